"""GPU parity: libsvl (HIP, through the C ABI) against the oracle on the same seeded inputs.

Bars:
  * quantization / dequantization of weights: bit-exact to the oracle's candle restatement
  * logits, attention, norms, hidden states: bit-exact to the oracle with an f32 KV cache (the
    GPU kernels perform the oracle's f32 operations in the oracle's order), hence within the
    step contract's max-abs 1e-4 (f32) / 2e-2 (bf16) with room to spare; a bf16 KV cache is
    held to 2e-2
  * greedy tokens: identical over 256 steps
  * lockstep batches: bit-identical to the same streams run one by one
Reduced shapes keep the structure (GQA/windows wrap, gated SiLU, RMSNorm / LayerNorm) and let
the oracle finish in seconds; the full-size STT-1B Q8_0 run checks the 256-step greedy
identity at the benchmark shape.
"""
import os

import numpy as np
import pytest

import oracle
import svl
from svl import workloads as W

pytestmark = pytest.mark.gpu

F32_TOL = 1e-4
LOWP_TOL = 2e-2


def build(shape, dtype, seed=0, kv_dtype=svl.F32):
    t = W.make_weights(shape, dtype, seed=seed)
    q = W.quantize_code(dtype)
    return t, svl.Model(shape.config(q), t, kv_dtype=kv_dtype), oracle.Model(shape.config(q), t)


def _tensor_for(name, shape):
    if name == "text_linear":
        return "text_linear.weight"
    layer, which = name.split(".")
    p = f"transformer.layers.{layer}."
    return p + {"in_proj": "self_attn.in_proj_weight", "out_proj": "self_attn.out_proj.weight",
                "ff1": "gating.linear_in.weight", "ff2": "gating.linear_out.weight"}[which]


def test_q8_0_quantize_and_dequantize_bit_exact():
    s = W.S1_SMALL
    t, g, _ = build(s, "q8_0", seed=1)
    for name in ["text_linear", "0.in_proj", "1.out_proj", "2.ff1", "2.ff2"]:
        w = t[_tensor_for(name, s)][2]
        f32, blocks = g.linear_weight(name)
        ob = oracle.quantize_q8_0(w)
        assert np.array_equal(blocks, ob), name
        assert np.array_equal(f32.view(np.uint32), oracle.dequantize_q8_0(ob, w.shape[1]).view(np.uint32)), name


def test_f16_widening_exhaustive():
    """Every binary16 bit pattern through the GPU's f16 -> f32 upload equals numpy's exact
    widening (NaNs stay NaN)."""
    s = W.S1_SMALL
    t = W.make_weights(s, "f32", seed=21)
    name = "transformer.layers.0.gating.linear_in.weight"
    shape = t[name][1]
    n = shape[0] * shape[1]
    assert n >= 65536
    bits = (np.arange(n) % 65536).astype(np.uint16).reshape(shape)
    t[name] = (W.F16, shape, bits)
    g = svl.Model(s.config(0), t)
    got, _ = g.linear_weight("0.ff1")
    want = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_q8_0_quantize_scales_across_the_f16_range():
    """Block maxima from 1e-9 to 4e6: scales d = amax / 127 cover f16 subnormals, normals and
    overflow; the GPU's blocks equal the oracle's."""
    s = W.S1_SMALL
    t = W.make_weights(s, "q8_0", seed=22)
    name = "transformer.layers.1.gating.linear_in.weight"
    shape = t[name][1]
    rng = np.random.default_rng(23)
    w = rng.standard_normal(shape).astype(np.float32)
    blocks = w.reshape(-1, 32)
    blocks *= (10.0 ** rng.uniform(-9, 6.6, size=(blocks.shape[0], 1))).astype(np.float32)
    t[name] = (W.F32, shape, blocks.reshape(shape))
    g = svl.Model(s.config(W.Q8_0), t)
    _, got = g.linear_weight("1.ff1")
    assert np.array_equal(got, oracle.quantize_q8_0(t[name][2]))


def test_q8_0_candle_blocks_round_trip():
    s = W.S1_SMALL
    t = W.make_weights(s, "q8_0", seed=2)
    blocked = dict(t)
    for name, (dt, shp, data) in t.items():
        if dt == W.F32 and len(shp) == 2:
            blocked[name] = (W.Q8_0, shp, oracle.quantize_q8_0(data))
    g = svl.Model(s.config(0), blocked)
    f32, blocks = g.linear_weight("0.in_proj")
    assert np.array_equal(blocks, blocked["transformer.layers.0.self_attn.in_proj_weight"][2])


def test_q4k_quantize_and_dequantize_bit_exact():
    """The GPU's Q4K quantizer (scale/min fit per 32-value sub-block, 6-bit packing) writes the
    oracle's block bytes; the GPU's dequantization equals the oracle's closed form."""
    s = W.S2_SMALL
    t, g, _ = build(s, "q4k", seed=30)
    for name in ["text_linear", "0.in_proj", "1.out_proj", "1.ff1", "0.ff2"]:
        w = t[_tensor_for(name, s)][2]
        f32, blocks = g.linear_weight(name)
        ob = oracle.quantize_q4k(w)
        assert blocks is not None and np.array_equal(blocks, ob), name
        assert np.array_equal(f32.view(np.uint32), oracle.dequantize_q4k(ob, w.shape[1]).view(np.uint32)), name


def test_q4k_quantize_across_magnitudes_and_offsets():
    """Super-blocks from 1e-6 to 1e3 in magnitude, some all-positive (min term zero), some
    constant (scale zero): GPU blocks equal the oracle's."""
    s = W.S2_SMALL
    t = W.make_weights(s, "q4k", seed=31)
    name = "transformer.layers.1.gating.linear_in.weight"
    shape = t[name][1]
    rng = np.random.default_rng(32)
    w = rng.standard_normal(shape).astype(np.float32).reshape(-1, 256)
    w *= (10.0 ** rng.uniform(-6, 3, size=(w.shape[0], 1))).astype(np.float32)
    w[::7] = np.abs(w[::7]) + np.float32(0.5)
    w[::11, :32] = np.float32(0.25)
    w[::13] = np.float32(-1.5)
    t[name] = (W.F32, shape, w.reshape(shape))
    g = svl.Model(s.config(W.Q4K), t)
    _, got = g.linear_weight("1.ff1")
    assert np.array_equal(got, oracle.quantize_q4k(t[name][2]))


def test_q4k_candle_blocks_round_trip():
    """Candle Q4K block bytes handed to the model come back unchanged, and the model computes
    with them as with its own quantization of the same floats."""
    s = W.S2_SMALL
    t = W.make_weights(s, "q4k", seed=33)
    blocked = dict(t)
    for name, (dt, shp, data) in t.items():
        if dt == W.F32 and len(shp) == 2 and shp[1] % 256 == 0:
            blocked[name] = (W.Q4K, shp, oracle.quantize_q4k(data))
    g = svl.Model(s.config(0), blocked)
    _, blocks = g.linear_weight("0.ff1")
    assert np.array_equal(blocks, blocked["transformer.layers.0.gating.linear_in.weight"][2])
    g2 = svl.Model(s.config(W.Q4K), t)
    audio = W.audio_tokens(s, 12, seed=34)[0]
    a = g.recognize(audio[:, None, :], g.init_state())[:, 0]
    b = g2.recognize(audio[:, None, :], g2.init_state())[:, 0]
    assert np.array_equal(a, b)


def test_q4k_steps_match_oracle():
    """Q4K linears (activations quantized to Q8K): 64 steps through a window of 40, logits
    bit-exact to the oracle's Q4K x Q8K vec_dot, tokens equal."""
    s = W.S2_SMALL
    _, g, o = build(s, "q4k", seed=35)
    gs, os_ = g.init_state(), o.new_state()
    audio = W.audio_tokens(s, 64, seed=36)[0]
    text = s.text_card
    for i in range(64):
        tg, lg = g.step([text], audio[i][None], gs, want_logits=True)
        to, lo = os_.stt_step(text, audio[i], want_logits=True)
        assert tg[0] == to, f"step {i}"
        assert np.array_equal(lg[0].view(np.uint32), lo.view(np.uint32)), \
            f"step {i}: max diff {float(np.max(np.abs(lg[0] - lo)))}"
        text = int(tg[0])


def test_q4k_recognize_matches_oracle_greedy():
    s = W.S2_SMALL
    _, g, o = build(s, "q4k", seed=37)
    audio = W.audio_tokens(s, 150, seed=38)[0]
    got = g.recognize(audio[:, None, :], g.init_state())[:, 0]
    assert np.array_equal(got, o.new_state().stt_greedy(audio))


@pytest.mark.parametrize("dtype", ["q8_0", "bf16", "f32"])
def test_stt_small_steps_match_oracle(dtype):
    """64 steps through a window of 24 (the ring wraps twice): logits bit-exact, tokens equal."""
    s = W.S1_SMALL
    _, g, o = build(s, dtype, seed=3)
    gs, os_ = g.init_state(), o.new_state()
    audio = W.audio_tokens(s, 64, seed=4)[0]
    text = s.text_card
    worst = 0.0
    for i in range(64):
        tg, lg = g.step([text], audio[i][None], gs, want_logits=True)
        to, lo = os_.stt_step(text, audio[i], want_logits=True)
        worst = max(worst, float(np.max(np.abs(lg[0] - lo))))
        assert tg[0] == to, f"step {i}"
        assert np.array_equal(lg[0].view(np.uint32), lo.view(np.uint32)), f"step {i}: max diff {worst}"
        text = int(tg[0])
    print(f"{dtype}: max |logit diff| over 64 steps = {worst:.3g}")


def _with_heads(shape, nh=4, hd=6):
    """The shape with extra (VAD) heads, 4 x 6 as in the reference's STT configs."""
    return W.Shape(**{**shape.__dict__, "extra_heads_num": nh, "extra_heads_dim": hd})


PROB_TOL = 1e-6  # the GPU's expf and the C library's differ by a few ulp at most


@pytest.mark.parametrize("dtype", ["q8_0", "bf16", "f32"])
def test_stt_extra_heads_match_oracle(dtype):
    """Extra heads (SVL/stt/model.rs:259-271): per step the first-class probabilities within
    PROB_TOL of the oracle's, logits bit-exact and tokens equal (the heads change neither); the
    recognize loop returns every step's probabilities."""
    s = _with_heads(W.S1_SMALL)
    _, g, o = build(s, dtype, seed=41)
    gs, os_ = g.init_state(), o.new_state()
    audio = W.audio_tokens(s, 40, seed=42)[0]
    text = s.text_card
    worst = 0.0
    for i in range(40):
        tg, lg, pg = g.step([text], audio[i][None], gs, want_logits=True, want_probs=True)
        to, lo, po = os_.stt_step(text, audio[i], want_logits=True, want_probs=True)
        assert tg[0] == to, f"step {i}"
        assert np.array_equal(lg[0].view(np.uint32), lo.view(np.uint32)), f"step {i}"
        worst = max(worst, float(np.max(np.abs(pg[0] - po))))
        assert worst < PROB_TOL, f"step {i}: {pg[0]} vs {po}"
        text = int(tg[0])
    toks, probs = g.recognize(audio[:, None, :], g.init_state(), want_probs=True)
    otoks, oprobs = o.new_state().stt_greedy(audio, want_probs=True)
    assert np.array_equal(toks[:, 0], otoks)
    assert float(np.max(np.abs(probs[:, 0] - oprobs))) < PROB_TOL
    print(f"{dtype}: max |probability diff| = {worst:.3g}")


@pytest.mark.parametrize("B", [3, 17])
def test_stt_extra_heads_batch_matches_oracle(B):
    """Lockstep batches (GEMV path at 3 streams, MFMA GEMMs at 17): each stream's tokens equal the
    oracle's independent greedy run and its probabilities are within PROB_TOL."""
    s = _with_heads(W.S1_SMALL)
    _, g, o = build(s, "q8_0", seed=43)
    n = 24
    audio = W.audio_tokens(s, n, seed=44, batch=B)
    toks, probs = g.recognize(np.ascontiguousarray(audio.transpose(1, 0, 2)), g.init_state(batch=B),
                              want_probs=True)
    for b in range(B):
        ot, op = o.new_state().stt_greedy(audio[b], want_probs=True)
        assert np.array_equal(toks[:, b], ot), f"stream {b}"
        assert float(np.max(np.abs(probs[:, b] - op))) < PROB_TOL, f"stream {b}"


def test_stt_small_recognize_matches_oracle_greedy():
    s = W.S1_SMALL
    _, g, o = build(s, "q8_0", seed=5)
    audio = W.audio_tokens(s, 200, seed=6)[0]
    got = g.recognize(audio[:, None, :], g.init_state())[:, 0]
    assert np.array_equal(got, o.new_state().stt_greedy(audio))


def test_lockstep_batch_equals_independent_streams():
    s = W.S1_SMALL
    _, g, _ = build(s, "q8_0", seed=7)
    B, n = 5, 40
    audio = W.audio_tokens(s, n, seed=8, batch=B)  # [B, n, n_q]
    st = g.init_state(batch=B)
    # streams start at different positions: prefill stream b with b*3 seeded keys
    caches = {}
    for b in range(B):
        ks, vs = W.prefill_caches(s, 3 * b, seed=20 + b)
        caches[b] = (ks, vs)
        st.load_stream(b, ks, vs)
    batched = g.recognize(audio.transpose(1, 0, 2), st)
    for b in range(B):
        one = g.init_state()
        one.load_stream(0, *caches[b])
        assert np.array_equal(g.recognize(audio[b][:, None, :], one)[:, 0], batched[:, b]), b


# text vocabulary 8000: text_linear runs in 32-row GEMM tiles, the other linears in 16-row tiles
S1_SMALL_VOCAB = W.stt_shape("stt-small-vocab", 256, 2, 4, 4.125, 24, card=64, n_q=4, text_card=8000)
# d_model 320: 10 blocks, three 128-byte chunks, the last one half full (an odd chunk count, fewer
# chunks than the loads issued ahead); FF hidden 672: 21 blocks, so the FF-out linear of the batch
# runs on the GEMV path (the GEMM's weight scales travel in pairs)
S1_ODD_CHUNKS = W.stt_shape("stt-odd-chunks", 320, 2, 5, 3.15, 24, card=64, n_q=4, text_card=100)


@pytest.mark.parametrize("shape", [W.S1_SMALL, S1_SMALL_VOCAB, S1_ODD_CHUNKS], ids=["small", "vocab8000", "odd-chunks"])
def test_mfma_batch_equals_independent_streams(shape):
    """A lockstep batch large enough for the MFMA GEMM path (20 streams at different positions):
    logits and tokens bit-identical to each stream stepped alone through the GEMV path."""
    s = shape
    _, g, _ = build(s, "q8_0", seed=24)
    B, n = 20, 10
    audio = W.audio_tokens(s, n, seed=25, batch=B)
    st = g.init_state(batch=B)
    caches = []
    for b in range(B):
        ks, vs = W.prefill_caches(s, (7 * b) % 30, seed=40 + b)
        caches.append((ks, vs))
        st.load_stream(b, ks, vs)
    singles = []
    for b in range(B):
        one = g.init_state()
        one.load_stream(0, *caches[b])
        singles.append(one)
    text = np.full(B, s.text_card, dtype=np.uint32)
    for i in range(n):
        tb, lb = g.step(text, audio[:, i], st, want_logits=True)
        for b in range(B):
            t1, l1 = g.step([text[b]], audio[b, i][None], singles[b], want_logits=True)
            assert np.array_equal(lb[b].view(np.uint32), l1[0].view(np.uint32)), (i, b)
            assert tb[b] == t1[0]
        text = tb.astype(np.uint32)


def test_state_duplicate_reset_and_caches():
    s = W.S1_SMALL
    _, g, o = build(s, "f32", seed=9)
    audio = W.audio_tokens(s, 30, seed=10)[0]
    st = g.init_state()
    g.recognize(audio[:10, None], st)
    dup = st.duplicate()
    a = g.recognize(audio[10:, None], st)
    b = g.recognize(audio[10:, None], dup)
    assert np.array_equal(a, b)
    # layer caches: the last `context` keys, equal to the oracle's within f32 tolerance
    os_ = o.new_state()
    os_.stt_greedy(audio)
    for layer, (k, v, first) in enumerate(st.layer_caches()):
        ok, ov, ostart = os_.cache(layer)
        n = k.shape[1]
        assert first == 30 - n and n == s.context
        assert np.array_equal(k, ok[0, :, -n:]) and np.array_equal(v, ov[0, :, -n:])
    st.reset()
    assert np.array_equal(g.recognize(audio[:10, None], st), g.recognize(audio[:10, None], g.init_state()))


def test_tts_small_prefilled_matches_oracle():
    s = W.T1_SMALL
    _, g, o = build(s, "f32", seed=11)
    ks, vs = W.prefill_caches(s, 40, seed=12)
    gs = g.state_from_layer_caches(ks, vs, capacity=128)
    os_ = o.state_from_layer_caches(ks, vs)
    lat = W.latents(s, 12, seed=13)
    for i in range(12):
        z = g.backbone_step(None if i == 0 else lat[i][None], gs)[0]
        zo = os_.tts_step(None if i == 0 else lat[i])
        assert np.array_equal(z, zo), (i, float(np.max(np.abs(z - zo))))


# FF hidden 2048: the FF-out linear (f32, K = 2048) has lane chains of 32 loads and one row per
# unit, so its units stage their rows in LDS before the chains run
T_STAGED = W.tts_shape("tts-staged-ff-out", 256, 2, 4, 2048, flow_dim=64, flow_depth=1)


def test_tts_staged_dense_rows_match_oracle_and_persistent(monkeypatch):
    s = T_STAGED
    _, g, o = build(s, "f32", seed=31)
    ks, vs = W.prefill_caches(s, 40, seed=32)
    gs = g.state_from_layer_caches(ks, vs, capacity=128)
    os_ = o.state_from_layer_caches(ks, vs)
    monkeypatch.setenv("SVL_STEP_LAUNCH", "persistent")  # read when a state is created
    gp = g.state_from_layer_caches(ks, vs, capacity=128)
    monkeypatch.delenv("SVL_STEP_LAUNCH")
    lat = W.latents(s, 8, seed=33)
    for i in range(8):
        x = None if i == 0 else lat[i][None]
        z = g.backbone_step(x, gs)[0]
        zp = g.backbone_step(x, gp)[0]
        zo = os_.tts_step(None if i == 0 else lat[i])
        assert np.array_equal(z, zo), (i, float(np.max(np.abs(z - zo))))
        assert np.array_equal(z, zp), i


def test_stt_bf16_staged_dense_rows_match_oracle():
    """bf16 linears with FF hidden 4096: the FF-out linear (K = 4096, bf16) has 32-load chains and
    stages its rows."""
    s = W.stt_shape("stt-staged-bf16", 256, 2, 4, 24.0, 24, card=64, n_q=4, text_card=100)
    assert s.ff_hidden == 4096
    _, g, o = build(s, "bf16", seed=34)
    gs, os_ = g.init_state(), o.new_state()
    audio = W.audio_tokens(s, 6, seed=35)[0]
    text = s.text_card
    for i in range(6):
        tg, lg = g.step([text], audio[i][None], gs, want_logits=True)
        to, lo = os_.stt_step(text, audio[i], want_logits=True)
        assert np.array_equal(lg[0].view(np.uint32), lo.view(np.uint32)), i
        assert tg[0] == to
        text = int(tg[0])


def test_transformer_forward_matches_oracle():
    s = W.Shape("fwd", W.MODEL_TRANSFORMER, 128, 2, 2, 1, 64, W.FF_PLAIN, 256, W.NORM_LAYER, 1e-5, 7,
                layer_scale=1)
    t = W.make_weights(s, "f32", seed=14)
    g, o = svl.Model(s.config(0), t), oracle.Model(s.config(0), t)
    xs = np.random.default_rng(15).standard_normal((1, 20, 128)).astype(np.float32)
    gs, os_ = g.init_state(), o.new_state()
    y1 = g.forward(xs[:, :13], gs)
    y2 = g.forward(xs[:, 13:], gs)
    yo = os_.forward(xs)
    assert np.array_equal(np.concatenate([y1, y2], axis=1), yo)
    assert gs.positions[0] == 20


def test_bf16_kv_cache_stays_within_low_precision_bar():
    s = W.S1_SMALL
    _, g, o = build(s, "f32", seed=16, kv_dtype=svl.BF16)
    gs, os_ = g.init_state(), o.new_state()
    audio = W.audio_tokens(s, 30, seed=17)[0]
    text = s.text_card
    for i in range(30):
        tg, lg = g.step([text], audio[i][None], gs, want_logits=True)
        _, lo = os_.stt_step(text, audio[i], want_logits=True)
        assert np.max(np.abs(lg[0] - lo)) < LOWP_TOL
        text = int(tg[0])


def test_input_errors():
    s = W.S1_SMALL
    _, g, _ = build(s, "f32", seed=18)
    st = g.init_state()
    with pytest.raises(svl.SvlError) as e:
        g.step([s.text_card + 1], np.zeros((1, s.n_q)), st)
    assert e.value.code == svl.ERR_INVALID_INPUT
    with pytest.raises(svl.SvlError) as e:
        g.recognize(np.full((2, 1, s.n_q), s.card + 1), st)
    assert e.value.code == svl.ERR_INVALID_INPUT
    assert st.positions[0] == 0  # rejected inputs leave the state untouched
    t = W.make_weights(W.T1_SMALL, "f32")
    gt = svl.Model(W.T1_SMALL.config(0), t)
    full = gt.init_state(capacity=2)
    gt.backbone_step(None, full)
    gt.backbone_step(None, full)
    with pytest.raises(svl.SvlError) as e:
        gt.backbone_step(None, full)
    assert e.value.code == svl.ERR_INVALID_INPUT
    with pytest.raises(svl.SvlError):
        gt.init_state(capacity=0)
    bad = dict(t)
    bad["input_linear.weight"] = (W.F32, (3, 3), np.zeros((3, 3), np.float32))
    with pytest.raises(svl.SvlError) as e:
        svl.Model(W.T1_SMALL.config(0), bad)
    assert e.value.code == svl.ERR_INVALID_INPUT


# ---- benchmark shapes -------------------------------------------------------------------------

@pytest.fixture(scope="module")
def s1_q8():
    oracle.set_threads(min(16, os.cpu_count() or 4))
    t, g, o = build(W.S1, "q8_0", seed=0)
    del t
    return g, o


def test_s1_q8_0_256_greedy_steps_token_identical(s1_q8):
    """STT-1B shape, Q8_0, batch 1, window 750: 256 greedy steps equal the oracle's."""
    g, o = s1_q8
    audio = W.audio_tokens(W.S1, 256, seed=1)[0]
    got = g.recognize(audio[:, None, :], g.init_state())[:, 0]
    expected = o.new_state().stt_greedy(audio)
    assert np.array_equal(got, expected), np.flatnonzero(got != expected)[:5]


def test_s1_q8_0_logits_within_bar(s1_q8):
    g, o = s1_q8
    audio = W.audio_tokens(W.S1, 6, seed=2)[0]
    gs, os_ = g.init_state(), o.new_state()
    text = W.S1.text_card
    for i in range(6):
        tg, lg = g.step([text], audio[i][None], gs, want_logits=True)
        to, lo = os_.stt_step(text, audio[i], want_logits=True)
        assert np.max(np.abs(lg[0] - lo)) < LOWP_TOL and tg[0] == to
        text = to


def _lockstep_fills(shape, B, seed=7):
    """The B = 64 benchmark's rings: stream b pre-filled with the first fills[b] positions of one
    seeded full-window cache, fills uniform in [1, window]."""
    fills = [int(f) for f in np.random.default_rng(seed).integers(1, shape.context + 1, size=B)]
    ks, vs = W.prefill_caches(shape, shape.context, seed=8)
    return fills, ks, vs


def test_s1_q8_0_64_stream_lockstep_matches_gemv_and_oracle(s1_q8):
    """The B = 64 benchmark configuration: STT-1B Q8_0, 64 streams with rings pre-filled to
    seeded fills in [1, 750], lockstep steps through the MFMA GEMM path.  Every stream's logits
    and tokens are bit-equal to the same stream stepped alone (GEMV path), and the first streams
    equal the oracle's."""
    g, o = s1_q8
    s, B, n = W.S1, 64, 4
    fills, ks, vs = _lockstep_fills(s, B)
    st = g.init_state(batch=B)
    for b in range(B):
        st.load_stream(b, [k[:, :, :fills[b]] for k in ks], [v[:, :, :fills[b]] for v in vs])
    audio = W.audio_tokens(s, n, seed=1, batch=B)  # [B, n, n_q]
    text = np.full(B, s.text_card, dtype=np.uint32)
    texts, logits, toks = [], [], []
    for i in range(n):
        tb, lb = g.step(text, audio[:, i], st, want_logits=True)
        texts.append(text.copy())
        logits.append(lb)
        toks.append(tb)
        text = tb.astype(np.uint32)
    del st
    for b in range(B):
        one = g.init_state()
        one.load_stream(0, [k[:, :, :fills[b]] for k in ks], [v[:, :, :fills[b]] for v in vs])
        ob = None
        if b < 4:
            ob = o.state_from_layer_caches([k[:, :, :fills[b]] for k in ks], [v[:, :, :fills[b]] for v in vs])
        for i in range(n):
            t1, l1 = g.step([texts[i][b]], audio[b, i][None], one, want_logits=True)
            assert np.array_equal(logits[i][b].view(np.uint32), l1[0].view(np.uint32)), (b, i, fills[b])
            assert toks[i][b] == t1[0], (b, i)
            if ob is not None:
                to, lo = ob.stt_step(int(texts[i][b]), audio[b, i], want_logits=True)
                assert np.array_equal(l1[0].view(np.uint32), lo.view(np.uint32)), (b, i, fills[b])
                assert to == t1[0]


def test_s1_q8_0_split_attention_through_the_window_wrap(s1_q8, monkeypatch):
    """Batch 1 at the full window: rings pre-filled to 740 positions, 24 steps through the wrap of
    the 750-slot window.  The split attention launches (16 units per head) give the bits of one
    unit per head, and the first 3 steps equal the oracle's."""
    g, o = s1_q8
    s = W.S1
    ks, vs = W.prefill_caches(s, 740, seed=72)
    audio = W.audio_tokens(s, 24, seed=73)[0]
    runs = []
    for split in ("0", "32"):
        monkeypatch.setenv("SVL_ATTN_SPLIT", split)
        st = g.init_state()
        st.load_stream(0, ks, vs)
        text, logits = s.text_card, []
        for i in range(24):
            tok, lg = g.step([text], audio[i][None], st, want_logits=True)
            logits.append(lg[0])
            text = int(tok[0])
        runs.append(np.stack(logits))
        del st
    assert np.array_equal(runs[0].view(np.uint32), runs[1].view(np.uint32))
    ob = o.state_from_layer_caches(ks, vs)
    text = s.text_card
    for i in range(3):
        to, lo = ob.stt_step(text, audio[i], want_logits=True)
        assert np.array_equal(runs[1][i].view(np.uint32), lo.view(np.uint32)), i
        text = int(to)


@pytest.fixture(scope="module")
def s1_bf16():
    oracle.set_threads(min(16, os.cpu_count() or 4))
    t, g, o = build(W.S1, "bf16", seed=0)
    del t
    return g, o


def test_s1_bf16_logits_bit_exact_and_greedy_tokens(s1_bf16):
    """STT-1B shape, bf16 weights (f32 arithmetic, 16-lane dot), window 750: the first 4 steps'
    logits bit-exact to the oracle, then 32 greedy steps token-identical."""
    g, o = s1_bf16
    audio = W.audio_tokens(W.S1, 32, seed=1)[0]
    gs, os_ = g.init_state(), o.new_state()
    text = W.S1.text_card
    for i in range(4):
        a = audio[i] if i else np.full(W.S1.n_q, W.S1.card, np.uint32)
        tg, lg = g.step([text], a[None], gs, want_logits=True)
        to, lo = os_.stt_step(text, a, want_logits=True)
        assert np.array_equal(lg[0].view(np.uint32), lo.view(np.uint32)), (i, float(np.max(np.abs(lg[0] - lo))))
        assert tg[0] == to
        text = to
    got = g.recognize(audio[:, None, :], g.init_state())[:, 0]
    assert np.array_equal(got, o.new_state().stt_greedy(audio))


def test_s2_q4k_window_3000_logits_and_greedy_tokens():
    """STT-2.6B shape, Q4K linears (Q8K activations), window 3000: 8 steps of bit-exact logits,
    then 16 greedy steps token-identical."""
    oracle.set_threads(min(16, os.cpu_count() or 4))
    t, g, o = build(W.S2, "q4k", seed=0)
    del t
    audio = W.audio_tokens(W.S2, 16, seed=1)[0]
    gs, os_ = g.init_state(), o.new_state()
    text = W.S2.text_card
    for i in range(8):
        a = audio[i] if i else np.full(W.S2.n_q, W.S2.card, np.uint32)
        tg, lg = g.step([text], a[None], gs, want_logits=True)
        to, lo = os_.stt_step(text, a, want_logits=True)
        assert np.array_equal(lg[0].view(np.uint32), lo.view(np.uint32)), (i, float(np.max(np.abs(lg[0] - lo))))
        assert tg[0] == to
        text = to
    got = g.recognize(audio[:, None, :], g.init_state())[:, 0]
    assert np.array_equal(got, o.new_state().stt_greedy(audio))


def test_t1_f32_prefilled_256_within_f32_bar():
    """Pocket-TTS shape, f32, 256 prefilled positions, 16 steps: z within 1e-4."""
    s = W.T1
    t, g, o = build(s, "f32", seed=0)
    ks, vs = W.prefill_caches(s, 256, seed=3)
    gs = g.state_from_layer_caches(ks, vs, capacity=512)
    os_ = o.state_from_layer_caches(ks, vs)
    lat = W.latents(s, 16, seed=4)
    for i in range(16):
        z = g.backbone_step(lat[i][None], gs)[0]
        zo = os_.tts_step(lat[i])
        assert np.array_equal(z, zo), (i, float(np.max(np.abs(z - zo))))


S_HD128 = W.stt_shape("stt-small-hd128", 512, 2, 4, 4.125, 24, card=64, n_q=4, text_card=100)


@pytest.mark.parametrize("kv", [svl.F32, svl.BF16], ids=["f32kv", "bf16kv"])
@pytest.mark.parametrize("shape", [W.S1_SMALL, S_HD128, W.T1_SMALL], ids=["hd64", "hd128", "tts-hd64"])
def test_attention_head_pairs_equal_single_heads(monkeypatch, shape, kv):
    """Two heads per attention unit (the schedule of large batches) gives the same bits as one
    head per unit: STT logits over 40 steps through a wrapping window, TTS z over 12 steps."""
    t = W.make_weights(shape, "q8_0" if shape.kind == W.MODEL_STT else "f32", seed=41)
    q = W.Q8_0 if shape.kind == W.MODEL_STT else 0
    results = []
    for pairs in ("0", "1"):
        monkeypatch.setenv("SVL_ATTN_PAIRS", pairs)
        g = svl.Model(shape.config(q), t, kv_dtype=kv)
        if shape.kind == W.MODEL_STT:
            st = g.init_state(batch=3)
            audio = W.audio_tokens(shape, 40, seed=42, batch=3)
            text = np.full(3, shape.text_card, dtype=np.uint32)
            logits = []
            for i in range(40):
                tok, lg = g.step(text, audio[:, i], st, want_logits=True)
                logits.append(lg)
                text = tok.astype(np.uint32)
            results.append(np.stack(logits))
        else:
            ks, vs = W.prefill_caches(shape, 20, seed=43)
            st = g.state_from_layer_caches(ks, vs, capacity=64)
            lat = W.latents(shape, 12, seed=44)
            results.append(np.stack([g.backbone_step(lat[i][None], st) for i in range(12)]))
    assert np.array_equal(results[0].view(np.uint32), results[1].view(np.uint32))


def test_persistent_and_per_phase_launches_agree(monkeypatch):
    """The persistent step kernel and one launch per phase run the same units: same bits."""
    s = W.S1_SMALL
    t = W.make_weights(s, "q8_0", seed=19)
    g = svl.Model(s.config(W.Q8_0), t)
    audio = W.audio_tokens(s, 30, seed=20)[0][:, None, :]
    monkeypatch.setenv("SVL_STEP_LAUNCH", "persistent")
    a = g.recognize(audio, g.init_state())
    monkeypatch.setenv("SVL_STEP_LAUNCH", "phases")
    st = g.init_state()
    b = g.recognize(audio, st)
    assert np.array_equal(a, b)


# ---- norm statistics on chosen rows -------------------------------------------------------------

def _stat_rows(k, seed):
    """Rows that stress an element-order sum: normal residuals, magnitudes over 40 binades, few
    distinct dyadic values (rounding ties at every step), a large first term, sparse spikes,
    zeros (leading, scattered, whole row), tiny values, and non-finite or huge terms."""
    rng = np.random.default_rng(seed)
    rows = []
    for kind in range(12):
        for _ in range(24 if kind < 8 else 4):
            if kind == 0:
                r = rng.standard_normal(k)
            elif kind == 1:
                r = rng.standard_normal(k) * 2.0 ** rng.integers(-20, 20, k)
            elif kind == 2:
                r = rng.integers(0, 7, k) * 0.25
            elif kind == 3:
                r = rng.standard_normal(k) * 0.01
                r[0] = 1000.0
            elif kind == 4:
                r = np.where(np.arange(k) % 97 == 0, rng.standard_normal(k) * 100, rng.standard_normal(k) * 1e-3)
            elif kind == 5:
                r = np.where(rng.integers(0, 3, k) == 0, 0.0, rng.standard_normal(k))
            elif kind == 6:
                r = np.where(np.arange(k) < k // 2, 0.0, rng.standard_normal(k))
            elif kind == 7:
                r = rng.integers(0, 4096, k) * 2.0 ** -12
            elif kind == 8:
                r = np.zeros(k)
            elif kind == 9:
                r = rng.standard_normal(k) * 1e-30
            elif kind == 10:
                r = rng.standard_normal(k) * 1e25
            else:
                r = rng.standard_normal(k)
                r[rng.integers(0, k)] = np.inf
            rows.append(r)
    return np.array(rows, dtype=np.float32)


@pytest.mark.parametrize("k", [2048, 2560, 1024, 4096, 256, 260, 36])
def test_norm_statistics_bit_exact_on_stress_rows(k):
    """The step's RMSNorm / LayerNorm statistics (exact parallel sum of squares, sequential
    LayerNorm sums) equal the oracle's element-order sums bit for bit, rows chosen to hit every
    branch: ties, binade edges, zeros, fallbacks."""
    x = _stat_rows(k, seed=k)
    alpha = np.ones(k, np.float32)
    got_rms = svl.row_stats(x, svl.NORM_RMS)
    got_ln = svl.row_stats(x, svl.NORM_LAYER)
    with np.errstate(over="ignore", invalid="ignore"):
        # numpy's accumulate adds in index order with one f32 accumulator (no pairwise blocking)
        seq2s = np.add.accumulate(x * x, axis=1, dtype=np.float32)[:, -1]
        seq1s = np.add.accumulate(x, axis=1, dtype=np.float32)[:, -1]
    for r in range(x.shape[0]):
        seq2, seq1 = seq2s[r], seq1s[r]
        for got, want in ((got_rms[r, 0], seq2), (got_ln[r, 0], seq2), (got_ln[r, 1], seq1)):
            assert (np.isnan(got) and np.isnan(want)) or np.float32(got).view(np.uint32) == np.float32(want).view(np.uint32), (k, r, got, want)
    # the oracle's RMSNorm from the same sums
    y = oracle.rms_norm(x[:24], alpha, 1e-8)
    m = np.sqrt(got_rms[:24, 0] / np.float32(k) + np.float32(1e-8), dtype=np.float32)
    assert np.array_equal((x[:24] / m[:, None]).view(np.uint32), y.view(np.uint32))


# ---- boundary: bounded RoPE storage, device-side input checks, LDS fit --------------------------

def test_rope_rows_past_the_table_cap_match_oracle(monkeypatch):
    """With the model's RoPE table capped at 64 positions every later position takes its rows from
    the per-call computation: 150 steps through a window of 24 stay bit-exact, and a lockstep batch
    whose streams straddle the cap equals its streams run alone."""
    monkeypatch.setenv("SVL_ROPE_TABLE_POSITIONS", "64")
    s = W.S1_SMALL
    t, g, o = build(s, "q8_0", seed=51)
    audio = W.audio_tokens(s, 150, seed=52)[0]
    gs, os_ = g.init_state(), o.new_state()
    text = s.text_card
    for i in range(150):
        a = audio[i] if i else np.full(s.n_q, s.card, np.uint32)
        tg, lg = g.step([text], a[None], gs, want_logits=True)
        to, lo = os_.stt_step(text, a, want_logits=True)
        assert np.array_equal(lg[0].view(np.uint32), lo.view(np.uint32)), i
        text = to
    got = g.recognize(audio[:, None, :], g.init_state())[:, 0]
    assert np.array_equal(got, o.new_state().stt_greedy(audio))
    B, n = 4, 12
    fills = [10, 58, 63, 90]
    batch = W.audio_tokens(s, n, seed=53, batch=B)
    st = g.init_state(batch=B)
    caches = []
    for b in range(B):
        ks, vs = W.prefill_caches(s, fills[b], seed=60 + b)
        caches.append((ks, vs))
        st.load_stream(b, ks, vs)
    together = g.recognize(np.ascontiguousarray(batch.transpose(1, 0, 2)), st)
    for b in range(B):
        one = g.init_state()
        one.load_stream(0, *caches[b])
        assert np.array_equal(g.recognize(batch[b][:, None, :], one)[:, 0], together[:, b]), b
        ob = o.state_from_layer_caches(*caches[b])
        assert np.array_equal(ob.stt_greedy(batch[b]), together[:, b]), b


def test_async_recognize_reports_bad_token_ids_at_synchronize():
    """The async entry point cannot see its device token ids on the host: an id past `card`
    raises the state's flag and svl_state_synchronize returns InvalidInput once, as the
    synchronous call rejects the same input up front."""
    from svl import hip

    s = W.S1_SMALL
    _, g, _ = build(s, "q8_0", seed=54)
    audio = W.audio_tokens(s, 6, seed=55)[0][:, None, :].copy()
    st = g.init_state()
    d_ok = hip.DeviceBuffer.from_array(audio)
    d_out = hip.DeviceBuffer(6 * 4)
    g.recognize_async(6, d_ok.address, d_out.address, st)
    st.synchronize()
    bad = audio.copy()
    bad[3, 0, 1] = s.card + 5
    with pytest.raises(svl.SvlError) as e:
        g.recognize(bad, g.init_state())
    assert e.value.code == svl.ERR_INVALID_INPUT
    d_bad = hip.DeviceBuffer.from_array(bad)
    st2 = g.init_state()
    g.recognize_async(6, d_bad.address, d_out.address, st2)
    with pytest.raises(svl.SvlError) as e:
        st2.synchronize()
    assert e.value.code == svl.ERR_INVALID_INPUT
    st2.synchronize()  # reported once
    st2.reset()
    g.recognize_async(6, d_ok.address, d_out.address, st2)
    st2.synchronize()


def test_large_capacity_batch_fits_lds_or_is_unsupported():
    """A TTS state with 10000 slots and 32 streams: two heads' scores per attention unit would
    exceed the LDS, so the state falls back to one head per unit and steps correctly; past the
    ring limit the library answers "unsupported" instead of failing at launch."""
    s = W.T1_SMALL
    t = W.make_weights(s, "f32", seed=56)
    g = svl.Model(s.config(0), t)
    o = oracle.Model(s.config(0), t)
    st = g.init_state(batch=32, capacity=10000)
    lat = W.latents(s, 3, seed=57)
    os_ = o.new_state()
    for i in range(3):
        z = g.backbone_step(np.repeat(lat[i][None], 32, axis=0), st)
        zo = os_.tts_step(lat[i])
        for b in (0, 31):
            assert np.array_equal(z[b].view(np.uint32), zo.view(np.uint32)), (i, b)
    with pytest.raises(svl.SvlUnsupported):
        g.init_state(batch=1, capacity=20000)
