"""GPU parity of the Q4_0 block format (candle BlockQ4_0 weights with Q8_0 activations): the GPU's
quantizer, block conversion, dequantization and GEMV against the oracle (oracle/formats.c).

Bar: bit-exact.  Block bytes equal the oracle's quantizer; dequantized values equal its closed
form; decode-step logits equal the oracle's bits (the GEMV forms candle's exact i32 block sum,
sum (code - 8) * q = sum code * q - 8 * sum q, and adds ((f32)sum * d_w) * d_x in block order).
"""
import os

import numpy as np
import pytest

import oracle
import svl
from svl import workloads as W

pytestmark = pytest.mark.gpu


def _name(layer, which):
    p = f"transformer.layers.{layer}."
    return p + {"in_proj": "self_attn.in_proj_weight", "out_proj": "self_attn.out_proj.weight",
                "ff1": "gating.linear_in.weight", "ff2": "gating.linear_out.weight"}[which]


def build(shape, seed):
    t = W.make_weights(shape, "q4_0", seed=seed)
    return t, svl.Model(shape.config(W.Q4_0), t), oracle.Model(shape.config(W.Q4_0), t)


def test_q4_0_quantize_and_dequantize_bit_exact():
    s = W.S1_SMALL
    t = W.make_weights(s, "q4_0", seed=50)
    # blocks across the f16 range, all-zero blocks and ties of magnitude in one linear
    name = _name(1, "ff1")
    shape = t[name][1]
    rng = np.random.default_rng(51)
    w = rng.standard_normal(shape).astype(np.float32).reshape(-1, 32)
    w *= (10.0 ** rng.uniform(-8, 5, size=(w.shape[0], 1))).astype(np.float32)
    w[::7] = 0.0
    w[3::11, 5] = -w[3::11, 2]
    t[name] = (W.F32, shape, w.reshape(shape))
    g = svl.Model(s.config(W.Q4_0), t)
    for lname, tname in [("text_linear", "text_linear.weight"), ("0.in_proj", _name(0, "in_proj")),
                         ("1.ff1", name), ("2.ff2", _name(2, "ff2"))]:
        x = t[tname][2]
        f32, blocks = g.linear_weight(lname)
        ob = oracle.quantize_q4_0(x)
        assert blocks is not None and blocks.shape[1] == x.shape[1] // 32 * 18, lname
        assert np.array_equal(blocks, ob), lname
        assert np.array_equal(f32.view(np.uint32), oracle.dequantize_q4_0(ob, x.shape[1]).view(np.uint32)), lname


def test_q4_0_candle_blocks_round_trip():
    s = W.S1_SMALL
    t = W.make_weights(s, "q4_0", seed=52)
    blocked = dict(t)
    for name, (dt, shp, data) in t.items():
        if dt == W.F32 and len(shp) == 2:
            blocked[name] = (W.Q4_0, shp, oracle.quantize_q4_0(data))
    g = svl.Model(s.config(0), blocked)
    _, blocks = g.linear_weight("0.in_proj")
    assert np.array_equal(blocks, blocked[_name(0, "in_proj")][2])


def test_q4_0_steps_match_oracle():
    """48 steps through a window of 24: logits bit-exact, tokens equal."""
    s = W.S1_SMALL
    _, g, o = build(s, seed=53)
    gs, os_ = g.init_state(), o.new_state()
    audio = W.audio_tokens(s, 48, seed=54)[0]
    text = s.text_card
    for i in range(48):
        tg, lg = g.step([text], audio[i][None], gs, want_logits=True)
        to, lo = os_.stt_step(text, audio[i], want_logits=True)
        assert tg[0] == to, f"step {i}"
        assert np.array_equal(lg[0].view(np.uint32), lo.view(np.uint32)), (i, float(np.max(np.abs(lg[0] - lo))))
        text = int(tg[0])


def test_q4_0_recognize_and_batches_match():
    """Greedy recognize = oracle; lockstep batches of 3 and 20 streams (Q4_0 linears stay on the
    GEMV path at any batch) = each stream alone, bit for bit."""
    s = W.S1_SMALL
    _, g, o = build(s, seed=55)
    audio = W.audio_tokens(s, 40, seed=56)[0]
    got = g.recognize(audio[:, None, :], g.init_state())[:, 0]
    assert np.array_equal(got, o.new_state().stt_greedy(audio))
    for B in (3, 20):
        n = 8
        aud = W.audio_tokens(s, n, seed=57 + B, batch=B)
        st = g.init_state(batch=B)
        caches = []
        for b in range(B):
            ks, vs = W.prefill_caches(s, (5 * b) % 30, seed=60 + b)
            caches.append((ks, vs))
            st.load_stream(b, ks, vs)
        batched = g.recognize(aud.transpose(1, 0, 2), st)
        for b in range(B):
            one = g.init_state()
            one.load_stream(0, *caches[b])
            assert np.array_equal(g.recognize(aud[b][:, None, :], one)[:, 0], batched[:, b]), (B, b)


def test_s1_q4_0_logits_bit_exact_and_greedy_tokens():
    """STT-1B shape with Q4_0 linears, window 750: 4 steps of bit-exact logits, 32 greedy tokens."""
    oracle.set_threads(min(16, os.cpu_count() or 4))
    _, g, o = build(W.S1, seed=0)
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
