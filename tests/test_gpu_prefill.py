"""GPU parity of the prompt prefill (Transformer::forward with T > 1, SVL/nn/transformer.rs:139-154,
as FlowLm::prompt_text / prompt_voice run it, SVL/tts/flow_lm.rs:137-158) and of the voice-state
format (Voice::load, SVL/tts/voice.rs:103-143), against the oracle.

Bar: bit-exact.  A block of positions runs as the rows of one pass of the step's kernels (each
row with a single step's arithmetic, attending causally within the block), and the oracle's
forward computes each position with the same arithmetic, so outputs, caches and the steps that
follow are identical bits.
"""
import time

import numpy as np
import pytest

import oracle
import svl
from svl import workloads as W

pytestmark = pytest.mark.gpu


def _models(shape, seed):
    t = W.make_weights(shape, "f32", seed=seed)
    return svl.Model(shape.config(0), t), oracle.Model(shape.config(0), t)


def _xs(shape, b, t, seed):
    rng = np.random.default_rng([seed, 0xF0])
    return rng.standard_normal((b, t, shape.d_model), dtype=np.float32)


@pytest.mark.parametrize("t", [2, 37, 300], ids=["t2", "t37", "t300-two-blocks"])
def test_prefill_block_matches_oracle_then_steps(t):
    s = W.T1_SMALL
    g, o = _models(s, seed=80)
    gs, os_ = g.init_state(1, 512), o.new_state()
    # a first block, then a second one continuing the positions
    for k, n in enumerate((t, 5)):
        xs = _xs(s, 1, n, seed=81 + k)
        ys = g.forward(xs, gs)
        yo = os_.forward(xs)
        assert np.array_equal(ys.view(np.uint32), yo.view(np.uint32)), (k, float(np.max(np.abs(ys - yo))))
    assert gs.positions[0] == t + 5
    for layer, (k, v, first) in enumerate(gs.layer_caches()):
        ok, ov, _ = os_.cache(layer)
        assert first == 0 and np.array_equal(k, ok[0]) and np.array_equal(v, ov[0]), layer
    lat = W.latents(s, 4, seed=82)
    for i in range(4):
        z = g.backbone_step(lat[i][None], gs)[0]
        assert np.array_equal(z, os_.tts_step(lat[i])), i


def test_prefill_batch_of_streams_matches_each_stream():
    s = W.T1_SMALL
    g, o = _models(s, seed=83)
    B, t = 3, 20
    gs = g.init_state(B, 128)
    # the streams start at different positions
    caches = [W.prefill_caches(s, 4 * b, seed=84 + b) for b in range(B)]
    for b in range(B):
        gs.load_stream(b, *caches[b])
    xs = _xs(s, B, t, seed=85)
    ys = g.forward(xs, gs)
    for b in range(B):
        ob = o.state_from_layer_caches(*caches[b]) if b else o.new_state()
        assert np.array_equal(ys[b], ob.forward(xs[b][None])[0]), b


def test_prefill_is_faster_than_position_by_position():
    s = W.T1
    g, _ = _models(s, seed=0)
    xs = _xs(s, 1, 200, seed=86)
    g.forward(xs[:, :8], g.init_state(1, 512))  # warm up (the block's shadow state)
    st = g.init_state(1, 512)
    t0 = time.perf_counter()
    g.forward(xs, st)
    block = time.perf_counter() - t0
    st2 = g.init_state(1, 512)
    t0 = time.perf_counter()
    for i in range(200):
        g.forward(xs[:, i:i + 1], st2)
    steps = time.perf_counter() - t0
    print(f"Pocket-TTS prefill of 200 positions: {block * 1e3:.1f} ms as a block, {steps * 1e3:.1f} ms one by one")
    assert block < steps


def test_voice_state_round_trip_matches_oracle():
    s = W.T1_SMALL
    g, o = _models(s, seed=87)
    ks, vs = W.prefill_caches(s, 30, seed=88)
    st = g.init_state(1, 128)
    st.load_voice(W.voice_tensors(ks, vs, pad_to=45))  # offset 30 of 45 cached rows
    os_ = o.state_from_layer_caches(ks, vs)
    assert st.positions[0] == 30
    lat = W.latents(s, 5, seed=89)
    for i in range(5):
        assert np.array_equal(g.backbone_step(lat[i][None], st)[0], os_.tts_step(lat[i])), i


def test_voice_state_errors():
    s = W.T1_SMALL
    g, _ = _models(s, seed=90)
    ks, vs = W.prefill_caches(s, 6, seed=91)
    good = W.voice_tensors(ks, vs)
    st = g.init_state(1, 64)
    bad = dict(good)
    bad["transformer.layers.0.self_attn/pad"] = (svl.I64, (1,), np.array([2], np.int64))
    with pytest.raises(svl.SvlError) as e:
        st.load_voice(bad)
    assert e.value.code == svl.ERR_INVALID_INPUT
    missing = {k: v for k, v in good.items() if not k.startswith("transformer.layers.1.")}
    with pytest.raises(svl.SvlError):
        st.load_voice(missing)
    with pytest.raises(svl.SvlError):
        st.load_voice({"unrelated": good["transformer.layers.0.self_attn/offset"]})
    two = dict(good)
    c = good["transformer.layers.0.self_attn/cache"][2]
    c2 = np.concatenate([c, c], axis=1)
    two["transformer.layers.0.self_attn/cache"] = (svl.F32, c2.shape, c2)
    with pytest.raises(svl.SvlUnsupported):
        st.load_voice(two)
