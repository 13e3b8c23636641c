"""GPU parity of the TTS step's heads: FlowLm::step's end-of-speech logit and flow-head decode
(SVL/tts/flow_lm.rs:162-185, 206-387) through svl_tts_step / svl_tts_step_async, against the
oracle (oracle/flow.c) on the same seeded weights, latents and noise.

Bar: bit-exact.  The kernels perform the oracle's f32 operations in the oracle's order (the
reference's 16-lane matvec dot and bias, its SiLU, candle-nn's layer_norm, the tensor-op norms
and affines), so the next latent and the logit are identical bits, frame after frame with the
latent fed back.
"""
import numpy as np
import pytest

import oracle
import svl
from svl import hip
from svl import workloads as W

pytestmark = pytest.mark.gpu

TINY = W.tts_shape("tts-flow-tiny", 128, 2, 2, 256, latent=8, flow_dim=64, flow_depth=2)


def _models(shape, seed):
    t = W.make_weights(shape, "f32", seed=seed)
    return svl.Model(shape.config(0), t), oracle.Model(shape.config(0), t)


def _noise(shape, frames, batch, seed):
    rng = np.random.default_rng([seed, 0x0015E])
    return rng.standard_normal((frames, batch, shape.latent_dim), dtype=np.float32)


def _run_pair(shape, g, o, frames, steps, seed, gs=None, os_=None, threshold=-4.0):
    gs = gs or g.init_state(1, 256)
    os_ = os_ or o.new_state()
    noise = _noise(shape, frames, 1, seed)
    lat_g = lat_o = None
    for f in range(frames):
        out, logit, flag = g.tts_step(lat_g, noise[f], gs, decode_steps=steps, eos_threshold=threshold)
        want, eos = os_.tts_full_step(lat_o, noise[f, 0], decode_steps=steps)
        assert np.array_equal(out[0], want), (f, float(np.max(np.abs(out[0] - want))))
        assert logit[0] == np.float32(eos), (f, logit[0], eos)
        assert flag[0] == int(eos > threshold)
        lat_g, lat_o = out, want
    return gs, os_


def test_tts_step_small_matches_oracle():
    g, o = _models(W.T1_SMALL, seed=21)
    _run_pair(W.T1_SMALL, g, o, frames=10, steps=1, seed=1)


@pytest.mark.parametrize("kind", [W.FLOW_LSD, W.FLOW_MATCHING, W.FLOW_DRIFTING, W.FLOW_POINTWISE],
                         ids=["lsd", "flow_matching", "drifting", "pointwise"])
@pytest.mark.parametrize("steps", [1, 2, 3])
def test_tts_step_every_flow_kind_and_step_count(kind, steps):
    shape = W.tts_shape("tts-flow-kind", 128, 2, 2, 256, latent=8, flow_dim=64, flow_depth=2, flow_kind=kind)
    g, o = _models(shape, seed=30 + kind)
    _run_pair(shape, g, o, frames=4, steps=steps, seed=steps)


def test_tts_step_batch_equals_streams_and_oracle():
    shape = TINY
    g, o = _models(shape, seed=23)
    B, frames = 3, 5
    noise = _noise(shape, frames, B, seed=4)
    gs = g.init_state(B, 64)
    ostates = [o.new_state() for _ in range(B)]
    lat = None
    lat_o = [None] * B
    for f in range(frames):
        out, logits, _ = g.tts_step(lat, noise[f], gs, decode_steps=2)
        for b in range(B):
            want, eos = ostates[b].tts_full_step(lat_o[b], noise[f, b], decode_steps=2)
            assert np.array_equal(out[b], want), (f, b)
            assert logits[b] == np.float32(eos)
            lat_o[b] = want
        lat = out


def test_t1_full_shape_prefilled_matches_oracle():
    """Pocket-TTS shape (d 1024, 6 layers, flow head 512 x 6 LSD), 256 prefilled positions."""
    s = W.T1
    g, o = _models(s, seed=0)
    ks, vs = W.prefill_caches(s, 256, seed=3)
    gs = g.state_from_layer_caches(ks, vs, capacity=512)
    os_ = o.state_from_layer_caches(ks, vs)
    _run_pair(s, g, o, frames=8, steps=1, seed=5, gs=gs, os_=os_)


def test_tts_step_async_chain_equals_sync():
    """Frames enqueued with device pointers, each fed the previous frame's device latent, give the
    synchronous call's bits."""
    shape = TINY
    g, _ = _models(shape, seed=25)
    frames, ld = 6, shape.latent_dim
    noise = _noise(shape, frames, 1, seed=6)
    s_sync, s_async = g.init_state(1, 64), g.init_state(1, 64)
    want, lat = [], None
    for f in range(frames):
        out, logit, _ = g.tts_step(lat, noise[f], s_sync, decode_steps=1)
        want.append((out[0].copy(), logit[0]))
        lat = out
    d_noise = hip.DeviceBuffer.from_array(noise)
    d_lat = [hip.DeviceBuffer(ld * 4) for _ in range(frames)]
    d_eos = hip.DeviceBuffer(frames * 4)
    for f in range(frames):
        g.tts_step_async(0 if f == 0 else d_lat[f - 1].address, d_noise.address + f * ld * 4, 1, d_lat[f].address,
                         d_eos.address + f * 4, s_async)
    s_async.synchronize()
    eos = d_eos.to_array(np.float32, frames)
    for f in range(frames):
        assert np.array_equal(d_lat[f].to_array(np.float32, ld), want[f][0]), f
        assert eos[f] == want[f][1]


def test_tts_step_needs_a_flow_head():
    shape = W.tts_shape("tts-no-flow", 128, 1, 2, 256, latent=8)
    g = svl.Model(shape.config(0), W.make_weights(shape, "f32", seed=1))
    st = g.init_state(1, 16)
    with pytest.raises(svl.SvlError) as e:
        g.tts_step(None, np.zeros((1, 8), np.float32), st)
    assert e.value.code == svl.ERR_CONFIG
