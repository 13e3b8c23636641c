"""The oracle's flow head and end-of-speech head (oracle/flow.c) against float64 brute force.

Reference: SVL/tts/flow_lm.rs:181-185 (out_eos, decode), 206-310 (FlowHead), 313-349
(TimestepEmbedder), 351-387 (ResBlock); SVL = crates/semantic-voice-local/src.  The float64
restatement below is written from those lines independently of the C code; each test also
checks that a plausible misreading (biased variance, swapped modulation chunks, a missing
`1 +` in modulate, the wrong time for an embedder) moves the result well outside the
tolerance, so the comparison can tell them apart.
"""
import numpy as np
import pytest

import oracle
from svl import workloads as W

SMALL = W.tts_shape("tts-flow-tiny", 64, 1, 2, 128, latent=8, flow_dim=32, flow_depth=2)


def _weights(shape, seed=5):
    return W.make_weights(shape, "f32", seed=seed)


def _t(ws, name):
    return ws[name][2].astype(np.float64)


def _silu(x):
    return x / (1.0 + np.exp(-x))


def _lin(ws, prefix, x):
    return _t(ws, prefix + ".weight") @ x + _t(ws, prefix + ".bias")


def np_time_embed(ws, i, t, ddof=1):
    p = f"flow_net.time_embed.{i}."
    args = _t(ws, p + "freqs") * t
    emb = np.concatenate([np.cos(args), np.sin(args)])
    e = _lin(ws, p + "mlp.2", _silu(_lin(ws, p + "mlp.0", emb)))
    return e / np.sqrt(e.var(ddof=ddof) + 1e-5) * _t(ws, p + "mlp.3.alpha")


def np_forward(ws, shape, cond, times, xs, swap=False, plus_one=True, ddof=1):
    D = shape.flow_dim
    y = _lin(ws, "flow_net.cond_embed", cond)
    if times:
        y = y + np.mean([np_time_embed(ws, i, t, ddof) for i, t in enumerate(times)], axis=0)
    sy = _silu(y)
    h = _lin(ws, "flow_net.input_proj", xs)

    def mod(x, shift, scale):
        if swap:
            shift, scale = scale, shift
        return x * ((1.0 if plus_one else 0.0) + scale) + shift

    for j in range(shape.flow_depth):
        r = f"flow_net.res_blocks.{j}."
        m = _lin(ws, r + "adaLN_modulation.1", sy)
        shift, scale, gate = m[:D], m[D:2 * D], m[2 * D:]
        hn = (h - h.mean()) / np.sqrt(h.var() + 1e-6) * _t(ws, r + "in_ln.weight") + _t(ws, r + "in_ln.bias")
        a = _silu(_lin(ws, r + "mlp.0", mod(hn, shift, scale)))
        h = h + gate * _lin(ws, r + "mlp.2", a)
    m = _lin(ws, "flow_net.final_layer.adaLN_modulation.1", sy)
    hn = (h - h.mean()) / np.sqrt(h.var() + 1e-6)
    return _lin(ws, "flow_net.final_layer.linear", mod(hn, m[:D], m[D:]))


def np_decode(ws, shape, cond, noise, steps, **kw):
    steps = max(steps, 1)
    x = noise.astype(np.float64)
    if shape.flow_kind == W.FLOW_LSD:
        for i in range(steps):
            x = x + np_forward(ws, shape, cond, [i / steps, (i + 1) / steps], x, **kw) / steps
        return x
    if shape.flow_kind == W.FLOW_MATCHING:
        for i in range(steps):
            x = x + np_forward(ws, shape, cond, [i / steps], x, **kw) / steps
        return x
    out = np_forward(ws, shape, cond, [], x, **kw)
    return out if shape.flow_kind == W.FLOW_DRIFTING else x + out


def _close(a, b, rtol=2e-5, atol=2e-6):
    return np.allclose(np.asarray(a, np.float64), b, rtol=rtol, atol=atol)


@pytest.fixture(scope="module")
def tiny():
    ws = _weights(SMALL)
    return ws, oracle.Model(SMALL.config(), ws)


def test_time_embedding_uses_the_unbiased_variance(tiny):
    ws, m = tiny
    for i, t in ((0, 0.0), (1, 1.0), (0, 0.25), (1, 0.75)):
        got = m.flow_time_embed(i, t)
        assert _close(got, np_time_embed(ws, i, t))
        assert not _close(got, np_time_embed(ws, i, t, ddof=0))
    # the conditioning of a flow step is the mean of the embedders' outputs
    tm = m.flow_time_mean([0.0, 1.0])
    assert _close(tm, (np_time_embed(ws, 0, 0.0) + np_time_embed(ws, 1, 1.0)) / 2)
    assert not _close(tm, (np_time_embed(ws, 0, 1.0) + np_time_embed(ws, 1, 0.0)) / 2)


def test_flow_forward_matches_float64(tiny):
    ws, m = tiny
    rng = np.random.default_rng(11)
    for _ in range(3):
        cond = rng.standard_normal(SMALL.d_model).astype(np.float32)
        xs = rng.standard_normal(SMALL.latent_dim).astype(np.float32)
        got = m.flow_forward(cond, [0.0, 1.0], xs)
        want = np_forward(ws, SMALL, cond, [0.0, 1.0], xs)
        assert _close(got, want), np.abs(got - want).max()
        assert not _close(got, np_forward(ws, SMALL, cond, [0.0, 1.0], xs, swap=True))
        assert not _close(got, np_forward(ws, SMALL, cond, [0.0, 1.0], xs, plus_one=False))


@pytest.mark.parametrize("kind", [W.FLOW_LSD, W.FLOW_MATCHING, W.FLOW_DRIFTING, W.FLOW_POINTWISE])
@pytest.mark.parametrize("steps", [1, 3])
def test_flow_decode_every_kind_matches_float64(kind, steps):
    shape = W.tts_shape("tts-flow-kind", 64, 1, 2, 128, latent=8, flow_dim=32, flow_depth=2, flow_kind=kind)
    ws = _weights(shape, seed=7)
    m = oracle.Model(shape.config(), ws)
    rng = np.random.default_rng(kind * 10 + steps)
    cond = rng.standard_normal(shape.d_model).astype(np.float32)
    noise = rng.standard_normal(shape.latent_dim).astype(np.float32)
    got = m.flow_decode(cond, noise, steps)
    want = np_decode(ws, shape, cond, noise, steps)
    assert _close(got, want), np.abs(got - want).max()


def test_decode_steps_below_one_count_as_one(tiny):
    _, m = tiny
    rng = np.random.default_rng(3)
    cond = rng.standard_normal(SMALL.d_model).astype(np.float32)
    noise = rng.standard_normal(SMALL.latent_dim).astype(np.float32)
    a = m.flow_decode(cond, noise, 1)
    assert np.array_equal(a, m.flow_decode(cond, noise, 0))
    assert np.array_equal(a, m.flow_decode(cond, noise, -2))


def test_eos_logit_is_the_out_eos_linear(tiny):
    ws, m = tiny
    z = np.random.default_rng(4).standard_normal(SMALL.d_model).astype(np.float32)
    want = float(_t(ws, "out_eos.weight")[0] @ z + _t(ws, "out_eos.bias")[0])
    assert abs(m.eos_logit(z) - want) < 1e-6


def test_tts_step_is_backbone_then_heads(tiny):
    """FlowLm::step = backbone z, out_eos(z), decode(z, noise): the full step equals its parts."""
    ws, m = tiny
    rng = np.random.default_rng(9)
    s1, s2 = m.new_state(), m.new_state()
    latent = None
    for step in range(4):
        noise = rng.standard_normal(SMALL.latent_dim).astype(np.float32)
        out, eos = s1.tts_full_step(latent, noise, decode_steps=2)
        z = s2.tts_step(latent)
        assert np.array_equal(out, m.flow_decode(z, noise, 2))
        assert eos == m.eos_logit(z)
        latent = out
