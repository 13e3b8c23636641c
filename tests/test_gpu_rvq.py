"""GPU parity of Mimi's split residual vector quantizer, encoding (svl_rvq_*, restating
SVL/stt/model.rs:84-174) against the oracle (oracle/rvq.c).

Bar: bit-exact codes.  The GPU follows the oracle's products (the 16-lane dot of the reference's
matvec kernel, SVL/nn/kernels/mod.rs:66-91) and its argmin (the first index of the minimum), so
codes are equal on every input, ties and entry counts that are not a multiple of the GPU's
entry blocks included.
"""
import numpy as np
import pytest

import oracle
import svl
from svl import hip
from svl import workloads as W

pytestmark = pytest.mark.gpu


def _pair(n_q, bins, seed, dtype=W.F32):
    w = W.rvq_weights(n_q, bins, seed=seed)
    t = W.rvq_tensors(*w)
    if dtype == W.BF16:  # the GPU widens bf16 tensors; the oracle sees the widened values
        t = {name: (W.BF16, shp, W.to_bf16_bits(data)) for name, (_, shp, data) in t.items()}
        w = tuple(W.bf16_round(x) for x in w)
    return svl.Rvq(t, n_q, bins), oracle.Rvq(*w)


@pytest.mark.parametrize("n_q,bins", [(8, 256), (1, 100), (5, 130)])
def test_rvq_codes_match_oracle(n_q, bins):
    g, o = _pair(n_q, bins, seed=11)
    for b, t in [(1, 1), (1, 7), (3, 5), (2, 40)]:
        x = W.rvq_latents(b, t, seed=12 + b * 100 + t)
        got, want = g.encode(x), o.encode(x)
        assert np.array_equal(got, want), (b, t, np.argwhere(got != want)[:5])


def test_rvq_full_size_matches_oracle():
    """32 codebooks of 2048 entries: 64 streams of one frame and 2 streams of 9 frames."""
    oracle.set_threads(16)
    g, o = _pair(W.RVQ_NQ, W.RVQ_BINS, seed=13)
    for b, t in [(64, 1), (2, 9)]:
        x = W.rvq_latents(b, t, seed=14 + b)
        got, want = g.encode(x), o.encode(x)
        assert np.array_equal(got, want), (b, t, np.argwhere(got != want)[:5])


def test_rvq_closed_form_and_ties():
    """Latents equal to codebook entries give those entries; equal entries give the first."""
    n_q, bins = 6, 96
    w_first = np.zeros((256, 512), np.float32)
    w_first[np.arange(256), 256 + np.arange(256)] = 1.0
    w_rest = np.zeros((256, 512), np.float32)
    w_rest[np.arange(256), np.arange(256)] = 1.0
    _, _, sums, usage = W.rvq_weights(n_q, bins, seed=15)
    sums[1, 40] = sums[1, 17]
    usage[1, 40] = usage[1, 17]
    o = oracle.Rvq(w_first, w_rest, sums, usage)
    g = svl.Rvq(W.rvq_tensors(w_first, w_rest, sums, usage), n_q, bins)
    x = np.zeros((4, 512, 1), np.float32)
    for i, (j1, j2) in enumerate([(0, 0), (95, 40), (17, 17), (50, 3)]):
        x[i, 256:, 0] = o.codebook(0)[0][j1]
        x[i, :256, 0] = o.codebook(1)[0][j2]
    got = g.encode(x)
    assert np.array_equal(got, o.encode(x))
    assert [tuple(got[i, 0, :2]) for i in range(4)] == [(0, 0), (95, 17), (17, 17), (50, 3)]


def test_rvq_bf16_tensors_and_async_calls():
    g, o = _pair(4, 128, seed=16, dtype=W.BF16)
    x = W.rvq_latents(2, 6, seed=17)
    want = o.encode(x)
    assert np.array_equal(g.encode(x), want)
    d_x = hip.DeviceBuffer.from_array(x)
    d_c = hip.DeviceBuffer(want.nbytes)
    g.encode_async(2, 6, d_x.address, d_c.address)
    g.synchronize()
    assert np.array_equal(d_c.to_array(np.uint32, want.size).reshape(want.shape), want)
    # a larger call after a smaller one (work buffers grow), then the small one again
    x2 = W.rvq_latents(3, 50, seed=18)
    assert np.array_equal(g.encode(x2), o.encode(x2))
    assert np.array_equal(g.encode(x), want)


def test_rvq_input_errors():
    g, _ = _pair(2, 64, seed=19)
    with pytest.raises(ValueError):
        g.encode(np.zeros((1, 256, 1), np.float32))
    t = W.rvq_tensors(*W.rvq_weights(2, 64, seed=19))
    del t["rvq_rest.vq.layers.0._codebook.cluster_usage"]
    with pytest.raises(svl.SvlError) as e:
        svl.Rvq(t, 2, 64)
    assert e.value.code == svl.ERR_INVALID_INPUT
    assert g.encode(np.zeros((0, 512, 3), np.float32)).shape == (0, 3, 2)
