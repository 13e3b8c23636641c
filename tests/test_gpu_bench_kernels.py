"""The measurement kernels bench.py prices the step's kernels against: libsvl's plain copy
(svl_bench_copy, the copy ceiling and the traffic counters' known-size reference) and its bare
streaming read (svl_bench_read, the per-launch read floor).  Their results are checked against
numpy on the host, so that a figure they give comes from kernels that moved every byte."""
import numpy as np
import pytest

import svl
from svl import hip

pytestmark = pytest.mark.gpu


def test_copy_moves_every_byte():
    L = svl.load_library()
    rng = np.random.default_rng(5)
    src = rng.integers(0, 2**32, size=4 * 100_003, dtype=np.uint32)
    d_src, d_dst = hip.DeviceBuffer.from_array(src), hip.DeviceBuffer(src.nbytes)
    svl._check(L.svl_bench_copy(0, d_src.address, d_dst.address, src.nbytes, None))
    hip.synchronize()
    assert np.array_equal(d_dst.to_array(np.uint32, src.size), src)


@pytest.mark.parametrize("pieces,blocks,threads", [(1000, 4, 64), (4 * 8 * 128 + 77, 8, 128), (3, 2, 64)])
def test_read_folds_every_piece(pieces, blocks, threads):
    """Piece i (16 bytes) is read by thread i mod (blocks x threads), through the four-deep loop
    and the tail loop; out[t] = xor over its pieces of their words 0 and 3."""
    L = svl.load_library()
    rng = np.random.default_rng(pieces)
    words = rng.integers(0, 2**32, size=(pieces, 4), dtype=np.uint32)
    nt = blocks * threads
    val = words[:, 0] ^ words[:, 3]
    want = np.bitwise_xor.reduce(np.concatenate([val, np.zeros(-pieces % nt, np.uint32)]).reshape(-1, nt), axis=0)
    d_src, d_out = hip.DeviceBuffer.from_array(words), hip.DeviceBuffer(nt * 4)
    svl._check(L.svl_bench_read(0, d_src.address, words.nbytes, blocks, threads, d_out.address, None))
    hip.synchronize()
    assert np.array_equal(d_out.to_array(np.uint32, nt), want)


def test_read_rejects_bad_grids():
    L = svl.load_library()
    d_src, d_out = hip.DeviceBuffer(1024), hip.DeviceBuffer(1024 * 4)
    for blocks, threads, nbytes in ((1, 100, 1024), (0, 64, 1024), (1, 2048, 1024), (1, 64, 1000)):
        assert L.svl_bench_read(0, d_src.address, nbytes, blocks, threads, d_out.address, None) != 0
