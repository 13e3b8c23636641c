"""Reduction-order identities the GPU kernels rely on for bit-exactness (CPU, numpy f32).

The reference's 16-lane dot ends with the pairwise tree a[i] = a[i] + a[i + w] for
w = 8, 4, 2, 1 (SVL/nn/kernels/mod.rs:66-91).  The kernels compute it with row rotations
(DPP row_ror) instead of lane exchanges: every lane adds its value to the value w lanes away
(mod 16).  Lane 0 then holds exactly the tree's result, because each addition sees the same two
operands as in the tree, possibly swapped, and f32 addition is commutative bit for bit.
"""
import numpy as np


def pairwise_tree(a):
    a = a.copy()
    for w in (8, 4, 2, 1):
        a[:w] = (a[:w] + a[w:2 * w]).astype(np.float32)
    return a[0]


def rotation_tree(a, direction):
    a = a.copy()
    for w in (8, 4, 2, 1):
        a = (a + np.roll(a, direction * w)).astype(np.float32)
    return a[0]


def test_rotations_reproduce_the_pairwise_lane_sum():
    rng = np.random.default_rng(11)
    vals = rng.standard_normal((20000, 16)) * 10.0 ** rng.uniform(-4, 4, (20000, 16))
    vals = vals.astype(np.float32)
    vals[::97] = np.float32(1e30) * np.sign(vals[::97])  # cancellations between huge values
    vals[::89, ::3] = np.float32(0.0)
    for direction in (1, -1):
        for row in vals:
            want = pairwise_tree(row)
            got = rotation_tree(row, direction)
            assert got.view(np.uint32) == want.view(np.uint32), (row, direction)


def test_a_plain_sequential_sum_is_not_the_tree():
    """The identity is not vacuous: summing lanes in order differs from the tree on some rows."""
    rng = np.random.default_rng(12)
    vals = (rng.standard_normal((2000, 16)) * 10.0 ** rng.uniform(-4, 4, (2000, 16))).astype(np.float32)
    differ = 0
    for row in vals:
        seq = np.float32(0)
        for v in row:
            seq = np.float32(seq + v)
        differ += int(seq.view(np.uint32) != pairwise_tree(row).view(np.uint32))
    assert differ > 0
