"""The step kernels' element functions on the GPU (svl_bench_activation) against the oracle on the
reference's own known-answer sweep (SVL/nn/kernels/activation.rs:89-122: 400k points over
[-100, 100) plus specials): exp, SiLU and GELU-tanh bit for bit (the FMA variant, the one the
reference selects on AVX2+FMA CPUs); the erf GELU within one float32 ulp of the oracle's (the GPU's
f64 erf is the device library's, the oracle's the C library's) and equal almost everywhere.
"""
import numpy as np
import pytest

import oracle
import svl

pytestmark = pytest.mark.gpu


def _points():
    xs = (-100.0 + np.arange(400_000, dtype=np.float32) * np.float32(5e-4)).astype(np.float32)
    specials = np.array([0.0, -0.0, 1e-30, -1e-30, -1e-7, 1e-3, -1e-3, 1e4, -1e4, np.inf, -np.inf, 88.7, 88.73,
                         -87.0, -87.5], dtype=np.float32)
    return np.concatenate([xs, specials])


def _bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def test_exp_silu_gelu_tanh_bit_exact():
    oracle.set_fma(True)
    x = _points()
    for kind, ref in ((0, lambda v: np.array([oracle.exp(t) for t in v], np.float32)),
                      (1, oracle.silu_n), (2, oracle.gelu_tanh_n)):
        got = svl.activation(kind, x)
        want = ref(x)
        same = (_bits(got) == _bits(want)) | (np.isnan(got) & np.isnan(want))
        assert same.all(), (kind, x[~same][:5], got[~same][:5], want[~same][:5])


def test_gelu_erf_within_one_ulp():
    x = _points()
    got = svl.activation(3, x)
    want = np.array([oracle.gelu_erf(t) for t in x], np.float32)
    fin = np.isfinite(want)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    ulp = np.abs(_bits(got)[fin].astype(np.int64) - _bits(want)[fin].astype(np.int64))
    assert ulp.max() <= 1 and np.mean(ulp == 0) > 0.9999, (ulp.max(), np.mean(ulp == 0))
    assert np.array_equal(got[~fin & ~np.isnan(want)], want[~fin & ~np.isnan(want)])
