"""GPU parity of the Kyutai STT Mimi's encoder transformer (SVL/nn/mimi.rs:87-127 with the config of
SVL/stt/model.rs:60-70): the shared transformer with LayerNorm, layer scale, context 250 and the
erf-GELU feed-forward, against the oracle.

Bar: the f32 bar of the step contract, max-abs 1e-4.  The erf GELU is evaluated in f64 and rounded
(candle's f32 gelu_erf); the GPU's f64 erf (the device library's) and the oracle's (the C
library's) may differ in the last f64 bit, which changes the f32 result only within an f64 ulp of
an f32 rounding boundary, so the outputs are bit-equal almost everywhere.
"""
import os

import numpy as np
import pytest

import oracle
import svl
from svl import workloads as W

pytestmark = pytest.mark.gpu

TOL = 1e-4


def _run(shape, positions, chunk, seed):
    t = W.make_weights(shape, "f32", seed=seed)
    g, o = svl.Model(shape.config(0), t), oracle.Model(shape.config(0), t)
    xs = np.random.default_rng(seed + 1).standard_normal((1, positions, shape.d_model)).astype(np.float32)
    gs, os_ = g.init_state(), o.new_state()
    ys = np.concatenate([g.forward(xs[:, i:i + chunk], gs) for i in range(0, positions, chunk)], axis=1)
    yo = os_.forward(xs)
    return ys, yo


def test_small_erf_gelu_transformer_matches_oracle():
    s = W.Shape("erf-small", W.MODEL_TRANSFORMER, 128, 2, 2, 2, 64, W.FF_PLAIN_ERF, 256, W.NORM_LAYER, 1e-5, 7,
                layer_scale=1)
    ys, yo = _run(s, 30, 4, seed=21)
    assert np.max(np.abs(ys - yo)) <= TOL
    assert np.mean(ys.view(np.uint32) == yo.view(np.uint32)) > 0.999


def test_mimi_encoder_transformer_through_the_window():
    """The full encoder transformer over 300 SEANet frames (12 s of audio) in calls of 20 frames,
    past the 250-frame context."""
    oracle.set_threads(min(16, os.cpu_count() or 4))
    ys, yo = _run(W.MIMI_ENC, 300, 20, seed=22)
    assert np.max(np.abs(ys - yo)) <= TOL, float(np.max(np.abs(ys - yo)))
    assert np.mean(ys.view(np.uint32) == yo.view(np.uint32)) > 0.999
