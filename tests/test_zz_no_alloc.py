"""The allocation-free recognize entry point (svl_stt_recognize_noalloc, include/svl.h) against
svl_stt_recognize, through the C ABI: the same tokens on consecutive calls, the second smaller
(the scratch keeps the previous call's contents), for one stream and a lockstep batch, and
sizes past the scratch rejected without touching the state."""
import ctypes as C

import numpy as np
import pytest

import svl
from svl import workloads as W

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 2 << 20


def _noalloc(model, state, audio):
    """audio [n, batch, n_q] -> tokens [n, batch] by svl_stt_recognize_noalloc."""
    L = svl.load_library()
    a = np.ascontiguousarray(audio, dtype=np.uint32)
    out = np.full((a.shape[0], state.batch), 0xFFFFFFFF, dtype=np.uint32)
    svl._check(L.svl_stt_recognize_noalloc(model.h, state.h, a.shape[0], a.ctypes.data_as(C.c_void_p),
                                           out.ctypes.data_as(C.c_void_p)))
    return out


@pytest.mark.parametrize("B", [1, 3])
def test_noalloc_recognize_equals_recognize_on_consecutive_calls(B):
    s = W.S1_SMALL
    g = svl.Model(s.config(W.Q8_0), W.make_weights(s, "q8_0", seed=61))
    audio = W.audio_tokens(s, 60, seed=62, batch=B).transpose(1, 0, 2).copy()  # [n, B, n_q]
    a, b = g.init_state(batch=B), g.init_state(batch=B)
    # first call 40 steps, then a smaller one that continues the streams
    assert np.array_equal(_noalloc(g, a, audio[:40]), g.recognize(audio[:40], b))
    assert np.array_equal(_noalloc(g, a, audio[40:47]), g.recognize(audio[40:47], b))
    assert np.array_equal(a.positions, b.positions)
    # a fresh state after a larger call: nothing of the previous call's scratch shows through
    c, d = g.init_state(batch=B), g.init_state(batch=B)
    assert np.array_equal(_noalloc(g, c, audio[50:55]), g.recognize(audio[50:55], d))


def test_noalloc_rejects_sizes_past_the_scratch():
    s = W.S1_SMALL
    g = svl.Model(s.config(W.Q8_0), W.make_weights(s, "q8_0", seed=63))
    st = g.init_state()
    n = SCRATCH_BYTES // (4 * (s.n_q + 1)) + 1
    audio = np.zeros((n, 1, s.n_q), dtype=np.uint32)
    with pytest.raises(svl.SvlError) as e:
        _noalloc(g, st, audio)
    assert e.value.code == svl.ERR_INVALID_INPUT
    assert st.positions[0] == 0
    ok = W.audio_tokens(s, 8, seed=64)[0][:, None, :]
    assert np.array_equal(_noalloc(g, st, ok), g.recognize(ok, g.init_state()))
