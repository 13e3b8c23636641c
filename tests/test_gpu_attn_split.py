"""GPU parity of the split attention launches: with few streams, each (stream, head) runs as up to
16 units that score a share of the keys, meet, and each form the whole softmax (max, exp, the sum
in key order, e / sum) and the key-order value chains of their share of the dims.

Bar: bit-exact -- the same bits as one unit per head (SVL_ATTN_SPLIT=0) and as the oracle.
SVL_ATTN_SPLIT=1 splits from two visible keys on (a split of S units once L >= S), so that short
reduced-shape runs pass through every split S = 2, 4, 8, 16, windows that wrap, batches whose
head count is and is not a multiple of 8 (the XCD-grouped and the plain unit order), f32 and bf16
caches and head dims 64 and 128 (the four piece layouts of the value columns).
"""
import numpy as np
import pytest

import oracle
import svl
from svl import workloads as W

pytestmark = pytest.mark.gpu

S_HD128 = W.stt_shape("stt-small-hd128", 512, 2, 4, 4.125, 24, card=64, n_q=4, text_card=100)


def _stt_logits(g, shape, B, n, seed):
    st = g.init_state(batch=B)
    audio = W.audio_tokens(shape, n, seed=seed, batch=B)
    text = np.full(B, shape.text_card, dtype=np.uint32)
    logits = []
    for i in range(n):
        tok, lg = g.step(text, audio[:, i], st, want_logits=True)
        logits.append(lg)
        text = tok.astype(np.uint32)
    return np.stack(logits)


@pytest.mark.parametrize("kv", [svl.F32, svl.BF16], ids=["f32kv", "bf16kv"])
@pytest.mark.parametrize("shape", [W.S1_SMALL, S_HD128], ids=["hd64", "hd128"])
def test_split_equals_unsplit_stt(monkeypatch, shape, kv):
    """STT logits over 40 steps through a window of 24, batches of 1, 2 (8 heads: grouped unit
    order) and 3 streams."""
    t = W.make_weights(shape, "q8_0", seed=61)
    for B in (1, 2, 3):
        results = []
        for split in ("0", "1"):
            monkeypatch.setenv("SVL_ATTN_SPLIT", split)
            g = svl.Model(shape.config(W.Q8_0), t, kv_dtype=kv)
            results.append(_stt_logits(g, shape, B, 40, seed=62 + B))
            del g
        assert np.array_equal(results[0].view(np.uint32), results[1].view(np.uint32)), B


@pytest.mark.parametrize("kv", [svl.F32, svl.BF16], ids=["f32kv", "bf16kv"])
def test_split_equals_unsplit_tts(monkeypatch, kv):
    """TTS backbone z over 12 steps after 20 pre-filled positions (unlimited context)."""
    shape = W.T1_SMALL
    t = W.make_weights(shape, "f32", seed=65)
    ks, vs = W.prefill_caches(shape, 20, seed=66)
    lat = W.latents(shape, 12, seed=67)
    results = []
    for split in ("0", "1"):
        monkeypatch.setenv("SVL_ATTN_SPLIT", split)
        g = svl.Model(shape.config(0), t, kv_dtype=kv)
        st = g.state_from_layer_caches(ks, vs, capacity=64)
        results.append(np.stack([g.backbone_step(lat[i][None], st) for i in range(12)]))
        del st, g
    assert np.array_equal(results[0].view(np.uint32), results[1].view(np.uint32))


def test_split_steps_match_oracle(monkeypatch):
    """f32 weights, batch 1: 40 split steps' logits equal the oracle's bits, tokens equal."""
    monkeypatch.setenv("SVL_ATTN_SPLIT", "1")
    s = W.S1_SMALL
    t = W.make_weights(s, "f32", seed=68)
    g, o = svl.Model(s.config(0), t), oracle.Model(s.config(0), t)
    gs, os_ = g.init_state(), o.new_state()
    audio = W.audio_tokens(s, 40, seed=69)[0]
    text = s.text_card
    for i in range(40):
        tg, lg = g.step([text], audio[i][None], gs, want_logits=True)
        to, lo = os_.stt_step(text, audio[i], want_logits=True)
        assert np.array_equal(lg[0].view(np.uint32), lo.view(np.uint32)), (i, float(np.max(np.abs(lg[0] - lo))))
        assert tg[0] == to, i
        text = int(to)


def test_split_recognize_and_state_calls(monkeypatch):
    """A split state through recognize, duplicate and reset: equal to the unsplit state's tokens."""
    s = W.S1_SMALL
    t = W.make_weights(s, "q8_0", seed=70)
    audio = W.audio_tokens(s, 30, seed=71)[0][:, None, :]
    got = []
    for split in ("0", "1"):
        monkeypatch.setenv("SVL_ATTN_SPLIT", split)
        g = svl.Model(s.config(W.Q8_0), t)
        st = g.init_state()
        a = g.recognize(audio[:20], st)
        c = st.duplicate()
        b = g.recognize(audio[20:], st)
        b2 = g.recognize(audio[20:], c)
        st.reset()
        r = g.recognize(audio, st)
        got.append((a, b, b2, r))
        del c, st, g
    for x, y in zip(got[0], got[1]):
        assert np.array_equal(x, y)
    assert np.array_equal(got[1][1], got[1][2])
