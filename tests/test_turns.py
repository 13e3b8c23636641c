"""The recognizer's word events and TurnDetector (SVL/stt/mod.rs:283-351, 564-590): the oracle's
restatement (oracle/turns.c) against the reference's own tests, and the GPU's on-device turn
signal (svl_stt_recognize_turns) against the oracle on the same token and probability stream."""
import numpy as np
import pytest

import oracle
from svl import workloads as W


def _activity(p):
    return [0.0, 0.0, p, 0.0]  # the reference test's event: pause probability at HEAD = 2


def test_reference_turns_end_after_words_only():
    """SVL/stt/mod.rs:636-646, the reference's test, restated."""
    d = oracle.TurnDetector()
    assert [d.activity(_activity(0.9)), d.activity(_activity(0.9))] == [False, False]
    got = [d.word(), d.activity(_activity(0.2)), d.activity(_activity(0.9)), d.activity(_activity(0.9))]
    assert got == [False, False, True, False]


def test_reference_turns_end_after_consecutive_frames():
    """SVL/stt/mod.rs:648-662, the reference's test, restated."""
    d = oracle.TurnDetector(threshold=0.6, frames=3)
    got = [d.word()] + [d.activity(_activity(p)) for p in (0.7, 0.7, 0.5, 0.7, 0.7, 0.7)]
    assert got == [False, False, False, False, False, False, True]


def test_word_events_follow_the_recognizer():
    """Recognizer::step (mod.rs:573-589): a padding token (0 or 3) after word tokens (> 3) emits
    words, which start a turn; tokens 1 and 2 and padding without pending tokens emit nothing;
    the step's VoiceActivity comes before its words."""
    d = oracle.TurnDetector()
    hi, lo = _activity(0.9), _activity(0.1)
    assert not d.step(3, hi)       # padding, no words pending: no turn yet
    assert not d.step(17, hi)      # a word token: pending, not emitted
    assert not d.step(1, hi)       # neither padding nor word: still pending
    assert not d.step(0, hi)       # end of padding: the words come after this step's activity
    assert d.step(3, hi)           # the next pause frame ends the turn
    assert not d.step(3, hi)       # ended; no new words
    assert not d.step(25, lo) and not d.step(3, hi)  # words emitted at the second step, after its activity
    assert d.step(0, hi)
    # frames.max(1) and a missing head (HEAD past the heads) never pause
    d0 = oracle.TurnDetector(frames=0)
    assert d0.t.frames == 1
    d5 = oracle.TurnDetector(head=5)
    d5.word()
    assert not any(d5.activity(_activity(0.99)) for _ in range(4))


@pytest.mark.gpu
def test_gpu_turn_signal_matches_oracle():
    import svl

    s = W.Shape(**{**W.S1_SMALL.__dict__, "extra_heads_num": 4, "extra_heads_dim": 6})
    t = W.make_weights(s, "q8_0", seed=70)
    # make the padding tokens frequent: rows 0 and 3 of text_linear scaled up
    w = t["text_linear.weight"][2].copy()
    w[[0, 3]] *= 3.0
    t["text_linear.weight"] = (t["text_linear.weight"][0], w.shape, w)
    g = svl.Model(s.config(W.Q8_0), t)
    o = oracle.Model(s.config(W.Q8_0), t)
    n = 96
    audio = W.audio_tokens(s, n, seed=71)[0]
    toks, probs = o.new_state().stt_greedy(audio, want_probs=True)
    assert np.sum((toks == 0) | (toks == 3)) >= 10 and np.sum(toks > 3) >= 10
    p2 = np.sort(probs[:, 2])
    for frames in (1, 2):
        # a threshold halfway between two probabilities near the median, away from every one
        k = len(p2) // 2
        threshold = float((p2[k - 1] + p2[k]) / 2)
        assert np.min(np.abs(probs[:, 2] - threshold)) > 1e-5
        det = oracle.TurnDetector(threshold=threshold, frames=frames)
        want = np.array([det.step(int(tk), pr) for tk, pr in zip(toks, probs)], dtype=np.int32)
        assert want.sum() >= 2
        st = g.init_state()
        # two calls: the recognizer's and the detector's state carry over
        a1, p1, e1 = g.recognize_turns(audio[:40, None, :], st, threshold=threshold, frames=frames)
        a2, _, e2 = g.recognize_turns(audio[40:, None, :], st, threshold=threshold, frames=frames)
        assert np.array_equal(np.concatenate([a1, a2])[:, 0], toks)
        assert np.allclose(p1[:, 0], probs[:40], atol=1e-6)
        assert np.array_equal(np.concatenate([e1, e2])[:, 0], want), (frames, np.flatnonzero(want))
        st.reset()
        _, _, e3 = g.recognize_turns(audio[:40, None, :], st, threshold=threshold, frames=frames)
        assert np.array_equal(e3[:, 0], want[:40])
