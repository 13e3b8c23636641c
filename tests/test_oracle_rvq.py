"""The oracle's restatement of Mimi's split residual vector quantizer (oracle/rvq.c, restating
SVL/stt/model.rs:84-174), pinned without the reference (which ships no quantizer vectors):
  * codebook preparation: exact on dyadic data, usages below 1e-5 clamped, IEEE division;
  * codes in closed form: latents equal to codebook entries give those entries (the first
    quantizer and the rest reading different projections of the same input), a zero residual
    then gives the entry of least half norm, ties give the first index;
  * a float64 brute force of the whole chain (argmin of half_norm - r.e, r -= e[code]) that the
    codes must follow up to float32 rounding.
"""
import numpy as np

import oracle
from svl import workloads as W


def _identity_projections():
    """proj_rest = x[:256], proj_first = x[256:] (exact 1x1 convolutions)."""
    w_rest = np.zeros((256, 512), np.float32)
    w_rest[np.arange(256), np.arange(256)] = 1.0
    w_first = np.zeros((256, 512), np.float32)
    w_first[np.arange(256), 256 + np.arange(256)] = 1.0
    return w_first, w_rest


def test_codebook_preparation_exact_and_clamped():
    rng = np.random.default_rng(1)
    n_q, bins = 3, 40
    sums = rng.integers(-8, 9, (n_q, bins, 256)).astype(np.float32)
    usage = np.full((n_q, bins), 2.0, np.float32)
    usage[1, :5] = [0.0, -1.0, 1e-7, 1e-5, 3.0]
    usage[2] = rng.uniform(0.3, 5.0, bins).astype(np.float32)
    q = oracle.Rvq(*_identity_projections(), sums, usage)
    for s in range(n_q):
        emb, hn = q.codebook(s)
        u = np.maximum(usage[s], np.float32(1e-5))
        assert np.array_equal(emb, sums[s] / u[:, None])  # one IEEE division per element
        if s == 0:  # dyadic: every square and partial sum exact
            exact = (emb.astype(np.float64) ** 2).sum(axis=1) / 2
            assert np.array_equal(hn.astype(np.float64), exact)
        else:
            ref = (emb.astype(np.float64) ** 2).sum(axis=1) / 2
            assert np.allclose(hn, ref, rtol=2e-6, atol=0)
    emb, _ = q.codebook(1)
    assert np.array_equal(emb[:3], sums[1, :3] / np.float32(1e-5))  # 0, -1 and 1e-7 clamp to 1e-5
    assert np.array_equal(emb[4], sums[1, 4] / np.float32(3.0))


def test_codes_closed_form():
    """x[256:] = an entry of the first codebook, x[:256] = an entry of the rest's first codebook:
    those entries are chosen; the rest's residual is then exactly zero, so its next codebook gives
    its entry of least half norm m, and the one after that the entry e minimizing hn(e) + e . e_m
    (the residual being -e_m)."""
    w_first, w_rest = _identity_projections()
    n_q, bins = 6, 96
    _, _, sums, usage = W.rvq_weights(n_q, bins, seed=3)
    q = oracle.Rvq(w_first, w_rest, sums, usage)
    cb = [q.codebook(s) for s in range(n_q)]
    for j1, j2 in [(0, 0), (17, 95), (95, 3), (40, 41)]:
        x = np.zeros((1, 512, 1), np.float32)
        x[0, 256:, 0] = cb[0][0][j1]
        x[0, :256, 0] = cb[1][0][j2]
        codes = q.encode(x)[0, 0]
        assert codes[0] == j1 and codes[1] == j2, (j1, j2, codes)
        m = int(np.argmin(cb[2][1]))
        assert codes[2] == m, codes
        sc3 = cb[3][1].astype(np.float64) + cb[3][0].astype(np.float64) @ cb[2][0][m].astype(np.float64)
        assert codes[3] == int(np.argmin(sc3)), codes


def test_ties_take_the_first_index():
    w_first, w_rest = _identity_projections()
    n_q, bins = 4, 64
    _, _, sums, usage = W.rvq_weights(n_q, bins, seed=4)
    sums[1, 9] = sums[1, 5]
    usage[1, 9] = usage[1, 5]
    # codebook 2 (which sees a zero residual): entries 7 and 3 equal and of least half norm
    sums[2, 7] = sums[2, 3] = 1e-3
    usage[2, 7] = usage[2, 3] = 1.0
    q = oracle.Rvq(w_first, w_rest, sums, usage)
    x = np.zeros((1, 512, 1), np.float32)
    x[0, :256, 0] = q.codebook(1)[0][9]
    codes = q.encode(x)[0, 0]
    assert codes[1] == 5 and codes[2] == 3, codes


def test_codes_follow_a_float64_chain():
    """Random weights and latents: at every stage the chosen entry's float64 score is within
    float32 rounding of the float64 minimum (and is the minimum almost always); the residual
    carried on is the float64 residual minus the chosen entry."""
    n_q, bins = 8, 256
    w_first, w_rest, sums, usage = W.rvq_weights(n_q, bins, seed=5)
    q = oracle.Rvq(w_first, w_rest, sums, usage)
    x = W.rvq_latents(3, 7, seed=6)
    codes = q.encode(x)
    cb = [(e.astype(np.float64), h.astype(np.float64)) for e, h in (q.codebook(s) for s in range(n_q))]
    exact, total = 0, 0
    for b in range(3):
        for t in range(7):
            xv = x[b, :, t].astype(np.float64)
            for part, stages in ((0, [0]), (1, list(range(1, n_q)))):
                r = (w_first if part == 0 else w_rest).astype(np.float64) @ xv
                for s in stages:
                    e, h = cb[s]
                    sc = h - e @ r
                    c = int(codes[b, t, s])
                    assert sc[c] - sc.min() <= 1e-3 * (1 + np.abs(sc).max()), (b, t, s)
                    exact += c == int(np.argmin(sc))
                    total += 1
                    r = r - e[c]
    assert exact >= total - 1, (exact, total)
