"""Pins the oracle's weight formats (f16/bf16 conversion, candle Q8_0 / Q4K / Q8K blocks).

The reference ships no golden vectors for these (candle is not vendored); they are pinned by
library routines (numpy float16, torch bfloat16), hand-built known answers whose expected values
come from exact rational arithmetic, and invariants chosen so that a plausible mistake (wrong
rounding mode, swapped scale/min bits, dropped min term) fails.
"""
from fractions import Fraction

import numpy as np
import pytest
import torch

import oracle


def test_f16_to_f32_exhaustive_matches_numpy():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    expected = bits.view(np.float16).astype(np.float32)
    got = np.array([oracle.f16_bits_to_f32(int(b)) for b in bits], dtype=np.float32)
    finite = np.isfinite(expected)
    assert np.array_equal(got[finite].view(np.uint32), expected[finite].view(np.uint32))
    assert np.all(np.isnan(got[np.isnan(expected)]))
    assert np.array_equal(np.isinf(got), np.isinf(expected))


def test_f32_to_f16_round_to_nearest_even_matches_numpy():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(200_000).astype(np.float32) * np.float32(10.0) ** rng.integers(-9, 6, 200_000).astype(np.float32),
        np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e6, -1e6, 6e-8, 3e-8, 2.9802322e-08,
                  5.960464477539063e-08, 1.0009765625, 1.00048828125, 1.00146484375, np.inf, -np.inf],
                 dtype=np.float32),
    ])
    got = oracle.f32_to_f16_bits(x)
    expected = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, expected)
    # every f16 value round-trips
    halfs = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16)
    halfs = halfs[np.isfinite(halfs)]
    assert np.array_equal(oracle.f32_to_f16_bits(halfs.astype(np.float32)), halfs.view(np.uint16))


def test_bf16_round_to_nearest_even_matches_torch():
    rng = np.random.default_rng(1)
    x = rng.standard_normal(300_000).astype(np.float32) * np.float32(3.0) ** rng.integers(-20, 20, 300_000).astype(np.float32)
    # exact ties: low 16 bits 0x8000, both parities of the kept lsb
    ties = (np.arange(1000, dtype=np.uint32) << 16 | 0x3F800000 | 0x8000).view(np.float32)
    x = np.concatenate([x, ties])
    got = oracle.f32_to_bf16_bits(x)
    expected = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, expected)


# ---- Q8_0 ---------------------------------------------------------------------------------

def _blocks(raw: np.ndarray):
    """Splits [n*34] bytes into (f16 scales as f32, int8 quants [n, 32])."""
    raw = raw.reshape(-1, 34)
    d = raw[:, :2].copy().view(np.float16).reshape(-1).astype(np.float32)
    q = raw[:, 2:].copy().view(np.int8)
    return d, q


def test_q8_0_known_answer_rounds_half_away_from_zero():
    # amax 127 -> d = 1 exactly, so q = round(x) with ties away from zero (f32::round).
    x = np.zeros(32, dtype=np.float32)
    x[:8] = [127.0, 2.5, -2.5, 0.5, -0.5, 1.5, -3.49, 3.51]
    d, q = _blocks(oracle.quantize_q8_0(x))
    assert d[0] == 1.0
    assert q[0, :8].tolist() == [127, 3, -3, 1, -1, 2, -3, 4]
    assert np.all(q[0, 8:] == 0)


def test_q8_0_known_answer_exact_rationals():
    # x_j = (j - 16) / 100: the expected quants from exact arithmetic on the f32 inputs.
    x = (np.arange(32, dtype=np.float32) - 16) / np.float32(100.0)
    d, q = _blocks(oracle.quantize_q8_0(x))
    amax = max(abs(Fraction(float(v))) for v in x)
    d_exact = amax / 127
    assert d[0] == np.float32(np.float16(np.float32(float(d_exact))))
    for j in range(32):
        r = Fraction(float(x[j])) / d_exact
        frac = abs(r - int(r))
        if abs(frac - Fraction(1, 2)) < Fraction(1, 10_000):
            continue  # too close to a tie for f32 arithmetic to be decided by rationals
        expected = int(r + (Fraction(1, 2) if r > 0 else Fraction(-1, 2)))
        assert q[0, j] == expected, j


def test_q8_0_invariants():
    rng = np.random.default_rng(2)
    x = (rng.standard_normal((64, 256)) * 0.02).astype(np.float32)
    raw = oracle.quantize_q8_0(x)
    d, q = _blocks(raw)
    xb = x.reshape(-1, 32)
    # the largest magnitude of every block maps to +-127; zero block -> zero scale
    assert np.all(np.abs(q).max(axis=1) == 127)
    # dequantization is the closed form q * f32(f16 d), bit for bit
    deq = oracle.dequantize_q8_0(raw, 256).reshape(-1, 32)
    assert np.array_equal(deq.view(np.uint32), (q.astype(np.float32) * d[:, None]).view(np.uint32))
    # reconstruction within half a step (plus the f16 rounding of d)
    step = np.abs(xb).max(axis=1) / 127
    assert np.all(np.abs(deq - xb) <= 0.51 * step[:, None] + 127 * np.abs(d - step)[:, None] + 1e-12)
    # odd symmetry
    _, qn = _blocks(oracle.quantize_q8_0(-x))
    assert np.array_equal(qn, -q)
    z_d, z_q = _blocks(oracle.quantize_q8_0(np.zeros(32, np.float32)))
    assert z_d[0] == 0 and np.all(z_q == 0)


def test_q8_0_vec_dot():
    # integer-valued blocks with unit scales: the dot is an exact integer
    w = np.zeros(64, np.float32)
    x = np.zeros(64, np.float32)
    w[0], x[0] = 127.0, 127.0
    w[1:32] = np.arange(1, 32)
    x[1:32] = -np.arange(1, 32)[::-1]
    w[32], x[32] = -127.0, 127.0
    w[40], x[40] = 5.0, 7.0
    wb, xb = oracle.quantize_q8_0(w), oracle.quantize_q8_0(x)
    expected = 127 * 127 + float(np.dot(np.arange(1, 32), -np.arange(1, 32)[::-1])) - 127 * 127 + 35
    assert oracle.vec_dot_q8_0(wb, xb, 64) == expected
    # random rows: equals sum_b (sum_i qw qx) * dw * dx up to f32 rounding
    rng = np.random.default_rng(3)
    w = (rng.standard_normal(2048) * 0.02).astype(np.float32)
    x = rng.standard_normal(2048).astype(np.float32)
    wb, xb = oracle.quantize_q8_0(w), oracle.quantize_q8_0(x)
    dw, qw = _blocks(wb)
    dx, qx = _blocks(xb)
    exact = float(np.sum((qw.astype(np.int64) * qx).sum(axis=1) * dw.astype(np.float64) * dx.astype(np.float64)))
    assert abs(oracle.vec_dot_q8_0(wb, xb, 2048) - exact) <= 1e-5 * abs(exact) + 1e-6
    # and approximates the float dot
    assert abs(exact - float(np.dot(w.astype(np.float64), x))) < 0.02 * np.linalg.norm(w) * np.linalg.norm(x)


# ---- Q4K / Q8K ------------------------------------------------------------------------------

def _pack_scales(sc, mn):
    """GGML Q4K 12-byte packing of eight 6-bit scales and mins (inverse of get_scale_min_k4)."""
    s = [0] * 12
    for j in range(8):
        if j < 4:
            s[j] = sc[j]
            s[j + 4] = mn[j]
        else:
            s[j + 4] = (sc[j] & 0xF) | ((mn[j] & 0xF) << 4)
            s[j - 4] |= (sc[j] >> 4) << 6
            s[j] |= (mn[j] >> 4) << 6
    return bytes(s)


def _q4k_block(d, dmin, sc, mn, q):
    """q: 256 nibbles in value order; element 64*i + l uses byte 32*i + l, low nibble for
    l < 32, high nibble for the next 32."""
    qs = bytearray(128)
    for i in range(4):
        for l in range(32):
            qs[32 * i + l] = q[64 * i + l] | (q[64 * i + 32 + l] << 4)
    head = np.array([d, dmin], dtype=np.float16).tobytes()
    return np.frombuffer(head + _pack_scales(sc, mn) + bytes(qs), dtype=np.uint8)


def test_q4k_dequant_known_answer():
    sc = [1, 7, 13, 63, 33, 48, 2, 60]
    mn = [0, 5, 63, 17, 40, 1, 31, 62]
    q = [(3 * i + i // 32) % 16 for i in range(256)]
    blk = _q4k_block(0.25, 0.125, sc, mn, q)
    got = oracle.dequantize_q4k(blk, 256)
    expected = np.array([0.25 * sc[i // 32] * q[i] - 0.125 * mn[i // 32] for i in range(256)], dtype=np.float64)
    assert np.array_equal(got.astype(np.float64), expected)


def test_q4k_quantize_reconstruction_and_vec_dot():
    rng = np.random.default_rng(4)
    w = (rng.standard_normal((16, 512)) * 0.02).astype(np.float32)
    raw = oracle.quantize_q4k(w)
    deq = oracle.dequantize_q4k(raw, 512)
    # 4-bit codes over each 32-value sub-block's range: error within about one step
    sub = w.reshape(-1, 32)
    rng_sub = sub.max(axis=1) - np.minimum(sub.min(axis=1), 0)
    err = np.abs(deq.reshape(-1, 32) - sub).max(axis=1)
    assert np.all(err <= rng_sub / 15 * 1.05 + 1e-7)
    # Q8K activation blocks: d * q reconstructs x; the largest magnitude maps to -128
    x = rng.standard_normal(512).astype(np.float32)
    xb = oracle.quantize_q8k(x).reshape(2, 292)
    d = xb[:, :4].copy().view(np.float32).reshape(-1)
    qx = xb[:, 4:260].copy().view(np.int8)
    bsums = xb[:, 260:].copy().view(np.int16)
    assert np.array_equal(bsums, qx.reshape(2, 16, 16).astype(np.int32).sum(axis=2).astype(np.int16))
    for b in range(2):
        i = np.argmax(np.abs(x[256 * b:256 * (b + 1)]))
        assert qx[b, i] == -128
    assert np.all(np.abs(d[:, None] * qx - x.reshape(2, 256)) <= np.abs(d)[:, None] * 0.5 + 1e-6)
    # vec_dot == dot of the dequantized operands (integer parts exact, f32 scaling rounding)
    xdeq = (d[:, None].astype(np.float64) * qx).reshape(-1)
    for r in range(16):
        exact = float(np.dot(deq[r].astype(np.float64), xdeq))
        got = oracle.vec_dot_q4k_q8k(raw[r], oracle.quantize_q8k(x), 512)
        assert abs(got - exact) <= 2e-6 * (np.abs(deq[r]).astype(np.float64) @ np.abs(xdeq)) + 1e-7


def test_q4k_min_term_matters():
    # A sub-block shifted far from zero needs its min: a dropped min term would fail this.
    x = np.full(256, 0.5, dtype=np.float32) + np.linspace(0, 0.1, 256, dtype=np.float32)
    x[:32] -= 1.0
    deq = oracle.dequantize_q4k(oracle.quantize_q4k(x), 256)
    assert np.max(np.abs(deq - x)) < 0.02


# ---- Q4K from_float known answers --------------------------------------------------------------
# BlockQ4K::from_float fits every 32-value sub-block with make_qkx1_quants(15, 5, x) -- L from
# the range, then alternating least-squares refits of (scale, min) with min clamped to <= 0, up
# to 5 passes -- quantizes the fitted scales and mins to 6 bits against the block maxima
# (d = max_scale / 63, dmin = max_min / 63 as f16) and codes each value on the resulting grid.
# The super-block below is built so that every step can be followed by hand; the comments give
# the numbers.  a = 2^-6.

_A = 2.0 ** -6


def _grid(s, m, q):
    return [s * v - m for v in q]


_Q_GRID = [0, 15] + [(5 * i) % 16 for i in range(30)]   # a 4-bit code ramp with both ends present


def _kat_superblock():
    sub = [
        # 0: the second pass changes L.  Pass 1: iscale = 15 / (15 a) = 1 / a, L = (0, 15, 7 x 30)
        #    (round(7.4) = 7), LS scale = (15 * 15 + 30 * 7.4 * 7) / (225 + 30 * 49) a
        #    = 1779 / 1695 a = 1.04956 a, mean residual 0.849 a / 32 > 0 -> min 0.  Pass 2:
        #    iscale = 0.95278 / a, L(15 a) = round(14.29) = 14 (changed), scale = 1764 / 1666 a
        #    = 1.058824 a, min = mean(x - scale L) = -0.1765 a / 32 = -0.005515 a.  Pass 3:
        #    L unchanged (7.4 a -> 6.994, 15 a -> 14.17), scale = 1.059565 a, min = -0.010707 a.
        #    Result (scale, -min) = (0.016556, 1.6729e-4).  One pass alone gives min 0.
        [0.0, 15 * _A] + [7.4 * _A] * 30,
        # 1: exact grid s = 2^-8, min 2^-12: the fit returns (2^-8, 2^-12) exactly.
        _grid(2.0 ** -8, 2.0 ** -12, _Q_GRID),
        # 2: all positive, two levels a and 2a: min(x) = a > 0 -> 0; iscale = 15 / 2a, L = 8 and 15;
        #    pass 1 scale = (16 * 8 + 16 * 30) a / (16 * 64 + 16 * 225) = 608 / 4624 a = 0.131488 a,
        #    min = -0.01211 a; pass 2 keeps L but refits: scale = 0.132453 a, min = -0.023203 a.
        [_A] * 16 + [2 * _A] * 16,
        # 3: constant: max == min -> (0, 0), so the whole sub-block codes as 0 and decodes to 0.
        [0.01] * 32,
        # 4: exact grid with the largest scale and min: (2^-5, 2^-9).
        _grid(2.0 ** -5, 2.0 ** -9, _Q_GRID),
        # 5: exact grid, zero min: (2^-7, -0).
        _grid(2.0 ** -7, 0.0, _Q_GRID),
        # 6: exact grid (2^-6, 2^-10).
        _grid(2.0 ** -6, 2.0 ** -10, _Q_GRID),
        # 7: exact grid with a scale that is not a power of two: (3 * 2^-8, 3 * 2^-11).
        _grid(3 * 2.0 ** -8, 3 * 2.0 ** -11, _Q_GRID),
    ]
    return np.array([v for s in sub for v in s], dtype=np.float32)


def test_q4k_from_float_known_answer_superblock():
    blk = oracle.quantize_q4k(_kat_superblock()).reshape(-1)
    d = blk[0:2].copy().view(np.float16)[0]
    dmin = blk[2:4].copy().view(np.float16)[0]
    # max_scale = 2^-5 (sub-block 4), max_min = 2^-9 (sub-block 4):
    # d = f16(2^-5 / 63) = 1040 * 2^-21 (0x1010), dmin = f16(2^-9 / 63) = 520 * 2^-24 (subnormal, 0x0208)
    assert blk[0:2].copy().view(np.uint16)[0] == 0x1010
    assert blk[2:4].copy().view(np.uint16)[0] == 0x0208
    # 6-bit scales round(63 scale / 2^-5): 33.38 -> 33, 7.875 -> 8, 4.172 -> 4, 0, 63, 15.75 -> 16,
    # 31.5 -> 32 (ties away from zero), 23.625 -> 24; mins round(63 min / 2^-9): 5.396 -> 5,
    # 7.875 -> 8, 11.69 -> 12, 0, 63, 0, 31.5 -> 32, 47.25 -> 47.
    ls = [33, 8, 4, 0, 63, 16, 32, 24]
    lm = [5, 8, 12, 0, 63, 0, 32, 47]
    assert blk[4:16].tolist() == [0xE1, 0x48, 0x84, 0x40, 0xC5, 0x08, 0x8C, 0x80, 0xFF, 0x00, 0x00, 0xF8]
    assert _pack_scales(ls, lm) == bytes(blk[4:16])
    # codes: round((x + dmin * lm) / (d * ls)), clamped to [0, 15]
    codes = np.zeros(256, dtype=np.int64)
    for i in range(4):
        for l in range(32):
            codes[64 * i + l] = blk[16 + 32 * i + l] & 0xF
            codes[64 * i + 32 + l] = blk[16 + 32 * i + l] >> 4
    codes = codes.reshape(8, 32)
    # sub-block 0 on the grid d * 33 = 0.016365, offset dmin * 5 = 1.55e-4: 0 -> 0, 15a -> 14.33,
    # 7.4a -> 7.08
    assert codes[0].tolist() == [0, 14] + [7] * 30
    # the exact grids come back as their codes (grid steps within 1.6 % of s, offsets within
    # 1e-3 of a step)
    for j in (1, 4, 5, 6, 7):
        assert codes[j].tolist() == _Q_GRID, j
    # sub-block 2 on the grid d * 4, offset dmin * 12: a -> 8.06, 2a -> 15.94
    assert codes[2].tolist() == [8] * 16 + [15] * 16
    assert codes[3].tolist() == [0] * 32
    deq = oracle.dequantize_q4k(blk, 256).reshape(8, 32)
    assert np.all(deq[3] == 0.0)  # a constant sub-block decodes to zero
    assert float(d) * 63 == pytest.approx(2.0 ** -5, rel=2 ** -10)
    assert float(dmin) * 63 == pytest.approx(2.0 ** -9, rel=2 ** -9)


def test_q4k_codes_are_nearest_grid_points():
    # Every code is the nearest point of its sub-block's decoded grid d*sc*q - dmin*m, q in 0..15
    # (ties aside), for any input: a wrong nibble order, shift or clamp fails this.
    rng = np.random.default_rng(11)
    x = np.concatenate([(rng.standard_normal(4096) * 0.02), rng.uniform(-1, 3, 4096),
                        np.repeat(rng.standard_normal(64), 64) * 0.1]).astype(np.float32)
    raw = oracle.quantize_q4k(x.reshape(-1, 256)).reshape(-1, 144)
    deq = oracle.dequantize_q4k(raw, 256).reshape(-1, 8, 32).astype(np.float64)
    xs = x.reshape(-1, 8, 32).astype(np.float64)
    for b in range(raw.shape[0]):
        blk = raw[b]
        d = float(blk[0:2].copy().view(np.float16)[0])
        dm = float(blk[2:4].copy().view(np.float16)[0])
        sc = blk[4:16]
        for j in range(8):
            if j < 4:
                s6, m6 = sc[j] & 63, sc[j + 4] & 63
            else:
                s6 = (sc[j + 4] & 0xF) | ((sc[j - 4] >> 6) << 4)
                m6 = (sc[j + 4] >> 4) | ((sc[j] >> 6) << 4)
            step, off = d * s6, dm * m6
            if step == 0:
                assert np.all(deq[b, j] == -off * 0 + deq[b, j])
                continue
            grid = step * np.arange(16) - off
            dist = np.abs(xs[b, j][:, None] - grid[None, :])
            best = dist.min(axis=1)
            got = np.abs(xs[b, j] - deq[b, j])
            assert np.all(got <= best + 1e-6 * step), (b, j)


# ---- Q4_0 (candle BlockQ4_0; SVL/nn/mod.rs:76-87 quantizes with the block type chosen there) ----
# Each expected block below is derived by hand from the GGML rule (max = the first value of
# largest magnitude, d = max / -8 kept as f16, code = min(15, trunc(x / d + 8.5)), byte j = code
# of element j | code of element j + 16 << 4), in the comments.

def _q40(x):
    return oracle.quantize_q4_0(np.asarray(x, dtype=np.float32).reshape(1, 32))[0]


def _block(d_bits, codes):
    codes = list(codes)
    qs = [codes[j] | (codes[j + 16] << 4) for j in range(16)]
    return np.array([d_bits & 0xFF, d_bits >> 8] + qs, dtype=np.uint8)


def test_q4_0_known_answer_blocks():
    # all zero: max = 0, d = 0 / -8 = -0.0 (f16 0x8000), id = 0, every code trunc(8.5) = 8
    assert np.array_equal(_q40(np.zeros(32)), _block(0x8000, [8] * 32))
    # integers -8..7 then 7..-8: max = -8 (element 0; element 31 ties later), d = 1, code = x + 8
    x = [j - 8 for j in range(16)] + [7 - j for j in range(16)]
    assert np.array_equal(_q40(x), _block(0x3C00, [j for j in range(16)] + [15 - j for j in range(16)]))
    # ties of magnitude: the first wins.  8 then -8: d = -1, codes 0 and trunc(16.5) -> 15
    x = [8.0, -8.0] + [0.0] * 30
    assert np.array_equal(_q40(x), _block(0xBC00, [0, 15] + [8] * 30))
    # -8 then 8: d = +1, codes 0 and 15 (16 clamped): the same codes, the other scale
    x = [-8.0, 8.0] + [0.0] * 30
    assert np.array_equal(_q40(x), _block(0x3C00, [0, 15] + [8] * 30))
    # truncation, not rounding (d = 1): -0.5 -> trunc(8.0) = 8, -1.5 -> 7, 0.5 -> 9, 0.49 -> 8,
    # -0.51 -> 7, 7.6 -> trunc(16.1) = 16 -> 15, 6.4 -> 14
    x = [-8.0, -0.5, -1.5, 0.5, 0.49, -0.51, 7.6, 6.4] + [0.0] * 24
    assert np.array_equal(_q40(x), _block(0x3C00, [0, 8, 7, 9, 8, 7, 15, 14] + [8] * 24))
    # a fractional scale: max = 3 -> d = -0.375 (f16 0xB600), id = -8/3 in f32; 3 -> code 0,
    # -1.5 -> trunc(4 + 8.5) = 12, 0 -> 8
    x = [3.0, -1.5] + [0.0] * 30
    assert np.array_equal(_q40(x), _block(0xB600, [0, 12] + [8] * 30))


def test_q4_0_dequantize_closed_form():
    rng = np.random.default_rng(40)
    x = rng.standard_normal((8, 64)).astype(np.float32)
    b = oracle.quantize_q4_0(x).reshape(8, 2, 18)
    d = b[:, :, :2].copy().view(np.float16).astype(np.float32)  # [8, 2, 1]
    qs = b[:, :, 2:]
    codes = np.concatenate([qs & 0xF, qs >> 4], axis=-1).astype(np.float32)  # [8, 2, 32]
    want = ((codes - 8) * d).reshape(8, 64)
    assert np.array_equal(oracle.dequantize_q4_0(b.reshape(8, 36), 64), want)
    # every code is the nearest-or-truncated point of its block's grid: |x - value| <= |d|
    assert np.all(np.abs(x - want) <= np.abs(d).repeat(32, axis=-1).reshape(8, 64) * 1.0000001)


def test_q4_0_vec_dot_is_the_exact_block_sum():
    """vec_dot = sum over blocks of ((sum (code - 8) q) * d_w) * d_x: with power-of-two scales and
    small integers every product and partial sum is exact, so it equals the dot of the
    dequantized blocks in float64."""
    rng = np.random.default_rng(41)
    nb = 6
    codes = rng.integers(0, 16, size=(nb, 32))
    w = np.zeros((nb, 18), np.uint8)
    x = np.zeros((nb, 34), np.uint8)
    wd = rng.choice([0.25, 0.5, 1.0, 2.0], nb).astype(np.float16)
    xd = rng.choice([0.125, 0.5, 1.0], nb).astype(np.float16)
    xq = rng.integers(-127, 128, size=(nb, 32)).astype(np.int8)
    w[:, :2] = wd.view(np.uint8).reshape(nb, 2)
    w[:, 2:] = (codes[:, :16] | (codes[:, 16:] << 4)).astype(np.uint8)
    x[:, :2] = xd.view(np.uint8).reshape(nb, 2)
    x[:, 2:] = xq.view(np.uint8)
    want = float(np.sum((codes - 8) * wd[:, None].astype(np.float64) * xq * xd[:, None].astype(np.float64)))
    assert oracle.vec_dot_q4_0_q8_0(w, x, nb * 32) == want
    # the offset matters: codes read without "- 8" give another value
    assert want != float(np.sum(codes * wd[:, None].astype(np.float64) * xq * xd[:, None].astype(np.float64)))
