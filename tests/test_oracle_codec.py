"""Pins the oracle's fp16 conversions and its restatement of MLX's affine codec.

The reference holds no stored affine-KV vectors (it calls MLX `quantize` as a
black box), so the codec is pinned by what the algorithm fixes: hand-derived
known answers on grid-aligned groups and on groups where MLX's scale refit
(scale = edge / q0) moves the stored scale, exact invariants (edge decodes
exactly, codes in range, constant groups), brute force (no other code is
nearer), a separate numpy restatement for the packing, and a count of the
exact .5 ties the tie rule decides on the config data. CPU only.
"""
import numpy as np
import pytest

from conftest import rng


# ----------------------------------------------------------------- fp16

def test_f16_to_f32_exhaustive(oracle_lib):
    o = oracle_lib
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ours = o.f16_to_f32(h.view(np.float16))
    ref = h.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(ours), nan)
    assert np.array_equal(ours[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_f32_to_f16_matches_numpy_rne(oracle_lib):
    o = oracle_lib
    r = rng(1)
    x = np.concatenate([
        r.standard_normal(200000).astype(np.float32) * 10.0,
        r.standard_normal(50000).astype(np.float32) * 1e-5,   # subnormal range
        np.array([65504, 65519.99, 65520, 65536, 1e9, -65520, 2.0**-24, 2.0**-25,
                  2.0**-25 * 1.0000001, 3 * 2.0**-26, 6.1035156e-05, 0.0, -0.0,
                  np.inf, -np.inf], np.float32),
    ])
    # all halfway points between consecutive fp16 values (ties)
    hs = np.arange(0, 0x7bff, dtype=np.uint16).view(np.float16).astype(np.float64)
    mids = ((hs[:-1] + hs[1:]) / 2).astype(np.float32)
    x = np.concatenate([x, mids, -mids])
    ours = o.f32_to_f16(x)
    ref = x.astype(np.float16)
    assert np.array_equal(ours.view(np.uint16), ref.view(np.uint16))


# ------------------------------------------------------- known answers

def _pack(codes, bits):
    codes = np.asarray(codes, np.uint64).reshape(-1, 32 // bits)
    sh = np.arange(32 // bits, dtype=np.uint64) * bits
    return (codes << sh).sum(axis=1).astype(np.uint32)


def _unpack(words, bits, n):
    words = np.asarray(words, np.uint64).reshape(-1, 1)
    sh = np.arange(32 // bits, dtype=np.uint64) * bits
    return ((words >> sh) & ((1 << bits) - 1)).reshape(-1)[:n].astype(np.int64)


@pytest.mark.parametrize("bits", [4, 8])
def test_known_answer_positive_edge(oracle_lib, bits):
    """Grid-aligned group whose larger-magnitude extreme is the max: the edge
    is the max, the scale is negative, code = n_bins - c, dequant is exact."""
    n_bins = (1 << bits) - 1
    step = 0.5 if bits == 4 else 0.25
    lo = -2.0 if bits == 4 else -10.0
    c = rng(bits).integers(0, n_bins + 1, 64)
    c[0], c[1] = 0, n_bins
    w = (lo + step * c).astype(np.float16)
    codes, s, b = oracle_lib.affine_quantize(w[None], bits)
    assert s[0, 0] == np.float16(-step) and b[0, 0] == np.float16(lo + step * n_bins)
    want = n_bins - c
    assert np.array_equal(_unpack(codes[0], bits, 64), want)
    assert np.array_equal(codes[0], _pack(want, bits))
    deq = oracle_lib.affine_dequantize(codes, s, b, bits)
    assert np.array_equal(deq[0], w)


@pytest.mark.parametrize("bits", [4, 8])
def test_known_answer_negative_edge(oracle_lib, bits):
    """Mirror case: |min| > |max| makes the min the edge, scale positive, code = c."""
    n_bins = (1 << bits) - 1
    step = 0.5 if bits == 4 else 0.25
    lo = -5.5 if bits == 4 else -60.0
    c = rng(10 + bits).integers(0, n_bins + 1, 64)
    c[5], c[9] = 0, n_bins
    w = (lo + step * c).astype(np.float16)
    codes, s, b = oracle_lib.affine_quantize(w[None], bits)
    assert s[0, 0] == np.float16(step) and b[0, 0] == np.float16(lo)
    assert np.array_equal(_unpack(codes[0], bits, 64), c)
    assert np.array_equal(oracle_lib.affine_dequantize(codes, s, b, bits)[0], w)


def test_known_answer_nibble_order(oracle_lib):
    """Codes are packed LSB-first: element k of a word sits in bits [4k, 4k+4)."""
    c = np.array(list(range(16)) * 4)
    w = (-5.5 + 0.5 * c).astype(np.float16)  # negative edge: code == c
    codes, _, _ = oracle_lib.affine_quantize(w[None], 4)
    assert codes[0, 0] == 0x76543210 and codes[0, 1] == 0xFEDCBA98


@pytest.mark.parametrize("bits", [4, 8])
def test_constant_and_zero_groups(oracle_lib, bits):
    for v in (0.0, 1.0, -3.25, 1000.0):
        w = np.full((1, 64), v, np.float16)
        codes, s, b = oracle_lib.affine_quantize(w, bits)
        assert np.all(codes == 0)
        assert b[0, 0] == np.float16(v)
        assert np.array_equal(oracle_lib.affine_dequantize(codes, s, b, bits), w)


def _codes_of(oracle_lib, vals, fill, bits):
    w = np.array(list(vals) + [fill[i % len(fill)] for i in range(64 - len(vals))], np.float16)
    codes, s, b = oracle_lib.affine_quantize(w[None], bits)
    return w, _unpack(codes[0], bits, 64), s[0, 0], b[0, 0]


# Hand-derived known answers on groups that are NOT grid-aligned, so MLX's
# refit `scale = edge / q0` (q0 = rint(edge / scale0)) moves the stored fp16
# scale away from f16((max - min) / n_bins). Each docstring carries the
# arithmetic; fp16 ulps: 2^-14 in [2^-4, 2^-3), 2^-13 in [2^-3, 2^-2),
# 2^-16 in [2^-6, 2^-5). The codes are chosen away from .5 ties except in the
# tie case, whose ties are exact.

def test_refit_known_answer_4bit_negative_edge(oracle_lib):
    """4-bit {-1.0, 0.3, 0, -0.5, 0.1, -0.25, fill 0 / -0.5}.
    f16(0.3) = 0.2998046875, f16(0.1) = 0.0999755859375. |min| > |max|: edge
    = -1.0, scale0 = 1.2998046875 / 15 = 0.0866536..., q0 = rint(-11.540) =
    -12, refit scale = -1 / -12 = 1/12, bias = -1. f16(1/12) = 1365 * 2^-14 =
    0.08331298828125 (without the refit: f16(0.0866536) = 0.086669921875).
    Codes (w + 1) * 12: -1 -> 0; 0.2998 -> 15.598 -> 16, clamped to 15;
    0 -> 12; -0.5 -> 6; 0.09998 -> 13.200 -> 13; -0.25 -> 9."""
    w, c, s, b = _codes_of(oracle_lib, [-1.0, 0.3, 0.0, -0.5, 0.1, -0.25], [0.0, -0.5], 4)
    assert s.view(np.uint16) == np.float16(0.08331298828125).view(np.uint16)
    assert b == np.float16(-1.0)
    assert c[:8].tolist() == [0, 15, 12, 6, 13, 9, 12, 6]
    # dequant of code 12 (the zero): 12 * 0.08331298828125 = 0.999755859375
    # = 2047.5 * 2^-11 is a tie in fp16 and rounds to even, 1.0; + (-1) = 0.
    # Code 13: 13 * s = 1.08306884765625 -> f16 1.0830078125 (2^-10 ulp),
    # - 1 = 0.0830078125.
    deq = oracle_lib.affine_dequantize(*oracle_lib.affine_quantize(w[None], 4), 4)[0]
    assert deq[2] == np.float16(0.0) and deq[4] == np.float16(0.0830078125)


def test_refit_known_answer_4bit_positive_edge(oracle_lib):
    """4-bit {2.0, -0.7, 0, 0.5, -0.5, 1.5, fill 0.5 / 1.5}. f16(0.7) =
    0.7001953125. |max| > |min|: edge = 2.0, scale0 = -2.7001953125 / 15 =
    -0.180013..., q0 = rint(-11.110) = -11, refit scale = 2 / -11 =
    -0.181818..., bias = 2. f16 = -(1489 * 2^-13) = -0.1817626953125 (without
    the refit: -(1475 * 2^-13) = -0.1800537109375). Codes (w - 2) / scale =
    (2 - w) * 5.5: 2 -> 0; -0.7002 -> 14.851 -> 15; 0 -> 11; 0.5 -> 8.25 -> 8;
    -0.5 -> 13.75 -> 14; 1.5 -> 2.75 -> 3."""
    _, c, s, b = _codes_of(oracle_lib, [2.0, -0.7, 0.0, 0.5, -0.5, 1.5], [0.5, 1.5], 4)
    assert s.view(np.uint16) == np.float16(-0.1817626953125).view(np.uint16)
    assert b == np.float16(2.0)
    assert c[:8].tolist() == [0, 15, 11, 8, 14, 3, 8, 3]


def test_refit_known_answer_8bit_negative_edge(oracle_lib):
    """8-bit {-3, 1, 0, 0.5, -2, fill 0 / 0.5}. edge = -3, scale0 = 4 / 255 =
    0.0156863, q0 = rint(-191.25) = -191, refit scale = 3 / 191 = 0.0157068,
    bias = -3. f16 = 1029 * 2^-16 = 0.0157012939453125 (without the refit:
    1028 * 2^-16 = 0.01568603515625). Codes (w + 3) * 191 / 3: -3 -> 0;
    1 -> 254.67 -> 255; 0 -> 191; 0.5 -> 222.83 -> 223; -2 -> 63.67 -> 64."""
    _, c, s, b = _codes_of(oracle_lib, [-3.0, 1.0, 0.0, 0.5, -2.0], [0.0, 0.5], 8)
    assert s.view(np.uint16) == np.float16(0.0157012939453125).view(np.uint16)
    assert b == np.float16(-3.0)
    assert c[:7].tolist() == [0, 255, 191, 223, 64, 191, 223]


def test_refit_known_answer_8bit_positive_edge(oracle_lib):
    """8-bit {5, -1.3, 0, 2.5, 1, -1, fill 0 / 2.5}. f16(1.3) = 1.2998046875.
    edge = 5, scale0 = -6.2998046875 / 255 = -0.0247051, q0 = rint(-202.39) =
    -202, refit scale = 5 / -202 = -0.0247525, bias = 5. f16 = -(1622 *
    2^-16) = -0.024749755859375 (without the refit: -(1619 * 2^-16) =
    -0.0247039794921875). Codes (5 - w) * 40.4: 5 -> 0; -1.2998 -> 254.51 ->
    255; 0 -> 202; 2.5 -> 101; 1 -> 161.6 -> 162; -1 -> 242.4 -> 242."""
    _, c, s, b = _codes_of(oracle_lib, [5.0, -1.3, 0.0, 2.5, 1.0, -1.0], [0.0, 2.5], 8)
    assert s.view(np.uint16) == np.float16(-0.024749755859375).view(np.uint16)
    assert b == np.float16(5.0)
    assert c[:8].tolist() == [0, 255, 202, 101, 162, 242, 202, 101]


def test_refit_known_answer_exact_ties(oracle_lib):
    """4-bit {-1, 0.8, -0.5625, -0.4375, ...}: f16(0.8) = 0.7998046875,
    scale0 = 1.7998046875 / 15 = 0.119987, q0 = rint(-8.334) = -8, refit
    scale = 1/8 exactly (without the refit f16(0.119987) = 0.1199951171875).
    (w + 1) * 8 is then exact: 0.7998 -> 14.398 -> 14 (15 without the refit);
    -0.5625 -> 3.5 and -0.4375 -> 4.5 are exact .5 ties, both rounding to the
    even code 4 (ties away from zero would give 4 and 5; without the refit
    they would be 3.646 -> 4 and 4.688 -> 5)."""
    _, c, s, b = _codes_of(oracle_lib, [-1.0, 0.8, -0.5625, -0.4375], [-0.5625, -0.4375], 4)
    assert s == np.float16(0.125) and b == np.float16(-1.0)
    assert c[:6].tolist() == [0, 14, 4, 4, 4, 4]


def _tie_count(w, bits):
    """Exact .5 ties of (w - bias) / scale in fp32 under the MLX formulas."""
    n_bins = np.float32((1 << bits) - 1)
    x = w.astype(np.float32).reshape(-1, 64)
    mx, mn = x.max(1), x.min(1)
    neg = np.abs(mn) > np.abs(mx)
    scale = np.maximum((mx - mn) / n_bins, np.float32(1e-7)).astype(np.float32)
    scale = np.where(neg, scale, -scale).astype(np.float32)
    edge = np.where(neg, mn, mx).astype(np.float32)
    q0 = np.rint(edge / scale).astype(np.float32)
    nz = q0 != 0
    scale = np.where(nz, edge / np.where(nz, q0, 1), scale).astype(np.float32)
    bias = np.where(nz, edge, 0).astype(np.float32)
    q = ((x - bias[:, None]) / scale[:, None]).astype(np.float32)
    tie = (q - np.floor(q)) == np.float32(0.5)
    return int(tie.sum()), tie, q


@pytest.mark.parametrize("case", ["c2", "c3"])
def test_tie_counts_on_config_data(oracle_lib, case):
    """Counts the exact .5 ties that the tie rule decides on the seeded
    config data (c2: K/V [4, 32769, 256] N(0,1) x per-head U(0.5, 2), 4-bit;
    c3: K/V [4, 18432, 256] N(0,1), 8-bit) and checks that the oracle gives
    each of them the even code. The counts are recorded so a change of the
    data or the formulas shows."""
    want = {"c2": (13361, 13271), "c3": (13168, 12940)}[case]
    r = np.random.default_rng(2 if case == "c2" else 3)
    T, bits = (32769, 4) if case == "c2" else (18432, 8)
    jit = r.uniform(0.5, 2.0, (4, 1, 1)) if case == "c2" else np.ones((4, 1, 1))
    got = []
    for _ in range(2):  # K, then V
        w = (r.standard_normal((4, T, 256)) * jit).astype(np.float16)
        n, tie, q = _tie_count(w, bits)
        got.append(n)
        rows = np.unique(np.nonzero(tie)[0])[:4000]  # groups holding a tie
        wg = w.reshape(-1, 64)[rows]
        codes, _, _ = oracle_lib.affine_quantize(wg, bits)
        c = _unpack(codes.reshape(-1), bits, wg.size).reshape(wg.shape)
        t = tie[rows]
        n_bins = (1 << bits) - 1
        want_c = np.clip(np.floor(q[rows]) + (np.floor(q[rows]) % 2 != 0), 0, n_bins)
        assert np.array_equal(c[t], want_c[t].astype(np.int64))
    assert tuple(got) == want, got
    """Exact .5 ties round to even (std::rint, MLX's CPU quantizer). Values
    0, 0.5, 1.5, 2.5, ..., 7.5 with the min as edge and scale 1: codes for the
    half-integers x.5 are the even neighbour."""
    vals = np.array([-8.0, 7.0] + [k + 0.5 - 8.0 for k in range(0, 15)] * 5, np.float32)[:64]
    w = vals.astype(np.float16)
    codes, s, b = oracle_lib.affine_quantize(w[None], 4)
    assert s[0, 0] == 1.0 and b[0, 0] == -8.0
    got = _unpack(codes[0], 4, 64)
    exact = vals + 8.0
    # explicit ties-to-even on the .5 values
    want = np.array([x if x % 1 == 0 else (np.floor(x) if np.floor(x) % 2 == 0 else np.ceil(x))
                     for x in exact])
    assert np.array_equal(got, want.astype(np.int64))


# ---------------------------------------------------------- invariants

@pytest.mark.parametrize("bits", [4, 8])
def test_invariants_and_brute_force(oracle_lib, bits):
    n_bins = (1 << bits) - 1
    r = rng(100 + bits)
    w = (r.standard_normal((512, 256)) * r.uniform(0.01, 4.0, (512, 1))
         + r.uniform(-2, 2, (512, 1))).astype(np.float16)
    codes, s, b = oracle_lib.affine_quantize(w, bits)
    deq = oracle_lib.affine_dequantize(codes, s, b, bits).astype(np.float64)
    c = _unpack(codes.reshape(-1), bits, w.size).reshape(w.shape)
    assert c.min() >= 0 and c.max() <= n_bins
    wg = w.astype(np.float64).reshape(512, 4, 64)
    sg = s.astype(np.float64)[..., None]
    bg = b.astype(np.float64)[..., None]
    cg = c.reshape(512, 4, 64)
    # edge: bias is the larger-magnitude extreme of the group and decodes exactly
    mx, mn = wg.max(-1), wg.min(-1)
    edge = np.where(np.abs(mn) > np.abs(mx), mn, mx)
    assert np.array_equal(bg[..., 0], edge)
    assert np.array_equal(deq.reshape(512, 4, 64)[cg == 0], np.broadcast_to(bg, cg.shape)[cg == 0])
    # scale sign is opposite to the edge's (code 0 is the edge, codes grow inward)
    nz = edge != 0
    assert np.all(np.sign(sg[..., 0][nz]) == -np.sign(edge[nz]))
    # |scale| = |edge / q0| with q0 = rint(edge / (range / n_bins)): within
    # a factor (k + 1/2) / k of range / n_bins, k = |q0|
    k = np.abs(np.rint(edge / (np.where(nz, (mx - mn) / n_bins, 1.0))))
    ratio = np.abs(sg[..., 0]) / np.maximum((mx - mn) / n_bins, 1e-30)
    ok = ~nz | (k == 0) | ((ratio <= (k + 0.5) / np.maximum(k, 1) * (1 + 2.0 ** -10)) &
                           (ratio >= (k - 0.5) / np.maximum(k, 1) * (1 - 2.0 ** -10)))
    assert np.all(ok)
    # brute force: no other code is nearer (up to the fp16 rounding of scale)
    grid = sg[..., None] * np.arange(n_bins + 1) + bg[..., None]  # [512,4,1,n_bins+1]
    d_all = np.abs(wg[..., None] - grid)
    d_own = np.take_along_axis(d_all, cg[..., None], axis=-1)[..., 0]
    slack = np.abs(sg) * n_bins * 2.0 ** -10 + 1e-7
    assert np.all(d_own <= d_all.min(-1) + slack)


def _numpy_quantize(w, bits):
    """Independent vectorized restatement, used only to cross-check packing and
    the C implementation's loops on random data."""
    n_bins = np.float32((1 << bits) - 1)
    x = w.astype(np.float32).reshape(-1, 64)
    mx, mn = x.max(1), x.min(1)
    neg = np.abs(mn) > np.abs(mx)
    scale = np.maximum((mx - mn) / n_bins, np.float32(1e-7)).astype(np.float32)
    scale = np.where(neg, scale, -scale).astype(np.float32)
    edge = np.where(neg, mn, mx).astype(np.float32)
    q0 = np.rint(edge / scale).astype(np.float32)
    nz = q0 != 0
    scale = np.where(nz, edge / np.where(nz, q0, 1), scale).astype(np.float32)
    bias = np.where(nz, edge, 0).astype(np.float32)
    c = np.clip(np.rint((x - bias[:, None]) / scale[:, None]), 0, n_bins).astype(np.uint64)
    epw = 32 // bits
    sh = np.arange(epw, dtype=np.uint64) * bits
    words = (c.reshape(-1, epw) << sh).sum(1).astype(np.uint32)
    rows = w.shape[0]
    return (words.reshape(rows, -1), scale.astype(np.float16).reshape(rows, -1),
            bias.astype(np.float16).reshape(rows, -1))


@pytest.mark.parametrize("bits", [4, 8])
def test_numpy_cross_check(oracle_lib, bits):
    r = rng(7 + bits)
    w = (r.standard_normal((300, 256)) * r.uniform(0.1, 3, (300, 1))).astype(np.float16)
    got = oracle_lib.affine_quantize(w, bits)
    want = _numpy_quantize(w, bits)
    for g_, w_ in zip(got, want):
        assert np.array_equal(np.asarray(g_).view(np.uint8), np.asarray(w_).view(np.uint8))


def test_dequantize_double_rounding(oracle_lib):
    """The composite dequant rounds code*scale to fp16 before adding the bias.
    code 255, scale 3.001953125 (fp16-exact): 255*s = 765.498046875 -> f16
    765.5; + 0.25 = 765.75 is a tie between 765.5 and 766.0 -> 766.0 (even).
    A single fused rounding of 765.748046875 would give 765.5."""
    codes = np.zeros((1, 64 * 8 // 32), np.uint32)
    codes[0, 0] = 255
    s = np.array([[3.001953125]], np.float16)
    b = np.array([[0.25]], np.float16)
    out = oracle_lib.affine_dequantize(codes, s, b, 8)
    assert out[0, 0] == np.float16(766.0)
    assert out[0, 1] == np.float16(0.25)


# ----------------------------------------------------------- Int8 per-token

def test_int8_reference_known_answer_round_trip(oracle_lib):
    """cache.rs:7480-7545 int8_kv_fetch_recovers_values_within_one_quant_step:
    the reference's own values (two real tokens and an all-zero token per side)
    come back within one step absmax/127 (x1.05, + 1e-3)."""
    k = np.array([[0.30, -1.20, 2.50, -0.80], [4.10, -3.30, 0.05, 1.90], [0, 0, 0, 0]],
                 np.float32)
    v = np.array([[-5.60, 0.90, 3.10, -2.20], [0.15, -0.45, 0.60, -0.30], [0, 0, 0, 0]],
                 np.float32)
    for orig in (k, v):
        x = orig.astype(np.float16)
        codes, scales = oracle_lib.int8_quantize(x)
        deq = oracle_lib.int8_dequantize(codes, scales).astype(np.float32)
        absmax = np.abs(orig).max(1, keepdims=True)
        tol = absmax / 127.0 * 1.05 + 1e-3
        assert (np.abs(orig - deq) <= tol).all()
        assert scales[2] == np.float16(1.0) and not codes[2].any()  # zero-token guard


def test_int8_hand_computed_known_answer(oracle_lib):
    """absmax 128: scale = f16(128/127 = 1.00787...) = 1.0078125 (1 + 8/1024).
    127/s = 126.0155 -> f16 126.0 -> 126; -128/s = -127.0077 -> f16 -127.0 ->
    -127 (the absmax element takes the extreme code); 63.5/s = 63.0078 -> f16
    63.0 -> 63; 0.25/s = 0.248 -> 0. A scale kept in fp32 would give 63/126
    differently only through the quotients' fp16 rounding, which this row
    fixes exactly."""
    x = np.zeros((1, 128), np.float16)
    x[0, :4] = [127.0, -128.0, 63.5, 0.25]
    codes, scales = oracle_lib.int8_quantize(x)
    assert scales[0] == np.float16(1.0078125)
    assert list(codes[0, :4]) == [126, -127, 63, 0] and not codes[0, 4:].any()
    deq = oracle_lib.int8_dequantize(codes, scales)
    assert deq[0, 0] == np.float16(126 * 1.0078125)  # 126.984375, exact in fp16


def test_int8_invariants_and_brute_force(oracle_lib):
    r = rng(808)
    x = (r.standard_normal((400, 256)) * r.uniform(0.01, 30, (400, 1))).astype(np.float16)
    x[7] = 0
    codes, scales = oracle_lib.int8_quantize(x)
    xf = x.astype(np.float64)
    s = scales.astype(np.float64)[:, None]
    absmax = np.abs(xf).max(1)
    # scale is the fp16 rounding of absmax / 127 (1 for the zero row)
    want_s = np.where(absmax == 0, 1.0, (absmax / 127.0).astype(np.float16).astype(np.float64))
    assert np.array_equal(s[:, 0], want_s)
    # the absmax element takes code +-127 (or 126/-128 at the fp16 edge)
    i = np.abs(xf).argmax(1)
    cm = np.abs(codes[np.arange(400), i].astype(int))
    assert (cm[absmax > 0] >= 126).all()
    # codes are the nearest integers to x / s up to the fp16 rounding of x / s
    q = xf / s
    c = codes.astype(np.float64)
    slack = 0.5 + np.abs(q) * 2.0 ** -11 + 1e-12
    inside = (q >= -128.5) & (q <= 127.5)
    assert (np.abs(c - q)[inside] <= slack[inside]).all()
    assert codes.min() >= -128 and codes.max() <= 127
    # dequantize is the fp16 product
    deq = oracle_lib.int8_dequantize(codes, scales)
    assert np.array_equal(deq, (c * s).astype(np.float16))
