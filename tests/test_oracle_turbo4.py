"""Pins the Turbo4 codec tables and the oracle's Turbo4 restatement (CPU).

Golden vectors: tests/golden/turbo_codebooks_hex.json is the reference's own
fixture tests/fixtures/turbo_codebooks/codebooks_hex.json (sha256
48e69fdc...6d34b, checked below), the float32 bit patterns of the Lloyd-Max
centroids for bits 2..4 and d in {64, 80, 96, 128, 192, 256}, against which the
reference tests its codebook (crates/mlxcel-core/src/cache/turbo/
codebook.rs:659-690). Both the oracle's scipy restatement and the library's
own host build (qw_turbo4_codebook, a C++ restatement with libm erfc) must
reproduce every entry bit for bit.

The rest is pinned by what the mathematics fixes:
  - the sign LCG against its closed form x_n = a^n x_0 + c (a^n - 1)/(a - 1)
    (mod 2^32), computed by jump-ahead, and hand-computed first steps;
  - the Hadamard matrix: symmetric, orthonormal, constant first row, the
    Sylvester recursion;
  - quantize: the boundary count equals the brute-force nearest centroid;
    rescale * |centroids| = norm to fp16 rounding; V's fetch has the stored
    norm; the codec's round trip is as close as a 4-bit Lloyd-Max quantizer
    allows (and as the reference's own tests require, quant.rs:873-930);
  - the nibble layout (low nibble = even coordinate, quant.rs:30-33, :1237).
"""
import ctypes
import hashlib
import json
import os

import numpy as np
import pytest

import oracle
from conftest import GOLDEN, rng

FIXTURE = os.path.join(GOLDEN, "turbo_codebooks_hex.json")


def _fixture():
    data = open(FIXTURE, "rb").read()
    assert hashlib.sha256(data).hexdigest() == (
        "48e69fdcb5ea7e8f0a473e446b72f659bce75ae0ae67e47d47da01eee3e6d34b")
    return json.loads(data)


def _hex(c):
    return [format(int(x), "08x") for x in np.asarray(c, np.float32).view(np.uint32)]


@pytest.fixture(scope="module")
def qwlib():
    import qw_amd

    if not os.path.exists(qw_amd.LIB_PATH):
        from qw_amd import build

        build.build()
    return qw_amd


def test_oracle_codebook_matches_reference_fixture():
    for key, want in _fixture().items():
        bits, d = map(int, key.split("_"))
        assert _hex(oracle.turbo4_centroids(bits, d)) == want, key


def test_library_codebook_matches_reference_fixture(qwlib):
    """Host-only call: no device work."""
    for key, want in _fixture().items():
        bits, d = map(int, key.split("_"))
        assert _hex(qwlib.turbo4_codebook(bits, d)) == want, key
    # the 1-bit closed form +-sqrt(2 / (pi d))
    c1 = qwlib.turbo4_codebook(1, 128)
    np.testing.assert_array_equal(c1, np.float32([-np.sqrt(2 / (np.pi * 128)),
                                                  np.sqrt(2 / (np.pi * 128))]))
    # symmetry of the Lloyd-Max solution for a symmetric density
    c4 = qwlib.turbo4_codebook(4, 256).astype(np.float64)
    np.testing.assert_allclose(c4, -c4[::-1], atol=1e-9)


def _lcg_closed_form(seed, n):
    """State after n steps by jump-ahead: x_n = A x_0 + C with (A, C) built by
    squaring the affine map x -> a x + c."""
    a, c, M = 1664525, 1013904223, 1 << 32
    A, C = 1, 0
    ma, mc = a, c
    k = n
    while k:
        if k & 1:
            A, C = (ma * A) % M, (ma * C + mc) % M
        ma, mc = (ma * ma) % M, (ma * mc + mc) % M
        k >>= 1
    x0 = seed or 0xDEADBEEF
    return (A * x0 + C) % M


def test_signs_match_lcg_closed_form(qwlib):
    for seed in (1, 0, 0x7B470404, 0xFFFFFFFF, oracle.TURBO_DEFAULT_SEED + 0x4B5F5345):
        lib = qwlib.turbo4_signs(300, seed)
        ora = oracle.lcg_signs(300, seed)
        np.testing.assert_array_equal(lib, ora)
        for n in (1, 2, 17, 255, 300):
            want = 1.0 if _lcg_closed_form(seed & 0xFFFFFFFF, n) >> 31 else -1.0
            assert lib[n - 1] == want, (seed, n)
    # by hand: seed 1 -> 1664525 + 1013904223 = 1015568748 < 2^31 -> -1
    assert qwlib.turbo4_signs(1, 1)[0] == -1.0
    # seed 0 starts from 0xDEADBEEF
    np.testing.assert_array_equal(qwlib.turbo4_signs(64, 0), qwlib.turbo4_signs(64, 0xDEADBEEF))


def test_hadamard_is_orthonormal_sylvester():
    for n in (64, 128, 256):
        H = oracle.hadamard_orthonormal(n)
        np.testing.assert_allclose(H @ H, np.eye(n), atol=1e-12)
        np.testing.assert_array_equal(H, H.T)
        np.testing.assert_allclose(H[0], np.full(n, 1 / np.sqrt(n)))
        h = oracle.hadamard_orthonormal(n // 2)
        np.testing.assert_allclose(H, np.block([[h, h], [h, -h]]) / np.sqrt(2), atol=1e-15)


def test_quantize_nearest_centroid_and_rescale():
    r = rng(5)
    for D in (128, 256):
        tab = oracle.turbo4_tables(D)
        x = (r.standard_normal((3, 40, D)) * r.uniform(0.1, 4, (3, 40, 1))).astype(np.float16)
        for s1, s2 in ((tab["v_s1"], tab["v_s2"]), (tab["k_s1"], tab["k_s2"])):
            idx, norms, rescale, y = oracle.turbo4_quantize(x, s1, s2, tab)
            cb = tab["cb"].astype(np.float64)
            brute = np.abs(y[..., None] - cb).argmin(-1)
            np.testing.assert_array_equal(idx, brute)
            np.testing.assert_allclose(norms.astype(np.float64),
                                       np.linalg.norm(x.astype(np.float64), axis=-1),
                                       rtol=2 ** -11)
            c = cb[idx]
            np.testing.assert_allclose(rescale.astype(np.float64) * np.linalg.norm(c, axis=-1),
                                       norms.astype(np.float64), rtol=2 ** -10)
            # the rotation preserves the norm of the unit row
            np.testing.assert_allclose(np.linalg.norm(y, axis=-1), 1.0, atol=1e-9)


def test_round_trip_quality_and_v_norm():
    r = rng(6)
    D = 256
    tab = oracle.turbo4_tables(D)
    x = r.standard_normal((4, 64, D)).astype(np.float16)
    idx, norms, _, _ = oracle.turbo4_quantize(x, tab["v_s1"], tab["v_s2"], tab)
    v = oracle.turbo4_fetch_v(oracle.turbo4_pack(idx), norms, tab).astype(np.float64)
    xf = x.astype(np.float64)
    cos = (v * xf).sum(-1) / (np.linalg.norm(v, axis=-1) * np.linalg.norm(xf, axis=-1))
    # 4-bit Lloyd-Max on N(0, 1/d): relative MSE ~0.0095, cos ~ 0.995
    assert cos.min() > 0.99, cos.min()
    np.testing.assert_allclose(np.linalg.norm(v, axis=-1), norms.astype(np.float64),
                               rtol=2e-3)
    idk, _, rk, _ = oracle.turbo4_quantize(x, tab["k_s1"], tab["k_s2"], tab)
    k = oracle.turbo4_fetch_k(oracle.turbo4_pack(idk), rk, tab).astype(np.float64)
    rel = np.linalg.norm(k - xf, axis=-1) / np.linalg.norm(xf, axis=-1)
    assert rel.max() < 0.15, rel.max()  # the reference's own bound (quant.rs:873-930)
    # K and V use independent rotations: different indices for the same rows
    assert (idk != idx).mean() > 0.5


def test_nibble_layout():
    idx = np.array([[1, 2, 15, 0, 7, 8]], np.uint8)
    packed = oracle.turbo4_pack(idx)
    np.testing.assert_array_equal(packed, [[0x21, 0x0F, 0x87]])
    np.testing.assert_array_equal(oracle.turbo4_unpack(packed), idx)


def test_expand_rotated_is_fp32_product_then_fp16():
    tab = oracle.turbo4_tables(128)
    packed = oracle.turbo4_pack(np.arange(16, dtype=np.uint8).repeat(8)[None])
    r = np.float16(0.7109375)
    got = oracle.turbo4_expand_rotated(packed, np.array([r]), tab)[0]
    want = np.array([np.float16(np.float32(c) * np.float32(r)) for c in tab["cb"]]).repeat(8)
    np.testing.assert_array_equal(got, want)


def _fused_case(seed, hkv=2, G=3, L=3, T=300, D=128):
    r = rng(seed)
    tab = oracle.turbo4_tables(D)
    k = r.standard_normal((hkv, T, D))
    v = r.standard_normal((hkv, T, D))
    ki, _, kr, _ = oracle.turbo4_quantize(k, tab["k_s1"], tab["k_s2"], tab)
    vi, _, vr, _ = oracle.turbo4_quantize(v, tab["v_s1"], tab["v_s2"], tab)
    q = r.standard_normal((hkv * G, L, D)).astype(np.float16)
    return q, oracle.turbo4_pack(ki), kr, oracle.turbo4_pack(vi), vr, tab


def test_fused_verify_zero_query_is_the_visible_value_mean():
    """q = 0 makes every visible score 0: each row's output is the plain mean of
    the V expansions it sees (rows see t <= pos), rotated back -- a closed form
    that fixes the causal cut and the V rotation."""
    q, kp, kr, vp, vr, tab = _fused_case(3)
    q[:] = 0
    hq, L, D = q.shape
    T = kp.shape[1]
    pos = oracle.causal_positions(L, T)
    out = oracle.turbo4_fused_verify(q, kp, kr, vp, vr, tab, 1.0 / 16, pos).astype(np.float64)
    v = oracle.turbo4_expand_rotated(vp, vr, tab).astype(np.float64)
    G = hq // kp.shape[0]
    for h in range(hq):
        for r_ in range(L):
            mean = v[h // G, : pos[r_] + 1].mean(0)
            want = oracle.turbo4_rotate(mean, tab["v_s2"], tab["v_s1"])
            np.testing.assert_allclose(out[h, r_], want, atol=2e-3, rtol=2e-3)


def test_fused_verify_agrees_with_the_dequantize_route():
    """The fused pass (fp32 scores, log2 domain) and the dequantize-then-SDPA
    route (fp16 scores) compute the same attention up to their roundings: a
    dropped log2(e), a wrong scale or a transposed rotation would move the
    outputs by far more than this bound."""
    q, kp, kr, vp, vr, tab = _fused_case(4)
    hq, L, D = q.shape
    T = kp.shape[1]
    pos = oracle.causal_positions(L, T)
    fused = oracle.turbo4_fused_verify(q, kp, kr, vp, vr, tab, 1.0 / 16, pos).astype(np.float64)
    route = oracle.turbo4_attention(q, kp, kr, vp, vr, tab, 1.0 / 16, pos).astype(np.float64)
    err = np.abs(fused - route).max()
    assert err < 1e-2, err
    wrong = oracle.turbo4_fused_verify(q, kp, kr, vp, vr, tab, 1.0 / 16 / 1.4426950408889634,
                                       pos).astype(np.float64)
    assert np.abs(wrong - route).max() > 3 * err
