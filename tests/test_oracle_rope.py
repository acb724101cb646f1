"""Pins the oracle's RoPE restatement (oracle.rope, following
crates/mlx-cpp/turbo/fused_rope_append.cpp:140-178) by what the mathematics
fixes, since MLX's fast::rope, the reference's parity target
(crates/mlxcel-core/src/fused_rope_parity_tests.rs:157-186), is not
available here:
  - position 0 is the identity, bit for bit;
  - pair 0 turns by exactly scale * position, and the sign convention is
    e1 -> (cos, sin), e2 -> (-sin, cos) (a counter-clockwise rotation);
  - pair p's frequency is base^(-p / (R/2)) (the textbook 1 / base^(2p/R));
  - each pair keeps its norm; rotations at a and b compose to a + b;
  - traditional and half-split layouts are the same rotation on permuted dims;
  - dims past rope_dims are copied (fused_rope_parity_tests.rs:274);
  - V is copied bit for bit (fused_rope_parity_tests.rs:330); layout 1 is
    layout 0 transposed (fused_rope_parity_tests.rs:302); token t turns at
    positions_base + t (fused_rope_parity_tests.rs:218).
A dropped minus sign, a swapped pair member, a wrong frequency exponent or a
position off by one fails one of these.
"""
import numpy as np

import oracle
from conftest import rng


def _x(r, shape):
    return r.standard_normal(shape).astype(np.float16)


def test_position_zero_is_identity():
    x = _x(rng(1), (3, 5, 128))
    for trad in (False, True):
        y = oracle.rope(x, 128, trad, 10000.0, 1.0, np.zeros(5))
        assert np.array_equal(y, x.astype(np.float64))


def test_pair0_angle_and_sign():
    D, R = 64, 64
    pos = np.array([0, 1, 7, 1000, 54321])
    for scale in (1.0, 0.25):
        for trad in (False, True):
            i1, i2 = oracle.rope_pairs(R, trad)
            e1 = np.zeros((len(pos), D))
            e1[:, i1[0]] = 1.0
            e2 = np.zeros((len(pos), D))
            e2[:, i2[0]] = 1.0
            th = (np.float32(scale) * pos.astype(np.float32)).astype(np.float64)
            y1 = oracle.rope(e1, R, trad, 10000.0, scale, pos)
            y2 = oracle.rope(e2, R, trad, 10000.0, scale, pos)
            np.testing.assert_allclose(y1[:, i1[0]], np.cos(th), atol=1e-12)
            np.testing.assert_allclose(y1[:, i2[0]], np.sin(th), atol=1e-12)
            np.testing.assert_allclose(y2[:, i1[0]], -np.sin(th), atol=1e-12)
            np.testing.assert_allclose(y2[:, i2[0]], np.cos(th), atol=1e-12)


def test_frequency_is_textbook_base_power():
    R, base = 128, 10000.0
    th = oracle.rope_theta(R, [1.0], base, 1.0)[0].astype(np.float64)
    p = np.arange(R // 2)
    np.testing.assert_allclose(th, base ** (-2.0 * p / R), rtol=2e-6)
    th5 = oracle.rope_theta(R, [1.0], 500000.0, 1.0)[0].astype(np.float64)
    np.testing.assert_allclose(th5, 500000.0 ** (-2.0 * p / R), rtol=2e-6)


def test_norm_preserved_and_composition():
    r = rng(2)
    R, D = 96, 128
    x = _x(r, (4, 9, D)).astype(np.float64)
    a = np.arange(9) * 3 + 5
    b = np.arange(9) * 2 + 11
    for trad in (False, True):
        i1, i2 = oracle.rope_pairs(R, trad)
        y = oracle.rope(x, R, trad, 10000.0, 1.0, a)
        np.testing.assert_allclose(y[..., i1] ** 2 + y[..., i2] ** 2,
                                   x[..., i1] ** 2 + x[..., i2] ** 2, rtol=1e-12, atol=1e-12)
        np.testing.assert_array_equal(y[..., R:], x[..., R:])
        yab = oracle.rope(y, R, trad, 10000.0, 1.0, b)
        ysum = oracle.rope(x, R, trad, 10000.0, 1.0, a + b)
        # fp32 angles: a few ulp of theta (<= ~60 rad here) apart
        np.testing.assert_allclose(yab, ysum, atol=1e-4)


def test_traditional_is_half_split_on_permuted_dims():
    r = rng(3)
    R, D = 64, 128
    x = _x(r, (2, 6, D)).astype(np.float64)
    pos = np.arange(6) + 100
    i1h, i2h = oracle.rope_pairs(R, False)
    i1t, i2t = oracle.rope_pairs(R, True)
    perm = np.arange(D)
    perm[i1t] = i1h
    perm[i2t] = i2h  # traditional dim j holds half-split dim perm[j]
    yt = oracle.rope(x[..., perm], R, True, 10000.0, 1.0, pos)
    yh = oracle.rope(x, R, False, 10000.0, 1.0, pos)
    np.testing.assert_array_equal(yt, yh[..., perm])


def test_fused_layouts_v_and_absolute_positions():
    r = rng(4)
    B, L, hq, hkv, D, R = 2, 5, 4, 2, 64, 32
    qkv = _x(r, (B, L, (hq + 2 * hkv) * D))
    q, k, v = oracle.fused_rope_qk_append(qkv, hq, hkv, D, R, 10000.0, 1.0, False, 37, 0)
    q1, k1, v1 = oracle.fused_rope_qk_append(qkv, hq, hkv, D, R, 10000.0, 1.0, False, 37, 1)
    x = qkv.reshape(B, L, hq + 2 * hkv, D)
    np.testing.assert_array_equal(v, x[:, :, hq + hkv:].transpose(0, 2, 1, 3))
    np.testing.assert_array_equal(k1, k.transpose(0, 2, 1, 3))
    np.testing.assert_array_equal(v1, v.transpose(0, 2, 1, 3))
    np.testing.assert_array_equal(q1, q)
    # token t alone at positions_base + t gives the same row
    for t in range(L):
        qt, kt, _ = oracle.fused_rope_qk_append(qkv[:, t:t + 1], hq, hkv, D, R, 10000.0, 1.0,
                                                False, 37 + t, 0)
        np.testing.assert_array_equal(qt[:, :, 0], q[:, :, t])
        np.testing.assert_array_equal(kt[:, :, 0], k[:, :, t])
