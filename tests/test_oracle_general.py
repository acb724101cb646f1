"""Pins oracle.sdpa_general, the restatement of the reference's general
attention options (layers::attention's mask and softcap, layers.rs:4010-4060;
causal_attention's sliding window, lib.rs:3185-3275; the softcap composite,
mlx_cxx_bridge.cpp:1573-1590; the float-mask cast, :3466-3497), CPU only.

Each check fixes a different part independently of the function's own code:
- no options / causal: the pinned C restatement of MLX's SDPA
  (qwo_sdpa_mlx_f16) on the same inputs;
- window: the C restatement run row by row on the window's keys only
  (what causal_attention's trailing-window slice does for one row);
- bool mask: the C restatement on each row's kept keys only, and the causal
  mask given as an array (an [L, T] orientation mistake fails it);
- additive mask: two-key known answers (softmax(a, b) weights), an additive
  0 / -inf mask equal to the bool mask, a large negative entry removing a key;
- softcap: closed forms of tanh capping (two keys at +-1000 capped at 5 give
  weights e^5, e^-5), the large-cap limit against the uncapped composite
  (within the fp16 budget), and the capped scores bounded by the cap.
"""
import numpy as np
import pytest

from conftest import rng


def _rand(r, hq, hkv, L, T, D):
    q = r.standard_normal((hq, L, D)).astype(np.float16)
    k = r.standard_normal((hkv, T, D)).astype(np.float16)
    v = r.standard_normal((hkv, T, D)).astype(np.float16)
    return q, k, v


def _close(a, b, tol):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    assert np.abs(a - b).max() <= tol, np.abs(a - b).max()


@pytest.mark.parametrize("causal", [False, True])
def test_no_options_is_the_mlx_sdpa_restatement(oracle_lib, causal):
    r = rng(41)
    q, k, v = _rand(r, 12, 2, 5, 300, 128)
    pos = oracle_lib.causal_positions(5, 300) if causal else None
    a = oracle_lib.sdpa_general(q, k, v, 1 / 16, causal=causal)
    b = oracle_lib.sdpa_mlx_f16(q, k, v, 1 / 16, pos)
    # the dot products accumulate in fp64 here, in fp32 in C, and the exp
    # differs in its last bits: equal except near fp16 rounding ties
    assert (a == b).mean() > 0.95
    _close(a, b, 2e-3)


@pytest.mark.parametrize("window", [1, 7, 64])
def test_window_is_the_sliced_keys(oracle_lib, window):
    r = rng(42 + window)
    hq, hkv, L, T, D = 6, 2, 4, 200, 64
    q, k, v = _rand(r, hq, hkv, L, T, D)
    got = oracle_lib.sdpa_general(q, k, v, 0.125, causal=True, window=window)
    for row in range(L):
        p = T - L + row
        lo = max(0, p - window + 1)
        want = oracle_lib.sdpa_mlx_f16(q[:, row:row + 1], k[:, lo:p + 1], v[:, lo:p + 1], 0.125)
        _close(got[:, row:row + 1], want, 2e-3)


def test_window_wider_than_the_context_is_causal(oracle_lib):
    r = rng(43)
    q, k, v = _rand(r, 4, 1, 3, 50, 64)
    a = oracle_lib.sdpa_general(q, k, v, 0.125, causal=True, window=500)
    b = oracle_lib.sdpa_general(q, k, v, 0.125, causal=True)
    np.testing.assert_array_equal(a, b)


def test_bool_mask_keeps_the_marked_keys(oracle_lib):
    r = rng(44)
    hq, hkv, L, T, D = 4, 2, 3, 120, 64
    q, k, v = _rand(r, hq, hkv, L, T, D)
    mask = r.random((L, T)) < 0.3
    mask[:, 5] = True
    got = oracle_lib.sdpa_general(q, k, v, 0.125, mask=mask)
    for row in range(L):
        keep = np.nonzero(mask[row])[0]
        want = oracle_lib.sdpa_mlx_f16(q[:, row:row + 1], k[:, keep], v[:, keep], 0.125)
        _close(got[:, row:row + 1], want, 2e-3)


def test_causal_mask_array_equals_causal_flag(oracle_lib):
    r = rng(45)
    L, T = 6, 40
    q, k, v = _rand(r, 4, 2, L, T, 64)
    causal = np.arange(T)[None, :] <= (T - L + np.arange(L))[:, None]
    a = oracle_lib.sdpa_general(q, k, v, 0.125, mask=causal)
    b = oracle_lib.sdpa_general(q, k, v, 0.125, causal=True)
    np.testing.assert_array_equal(a, b)
    # the transposed-orientation mistake would differ
    assert not np.array_equal(a, oracle_lib.sdpa_general(q, k, v, 0.125, mask=causal[::-1]))


def test_additive_zero_neg_inf_equals_bool(oracle_lib):
    r = rng(46)
    L, T = 4, 90
    q, k, v = _rand(r, 6, 2, L, T, 128)
    keep = r.random((6, L, T)) < 0.5
    keep[..., 0] = True
    add = np.where(keep, 0.0, -np.inf).astype(np.float32)
    a = oracle_lib.sdpa_general(q, k, v, 0.1, mask=add)
    b = oracle_lib.sdpa_general(q, k, v, 0.1, mask=keep)
    np.testing.assert_array_equal(a, b)
    # a large negative (finite) entry removes its key as well
    add2 = np.where(keep, 0.0, -60000.0).astype(np.float16)
    np.testing.assert_array_equal(oracle_lib.sdpa_general(q, k, v, 0.1, mask=add2), b)


@pytest.mark.parametrize("a_add,b_add", [(0.0, 0.0), (1.0, 0.0), (-2.0, 0.5), (3.25, -1.5)])
def test_additive_mask_two_key_known_answer(oracle_lib, a_add, b_add):
    # q = 0: every score is 0, so the weights are softmax(a_add, b_add)
    q = np.zeros((1, 1, 64), np.float16)
    k = np.ones((1, 2, 64), np.float16)
    v = np.zeros((1, 2, 64), np.float16)
    v[0, 0, :] = 1.0
    v[0, 1, :] = -1.0
    mask = np.array([[[a_add, b_add]]], np.float32)
    out = oracle_lib.sdpa_general(q, k, v, 0.125, mask=mask)
    w0 = np.exp(a_add) / (np.exp(a_add) + np.exp(b_add))
    # P is rounded to fp16 on this path, the output too
    want = np.float16(np.float16(w0) * 1.0 - np.float16(1 - w0) * 1.0)
    assert abs(float(out[0, 0, 0]) - float(want)) <= 2e-3


def test_softcap_two_key_closed_form(oracle_lib):
    # q . k0 = +1000, q . k1 = -1000 (exact in fp16), cap 5: scores +-5
    D = 64
    q = np.zeros((1, 1, D), np.float16)
    q[0, 0, 0] = 10.0
    k = np.zeros((1, 2, D), np.float16)
    k[0, 0, 0] = 100.0
    k[0, 1, 0] = -100.0
    v = np.zeros((1, 2, D), np.float16)
    v[0, 0, 1] = 1.0
    v[0, 1, 2] = 1.0
    out = oracle_lib.sdpa_general(q, k, v, 1.0, softcap=5.0).astype(np.float64)
    w0 = np.exp(5.0) / (np.exp(5.0) + np.exp(-5.0))
    assert abs(out[0, 0, 1] - w0) < 1e-3 and abs(out[0, 0, 2] - (1 - w0)) < 1e-4
    # uncapped, the second key's weight underflows entirely
    plain = oracle_lib.sdpa_general(q, k, v, 1.0).astype(np.float64)
    assert plain[0, 0, 2] == 0.0


def test_softcap_scale_enters_before_the_cap(oracle_lib):
    # S = 8, scale 0.25, cap 1: s = tanh(2) (the cap sees the scaled score)
    D = 64
    q = np.zeros((1, 1, D), np.float16)
    q[0, 0, 0] = 2.0
    k = np.zeros((1, 2, D), np.float16)
    k[0, 0, 0] = 4.0
    v = np.zeros((1, 2, D), np.float16)
    v[0, 0, 1] = 1.0
    v[0, 1, 2] = 1.0
    out = oracle_lib.sdpa_general(q, k, v, 0.25, softcap=1.0).astype(np.float64)
    s0 = np.tanh(2.0)
    w0 = np.exp(s0) / (np.exp(s0) + 1.0)
    assert abs(out[0, 0, 1] - w0) < 1e-3


def test_softcap_large_cap_is_the_uncapped_composite(oracle_lib):
    r = rng(47)
    q, k, v = _rand(r, 6, 2, 3, 150, 64)
    got = oracle_lib.sdpa_general(q, k, v, 0.125, causal=True, softcap=1e6)
    # the uncapped composite differs from MLX's SDPA only by where scale
    # enters (q pre-scaled and rounded there) and P's fp16 rounding
    want = oracle_lib.sdpa_mlx_f16(q, k, v, 0.125, oracle_lib.causal_positions(3, 150))
    _close(got, want, 4e-3)


def test_rows_without_a_visible_key_are_zero(oracle_lib):
    r = rng(48)
    q, k, v = _rand(r, 2, 1, 2, 30, 64)
    mask = np.ones((2, 30), bool)
    mask[1] = False
    out = oracle_lib.sdpa_general(q, k, v, 0.125, mask=mask)
    assert np.all(out[:, 1] == 0) and np.any(out[:, 0] != 0)
