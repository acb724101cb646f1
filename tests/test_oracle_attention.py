"""Pins the oracle's attention functions (CPU only).

- qwo_sdpa_f64 against an independent numpy fp64 softmax attention.
- qwo_sdpa_mlx_f16 (MLX CPU-stream roundings) against fp64 within the fp16
  budget, and on known answers (one key, equal keys, one-hot softmax).
- qwo_dlsa_attention against the reference's golden fixtures
  (tests/golden/dlsa_*.safetensors, extracted from the reference's
  tests/fixtures/dlsa), the identity "a full-coverage list equals dense causal
  attention" (reference gpu_attend_tests.rs:260), list-order invariance and the
  skip/empty-row rules of the K2 contract (dlsa_attention.rs:1-14).
"""
import os

import numpy as np
import pytest
from safetensors.numpy import load_file

from conftest import GOLDEN, rng


def _np_attention(q, k, v, scale, pos=None):
    q, k, v = (x.astype(np.float64) for x in (q, k, v))
    hq, L, D = q.shape
    hkv = k.shape[0]
    G = hq // hkv
    out = np.empty((hq, L, D))
    for h in range(hq):
        s = q[h] @ k[h // G].T * scale
        if pos is not None:
            s = np.where(np.arange(k.shape[1])[None, :] > pos[:, None], -np.inf, s)
        s = s - s.max(1, keepdims=True)
        p = np.exp(s)
        p /= p.sum(1, keepdims=True)
        out[h] = p @ v[h // G]
    return out


@pytest.mark.parametrize("causal", [False, True])
def test_sdpa_f64_matches_numpy(oracle_lib, causal):
    r = rng(3)
    q = r.standard_normal((12, 5, 64)).astype(np.float16)
    k = r.standard_normal((2, 40, 64)).astype(np.float16)
    v = r.standard_normal((2, 40, 64)).astype(np.float16)
    pos = oracle_lib.causal_positions(5, 40) if causal else None
    got = oracle_lib.sdpa_f64(q, k, v, 0.125, q_pos=pos)
    assert np.abs(got - _np_attention(q, k, v, 0.125, pos)).max() < 1e-12


@pytest.mark.parametrize("T,L,causal", [(300, 1, False), (1000, 4, True), (4096, 1, False)])
def test_sdpa_mlx_f16_within_fp16_budget(oracle_lib, T, L, causal):
    r = rng(T)
    q = r.standard_normal((24, L, 256)).astype(np.float16)
    k = r.standard_normal((4, T, 256)).astype(np.float16)
    v = r.standard_normal((4, T, 256)).astype(np.float16)
    pos = oracle_lib.causal_positions(L, T) if causal else None
    o16 = oracle_lib.sdpa_mlx_f16(q, k, v, 1 / 16, q_pos=pos).astype(np.float64)
    o64 = oracle_lib.sdpa_f64(q, k, v, 1 / 16, q_pos=pos)
    err = o16 - o64
    assert np.abs(err).max() < 2e-3
    assert np.linalg.norm(err) / np.linalg.norm(o64) < 2e-3
    # ... and it is not exact: the fp16 roundings are really there
    assert np.abs(err).max() > 0


def test_sdpa_mlx_known_answers(oracle_lib):
    r = rng(5)
    D = 64
    v = r.standard_normal((1, 3, D)).astype(np.float16)
    q = r.standard_normal((2, 1, D)).astype(np.float16)
    # one key: softmax is exactly 1, the output is that value row
    k1 = r.standard_normal((1, 1, D)).astype(np.float16)
    out = oracle_lib.sdpa_mlx_f16(q, k1, v[:, :1], 0.125)
    assert np.array_equal(out[0, 0], v[0, 0]) and np.array_equal(out[1, 0], v[0, 0])
    # equal keys: uniform weights, the output is the mean of the values
    keq = np.repeat(k1, 3, axis=1)
    out = oracle_lib.sdpa_mlx_f16(q, keq, v, 0.125).astype(np.float64)
    assert np.abs(out[0, 0] - v[0].astype(np.float64).mean(0)).max() < 4e-3
    # one-hot: a key aligned with q by a huge margin takes all the weight
    qh = np.zeros((1, 1, D), np.float16)
    qh[0, 0, 0] = 8.0
    kh = np.zeros((1, 3, D), np.float16)
    kh[0, 1, 0] = 8.0  # score 64 * scale 1 vs 0
    out = oracle_lib.sdpa_mlx_f16(qh, kh, v, 1.0)
    assert np.array_equal(out[0, 0], v[0, 1])


def test_sdpa_mlx_causal_rows_match_prefix_attention(oracle_lib):
    """Bottom-right causal row r equals unmasked attention over keys [0, T-L+r]."""
    r = rng(9)
    q = r.standard_normal((6, 3, 64)).astype(np.float16)
    k = r.standard_normal((1, 20, 64)).astype(np.float16)
    v = r.standard_normal((1, 20, 64)).astype(np.float16)
    full = oracle_lib.sdpa_mlx_f16(q, k, v, 0.125, q_pos=oracle_lib.causal_positions(3, 20))
    for row in range(3):
        n = 20 - 3 + row + 1
        one = oracle_lib.sdpa_mlx_f16(q[:, row:row + 1], k[:, :n], v[:, :n], 0.125)
        assert np.array_equal(full[:, row], one[:, 0])


# ---------------------------------------------------------------- D-LSA

def _golden(case):
    return load_file(os.path.join(GOLDEN, f"dlsa_{case}.safetensors"))


@pytest.mark.parametrize("m", ["real", "random"])
def test_dlsa_qwen_layer_golden(oracle_lib, m):
    d = _golden("qwen_layer")
    q = d["q_rows"].transpose(1, 0, 2)      # [Hq, R, D]
    k = d["k"].transpose(1, 0, 2)           # strided [Hkv, T, D]
    v = d["v"].transpose(1, 0, 2)
    out = oracle_lib.dlsa_attention(q, k, v, d[f"{m}.selected"], d[f"{m}.selected_lengths"],
                                    256 ** -0.5)
    ref = d[f"{m}.attention_out"].transpose(1, 0, 2)
    assert np.abs(out - ref).max() < 1e-5


@pytest.mark.parametrize("case", ["tiny", "short_dense"])
def test_dlsa_tiny_golden_and_dense(oracle_lib, case):
    d = _golden(case)
    q = d["q"].transpose(1, 0, 2)
    k = d["k"].transpose(1, 0, 2)
    v = d["v"].transpose(1, 0, 2)
    T = k.shape[1]
    out = oracle_lib.dlsa_attention(q, k, v, d["selected"], d["selected_lengths"], 16 ** -0.5)
    assert np.abs(out - d["attention_out"].transpose(1, 0, 2)).max() < 1e-5
    dense = oracle_lib.sdpa_f64(q, k, v, 16 ** -0.5, q_pos=np.arange(T, dtype=np.int32))
    assert np.abs(dense - d["dense_out"].transpose(1, 0, 2)).max() < 1e-5


def test_dlsa_full_list_equals_dense_causal(oracle_lib):
    r = rng(11)
    T, D = 70, 64
    q = r.standard_normal((8, T, D)).astype(np.float16)
    k = r.standard_normal((2, T, D)).astype(np.float16)
    v = r.standard_normal((2, T, D)).astype(np.float16)
    lists = np.full((T, T), -1, np.int32)
    for p in range(T):
        lists[p, :p + 1] = r.permutation(p + 1)
    lengths = np.arange(1, T + 1, dtype=np.int32)
    out = oracle_lib.dlsa_attention(q, k, v, lists, lengths, D ** -0.5)
    dense = oracle_lib.sdpa_f64(q, k, v, D ** -0.5, q_pos=np.arange(T, dtype=np.int32))
    assert np.abs(out - dense).max() < 1e-6


def test_dlsa_skips_and_empty_rows(oracle_lib):
    r = rng(12)
    q = r.standard_normal((6, 3, 64)).astype(np.float16)
    k = r.standard_normal((1, 50, 64)).astype(np.float16)
    v = r.standard_normal((1, 50, 64)).astype(np.float16)
    base = np.array([[3, 7, 11, 19, -1, -1],
                     [5, 9, -1, -1, -1, -1],
                     [-1, -1, -1, -1, -1, -1]], np.int32)
    dirty = base.copy()
    dirty[0, 4] = 50      # out of range (== T): skipped
    dirty[1, 2] = -7      # negative: skipped
    lengths = np.array([5, 3, 0], np.int32)
    a = oracle_lib.dlsa_attention(q, k, v, base, np.array([4, 2, 0], np.int32), 0.125)
    b = oracle_lib.dlsa_attention(q, k, v, dirty, lengths, 0.125)
    assert np.array_equal(a, b)
    assert np.all(a[:, 2] == 0)


# dlsa_attention_f64: the typed read's checker (any input dtype, fp64). Pinned
# by the reference's golden outputs, by the fp32 C restatement on the same
# inputs, by the dense-causal identity and by hand-computed answers.
@pytest.mark.parametrize("m", ["real", "random"])
def test_dlsa_f64_qwen_layer_golden(oracle_lib, m):
    d = _golden("qwen_layer")
    q = d["q_rows"].transpose(1, 0, 2)
    k = d["k"].transpose(1, 0, 2)
    v = d["v"].transpose(1, 0, 2)
    out = oracle_lib.dlsa_attention_f64(q, k, v, d[f"{m}.selected"], d[f"{m}.selected_lengths"],
                                        256 ** -0.5)
    assert np.abs(out - d[f"{m}.attention_out"].transpose(1, 0, 2)).max() < 1e-5


def test_dlsa_f64_matches_the_fp32_restatement(oracle_lib):
    r = rng(13)
    q = r.standard_normal((8, 5, 128)).astype(np.float16)
    k = r.standard_normal((2, 300, 128)).astype(np.float16)
    v = r.standard_normal((2, 300, 128)).astype(np.float16)
    lists = np.full((5, 120), -1, np.int32)
    lengths = np.array([120, 1, 60, 0, 99], np.int32)
    for row in range(5):
        lists[row, :lengths[row]] = r.choice(300, lengths[row], replace=False)
    lists[2, 3] = 300  # past the end: skipped
    a = oracle_lib.dlsa_attention_f64(q, k, v, lists, lengths, 128 ** -0.5)
    b = oracle_lib.dlsa_attention(q, k, v, lists, lengths, 128 ** -0.5)
    assert np.abs(a - b).max() < 1e-5
    assert np.all(a[:, 3] == 0)


def test_dlsa_f64_known_answers(oracle_lib):
    # one entry: that key's value row exactly; two keys with equal scores:
    # their mean; a key scored log(3) above another: weights 3/4, 1/4
    k = np.zeros((1, 4, 32))
    v = np.arange(4 * 32, dtype=np.float64).reshape(1, 4, 32)
    k[0, 2, 0] = np.log(3.0)
    q = np.zeros((2, 1, 32))
    q[:, 0, 0] = 1.0
    lists = np.array([[1, 3, -1]], np.int32)
    one = oracle_lib.dlsa_attention_f64(q, k, v, lists, np.array([1], np.int32), 1.0)
    assert np.array_equal(one[0, 0], v[0, 1])
    two = oracle_lib.dlsa_attention_f64(q, k, v, lists, np.array([2], np.int32), 1.0)
    assert np.allclose(two[1, 0], (v[0, 1] + v[0, 3]) / 2, rtol=0, atol=1e-12)
    w = oracle_lib.dlsa_attention_f64(q, k, v, np.array([[2, 0]], np.int32),
                                      np.array([2], np.int32), 1.0)
    assert np.allclose(w[0, 0], 0.75 * v[0, 2] + 0.25 * v[0, 0], rtol=0, atol=1e-12)


def test_dlsa_f64_full_list_equals_dense_causal(oracle_lib):
    r = rng(14)
    T, D = 50, 32
    q = r.standard_normal((6, T, D)).astype(np.float32)
    k = r.standard_normal((2, T, D)).astype(np.float32)
    v = r.standard_normal((2, T, D)).astype(np.float32)
    lists = np.full((T, T), -1, np.int32)
    for p in range(T):
        lists[p, :p + 1] = r.permutation(p + 1)
    out = oracle_lib.dlsa_attention_f64(q, k, v, lists, np.arange(1, T + 1, dtype=np.int32),
                                        D ** -0.5)
    pos = np.arange(T)
    assert np.abs(out - _np_attention(q, k, v, D ** -0.5, pos)).max() < 1e-12
