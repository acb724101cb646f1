"""GPU parity of the D-LSA read over a KV cache in place (qw_kv_dlsa_attention),
the reference's update_and_fetch + sparse_attention pair
(crates/runtime/src/qwen3_next/dlsa.rs:161-177) without the fetch.

* fp16 cache: K rows and the 8-key V blocks are read in place; the result
  equals the strided read of the same rows (qw_dlsa_sparse_attention) bit for
  bit, over the golden qwen_layer lists (general, unaligned entries) and the
  config-5 list (whole 512-key runs: the aligned block loads).
* affine 4/8-bit and Int8 caches: rows dequantized inside the gather, checked
  against the oracle's fetch (MLX's composite dequant) fed to the oracle's
  K2 restatement, within the stated bar (2e-3 max-abs, 1e-3 rel-L2), and
  against the strided read of the device fetch within fp32 rounding.
* Turbo4: fetched to fp16 first, as the reference does: bit-equal to the
  strided read of qw_kv_dequantize's rows.
"""
import os

import numpy as np
import pytest
from safetensors.numpy import load_file

from conftest import GOLDEN, rng
from test_gpu_dlsa import c5_list
from test_gpu_kv import _gpu, _np, assert_close

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


def _cache(mode, k, v, cap=None):
    import qw_amd

    H, T, D = k.shape
    c = qw_amd.KVCache(mode, H, D, capacity=cap or T)
    c.update(_gpu(k), _gpu(v))
    return c


def _strided_of(cache):
    """The strided read of the cache's fetched fp16 rows (the reference's
    update_and_fetch then sparse_attention)."""
    k, v = cache.dequantize()
    return k[0], v[0]


def test_fp16_cache_golden_lists_bit_equal_to_strided():
    import qw_amd

    d = load_file(os.path.join(GOLDEN, "dlsa_qwen_layer.safetensors"))
    q = _gpu(d["q_rows"].transpose(1, 0, 2))                 # [24, 10, 256]
    k = np.ascontiguousarray(d["k"].transpose(1, 0, 2))      # [4, 260, 256]
    v = np.ascontiguousarray(d["v"].transpose(1, 0, 2))
    c = _cache("fp16", k, v, cap=512)
    for m in ("real", "random"):
        lists = _gpu(d[f"{m}.selected"])
        lengths = _gpu(d[f"{m}.selected_lengths"])
        out = _np(c.dlsa_attention(q, lists, lengths, 256 ** -0.5))[0]
        ref = d[f"{m}.attention_out"].transpose(1, 0, 2)
        assert_close(out, ref, f"qwen_layer {m} through an fp16 cache")
        strided = _np(qw_amd.sparse_attention(q, _gpu(k), _gpu(v), lists, lengths, 256 ** -0.5))[0]
        np.testing.assert_array_equal(out, strided)
    c.close()


def test_fp16_cache_config5_bit_equal_to_strided(oracle_lib):
    """Config 5 geometry (131072 keys, the 4612-entry sink + window + whole
    512-key blocks list) on an fp16 cache: equal to the strided read, and to
    the oracle within the bar."""
    import qw_amd

    T, H, G, D = 131072, 4, 6, 256
    r = rng(5)
    k = r.standard_normal((H, T, D)).astype(np.float16)
    v = r.standard_normal((H, T, D)).astype(np.float16)
    q = r.standard_normal((H * G, 1, D)).astype(np.float16)
    lists = c5_list(T, 5)[None]
    lengths = np.array([lists.shape[1]], np.int32)
    c = _cache("fp16", k, v)
    out = _np(c.dlsa_attention(_gpu(q), _gpu(lists), _gpu(lengths), D ** -0.5))[0]
    strided = _np(qw_amd.sparse_attention(_gpu(q), _gpu(k), _gpu(v), _gpu(lists), _gpu(lengths),
                                          D ** -0.5))[0]
    np.testing.assert_array_equal(out, strided)
    ref = oracle_lib.dlsa_attention(q, k, v, lists, lengths, D ** -0.5)
    assert_close(out, ref, "config5 through an fp16 cache")
    c.close()


@pytest.mark.parametrize("mode", ["affine4", "affine8", "int8"])
@pytest.mark.parametrize("D", [256, 128])
@pytest.mark.parametrize("lists_kind", ["runs", "random"])
def test_quantized_cache_vs_oracle(oracle_lib, mode, D, lists_kind):
    import qw_amd

    H, G, T, L, W = 4, 6, 6000, 3, 1200
    r = rng({"affine4": 1, "affine8": 2, "int8": 3}[mode] * 100 + D + (lists_kind == "runs"))
    jit = r.uniform(0.5, 2.0, (H, 1, 1))
    k = (r.standard_normal((H, T, D)) * jit).astype(np.float16)
    v = (r.standard_normal((H, T, D)) * jit).astype(np.float16)
    q = r.standard_normal((H * G, L, D)).astype(np.float16)
    lists = np.full((L, W), -1, np.int32)
    lengths = np.array([W, 700, 0], np.int32)
    for row in range(L):
        n = lengths[row]
        if lists_kind == "runs":  # whole aligned runs, a window and sinks
            blocks = np.sort(r.choice(np.arange(1, (T - 256) // 128), n // 128, replace=False))
            lst = np.concatenate([np.arange(b * 128, b * 128 + 128) for b in blocks]
                                 + [np.arange(T - (n % 128), T)])[:n]
        else:
            lst = r.choice(T, n, replace=False)
        lists[row, :n] = lst
    lists[1, 3] = T + 5   # past the cached rows: skipped
    c = _cache(mode, k, v)
    out = _np(c.dlsa_attention(_gpu(q), _gpu(lists), _gpu(lengths), D ** -0.5))[0]
    orc = (oracle_lib.Int8CacheOracle(H, D, T) if mode == "int8"
           else oracle_lib.AffineCacheOracle(H, D, T, 4 if mode == "affine4" else 8))
    orc.update(k, v)
    kf, vf = orc.fetch()
    ref = oracle_lib.dlsa_attention(q, kf, vf, lists, lengths, D ** -0.5)
    assert_close(out, ref, f"{mode} D={D} {lists_kind} through the cache")
    assert np.all(out[:, 2] == 0)  # the empty row
    # the device fetch read strided agrees to fp32 rounding (only the order of
    # the QK accumulation differs)
    ks, vs = _strided_of(c)
    strided = _np(qw_amd.sparse_attention(_gpu(q), ks, vs, _gpu(lists), _gpu(lengths),
                                          D ** -0.5))[0]
    assert np.abs(out.astype(np.float64) - strided).max() <= 2e-3 * max(1.0, np.abs(strided).max())
    c.close()


@pytest.mark.parametrize("mode", ["affine4", "affine8"])
def test_quantized_cache_separately_rounded_dequant(oracle_lib, mode):
    """Rows with scales outside the 2-op dequant's exact range clear the
    cache's fast flag: the read then takes the separately rounded dequant."""
    H, G, T, D, W = 2, 6, 2048, 256, 600
    r = rng(31)
    k = r.standard_normal((H, T, D)).astype(np.float16)
    v = r.standard_normal((H, T, D)).astype(np.float16)
    k[:, 100:104] *= 3000.0   # |scale| > 64 in those groups
    v[:, 200:208] *= 1e-4     # tiny scales
    q = (r.standard_normal((H * G, 2, D)) * 0.01).astype(np.float16)
    lists = np.stack([np.arange(0, W), r.choice(T, W, replace=False)]).astype(np.int32)
    lengths = np.array([W, W], np.int32)
    c = _cache(mode, k, v)
    out = _np(c.dlsa_attention(_gpu(q), _gpu(lists), _gpu(lengths), D ** -0.5))[0]
    orc = oracle_lib.AffineCacheOracle(H, D, T, 4 if mode == "affine4" else 8)
    orc.update(k, v)
    kf, vf = orc.fetch()
    ref = oracle_lib.dlsa_attention(q, kf, vf, lists, lengths, D ** -0.5)
    assert_close(out, ref, f"{mode} extreme scales")
    c.close()


def test_turbo4_cache_equals_fetch_then_read():
    import qw_amd

    H, G, T, D, W = 4, 6, 5000, 256, 900
    r = rng(41)
    k = r.standard_normal((H, T, D)).astype(np.float16)
    v = r.standard_normal((H, T, D)).astype(np.float16)
    q = _gpu(r.standard_normal((H * G, 2, D)).astype(np.float16))
    lists = _gpu(np.stack([r.choice(T, W, replace=False) for _ in range(2)]).astype(np.int32))
    lengths = _gpu(np.array([W, W - 100], np.int32))
    c = _cache("turbo4", k, v)
    out = _np(c.dlsa_attention(q, lists, lengths, D ** -0.5))
    ks, vs = _strided_of(c)
    want = _np(qw_amd.sparse_attention(q, ks, vs, lists, lengths, D ** -0.5))
    np.testing.assert_array_equal(out, want)
    c.close()


@pytest.mark.parametrize("mode", ["fp16", "affine4"])
def test_update_and_dlsa_attention(oracle_lib, mode):
    """Append L new rows, then read lists that include them: equal to update
    followed by the read."""
    H, G, T, D, L, W = 4, 6, 3000, 256, 2, 500
    r = rng(51)
    k = r.standard_normal((H, T + L, D)).astype(np.float16)
    v = r.standard_normal((H, T + L, D)).astype(np.float16)
    q = _gpu(r.standard_normal((H * G, L, D)).astype(np.float16))
    lists = np.stack([np.concatenate([r.choice(T, W - 2, replace=False), [T, T + 1]])
                      for _ in range(L)]).astype(np.int32)
    lengths = np.array([W, W - 1], np.int32)
    a = _cache(mode, k[:, :T], v[:, :T], cap=T + 256)
    b = _cache(mode, k[:, :T], v[:, :T], cap=T + 256)
    got = _np(a.update_and_dlsa_attention(q, _gpu(k[:, T:]), _gpu(v[:, T:]), _gpu(lists),
                                          _gpu(lengths), D ** -0.5))
    b.update(_gpu(k[:, T:]), _gpu(v[:, T:]))
    want = _np(b.dlsa_attention(q, _gpu(lists), _gpu(lengths), D ** -0.5))
    np.testing.assert_array_equal(got, want)
    assert a.offset == T + L
    a.close()
    b.close()


def test_empty_cache_is_an_error():
    import qw_amd

    c = qw_amd.KVCache("fp16", 4, 256, capacity=256)
    q = _gpu(np.zeros((24, 1, 256), np.float16))
    lists = _gpu(np.zeros((1, 4), np.int32))
    lengths = _gpu(np.array([4], np.int32))
    with pytest.raises(qw_amd.QwError) as ei:
        c.dlsa_attention(q, lists, lengths, 1 / 16)
    assert ei.value.status == 1 and "empty" in str(ei.value)
    c.close()


# The two-rows-a-workgroup D-LSA kernel (RP = 2) on cache sources: one-pass
# calls (rows x kv_heads >= 192), 2G <= 16 and rows x kv_heads >= 384, at
# head_dim 128 (the cache sources' pair form). 203 rows over 2 KV heads
# (406 units, an odd row count so the last workgroup holds one row),
# unequal lengths with -1 padding and past-the-end entries. Both list kinds:
# whole aligned runs (the aligned block gathers, the pair's shared tiles)
# and random entries (the unaligned gathers). One affine case holds scales
# outside the 2-op dequant's exact range, so the separately rounded second
# pass runs under the pair form too.
@pytest.mark.parametrize("mode,extreme", [("fp16", False), ("affine4", False),
                                          ("affine8", False), ("int8", False),
                                          ("affine4", True)])
@pytest.mark.parametrize("lists_kind", ["runs", "random"])
def test_row_pairs_over_cache_sources_vs_oracle(oracle_lib, mode, extreme, lists_kind):
    import qw_amd

    H, G, D, T, L, W = 2, 6, 128, 3000, 203, 400
    r = rng(8100 + 10 * ["fp16", "affine4", "affine8", "int8"].index(mode) + extreme
            + 2 * (lists_kind == "runs"))
    jit = r.uniform(0.5, 2.0, (H, 1, 1))
    k = (r.standard_normal((H, T, D)) * jit).astype(np.float32)
    v = (r.standard_normal((H, T, D)) * jit).astype(np.float32)
    if extreme:
        k[:, 100:140, :64] *= 1e-3       # |scale| < 2^-10
        k[:, 900:905, 64:] *= 300.0      # |scale| >= 64
        v[:, 200:260, 64:] *= 1e-3
    k, v = k.astype(np.float16), v.astype(np.float16)
    q = r.standard_normal((H * G, L, D)).astype(np.float16)
    lists = np.full((L, W), -1, np.int32)
    lengths = r.integers(1, W + 1, L).astype(np.int32)
    lengths[::7] = W
    lengths[5] = 0
    for row in range(L):
        n = int(lengths[row])
        if lists_kind == "runs":
            # whole aligned 16-key runs, then a ragged tail; the two rows of a
            # workgroup (2j, 2j + 1) draw from the same runs, so their tiles
            # are shared (gathered and multiplied once) up to the shorter list
            if row % 2 == 0:
                blocks = np.sort(r.choice(np.arange(T // 16 - 1), W // 16, replace=False))
            lst = np.concatenate([np.arange(b * 16, b * 16 + 16) for b in blocks[:n // 16]]
                                 + [np.arange(T - (n % 16), T)])[:n]
        else:
            lst = r.choice(T, n, replace=False)
        lists[row, :n] = lst
    lists[3, 1] = T + 7      # past the cached rows: skipped
    lists[8, 0] = T + 100
    c = _cache(mode, k, v)
    assert (lengths.size * H) >= 384
    out = _np(c.dlsa_attention(_gpu(q), _gpu(lists), _gpu(lengths), D ** -0.5))[0]
    if mode == "fp16":
        kf, vf = k, v
    else:
        orc = (oracle_lib.Int8CacheOracle(H, D, T) if mode == "int8"
               else oracle_lib.AffineCacheOracle(H, D, T, 4 if mode == "affine4" else 8))
        orc.update(k, v)
        kf, vf = orc.fetch()
    ref = oracle_lib.dlsa_attention(q, kf, vf, lists, lengths, D ** -0.5)
    assert_close(out, ref, f"row pairs {mode}{' extreme' if extreme else ''} {lists_kind}")
    assert np.all(out[:, 5] == 0)  # the empty row
    c.close()
