"""qw_dlsa_sparse_attention_noalloc: the D-LSA read with its split-K partials
in the library's fixed device scratch (no allocation). Through the C ABI, its
output must equal qw_dlsa_sparse_attention_with's bit for bit (same kernels,
same part count), on two calls in a row, the second smaller; an explicit part
count whose partials exceed the scratch is refused; an automatic part count
is lowered to fit."""
import ctypes

import numpy as np
import pytest

from conftest import rng
from test_gpu_kv import _gpu, _np, assert_close

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

_p, _i, _i64, _f = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_float
SCRATCH_BYTES = 4 << 20


def _lib():
    import qw_amd

    L = qw_amd.lib()
    fn = L.qw_dlsa_sparse_attention_noalloc
    fn.restype = _i
    fn.argtypes = [_p, _p, _p, _i64, _i64, _i64, _i64, _p, _p, _i, _i, _i, _i, _i, _i, _f, _i, _i,
                   _p, _p]
    return L


def _call(L, name, q, k, v, lists, lengths, scale, parts):
    hq, rows, D = q.shape
    hkv, T, _ = k.shape
    out = torch.empty_like(q)
    st = torch.cuda.current_stream().cuda_stream
    rc = getattr(L, name)(q.data_ptr(), k.data_ptr(), v.data_ptr(), k.stride(0), k.stride(1),
                          v.stride(0), v.stride(1), lists.data_ptr(), lengths.data_ptr(), rows,
                          lists.shape[1], hq, hkv, D, T, scale, parts, 0, out.data_ptr(), st)
    return rc, out


def _case(seed, T, H, G, D, L, W):
    r = rng(seed)
    k = _gpu(r.standard_normal((H, T, D)).astype(np.float16))
    v = _gpu(r.standard_normal((H, T, D)).astype(np.float16))
    q = _gpu(r.standard_normal((H * G, L, D)).astype(np.float16))
    lists = np.full((L, W), -1, np.int32)
    lens = r.integers(W // 2, W + 1, L).astype(np.int32)
    for row in range(L):
        lists[row, :lens[row]] = r.choice(T, lens[row], replace=False)
    return q, k, v, _gpu(lists), _gpu(lens)


def test_noalloc_equals_allocating_entry():
    L = _lib()
    scale = 256 ** -0.5
    # config-5 shape (one row, 4612 entries, automatic parts: 48), then a
    # smaller call (3 rows, 700 entries) reusing the same scratch
    big = _case(1, 131072 // 8, 4, 6, 256, 1, 4612)
    small = _case(2, 3000, 4, 6, 256, 3, 700)
    for inputs, knobs in ((big, (0, 16, 64)), (small, (0, 16, 32))):
        for parts in knobs:
            rc_a, a = _call(L, "qw_dlsa_sparse_attention_with", *inputs, scale, parts)
            rc_b, b = _call(L, "qw_dlsa_sparse_attention_noalloc", *inputs, scale, parts)
            torch.cuda.synchronize()
            assert rc_a == 0 and rc_b == 0, L.qw_last_error()
            np.testing.assert_array_equal(_np(b), _np(a))


def test_noalloc_scratch_limit():
    L = _lib()
    scale = 256 ** -0.5
    # 40 rows x 64 q heads: 2.6 MB of partials a part, so one part fits
    q, k, v, lists, lens = _case(3, 3000, 4, 16, 256, 40, 100)
    part_bytes = 40 * 64 * (256 * 4 + 8)           # rows x q heads x (fp32 row + (m, l))
    fit = SCRATCH_BYTES // part_bytes
    assert fit == 1
    rc, _ = _call(L, "qw_dlsa_sparse_attention_noalloc", q, k, v, lists, lens, scale, fit + 1)
    assert rc == 1 and b"scratch" in L.qw_last_error()
    # automatic parts (2 here: 160 workgroups a part) are lowered to what fits:
    # equal to one explicit part
    rc_a, a = _call(L, "qw_dlsa_sparse_attention_with", q, k, v, lists, lens, scale, fit)
    rc_b, b = _call(L, "qw_dlsa_sparse_attention_noalloc", q, k, v, lists, lens, scale, 0)
    torch.cuda.synchronize()
    assert rc_a == 0 and rc_b == 0
    np.testing.assert_array_equal(_np(b), _np(a))
    rc_c, c = _call(L, "qw_dlsa_sparse_attention_with", q, k, v, lists, lens, scale, 0)
    torch.cuda.synchronize()
    assert rc_c == 0
    assert_close(_np(b), _np(c), "noalloc auto (1 part) vs auto (2 parts)")
