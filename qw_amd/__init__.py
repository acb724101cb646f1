"""qw_amd - MI355X (gfx950) full-attention hot path of cr0sh/qw.

The compute lives in ``libqwattn.so`` (hand-written HIP kernels behind the C
ABI of ``include/qwattn.h``). This module is the thin host mirror of the
reference's Rust interface for the path, over ctypes, so that Python callers
and the tests use the reference's names:

* :class:`KVCache` mirrors ``crates/mlxcel-core/src/cache.rs`` ``KVCache``
  (``update`` :922, ``update_and_fetch`` :2709, ``update_and_turbo4_attention``
  :3495 / ``update_and_turbo4_causal_attention`` :3520 with the affine codec,
  ``trim`` :2251, ``offset``, ``nbytes`` :3063, snapshot tensors :570-626).
* :func:`sparse_attention` / :func:`sparse_attention_with` mirror
  ``crates/mlxcel-core/src/dlsa_attention.rs:31`` / ``:44``.
* :func:`attention` / :func:`causal_attention` mirror ``layers::attention(q, k,
  v, scale, mask, softcap, window)`` (``layers.rs:4010``) and
  ``causal_attention(q, k, v, scale, softcap, window)`` (``lib.rs:3185``);
  ``KVCache.update_and_attention(..., mask)`` and
  :meth:`KVCache.attention_general` take the same options over a cache.

Torch is used only to hold device memory and to name the current stream.
Tensors follow the reference's layouts: ``[1, H, L, D]`` (the batch of 1 may
be omitted). There is no CPU fallback: every call goes through the HIP
library and raises :class:`QwError` when it is missing or a call fails.
"""
from __future__ import annotations

import ctypes
import os

__all__ = ["KVCacheMode", "KVCache", "QwError", "attention", "causal_attention",
           "sparse_attention", "sparse_attention_with",
           "fused_rope_qk_append", "dlsa_select", "dlsa_select_with", "turbo4_codebook",
           "turbo4_signs",
           "lib", "LIB_PATH"]

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libqwattn.so")
_lib = None

QW_OK = 0
_STATUS = {1: "invalid argument", 2: "unsupported", 3: "out of memory", 4: "HIP error",
           5: "invalid state"}


class QwError(RuntimeError):
    """A libqwattn call failed; ``status`` is the C status code."""

    def __init__(self, status: int, message: str):
        super().__init__(f"{_STATUS.get(status, status)}: {message}")
        self.status = status


_p = ctypes.c_void_p
_i = ctypes.c_int
_i64 = ctypes.c_int64
_f = ctypes.c_float

_SIGNATURES = {
    "qw_abi_version": (_i, []),
    "qw_last_error": (ctypes.c_char_p, []),
    "qw_kv_create": (_i, [_i, _i, _i, _i, _i, _i, ctypes.POINTER(_p)]),
    "qw_kv_create_seeded": (_i, [_i, _i, _i, _i, _i, _i, ctypes.c_uint32, ctypes.POINTER(_p)]),
    "qw_kv_export_turbo4": (_i, [_p, _p, _p, _p, _p, _p, _p]),
    "qw_kv_import_turbo4": (_i, [_p, _i, _p, _p, _p, _p, _p, _p]),
    "qw_turbo4_codebook": (_i, [_i, _i, _p]),
    "qw_turbo4_signs": (_i, [_i, ctypes.c_uint32, _p]),
    "qw_kv_destroy": (_i, [_p]),
    "qw_kv_reserve": (_i, [_p, _i, _p]),
    "qw_kv_offset": (_i, [_p, ctypes.POINTER(_i)]),
    "qw_kv_capacity": (_i, [_p, ctypes.POINTER(_i)]),
    "qw_kv_nbytes": (_i, [_p, ctypes.POINTER(_i64)]),
    "qw_kv_update": (_i, [_p, _p, _p, _i, _p]),
    "qw_kv_update_and_fetch": (_i, [_p, _p, _p, _i, _p, _p, _p]),
    "qw_kv_dequantize": (_i, [_p, _i, _i, _p, _p, _p]),
    "qw_kv_update_and_attention": (_i, [_p, _p, _i, _i, _p, _p, _f, _i, _p, _p]),
    "qw_kv_attention": (_i, [_p, _p, _i, _i, _f, _i, _p, _p]),
    "qw_sdpa": (_i, [_p, _i, _i, _p, _p, _i, _i, _i, _i64, _i64, _i64, _i64, _f, _i, _i, _f,
                     _p, _i, _i64, _i64, _p, _p]),
    "qw_kv_attention_general": (_i, [_p, _p, _i, _i, _f, _i, _i, _f, _p, _i, _i64, _i64, _p,
                                     _p]),
    "qw_kv_update_and_attention_general": (_i, [_p, _p, _i, _i, _p, _p, _f, _i, _i, _f, _p, _i,
                                                _i64, _i64, _p, _p]),
    "qw_kv_trim": (_i, [_p, _i, ctypes.POINTER(_i)]),
    "qw_kv_dlsa_attention": (_i, [_p, _p, _i, _i, _p, _p, _i, _f, _p, _p]),
    "qw_kv_update_and_dlsa_attention": (_i, [_p, _p, _i, _i, _p, _p, _p, _p, _i, _f, _p, _p]),
    "qw_kv_demote": (_i, [_p, _i, _p, ctypes.POINTER(_i)]),
    "qw_kv_export": (_i, [_p, _p, _p, _p, _p, _p, _p, _p]),
    "qw_kv_import": (_i, [_p, _i, _p, _p, _p, _p, _p, _p, _p]),
    "qw_dlsa_select": (_i, [_p, _i64, _p, _i, _i, _p, _i, _i, _i, _i, _i, _i, _i, _i, _p, _p, _p,
                            _p, _p]),
    "qw_fused_rope_qk_append": (_i, [_p, _i, _i, _i, _i, _i, _i, _f, _f, _i, _i, _i, _p, _p, _p,
                                     _p]),
    "qw_kv_rope_update": (_i, [_p, _p, _i, _i, _i, _i, _f, _f, _i, _p, _p]),
    "qw_kv_rope_update_and_attention": (_i, [_p, _p, _i, _i, _i, _i, _f, _f, _i, _f, _i, _p, _p,
                                             _p]),
    "qw_dlsa_sparse_attention": (_i, [_p, _p, _p, _i64, _i64, _i64, _i64, _p, _p, _i, _i, _i,
                                      _i, _i, _i, _f, _p, _p]),
    "qw_dlsa_sparse_attention_with": (_i, [_p, _p, _p, _i64, _i64, _i64, _i64, _p, _p, _i, _i,
                                           _i, _i, _i, _i, _f, _i, _i, _p, _p]),
    "qw_dlsa_sparse_attention_noalloc": (_i, [_p, _p, _p, _i64, _i64, _i64, _i64, _p, _p, _i, _i,
                                              _i, _i, _i, _i, _f, _i, _i, _p, _p]),
    "qw_dlsa_sparse_attention_typed": (_i, [_p, _i, _p, _p, _i, _i64, _i64, _i64, _i64, _p, _p, _i,
                                            _i, _i, _i, _i, _i, _f, _i, _i, _p, _p]),
}


def lib() -> ctypes.CDLL:
    """Load libqwattn.so (built by ``qw_amd.build``); raise if it is absent."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise QwError(4, f"{LIB_PATH} is not built; run `python -m qw_amd.build`")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _check(rc: int) -> None:
    if rc != QW_OK:
        raise QwError(rc, lib().qw_last_error().decode())


def _torch():
    import torch  # imported lazily: the ABI itself needs no torch

    return torch


def _stream(device) -> int:
    torch = _torch()
    return torch.cuda.current_stream(device).cuda_stream


def _as3(t, name: str):
    """Reference tensors are [1, H, L, D]; accept [H, L, D] as well."""
    if t.dim() == 4:
        if t.shape[0] != 1:
            raise QwError(1, f"{name}: batch must be 1")
        t = t[0]
    if t.dim() != 3:
        raise QwError(1, f"{name}: expected [1, H, L, D] or [H, L, D]")
    torch = _torch()
    if t.dtype != torch.float16:
        raise QwError(2, f"{name}: fp16 expected, got {t.dtype}")
    if not t.is_cuda:
        raise QwError(1, f"{name}: must be a device tensor")
    return t.contiguous()


class KVCacheMode:
    """Storage modes (reference ``KVCacheMode``, cache.rs:172, plus the affine codec)."""

    FP16 = 0
    AFFINE8 = 1
    AFFINE4 = 2
    INT8 = 3  # per-token absmax Int8 (cache.rs:262-316)
    TURBO4 = 4  # symmetric PolarQuant, the reference's served default (cache.rs:1438)

    BITS = {0: 16, 1: 8, 2: 4, 3: 8, 4: 4}
    DEFAULT_TURBO_SEED = 0x7B470404  # cache.rs:324

    @staticmethod
    def from_str(s: str) -> int:
        key = s.lower()
        table = {"fp16": 0, "float16": 0, "affine8": 1, "uniform8": 1, "affine4": 2,
                 "uniform4": 2, "int8": 3, "turbo4": 4}
        if key not in table:
            raise ValueError(f'unknown kv-cache-mode "{s}"; expected "fp16", "affine8", '
                             f'"affine4", "int8" or "turbo4"')
        return table[key]


class KVCache:
    """One layer's KV cache on a GPU (reference ``KVCache``, cache.rs:354)."""

    def __init__(self, mode: int | str, n_kv_heads: int, head_dim: int, capacity: int = 0,
                 group_size: int = 64, device=None, turbo_seed: int | None = None):
        torch = _torch()
        if isinstance(mode, str):
            mode = KVCacheMode.from_str(mode)
        self.mode = mode
        self.n_kv_heads = n_kv_heads
        self.head_dim = head_dim
        self.bits = KVCacheMode.BITS[mode]
        self.device = torch.device("cuda", torch.cuda.current_device() if device is None else
                                   torch.device(device).index or 0)
        self.turbo_seed = (KVCacheMode.DEFAULT_TURBO_SEED if turbo_seed is None
                           else int(turbo_seed) & 0xFFFFFFFF)
        h = _p()
        # KVCache::new_with_mode_and_seed (cache.rs:537)
        _check(lib().qw_kv_create_seeded(mode, group_size, n_kv_heads, head_dim, capacity,
                                         self.device.index, self.turbo_seed, ctypes.byref(h)))
        self._h = h

    def close(self) -> None:
        if getattr(self, "_h", None):
            lib().qw_kv_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # -- state
    @property
    def offset(self) -> int:
        v = _i()
        _check(lib().qw_kv_offset(self._h, ctypes.byref(v)))
        return v.value

    @property
    def capacity(self) -> int:
        v = _i()
        _check(lib().qw_kv_capacity(self._h, ctypes.byref(v)))
        return v.value

    def nbytes(self) -> int:
        v = _i64()
        _check(lib().qw_kv_nbytes(self._h, ctypes.byref(v)))
        return v.value

    def reserve(self, capacity: int) -> None:
        _check(lib().qw_kv_reserve(self._h, capacity, _stream(self.device)))

    # -- append / fetch
    def update(self, keys, values) -> None:
        k, v = _as3(keys, "keys"), _as3(values, "values")
        if k.shape != v.shape or k.shape[0] != self.n_kv_heads or k.shape[2] != self.head_dim:
            raise QwError(1, "update: keys/values must be [n_kv_heads, L, head_dim]")
        _check(lib().qw_kv_update(self._h, k.data_ptr(), v.data_ptr(), k.shape[1],
                                  _stream(self.device)))

    def rope_update(self, qkv, n_q_heads: int, rope_dims: int, rope_base: float,
                    rope_scale: float = 1.0, traditional: bool = False,
                    position0: int | None = None):
        """q/k RoPE out of the fused QKV projection with the append fused in
        (reference ``Attention::forward_fused_rope_append``, layers.rs:2852,
        then ``KVCache::update``): ``qkv`` is [1, L, (Hq + 2 Hkv) D] or
        [L, (Hq + 2 Hkv) D] fp16; token t rotates at position0 + t (default:
        the cache offset). Returns the rotated q as [1, Hq, L, D]."""
        torch = _torch()
        x = qkv[0] if qkv.dim() == 3 else qkv
        if x.dim() != 2 or x.dtype != torch.float16 or not x.is_cuda:
            raise QwError(1, "rope_update: qkv must be a [1, L, W] or [L, W] fp16 device tensor")
        x = x.contiguous()
        L, W = x.shape
        if W != (n_q_heads + 2 * self.n_kv_heads) * self.head_dim:
            raise QwError(1, "rope_update: qkv width does not match the head geometry")
        pos = self.offset if position0 is None else position0
        q = torch.empty((n_q_heads, L, self.head_dim), dtype=torch.float16, device=self.device)
        _check(lib().qw_kv_rope_update(self._h, x.data_ptr(), n_q_heads, L, rope_dims,
                                       int(traditional), float(rope_base), float(rope_scale),
                                       pos, q.data_ptr(), _stream(self.device)))
        return q.unsqueeze(0)

    def rope_update_and_attention(self, qkv, n_q_heads: int, rope_dims: int, rope_base: float,
                                  scale: float, rope_scale: float = 1.0, traditional: bool = False,
                                  position0: int | None = None, causal: bool = False):
        """RoPE, append and attention of one projection (rope_update, then
        attention of the rotated q over the cache; one decode launch for
        decode-route shapes). Returns (out [1, Hq, L, D], rotated q [1, Hq,
        L, D])."""
        torch = _torch()
        x = qkv[0] if qkv.dim() == 3 else qkv
        if x.dim() != 2 or x.dtype != torch.float16 or not x.is_cuda:
            raise QwError(1, "rope_update_and_attention: qkv must be a [1, L, W] or [L, W] fp16 "
                             "device tensor")
        x = x.contiguous()
        L, W = x.shape
        if W != (n_q_heads + 2 * self.n_kv_heads) * self.head_dim:
            raise QwError(1, "rope_update_and_attention: qkv width does not match the head geometry")
        pos = self.offset if position0 is None else position0
        q = torch.empty((n_q_heads, L, self.head_dim), dtype=torch.float16, device=self.device)
        out = torch.empty_like(q)
        _check(lib().qw_kv_rope_update_and_attention(
            self._h, x.data_ptr(), n_q_heads, L, rope_dims, int(traditional), float(rope_base),
            float(rope_scale), pos, float(scale), int(causal), q.data_ptr(), out.data_ptr(),
            _stream(self.device)))
        return out.unsqueeze(0), q.unsqueeze(0)

    def dequantize(self, start: int = 0, n: int | None = None):
        torch = _torch()
        n = self.offset - start if n is None else n
        k = torch.empty((self.n_kv_heads, n, self.head_dim), dtype=torch.float16,
                        device=self.device)
        v = torch.empty_like(k)
        _check(lib().qw_kv_dequantize(self._h, start, n, k.data_ptr(), v.data_ptr(),
                                      _stream(self.device)))
        return k.unsqueeze(0), v.unsqueeze(0)

    def update_and_fetch(self, keys, values):
        self.update(keys, values)
        return self.dequantize(0, self.offset)

    # -- attention
    def _attn(self, q, keys, values, scale: float, causal: bool):
        torch = _torch()
        qq = _as3(q, "q")
        hq, L, D = qq.shape
        out = torch.empty_like(qq)
        st = _stream(self.device)
        if keys is None:
            _check(lib().qw_kv_attention(self._h, qq.data_ptr(), hq, L, float(scale),
                                         int(causal), out.data_ptr(), st))
        else:
            k, v = _as3(keys, "keys"), _as3(values, "values")
            if k.shape != v.shape or k.shape[1] != L:
                raise QwError(1, "attention: new keys/values must have q's row count")
            _check(lib().qw_kv_update_and_attention(self._h, qq.data_ptr(), hq, L, k.data_ptr(),
                                                    v.data_ptr(), float(scale), int(causal),
                                                    out.data_ptr(), st))
        return out.unsqueeze(0)

    def update_and_attention(self, q, keys, values, scale: float, mask=None):
        """Append, then attend (reference ``update_and_turbo4_attention(q, k, v,
        scale, mask)``, cache.rs:3495). With a mask (bool, or additive f16 /
        bf16 / f32, broadcastable to [1, Hq, L, T]) the general route runs."""
        if mask is None:
            return self._attn(q, keys, values, scale, False)
        return self._general(q, keys, values, scale, False, 0, 0.0, mask)

    def update_and_causal_attention(self, q, keys, values, scale: float):
        """Append, then bottom-right causal attention (``update_and_turbo4_causal_attention``)."""
        return self._attn(q, keys, values, scale, True)

    def attention(self, q, scale: float, causal: bool = False):
        """Attend the cache as it is (fused prefix attention, cache.rs:3607)."""
        return self._attn(q, None, None, scale, causal)

    def attention_general(self, q, scale: float, causal: bool = False, window: int = 0,
                          softcap: float = 0.0, mask=None):
        """Attend the cache as it is with the general options (``layers::attention``'s
        mask and softcap, ``causal_attention``'s window) over its dequantized rows."""
        return self._general(q, None, None, scale, causal, window, softcap, mask)

    def update_and_attention_general(self, q, keys, values, scale: float, causal: bool = False,
                                     window: int = 0, softcap: float = 0.0, mask=None):
        """Append, then :meth:`attention_general`."""
        return self._general(q, keys, values, scale, causal, window, softcap, mask)

    def _general(self, q, keys, values, scale, causal, window, softcap, mask):
        torch = _torch()
        qq = _as3(q, "q")
        hq, L, D = qq.shape
        out = torch.empty_like(qq)
        T = self.offset + (0 if keys is None else L)
        m, md, mhs, mrs, _keep = _mask_args(mask, hq, L, T)
        st = _stream(self.device)
        if keys is None:
            _check(lib().qw_kv_attention_general(self._h, qq.data_ptr(), hq, L, float(scale),
                                                 int(causal), int(window), float(softcap), m, md,
                                                 mhs, mrs, out.data_ptr(), st))
        else:
            k, v = _as3(keys, "keys"), _as3(values, "values")
            if k.shape != v.shape or k.shape[1] != L:
                raise QwError(1, "attention: new keys/values must have q's row count")
            _check(lib().qw_kv_update_and_attention_general(
                self._h, qq.data_ptr(), hq, L, k.data_ptr(), v.data_ptr(), float(scale),
                int(causal), int(window), float(softcap), m, md, mhs, mrs, out.data_ptr(), st))
        return out.unsqueeze(0)

    # -- D-LSA read over the cache (qwen3_next/dlsa.rs:161-177)
    def _dlsa(self, q, keys, values, lists, lengths, scale: float):
        torch = _torch()
        qq = _as3(q, "q")
        hq, L, D = qq.shape
        if lists.dim() != 2 or lists.dtype != torch.int32 or lengths.dim() != 1 or \
                lengths.dtype != torch.int32 or lists.shape[0] != L or lengths.shape[0] != L:
            raise QwError(1, "dlsa_attention: lists [L,W] i32 and lengths [L] i32 expected")
        lists, lengths = lists.contiguous(), lengths.contiguous()
        out = torch.empty_like(qq)
        st = _stream(self.device)
        if keys is None:
            _check(lib().qw_kv_dlsa_attention(self._h, qq.data_ptr(), hq, L, lists.data_ptr(),
                                              lengths.data_ptr(), lists.shape[1], float(scale),
                                              out.data_ptr(), st))
        else:
            k, v = _as3(keys, "keys"), _as3(values, "values")
            if k.shape != v.shape or k.shape[1] != L:
                raise QwError(1, "dlsa_attention: new keys/values must have q's row count")
            _check(lib().qw_kv_update_and_dlsa_attention(
                self._h, qq.data_ptr(), hq, L, k.data_ptr(), v.data_ptr(), lists.data_ptr(),
                lengths.data_ptr(), lists.shape[1], float(scale), out.data_ptr(), st))
        return out.unsqueeze(0)

    def dlsa_attention(self, q, lists, lengths, scale: float):
        """D-LSA K2 over the cached rows in place: the reference's
        ``update_and_fetch`` + ``sparse_attention`` read without the fetch
        (``[1, Hq, L, D]`` q, ``[L, W]`` i32 lists, ``[L]`` i32 lengths)."""
        return self._dlsa(q, None, None, lists, lengths, scale)

    def update_and_dlsa_attention(self, q, keys, values, lists, lengths, scale: float):
        """Append the L new rows, then :meth:`dlsa_attention`."""
        return self._dlsa(q, keys, values, lists, lengths, scale)

    # -- lifecycle
    def demote_fp16_to_affine(self, target_mode: int | str) -> bool:
        """Re-store a populated fp16 cache in an affine mode (reference
        ``demote_fp16_to_turbo4``, cache.rs:3591): False, and nothing done,
        when the cache is not fp16 or holds no rows."""
        if isinstance(target_mode, str):
            target_mode = KVCacheMode.from_str(target_mode)
        d = _i()
        _check(lib().qw_kv_demote(self._h, target_mode, _stream(self.device), ctypes.byref(d)))
        if d.value:
            self.mode = target_mode
            self.bits = KVCacheMode.BITS[target_mode]
        return bool(d.value)

    def demote_fp16_to_turbo4(self) -> bool:
        """The reference's own demote (cache.rs:3591): fp16 -> Turbo4."""
        return self.demote_fp16_to_affine(KVCacheMode.TURBO4)

    def trim(self, n: int) -> int:
        v = _i()
        _check(lib().qw_kv_trim(self._h, n, ctypes.byref(v)))
        return v.value

    def snapshot_tensors(self) -> dict:
        """Packed tensors in the reference layout (cache.rs:570-626)."""
        torch = _torch()
        n, H, D = self.offset, self.n_kv_heads, self.head_dim
        st = _stream(self.device)
        if self.mode == KVCacheMode.FP16:
            k = torch.empty((H, n, D), dtype=torch.float16, device=self.device)
            v = torch.empty_like(k)
            _check(lib().qw_kv_export(self._h, k.data_ptr(), None, None, v.data_ptr(), None, None,
                                      st))
            return {"keys": k, "values": v}
        if self.mode == KVCacheMode.TURBO4:
            # turbo4_snapshot_tensors (cache.rs:570): packed [H, T, D/2] u8, sidecars [H, T, 1]
            t = {name: torch.empty((H, n, D // 2), dtype=torch.uint8, device=self.device)
                 for name in ("k_packed", "v_packed")}
            for name in ("k_rescale", "v_norms", "v_rescale"):
                t[name] = torch.empty((H, n, 1), dtype=torch.float16, device=self.device)
            _check(lib().qw_kv_export_turbo4(self._h, t["k_packed"].data_ptr(),
                                             t["k_rescale"].data_ptr(), t["v_packed"].data_ptr(),
                                             t["v_norms"].data_ptr(), t["v_rescale"].data_ptr(),
                                             st))
            return t
        if self.mode == KVCacheMode.INT8:
            # the reference's keys, values [H, T, D] int8; key_scales, val_scales [H, T, 1] f16
            t = {name: torch.empty((H, n, D), dtype=torch.int8, device=self.device)
                 for name in ("keys", "values")}
            for name in ("key_scales", "val_scales"):
                t[name] = torch.empty((H, n, 1), dtype=torch.float16, device=self.device)
            _check(lib().qw_kv_export(self._h, t["keys"].data_ptr(), t["key_scales"].data_ptr(),
                                      None, t["values"].data_ptr(), t["val_scales"].data_ptr(),
                                      None, st))
            return t
        w = D * self.bits // 32
        t = {name: torch.empty((H, n, w), dtype=torch.int32, device=self.device)
             for name in ("k_codes", "v_codes")}
        for name in ("k_scales", "k_biases", "v_scales", "v_biases"):
            t[name] = torch.empty((H, n, D // 64), dtype=torch.float16, device=self.device)
        _check(lib().qw_kv_export(self._h, t["k_codes"].data_ptr(), t["k_scales"].data_ptr(),
                                  t["k_biases"].data_ptr(), t["v_codes"].data_ptr(),
                                  t["v_scales"].data_ptr(), t["v_biases"].data_ptr(), st))
        return t

    def restore_snapshot(self, tensors: dict) -> None:
        st = _stream(self.device)
        if self.mode == KVCacheMode.FP16:
            k, v = tensors["keys"].contiguous(), tensors["values"].contiguous()
            _check(lib().qw_kv_import(self._h, k.shape[1], k.data_ptr(), None, None, v.data_ptr(),
                                      None, None, st))
            return
        t = {k2: v2.contiguous() for k2, v2 in tensors.items()}
        if self.mode == KVCacheMode.TURBO4:
            # restore_turbo4_snapshot (cache.rs:581)
            n = t["k_packed"].shape[-2]
            _check(lib().qw_kv_import_turbo4(self._h, n, t["k_packed"].data_ptr(),
                                             t["k_rescale"].data_ptr(), t["v_packed"].data_ptr(),
                                             t["v_norms"].data_ptr(), t["v_rescale"].data_ptr(),
                                             st))
            return
        if self.mode == KVCacheMode.INT8:
            n = t["keys"].shape[1]
            _check(lib().qw_kv_import(self._h, n, t["keys"].data_ptr(), t["key_scales"].data_ptr(),
                                      None, t["values"].data_ptr(), t["val_scales"].data_ptr(),
                                      None, st))
            return
        n = t["k_codes"].shape[1]
        _check(lib().qw_kv_import(self._h, n, t["k_codes"].data_ptr(), t["k_scales"].data_ptr(),
                                  t["k_biases"].data_ptr(), t["v_codes"].data_ptr(),
                                  t["v_scales"].data_ptr(), t["v_biases"].data_ptr(), st))


def _kv_view(t, name: str):
    """K/V [1, Hkv, T, D] or [Hkv, T, D], any head/row strides, unit last stride."""
    torch = _torch()
    if t.dim() == 4:
        if t.shape[0] != 1:
            raise QwError(1, f"{name}: batch must be 1")
        t = t[0]
    if t.dim() != 3 or t.dtype != torch.float16 or not t.is_cuda:
        raise QwError(1, f"{name}: fp16 device tensor [1, Hkv, T, D] expected")
    if t.stride(2) != 1:
        t = t.contiguous()
    return t


def sparse_attention_with(q, k, v, lists, lengths, scale: float, parts: int = 0,
                          waves: int = 0):
    """D-LSA gathered read with launch knobs (dlsa_attention.rs:44)."""
    torch = _torch()
    qq = _as3(q, "q")
    kk, vv = _kv_view(k, "k"), _kv_view(v, "v")
    if kk.shape != vv.shape or kk.shape[2] != qq.shape[2]:
        raise QwError(1, "sparse_attention: k/v shapes disagree with q")
    if lists.dim() != 2 or lists.dtype != torch.int32 or lengths.dim() != 1 or \
            lengths.dtype != torch.int32 or lists.shape[0] != qq.shape[1] or \
            lengths.shape[0] != qq.shape[1]:
        raise QwError(1, "sparse_attention: lists [L,W] i32 and lengths [L] i32 expected")
    lists = lists.contiguous()
    lengths = lengths.contiguous()
    out = torch.empty_like(qq)
    hq, L, D = qq.shape
    hkv, T, _ = kk.shape
    _check(lib().qw_dlsa_sparse_attention_with(
        qq.data_ptr(), kk.data_ptr(), vv.data_ptr(), kk.stride(0), kk.stride(1), vv.stride(0),
        vv.stride(1), lists.data_ptr(), lengths.data_ptr(), L, lists.shape[1], hq, hkv, D, T,
        float(scale), parts, waves, out.data_ptr(), _stream(qq.device)))
    return out.unsqueeze(0)


QW_MASK_BOOL = 3


def _mask_args(mask, hq: int, L: int, T: int):
    """(pointer, dtype code, head stride, row stride, tensor kept alive) of a
    mask broadcastable to [1, hq, L, T]: bool / uint8 (nonzero attends) or an
    additive f16 / bf16 / f32 mask."""
    if mask is None:
        return None, 0, 0, 0, None
    torch = _torch()
    m = mask
    while m.dim() > 3:
        if m.shape[0] != 1:
            raise QwError(1, "mask: batch must be 1")
        m = m[0]
    if m.dim() == 2:
        m = m.unsqueeze(0)
    if m.dim() != 3 or m.shape[0] not in (1, hq) or m.shape[1] != L or m.shape[2] != T:
        raise QwError(1, f"mask: shape {tuple(mask.shape)} does not broadcast to [1, {hq}, {L}, {T}]")
    if not m.is_cuda:
        raise QwError(1, "mask: device tensor expected")
    codes = {torch.float16: 0, torch.bfloat16: 1, torch.float32: 2, torch.bool: QW_MASK_BOOL,
             torch.uint8: QW_MASK_BOOL}
    if m.dtype not in codes:
        raise QwError(1, f"mask: bool or f16/bf16/f32 expected, got {m.dtype}")
    if m.stride(2) != 1:
        m = m.contiguous()
    hs = 0 if m.shape[0] == 1 else m.stride(0)
    return m.data_ptr(), codes[m.dtype], hs, m.stride(1), m


def attention(q, k, v, scale: float, mask=None, softcap: float = 0.0, window: int = 0,
              causal: bool = False):
    """``layers::attention(q, k, v, scale, mask, softcap, window)`` (layers.rs:4010)
    over fp16 K/V [1, Hkv, T, D] (any head/row strides); ``causal`` and
    ``window`` give ``causal_attention``'s masks (lib.rs:3185)."""
    torch = _torch()
    qq = _as3(q, "q")
    kk, vv = _kv_view(k, "k"), _kv_view(v, "v")
    if kk.shape != vv.shape or kk.shape[2] != qq.shape[2]:
        raise QwError(1, "attention: k/v shapes disagree with q")
    hq, L, D = qq.shape
    hkv, T, _ = kk.shape
    m, md, mhs, mrs, _keep = _mask_args(mask, hq, L, T)
    out = torch.empty_like(qq)
    _check(lib().qw_sdpa(qq.data_ptr(), hq, L, kk.data_ptr(), vv.data_ptr(), hkv, T, D,
                         kk.stride(0), kk.stride(1), vv.stride(0), vv.stride(1), float(scale),
                         int(causal), int(window), float(softcap), m, md, mhs, mrs,
                         out.data_ptr(), _stream(qq.device)))
    return out.unsqueeze(0)


def causal_attention(q, k, v, scale: float, softcap: float = 0.0, window: int = 0):
    """``causal_attention(q, k, v, scale, softcap, window)`` (lib.rs:3185):
    bottom-right causal, with the sliding window when ``window`` > 0."""
    return attention(q, k, v, scale, None, softcap, window, True)


def sparse_attention(q, k, v, lists, lengths, scale: float):
    """D-LSA gathered read with the automatic launch policy (dlsa_attention.rs:31)."""
    return sparse_attention_with(q, k, v, lists, lengths, scale, 0, 0)


def _dtype_code(t, name: str) -> int:
    torch = _torch()
    codes = {torch.float16: 0, torch.bfloat16: 1, torch.float32: 2}
    if t.dtype not in codes:
        raise QwError(1, f"{name}: f16/bf16/f32 expected, got {t.dtype}")
    return codes[t.dtype]


def sparse_attention_typed(q, k, v, lists, lengths, scale: float, parts: int = 0,
                           waves: int = 0):
    """The D-LSA read over the reference's whole dtype and head-dim contract
    (mlx_cxx_dlsa_attention.cpp:429-470): q f16/bf16/f32, K and V alike in one
    of the three, head_dim 32..256, at most 8 query heads a KV head; the output
    has q's dtype (dlsa_attention.rs:5-9). fp32 arithmetic throughout."""
    torch = _torch()

    def as3(t, name, any_stride=False):
        if t.dim() == 4:
            if t.shape[0] != 1:
                raise QwError(1, f"{name}: batch must be 1")
            t = t[0]
        if t.dim() != 3 or not t.is_cuda:
            raise QwError(1, f"{name}: device tensor [1, H, L, D] expected")
        return t if (any_stride and t.stride(2) == 1) else t.contiguous()

    qq = as3(q, "q")
    kk, vv = as3(k, "k", True), as3(v, "v", True)
    qd, kd = _dtype_code(qq, "q"), _dtype_code(kk, "k")
    if vv.dtype != kk.dtype:
        raise QwError(1, "sparse_attention: k and v must share a dtype")
    if kk.shape != vv.shape or kk.shape[2] != qq.shape[2]:
        raise QwError(1, "sparse_attention: k/v shapes disagree with q")
    if lists.dim() != 2 or lists.dtype != torch.int32 or lengths.dim() != 1 or \
            lengths.dtype != torch.int32 or lists.shape[0] != qq.shape[1] or \
            lengths.shape[0] != qq.shape[1]:
        raise QwError(1, "sparse_attention: lists [L,W] i32 and lengths [L] i32 expected")
    lists = lists.contiguous()
    lengths = lengths.contiguous()
    out = torch.empty_like(qq)
    hq, L, D = qq.shape
    hkv, T, _ = kk.shape
    _check(lib().qw_dlsa_sparse_attention_typed(
        qq.data_ptr(), qd, kk.data_ptr(), vv.data_ptr(), kd, kk.stride(0), kk.stride(1),
        vv.stride(0), vv.stride(1), lists.data_ptr(), lengths.data_ptr(), L, lists.shape[1], hq,
        hkv, D, T, float(scale), parts, waves, out.data_ptr(), _stream(qq.device)))
    return out.unsqueeze(0)


# ------------------------------------------------------------ D-LSA K1 select

DLSA_SELECT_STATUS_NAN = 1
DLSA_SELECT_STATUS_SHORT_SCORES = 2
DLSA_TOP_P_MAX = 2048


class DlsaSelectParams:
    """The flat-design knobs the select reads (dlsa_kernels.rs:24-38)."""

    def __init__(self, window: int, sink: int, top_k: int, top_p: int, bucket_cap: int,
                 buckets_per_block: int):
        self.window, self.sink, self.top_k, self.top_p = window, sink, top_k, top_p
        self.bucket_cap, self.buckets_per_block = bucket_cap, buckets_per_block

    def list_width(self) -> int:
        return self.top_k + self.window + self.sink


def dlsa_select_with(scores, members, positions, total_rows: int, params: DlsaSelectParams,
                     threads: int = 0):
    """D-LSA K1 on the device (dlsa_kernels.rs:88 ``dlsa_select_with``): scores
    ``[R, S]`` f32, members ``[N, bucket_cap]`` i32, positions ``[R]`` i32.
    Returns ``(lists [R, top_k+window+sink], lengths [R], picked [R, top_p],
    status [R])``, all int32 device tensors."""
    torch = _torch()
    if scores.dim() != 2 or scores.dtype != torch.float32 or not scores.is_cuda:
        raise QwError(1, "dlsa_select: scores must be a [R, S] f32 device tensor")
    if members.dim() != 2 or members.dtype != torch.int32 or not members.is_cuda:
        raise QwError(1, "dlsa_select: members must be a [N, cap] i32 device tensor")
    if positions.dim() != 1 or positions.dtype != torch.int32 or \
            positions.shape[0] != scores.shape[0]:
        raise QwError(1, "dlsa_select: positions must be [R] i32")
    if members.shape[1] != params.bucket_cap:
        raise QwError(1, "dlsa_select: members width differs from bucket_cap")
    sc, mb, pos = scores.contiguous(), members.contiguous(), positions.contiguous()
    R = sc.shape[0]
    dev = sc.device
    lists = torch.empty((R, params.list_width()), dtype=torch.int32, device=dev)
    lengths = torch.empty((R,), dtype=torch.int32, device=dev)
    picked = torch.empty((R, params.top_p), dtype=torch.int32, device=dev)
    status = torch.empty((R,), dtype=torch.int32, device=dev)
    _check(lib().qw_dlsa_select(sc.data_ptr(), sc.shape[1], mb.data_ptr(), mb.shape[0],
                                params.bucket_cap, pos.data_ptr(), R, total_rows, params.window,
                                params.sink, params.top_k, params.top_p,
                                params.buckets_per_block, threads, lists.data_ptr(),
                                lengths.data_ptr(), picked.data_ptr(), status.data_ptr(),
                                _stream(dev)))
    return lists, lengths, picked, status


def dlsa_select(scores, members, positions, total_rows: int, params: DlsaSelectParams):
    """D-LSA K1 with the automatic workgroup size (dlsa_kernels.rs:73)."""
    return dlsa_select_with(scores, members, positions, total_rows, params, 0)



def fused_rope_qk_append(qkv, n_q_heads: int, n_kv_heads: int, head_dim: int, rope_dims: int,
                         rope_base: float, rope_scale: float = 1.0, traditional: bool = False,
                         positions_base: int = 0, dest_layout: int = 0):
    """q/k RoPE + append-layout relayout out of the fused QKV projection
    (reference ``fused_rope_qk_append``, lib.rs:1462; kernel
    fused_rope_append.cpp:80-180). ``qkv`` [B, L, (Hq + 2 Hkv) D] fp16 on the
    device. Returns (q [B, Hq, L, D], k, v) with k / v [B, Hkv, L, D]
    (dest_layout 0) or [B, L, Hkv, D] (dest_layout 1); q and k rotated."""
    torch = _torch()
    if qkv.dim() != 3 or qkv.dtype != torch.float16 or not qkv.is_cuda:
        raise QwError(1, "fused_rope_qk_append: qkv must be [B, L, W] fp16 on the device")
    x = qkv.contiguous()
    B, L, W = x.shape
    if W != (n_q_heads + 2 * n_kv_heads) * head_dim:
        raise QwError(1, "fused_rope_qk_append: qkv trailing dim does not match the head geometry")
    q = torch.empty((B, n_q_heads, L, head_dim), dtype=torch.float16, device=x.device)
    kv_shape = (B, n_kv_heads, L, head_dim) if dest_layout == 0 else (B, L, n_kv_heads, head_dim)
    k = torch.empty(kv_shape, dtype=torch.float16, device=x.device)
    v = torch.empty_like(k)
    _check(lib().qw_fused_rope_qk_append(x.data_ptr(), B, L, n_q_heads, n_kv_heads, head_dim,
                                         rope_dims, float(rope_base), float(rope_scale),
                                         int(traditional), positions_base, dest_layout,
                                         q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                         _stream(x.device)))
    return q, k, v


def turbo4_codebook(bits: int, head_dim: int):
    """The 2^bits Lloyd-Max centroids for N(0, 1/head_dim) the library builds
    (reference ``optimal_centroids``, turbo/codebook.rs:139), float32 numpy."""
    import numpy as np

    out = np.zeros(1 << bits, np.float32)
    _check(lib().qw_turbo4_codebook(bits, head_dim, out.ctypes.data))
    return out


def turbo4_signs(length: int, seed: int):
    """The +-1 LCG sign vector (reference ``generate_signs``, turbo/quant.rs:217)."""
    import numpy as np

    out = np.zeros(length, np.float32)
    _check(lib().qw_turbo4_signs(length, seed & 0xFFFFFFFF, out.ctypes.data))
    return out
