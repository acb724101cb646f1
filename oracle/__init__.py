"""CPU oracle for the full-attention hot path (TEST INFRASTRUCTURE ONLY).

This package is the parity checker and the reported CPU baseline. Only
``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg
may import it; the product (``qw_amd`` / ``libqwattn.so``) never does.

It wraps ``libqw_oracle.so`` (``qw_oracle.c``, a C restatement of the
reference's MLX semantics) with numpy-facing helpers. Array conventions follow
the reference's tensors with the batch dimension of 1 dropped:
q ``[Hq, L, D]``, k/v ``[Hkv, T, D]``, out ``[Hq, L, D]``.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libqw_oracle.so")
_lib = None


def build() -> str:
    """Compile ``libqw_oracle.so`` with the committed Makefile."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        _declare(_lib)
    return _lib


_p = ctypes.c_void_p
_i32 = ctypes.c_int
_i64 = ctypes.c_int64
_f32 = ctypes.c_float
_f64 = ctypes.c_double


def _declare(L: ctypes.CDLL) -> None:
    L.qwo_f32_to_f16.restype = ctypes.c_uint16
    L.qwo_f32_to_f16.argtypes = [_f32]
    L.qwo_f16_to_f32.restype = _f32
    L.qwo_f16_to_f32.argtypes = [ctypes.c_uint16]
    L.qwo_f32_to_f16_array.argtypes = [_p, _p, _i64]
    L.qwo_f16_to_f32_array.argtypes = [_p, _p, _i64]
    L.qwo_affine_quantize.restype = _i32
    L.qwo_affine_quantize.argtypes = [_p, _i64, _i32, _i32, _i32, _p, _p, _p]
    L.qwo_affine_dequantize.restype = _i32
    L.qwo_affine_dequantize.argtypes = [_p, _p, _p, _i64, _i32, _i32, _i32, _p]
    L.qwo_int8_quantize.restype = _i32
    L.qwo_int8_quantize.argtypes = [_p, _i64, _i32, _p, _p]
    L.qwo_int8_dequantize.restype = _i32
    L.qwo_int8_dequantize.argtypes = [_p, _p, _i64, _i32, _p]
    L.qwo_sdpa_mlx_f16.restype = _i32
    L.qwo_sdpa_mlx_f16.argtypes = [_p, _p, _p, _i32, _i32, _i32, _i32, _i32, _f32, _p, _p, _i32]
    L.qwo_sdpa_f64.restype = _i32
    L.qwo_sdpa_f64.argtypes = [_p, _p, _p, _i32, _i32, _i32, _i32, _i32, _f64, _p, _p, _i32]
    L.qwo_dlsa_attention.restype = _i32
    L.qwo_dlsa_attention.argtypes = [_p, _p, _p, _i64, _i64, _i64, _i64, _p, _p,
                                     _i32, _i32, _i32, _i32, _i32, _i32, _f32, _p, _i32]
    L.qwo_affine_layer_call.restype = _i32
    L.qwo_affine_layer_call.argtypes = [_p, _p, _p, _p, _p, _p, _i64, _i32, _p, _p, _p,
                                        _i32, _i32, _i32, _i32, _i32, _i32, _f32, _i32,
                                        _p, _i32, _p, _i32]


def _ptr(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _c(a: np.ndarray, dtype) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=dtype)


def default_threads() -> int:
    return max(1, os.cpu_count() or 1)


def _check(rc: int, what: str) -> None:
    if rc != 0:
        raise ValueError(f"oracle {what}: bad arguments (rc={rc})")


# ------------------------------------------------------------------ fp16

def f32_to_f16(x: np.ndarray) -> np.ndarray:
    x = _c(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().qwo_f32_to_f16_array(_ptr(x), _ptr(out), x.size)
    return out.view(np.float16)


def f16_to_f32(x: np.ndarray) -> np.ndarray:
    x = _c(np.asarray(x, np.float16).view(np.uint16), np.uint16)
    out = np.empty(x.shape, np.float32)
    lib().qwo_f16_to_f32_array(_ptr(x), _ptr(out), x.size)
    return out


# ----------------------------------------------------------- affine codec

def affine_quantize(w: np.ndarray, bits: int, group: int = 64):
    """MLX affine quantize of fp16 rows ``w[..., dim]``.

    Returns ``(codes uint32 [..., dim*bits/32], scales f16 [..., dim/group],
    biases f16 [..., dim/group])``.
    """
    w = _c(w, np.float16)
    dim = w.shape[-1]
    rows = int(np.prod(w.shape[:-1])) if w.ndim > 1 else 1
    codes = np.empty(w.shape[:-1] + (dim * bits // 32,), np.uint32)
    scales = np.empty(w.shape[:-1] + (dim // group,), np.float16)
    biases = np.empty_like(scales)
    _check(lib().qwo_affine_quantize(_ptr(w), rows, dim, group, bits, _ptr(codes),
                                     _ptr(scales), _ptr(biases)), "affine_quantize")
    return codes, scales, biases


def affine_dequantize(codes: np.ndarray, scales: np.ndarray, biases: np.ndarray,
                      bits: int, group: int = 64) -> np.ndarray:
    codes = _c(codes, np.uint32)
    scales = _c(scales, np.float16)
    biases = _c(biases, np.float16)
    dim = codes.shape[-1] * 32 // bits
    rows = int(np.prod(codes.shape[:-1])) if codes.ndim > 1 else 1
    out = np.empty(codes.shape[:-1] + (dim,), np.float16)
    _check(lib().qwo_affine_dequantize(_ptr(codes), _ptr(scales), _ptr(biases), rows, dim,
                                       group, bits, _ptr(out)), "affine_dequantize")
    return out


# ------------------------------------------------------------ Int8 codec

def int8_quantize(w: np.ndarray):
    """quantize_per_token of fp16 rows ``w[..., dim]``: (codes int8 [..., dim],
    scales f16 [...])."""
    w = _c(w, np.float16)
    dim = w.shape[-1]
    rows = int(np.prod(w.shape[:-1])) if w.ndim > 1 else 1
    codes = np.empty(w.shape, np.int8)
    scales = np.empty(w.shape[:-1], np.float16)
    _check(lib().qwo_int8_quantize(_ptr(w), rows, dim, _ptr(codes), _ptr(scales)),
           "int8_quantize")
    return codes, scales


def int8_dequantize(codes: np.ndarray, scales: np.ndarray) -> np.ndarray:
    codes = _c(codes, np.int8)
    scales = _c(scales, np.float16)
    dim = codes.shape[-1]
    rows = int(np.prod(codes.shape[:-1])) if codes.ndim > 1 else 1
    out = np.empty(codes.shape, np.float16)
    _check(lib().qwo_int8_dequantize(_ptr(codes), _ptr(scales), rows, dim, _ptr(out)),
           "int8_dequantize")
    return out


# ------------------------------------------------------------------ SDPA

def _pos(q_pos, L):
    if q_pos is None:
        return None
    q_pos = _c(q_pos, np.int32)
    assert q_pos.shape == (L,)
    return q_pos


def causal_positions(L: int, T: int) -> np.ndarray:
    """Bottom-right causal positions: row r sees keys t <= T - L + r."""
    return np.arange(T - L, T, dtype=np.int32)


def sdpa_mlx_f16(q, k, v, scale: float, q_pos=None, threads: int | None = None):
    """MLX CPU-stream SDPA with its fp16 roundings. q [Hq,L,D], k/v [Hkv,T,D]."""
    q, k, v = _c(q, np.float16), _c(k, np.float16), _c(v, np.float16)
    hq, L, D = q.shape
    hkv, T, _ = k.shape
    pos = _pos(q_pos, L)
    out = np.empty((hq, L, D), np.float16)
    _check(lib().qwo_sdpa_mlx_f16(_ptr(q), _ptr(k), _ptr(v), hq, hkv, L, T, D, scale,
                                  _ptr(pos), _ptr(out), threads or default_threads()),
           "sdpa_mlx_f16")
    return out


def sdpa_f64(q, k, v, scale: float, q_pos=None, threads: int | None = None):
    """Closed-form softmax attention in fp64 (no intermediate rounding)."""
    q, k, v = _c(q, np.float16), _c(k, np.float16), _c(v, np.float16)
    hq, L, D = q.shape
    hkv, T, _ = k.shape
    pos = _pos(q_pos, L)
    out = np.empty((hq, L, D), np.float64)
    _check(lib().qwo_sdpa_f64(_ptr(q), _ptr(k), _ptr(v), hq, hkv, L, T, D, float(scale),
                              _ptr(pos), _ptr(out), threads or default_threads()), "sdpa_f64")
    return out


def sdpa_general(q, k, v, scale: float, causal: bool = False, window: int = 0,
                 softcap: float = 0.0, mask=None) -> np.ndarray:
    """Attention with the reference's general options (numpy): layers::attention
    (layers.rs:4010-4060) and causal_attention (lib.rs:3185-3275) reduce to
    MLX's SDPA with an array mask, or with softcap to the composite of
    mlx_cxx_bridge.cpp:1573-1590.

    q [Hq, L, D] fp16, k / v [Hkv, T, D] fp16. Position of row r:
    p = T - L + r. causal keeps keys t <= p; window > 0 also t >= p - window + 1
    (create_causal_mask_with_window, utils.rs:95-140). mask broadcastable to
    [Hq, L, T]: bool / uint8 keeps the scores where nonzero; a float mask is
    cast to fp16 (mlx_cxx_bridge.cpp:3466-3497) and added.
      softcap == 0: S = f16(f16(f16(scale) q) . k); S = f16(S + mask);
        P = f16(softmax_fp32(S)); out = f16(P . V).
      softcap > 0: S = f16(q . k); s = tanh(S scale / cap) cap, + mask, in
        fp32; P = softmax_fp32(s) (not rounded); out = f16(P . V).
    Dot products and P . V accumulate in fp64 (MLX accumulates in fp32; the
    two differ only at fp16 rounding ties of S). A row with no visible key is
    zeros. Returns fp16 [Hq, L, D]."""
    q = np.asarray(q, np.float16)
    k = np.asarray(k, np.float16)
    v = np.asarray(v, np.float16)
    hq, L, D = q.shape
    hkv, T, _ = k.shape
    G = hq // hkv
    kk = np.repeat(k.astype(np.float64), G, axis=0)
    vv = np.repeat(v.astype(np.float64), G, axis=0)
    t = np.arange(T)
    p = T - L + np.arange(L)
    vis = np.ones((L, T), bool)
    if causal:
        vis &= t[None, :] <= p[:, None]
    if window > 0:
        vis &= t[None, :] >= (p - window + 1)[:, None]
    vis = np.broadcast_to(vis, (hq, L, T)).copy()
    add = None
    if mask is not None:
        m = np.asarray(mask)
        m = np.broadcast_to(m.reshape((-1, L, T)), (hq, L, T))
        if m.dtype == np.bool_ or m.dtype == np.uint8:
            vis &= m != 0
        else:
            add = m.astype(np.float16).astype(np.float32)
    if softcap <= 0:
        sh = np.float32(np.float16(scale))
        qs = (sh * q.astype(np.float32)).astype(np.float16).astype(np.float64)
        s = np.matmul(qs, kk.transpose(0, 2, 1)).astype(np.float16).astype(np.float32)
        if add is not None:
            s = (s + add).astype(np.float16).astype(np.float32)
    else:
        S = np.matmul(q.astype(np.float64), kk.transpose(0, 2, 1)).astype(np.float16)
        s = S.astype(np.float32) * np.float32(scale)
        s = np.tanh(s / np.float32(softcap)).astype(np.float32) * np.float32(softcap)
        if add is not None:
            s = s + add
    s = np.where(vis, s, np.float32(-np.inf)).astype(np.float32)
    mx = s.max(axis=-1, keepdims=True)
    any_vis = np.isfinite(mx)
    e = np.exp(s - np.where(any_vis, mx, np.float32(0.0))).astype(np.float32)
    den = e.sum(axis=-1, keepdims=True, dtype=np.float32)
    P = np.where(any_vis, e / np.where(den > 0, den, np.float32(1.0)), np.float32(0.0))
    if softcap <= 0:
        P = P.astype(np.float16)
    return np.matmul(P.astype(np.float64), vv).astype(np.float16)


def dlsa_attention_f64(q, k, v, lists, lengths, scale: float):
    """The K2 contract in fp64 for inputs of any float dtype (numpy; the
    reference's own host check, dlsa_attention.rs:140-170): for row r and
    head h, the valid entries p of lists[r, :lengths[r]] (0 <= p < T) give
    s_p = scale * q[h, r] . k[h / G, p] and out = sum_p softmax(s)_p v[h / G, p];
    a row without a valid entry is zeros. q [Hq,L,D]; k, v [Hkv,T,D];
    returns fp64 [Hq,L,D]."""
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    lists = np.asarray(lists, np.int64)
    lengths = np.asarray(lengths, np.int64)
    hq, L, D = q.shape
    hkv, T, _ = k.shape
    G = hq // hkv
    out = np.zeros((hq, L, D))
    for r in range(L):
        lst = lists[r, :max(0, min(int(lengths[r]), lists.shape[1]))]
        lst = lst[(lst >= 0) & (lst < T)]
        if lst.size == 0:
            continue
        for h in range(hq):
            kh = k[h // G, lst]
            s = (kh @ q[h, r]) * float(scale)
            w = np.exp(s - s.max())
            out[h, r] = (w @ v[h // G, lst]) / w.sum()
    return out


def dlsa_attention(q, k, v, lists, lengths, scale: float, threads: int | None = None):
    """D-LSA gathered read (K2 contract). q [Hq,L,D] f16; k/v [Hkv,T,D] f16
    (any element strides with a unit last stride); lists [L,W] i32;
    lengths [L] i32. Returns fp32 [Hq,L,D]."""
    q = _c(q, np.float16)
    k = np.asarray(k, np.float16)
    v = np.asarray(v, np.float16)
    if k.strides[-1] != 2:
        k = np.ascontiguousarray(k)
    if v.strides[-1] != 2:
        v = np.ascontiguousarray(v)
    lists, lengths = _c(lists, np.int32), _c(lengths, np.int32)
    hq, L, D = q.shape
    hkv, T, _ = k.shape
    W = lists.shape[1]
    out = np.empty((hq, L, D), np.float32)
    _check(lib().qwo_dlsa_attention(
        _ptr(q), k.ctypes.data_as(ctypes.c_void_p), v.ctypes.data_as(ctypes.c_void_p),
        k.strides[0] // 2, k.strides[1] // 2, v.strides[0] // 2, v.strides[1] // 2,
        _ptr(lists), _ptr(lengths), L, W, hq, hkv, D, T, scale, _ptr(out),
        threads or default_threads()), "dlsa_attention")
    return out


# ------------------------------------------------------ quantized layer call

class Int8CacheOracle:
    """Host-side Int8 KV cache (keys/values int8 [Hkv, cap, D], key/value
    scales f16 [Hkv, cap]); attention is the reference's: fetch (dequantize
    the visible cache, a6) then the MLX SDPA restatement."""

    def __init__(self, n_kv_heads: int, head_dim: int, capacity: int):
        self.hkv, self.D, self.cap = n_kv_heads, head_dim, capacity
        self.keys = np.zeros((n_kv_heads, capacity, head_dim), np.int8)
        self.values = np.zeros_like(self.keys)
        self.key_scales = np.zeros((n_kv_heads, capacity), np.float16)
        self.val_scales = np.zeros_like(self.key_scales)
        self.offset = 0

    def update(self, k_new: np.ndarray, v_new: np.ndarray) -> None:
        L = k_new.shape[1]
        assert self.offset + L <= self.cap
        sl = slice(self.offset, self.offset + L)
        self.keys[:, sl], self.key_scales[:, sl] = int8_quantize(k_new)
        self.values[:, sl], self.val_scales[:, sl] = int8_quantize(v_new)
        self.offset += L

    def fetch(self):
        T = self.offset
        return (int8_dequantize(self.keys[:, :T], self.key_scales[:, :T]),
                int8_dequantize(self.values[:, :T], self.val_scales[:, :T]))

    def update_and_attention(self, q, k_new, v_new, scale: float, causal: bool,
                             rows=None, threads: int | None = None) -> np.ndarray:
        L = q.shape[1]
        self.update(k_new, v_new)
        k, v = self.fetch()
        sel = np.arange(L) if rows is None else np.asarray(rows)
        pos = causal_positions(L, self.offset)[sel] if causal else None
        return sdpa_mlx_f16(np.ascontiguousarray(q[:, sel]), k, v, scale,
                            q_pos=None if pos is None else np.ascontiguousarray(pos),
                            threads=threads)

class AffineCacheOracle:
    """Host-side quantized KV cache in the reference's layout (row-major codes,
    separate fp16 scale and bias planes), used to restate one layer call."""

    def __init__(self, n_kv_heads: int, head_dim: int, capacity: int, bits: int,
                 group: int = 64):
        self.hkv, self.D, self.cap, self.bits, self.group = n_kv_heads, head_dim, capacity, bits, group
        wpr, gpr = head_dim * bits // 32, head_dim // group
        self.k_codes = np.zeros((n_kv_heads, capacity, wpr), np.uint32)
        self.v_codes = np.zeros_like(self.k_codes)
        self.k_scales = np.zeros((n_kv_heads, capacity, gpr), np.float16)
        self.k_biases = np.zeros_like(self.k_scales)
        self.v_scales = np.zeros_like(self.k_scales)
        self.v_biases = np.zeros_like(self.k_scales)
        self.offset = 0

    def update(self, k_new: np.ndarray, v_new: np.ndarray) -> None:
        """Quantize-on-append of [Hkv, L, D] fp16 rows."""
        L = k_new.shape[1]
        assert self.offset + L <= self.cap
        for name, src in (("k", k_new), ("v", v_new)):
            c, s, b = affine_quantize(src, self.bits, self.group)
            getattr(self, name + "_codes")[:, self.offset:self.offset + L] = c
            getattr(self, name + "_scales")[:, self.offset:self.offset + L] = s
            getattr(self, name + "_biases")[:, self.offset:self.offset + L] = b
        self.offset += L

    def fetch(self):
        """Dequantized visible K and V, [Hkv, offset, D] fp16 (update_and_fetch)."""
        T = self.offset
        k = affine_dequantize(self.k_codes[:, :T], self.k_scales[:, :T], self.k_biases[:, :T],
                              self.bits, self.group)
        v = affine_dequantize(self.v_codes[:, :T], self.v_scales[:, :T], self.v_biases[:, :T],
                              self.bits, self.group)
        return k, v

    def update_and_attention(self, q, k_new, v_new, scale: float, causal: bool,
                             rows=None, threads: int | None = None) -> np.ndarray:
        """Append then attend, in C (quantize, MLX dequantize, MLX SDPA).
        ``rows`` restricts the computed query rows (attention rows are
        independent, so a subset is exact)."""
        q = _c(q, np.float16)
        k_new, v_new = _c(k_new, np.float16), _c(v_new, np.float16)
        hq, L, D = q.shape
        assert self.offset + L <= self.cap
        sel = None if rows is None else _c(rows, np.int32)
        n_sel = 0 if sel is None else sel.size
        out = np.empty((hq, n_sel or L, D), np.float16)
        _check(lib().qwo_affine_layer_call(
            _ptr(self.k_codes), _ptr(self.k_scales), _ptr(self.k_biases), _ptr(self.v_codes),
            _ptr(self.v_scales), _ptr(self.v_biases), self.cap, self.offset, _ptr(q),
            _ptr(k_new), _ptr(v_new), hq, self.hkv, L, D, self.group, self.bits, scale,
            1 if causal else 0, _ptr(sel), n_sel, _ptr(out), threads or default_threads()),
            "affine_layer_call")
        self.offset += L
        return out


# ------------------------------------------------------------ D-LSA K1 select

SELECT_STATUS_NAN = 1
SELECT_STATUS_SHORT_SCORES = 2


def dlsa_select(scores: np.ndarray, members: np.ndarray, positions: np.ndarray,
                total_rows: int, window: int, sink: int, top_k: int, top_p: int,
                buckets_per_block: int):
    """Read lists from bucket scores (crates/runtime/src/dlsa/select.rs:65-115,
    the device contract of crates/mlxcel-core/src/dlsa_kernels.rs:57-84).

    scores ``[R, S]`` f32, members ``[N, cap]`` i32 (ascending, -1 padded),
    positions ``[R]``. Row r ranks its first ``min(floor(p / window) * m,
    total_rows)`` columns (clipped to S, with status bit 2): score descending,
    -0 == +0, a NaN below every number (status bit 1), ties to the lower
    bucket; keeps the best ``top_p``; the list is the picked buckets' members
    in ``[sink, window_start)`` (pick order, members ascending, at most
    ``top_k``), then the window ``[window_start, p]``, then the sinks
    ``[0, min(sink, window_start, p + 1))``, -1 padded.
    Returns (lists [R, top_k+window+sink], lengths [R], picked [R, top_p],
    status [R]), all int32."""
    scores = np.asarray(scores, np.float32)
    members = np.asarray(members, np.int32)
    R = len(positions)
    S = scores.shape[1] if scores.ndim == 2 else 0
    cap = members.shape[1] if members.ndim == 2 else 0
    width = top_k + window + sink
    lists = np.full((R, width), -1, np.int32)
    lengths = np.zeros(R, np.int32)
    picked = np.full((R, top_p), -1, np.int32)
    status = np.zeros(R, np.int32)
    for r in range(R):
        p = int(positions[r])
        v = min(p // window * buckets_per_block, total_rows)
        if v > S:
            v = S
            status[r] |= SELECT_STATUS_SHORT_SCORES
        row = scores[r, :v]
        nan = np.isnan(row)
        if nan.any():
            status[r] |= SELECT_STATUS_NAN
        neg = np.where(nan, 0.0, -row.astype(np.float64))
        neg = np.where(neg == 0.0, 0.0, neg)  # -0 == +0
        order = np.lexsort((np.arange(v), neg, nan.astype(np.int8)))[:top_p]
        picked[r, :len(order)] = order
        ws = max(0, p + 1 - window)
        out = []
        for b in order:
            for x in members[b, :cap]:
                if x >= 0 and sink <= x < ws:
                    if len(out) == top_k:
                        break
                    out.append(int(x))
            if len(out) == top_k:
                break
        out.extend(range(ws, p + 1))
        out.extend(range(min(sink, ws, p + 1)))
        lists[r, :len(out)] = out
        lengths[r] = len(out)
    return lists, lengths, picked, status


# ------------------------------------------------- fused q/k RoPE + append

def rope_theta(rope_dims: int, positions, base: float, scale: float = 1.0) -> np.ndarray:
    """Angles [len(positions), rope_dims/2] as the reference forms them, all in
    fp32 (crates/mlx-cpp/turbo/fused_rope_append.cpp:163-168, host log2 at
    :435-441): inv_freq = exp2(-(p / (R/2)) * log2(base)),
    theta = (scale * position) * inv_freq."""
    rhalf = rope_dims // 2
    log2b = np.float32(np.log2(np.float32(base)))
    d = np.arange(rhalf, dtype=np.float32) / np.float32(rhalf)
    inv = np.exp2(-d * log2b).astype(np.float32)
    pos = np.asarray(positions, dtype=np.float32)
    return ((np.float32(scale) * pos)[:, None] * inv[None, :]).astype(np.float32)


def rope_pairs(rope_dims: int, traditional: bool):
    """Dim indices (first, second) of each rotated pair p
    (fused_rope_append.cpp:142-151): (2p, 2p+1) traditional, else (p, p + R/2)."""
    rhalf = rope_dims // 2
    p = np.arange(rhalf)
    return (2 * p, 2 * p + 1) if traditional else (p, p + rhalf)


def rope(x: np.ndarray, rope_dims: int, traditional: bool, base: float, scale: float,
         positions) -> np.ndarray:
    """RoPE of x [..., T, D] (fp16 or wider) at the given per-row positions,
    returned unrounded in float64 from the fp32 angles of ``rope_theta``:
    r1 = x1 cos - x2 sin, r2 = x1 sin + x2 cos on each pair; dims past R are
    copied (fused_rope_append.cpp:152-178)."""
    x = np.asarray(x, np.float64)
    out = x.copy()
    th = rope_theta(rope_dims, positions, base, scale).astype(np.float64)
    c, s = np.cos(th), np.sin(th)
    i1, i2 = rope_pairs(rope_dims, traditional)
    x1, x2 = x[..., i1], x[..., i2]
    out[..., i1] = x1 * c - x2 * s
    out[..., i2] = x1 * s + x2 * c
    return out


def fused_rope_qk_append(qkv: np.ndarray, hq: int, hkv: int, D: int, rope_dims: int,
                         base: float, scale: float, traditional: bool, positions_base: int,
                         dest_layout: int = 0):
    """The reference op end to end (lib.rs:1462-1476): qkv [B, L, (Hq+2Hkv) D]
    -> q [B, Hq, L, D], k / v [B, Hkv, L, D] (layout 0) or [B, L, Hkv, D]
    (layout 1), q and k rotated (float64, unrounded), v copied."""
    B, L, _ = qkv.shape
    x = np.asarray(qkv).reshape(B, L, hq + 2 * hkv, D).transpose(0, 2, 1, 3)
    pos = positions_base + np.arange(L)
    q = rope(x[:, :hq], rope_dims, traditional, base, scale, pos)
    k = rope(x[:, hq:hq + hkv], rope_dims, traditional, base, scale, pos)
    v = np.asarray(x[:, hq + hkv:], np.float64)
    if dest_layout == 1:
        k, v = k.transpose(0, 2, 1, 3), v.transpose(0, 2, 1, 3)
    return q, k, v


# ------------------------------------------------------------------ Turbo4

TURBO_DEFAULT_SEED = 0x7B470404   # crates/mlxcel-core/src/cache.rs:324
TURBO_SUB_SEED = 0x9E3779B9       # turbo/quant.rs:196 (second vector of a pair)
TURBO_K_SEED_OFFSET = 0x4B5F5345  # turbo/quant.rs:101


def turbo4_centroids(bits: int, head_dim: int) -> np.ndarray:
    """Lloyd-Max centroids for N(0, 1/head_dim), float32 (turbo/codebook.rs:
    208-361, the published turboquant_plus `optimal_centroids`): b = 1, 2 in
    closed form; b >= 3 from uniform-quantile boundaries (scipy's norm.ppf),
    100 rounds of midpoint boundaries and conditional-expectation centroids,
    in float64."""
    from scipy import stats

    d = float(head_dim)
    if bits == 1:
        c = np.sqrt(2.0 / (np.pi * d))
        return np.array([-c, c]).astype(np.float32)
    if bits == 2:
        return (np.array([-1.51, -0.453, 0.453, 1.51]) / np.sqrt(d)).astype(np.float32)
    n = 1 << bits
    sigma = 1.0 / np.sqrt(d)
    bnd = stats.norm.ppf(np.linspace(0.0, 1.0, n + 1)[1:-1], scale=sigma)

    def cond(bnd):
        lo = np.concatenate([[-np.inf], bnd]) / sigma
        hi = np.concatenate([bnd, [np.inf]]) / sigma
        prob = stats.norm.cdf(hi) - stats.norm.cdf(lo)
        prob[-1] = stats.norm.sf(lo[-1])
        return sigma * (stats.norm.pdf(lo) - stats.norm.pdf(hi)) / prob

    c = cond(bnd)
    for _ in range(100):
        c = cond((c[:-1] + c[1:]) * 0.5)
    return c.astype(np.float32)


def turbo4_boundaries(c: np.ndarray) -> np.ndarray:
    """Midpoints in float32 (codebook.rs:84-90)."""
    c = c.astype(np.float32)
    return ((c[:-1] + c[1:]) * np.float32(0.5)).astype(np.float32)


def lcg_signs(n: int, seed: int) -> np.ndarray:
    """+-1 from the 32-bit LCG x <- 1664525 x + 1013904223 (mod 2^32), a
    zero seed starting from 0xDEADBEEF; + when bit 31 of the new state is set
    (turbo/quant.rs:119-139, :217-236)."""
    s = seed & 0xFFFFFFFF or 0xDEADBEEF
    out = np.empty(n, np.float32)
    for i in range(n):
        s = (1664525 * s + 1013904223) & 0xFFFFFFFF
        out[i] = 1.0 if s >> 31 else -1.0
    return out


def turbo4_tables(head_dim: int, seed: int = TURBO_DEFAULT_SEED) -> dict:
    """The per-cache codec state (TurboQuantParams::new, turbo/quant.rs:188-214)."""
    ks = (seed + TURBO_K_SEED_OFFSET) & 0xFFFFFFFF
    cb = turbo4_centroids(4, head_dim)
    return {
        "v_s1": lcg_signs(head_dim, seed),
        "v_s2": lcg_signs(head_dim, (seed + TURBO_SUB_SEED) & 0xFFFFFFFF),
        "k_s1": lcg_signs(head_dim, ks),
        "k_s2": lcg_signs(head_dim, (ks + TURBO_SUB_SEED) & 0xFFFFFFFF),
        "cb": cb,
        "bnd": turbo4_boundaries(cb),
    }


def hadamard_orthonormal(n: int) -> np.ndarray:
    """Sylvester Walsh-Hadamard matrix / sqrt(n) (MLX hadamard_transform with
    its default scale, the reference's `wht`, ops.rs:72-111)."""
    from scipy.linalg import hadamard

    return hadamard(n).astype(np.float64) / np.sqrt(n)


def turbo4_rotate(x: np.ndarray, s1: np.ndarray, s2: np.ndarray) -> np.ndarray:
    """s2 . H . s1 along the last axis, float64."""
    H = hadamard_orthonormal(x.shape[-1])
    return ((np.asarray(x, np.float64) * s1) @ H) * s2


def turbo4_quantize(x: np.ndarray, s1: np.ndarray, s2: np.ndarray, tab: dict):
    """quantize_into_packed (turbo/quant.rs:270-440 with the pack kernel,
    mlx_cxx_kernels.cpp:186-212) in float64 on fp16 rows x [..., D]: returns
    (indices uint8 [..., D], norms f16 [...], rescale f16 [...], rotated
    float64 [..., D])."""
    x = np.asarray(x, np.float64)
    norm = np.sqrt((x * x).sum(-1))
    safe = np.where(norm > 0, norm, 1.0)
    y = turbo4_rotate(x / safe[..., None], s1, s2)
    idx = (y[..., None] > tab["bnd"].astype(np.float64)).sum(-1).astype(np.uint8)
    c = tab["cb"].astype(np.float64)[idx]
    rn = np.maximum(np.sqrt((c * c).sum(-1)), 1e-10)
    return idx, norm.astype(np.float16), (norm / rn).astype(np.float16), y


def turbo4_pack(idx: np.ndarray) -> np.ndarray:
    """Two indices a byte, low nibble = even coordinate (turbo/quant.rs:30-33)."""
    idx = np.asarray(idx, np.uint8)
    return (idx[..., 0::2] | (idx[..., 1::2] << 4)).astype(np.uint8)


def turbo4_unpack(packed: np.ndarray) -> np.ndarray:
    p = np.asarray(packed, np.uint8)
    out = np.empty(p.shape[:-1] + (2 * p.shape[-1],), np.uint8)
    out[..., 0::2] = p & 15
    out[..., 1::2] = p >> 4
    return out


def turbo4_expand_rotated(packed: np.ndarray, rescale: np.ndarray, tab: dict) -> np.ndarray:
    """f16(f32(centroid) * f32(rescale)) in the rotated basis (quant.rs:586-600,
    turbo4_delegated_sdpa.cpp:193-221): an fp32 product, then the fp16 cast."""
    c = tab["cb"].astype(np.float32)[turbo4_unpack(packed)]
    r = np.asarray(rescale, np.float16).astype(np.float32).reshape(c.shape[:-1] + (1,))
    return (c * r).astype(np.float32).astype(np.float16)


def turbo4_fetch_k(packed, k_rescale, tab) -> np.ndarray:
    """dequantize_k_turbo4 (quant.rs:676-691): expansion, then s1 . H . s2, fp16."""
    rot = turbo4_expand_rotated(packed, k_rescale, tab).astype(np.float64)
    return turbo4_rotate(rot, tab["k_s2"], tab["k_s1"]).astype(np.float16)


def turbo4_fetch_v(packed, v_norms, tab) -> np.ndarray:
    """dequantize_v_turbo4 (quant.rs:486-546): unit-normalised centroids, the
    inverse rotation, times the stored norm, fp16."""
    c = tab["cb"].astype(np.float64)[turbo4_unpack(packed)]
    u = c / np.maximum(np.sqrt((c * c).sum(-1, keepdims=True)), 1e-10)
    n = np.asarray(v_norms, np.float16).astype(np.float64).reshape(c.shape[:-1] + (1,))
    return (turbo4_rotate(u, tab["v_s2"], tab["v_s1"]) * n).astype(np.float16)


def turbo4_fused_verify(q, k_packed, k_rescale, v_packed, v_rescale, tab, scale: float,
                        q_pos) -> np.ndarray:
    """The reference's fused Turbo4 verify pass (crates/mlx-cpp/turbo/
    turbo4_attention.cpp:45-193 partial, :198-264 merge; wrapper
    cache/turbo/fused_attention.rs:119-160): q rotated into the K basis in
    fp32 (quant.rs:728-744), q' = f16(f32(q_rot * f32(scale * log2 e)))
    (turbo4_attention.cpp:67-79), K and V expanded as f16(f32(centroid) *
    f32(rescale)), then the closed form of its fp32 scores / softmax / P.V,
    here in float64, with each row r seeing keys t <= q_pos[r]; the output
    rotated back through the V basis (quant.rs:752-769) and cast to fp16.
    q [Hq, L, D] fp16; packed [Hkv, T, D/2]; rescales [Hkv, T]."""
    q = np.asarray(q, np.float16)
    hq, L, D = q.shape
    sl2e = np.float32(scale) * np.float32(1.4426950408889634)
    q_rot = turbo4_rotate(q, tab["k_s1"], tab["k_s2"]).astype(np.float32)
    qs = (q_rot * sl2e).astype(np.float32).astype(np.float16).astype(np.float64)
    k = turbo4_expand_rotated(k_packed, k_rescale, tab).astype(np.float64)
    v = turbo4_expand_rotated(v_packed, v_rescale, tab).astype(np.float64)
    hkv, T, _ = k.shape
    G = hq // hkv
    pos = np.asarray(q_pos, np.int64)
    o = np.empty((hq, L, D), np.float64)
    for h in range(hq):
        s = qs[h] @ k[h // G].T                        # [L, T], log2 domain
        s = np.where(np.arange(T)[None, :] <= pos[:, None], s, -np.inf)
        p = np.exp2(s - s.max(-1, keepdims=True))
        o[h] = (p @ v[h // G]) / p.sum(-1, keepdims=True)
    return turbo4_rotate(o, tab["v_s2"], tab["v_s1"]).astype(np.float16)


def turbo4_attention(q, k_packed, k_rescale, v_packed, v_rescale, tab, scale: float,
                     q_pos=None, threads: int | None = None) -> np.ndarray:
    """attention_turbo4_dequant_sdpa (turbo/sparse_v.rs:1051-1072): q rotated
    into the K basis and cast to fp16, rotated K/V expansions, MLX fp16 SDPA,
    the output rotated back through the V basis and cast to fp16. q [Hq, L, D];
    the packed tensors [Hkv, T, D/2], rescales [Hkv, T]."""
    q_rot = turbo4_rotate(np.asarray(q, np.float16), tab["k_s1"], tab["k_s2"]).astype(np.float16)
    k_rot = turbo4_expand_rotated(k_packed, k_rescale, tab)
    v_rot = turbo4_expand_rotated(v_packed, v_rescale, tab)
    o_rot = sdpa_mlx_f16(q_rot, k_rot, v_rot, scale, q_pos, threads)
    return turbo4_rotate(o_rot.astype(np.float64), tab["v_s2"], tab["v_s1"]).astype(np.float16)
