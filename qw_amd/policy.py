"""KV-cache mode policy of the model runtime (reference qwen3_5.rs:53, :929-986).

A cache configured for a quantized mode prefills in fp16 and is quantized once,
when the longest cache passes a threshold: at the end of the initial prefill,
or before the first forward that would carry it past the threshold. The
reference applies this to Turbo4; here it applies to Turbo4 and, in Turbo4's
place, to the affine modes, and the quantization is
``KVCache.demote_fp16_to_affine(configured)`` (for Turbo4 the reference's own
``demote_fp16_to_turbo4``). Int8 and fp16 caches start in their own mode.
Caches other than attention KV caches (the linear-attention state of hybrid
models) are passed through untouched.
"""
from __future__ import annotations

from typing import Iterable

from . import KVCacheMode

# qwen3_5.rs:53 TURBO4_PACKED_MTP_THRESHOLD_TOKENS
QUANTIZE_THRESHOLD_TOKENS = 2048


def _is_quantized(mode: int) -> bool:
    return mode in (KVCacheMode.TURBO4, KVCacheMode.AFFINE4, KVCacheMode.AFFINE8)


def _attention_caches(caches: Iterable):
    return [c for c in caches if hasattr(c, "demote_fp16_to_affine")]


def _offset(cache) -> int:
    return int(getattr(cache, "offset", 0))


def initial_attention_cache_mode(configured: int) -> int:
    """qwen3_5.rs:933 initial_attention_cache_mode: quantized modes start in fp16."""
    return KVCacheMode.FP16 if _is_quantized(configured) else configured


def demote_populated_attention_caches(caches: Iterable, configured: int) -> int:
    """qwen3_5.rs:947: every populated fp16 attention cache becomes `configured`.
    Returns how many were demoted."""
    n = 0
    for cache in _attention_caches(caches):
        if cache.mode == KVCacheMode.FP16 and cache.offset > 0:
            demoted = cache.demote_fp16_to_affine(configured)
            assert demoted, "populated fp16 cache must demote"
            n += 1
    return n


def finish_initial_attention_prefill(caches, configured: int) -> int:
    """qwen3_5.rs:959: after the initial prefill, demote once the longest cache
    is past the threshold."""
    caches = list(caches)
    longest = max((_offset(c) for c in caches), default=0)
    if _is_quantized(configured) and longest > QUANTIZE_THRESHOLD_TOKENS:
        return demote_populated_attention_caches(caches, configured)
    return 0


def prepare_attention_forward(caches, configured: int, input_len: int,
                              initial_prefill_complete: bool) -> int:
    """qwen3_5.rs:968: before a forward of `input_len` rows, demote when the
    longest cache would pass the threshold."""
    if not _is_quantized(configured) or not initial_prefill_complete:
        return 0
    caches = list(caches)
    projected = max((_offset(c) for c in caches), default=0) + input_len
    if projected > QUANTIZE_THRESHOLD_TOKENS:
        return demote_populated_attention_caches(caches, configured)
    return 0
