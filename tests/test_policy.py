"""KV-cache mode policy (qw_amd.policy), the host logic of qwen3_5.rs:929-986.

Mirrors the reference's own tests of that policy (qwen3_5.rs:3248-3620:
fresh_turbo4_attention_cache_begins_prefill_in_fp16,
short_populated_turbo4_prefill_stays_fp16, the long-prefill demotion,
threshold_crossing_demotes_once_before_target_forward,
restored_turbo4_attention_cache_is_not_demoted_again,
requested_fp16_attention_cache_stays_fp16_after_prefill) with the affine
modes in Turbo4's place. Runs on the CPU: the caches here are stand-ins that
record demotions; tests/test_gpu_kv.py checks the real demotion on a GPU.
"""
import pytest

from qw_amd import KVCacheMode
from qw_amd import policy

A4 = KVCacheMode.AFFINE4
THR = policy.QUANTIZE_THRESHOLD_TOKENS


class FakeAttentionCache:
    def __init__(self, mode, offset=0):
        self.mode = mode
        self.offset = offset
        self.demotions = 0

    def demote_fp16_to_affine(self, target):
        if self.mode != KVCacheMode.FP16 or self.offset <= 0:
            return False
        self.mode = target
        self.demotions += 1
        return True


class FakeLinearCache:
    """A hybrid model's recurrent state: has an offset, is never demoted."""

    def __init__(self, offset=0):
        self.offset = offset


def test_quantized_configuration_begins_prefill_in_fp16():
    assert policy.initial_attention_cache_mode(A4) == KVCacheMode.FP16
    assert policy.initial_attention_cache_mode(KVCacheMode.AFFINE8) == KVCacheMode.FP16
    assert policy.initial_attention_cache_mode(KVCacheMode.FP16) == KVCacheMode.FP16
    c = FakeAttentionCache(policy.initial_attention_cache_mode(A4))
    assert policy.finish_initial_attention_prefill([c], A4) == 0
    assert c.mode == KVCacheMode.FP16, "an empty initial cache must not be demoted"


def test_short_populated_prefill_stays_fp16():
    c, lin = FakeAttentionCache(KVCacheMode.FP16, 2), FakeLinearCache()
    policy.finish_initial_attention_prefill([c, lin], A4)
    assert c.mode == KVCacheMode.FP16 and c.offset == 2
    assert lin.offset == 0


def test_long_prefill_is_demoted_at_its_end():
    c = FakeAttentionCache(KVCacheMode.FP16, THR + 1)
    assert policy.finish_initial_attention_prefill([c], A4) == 1
    assert c.mode == A4 and c.offset == THR + 1


def test_prefill_exactly_at_the_threshold_stays_fp16():
    c = FakeAttentionCache(KVCacheMode.FP16, THR)
    policy.finish_initial_attention_prefill([c], A4)
    assert c.mode == KVCacheMode.FP16


def test_threshold_crossing_demotes_once_before_the_forward():
    c = FakeAttentionCache(KVCacheMode.FP16, 2)
    policy.finish_initial_attention_prefill([c], A4)
    policy.prepare_attention_forward([c], A4, THR - 2, True)  # projected == THR: not past it
    assert c.mode == KVCacheMode.FP16
    policy.prepare_attention_forward([c], A4, THR - 1, True)
    assert c.mode == A4 and c.demotions == 1
    policy.prepare_attention_forward([c], A4, THR - 1, True)
    assert c.demotions == 1, "a quantized cache is not demoted again"


def test_forward_before_the_initial_prefill_completes_never_demotes():
    c = FakeAttentionCache(KVCacheMode.FP16, 10)
    assert policy.prepare_attention_forward([c], A4, 10 * THR, False) == 0
    assert c.mode == KVCacheMode.FP16


def test_restored_quantized_cache_is_not_demoted_again():
    c = FakeAttentionCache(A4, THR + 10)
    policy.finish_initial_attention_prefill([c], A4)
    assert c.mode == A4 and c.demotions == 0


def test_requested_fp16_cache_stays_fp16():
    c = FakeAttentionCache(KVCacheMode.FP16, THR + 100)
    assert policy.finish_initial_attention_prefill([c], KVCacheMode.FP16) == 0
    assert policy.prepare_attention_forward([c], KVCacheMode.FP16, THR, True) == 0
    assert c.mode == KVCacheMode.FP16


def test_longest_cache_of_any_kind_sets_the_trigger():
    """The reference takes the max offset over all caches of the model."""
    short = FakeAttentionCache(KVCacheMode.FP16, 5)
    long_linear = FakeLinearCache(THR + 1)
    assert policy.finish_initial_attention_prefill([short, long_linear], A4) == 1
    assert short.mode == A4


def test_unpopulated_attention_caches_stay_fp16_when_others_demote():
    a, b = FakeAttentionCache(KVCacheMode.FP16, THR + 1), FakeAttentionCache(KVCacheMode.FP16, 0)
    policy.finish_initial_attention_prefill([a, b], A4)
    assert a.mode == A4 and b.mode == KVCacheMode.FP16


def test_turbo4_configuration_follows_the_reference_policy():
    """The reference's own case (qwen3_5.rs:933-986): Turbo4 starts in fp16 and
    is demoted to Turbo4 past the threshold; Int8 starts and stays Int8."""
    T4 = KVCacheMode.TURBO4
    assert policy.initial_attention_cache_mode(T4) == KVCacheMode.FP16
    assert policy.initial_attention_cache_mode(KVCacheMode.INT8) == KVCacheMode.INT8
    c = FakeAttentionCache(KVCacheMode.FP16, THR)
    assert policy.prepare_attention_forward([c], T4, 1, True) == 1
    assert c.mode == T4 and c.demotions == 1
    assert policy.prepare_attention_forward([c], T4, 1, True) == 0


@pytest.mark.parametrize("bad", [KVCacheMode.FP16, KVCacheMode.INT8])
def test_demoting_into_a_non_quantized_mode_is_a_no_op_policy(bad):
    c = FakeAttentionCache(KVCacheMode.FP16, THR + 1)
    assert policy.finish_initial_attention_prefill([c], bad) == 0
