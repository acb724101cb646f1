"""GPU parity of the D-LSA K1 select (qw_dlsa_select) through the C ABI.

Exact (picked buckets, lists, lengths, status) against the reference's golden
fixtures (tiny, tiny_ties, qwen_layer random/real, qwen_index_defaults: the
served defaults with 4,612-entry lists) and against the CPU oracle
(oracle.dlsa_select, itself pinned by the same fixtures) on random cases built
like the reference's own kernel tests (dlsa_kernels_tests.rs:236-425): score
kinds with many ties and signed zeros, top_k / top_p / sink variants, up to
40,000 buckets, top_p 2048 with 8,192-key expansions, every workgroup size, a
NaN score, too few score columns, an empty cache and bad arguments. Then K1
feeds K2: lists selected on the device drive the gathered read to the
fixture's attention output.
"""
import os

import numpy as np
import pytest
from safetensors.numpy import load_file

from conftest import GOLDEN, rng
from test_gpu_kv import assert_close, _gpu, _np
from test_oracle_select import CASES, select_args

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

SMALL = dict(window=16, sink=2, top_k=20, top_p=6, bucket_cap=8, buckets_per_block=4)
QWEN = dict(window=512, sink=4, top_k=4096, top_p=1024, bucket_cap=16, buckets_per_block=64)


def _params(d):
    import qw_amd

    return qw_amd.DlsaSelectParams(d["window"], d["sink"], d["top_k"], d["top_p"],
                                   d["bucket_cap"], d["buckets_per_block"])


def _run(scores, members, positions, total_rows, p, threads=0):
    import qw_amd

    sc = torch.tensor(np.asarray(scores, np.float32), device="cuda:0")
    mb = torch.tensor(np.asarray(members, np.int32), device="cuda:0")
    pos = torch.tensor(np.asarray(positions, np.int32), device="cuda:0")
    out = qw_amd.dlsa_select_with(sc, mb, pos, total_rows, _params(p), threads)
    return [_np(t) for t in out]


def _check(oracle_lib, scores, members, positions, total_rows, p, threads=0, what=""):
    got = _run(scores, members, positions, total_rows, p, threads)
    want = oracle_lib.dlsa_select(np.asarray(scores, np.float32), members, positions, total_rows,
                                  p["window"], p["sink"], p["top_k"], p["top_p"],
                                  p["buckets_per_block"])
    for name, g, w in zip(("lists", "lengths", "picked", "status"), got, want):
        assert np.array_equal(g, w), (what, name, np.argwhere(g != w)[:5])


def _members(r, p, rows):
    """[rows, cap]: bucket b of block b / m holds an ascending random subset of
    that block's positions, -1 padded (dlsa_kernels_tests.rs:61-84)."""
    w, m, cap = p["window"], p["buckets_per_block"], p["bucket_cap"]
    out = np.full((rows, cap), -1, np.int32)
    for b in range(rows):
        base = (b // m) * w
        n = int(r.integers(0, min(cap, w) + 1))
        picks = np.sort(r.choice(w, n, replace=False)) + base
        out[b, :n] = picks
    return out


def _scores(r, kind, n):
    if kind == "float":
        return r.random(n, dtype=np.float32)
    if kind == "ternary":
        return np.array([-1.0, 0.0, 1.0], np.float32)[r.integers(0, 3, n)]
    if kind == "signed_zeros":
        return np.array([-0.0, 0.0, 0.5], np.float32)[r.integers(0, 3, n)]
    return np.array([0.25, -0.125, 0.75, 0.75, 1e-30], np.float32)[r.integers(0, 5, n)]


def _random_case(oracle_lib, seed, p, t, rows, kind, threads_list=(0, 256)):
    r = rng(seed)
    w = p["window"]
    total_rows = t // w * p["buckets_per_block"]
    members = _members(r, p, max(total_rows, 1))
    positions = list(r.integers(0, t, rows))
    positions += [e for e in (0, w - 1, w, 2 * w - 1, 2 * w, t - 1) if e < t]
    positions = np.array(positions, np.int32)
    stride = int(max(min(x // w * p["buckets_per_block"], total_rows) for x in positions))
    scores = _scores(r, kind, len(positions) * stride).reshape(len(positions), stride)
    for threads in threads_list:
        _check(oracle_lib, scores, members, positions, total_rows, p, threads,
               f"seed {seed} {kind} t {t} threads {threads} {p}")


@pytest.mark.parametrize("tag", sorted(CASES))
def test_select_matches_golden_fixtures(tag):
    cfg, t = CASES[tag]
    a = select_args(cfg, t)
    p = dict(window=a["window"], sink=a["sink"], top_k=a["top_k"], top_p=a["top_p"],
             bucket_cap=t["bucket_members"].shape[1], buckets_per_block=a["buckets_per_block"])
    for threads in (0, 64, 1024):
        lists, lengths, picked, status = _run(t["bucket_scores"], t["bucket_members"],
                                              t["positions"], a["total_rows"], p, threads)
        assert not status.any()
        assert np.array_equal(picked, t["picked_buckets"]), (tag, threads)
        assert np.array_equal(lengths, t["selected_lengths"]), (tag, threads)
        assert np.array_equal(lists, t["selected"]), (tag, threads)


VARIANTS = [SMALL, dict(SMALL, top_k=3), dict(SMALL, top_p=1, sink=0), dict(SMALL, sink=40),
            dict(SMALL, top_p=2, top_k=64)]


@pytest.mark.parametrize("vi", range(len(VARIANTS)))
def test_small_configs_match_oracle(oracle_lib, vi):
    seed = 1 + 100 * vi
    for t in (1, 15, 16, 17, 33, 100, 400):
        for kind in ("float", "ternary", "signed_zeros", "few_values"):
            _random_case(oracle_lib, seed, VARIANTS[vi], t, 24, kind)
            seed += 1


def test_qwen_defaults_match_oracle_up_to_40k_buckets(oracle_lib):
    seed = 1000
    for t in (511, 1024, 8704, 9216, 93_696, 320_000):
        for kind in ("float", "ternary", "signed_zeros"):
            _random_case(oracle_lib, seed, QWEN, t, 12, kind)
            seed += 1


def test_top_p_limit_and_wide_lists(oracle_lib):
    import qw_amd

    p = dict(QWEN, top_p=qw_amd.DLSA_TOP_P_MAX, top_k=8192)
    for seed, kind in ((7, "float"), (8, "ternary")):
        _random_case(oracle_lib, seed, p, 70_000, 6, kind)


def test_workgroup_size_does_not_change_outputs(oracle_lib):
    _random_case(oracle_lib, 42, QWEN, 40_000, 8, "ternary", threads_list=(64, 128, 512, 1024))


def test_nan_ranks_last_and_sets_status(oracle_lib):
    r = rng(5)
    t = 4096
    total_rows = t // 16 * 4
    members = _members(r, SMALL, total_rows)
    positions = np.array([4095, 200, 15], np.int32)
    scores = r.random((3, total_rows), dtype=np.float32)
    scores[0, 3] = np.nan
    scores[1, 1] = -np.nan
    scores[1, 2] = -np.inf
    scores[2, 0] = np.nan  # row 2 sees no bucket: never read
    _check(oracle_lib, scores, members, positions, total_rows, SMALL)
    status = _run(scores, members, positions, total_rows, SMALL)[3]
    assert list(status) == [1, 1, 0]


def test_short_scores_and_spare_member_rows(oracle_lib):
    r = rng(6)
    total_rows = 64
    members = _members(r, SMALL, total_rows + 40)
    positions = np.array([1000, 60], np.int32)
    scores = r.random((2, 20), dtype=np.float32)  # 20 columns: < visible(1000) = 64, > visible(60) = 12
    _check(oracle_lib, scores, members, positions, total_rows, SMALL)
    assert list(_run(scores, members, positions, total_rows, SMALL)[3]) == [2, 0]


def test_empty_cache_and_no_rows(oracle_lib):
    import qw_amd

    positions = np.array([0, 5, 300], np.int32)
    _check(oracle_lib, np.zeros((3, 0), np.float32), np.zeros((0, 8), np.int32), positions, 0,
           SMALL)
    out = qw_amd.dlsa_select(torch.zeros((0, 4), dtype=torch.float32, device="cuda:0"),
                             torch.full((1, 8), -1, dtype=torch.int32, device="cuda:0"),
                             torch.zeros((0,), dtype=torch.int32, device="cuda:0"), 1,
                             _params(SMALL))
    assert tuple(out[0].shape) == (0, 38) and tuple(out[2].shape) == (0, 6)


def test_bad_arguments_are_errors():
    import qw_amd

    sc = torch.zeros((1, 4), dtype=torch.float32, device="cuda:0")
    mem = torch.full((4, 8), -1, dtype=torch.int32, device="cuda:0")
    pos = torch.tensor([100], dtype=torch.int32, device="cuda:0")
    with pytest.raises(qw_amd.QwError):
        qw_amd.dlsa_select(sc, mem, pos, 4, _params(dict(SMALL, top_p=qw_amd.DLSA_TOP_P_MAX + 1)))
    with pytest.raises(qw_amd.QwError):
        qw_amd.dlsa_select(sc, mem, pos, 4, _params(dict(SMALL, bucket_cap=4)))
    with pytest.raises(qw_amd.QwError):
        qw_amd.dlsa_select(sc, mem, pos, 5, _params(SMALL))
    with pytest.raises(qw_amd.QwError):
        qw_amd.dlsa_select_with(sc, mem, pos, 4, _params(SMALL), 100)


@pytest.mark.parametrize("m", ["real", "random"])
def test_device_lists_drive_the_gathered_read(m):
    """K1 then K2 on the device reproduce the fixture's attention output."""
    import qw_amd

    cfg, t = CASES[f"qwen_layer.{m}"]
    a = select_args(cfg, t)
    p = dict(window=a["window"], sink=a["sink"], top_k=a["top_k"], top_p=a["top_p"],
             bucket_cap=t["bucket_members"].shape[1], buckets_per_block=a["buckets_per_block"])
    d = load_file(os.path.join(GOLDEN, "dlsa_qwen_layer.safetensors"))
    rows = d["attention_rows"]
    sc = torch.tensor(t["bucket_scores"][rows], device="cuda:0")
    mb = torch.tensor(t["bucket_members"], device="cuda:0")
    pos = torch.tensor(rows.astype(np.int32), device="cuda:0")
    lists, lengths, _, status = qw_amd.dlsa_select(sc, mb, pos, a["total_rows"], _params(p))
    assert not _np(status).any()
    q = _gpu(d["q_rows"].transpose(1, 0, 2))
    k = _gpu(d["k"]).permute(1, 0, 2)
    v = _gpu(d["v"]).permute(1, 0, 2)
    out = _np(qw_amd.sparse_attention(q, k, v, lists, lengths, 256 ** -0.5))[0]
    assert_close(out, d[f"{m}.attention_out"].transpose(1, 0, 2), f"K1->K2 {m}")
