"""GPU parity of the D-LSA gathered read (K2 contract) through the C ABI.

Against the reference's golden fixtures (qwen_layer real/random lists, fp32
attention_out) and against the oracle at BASELINE config 5 size (131072 keys,
a 4612-entry sink + window + 8 whole 512-key blocks list). fp16 output: within
2e-3 max-abs and 1e-3 relative-L2 (the reference's own K2 fp16 check vs an f64
host softmax uses 1.5e-3, gpu_attend_tests.rs:184-258).
"""
import os

import numpy as np
import pytest
from safetensors.numpy import load_file

from conftest import GOLDEN, rng
from test_gpu_kv import assert_close, _gpu, _np

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


def c5_list(T, seed, sinks=4, window=512, block=512, n_blocks=8):
    """Config 5 read list: expansion (whole 512-key cluster blocks drawn without
    replacement among the blocks lying fully inside [sinks, T - window)), then
    the trailing window, then the sinks (the list order of the reference's
    `selected`, tests/fixtures/dlsa/README.md). Sorted, unique."""
    r = rng(seed)
    first = (sinks + block - 1) // block
    last = (T - window) // block - 1
    blocks = np.sort(r.choice(np.arange(first, last + 1), n_blocks, replace=False))
    exp = np.concatenate([np.arange(b * block, (b + 1) * block) for b in blocks])
    win = np.arange(T - window, T)
    sk = np.arange(sinks)
    return np.concatenate([exp, win, sk]).astype(np.int32)


@pytest.mark.parametrize("m", ["real", "random"])
def test_golden_qwen_layer(m):
    import qw_amd

    d = load_file(os.path.join(GOLDEN, "dlsa_qwen_layer.safetensors"))
    q = _gpu(d["q_rows"].transpose(1, 0, 2))         # [24, 10, 256]
    kstore = _gpu(d["k"])                             # [260, 4, 256]: strided heads
    vstore = _gpu(d["v"])
    k = kstore.permute(1, 0, 2)
    v = vstore.permute(1, 0, 2)
    lists = _gpu(d[f"{m}.selected"])
    lengths = _gpu(d[f"{m}.selected_lengths"])
    out = _np(qw_amd.sparse_attention(q, k, v, lists, lengths, 256 ** -0.5))[0]
    ref = d[f"{m}.attention_out"].transpose(1, 0, 2)
    assert_close(out, ref, f"qwen_layer {m}")
    # one pass, ragged splits, and part counts that put one or two workgroups on a CU
    for parts in (1, 3, 16, 64, 128):
        o2 = _np(qw_amd.sparse_attention_with(q, k, v, lists, lengths, 256 ** -0.5, parts, 0))[0]
        assert_close(o2, ref, f"qwen_layer {m} parts={parts}")


def test_config5_decode_vs_oracle(oracle_lib):
    import qw_amd

    T, H, G, D = 131072, 4, 6, 256
    r = rng(5)
    k = r.standard_normal((H, T, D)).astype(np.float16)
    v = r.standard_normal((H, T, D)).astype(np.float16)
    q = r.standard_normal((H * G, 1, D)).astype(np.float16)
    lst = c5_list(T, 5)
    assert lst.size == 4612 and np.unique(lst).size == 4612
    lists = lst[None]
    lengths = np.array([4612], np.int32)
    ref = oracle_lib.dlsa_attention(q, k, v, lists, lengths, D ** -0.5)
    out = _np(qw_amd.sparse_attention(_gpu(q), _gpu(k), _gpu(v), _gpu(lists), _gpu(lengths),
                                      D ** -0.5))[0]
    assert_close(out, ref, "config5")
    # list order is irrelevant up to fp32 rounding
    perm = r.permutation(lst)[None].astype(np.int32)
    out2 = _np(qw_amd.sparse_attention(_gpu(q), _gpu(k), _gpu(v), _gpu(perm), _gpu(lengths),
                                       D ** -0.5))[0]
    assert np.abs(out2.astype(np.float64) - out).max() <= 1e-3


@pytest.mark.parametrize("D,G", [(256, 6), (128, 8), (64, 4), (256, 16)])
def test_ragged_lists_skips_and_empty_rows(oracle_lib, D, G):
    import qw_amd

    r = rng(D + G)
    T, H, L, W = 3000, 2, 5, 700
    k = r.standard_normal((H, T, D)).astype(np.float16)
    v = r.standard_normal((H, T, D)).astype(np.float16)
    q = r.standard_normal((H * G, L, D)).astype(np.float16)
    lists = np.full((L, W), -1, np.int32)
    lengths = np.array([700, 1, 0, 333, 650], np.int32)
    for row in range(L):
        n = lengths[row]
        lists[row, :n] = r.choice(T, n, replace=False)
    lists[3, 5] = T + 9        # out of range: skipped
    lists[4, 0] = -3           # negative: skipped
    ref = oracle_lib.dlsa_attention(q, k, v, lists, lengths, D ** -0.5)
    out = _np(qw_amd.sparse_attention(_gpu(q), _gpu(k), _gpu(v), _gpu(lists), _gpu(lengths),
                                      D ** -0.5))[0]
    assert_close(out, ref, f"ragged D={D} G={G}")
    assert np.all(out[:, 2] == 0)


def prefill_lists(T0, L, seed, sinks=4, window=512, block=512, n_blocks=4):
    """Lists of an L-row prefill chunk at positions T0 .. T0 + L - 1: the sinks,
    the row's own trailing window (ending at its position) and n_blocks whole
    512-key blocks drawn once for the chunk from below the first row's window
    (the rows of a chunk pick mostly the same clusters). Width sinks + window +
    n_blocks * block; every entry is visible to its row."""
    r = rng(seed)
    last = (T0 - window) // block - 1
    blocks = np.sort(r.choice(np.arange(1, last + 1), n_blocks, replace=False))
    exp = np.concatenate([np.arange(b * block, (b + 1) * block) for b in blocks])
    lists = np.empty((L, sinks + window + exp.size), np.int32)
    for row in range(L):
        pos = T0 + row
        lists[row] = np.concatenate([exp, np.arange(pos - window + 1, pos + 1), np.arange(sinks)])
    return lists


@pytest.mark.parametrize("L", [256, 24])
def test_prefill_rows_vs_oracle(oracle_lib, L):
    """K2 at prefill row counts: 256 rows x 4 KV heads take one pass (one
    workgroup a row and head, mlx_cxx_dlsa_attention.cpp:379-418 switches at
    L * Hkv >= 160), 24 rows split each list; checked against the oracle on a
    spread of rows (first, last, and between)."""
    import qw_amd

    T0, H, G, D = 8192, 4, 6, 256
    T = T0 + L
    r = rng(9000 + L)
    k = r.standard_normal((H, T, D)).astype(np.float16)
    v = r.standard_normal((H, T, D)).astype(np.float16)
    q = r.standard_normal((H * G, L, D)).astype(np.float16)
    lists = prefill_lists(T0, L, 77 + L)
    lengths = np.full(L, lists.shape[1], np.int32)
    out = _np(qw_amd.sparse_attention(_gpu(q), _gpu(k), _gpu(v), _gpu(lists), _gpu(lengths),
                                      D ** -0.5))[0]
    sel = np.unique(np.array([0, 1, L // 3, L // 2, L - 2, L - 1]))
    ref = oracle_lib.dlsa_attention(np.ascontiguousarray(q[:, sel]), k, v,
                                    np.ascontiguousarray(lists[sel]), lengths[sel], D ** -0.5)
    assert np.isfinite(out).all()
    assert_close(out[:, sel], ref, f"prefill rows L={L}")


@pytest.mark.parametrize("D,H,G", [(256, 4, 6), (128, 2, 8)])
def test_prefill_row_pairs_vs_oracle(oracle_lib, D, H, G):
    """One-pass prefill calls take two rows a workgroup: a tile whose 16
    entries are the same keys for both rows (sinks, the chunk's blocks) is
    gathered once for both, other tiles once a row. An odd row count leaves
    the last workgroup one row; the rows' lengths differ (so some tiles split
    inside the shared part) and some entries are -1 or past the keys (skipped)."""
    import qw_amd

    T0, L = 4096, 203
    T = T0 + L
    r = rng(9100 + D)
    k = r.standard_normal((H, T, D)).astype(np.float16)
    v = r.standard_normal((H, T, D)).astype(np.float16)
    q = r.standard_normal((H * G, L, D)).astype(np.float16)
    lists = prefill_lists(T0, L, 81 + D, n_blocks=2)
    W = lists.shape[1]
    lengths = (W - (np.arange(L) % 5) * 37).astype(np.int32)
    lists[::11, 5] = -1
    lists[::13, 9] = T + 5
    out = _np(qw_amd.sparse_attention(_gpu(q), _gpu(k), _gpu(v), _gpu(lists), _gpu(lengths),
                                      D ** -0.5))[0]
    sel = np.array([0, 1, 2, 11, 13, 100, 101, 200, 201, 202])
    ref = oracle_lib.dlsa_attention(np.ascontiguousarray(q[:, sel]), k, v,
                                    np.ascontiguousarray(lists[sel]), lengths[sel], D ** -0.5)
    assert np.isfinite(out).all()
    assert_close(out[:, sel], ref, f"prefill row pairs D={D} G={G}")


def test_workspace_per_stream_growth():
    """Split-K partials live in a workspace per (device, stream): calls
    alternating on two streams, with a growth of one stream's workspace in
    between, give the single-stream outputs bit for bit."""
    import qw_amd

    r = rng(77)
    T, H, G, D, L, W = 3000, 4, 6, 256, 3, 700
    k = _gpu(r.standard_normal((H, T, D)).astype(np.float16))
    v = _gpu(r.standard_normal((H, T, D)).astype(np.float16))
    q = _gpu(r.standard_normal((H * G, L, D)).astype(np.float16))
    lists = _gpu(np.stack([r.choice(T, W, replace=False) for _ in range(L)]).astype(np.int32))
    lengths = _gpu(np.array([W, 500, 650], np.int32))
    knobs = (16, 128, 32)  # 128 parts need ~9.5 MB of partials: a growth
    torch.cuda.synchronize()
    want = [_np(qw_amd.sparse_attention_with(q, k, v, lists, lengths, D ** -0.5, p, 0))
            for p in knobs]
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    outs = []
    for rep in range(3):
        for i, p in enumerate(knobs):
            with torch.cuda.stream(s1 if (i + rep) % 2 == 0 else s2):
                outs.append((i, qw_amd.sparse_attention_with(q, k, v, lists, lengths,
                                                             D ** -0.5, p, 0)))
    torch.cuda.synchronize()
    for i, o in outs:
        np.testing.assert_array_equal(_np(o), want[i])
