#!/usr/bin/env python3
"""Benchmark of the MI355X full-attention hot path (BASELINE.json metric).

Headline (config 2): one decode layer call on a 4-bit affine KV cache at 32k
context, GQA 24q/4kv, head_dim 256: quantize-and-append one token, then the
fused dequant-in-attention over 32769 keys. A "step" is one such layer call.
Timed steps rotate over 16 distinct layer caches (16 x 37.7 MB = 604 MB, more
than the 256 MB Infinity Cache), so every step reads HBM.

value = algorithmic bytes of a layer call / its time, GB/s (inputs resident in
HBM). The 16 layer calls of a round are replayed as one HIP graph, so the
figure is device time, not Python launch overhead (the eager figure is
reported beside it). The other configurations are reported under "extra":
config 3 (2048-row prefill chunk, TFLOP/s against the MFMA peak), config 4
(16-row verify block), config 5 (D-LSA gathered read), config 1, and the
neighbouring paths at the config-2 geometry: Int8 decode, the D-LSA K1 select,
the fused q/k RoPE, Turbo4 decode and the Turbo4 fused causal verify. The CPU
baseline is the oracle's restatement of the MLX CPU stream, timed on a bounded
sample on this host.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-extra]
    python bench.py --pmc-workload          # short run for rocprofv3 --pmc passes
    python bench.py --summarize-pmc FETCH_DB WRITE_DB --out profiles/<name>.txt
    python bench.py --summarize-trace DB --out profiles/<name>.txt
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "decode attn µs/layer + HBM GB/s @32k ctx 4-bit KV; prefill TFLOP/s"
HBM_PEAK_GBS = 8000.0
MFMA_PEAK_TFLOPS = 2500.0  # dense fp16
LAYERS = 16
HQ, HKV, D = 24, 4, 256
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "attend_decode_c2_traffic.txt")
COPY_BYTES = 256 << 20  # the calibration copy of --pmc-workload


def kv_bytes_per_token_head(bits: int) -> int:
    """Algorithmic bytes of one (token, KV head) row of K plus V: codes plus one
    fp16 scale and bias per 64-dim group (288 B at 4-bit, 544 B at 8-bit)."""
    if bits == 16:
        return 2 * D * 2
    return 2 * (D * bits // 8 + (D // 64) * 2 * 2)


def attn_flops(n_rows: int, T: int, causal: bool) -> int:
    """4 * D * Hq * sum over rows of visible keys (QK and PV, 2 flops a MAC)."""
    vis = sum(T - n_rows + r + 1 for r in range(n_rows)) if causal else n_rows * T
    return 4 * D * HQ * vis


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=320)
    ap.add_argument("--warmup", type=int, default=32)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-extra", action="store_true", help="only the headline workload")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--pmc-workload", action="store_true",
                    help="a 256 MiB copy then 16 config-2 attention calls, for counter runs")
    ap.add_argument("--summarize-pmc", nargs=2, metavar=("FETCH_DB", "WRITE_DB"))
    ap.add_argument("--summarize-trace", metavar="DB")
    ap.add_argument("--command", default="rocprofv3 --kernel-trace --stats -d gpurun_out/ktrace "
                    "-o run -- python3 bench.py --no-cpu")
    ap.add_argument("--out", default=TRAFFIC_FILE)
    return ap.parse_args()


class Timer:
    """HIP events on torch's current stream (the stream the library launches on)."""

    def __init__(self, torch):
        self.torch = torch

    def run(self, fn, iters: int) -> float:
        torch = self.torch
        s = torch.cuda.Event(enable_timing=True)
        e = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        s.record()
        for _ in range(iters):
            fn()
        e.record()
        torch.cuda.synchronize()
        return s.elapsed_time(e)  # ms


def _mode(bits: int) -> str:
    return {4: "affine4", 8: "affine8", 16: "fp16"}[bits]


def make_caches(torch, qw_amd, g, bits, T_prefix, cap, layers, jitter=True, mode=None):
    dev = torch.device("cuda:0")
    caches = []
    for _ in range(layers):
        c = qw_amd.KVCache(mode or _mode(bits), HKV, D, capacity=cap)
        jit = (torch.empty((HKV, 1, 1), device=dev).uniform_(0.5, 2.0, generator=g) if jitter
               else torch.ones((HKV, 1, 1), device=dev))
        chunk = 8192
        for t0 in range(0, T_prefix, chunk):
            n = min(chunk, T_prefix - t0)
            k = (torch.randn((HKV, n, D), device=dev, generator=g) * jit).half()
            v = (torch.randn((HKV, n, D), device=dev, generator=g) * jit).half()
            c.update(k, v)
        caches.append((c, jit))
    return caches


def graph_time(torch, body, rounds: int, calls_per_round: int) -> float:
    """Capture body() (calls_per_round library calls) once as a HIP graph,
    replay it `rounds` times between events; ms per call."""
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        body()
    for _ in range(3):
        g.replay()
    ms = Timer(torch).run(g.replay, rounds) / (rounds * calls_per_round)
    del g
    return ms


class LayerSet:
    """`layers` caches of one configuration plus per-layer q / new K,V / out,
    called through the raw C ABI with prebuilt arguments."""

    def __init__(self, torch, qw_amd, seed, bits, T_prefix, L, layers, causal, mode=None):
        dev = torch.device("cuda:0")
        g = torch.Generator(device=dev)
        g.manual_seed(seed)
        self.torch, self.qw, self.L, self.causal = torch, qw_amd, L, causal
        self.caches = make_caches(torch, qw_amd, g, bits, T_prefix, T_prefix + L, layers,
                                  mode=mode)
        self.q, self.kn, self.vn, self.out = [], [], [], []
        for _, jit in self.caches:
            self.q.append(torch.randn((1, HQ, L, D), device=dev, generator=g).half())
            self.kn.append((torch.randn((HKV, L, D), device=dev, generator=g) * jit).half())
            self.vn.append((torch.randn((HKV, L, D), device=dev, generator=g) * jit).half())
            self.out.append(torch.empty((HQ, L, D), dtype=torch.float16, device=dev))
        self.lib = qw_amd.lib()
        self.T = T_prefix + L
        torch.cuda.synchronize()

    def _check(self, rc):
        if rc:
            raise self.qw.QwError(rc, self.lib.qw_last_error().decode())

    def layer_call(self, i, st):
        """update_and_attention (append L rows, attend), then trim the rows so
        the next call sees the same cache."""
        c = self.caches[i][0]
        self._check(self.lib.qw_kv_update_and_attention(
            c._h, self.q[i].data_ptr(), HQ, self.L, self.kn[i].data_ptr(),
            self.vn[i].data_ptr(), 1.0 / 16, int(self.causal), self.out[i].data_ptr(), st))
        c.trim(self.L)

    def attn_call(self, i, st):
        c = self.caches[i][0]
        self._check(self.lib.qw_kv_attention(c._h, self.q[i].data_ptr(), HQ, self.L, 1.0 / 16,
                                             int(self.causal), self.out[i].data_ptr(), st))

    def stream(self):
        return self.torch.cuda.current_stream(self.torch.device("cuda:0")).cuda_stream

    def time_layers(self, rounds):
        n = len(self.caches)
        ms = graph_time(self.torch, lambda: [self.layer_call(i, self.stream()) for i in range(n)],
                        rounds, n)
        return ms

    def time_eager(self, rounds):
        n = len(self.caches)
        return Timer(self.torch).run(lambda: [self.layer_call(i, self.stream()) for i in range(n)],
                                     rounds) / (rounds * n)

    def time_attention(self, rounds):
        n = len(self.caches)
        for i in range(n):
            c = self.caches[i][0]
            c.update(self.kn[i], self.vn[i])
        ms = graph_time(self.torch, lambda: [self.attn_call(i, self.stream()) for i in range(n)],
                        rounds, n)
        for i in range(n):
            self.caches[i][0].trim(self.L)
        return ms

    def warm(self, n_calls):
        n = len(self.caches)
        for j in range(max(1, n_calls // n)):
            for i in range(n):
                self.layer_call(i, self.stream())
        self.torch.cuda.synchronize()

    def close(self):
        for c, _ in self.caches:
            c.close()
        self.caches = []
        self.torch.cuda.empty_cache()


def bench_decode(torch, qw_amd, steps: int, warmup: int, bits: int = 4, T_prefix: int = 32768,
                 mode=None):
    """Config 2 (bits 4, 32768 + 1) or config 1 (bits 8, 4095 + 1); `mode`
    overrides the cache mode (e.g. "int8", stored in the 8-bit layout)."""
    ls = LayerSet(torch, qw_amd, 2, bits, T_prefix, 1, LAYERS, causal=False, mode=mode)
    ls.warm(warmup)
    # one attention-only round too, so the split-K workspace exists before capture
    ls.time_attention(1)
    rounds = max(1, steps // LAYERS)
    eager_ms = ls.time_eager(rounds)
    layer_ms = ls.time_layers(rounds)
    attn_ms = ls.time_attention(rounds)
    T = ls.T
    ls.close()
    bytes_attn = T * HKV * kv_bytes_per_token_head(bits) + 2 * HQ * D * 2
    bytes_layer = bytes_attn + 2 * HKV * D * 2 + HKV * kv_bytes_per_token_head(bits) // 2
    return {"T": T, "bits": bits, "rounds": rounds, "layer_ms": layer_ms, "eager_layer_ms": eager_ms,
            "attn_ms": attn_ms, "bytes_layer": bytes_layer, "bytes_attn": bytes_attn}


def bench_turbo4_verify(torch, qw_amd, steps: int, warmup: int, T_prefix: int = 32768,
                        L: int = 4):
    """A Turbo4 causal verify block (L draft rows, the reference's fused-pass
    case) at the config-2 geometry: update_and_causal_attention of L tokens,
    routed to the fused verify kernel (scored straight from the packed codes).
    Timed eagerly, like the decode route."""
    ls = LayerSet(torch, qw_amd, 4, 4, T_prefix, L, LAYERS, causal=True, mode="turbo4")
    ls.warm(warmup)
    rounds = max(1, steps // LAYERS)
    ms = ls.time_eager(rounds)
    T = ls.T
    ls.close()
    return {"T": T, "L": L, "layer_ms": ms}


def bench_turbo4_decode(torch, qw_amd, steps: int, warmup: int, T_prefix: int = 32768):
    """The reference's served default KV mode at the config-2 geometry:
    update_and_attention of one token on a Turbo4 cache (rotate q, expand the
    rotated K/V to fp16, the fp16 decode kernels, rotate the output back).
    Timed eagerly: the route's shared workspace orders its users with an
    event, which a HIP graph capture does not take."""
    ls = LayerSet(torch, qw_amd, 3, 4, T_prefix, 1, LAYERS, causal=False, mode="turbo4")
    ls.warm(warmup)
    rounds = max(1, steps // LAYERS)
    ms = ls.time_eager(rounds)
    T = ls.T
    ls.close()
    return {"T": T, "layer_ms": ms, "rounds": rounds}


def bench_select(torch, qw_amd, steps: int, T: int = 131072):
    """D-LSA K1 select at the served defaults (window 512, sink 4, top-k 4096,
    top-p 1024, 8-key buckets, 64 buckets a block) for one decode row at
    context T: synthetic N(0,1) bucket scores. Raw ABI calls with preallocated
    outputs, graph-replayed."""
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(5)
    n_b = T // 8
    scores = torch.randn((1, n_b), device=dev, generator=g, dtype=torch.float32)
    members = torch.full((n_b, 16), -1, dtype=torch.int32, device=dev)
    members[:, :8] = torch.arange(n_b * 8, dtype=torch.int32, device=dev).view(n_b, 8)
    pos = torch.tensor([T - 1], dtype=torch.int32, device=dev)
    window, sink, top_k, top_p, bpb = 512, 4, 4096, 1024, 64
    W = top_k + window + sink
    lists = torch.empty((1, W), dtype=torch.int32, device=dev)
    lengths = torch.empty((1,), dtype=torch.int32, device=dev)
    picked = torch.empty((1, top_p), dtype=torch.int32, device=dev)
    status = torch.empty((1,), dtype=torch.int32, device=dev)
    lib = qw_amd.lib()

    def call():
        st = torch.cuda.current_stream(dev).cuda_stream
        rc = lib.qw_dlsa_select(scores.data_ptr(), n_b, members.data_ptr(), n_b, 16,
                                pos.data_ptr(), 1, n_b, window, sink, top_k, top_p, bpb, 0,
                                lists.data_ptr(), lengths.data_ptr(), picked.data_ptr(),
                                status.data_ptr(), st)
        if rc:
            raise qw_amd.QwError(rc, lib.qw_last_error().decode())

    for _ in range(5):
        call()
    torch.cuda.synchronize()
    ms = graph_time(torch, lambda: [call() for _ in range(LAYERS)], max(1, steps // LAYERS),
                    LAYERS)
    return {"ms": ms, "buckets": n_b, "list_len": int(lengths.item()), "width": W}


def bench_rope(torch, qw_amd, steps: int, L: int = 2048):
    """Fused q/k RoPE: the standalone op over a 2048-token QKV chunk (bytes:
    the chunk read once, q/k/v written once), and the RoPE-append of one
    decode token into a 4-bit cache (append then trim, graph-replayed)."""
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(6)
    W = (HQ + 2 * HKV) * D
    qkv = torch.randn((1, L, W), device=dev, generator=g).half()
    q = torch.empty((1, HQ, L, D), dtype=torch.float16, device=dev)
    k = torch.empty((1, HKV, L, D), dtype=torch.float16, device=dev)
    v = torch.empty_like(k)
    lib = qw_amd.lib()

    def chunk():
        st = torch.cuda.current_stream(dev).cuda_stream
        rc = lib.qw_fused_rope_qk_append(qkv.data_ptr(), 1, L, HQ, HKV, D, D, 1e7, 1.0, 0, 1000,
                                         0, q.data_ptr(), k.data_ptr(), v.data_ptr(), st)
        if rc:
            raise qw_amd.QwError(rc, lib.qw_last_error().decode())

    chunk()
    torch.cuda.synchronize()
    chunk_ms = graph_time(torch, lambda: [chunk() for _ in range(LAYERS)], max(1, steps // LAYERS),
                          LAYERS)
    cache = qw_amd.KVCache("affine4", HKV, D, capacity=4096)
    cache.update(torch.randn((HKV, 4000, D), device=dev, generator=g).half(),
                 torch.randn((HKV, 4000, D), device=dev, generator=g).half())
    tok = qkv[:, :1].contiguous()
    q1 = torch.empty((HQ, 1, D), dtype=torch.float16, device=dev)

    def one():
        st = torch.cuda.current_stream(dev).cuda_stream
        rc = lib.qw_kv_rope_update(cache._h, tok.data_ptr(), HQ, 1, D, 0, 1e7, 1.0, 4000,
                                   q1.data_ptr(), st)
        if rc:
            raise qw_amd.QwError(rc, lib.qw_last_error().decode())
        cache.trim(1)

    one()
    torch.cuda.synchronize()
    one_ms = graph_time(torch, lambda: [one() for _ in range(LAYERS)], max(1, steps // LAYERS),
                        LAYERS)
    cache.close()
    return {"chunk_ms": chunk_ms, "chunk_bytes": 2 * L * W * 2, "token_ms": one_ms}


def bench_block(torch, qw_amd, steps: int, bits: int, T_prefix: int, L: int, layers: int):
    """Config 3 (prefill chunk) / config 4 (verify block): append L rows and
    attend them causally; graph-replayed over `layers` caches."""
    ls = LayerSet(torch, qw_amd, 3 + L, bits, T_prefix, L, layers, causal=True)
    ls.warm(2 * layers)
    ls.time_attention(1)
    rounds = max(2, steps // (4 * layers))
    layer_ms = ls.time_layers(rounds)
    attn_ms = ls.time_attention(rounds)
    T = ls.T
    ls.close()
    flops = attn_flops(L, T, True)
    kv = T * HKV * kv_bytes_per_token_head(bits)
    return {"T": T, "L": L, "bits": bits, "layer_ms": layer_ms, "attn_ms": attn_ms,
            "flops": flops, "kv_bytes": kv}


def bench_dlsa(torch, qw_amd, steps: int, T: int = 131072, layers: int = LAYERS):
    """Config 5: one decode row, 4612-entry list (4 sinks + 512 window + 8 whole
    512-key blocks drawn without replacement from the blocks fully inside
    [4, window start)), fp16 KV [4, 131072, 256] per layer, 16 layers rotated."""
    import numpy as np

    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(5)
    rng = np.random.default_rng(5)
    ks, vs, qs, lists, lens, outs = [], [], [], [], [], []
    for layer in range(layers):
        ks.append(torch.randn((1, HKV, T, D), device=dev, generator=g).half())
        vs.append(torch.randn((1, HKV, T, D), device=dev, generator=g).half())
        qs.append(torch.randn((1, HQ, 1, D), device=dev, generator=g).half())
        blocks = np.sort(rng.choice(np.arange(1, (T - 512) // 512), 8, replace=False))
        lst = np.concatenate([np.concatenate([np.arange(b * 512, b * 512 + 512) for b in blocks]),
                              np.arange(T - 512, T), np.arange(4)]).astype(np.int32)
        lists.append(torch.from_numpy(lst[None]).to(dev))
        lens.append(torch.tensor([lst.size], dtype=torch.int32, device=dev))
        outs.append(torch.empty((HQ, 1, D), dtype=torch.float16, device=dev))
    W = lists[0].shape[1]
    L = qw_amd.lib()

    def call(i, st):
        k, v = ks[i][0], vs[i][0]
        rc = L.qw_dlsa_sparse_attention(qs[i].data_ptr(), k.data_ptr(), v.data_ptr(), k.stride(0),
                                        k.stride(1), v.stride(0), v.stride(1),
                                        lists[i].data_ptr(), lens[i].data_ptr(), 1, W, HQ, HKV, D,
                                        T, D ** -0.5, outs[i].data_ptr(), st)
        assert rc == 0, L.qw_last_error()

    st = torch.cuda.current_stream(dev).cuda_stream
    for i in range(layers):
        call(i, st)
    torch.cuda.synchronize()
    rounds = max(1, steps // layers)
    ms = graph_time(torch, lambda: [call(i, torch.cuda.current_stream(dev).cuda_stream)
                                    for i in range(layers)], rounds, layers)
    bytes_call = W * HKV * 2 * D * 2 + HQ * D * 2 * 2 + W * 4
    del ks, vs
    torch.cuda.empty_cache()
    return {"T": T, "W": int(W), "ms": ms, "bytes": bytes_call}


def cpu_baseline(seconds: float, threads: int):
    """Oracle restatement of the MLX CPU stream for the config 2 layer call
    (quantize the new token, dequantize the whole cache, SDPA with fp16
    roundings), timed on this host over a bounded number of calls."""
    import numpy as np

    import oracle

    oracle.build()
    r = np.random.default_rng(2)
    T0 = 32768
    jit = r.uniform(0.5, 2.0, (HKV, 1, 1))
    k = (r.standard_normal((HKV, T0 + 1, D)) * jit).astype(np.float16)
    v = (r.standard_normal((HKV, T0 + 1, D)) * jit).astype(np.float16)
    q = r.standard_normal((HQ, 1, D)).astype(np.float16)
    orc = oracle.AffineCacheOracle(HKV, D, T0 + 1, 4)
    orc.update(k[:, :T0], v[:, :T0])
    n, t_total = 0, 0.0
    while t_total < seconds and n < 50:
        t = time.perf_counter()
        orc.update_and_attention(q, k[:, T0:], v[:, T0:], 1 / 16, False, threads=threads)
        t_total += time.perf_counter() - t
        orc.offset -= 1
        n += 1
    return {"calls": n, "s_per_call": t_total / n}


# ----------------------------------------------------------- counter runs

def pmc_workload() -> int:
    """What the rocprofv3 --pmc passes profile: one plain 256 MiB device copy
    (the calibration kernel, HIP's copyBuffer: FETCH_SIZE / WRITE_SIZE of a
    known byte count; the largest copyBuffer dispatch of the run),
    then 16 config-2 attention calls over 16 distinct caches."""
    import torch

    import qw_amd

    qw_amd.lib()
    torch.cuda.set_device(0)
    src = torch.full((COPY_BYTES // 2,), 1.5, dtype=torch.float16, device="cuda:0")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)  # a device-to-device memcpy: HIP's copyBuffer kernel
    torch.cuda.synchronize()
    del src, dst
    ls = LayerSet(torch, qw_amd, 2, 4, 32768, 1, LAYERS, causal=False)
    for i in range(LAYERS):
        ls.caches[i][0].update(ls.kn[i], ls.vn[i])
    torch.cuda.synchronize()
    for i in range(LAYERS):
        ls.attn_call(i, ls.stream())
    torch.cuda.synchronize()
    ls.close()
    print("pmc workload done", flush=True)
    return 0


def _pmc_per_kernel(db_path: str, counter: str):
    import sqlite3

    con = sqlite3.connect(db_path)
    tabs = [r[0] for r in con.execute("select name from sqlite_master where type in ('table', 'view')")]
    ctab = next(t for t in tabs if t.startswith("counters_collection"))
    rows = con.execute(f"select * from {ctab} limit 1")
    cols = [d[0] for d in rows.description]
    name_col = next(c for c in cols if c in ("kernel_name", "name"))
    cnt_col = next(c for c in cols if c in ("counter_name", "counter"))
    val_col = next(c for c in cols if c in ("value", "counter_value"))
    disp_col = next((c for c in cols if "dispatch" in c and "id" in c), None)
    if disp_col:
        q = (f"select {name_col}, sum({val_col}) from {ctab} where {cnt_col} = ? "
             f"group by {name_col}, {disp_col}")
    else:
        q = f"select {name_col}, {val_col} from {ctab} where {cnt_col} = ?"
    per = {}
    for name, v in con.execute(q, (counter,)):
        per.setdefault(name, []).append(float(v))
    return per


def summarize_pmc(fetch_db: str, write_db: str, out: str) -> int:
    fetch = _pmc_per_kernel(fetch_db, "FETCH_SIZE")
    write = _pmc_per_kernel(write_db, "WRITE_SIZE")

    def pick(d, key):
        k = next(n for n in d if key in n)
        v = d[k]
        return k, sum(v) / len(v), len(v)

    # the calibration copy is the largest copyBuffer dispatch of the run
    copy_k = next(n for n in fetch if "copyBuffer" in n)
    copy_fetch = max(fetch[copy_k])
    copy_write = max(write[next(n for n in write if "copyBuffer" in n)])
    f_scale = (COPY_BYTES / 1024.0) / copy_fetch    # true KiB per counted KiB
    w_scale = (COPY_BYTES / 1024.0) / copy_write
    att_k, att_fetch, n_f = pick(fetch, "attend_decode_kernel")
    _, att_write, n_w = pick(write, "attend_decode_kernel")
    mer_key = next(k for k in ("merge_append_kernel", "decode_merge_kernel") if any(k in n for n in fetch))
    mer_k, mer_fetch, _ = pick(fetch, mer_key)
    _, mer_write, _ = pick(write, mer_key)
    traffic = (att_fetch * f_scale + att_write * w_scale) * 1024.0
    alg = 32769 * HKV * kv_bytes_per_token_head(4) + 2 * HQ * D * 2
    lines = [
        "# HBM traffic of the config-2 attention kernel (rocprofv3 --pmc)",
        "",
        "commands:",
        "  rocprofv3 --pmc FETCH_SIZE -d gpurun_out/pmc_fetch -o run -- python3 bench.py --pmc-workload",
        "  rocprofv3 --pmc WRITE_SIZE -d gpurun_out/pmc_write -o run -- python3 bench.py --pmc-workload",
        "  python3 bench.py --summarize-pmc <fetch db> <write db>",
        "",
        f"calibration kernel: {copy_k[:90]}",
        f"  copy of {COPY_BYTES} B: FETCH_SIZE {copy_fetch:.1f} KiB, WRITE_SIZE {copy_write:.1f} KiB",
        f"  scale factors (true / counted): fetch {f_scale:.4f}, write {w_scale:.4f}",
        f"kernel: {att_k[:90]} ({n_f} / {n_w} dispatches)",
        f"  FETCH_SIZE {att_fetch:.1f} KiB/dispatch, WRITE_SIZE {att_write:.1f} KiB/dispatch",
        f"merge kernel: {mer_k[:90]}",
        f"  FETCH_SIZE {mer_fetch:.1f} KiB/dispatch, WRITE_SIZE {mer_write:.1f} KiB/dispatch",
        f"algorithmic bytes per dispatch: {alg}",
        f"traffic_bytes_per_dispatch = {traffic:.0f}",
        f"traffic / algorithmic = {traffic / alg:.4f}",
    ]
    os.makedirs(os.path.dirname(os.path.abspath(out)), exist_ok=True)
    with open(out, "w") as f:
        f.write("\n".join(lines) + "\n")
    print("\n".join(lines))
    return 0


def summarize_trace(db_path: str, out: str, command: str) -> int:
    """Per-kernel dispatch count and duration (avg / min / max, µs) from a
    rocprofv3 --kernel-trace database, as a short text table: every kernel of
    this library, then the others (torch's input generation) by total time."""
    import sqlite3

    con = sqlite3.connect(db_path)
    rows = con.execute("select name, count(*), avg(end - start), min(end - start), "
                       "max(end - start), sum(end - start) from kernels group by name "
                       "order by sum(end - start) desc").fetchall()
    lines = ["# rocprofv3 kernel trace summary", "", "command:", f"  {command}",
             "  python3 bench.py --summarize-trace <db> --out <this file>", "",
             f"{'kernel':<72} {'n':>6} {'avg_us':>9} {'min_us':>9} {'max_us':>9}"]
    ours = [r for r in rows if "qw::" in r[0] or "_ZN2qw" in r[0]]
    rows = ours + [r for r in rows if r not in ours][:4]
    for name, n, avg, mn, mx, _ in rows:
        short = name if len(name) <= 72 else name[:69] + "..."
        lines.append(f"{short:<72} {n:>6} {avg / 1e3:>9.2f} {mn / 1e3:>9.2f} {mx / 1e3:>9.2f}")
    os.makedirs(os.path.dirname(os.path.abspath(out)), exist_ok=True)
    with open(out, "w") as f:
        f.write("\n".join(lines) + "\n")
    print("\n".join(lines))
    return 0


def read_traffic():
    try:
        with open(TRAFFIC_FILE) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_dispatch"):
                    return int(float(line.split("=")[1]))
    except OSError:
        pass
    return None


def main() -> int:
    args = parse()
    if args.summarize_pmc:
        return summarize_pmc(args.summarize_pmc[0], args.summarize_pmc[1], args.out)
    if args.summarize_trace:
        return summarize_trace(args.summarize_trace, args.out, args.command)
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only: the path shards by KV head "
                          "across GPUs in design, which is not implemented; run with --gpus 1"}))
        return 2
    if args.pmc_workload:
        return pmc_workload()
    import torch

    import qw_amd

    qw_amd.lib()  # fail loudly if the HIP library is missing
    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU visible"}))
        return 2
    torch.cuda.set_device(0)
    steps = max(LAYERS, args.steps // LAYERS * LAYERS)
    log(f"bench: config 2 decode, {steps} steps, warmup {args.warmup}")
    dec = bench_decode(torch, qw_amd, steps, args.warmup)
    us_layer = dec["layer_ms"] * 1e3
    value = dec["bytes_layer"] / (dec["layer_ms"] * 1e-3) / 1e9
    achieved = dec["bytes_attn"] / (dec["attn_ms"] * 1e-3) / 1e9
    line = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": round(dec["layer_ms"], 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u4 codes / fp16",
        "data": "synthetic: N(0,1) fp16 K/V x per-head U(0.5,2), N(0,1) q, seeded",
        "config": {"workload": "config 2: decode layer call, append 1 token (4-bit affine, "
                               "group 64) + fused dequant-SDPA over 32769 keys",
                   "q_heads": HQ, "kv_heads": HKV, "head_dim": D, "context": dec["T"],
                   "kv_bits": 4, "layers_rotated": LAYERS},
        "us_per_layer": round(us_layer, 3),
        "us_per_layer_eager": round(dec["eager_layer_ms"] * 1e3, 3),
        "us_attention": round(dec["attn_ms"] * 1e3, 3),
        "tokens_per_s": round(1.0 / (dec["layer_ms"] * 1e-3), 1),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": read_traffic(),
                     "kernel": "qw_kv_attention: attend_decode_kernel + decode_merge_kernel, "
                               "graph-replayed over 16 caches",
                     "algorithmic_bytes": dec["bytes_attn"]},
    }
    if not args.no_extra:
        extra = {}
        log("bench: config 3 prefill chunk")
        pf = bench_block(torch, qw_amd, steps, 8, 16384, 2048, 2)
        tf = pf["flops"] / (pf["attn_ms"] * 1e-3) / 1e12
        extra["config3_prefill"] = {
            "us_per_layer": round(pf["layer_ms"] * 1e3, 1),
            "us_attention": round(pf["attn_ms"] * 1e3, 1),
            "TFLOP_s": round(tf, 1), "frac_mfma": round(tf / MFMA_PEAK_TFLOPS, 4),
            "TFLOP_s_layer": round(pf["flops"] / (pf["layer_ms"] * 1e-3) / 1e12, 1),
            "tokens_per_s": round(2048 / (pf["layer_ms"] * 1e-3), 1),
            "flops": pf["flops"], "keys": pf["T"], "rows": 2048, "kv_bits": 8}
        log("bench: config 4 verify block")
        vf = bench_block(torch, qw_amd, steps, 4, 65536, 16, LAYERS)
        vt = vf["flops"] / (vf["attn_ms"] * 1e-3) / 1e12
        vg = vf["kv_bytes"] / (vf["attn_ms"] * 1e-3) / 1e9
        extra["config4_verify"] = {
            "us_per_layer": round(vf["layer_ms"] * 1e3, 2),
            "us_attention": round(vf["attn_ms"] * 1e3, 2),
            "TFLOP_s": round(vt, 1), "frac_mfma": round(vt / MFMA_PEAK_TFLOPS, 4),
            "GB_s": round(vg, 1), "frac_hbm": round(vg / HBM_PEAK_GBS, 4),
            "flops": vf["flops"], "kv_bytes": vf["kv_bytes"], "keys": vf["T"], "rows": 16,
            "kv_bits": 4}
        log("bench: config 5 D-LSA read")
        ds = bench_dlsa(torch, qw_amd, steps)
        gbs = ds["bytes"] / (ds["ms"] * 1e-3) / 1e9
        extra["config5_dlsa_decode"] = {
            "us_per_layer": round(ds["ms"] * 1e3, 3), "GB_s": round(gbs, 1),
            "frac_hbm": round(gbs / HBM_PEAK_GBS, 4), "list_width": ds["W"],
            "context": ds["T"], "algorithmic_bytes": ds["bytes"]}
        log("bench: config 1 decode (8-bit, 4096 keys)")
        c1 = bench_decode(torch, qw_amd, steps, args.warmup, bits=8, T_prefix=4095)
        extra["config1_decode"] = {
            "us_per_layer": round(c1["layer_ms"] * 1e3, 3),
            "us_attention": round(c1["attn_ms"] * 1e3, 3),
            "GB_s": round(c1["bytes_attn"] / (c1["attn_ms"] * 1e-3) / 1e9, 1)}
        log("bench: Int8 decode (config-2 geometry)")
        i8 = bench_decode(torch, qw_amd, steps, args.warmup, bits=8, T_prefix=32768, mode="int8")
        extra["int8_decode"] = {
            "us_per_layer": round(i8["layer_ms"] * 1e3, 2),
            "us_attention": round(i8["attn_ms"] * 1e3, 2),
            "GB_s": round(i8["bytes_attn"] / (i8["attn_ms"] * 1e-3) / 1e9, 1)}
        log("bench: D-LSA K1 select")
        k1 = bench_select(torch, qw_amd, steps)
        extra["dlsa_k1_select"] = {
            "us_per_row": round(k1["ms"] * 1e3, 2), "buckets": k1["buckets"],
            "list_width": k1["width"], "list_len": k1["list_len"]}
        log("bench: fused q/k RoPE")
        rp = bench_rope(torch, qw_amd, steps)
        extra["rope"] = {
            "us_chunk_2048": round(rp["chunk_ms"] * 1e3, 2),
            "GB_s_chunk": round(rp["chunk_bytes"] / (rp["chunk_ms"] * 1e-3) / 1e9, 1),
            "us_rope_append_1_token": round(rp["token_ms"] * 1e3, 2)}
        log("bench: Turbo4 decode (config-2 geometry)")
        t4 = bench_turbo4_decode(torch, qw_amd, steps, args.warmup)
        extra["turbo4_decode"] = {
            "us_per_layer_eager": round(t4["layer_ms"] * 1e3, 2), "keys": t4["T"],
            "route": "rotate q, expand rotated K/V to fp16, fp16 decode, rotate back"}
        log("bench: Turbo4 fused causal verify (4 rows, config-2 geometry)")
        tv = bench_turbo4_verify(torch, qw_amd, steps, args.warmup)
        extra["turbo4_verify"] = {
            "us_per_layer_eager": round(tv["layer_ms"] * 1e3, 2), "keys": tv["T"], "rows": tv["L"],
            "route": "rotate q, fused verify kernel on the packed codes, merge, rotate back"}
        line["extra"] = extra
    if not args.no_cpu:
        threads = min(16, os.cpu_count() or 1)
        log(f"bench: CPU baseline ({threads} threads, ~{args.cpu_seconds:.0f} s)")
        cb = cpu_baseline(args.cpu_seconds, threads)
        line["cpu_baseline"] = {
            "value": round(dec["bytes_layer"] / cb["s_per_call"] / 1e9, 3),
            "unit": "GB/s",
            "cores": threads,
            "kind": "port",
            "us_per_layer": round(cb["s_per_call"] * 1e6, 1),
            "sample": f"{cb['calls']} config-2 layer calls (quantize 1 token, dequantize 32769 "
                      f"keys, MLX-rounding SDPA) by the C oracle, a restatement of the MLX CPU "
                      f"stream (not MLX)",
        }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
