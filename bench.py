#!/usr/bin/env python3
"""Benchmark of the MI355X full-attention hot path (BASELINE.json metric).

Headline (config 2): one decode layer call on a 4-bit affine KV cache at 32k
context, GQA 24q/4kv, head_dim 256: quantize-and-append one token, then the
fused dequant-in-attention over 32769 keys. A "step" is one such layer call.
Timed steps rotate over 16 distinct layer caches (16 x 37.7 MB = 604 MB, more
than the 256 MB Infinity Cache), so every step reads HBM.

value = algorithmic bytes of a layer call / its time, GB/s (inputs resident in
HBM). The timed region of a measurement is exactly K = --steps layer calls,
cycling over the 16 caches, captured as one HIP graph and replayed between two
HIP events; --reps (at least 50) such replays are timed and ms_per_step is
their median (min and max are reported beside it), so the figure is device
time, not Python launch overhead (the eager figure is reported too). The other
configurations are reported under "extra", each the median of at least 50
replays: config 3 (2048-row prefill chunk over 4 rotated caches, 392 MB,
TFLOP/s against the MFMA peak), config 4 (16-row verify block), the served 4-
and 5-row verify blocks, config 5 (D-LSA gathered read), config 1, and the
neighbouring paths at the config-2 geometry: Int8 decode, the D-LSA K1
select, the fused q/k RoPE, Turbo4 decode and the Turbo4 fused causal
verify. Counter-derived figures (bytes read from memory, MFMA busy cycles)
come from the committed profiles/counters_<cfg>.txt summaries. The CPU
baseline is the oracle's restatement of the MLX CPU stream, timed on a
bounded sample on this host.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--reps R] [--no-cpu] [--no-extra]
    python bench.py --pmc-workload c1|c2|c3|c4|c5   # short run for rocprofv3 --pmc passes
    python bench.py --summarize-counters CFG DIR --out profiles/counters_<cfg>.txt
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
    ap.add_argument("--reps", type=int, default=50, help="timed graph replays (at least 50)")
    ap.add_argument("--pmc-workload", choices=["c1", "c2", "c3", "c4", "c5", "gemm"],
                    help="a 256 MiB copy then the configuration's attention calls, for counter runs")
    ap.add_argument("--summarize-counters", nargs=2, metavar=("CFG", "DIR"))
    ap.add_argument("--summarize-trace", metavar="DB")
    ap.add_argument("--command", default="rocprofv3 --kernel-trace --stats -d gpurun_out/ktrace "
                    "-o run -- python3 bench.py --no-cpu")
    ap.add_argument("--out", default=os.path.join(ROOT, "profiles", "summary.txt"))
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


def _stats(ms):
    ms = sorted(ms)
    n = len(ms)
    med = ms[n // 2] if n % 2 else 0.5 * (ms[n // 2 - 1] + ms[n // 2])
    return {"median": med, "min": ms[0], "max": ms[-1], "n": n}


def replay_stats(torch, call, n_units: int, steps: int, reps: int):
    """Time `steps` consecutive calls, call(u) for u = j, j+1, ... (mod
    n_units), as one HIP graph replay between two events; `reps` replays.
    Graph j starts at unit (j * steps) mod n_units, and the graphs are
    replayed in turn, so successive replays keep walking the units (every
    unit's data leaves the 256 MB Infinity Cache before it is read again).
    Returns ms per call: median, min and max over the replays."""
    import math

    n_graphs = n_units // math.gcd(steps, n_units)
    # Capture on a stream of our own, after one eager pass over the units on
    # it, so split-K workspaces kept per stream exist before the capture.
    cs = torch.cuda.Stream()
    cs.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(cs):
        for u in range(n_units):
            call(u)
    torch.cuda.synchronize()
    graphs = []
    for j in range(n_graphs):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=cs):
            for i in range(steps):
                call((j * steps + i) % n_units)
        graphs.append(g)
    for g in graphs:  # one untimed replay each
        g.replay()
    torch.cuda.synchronize()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(reps)]
    for k, (s, e) in enumerate(evs):
        s.record()
        graphs[k % n_graphs].replay()
        e.record()
    torch.cuda.synchronize()
    out = _stats([s.elapsed_time(e) / steps for s, e in evs])
    del graphs
    return out


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

    def time_layers(self, steps, reps):
        """update_and_attention layer calls: `steps` per graph replay, `reps`
        replays; ms per call (median / min / max)."""
        return replay_stats(self.torch, lambda i: self.layer_call(i, self.stream()),
                            len(self.caches), steps, reps)

    def time_eager(self, steps):
        """`steps` eager layer calls (launch overhead included), bracketed by
        synchronizations; ms per call."""
        n = len(self.caches)
        it = iter(range(steps))
        return Timer(self.torch).run(lambda: self.layer_call(next(it) % n, self.stream()),
                                     steps) / steps

    def time_attention(self, steps, reps):
        """Attention-only calls over the caches with the L new rows appended."""
        n = len(self.caches)
        for i in range(n):
            self.caches[i][0].update(self.kn[i], self.vn[i])
        st = replay_stats(self.torch, lambda i: self.attn_call(i, self.stream()), n, steps, reps)
        for i in range(n):
            self.caches[i][0].trim(self.L)
        return st

    def warm(self, n_calls):
        n = len(self.caches)
        for j in range(max(1, n_calls)):
            self.layer_call(j % n, self.stream())
        self.torch.cuda.synchronize()

    def close(self):
        for c, _ in self.caches:
            c.close()
        self.caches = []
        self.torch.cuda.empty_cache()


def bench_decode(torch, qw_amd, steps: int, warmup: int, reps: int, bits: int = 4,
                 T_prefix: int = 32768, mode=None):
    """Config 2 (bits 4, 32768 + 1) or config 1 (bits 8, 4095 + 1); `mode`
    overrides the cache mode (e.g. "int8", stored in the 8-bit layout)."""
    ls = LayerSet(torch, qw_amd, 2, bits, T_prefix, 1, LAYERS, causal=False, mode=mode)
    ls.warm(warmup)
    eager_ms = ls.time_eager(steps)
    layer = ls.time_layers(steps, reps)
    attn = ls.time_attention(steps, reps)
    T = ls.T
    ls.close()
    bytes_attn = T * HKV * kv_bytes_per_token_head(bits) + 2 * HQ * D * 2
    bytes_layer = bytes_attn + 2 * HKV * D * 2 + HKV * kv_bytes_per_token_head(bits) // 2
    return {"T": T, "bits": bits, "layer": layer, "layer_ms": layer["median"],
            "eager_layer_ms": eager_ms, "attn": attn, "attn_ms": attn["median"],
            "bytes_layer": bytes_layer, "bytes_attn": bytes_attn}


def bench_rope_decode(torch, qw_amd, reps: int, mode=None, T_prefix: int = 32768,
                      rope_dims: int = 64, L: int = 1):
    """The served decode step from the QKV projection at the config-2
    geometry (4-bit unless `mode`): RoPE of L tokens (a quarter of the dims
    rotated, Qwen3-Next's partial rotary), their append and the attention
    (causal for a verify block, L > 1). Three forms, graph-replayed over 16
    caches, each call then trimmed: qw_kv_rope_update_and_attention (one
    attention launch plus the merge); the reference's two calls
    (qw_fused_rope_qk_append, then qw_kv_update_and_attention on its q, k,
    v); qw_kv_rope_update then qw_kv_attention."""
    causal = L > 1
    ls = LayerSet(torch, qw_amd, 7, 4, T_prefix, L, LAYERS, causal=causal, mode=mode)
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(8)
    W = (HQ + 2 * HKV) * D
    qkv = [torch.randn((1, L, W), device=dev, generator=g).half() for _ in ls.caches]
    qo = [torch.empty((HQ, L, D), dtype=torch.float16, device=dev) for _ in ls.caches]
    kr = [torch.empty((HKV, L, D), dtype=torch.float16, device=dev) for _ in ls.caches]
    vr = [torch.empty((HKV, L, D), dtype=torch.float16, device=dev) for _ in ls.caches]
    cz = int(causal)
    lib = ls.lib
    base, pos = 1e7, T_prefix

    def one(i, st):
        c = ls.caches[i][0]
        ls._check(lib.qw_kv_rope_update_and_attention(c._h, qkv[i].data_ptr(), HQ, L, rope_dims,
                                                      0, base, 1.0, pos, 1.0 / 16, cz,
                                                      qo[i].data_ptr(), ls.out[i].data_ptr(), st))
        c.trim(L)

    def two(i, st):
        c = ls.caches[i][0]
        ls._check(lib.qw_fused_rope_qk_append(qkv[i].data_ptr(), 1, L, HQ, HKV, D, rope_dims, base,
                                              1.0, 0, pos, 0, qo[i].data_ptr(), kr[i].data_ptr(),
                                              vr[i].data_ptr(), st))
        ls._check(lib.qw_kv_update_and_attention(c._h, qo[i].data_ptr(), HQ, L, kr[i].data_ptr(),
                                                 vr[i].data_ptr(), 1.0 / 16, cz,
                                                 ls.out[i].data_ptr(), st))
        c.trim(L)

    def split(i, st):
        c = ls.caches[i][0]
        ls._check(lib.qw_kv_rope_update(c._h, qkv[i].data_ptr(), HQ, L, rope_dims, 0, base, 1.0,
                                        pos, qo[i].data_ptr(), st))
        ls._check(lib.qw_kv_attention(c._h, qo[i].data_ptr(), HQ, L, 1.0 / 16, cz,
                                      ls.out[i].data_ptr(), st))
        c.trim(L)

    n = len(ls.caches)
    res = {}
    for name, fn in (("one_launch", one), ("reference_calls", two), ("rope_update_then_attention", split)):
        res[name] = replay_stats(torch, lambda i, f=fn: f(i, ls.stream()), n, n, reps)["median"]
    ls.close()
    return res


def bench_general_options(torch, qw_amd, reps: int, L: int = 1, T_prefix: int = 32768,
                          window: int = 4096, softcap: float = 30.0):
    """causal_attention's sliding window and softcap (lib.rs:3185) over the
    config-2 caches as they are (4-bit, L causal rows), graph-replayed over 16
    caches like the headline: qw_kv_attention (no option), then
    qw_kv_attention_general with the window, and with the softcap (both run
    the fused block kernel on the codes)."""
    ls = LayerSet(torch, qw_amd, 11, 4, T_prefix, L, LAYERS, causal=True)
    lib = ls.lib

    def plain(i, st):
        c = ls.caches[i][0]
        ls._check(lib.qw_kv_attention(c._h, ls.q[i].data_ptr(), HQ, L, 1.0 / 16, 1,
                                      ls.out[i].data_ptr(), st))

    def general(i, st, w, cap):
        c = ls.caches[i][0]
        ls._check(lib.qw_kv_attention_general(c._h, ls.q[i].data_ptr(), HQ, L, 1.0 / 16, 1, w,
                                              cap, None, 0, 0, 0, ls.out[i].data_ptr(), st))

    n = len(ls.caches)
    res = {}
    for name, fn in (("attention", plain),
                     (f"window_{window}", lambda i, st: general(i, st, window, 0.0)),
                     (f"softcap_{int(softcap)}", lambda i, st: general(i, st, 0, softcap))):
        res[name] = replay_stats(torch, lambda i, f=fn: f(i, ls.stream()), n, n, reps)["median"]
    ls.close()
    return res


def bench_turbo4_verify(torch, qw_amd, steps: int, warmup: int, reps: int,
                        T_prefix: int = 32768, L: int = 4):
    """A Turbo4 causal verify block (L draft rows, the reference's fused-pass
    case) at the config-2 geometry: update_and_causal_attention of L tokens,
    routed to the fused verify kernel (scored straight from the packed codes).
    Graph-replayed like the affine paths; the eager figure beside it."""
    ls = LayerSet(torch, qw_amd, 4, 4, T_prefix, L, LAYERS, causal=True, mode="turbo4")
    ls.warm(warmup)
    eager_ms = ls.time_eager(steps)
    layer = ls.time_layers(steps, reps)
    T = ls.T
    ls.close()
    return {"T": T, "L": L, "layer_ms": layer["median"], "eager_layer_ms": eager_ms}


def bench_turbo4_decode(torch, qw_amd, steps: int, warmup: int, reps: int,
                        T_prefix: int = 32768):
    """The reference's served default KV mode at the config-2 geometry:
    update_and_attention of one token on a Turbo4 cache (append the token; the
    decode kernel rotates q and reads the packed indices in place; the merge
    rotates the output back). Graph-replayed like the affine paths; the eager
    figure beside it."""
    ls = LayerSet(torch, qw_amd, 3, 4, T_prefix, 1, LAYERS, causal=False, mode="turbo4")
    ls.warm(warmup)
    eager_ms = ls.time_eager(steps)
    layer = ls.time_layers(steps, reps)
    T = ls.T
    ls.close()
    return {"T": T, "layer_ms": layer["median"], "eager_layer_ms": eager_ms}


def bench_select(torch, qw_amd, reps: int, T: int = 131072):
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
    ms = replay_stats(torch, lambda i: call(), 1, LAYERS, reps)["median"]
    return {"ms": ms, "buckets": n_b, "list_len": int(lengths.item()), "width": W}


def bench_rope(torch, qw_amd, reps: int, L: int = 2048):
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
    chunk_ms = replay_stats(torch, lambda i: chunk(), 1, LAYERS, reps)["median"]
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
    one_ms = replay_stats(torch, lambda i: one(), 1, LAYERS, reps)["median"]
    cache.close()
    return {"chunk_ms": chunk_ms, "chunk_bytes": 2 * L * W * 2, "token_ms": one_ms}


def bench_block(torch, qw_amd, reps: int, bits: int, T_prefix: int, L: int, layers: int,
                causal: bool = True):
    """Config 3 (prefill chunk) / config 4 (verify block) and the served
    verify blocks: append L rows and attend them causally, graph-replayed over
    `layers` caches (one call a cache a replay, `reps` replays)."""
    ls = LayerSet(torch, qw_amd, 3 + L, bits, T_prefix, L, layers, causal=causal)
    ls.warm(layers)
    layer = ls.time_layers(layers, reps)
    attn = ls.time_attention(layers, reps)
    T = ls.T
    ls.close()
    flops = attn_flops(L, T, causal)
    kv = T * HKV * kv_bytes_per_token_head(bits)
    return {"T": T, "L": L, "bits": bits, "layer": layer, "layer_ms": layer["median"],
            "attn": attn, "attn_ms": attn["median"], "flops": flops, "kv_bytes": kv}


def bench_dlsa(torch, qw_amd, reps: int, T: int = 131072, layers: int = LAYERS):
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
    for i in range(layers):  # reps = 0: these `layers` calls only (the counter workload)
        call(i, st)
    torch.cuda.synchronize()
    if reps == 0:
        return {"T": T, "W": int(W)}
    st = replay_stats(torch, lambda i: call(i, torch.cuda.current_stream(dev).cuda_stream),
                      layers, layers, reps)
    ms = st["median"]
    bytes_call = W * HKV * 2 * D * 2 + HQ * D * 2 * 2 + W * 4
    del ks, vs
    torch.cuda.empty_cache()
    return {"T": T, "W": int(W), "ms": ms, "stats": st, "bytes": bytes_call}


def bench_dlsa_prefill(torch, qw_amd, reps: int, rows: int = 1536, depth: int = 32768,
                       layers: int = 2):
    """The K2 read at a prefill chunk (the reference's one-pass case, L x Hkv
    >= 160): `rows` query rows at positions depth .. depth + rows - 1 over fp16
    KV [4, depth + rows, 256], each row's list the 4 sinks, its own 512-key
    trailing window and 8 whole 512-key blocks drawn once for the chunk below
    the first row's window (4612 entries a row, as config 5). Two layers
    rotated (280 MB)."""
    import numpy as np

    dev = torch.device("cuda:0")
    T = depth + rows
    g = torch.Generator(device=dev)
    g.manual_seed(15)
    rng = np.random.default_rng(15)
    ks, vs, qs, lists, lens, outs = [], [], [], [], [], []
    for layer in range(layers):
        ks.append(torch.randn((HKV, T, D), device=dev, generator=g).half())
        vs.append(torch.randn((HKV, T, D), device=dev, generator=g).half())
        qs.append(torch.randn((HQ, rows, D), device=dev, generator=g).half())
        blocks = np.sort(rng.choice(np.arange(1, (depth - 512) // 512), 8, replace=False))
        exp = np.concatenate([np.arange(b * 512, b * 512 + 512) for b in blocks])
        pos = depth + np.arange(rows)[:, None]
        win = pos - 511 + np.arange(512)[None, :]
        lst = np.concatenate([np.broadcast_to(exp, (rows, exp.size)), win,
                              np.broadcast_to(np.arange(4), (rows, 4))], axis=1).astype(np.int32)
        lists.append(torch.from_numpy(np.ascontiguousarray(lst)).to(dev))
        lens.append(torch.full((rows,), lst.shape[1], dtype=torch.int32, device=dev))
        outs.append(torch.empty((HQ, rows, D), dtype=torch.float16, device=dev))
    W = lists[0].shape[1]
    L = qw_amd.lib()

    def call(i, st):
        k, v = ks[i], vs[i]
        rc = L.qw_dlsa_sparse_attention(qs[i].data_ptr(), k.data_ptr(), v.data_ptr(), k.stride(0),
                                        k.stride(1), v.stride(0), v.stride(1),
                                        lists[i].data_ptr(), lens[i].data_ptr(), rows, W, HQ, HKV,
                                        D, T, D ** -0.5, outs[i].data_ptr(), st)
        assert rc == 0, L.qw_last_error()

    st = replay_stats(torch, lambda i: call(i, torch.cuda.current_stream(dev).cuda_stream),
                      layers, layers, reps)
    del ks, vs
    torch.cuda.empty_cache()
    gathered = rows * W * HKV * 2 * D * 2  # K and V rows each row's list reads
    flops = 4 * D * HQ * rows * W
    return {"T": T, "W": int(W), "rows": rows, "ms": st["median"], "stats": st,
            "gathered_bytes": gathered, "flops": flops}


def bench_dlsa_cache(torch, qw_amd, reps: int, T: int = 131072, layers: int = LAYERS):
    """Config 5 through an fp16 KV cache read in place (qw_kv_dlsa_attention):
    the same lists as bench_dlsa over caches holding the same kind of rows."""
    import numpy as np

    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(5)
    rng = np.random.default_rng(5)
    caches, qs, lists, lens, outs = [], [], [], [], []
    for layer in range(layers):
        c = qw_amd.KVCache("fp16", HKV, D, capacity=T)
        for t0 in range(0, T, 16384):
            c.update(torch.randn((HKV, 16384, D), device=dev, generator=g).half(),
                     torch.randn((HKV, 16384, D), device=dev, generator=g).half())
        caches.append(c)
        qs.append(torch.randn((HQ, 1, D), device=dev, generator=g).half())
        blocks = np.sort(rng.choice(np.arange(1, (T - 512) // 512), 8, replace=False))
        lst = np.concatenate([np.concatenate([np.arange(b * 512, b * 512 + 512) for b in blocks]),
                              np.arange(T - 512, T), np.arange(4)]).astype(np.int32)
        lists.append(torch.from_numpy(lst[None]).to(dev))
        lens.append(torch.tensor([lst.size], dtype=torch.int32, device=dev))
        outs.append(torch.empty((HQ, 1, D), dtype=torch.float16, device=dev))
    W = lists[0].shape[1]
    L = qw_amd.lib()

    def call(i, st):
        rc = L.qw_kv_dlsa_attention(caches[i]._h, qs[i].data_ptr(), HQ, 1, lists[i].data_ptr(),
                                    lens[i].data_ptr(), W, D ** -0.5, outs[i].data_ptr(), st)
        assert rc == 0, L.qw_last_error()

    st = replay_stats(torch, lambda i: call(i, torch.cuda.current_stream(dev).cuda_stream),
                      layers, layers, reps)
    for c in caches:
        c.close()
    torch.cuda.empty_cache()
    bytes_call = W * HKV * 2 * D * 2 + HQ * D * 2 * 2 + W * 4
    return {"T": T, "W": int(W), "ms": st["median"], "stats": st, "bytes": bytes_call}


def _ceil_lib(qw_amd):
    import ctypes

    path = os.path.join(os.path.dirname(os.path.abspath(qw_amd.__file__)), "libqwceil.so")
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is missing: run `python -m qw_amd.build`")
    L = ctypes.CDLL(path)
    L.qwc_read.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int,
                           ctypes.c_int, ctypes.c_void_p]
    L.qwc_copy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int,
                           ctypes.c_void_p]
    return L


def bench_ceilings(torch, qw_amd, reps: int):
    """The box's ceilings, measured:
    - a 2 GiB device-to-device copy (a 128-bit grid-stride copy kernel, and
      torch's copy_), reported as bytes moved (read + write) per second;
    - the config-2 read floor: every byte of 16 rotated 37.8 MB buffers (the
      size of one config-2 attention call's KV, 604 MB in all, more than the
      256 MB MALL) read once by a plain load-and-XOR kernel, graph-replayed
      like the headline; the best of a sweep of grids and loads in flight;
    - the same read kernel over one 2 GiB buffer (the stream rate);
    - torch.matmul fp16 8192^3 (hipBLASLt), TFLOP/s."""
    dev = torch.device("cuda:0")
    L = _ceil_lib(qw_amd)
    out = {}

    def st():
        return torch.cuda.current_stream(dev).cuda_stream

    def time_fn(fn, iters):
        fn()
        torch.cuda.synchronize()
        ms = []
        for _ in range(iters):
            s = torch.cuda.Event(enable_timing=True)
            e = torch.cuda.Event(enable_timing=True)
            s.record()
            fn()
            e.record()
            torch.cuda.synchronize()
            ms.append(s.elapsed_time(e))
        return _stats(ms)

    nb = 2 << 30
    src = torch.empty(nb, dtype=torch.uint8, device=dev)
    dst = torch.empty(nb, dtype=torch.uint8, device=dev)
    src.fill_(1)
    sink = torch.zeros(2048 * 512, dtype=torch.int32, device=dev)

    def copy_k():
        rc = L.qwc_copy(dst.data_ptr(), src.data_ptr(), nb, 4096, st())
        assert rc == 0, rc

    ck = time_fn(copy_k, 20)
    ct = time_fn(lambda: dst.copy_(src), 20)
    out["copy_2GiB"] = {
        "GB_s_kernel": round(2 * nb / (ck["median"] * 1e-3) / 1e9, 1),
        "GB_s_torch_copy": round(2 * nb / (ct["median"] * 1e-3) / 1e9, 1),
        "ms_kernel": round(ck["median"], 4), "bytes_moved": 2 * nb,
        "note": "GB/s counts the bytes read plus the bytes written"}

    def read_big(blocks, unroll):
        rc = L.qwc_read(src.data_ptr(), nb, sink.data_ptr(), blocks, unroll, st())
        assert rc == 0, rc

    best = None
    for blocks in (1024, 2048):
        for unroll in (2, 4, 8):
            r = time_fn(lambda: read_big(blocks, unroll), 10)
            gbs = nb / (r["median"] * 1e-3) / 1e9
            if best is None or gbs > best[0]:
                best = (gbs, blocks, unroll)
    out["read_2GiB"] = {"GB_s": round(best[0], 1), "blocks": best[1], "unroll": best[2]}
    del src, dst
    torch.cuda.empty_cache()

    # the config-2-sized read floor
    c2_bytes = 32769 * HKV * kv_bytes_per_token_head(4) + 2 * HQ * D * 2
    rb = (c2_bytes + 1023) // 1024 * 1024
    bufs = [torch.empty(rb, dtype=torch.uint8, device=dev).fill_(i + 1) for i in range(LAYERS)]
    sweep = {}
    best = None
    for blocks in (256, 512, 1024):
        for unroll in (1, 2, 4):
            def call(i, blocks=blocks, unroll=unroll):
                rc = L.qwc_read(bufs[i].data_ptr(), rb, sink.data_ptr(), blocks, unroll, st())
                assert rc == 0, rc
            r = replay_stats(torch, call, LAYERS, LAYERS, reps)
            sweep[f"{blocks}x{unroll}"] = round(r["median"] * 1e3, 3)
            if best is None or r["median"] < best[0]["median"]:
                best = (r, blocks, unroll)
    r, blocks, unroll = best
    out["read_c2_size"] = {
        "us": round(r["median"] * 1e3, 3), "GB_s": round(rb / (r["median"] * 1e-3) / 1e9, 1),
        "bytes": rb, "blocks": blocks, "unroll": unroll, "sweep_us": sweep,
        "note": "16 rotated buffers, one graph of 16 reads, median of the replays"}
    del bufs
    torch.cuda.empty_cache()

    n = 8192
    a = torch.randn((n, n), device=dev, dtype=torch.float16)
    b = torch.randn((n, n), device=dev, dtype=torch.float16)
    r = time_fn(lambda: torch.matmul(a, b), 20)
    out["gemm_fp16_8192"] = {"TFLOP_s": round(2 * n ** 3 / (r["median"] * 1e-3) / 1e12, 1),
                             "ms": round(r["median"], 4), "route": "torch.matmul (hipBLASLt)"}
    del a, b
    torch.cuda.empty_cache()
    return out


def cpu_threads():
    """Threads for the CPU baseline: every core this process may run on,
    capped by OMP_NUM_THREADS when the environment sets it (the GPU box's
    harness sets it to the box's CPU share)."""
    try:
        n = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        n = os.cpu_count() or 1
    omp = os.environ.get("OMP_NUM_THREADS", "")
    if omp.isdigit() and int(omp) > 0:
        n = min(n, int(omp))
    return max(1, n)


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


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
#
# Per configuration, four rocprofv3 --pmc passes of `bench.py --pmc-workload
# <cfg>` (one pass a counter group; rocprofv3 does not split counters over
# passes), then `bench.py --summarize-counters <cfg> <dir>` writes
# profiles/counters_<cfg>.txt:
#   fetch  FETCH_SIZE                      (KiB read from memory per dispatch)
#   write  WRITE_SIZE                      (KiB written)
#   ea     TCC_EA0_RDREQ_{32B,64B,128B,DRAM}_sum (read requests by size, and
#          those addressed to DRAM: bytes = 32 n32 + 64 n64 + 128 n128)
#   mfma   SQ_VALU_MFMA_BUSY_CYCLES SQ_INSTS_VALU_MFMA_MOPS_F16 SQ_INSTS_VALU
#          SQ_INSTS_MFMA SQ_BUSY_CYCLES GRBM_GUI_ACTIVE
# Each workload first runs one plain 256 MiB device copy (HIP's copyBuffer):
# its counter readings for a known byte count calibrate the byte counters.

PMC_PASSES = {
    "fetch": "FETCH_SIZE",
    "write": "WRITE_SIZE",
    "ea": "TCC_EA0_RDREQ_32B_sum TCC_EA0_RDREQ_64B_sum TCC_EA0_RDREQ_128B_sum "
          "TCC_EA0_RDREQ_DRAM_sum",
    "mfma": "SQ_VALU_MFMA_BUSY_CYCLES SQ_INSTS_VALU_MFMA_MOPS_F16 SQ_INSTS_VALU SQ_INSTS_MFMA "
            "SQ_BUSY_CYCLES GRBM_GUI_ACTIVE",
}
PMC_CONFIGS = {
    # cfg: (what the dispatches are, algorithmic bytes a call, algorithmic flops a call)
    "c1": "config 1: 16 qw_kv_attention calls, 8-bit, 4096 keys, 16 caches",
    "c2": "config 2: 16 qw_kv_attention calls, 4-bit, 32769 keys, 16 caches",
    "c3": "config 3: 4 qw_kv_attention calls, 2048 causal rows over 18432 keys, 8-bit, 4 caches",
    "c4": "config 4: 16 qw_kv_attention calls, 16 causal rows over 65552 keys, 4-bit, 16 caches",
    "c5": "config 5: 16 qw_dlsa_sparse_attention calls, 4612-entry list, fp16 KV, 16 layers",
    "gemm": "the MFMA ceiling: 3 torch.matmul calls, fp16 8192 x 8192 x 8192 (hipBLASLt)",
}
GEMM_N = 8192


def pmc_algorithmic(cfg: str):
    """(bytes, flops) of one call of the configuration's attention."""
    if cfg == "c1":
        T = 4096
        return T * HKV * kv_bytes_per_token_head(8) + 2 * HQ * D * 2, attn_flops(1, T, False)
    if cfg == "c2":
        T = 32769
        return T * HKV * kv_bytes_per_token_head(4) + 2 * HQ * D * 2, attn_flops(1, T, False)
    if cfg == "c3":
        T, L = 18432, 2048
        return T * HKV * kv_bytes_per_token_head(8) + 2 * HQ * L * D * 2, attn_flops(L, T, True)
    if cfg == "c4":
        T, L = 65552, 16
        return T * HKV * kv_bytes_per_token_head(4) + 2 * HQ * L * D * 2, attn_flops(L, T, True)
    if cfg == "gemm":
        return 3 * GEMM_N * GEMM_N * 2, 2 * GEMM_N ** 3
    W = 4612
    return W * HKV * 2 * D * 2 + HQ * D * 2 * 2 + W * 4, 4 * D * HQ * W


def pmc_workload(cfg: str) -> int:
    """What the rocprofv3 --pmc passes profile: one plain 256 MiB device copy
    (the calibration kernel, HIP's copyBuffer), then the configuration's
    attention calls over distinct caches."""
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
    if cfg == "gemm":
        a = torch.randn((GEMM_N, GEMM_N), device="cuda:0", dtype=torch.float16)
        b = torch.randn((GEMM_N, GEMM_N), device="cuda:0", dtype=torch.float16)
        for _ in range(PMC_CALLS["gemm"]):
            torch.matmul(a, b)
        torch.cuda.synchronize()
        print("pmc workload gemm done", flush=True)
        return 0
    if cfg == "c5":
        bench_dlsa(torch, qw_amd, 0)
        print("pmc workload c5 done", flush=True)
        return 0
    bits, T0, L, n, causal = {"c1": (8, 4095, 1, LAYERS, False),
                              "c2": (4, 32768, 1, LAYERS, False),
                              "c3": (8, 16384, 2048, 4, True),
                              "c4": (4, 65536, 16, LAYERS, True)}[cfg]
    ls = LayerSet(torch, qw_amd, 2, bits, T0, L, n, causal=causal)
    for i in range(n):
        ls.caches[i][0].update(ls.kn[i], ls.vn[i])
    torch.cuda.synchronize()
    for i in range(n):
        ls.attn_call(i, ls.stream())
    torch.cuda.synchronize()
    ls.close()
    print(f"pmc workload {cfg} done", flush=True)
    return 0


PMC_CALLS = {"c1": LAYERS, "c2": LAYERS, "c3": 4, "c4": LAYERS, "c5": LAYERS, "gemm": 3}
# the kernels a call of the configuration launches (set-up appends excluded)
PMC_KERNELS = ("attend_decode_kernel", "attend_block_kernel", "decode_merge_kernel",
               "merge_rows_", "t4_merge_rotate_kernel", "dlsa_kernel", "dlsa_merge_kernel")
N_XCD, N_SIMD = 8, 1024  # MI355X: 8 XCDs, 256 CUs x 4 SIMDs


def _pmc_rows(root: str, ps: str):
    """(kernel, dispatch, counter, value, duration_ns) rows of one pass, from a
    rocprofv3 results database under root/ps, or from root/ps.tsv (the same
    table's rows dumped as text)."""
    import csv
    import glob
    import sqlite3

    tsv = os.path.join(root, f"{ps}.tsv")
    if os.path.exists(tsv):
        with open(tsv) as f:
            rd = csv.DictReader(f, delimiter="\t")
            return [(r["kernel_name"], r["dispatch_id"], r["counter_name"], float(r["value"]),
                     float(r["duration"])) for r in rd]
    hits = sorted(glob.glob(os.path.join(root, ps, "**", "*results.db"), recursive=True))
    if not hits:
        raise FileNotFoundError(f"no rocprofv3 results under {root}/{ps}")
    con = sqlite3.connect(hits[-1])
    tabs = [r[0] for r in con.execute("select name from sqlite_master where type in ('table', 'view')")]
    ctab = next(t for t in tabs if t.startswith("counters_collection"))
    q = f"select kernel_name, dispatch_id, counter_name, value, duration from {ctab}"
    return [(n, d, c, float(v), float(du)) for n, d, c, v, du in con.execute(q)]


def _short(name: str) -> str:
    base = name.split("(")[0]
    return base.replace("void ", "").replace("qw::", "")[:60]


def summarize_counters(cfg: str, root: str, out: str) -> int:
    """profiles/counters_<cfg>.txt from the four passes under root: per call
    of the configuration's attention (every dispatch of its kernels summed and
    divided by the number of calls), bytes read and written, and MFMA
    figures."""
    per = {}   # kernel -> dispatch -> {counter: value, "dur": ns}
    for ps in PMC_PASSES:
        for name, disp, counter, value, dur in _pmc_rows(root, ps):
            d = per.setdefault(name, {}).setdefault((ps, disp), {})
            d[counter] = d.get(counter, 0.0) + value
            d["dur"] = dur

    def total(name, counter):
        return sum(d.get(counter, 0.0) for d in per[name].values())

    def biggest(name, counter):
        return max(d.get(counter, 0.0) for d in per[name].values())

    copy_k = next(n for n in per if "copyBuffer" in n)
    cf, cw = biggest(copy_k, "FETCH_SIZE"), biggest(copy_k, "WRITE_SIZE")
    n32, n64, n128 = (biggest(copy_k, f"TCC_EA0_RDREQ_{b}_sum") for b in ("32B", "64B", "128B"))
    copy_ea = 32 * n32 + 64 * n64 + 128 * n128
    f_scale = (COPY_BYTES / 1024.0) / cf
    w_scale = (COPY_BYTES / 1024.0) / cw
    alg_bytes, alg_flops = pmc_algorithmic(cfg)
    calls = PMC_CALLS[cfg]
    ours = [n for n in per if any(k in n for k in PMC_KERNELS)] if cfg != "gemm" else \
        [n for n in per if "copyBuffer" not in n and "elementwise" not in n.lower()
         and "distribution" not in n.lower()]
    lines = [f"# Counters of {PMC_CONFIGS[cfg]} (rocprofv3 --pmc)", "", "commands:"]
    for ps, counters in PMC_PASSES.items():
        lines.append(f"  rocprofv3 --pmc {counters} -d gpurun_out/pmc_{cfg}/{ps} -o run -- "
                     f"python3 bench.py --pmc-workload {cfg}")
    lines += [f"  python3 bench.py --summarize-counters {cfg} gpurun_out/pmc_{cfg} "
              f"--out profiles/counters_{cfg}.txt", "",
              f"calibration, a copy of {COPY_BYTES} B ({_short(copy_k)}):",
              f"  FETCH_SIZE {cf:.1f} KiB -> x{f_scale:.4f} (it counts a 128-byte request as 64); "
              f"WRITE_SIZE {cw:.1f} KiB -> x{w_scale:.4f}",
              f"  EA read requests 32B/64B/128B {n32:.0f}/{n64:.0f}/{n128:.0f} = {copy_ea:.0f} B "
              f"({copy_ea / COPY_BYTES:.4f} of the true count)",
              f"per call: algorithmic {alg_bytes} B and {alg_flops} flop; {calls} calls profiled",
              "MFMA busy = SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE / 8 XCDs x 1024 SIMDs); "
              "clock = GRBM_GUI_ACTIVE / 8 / duration",
              "(GRBM_GUI_ACTIVE spans the profiler's whole dispatch window: for kernels of a few "
              "tens of us the clock reads high and MFMA busy low; trust them on long kernels)", ""]
    tot = {"read": 0.0, "write": 0.0, "ea": 0.0, "dram": 0.0, "flop": 0.0, "busy": 0.0,
           "simd_cycles": 0.0}
    for name in sorted(ours):
        disp = {d for (ps, d) in per[name] if ps == "fetch"}
        n = max(1, len(disp))
        rd = total(name, "FETCH_SIZE") * f_scale * 1024.0 / calls
        wr = total(name, "WRITE_SIZE") * w_scale * 1024.0 / calls
        e32, e64, e128 = (total(name, f"TCC_EA0_RDREQ_{b}_sum") for b in ("32B", "64B", "128B"))
        ea = (32 * e32 + 64 * e64 + 128 * e128) / calls
        req = e32 + e64 + e128
        dram = ea * (total(name, "TCC_EA0_RDREQ_DRAM_sum") / req if req else 0.0)
        busy = total(name, "SQ_VALU_MFMA_BUSY_CYCLES") / calls
        gui = total(name, "GRBM_GUI_ACTIVE") / calls
        mfd = [d for (ps, _), d in per[name].items() if ps == "mfma"]
        dur = sum(d["dur"] for d in mfd) / calls
        flop = total(name, "SQ_INSTS_VALU_MFMA_MOPS_F16") * 512 / calls
        simd = gui / N_XCD * N_SIMD
        clk = gui / N_XCD / dur if dur else 0.0
        for k, v in (("read", rd), ("write", wr), ("ea", ea), ("dram", dram), ("flop", flop),
                     ("busy", busy), ("simd_cycles", simd)):
            tot[k] += v
        lines += [f"kernel {_short(name)}: {n} dispatches, {n / calls:g} a call; per call:",
                  f"  read {rd:.0f} B (FETCH_SIZE), {ea:.0f} B (EA requests, "
                  f"{dram / ea if ea else 0:.3f} to DRAM); write {wr:.0f} B",
                  f"  {dur / 1e3:.2f} us under the profiler, clock {clk:.2f} GHz; MFMA busy "
                  f"{busy / simd if simd else 0:.4f}, MFMA flop {flop:.4g}, SQ_INSTS_VALU "
                  f"{total(name, 'SQ_INSTS_VALU') / calls:.0f}, SQ_INSTS_MFMA "
                  f"{total(name, 'SQ_INSTS_MFMA') / calls:.0f}"]
    lines += ["", "per call, all of the call's kernels:",
              f"traffic_bytes_per_call = {tot['read'] + tot['write']:.0f}",
              f"read_bytes_per_call = {tot['read']:.0f}",
              f"write_bytes_per_call = {tot['write']:.0f}",
              f"dram_read_bytes_per_call = {tot['dram']:.0f}",
              f"traffic / algorithmic = {(tot['read'] + tot['write']) / alg_bytes:.4f}",
              f"mfma_flop_per_call = {tot['flop']:.0f}",
              f"mfma_flop / algorithmic = {tot['flop'] / alg_flops:.4f}",
              f"mfma_busy = {tot['busy'] / tot['simd_cycles'] if tot['simd_cycles'] else 0:.4f}"]
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


def read_counters(cfg: str):
    """The committed counter summary of a configuration, as numbers (per call
    of its attention): bytes read/written, DRAM read bytes, MFMA busy."""
    out = {}
    keys = ("traffic_bytes_per_call", "read_bytes_per_call", "write_bytes_per_call",
            "dram_read_bytes_per_call", "mfma_flop_per_call", "mfma_busy")
    try:
        with open(os.path.join(ROOT, "profiles", f"counters_{cfg}.txt")) as f:
            for line in f:
                for key in keys:
                    if line.startswith(key + " ="):
                        v = float(line.split("=")[1])
                        out[key] = v if key == "mfma_busy" else int(v)
    except OSError:
        pass
    return out


def _round_stats(st, scale=1e3, nd=3):
    return {k: (round(v * scale, nd) if k != "n" else v) for k, v in st.items()}


def main() -> int:
    args = parse()
    if args.summarize_counters:
        return summarize_counters(args.summarize_counters[0], args.summarize_counters[1],
                                  args.out)
    if args.summarize_trace:
        return summarize_trace(args.summarize_trace, args.out, args.command)
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only: the path shards by KV head "
                          "across GPUs in design, which is not implemented; run with --gpus 1"}))
        return 2
    if args.pmc_workload:
        return pmc_workload(args.pmc_workload)
    import torch

    import qw_amd

    qw_amd.lib()  # fail loudly if the HIP library is missing
    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU visible"}))
        return 2
    torch.cuda.set_device(0)
    steps, reps = max(1, args.steps), max(50, args.reps)
    log("bench: measured ceilings (copy, config-2-sized read floor, fp16 GEMM)")
    ceil = bench_ceilings(torch, qw_amd, reps)
    log(f"bench: config 2 decode, {steps} steps a replay, {reps} replays, warmup {args.warmup}")
    dec = bench_decode(torch, qw_amd, steps, args.warmup, reps)
    us_layer = dec["layer_ms"] * 1e3
    value = dec["bytes_layer"] / (dec["layer_ms"] * 1e-3) / 1e9
    achieved = dec["bytes_attn"] / (dec["attn_ms"] * 1e-3) / 1e9
    c2c = read_counters("c2")
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
        "timing": {"method": f"HIP graph of exactly {steps} layer calls (cycling the "
                             f"{LAYERS} caches), {reps} replays, each between its own events; "
                             "ms_per_step is the median",
                   "ms_per_step": _round_stats(dec["layer"], 1.0, 6)},
        "us_per_layer": round(us_layer, 3),
        "us_per_layer_eager": round(dec["eager_layer_ms"] * 1e3, 3),
        "us_attention": round(dec["attn_ms"] * 1e3, 3),
        "us_attention_stats": _round_stats(dec["attn"]),
        "layer_calls_per_s": round(1.0 / (dec["layer_ms"] * 1e-3), 1),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "peak_measured": ceil["read_2GiB"]["GB_s"],
                     "frac_measured": round(achieved / ceil["read_2GiB"]["GB_s"], 4),
                     "read_floor_us": ceil["read_c2_size"]["us"],
                     "peak_measured_note": "peak_measured: a plain read kernel over 2 GiB on this "
                                           "box; read_floor_us: the same kernel reading 16 rotated "
                                           "config-2-sized buffers, timed like the headline",
                     "traffic": c2c.get("traffic_bytes_per_call"),
                     "kernel": "qw_kv_attention: attend_decode_kernel + decode_merge_kernel, "
                               "graph-replayed over 16 caches",
                     "algorithmic_bytes": dec["bytes_attn"],
                     "dram_read_bytes": c2c.get("dram_read_bytes_per_call")},
    }
    if not args.no_extra:
        extra = {"ceilings": ceil}
        log("bench: config 3 prefill chunk")
        pf = bench_block(torch, qw_amd, reps, 8, 16384, 2048, 4)
        tf = pf["flops"] / (pf["attn_ms"] * 1e-3) / 1e12
        c3c = read_counters("c3")
        extra["config3_prefill"] = {
            "us_per_layer": round(pf["layer_ms"] * 1e3, 1),
            "us_attention": round(pf["attn_ms"] * 1e3, 1),
            "us_attention_stats": _round_stats(pf["attn"], 1e3, 1),
            "TFLOP_s": round(tf, 1), "frac_mfma": round(tf / MFMA_PEAK_TFLOPS, 4),
            "frac_mfma_measured": round(tf / ceil["gemm_fp16_8192"]["TFLOP_s"], 4),
            "TFLOP_s_layer": round(pf["flops"] / (pf["layer_ms"] * 1e-3) / 1e12, 1),
            "chunk_rows_per_s_one_layer": round(2048 / (pf["layer_ms"] * 1e-3), 1),
            "flops": pf["flops"], "keys": pf["T"], "rows": 2048, "kv_bits": 8,
            "layers_rotated": 4, "counters": c3c}
        log("bench: config 4 verify block")
        vf = bench_block(torch, qw_amd, reps, 4, 65536, 16, LAYERS)
        vt = vf["flops"] / (vf["attn_ms"] * 1e-3) / 1e12
        vg = vf["kv_bytes"] / (vf["attn_ms"] * 1e-3) / 1e9
        extra["config4_verify"] = {
            "us_per_layer": round(vf["layer_ms"] * 1e3, 2),
            "us_attention": round(vf["attn_ms"] * 1e3, 2),
            "us_attention_stats": _round_stats(vf["attn"], 1e3, 2),
            "TFLOP_s": round(vt, 1), "frac_mfma": round(vt / MFMA_PEAK_TFLOPS, 4),
            "GB_s": round(vg, 1), "frac_hbm": round(vg / HBM_PEAK_GBS, 4),
            "flops": vf["flops"], "kv_bytes": vf["kv_bytes"], "keys": vf["T"], "rows": 16,
            "kv_bits": 4, "counters": read_counters("c4")}
        for rows, ctx in ((4, 32768), (5, 65536)):
            log(f"bench: served verify block, {rows} rows at {ctx} (4-bit)")
            sv = bench_block(torch, qw_amd, reps, 4, ctx, rows, LAYERS)
            st = sv["flops"] / (sv["attn_ms"] * 1e-3) / 1e12
            sg = sv["kv_bytes"] / (sv["attn_ms"] * 1e-3) / 1e9
            extra[f"verify_{rows}rows_{ctx // 1024}k"] = {
                "us_per_layer": round(sv["layer_ms"] * 1e3, 2),
                "us_attention": round(sv["attn_ms"] * 1e3, 2),
                "TFLOP_s": round(st, 1), "GB_s": round(sg, 1),
                "frac_hbm": round(sg / HBM_PEAK_GBS, 4), "keys": sv["T"], "rows": rows,
                "kv_bits": 4}
        log("bench: config 5 D-LSA read")
        ds = bench_dlsa(torch, qw_amd, reps)
        gbs = ds["bytes"] / (ds["ms"] * 1e-3) / 1e9
        extra["config5_dlsa_decode"] = {
            "us_per_layer": round(ds["ms"] * 1e3, 3), "GB_s": round(gbs, 1),
            "us_stats": _round_stats(ds["stats"]),
            "frac_hbm": round(gbs / HBM_PEAK_GBS, 4), "list_width": ds["W"],
            "context": ds["T"], "algorithmic_bytes": ds["bytes"],
            "counters": read_counters("c5")}
        log("bench: config 5 D-LSA read over fp16 KV caches in place")
        dc = bench_dlsa_cache(torch, qw_amd, reps)
        gbc = dc["bytes"] / (dc["ms"] * 1e-3) / 1e9
        extra["config5_dlsa_from_cache"] = {
            "us_per_layer": round(dc["ms"] * 1e3, 3), "GB_s": round(gbc, 1),
            "frac_hbm": round(gbc / HBM_PEAK_GBS, 4), "list_width": dc["W"],
            "route": "qw_kv_dlsa_attention: K rows and 8-key V blocks of the cache read in place"}
        log("bench: D-LSA K2 read at a 1536-row prefill chunk")
        dp = bench_dlsa_prefill(torch, qw_amd, max(20, reps // 2))
        extra["dlsa_prefill_1536rows"] = {
            "ms_per_chunk": round(dp["ms"], 3), "ms_stats": _round_stats(dp["stats"], scale=1.0),
            "gathered_GB_s": round(dp["gathered_bytes"] / (dp["ms"] * 1e-3) / 1e9, 1),
            "TFLOP_s": round(dp["flops"] / (dp["ms"] * 1e-3) / 1e12, 1), "rows": dp["rows"],
            "list_width": dp["W"], "context": dp["T"],
            "note": "rows' lists share the chunk's 8 blocks; gathers hit the L2 and the MALL; "
                    "the reference publishes 38.3-44.9 ms for a 1536-row chunk on an M4 Max"}
        log("bench: config 1 decode (8-bit, 4096 keys)")
        c1 = bench_decode(torch, qw_amd, LAYERS, args.warmup, reps, bits=8, T_prefix=4095)
        extra["config1_decode"] = {
            "us_per_layer": round(c1["layer_ms"] * 1e3, 3),
            "us_attention": round(c1["attn_ms"] * 1e3, 3),
            "GB_s": round(c1["bytes_attn"] / (c1["attn_ms"] * 1e-3) / 1e9, 1)}
        log("bench: Int8 decode (config-2 geometry)")
        i8 = bench_decode(torch, qw_amd, LAYERS, args.warmup, reps, bits=8, T_prefix=32768,
                          mode="int8")
        extra["int8_decode"] = {
            "us_per_layer": round(i8["layer_ms"] * 1e3, 2),
            "us_attention": round(i8["attn_ms"] * 1e3, 2),
            "GB_s": round(i8["bytes_attn"] / (i8["attn_ms"] * 1e-3) / 1e9, 1)}
        log("bench: D-LSA K1 select")
        k1 = bench_select(torch, qw_amd, reps)
        extra["dlsa_k1_select"] = {
            "us_per_row": round(k1["ms"] * 1e3, 2), "buckets": k1["buckets"],
            "list_width": k1["width"], "list_len": k1["list_len"]}
        log("bench: fused q/k RoPE")
        rp = bench_rope(torch, qw_amd, reps)
        extra["rope"] = {
            "us_chunk_2048": round(rp["chunk_ms"] * 1e3, 2),
            "GB_s_chunk": round(rp["chunk_bytes"] / (rp["chunk_ms"] * 1e-3) / 1e9, 1),
            "us_rope_append_1_token": round(rp["token_ms"] * 1e3, 2)}
        log("bench: the decode step from the projection (RoPE, append, attention)")
        sd = {}
        for m in ("affine4", "turbo4"):
            for L_ in (1, 4):
                r_ = bench_rope_decode(torch, qw_amd, reps, mode=None if m == "affine4" else m, L=L_)
                sd[f"{m}_{L_}row" + ("s" if L_ > 1 else "")] = {k: round(v * 1e3, 2) for k, v in r_.items()}
        extra["decode_step_from_projection"] = {
            "us": sd, "rope_dims": 64, "keys": "32768 + rows", "verify": "4 rows, causal",
            "forms": "one_launch: qw_kv_rope_update_and_attention; reference_calls: "
                     "qw_fused_rope_qk_append then qw_kv_update_and_attention; "
                     "rope_update_then_attention: qw_kv_rope_update then qw_kv_attention"}
        log("bench: the general options over the config-2 caches (window, softcap)")
        go = {}
        for L_ in (1, 4):
            r_ = bench_general_options(torch, qw_amd, reps, L=L_)
            go[f"{L_}row" + ("s" if L_ > 1 else "")] = {k: round(v * 1e3, 2) for k, v in r_.items()}
        extra["general_options"] = {
            "us": go, "keys": 32768, "causal": True,
            "forms": "attention: qw_kv_attention; window_4096 / softcap_30: "
                     "qw_kv_attention_general (the fused block kernel on the codes)"}
        log("bench: Turbo4 decode (config-2 geometry)")
        t4 = bench_turbo4_decode(torch, qw_amd, LAYERS, args.warmup, reps)
        extra["turbo4_decode"] = {
            "us_per_layer": round(t4["layer_ms"] * 1e3, 2),
            "us_per_layer_eager": round(t4["eager_layer_ms"] * 1e3, 2), "keys": t4["T"],
            "route": "decode kernel: q rotated in the kernel, packed indices read in place, the new token appended in its launch; merge kernel rotates the rows back"}
        log("bench: Turbo4 fused causal verify (4 rows, config-2 geometry)")
        tv = bench_turbo4_verify(torch, qw_amd, LAYERS, args.warmup, reps)
        extra["turbo4_verify"] = {
            "us_per_layer": round(tv["layer_ms"] * 1e3, 2),
            "us_per_layer_eager": round(tv["eager_layer_ms"] * 1e3, 2), "keys": tv["T"], "rows": tv["L"],
            "route": "fused verify pass in the block kernel on the packed indices (q rotated in the kernel, rows appended in its launch); merge kernel rotates the rows back"}
        line["extra"] = extra
    if not args.no_cpu:
        threads = cpu_threads()
        log(f"bench: CPU baseline ({threads} threads, ~{args.cpu_seconds:.0f} s)")
        cb = cpu_baseline(args.cpu_seconds, threads)
        line["cpu_baseline"] = {
            "value": round(dec["bytes_layer"] / cb["s_per_call"] / 1e9, 3),
            "unit": "GB/s",
            "cores": threads,
            "kind": "port",
            "us_per_layer": round(cb["s_per_call"] * 1e6, 1),
            "nproc": os.cpu_count(),
            "cpu_model": cpu_model(),
            "sample": f"{cb['calls']} config-2 layer calls (quantize 1 token, dequantize 32769 "
                      f"keys, MLX-rounding SDPA) by the C oracle, a restatement of the MLX CPU "
                      f"stream (not MLX), threaded over (KV head x query head) on every core "
                      f"this process may use, capped by OMP_NUM_THREADS",
        }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
