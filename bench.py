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
reported beside it). Extra workloads (D-LSA config 5, config 1) are reported
under "extra"; the CPU baseline is the oracle's restatement of the MLX CPU
stream, timed on a bounded sample on this host.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-extra]
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
LAYERS = 16
HQ, HKV, D = 24, 4, 256


def kv_bytes_per_token_head(bits: int) -> int:
    """Algorithmic bytes of one (token, KV head) row of K plus V: codes plus one
    fp16 scale and bias per 64-dim group (288 B at 4-bit, 544 B at 8-bit)."""
    if bits == 16:
        return 2 * D * 2
    return 2 * (D * bits // 8 + (D // 64) * 2 * 2)


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


def bench_decode(torch, qw_amd, steps: int, warmup: int, bits: int = 4, T_prefix: int = 32768):
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(2)
    mode = {4: "affine4", 8: "affine8", 16: "fp16"}[bits]
    caches, qs, kns, vns, outs = [], [], [], [], []
    for layer in range(LAYERS):
        c = qw_amd.KVCache(mode, HKV, D, capacity=T_prefix + 1)
        jit = torch.empty((HKV, 1, 1), device=dev).uniform_(0.5, 2.0, generator=g)
        chunk = 8192
        for t0 in range(0, T_prefix, chunk):
            n = min(chunk, T_prefix - t0)
            k = (torch.randn((HKV, n, D), device=dev, generator=g) * jit).half()
            v = (torch.randn((HKV, n, D), device=dev, generator=g) * jit).half()
            c.update(k, v)
        caches.append(c)
        qs.append(torch.randn((1, HQ, 1, D), device=dev, generator=g).half())
        kns.append((torch.randn((1, HKV, 1, D), device=dev, generator=g) * jit).half())
        vns.append((torch.randn((1, HKV, 1, D), device=dev, generator=g) * jit).half())
    torch.cuda.synchronize()
    T = T_prefix + 1
    bytes_attn = T * HKV * kv_bytes_per_token_head(bits) + 2 * HQ * D * 2
    bytes_layer = bytes_attn + 2 * HKV * D * 2 + HKV * kv_bytes_per_token_head(bits) // 2

    # The raw ABI call with prebuilt arguments (no per-call Python checks).
    L = qw_amd.lib()
    stream = torch.cuda.current_stream(dev).cuda_stream
    for layer in range(LAYERS):
        outs.append(torch.empty((HQ, 1, D), dtype=torch.float16, device=dev))

    def layer_call(i):
        c = caches[i]
        rc = L.qw_kv_update_and_attention(c._h, qs[i].data_ptr(), HQ, 1, kns[i].data_ptr(),
                                          vns[i].data_ptr(), 1.0 / 16, 0, outs[i].data_ptr(),
                                          stream)
        if rc:
            raise qw_amd.QwError(rc, L.qw_last_error().decode())
        c.trim(1)  # host-side: the next step again attends 32769 keys

    def attn_call(i):
        c = caches[i]
        rc = L.qw_kv_attention(c._h, qs[i].data_ptr(), HQ, 1, 1.0 / 16, 0, outs[i].data_ptr(),
                               stream)
        if rc:
            raise qw_amd.QwError(rc, L.qw_last_error().decode())

    def round_layers():
        for i in range(LAYERS):
            layer_call(i)

    def round_attn():
        for i in range(LAYERS):
            attn_call(i)

    # caches hold T_prefix rows; attn_call needs the appended token present
    for i in range(LAYERS):
        caches[i].update(kns[i], vns[i])
    # warmup (also allocates the split-K workspaces before graph capture)
    for _ in range(max(1, warmup // LAYERS)):
        round_attn()
    for i in range(LAYERS):
        caches[i].trim(1)
    for _ in range(max(1, warmup // LAYERS)):
        round_layers()
    torch.cuda.synchronize()
    timer = Timer(torch)
    rounds = max(1, steps // LAYERS)
    eager_ms = timer.run(round_layers, rounds) / (rounds * LAYERS)

    # One graph per round: 16 layer calls (append + attention each).
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(LAYERS):
            c = caches[i]
            st = torch.cuda.current_stream(dev).cuda_stream
            rc = L.qw_kv_update_and_attention(c._h, qs[i].data_ptr(), HQ, 1, kns[i].data_ptr(),
                                              vns[i].data_ptr(), 1.0 / 16, 0,
                                              outs[i].data_ptr(), st)
            assert rc == 0, L.qw_last_error()
            c.trim(1)
    for _ in range(3):
        graph.replay()
    layer_ms = timer.run(graph.replay, rounds) / (rounds * LAYERS)

    # The attention alone (dominant kernel + its split-K merge), also as a graph.
    for i in range(LAYERS):
        caches[i].update(kns[i], vns[i])
    agraph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(agraph):
        for i in range(LAYERS):
            c = caches[i]
            st = torch.cuda.current_stream(dev).cuda_stream
            rc = L.qw_kv_attention(c._h, qs[i].data_ptr(), HQ, 1, 1.0 / 16, 0,
                                   outs[i].data_ptr(), st)
            assert rc == 0, L.qw_last_error()
    for _ in range(3):
        agraph.replay()
    attn_ms = timer.run(agraph.replay, rounds) / (rounds * LAYERS)
    for i in range(LAYERS):
        caches[i].trim(1)
    torch.cuda.synchronize()
    del graph, agraph
    for c in caches:
        c.close()
    torch.cuda.empty_cache()
    return {
        "T": T, "bits": bits, "rounds": rounds, "layer_ms": layer_ms, "eager_layer_ms": eager_ms,
        "attn_ms": attn_ms, "bytes_layer": bytes_layer, "bytes_attn": bytes_attn,
    }


def bench_dlsa(torch, qw_amd, steps: int, T: int = 131072, layers: int = LAYERS):
    """Config 5: one decode row, 4612-entry list (4 sinks + 512 window + 8 whole
    512-key blocks), fp16 KV [4, 131072, 256] per layer, 16 layers rotated."""
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
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        st = torch.cuda.current_stream(dev).cuda_stream
        for i in range(layers):
            call(i, st)
    for _ in range(3):
        graph.replay()
    rounds = max(1, steps // layers)
    ms = Timer(torch).run(graph.replay, rounds) / (rounds * layers)
    bytes_call = W * HKV * 2 * D * 2 + HQ * D * 2 * 2 + W * 4
    del graph
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


def main() -> int:
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only: the path is sharded by KV "
                          "head across GPUs in design (DESIGN.md), not implemented; run with "
                          "--gpus 1"}))
        return 2
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
        "dtype": "fp16",
        "data": "synthetic: N(0,1) fp16 K/V x per-head U(0.5,2), N(0,1) q, seeded",
        "config": {"workload": "config 2: decode layer call, append 1 token (4-bit affine, "
                               "group 64) + fused dequant-SDPA over 32769 keys",
                   "q_heads": HQ, "kv_heads": HKV, "head_dim": D, "context": dec["T"],
                   "kv_bits": 4, "layers_rotated": LAYERS},
        "us_per_layer": round(us_layer, 3),
        "us_per_layer_eager": round(dec["eager_layer_ms"] * 1e3, 3),
        "us_attention": round(dec["attn_ms"] * 1e3, 3),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": None,
                     "kernel": "attend_decode_kernel + decode_merge_kernel (one qw_kv_attention "
                               "call)",
                     "algorithmic_bytes": dec["bytes_attn"]},
    }
    if not args.no_extra:
        log("bench: config 5 D-LSA read")
        ds = bench_dlsa(torch, qw_amd, steps)
        gbs = ds["bytes"] / (ds["ms"] * 1e-3) / 1e9
        line["extra"] = {
            "config5_dlsa_decode": {"us_per_layer": round(ds["ms"] * 1e3, 3),
                                    "GB_s": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4),
                                    "list_width": ds["W"], "context": ds["T"],
                                    "algorithmic_bytes": ds["bytes"]},
        }
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
