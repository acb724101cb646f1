"""Seeded random shapes through the cache and D-LSA entry points against the
oracle: every cache mode (affine 4/8-bit, Int8, fp16, Turbo4), head_dim
128/256, 1..8 KV heads, 1..8 query heads a KV head, 1..100 appended rows over
0..9000 cached ones, causal or not (Turbo4: the route the reference's gate
picks, the fused pass held to its one-ulp bar), and D-LSA reads with ragged,
unsorted lists holding entries past the end. The seeds are fixed, so a
failure names its case and reproduces exactly."""
import numpy as np
import pytest

import oracle
from conftest import rng
from test_gpu_kv import assert_close
from test_gpu_turbo4 import _snap, assert_fused_exact, fused_verify_route

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


def _g(x):
    return torch.from_numpy(np.ascontiguousarray(x)).to("cuda:0")


def _kv(r, hkv, T, D):
    s = r.uniform(0.5, 2.0, (hkv, 1, 1))
    return ((r.standard_normal((hkv, T, D)) * s).astype(np.float16),
            (r.standard_normal((hkv, T, D)) * s).astype(np.float16))


@pytest.mark.parametrize("seed", range(6))
def test_cache_modes_random_shapes(oracle_lib, seed):
    import qw_amd

    r = rng(7000 + seed)
    for case in range(12):
        mode = str(r.choice(["affine4", "affine8", "int8", "fp16"]))
        D = int(r.choice([128, 256]))
        hkv = int(r.choice([1, 2, 4, 8]))
        G = int(r.choice([1, 2, 3, 6, 8]))
        L = int(r.choice([1, 1, 2, 3, 4, 5, 7, 16, 33, 100]))
        T0 = int(r.integers(0, 6000)) if L < 50 else int(r.integers(0, 1500))
        causal = bool(r.integers(0, 2)) if L > 1 else False
        what = f"seed {seed} case {case}: {mode} D={D} hkv={hkv} G={G} T0={T0} L={L} causal={causal}"
        print(what, flush=True)
        k, v = _kv(r, hkv, T0 + L, D)
        q = r.standard_normal((hkv * G, L, D)).astype(np.float16)
        c = qw_amd.KVCache(mode, hkv, D)
        if T0:
            c.update(_g(k[:, :T0]), _g(v[:, :T0]))
        fn = c.update_and_causal_attention if causal else c.update_and_attention
        out = fn(_g(q), _g(k[:, T0:]), _g(v[:, T0:]), 1.0 / 16)[0].cpu().numpy()
        kd, vd = (x[0].cpu().numpy() for x in c.dequantize())
        pos = oracle_lib.causal_positions(L, T0 + L) if causal else None
        ref = oracle_lib.sdpa_mlx_f16(q, kd, vd, 1.0 / 16, pos)
        assert np.isfinite(out).all(), what
        assert_close(out, ref, what)
        c.close()


@pytest.mark.parametrize("seed", range(4))
def test_turbo4_and_dlsa_random_shapes(oracle_lib, seed):
    import qw_amd

    r = rng(8000 + seed)
    for case in range(10):
        D = int(r.choice([128, 256]))
        hkv = int(r.choice([1, 2, 4]))
        G = int(r.choice([1, 3, 6, 8]))
        if case % 2 == 0:
            L = int(r.choice([1, 2, 3, 4, 5, 9, 40]))
            T0 = int(r.choice([int(r.integers(1, 2000)), int(r.integers(2048, 9000))]))
            causal = bool(r.integers(0, 2))
            what = f"seed {seed} case {case}: turbo4 D={D} hkv={hkv} G={G} T0={T0} L={L} causal={causal}"
            print(what, flush=True)
            k, v = _kv(r, hkv, T0 + L, D)
            q = r.standard_normal((hkv * G, L, D)).astype(np.float16)
            c = qw_amd.KVCache("turbo4", hkv, D)
            c.update(_g(k[:, :T0]), _g(v[:, :T0]))
            fn = c.update_and_causal_attention if causal else c.update_and_attention
            out = fn(_g(q), _g(k[:, T0:]), _g(v[:, T0:]), 1.0 / 16)[0].cpu().numpy()
            snap = _snap(c)
            tab = oracle.turbo4_tables(D)
            pos = oracle.causal_positions(L, T0 + L) if causal else None
            args = (q, snap["k_packed"], snap["k_rescale"], snap["v_packed"], snap["v_rescale"], tab,
                    1.0 / 16, pos)
            if fused_verify_route(T0 + L, L, causal, G):
                assert_fused_exact(out, oracle.turbo4_fused_verify(*args), what)
            else:
                assert_close(out, oracle.turbo4_attention(*args), what)
            c.close()
        else:
            G = min(G, 8)
            L = int(r.choice([1, 1, 2, 5, 37, 200]))
            T = int(r.integers(100, 20000))
            W = int(r.integers(1, min(T, 3000) + 1))
            what = f"seed {seed} case {case}: dlsa D={D} hkv={hkv} G={G} T={T} L={L} W={W}"
            print(what, flush=True)
            q = r.standard_normal((hkv * G, L, D)).astype(np.float16)
            k = r.standard_normal((hkv, T, D)).astype(np.float16)
            v = r.standard_normal((hkv, T, D)).astype(np.float16)
            lists = np.full((L, W), -1, np.int32)
            lengths = r.integers(0, W + 1, L).astype(np.int32)
            for row in range(L):  # unsorted, some entries past the end
                lists[row, :lengths[row]] = r.choice(T + 5, lengths[row], replace=False)
            out = qw_amd.sparse_attention(_g(q), _g(k), _g(v), _g(lists), _g(lengths),
                                          D ** -0.5)[0].cpu().numpy()
            ref = oracle_lib.dlsa_attention(q, k, v, lists, lengths, D ** -0.5)
            assert_close(out, ref, what)
