"""GPU parity of the typed D-LSA read (qw_dlsa_sparse_attention_typed): the
reference's whole K2 contract, q f16 / bf16 / f32 with K and V alike in one of
the three, head_dim 32..256, at most 8 query heads a KV head
(mlx_cxx_dlsa_attention.cpp:429-470).

* f32 mirrors the reference's own test (dlsa_attention.rs:213-255): the same
  geometries (hq/hkv/d 6/2/32, 24/4/256, 8/8/64, 16/2/128, 6/1/32), context
  and row counts, its list construction (row r at t - rows + r reads a
  scattered unsorted subset of its causal keys, itself included, -1 padded),
  its value generator and its launch knobs (automatic, 1 part x 1 and 16
  waves, 7 parts x 4, 64 parts x 2), held to max-abs < 1e-5 of the fp64
  softmax (oracle.dlsa_attention_f64).
* bf16 and mixed dtypes, against the fp64 softmax of the same (widened)
  inputs: an f32 output within 1e-5, an f16 output within the stated bar
  (2e-3 max-abs, 1e-3 rel-L2), a bf16 output within half a bf16 ulp (its own
  rounding is ~1e-3 rel-L2 by itself: the output rounding to q's dtype is the
  only rounding below fp32).
* f16 with f16 K/V at head_dim >= 64 is the served fp16 read, bit for bit.
"""
import numpy as np
import pytest

from conftest import rng
from test_gpu_kv import _gpu, _np, assert_close

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

MASK64 = (1 << 64) - 1


def ref_values(n, seed):
    """The reference test's values(): xorshift64 into about [-1.5, 1.5]
    (dlsa_attention.rs:80-91)."""
    s = ((seed * 0x9E3779B97F4A7C15) & MASK64) | 1
    hi = []
    for _ in range(n):
        s ^= (s << 13) & MASK64
        s ^= s >> 7
        s ^= (s << 17) & MASK64
        hi.append(s >> 40)
    # (hi / 2^24 - 0.5) is exact in fp32; the product by 3 rounds once either
    # way, so fp64 arithmetic then one cast equals the reference's fp32 steps
    return ((np.array(hi, np.float64) / (1 << 24) - 0.5) * 3.0).astype(np.float32)


def ref_case(t, rows, seed):
    """The reference test's case(): lists [rows, width] i32 and lengths
    (dlsa_attention.rs:104-138)."""
    raw = []
    for r in range(rows):
        p = t - rows + r
        lst = [k for k in range(p) if (k * 7 + p + seed) % 3 == 0] + [p]
        mid = len(lst) // 2
        lst[:mid] = lst[:mid][::-1]
        rot = mid // 3
        lst = lst[rot:] + lst[:rot]
        raw.append(lst)
    width = max(len(x) for x in raw) + 5
    lists = np.full((rows, width), -1, np.int32)
    lengths = np.array([len(x) for x in raw], np.int32)
    for r, x in enumerate(raw):
        lists[r, :len(x)] = x
    return lists, lengths


def _typed(q, k, v, lists, lengths, scale, parts=0, waves=0):
    import qw_amd

    return qw_amd.sparse_attention_typed(q, k, v, _gpu(lists), _gpu(lengths), scale, parts,
                                         waves)[0]


GEOMS = [(6, 2, 32), (24, 4, 256), (8, 8, 64), (16, 2, 128), (6, 1, 32)]
LAUNCHES = [(0, 0), (1, 1), (1, 16), (7, 4), (64, 2)]


@pytest.mark.parametrize("hq,hkv,d", GEOMS)
def test_f32_matches_fp64_softmax_across_launches(oracle_lib, hq, hkv, d):
    failures = []
    for t, rows in [(40, 1), (97, 3), (200, 8), (300, 37)]:
        lists, lengths = ref_case(t, rows, t + rows)
        q = ref_values(hq * rows * d, 1).reshape(hq, rows, d)
        k = ref_values(hkv * t * d, 2).reshape(hkv, t, d)
        v = ref_values(hkv * t * d, 3).reshape(hkv, t, d)
        scale = 1.0 / np.sqrt(np.float32(d))
        want = oracle_lib.dlsa_attention_f64(q, k, v, lists, lengths, float(np.float32(scale)))
        qg, kg, vg = _gpu(q), _gpu(k), _gpu(v)
        for parts, waves in LAUNCHES:
            got = _np(_typed(qg, kg, vg, lists, lengths, float(scale), parts, waves))
            assert got.dtype == np.float32
            err = np.where(np.isfinite(got), np.abs(got - want), np.inf).max()
            if not err < 1e-5:
                failures.append(f"{hq}/{hkv}/{d} t={t} rows={rows} parts={parts} waves={waves}: {err:e}")
    assert not failures, "\n".join(failures)


def _bf16(x):
    """Round fp32 to bf16 (nearest even) and back, as numpy fp32."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    u = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    return u.astype(np.uint32).view(np.float32)


def _within_half_bf16_ulp(got, want):
    ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(want), 1e-30))) - 7)
    err = np.abs(got - want) - 0.5 * ulp
    print(f"  bf16 output: worst excess over half an ulp {err.max():.3e}", flush=True)
    return bool(np.all(err <= 1e-6))


def _case(r, hq, hkv, d, t, rows, width):
    lists = np.full((rows, width), -1, np.int32)
    lengths = r.integers(1, width + 1, rows).astype(np.int32)
    lengths[0] = width
    for row in range(rows):
        lists[row, :lengths[row]] = r.choice(t, lengths[row], replace=False)
    return lists, lengths


@pytest.mark.parametrize("q_dt,kv_dt", [("bf16", "bf16"), ("f32", "bf16"), ("bf16", "f32"),
                                        ("f16", "f32"), ("f32", "f16"), ("f16", "bf16")])
@pytest.mark.parametrize("d", [32, 128, 256])
def test_mixed_dtypes_within_the_bar(oracle_lib, q_dt, kv_dt, d):
    tdt = {"f16": torch.float16, "bf16": torch.bfloat16, "f32": torch.float32}
    r = rng(900 + d + 7 * len(q_dt) + len(kv_dt))
    hq, hkv, t, rows, width = 24, 4, 3000, 5, 700
    q = r.standard_normal((hq, rows, d)).astype(np.float32)
    k = r.standard_normal((hkv, t, d)).astype(np.float32)
    v = r.standard_normal((hkv, t, d)).astype(np.float32)
    lists, lengths = _case(r, hq, hkv, d, t, rows, width)
    lists[1, 2] = t + 3   # past the end: skipped
    qg = torch.from_numpy(q).to("cuda:0").to(tdt[q_dt])
    kg = torch.from_numpy(k).to("cuda:0").to(tdt[kv_dt])
    vg = torch.from_numpy(v).to("cuda:0").to(tdt[kv_dt])
    # the checker sees exactly the inputs the device holds
    qw, kw, vw = (x.float().cpu().numpy() for x in (qg, kg, vg))
    scale = d ** -0.5
    want = oracle_lib.dlsa_attention_f64(qw, kw, vw, lists, lengths, scale)
    got = _typed(qg, kg, vg, lists, lengths, scale)
    assert got.dtype == tdt[q_dt]
    got = got.float().cpu().numpy()
    what = f"typed q={q_dt} kv={kv_dt} d={d}"
    if q_dt == "f32":
        assert np.abs(got - want).max() < 1e-5, what
    elif q_dt == "f16":
        assert_close(got, want, what)
    else:
        # a bf16 output carries bf16's own rounding (rel-L2 ~1e-3 by itself):
        # it is the fp32 result rounded once, within half a bf16 ulp of fp64
        assert _within_half_bf16_ulp(got, want), what


def test_bf16_output_is_the_rounded_fp32_result(oracle_lib):
    """bf16 everywhere: the result is the fp32 computation rounded once to
    bf16, so it is within half a bf16 ulp (plus fp32 noise) of the fp64
    softmax of the same inputs."""
    r = rng(951)
    hq, hkv, d, t, rows, width = 16, 2, 128, 900, 3, 400
    q = _bf16(r.standard_normal((hq, rows, d)))
    k = _bf16(r.standard_normal((hkv, t, d)))
    v = _bf16(r.standard_normal((hkv, t, d)))
    lists, lengths = _case(r, hq, hkv, d, t, rows, width)
    want = oracle_lib.dlsa_attention_f64(q, k, v, lists, lengths, d ** -0.5)
    g = lambda x: torch.from_numpy(x).to("cuda:0").to(torch.bfloat16)  # noqa: E731
    got = _typed(g(q), g(k), g(v), lists, lengths, d ** -0.5).float().cpu().numpy()
    assert _within_half_bf16_ulp(got, want)


def test_f16_head_dim_32(oracle_lib):
    """f16 at head_dim 32 (below the fp16 MFMA kernel's range) goes through the
    typed kernel, within the bar of the fp64 softmax."""
    r = rng(952)
    hq, hkv, d, t, rows, width = 6, 2, 32, 500, 4, 200
    q = r.standard_normal((hq, rows, d)).astype(np.float16)
    k = r.standard_normal((hkv, t, d)).astype(np.float16)
    v = r.standard_normal((hkv, t, d)).astype(np.float16)
    lists, lengths = _case(r, hq, hkv, d, t, rows, width)
    want = oracle_lib.dlsa_attention_f64(q, k, v, lists, lengths, d ** -0.5)
    got = _np(_typed(_gpu(q), _gpu(k), _gpu(v), lists, lengths, d ** -0.5))
    assert_close(got, want, "typed f16 d=32")


def test_f16_served_shapes_are_the_fp16_read():
    import qw_amd

    r = rng(953)
    hq, hkv, d, t, rows, width = 24, 4, 256, 2000, 3, 600
    q = _gpu(r.standard_normal((hq, rows, d)).astype(np.float16))
    k = _gpu(r.standard_normal((hkv, t, d)).astype(np.float16))
    v = _gpu(r.standard_normal((hkv, t, d)).astype(np.float16))
    lists, lengths = _case(r, hq, hkv, d, t, rows, width)
    a = _np(_typed(q, k, v, lists, lengths, d ** -0.5))
    b = _np(qw_amd.sparse_attention(q, k, v, _gpu(lists), _gpu(lengths), d ** -0.5)[0])
    np.testing.assert_array_equal(a, b)


def test_typed_contract_errors():
    import qw_amd

    q = torch.zeros((9, 1, 64), device="cuda:0")
    k = torch.zeros((1, 10, 64), device="cuda:0")
    lists = torch.zeros((1, 4), dtype=torch.int32, device="cuda:0")
    lengths = torch.ones((1,), dtype=torch.int32, device="cuda:0")
    with pytest.raises(qw_amd.QwError):  # G = 9 > 8
        qw_amd.sparse_attention_typed(q, k, k, lists, lengths, 0.1)
    q = torch.zeros((2, 1, 48), device="cuda:0")
    k = torch.zeros((1, 10, 48), device="cuda:0")
    with pytest.raises(qw_amd.QwError):  # head_dim 48
        qw_amd.sparse_attention_typed(q, k, k, lists, lengths, 0.1)
    q = torch.zeros((2, 1, 64), device="cuda:0")
    k = torch.zeros((1, 10, 64), device="cuda:0")
    with pytest.raises(qw_amd.QwError):  # K and V in different dtypes
        qw_amd.sparse_attention_typed(q, k, k.half(), lists, lengths, 0.1)
