"""GPU parity of the Turbo4 KV mode (MI355X, through the C ABI).

Reference: KVCache::update_turbo4_sym and the Turbo4 attention routes
(crates/mlxcel-core/src/cache.rs:1438-1597, :3495-3589, :3652-3697), the codec
in crates/mlxcel-core/src/cache/turbo/quant.rs and sparse_v.rs:1051-1072.

Bars (the oracle restates the codec in float64, the library computes in
fp32 as the reference's MLX graph does):
  - stored indices equal the oracle's except where the oracle's rotated
    coordinate lies within 2e-6 of a centroid boundary (fp32 rounding of the
    rotation decides those), and there by one step; norms and rescales within
    one fp16 ulp;
  - the fetched rows (update_and_fetch) within one fp16 ulp of the oracle's
    float64 inverse rotation of the same stored tensors, plus 1e-6 of the
    row's norm (fp32 rotation error near zero);
  - attention within 2e-3 max-abs and 1e-3 relative L2 of the oracle's
    attention_turbo4_dequant_sdpa over the same stored tensors;
  - snapshot, trim, growth, demote and the fused RoPE append bit-exact
    against their plain counterparts.
"""
import numpy as np
import pytest

import oracle
from conftest import rng

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

MAX_ABS = 2e-3
REL_L2 = 1e-3


def _gpu(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0")


def _np(t):
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


def _snap(cache):
    t = cache.snapshot_tensors()
    out = {k: _np(v) for k, v in t.items()}
    for k in ("k_rescale", "v_norms", "v_rescale"):
        out[k] = out[k][..., 0]
    return out


def _kv(r, H, T, D):
    s = r.uniform(0.5, 2.0, (H, 1, 1))
    return ((r.standard_normal((H, T, D)) * s).astype(np.float16),
            (r.standard_normal((H, T, D)) * s).astype(np.float16))


def _ulps(a, b):
    a = np.asarray(a, np.float16).view(np.int16).astype(np.int64)
    b = np.asarray(b, np.float16).view(np.int16).astype(np.int64)
    return np.abs(a - b)


def assert_close(out, ref, what=""):
    out = np.asarray(out, np.float64)
    ref = np.asarray(ref, np.float64)
    err = out - ref
    mx = np.abs(err).max()
    rel = np.linalg.norm(err) / max(np.linalg.norm(ref), 1e-30)
    mag = max(1.0, float(np.abs(ref).max()))
    print(f"{what}: max_abs={mx:.3e} rel_l2={rel:.3e}", flush=True)
    assert mx <= MAX_ABS * mag and rel <= REL_L2, (what, mx, rel, mag)


def _check_stored(snap, k, v, tab, what=""):
    """Indices, norms and rescales of the GPU's snapshot against the oracle
    quantize of the same fp16 rows."""
    bnd = tab["bnd"].astype(np.float64)
    for name, x, s1, s2 in (("k", k, tab["k_s1"], tab["k_s2"]),
                            ("v", v, tab["v_s1"], tab["v_s2"])):
        idx, norms, rescale, y = oracle.turbo4_quantize(x, s1, s2, tab)
        got = oracle.turbo4_unpack(snap[name + "_packed"])
        diff = got != idx
        near = np.abs(y[..., None] - bnd).min(-1) < 2e-6
        print(f"{what} {name}: {int(diff.sum())} of {diff.size} indices differ, "
              f"{int(near.sum())} coordinates near a boundary", flush=True)
        assert not (diff & ~near).any(), (what, name)
        assert (np.abs(got.astype(int) - idx.astype(int)) <= 1).all()
        rs = snap[name + "_rescale"]
        ok_rows = ~diff.any(-1)  # a flipped index changes |centroids| legitimately
        assert (_ulps(rs, rescale)[ok_rows] <= 1).all(), (what, name)
        if name == "v":
            assert (_ulps(snap["v_norms"], norms) <= 1).all(), what
        exact = (_ulps(rs, rescale) == 0).mean()
        assert exact > 0.99, (what, name, exact)


@pytest.mark.parametrize("D", [256, 128])
def test_turbo4_append_and_fetch_match_oracle(D):
    import qw_amd

    H = 4
    r = rng(300 + D)
    k, v = _kv(r, H, 346, D)
    k[1, 5] = 0.0  # an all-zero row: norm 0, divided by 1, rescale 0
    v[2, 9] = 0.0
    cache = qw_amd.KVCache("turbo4", H, D, capacity=64)  # grows twice
    off = 0
    for n in (37, 1, 8, 300):
        cache.update(_gpu(k[:, off:off + n]), _gpu(v[:, off:off + n]))
        off += n
    assert cache.offset == 346
    tab = oracle.turbo4_tables(D)
    snap = _snap(cache)
    _check_stored(snap, k, v, tab, f"D{D}")
    assert snap["k_rescale"][1, 5] == 0 and snap["v_norms"][2, 9] == 0
    # fetch: the inverse rotation of the stored tensors
    kf, vf = map(_np, cache.dequantize())
    kf, vf = kf[0], vf[0]
    rk = oracle.turbo4_fetch_k(snap["k_packed"], snap["k_rescale"], tab)
    rv = oracle.turbo4_fetch_v(snap["v_packed"], snap["v_norms"], tab)
    for name, got, ref, x in (("k", kf, rk, k), ("v", vf, rv, v)):
        rn = np.linalg.norm(x.astype(np.float64), axis=-1, keepdims=True)
        spacing = np.spacing(np.abs(ref).astype(np.float16)).astype(np.float64)
        tol = spacing + 1e-6 * rn
        err = np.abs(got.astype(np.float64) - ref.astype(np.float64))
        print(f"fetch {name}: worst err/tol {float((err / tol).max()):.3f}", flush=True)
        assert (err <= tol).all(), name
    # a 4-bit Lloyd-Max quantizer's error on Gaussian rows: relative L2 ~0.097
    xf = k.astype(np.float64)
    rel = np.linalg.norm(kf - xf, axis=-1) / np.maximum(np.linalg.norm(xf, axis=-1), 1e-9)
    rel[1, 5] = 0.0
    assert rel.mean() < 0.11, rel.mean()
    # stored_norms_match_input_l2 (quant.rs:1261-1285): 2 %
    np.testing.assert_allclose(snap["v_norms"].astype(np.float64),
                               np.linalg.norm(v.astype(np.float64), axis=-1), rtol=0.02)


def test_turbo4_reference_round_trip_case():
    """k_side_quantize_dequantize_round_trip_bounded_error (turbo/quant.rs:
    873-930) on its own input: head_dim 128, params seed 0xCAFEF00D, four
    tokens of (sum of six LCG(0xBEEFCACE) signs) / 6 scaled by 0.5, 1.5, 4,
    12; relative L2 error under 15 % per token, in the full and in the
    rotated basis."""
    import qw_amd

    D, seed = 128, 0xCAFEF00D
    bits = (oracle.lcg_signs(4 * D * 6, 0xBEEFCACE) > 0).reshape(4, D, 6)
    acc = np.where(bits, 1.0, -1.0).sum(-1) / 6.0
    k = (acc * np.array([0.5, 1.5, 4.0, 12.0])[:, None]).astype(np.float16)[None]
    cache = qw_amd.KVCache("turbo4", 1, D, turbo_seed=seed)
    cache.update(_gpu(k), _gpu(k))
    kf = _np(cache.dequantize()[0])[0].astype(np.float64)
    snap = _snap(cache)
    tab = oracle.turbo4_tables(D, seed)
    kx = k[0].astype(np.float64)
    rel = np.linalg.norm(kf - kx, axis=-1) / np.linalg.norm(kx, axis=-1)
    k_rot = oracle.turbo4_rotate(kx, tab["k_s1"], tab["k_s2"])
    k_rot_hat = oracle.turbo4_expand_rotated(snap["k_packed"], snap["k_rescale"],
                                             tab)[0].astype(np.float64)
    rel_rot = np.linalg.norm(k_rot_hat - k_rot, axis=-1) / np.linalg.norm(k_rot, axis=-1)
    print("full", rel, "rotated", rel_rot, flush=True)
    assert rel.max() < 0.15 and rel_rot.max() < 0.15
    # k_and_v_packed_outputs_differ_for_same_input (quant.rs:938-960)
    assert (snap["k_packed"] != snap["v_packed"]).any()


def _turbo4_layer(qw_amd, T_prefix, L, causal, seed, D=256, hq=24, hkv=4, rows=None):
    r = rng(seed)
    k, v = _kv(r, hkv, T_prefix + L, D)
    q = r.standard_normal((hq, L, D)).astype(np.float16)
    cache = qw_amd.KVCache("turbo4", hkv, D, capacity=T_prefix + L)
    if T_prefix:
        cache.update(_gpu(k[:, :T_prefix]), _gpu(v[:, :T_prefix]))
    fn = cache.update_and_causal_attention if causal else cache.update_and_attention
    out = _np(fn(_gpu(q), _gpu(k[:, T_prefix:]), _gpu(v[:, T_prefix:]), 1.0 / 16))[0]
    snap = _snap(cache)
    tab = oracle.turbo4_tables(D)
    sel = np.arange(L) if rows is None else np.asarray(rows)
    pos = oracle.causal_positions(L, T_prefix + L) if causal else None
    if fused_verify_route(T_prefix + L, L, causal, hq // hkv):
        ref = oracle.turbo4_fused_verify(np.ascontiguousarray(q[:, sel]), snap["k_packed"],
                                         snap["k_rescale"], snap["v_packed"], snap["v_rescale"],
                                         tab, 1.0 / 16, np.ascontiguousarray(pos[sel]))
    else:
        ref = oracle.turbo4_attention(np.ascontiguousarray(q[:, sel]), snap["k_packed"],
                                      snap["k_rescale"], snap["v_packed"], snap["v_rescale"], tab,
                                      1.0 / 16,
                                      None if pos is None else np.ascontiguousarray(pos[sel]))
    return out[:, sel], ref, cache, (q, k, v)


def assert_fused_exact(out, ref, what=""):
    """The fused verify route keeps the merged rotated output in fp32 and casts
    to fp16 once after the rotation back, as the reference does; the oracle
    computes the same closed form in float64 and casts once. So the outputs
    agree to the final fp16 rounding: every element within one fp16 ulp of the
    reference plus 1e-5 (the fp32 error of scores, exp2 and the rotation, which
    matters only for outputs near zero), and at least 99 % equal bit for bit
    (measured 99.7-99.9 %; an extra fp16 rounding before the rotation gave
    57 %, with errors up to hundreds of ulps on small outputs)."""
    o = out.astype(np.float64)
    r = ref.astype(np.float64)
    ulp = np.spacing(np.abs(ref).astype(np.float16)).astype(np.float64)
    err = np.abs(o - r)
    bad = err > ulp + 1e-5
    assert not bad.any(), f"{what}: {int(bad.sum())} elements beyond one ulp, worst {err.max():.3e}"
    exact = float((o == r).mean())
    assert exact >= 0.99, f"{what}: only {exact:.4f} of the outputs equal"


def fused_verify_route(T, L, causal, G):
    """The reference's gate for its fused Turbo4 verify pass (fused_attention.rs:
    69-110): causal, 1..5 rows, more than 2048 cached tokens, at most 32 query
    heads a KV head; everything else takes the dequantize-then-SDPA route."""
    return causal and 1 <= L <= 5 and T > 2048 and G <= 32


@pytest.mark.parametrize("T_prefix,L,causal,D", [
    (4095, 1, False, 256),    # decode: the decode kernel on the packed indices, rotated basis
    (12286, 1, False, 256),   # decode over 12287 keys (a partial last 32-key sub-chunk)
    (1500, 2, True, 256),     # 2 causal rows below the gate (G * L = 12): the decode kernel
    (2999, 2, True, 256),     # 2-row verify past 2048 tokens: the fused verify kernel
    (4090, 5, True, 256),     # 5-row verify (G * L = 30 rows): fused
    (2046, 3, True, 256),     # 2049 tokens: fused, one partial key stage per split
    (2040, 3, True, 256),     # 2043 tokens: below the gate, the dequantize route
    (5000, 1, True, 256),     # causal single row: fused
    (3333, 4, True, 128),     # head_dim 128: fused
    (65532, 4, True, 256),    # 65536 tokens, 64 key stages a split
    (1000, 16, True, 256),    # 16-row verify block
    (900, 128, True, 256),    # prefill chunk, 768 rows a KV head: block kernel on the packed cache
    (700, 200, True, 256),    # 1200 rows a KV head: the block kernel from LDS tile images
    (600, 520, True, 256),    # 3120 rows a KV head, likewise
    (400, 520, False, 128),   # the same at head_dim 128, non-causal
    (2000, 40, False, 128),   # non-causal 240 rows a KV head, head_dim 128: block kernel
    (777, 1, False, 128),     # head_dim 128 decode
    (0, 1, False, 256),       # first token
])
def test_turbo4_attention_matches_oracle(T_prefix, L, causal, D):
    import qw_amd

    rows = None if L <= 16 else np.unique([r for r in (0, 1, 63, 64, 100, L - 1) if r < L])
    out, ref, _, _ = _turbo4_layer(qw_amd, T_prefix, L, causal, seed=T_prefix + L + D,
                                   D=D, rows=rows)
    assert np.isfinite(out).all()
    assert_close(out, ref, f"turbo4 T{T_prefix}+{L} causal={causal} D{D}")
    if fused_verify_route(T_prefix + L, L, causal, 24 // 4):
        assert_fused_exact(out, ref, f"turbo4 fused T{T_prefix}+{L} D{D}")


@pytest.mark.parametrize("T_prefix,L,hq,hkv,D", [
    (3000, 4, 32, 4, 256),    # G * L = 32: both row tiles of the fused kernel full
    (2500, 5, 8, 8, 256),     # no GQA sharing (G = 1), 5 rows
    (4000, 3, 16, 2, 128),    # head_dim 128, two KV heads
    (3000, 5, 56, 8, 256),    # G * L = 35: fused (one 128-row query tile)
    (2600, 5, 64, 8, 256),    # G = 8 with 5 rows (40)
    (4000, 4, 64, 2, 128),    # G = 32 with 4 rows: exactly one query tile, head_dim 128
    (2500, 5, 128, 4, 256),   # G = 32 with 5 rows (160): two query tiles, every key split
    (3000, 3, 132, 4, 256),   # G = 33 > 32: the dequantize route
])
def test_turbo4_verify_geometries(T_prefix, L, hq, hkv, D):
    import qw_amd

    out, ref, _, _ = _turbo4_layer(qw_amd, T_prefix, L, True, seed=T_prefix + 7 * L + hq,
                                   D=D, hq=hq, hkv=hkv)
    assert np.isfinite(out).all()
    assert_close(out, ref, f"turbo4 verify T{T_prefix}+{L} hq{hq} hkv{hkv} D{D}")
    if fused_verify_route(T_prefix + L, L, True, hq // hkv):
        assert_fused_exact(out, ref, f"turbo4 fused verify T{T_prefix}+{L} hq{hq} hkv{hkv} D{D}")


def test_turbo4_attention_without_append_and_reuse():
    """attention() over the cache as it is equals update_and_attention's
    output (which attends the new key in the decode launch's append unit, so
    within the stated tolerance), and repeated calls (shared workspace reuse)
    repeat it exactly."""
    import qw_amd

    out, _, cache, (q, k, v) = _turbo4_layer(qw_amd, 2000, 1, False, seed=9)
    again = _np(cache.attention(_gpu(q), 1.0 / 16))[0]
    assert_close(again, out, "turbo4 attention() vs update_and_attention")
    # a second, smaller cache in between uses the same device workspace
    other = qw_amd.KVCache("turbo4", 4, 256)
    other.update(_gpu(k[:, :300]), _gpu(v[:, :300]))
    _np(other.attention(_gpu(q), 1.0 / 16))
    np.testing.assert_array_equal(_np(cache.attention(_gpu(q), 1.0 / 16))[0], again)


@pytest.mark.parametrize("T0,L,causal,D", [
    (3000, 4, True, 256),     # the fused verify pass, its rows appended in the block launch
    (2040, 3, True, 256),     # below the gate: the fp16 arithmetic in the block kernel, likewise
    (1000, 16, True, 128),    # 96 rows a KV head at head_dim 128
    (600, 5, False, 256),     # non-causal block
    (4095, 1, False, 256),    # the decode step: the decode launch's append unit
    (12286, 1, False, 256),
    (1500, 2, True, 256),     # 2 causal rows below the fused gate: decode route
    (777, 1, False, 128),     # head_dim 128 decode
])
def test_turbo4_append_in_launch_equals_separate_update(T0, L, causal, D):
    """Update-and-attention calls append their rows inside the attention
    launch (the block kernel's, or the decode kernel's append unit): the cache
    then holds exactly what one bulk update stores (every snapshot tensor
    equal bit for bit), and the output equals attending the updated cache,
    within the stated tolerance."""
    import qw_amd

    r = rng(8100 + T0 + L + D)
    k, v = _kv(r, 4, T0 + L, D)
    q = r.standard_normal((24, L, D)).astype(np.float16)
    a = qw_amd.KVCache("turbo4", 4, D)
    a.update(_gpu(k[:, :T0]), _gpu(v[:, :T0]))
    fn = a.update_and_causal_attention if causal else a.update_and_attention
    o1 = _np(fn(_gpu(q), _gpu(k[:, T0:]), _gpu(v[:, T0:]), 1.0 / 16))[0]
    b = qw_amd.KVCache("turbo4", 4, D)
    b.update(_gpu(k), _gpu(v))
    o2 = _np(b.attention(_gpu(q), 1.0 / 16, causal))[0]
    assert a.offset == b.offset == T0 + L
    sa, sb = a.snapshot_tensors(), b.snapshot_tensors()
    for name, t in sa.items():
        assert torch.equal(t, sb[name]), name
    assert np.isfinite(o1).all()
    assert_close(o1, o2, f"turbo4 D{D} T{T0}+{L} causal={causal}: append in launch vs cached")


def test_turbo4_snapshot_trim_and_seed():
    import qw_amd

    H, D = 4, 256
    r = rng(31)
    k, v = _kv(r, H, 500, D)
    a = qw_amd.KVCache("turbo4", H, D)
    a.update(_gpu(k[:, :480]), _gpu(v[:, :480]))
    snap = a.snapshot_tensors()
    b = qw_amd.KVCache("turbo4", H, D)
    b.restore_snapshot(snap)
    assert b.offset == 480
    for key, val in _snap(b).items():
        np.testing.assert_array_equal(val, _snap(a)[key], err_msg=key)
    q = _gpu(r.standard_normal((H * 6, 1, D)).astype(np.float16))
    np.testing.assert_array_equal(_np(a.attention(q, 0.0625)), _np(b.attention(q, 0.0625)))
    # trim then re-append == never appended
    c = qw_amd.KVCache("turbo4", H, D)
    c.update(_gpu(k[:, :450]), _gpu(v[:, :450]))
    c.update(_gpu(k[:, 100:130]), _gpu(v[:, 100:130]))  # rows to roll back
    assert c.trim(30) == 30
    c.update(_gpu(k[:, 450:480]), _gpu(v[:, 450:480]))
    for key, val in _snap(c).items():
        np.testing.assert_array_equal(val, _snap(a)[key], err_msg=key)
    # the seed picks the rotation: another seed stores other indices, the
    # oracle's tables for that seed reproduce them
    s = qw_amd.KVCache("turbo4", H, D, turbo_seed=12345)
    s.update(_gpu(k[:, :64]), _gpu(v[:, :64]))
    ss = _snap(s)
    assert (ss["k_packed"] != _snap(a)["k_packed"][:, :64]).mean() > 0.5
    _check_stored(ss, k[:, :64], v[:, :64], oracle.turbo4_tables(D, 12345), "seed 12345")
    # the Turbo4 snapshot calls refuse another mode's cache (QW_ERR_STATE)
    aff = qw_amd.KVCache("affine4", H, D)
    ptrs = [snap[n].data_ptr() for n in ("k_packed", "k_rescale", "v_packed", "v_norms",
                                         "v_rescale")]
    assert qw_amd.lib().qw_kv_import_turbo4(aff._h, 480, *ptrs, None) == 5
    assert qw_amd.lib().qw_kv_export_turbo4(aff._h, *ptrs, None) == 5


def test_turbo4_demote_and_rope_update():
    import qw_amd

    H, D, hq = 4, 256, 24
    r = rng(41)
    k, v = _kv(r, H, 2100, D)
    # demote_fp16_to_turbo4 (cache.rs:3591) stores what a Turbo4 update stores
    f = qw_amd.KVCache("fp16", H, D)
    f.update(_gpu(k), _gpu(v))
    assert f.demote_fp16_to_turbo4()
    assert f.mode == qw_amd.KVCacheMode.TURBO4 and f.offset == 2100
    t = qw_amd.KVCache("turbo4", H, D)
    t.update(_gpu(k), _gpu(v))
    for key, val in _snap(f).items():
        np.testing.assert_array_equal(val, _snap(t)[key], err_msg=key)
    assert not f.demote_fp16_to_turbo4()  # no longer fp16
    # the fused RoPE append stores what RoPE then update stores
    a = qw_amd.KVCache("turbo4", H, D)
    b = qw_amd.KVCache("turbo4", H, D)
    pos = 0
    for L in (33, 1, 5):
        qkv = _gpu(r.standard_normal((1, L, (hq + 2 * H) * D)).astype(np.float16))
        qa = a.rope_update(qkv, hq, 256, 1e7)
        qr, kr, vr = qw_amd.fused_rope_qk_append(qkv, hq, H, D, 256, 1e7, 1.0, False, pos, 0)
        b.update(kr, vr)
        pos += L
        np.testing.assert_array_equal(_np(qa), _np(qr))
    for key, val in _snap(a).items():
        np.testing.assert_array_equal(val, _snap(b)[key], err_msg=key)


def test_turbo4_workspace_growth_and_streams():
    """The shared per-device workspace grows with the context and is ordered
    across streams by its event: caches attended alternately on two streams
    (with a growth in between) give the same rows as on one stream."""
    import qw_amd

    H, D, hq = 4, 256, 24
    r = rng(51)
    sizes = (300, 2500, 700, 4000)  # the last is first attended on a side stream (growth)
    caches, qs, want = [], [], []
    for T in sizes:
        k, v = _kv(r, H, T, D)
        c = qw_amd.KVCache("turbo4", H, D)
        c.update(_gpu(k), _gpu(v))
        caches.append(c)
        qs.append(_gpu(r.standard_normal((hq, 1, D)).astype(np.float16)))
    torch.cuda.synchronize()
    for c, q in zip(caches[:3], qs[:3]):  # reference: one stream, in order
        want.append(_np(c.attention(q, 1.0 / 16)))
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    outs = []
    for rep in range(3):
        for i, (c, q) in enumerate(zip(caches, qs)):
            with torch.cuda.stream(s1 if (i + rep) % 2 == 0 else s2):
                outs.append((i, c.attention(q, 1.0 / 16)))
    torch.cuda.synchronize()
    want.append(_np(caches[3].attention(qs[3], 1.0 / 16)))
    for i, o in outs:
        np.testing.assert_array_equal(_np(o), want[i])


def _ref_synth(n, seed):
    """The reference test's synth_kv_tensor values (turbo_tests.rs:79-91): an
    LCG (state * 1664525 + 1013904223 mod 2^32, seed 0 -> 0xDEADBEEF), each
    value (state >> 1) / i32::MAX in fp32; vectorized by jump-ahead."""
    a, c, M = 1664525, 1013904223, 1 << 32
    s0 = 0xDEADBEEF if seed == 0 else seed
    B = 4096
    Ak = np.empty(B, np.uint64)
    Ck = np.empty(B, np.uint64)
    ak, ck = 1, 0
    for k in range(B):  # state_{i+k+1} = A[k] state_i + C[k]
        ak = (ak * a) % M
        ck = (ck * a + c) % M
        Ak[k], Ck[k] = ak, ck
    out = np.empty(n, np.uint64)
    s = s0
    for i in range(0, n, B):
        blk = (Ak * np.uint64(s) + Ck) % np.uint64(M)
        m = min(B, n - i)
        out[i:i + m] = blk[:m]
        s = int(blk[B - 1])
    return ((out >> np.uint64(1)).astype(np.float32) / np.float32(2147483647.0)).astype(np.float32)


def _fixed_projection_argmax(values, dim):
    """turbo_tests.rs:1146-1164: argmax over 11 fixed projections of each row."""
    rows = values.reshape(-1, dim).astype(np.float32)
    d = np.arange(dim)[:, None]
    cls = np.arange(11)[None, :]
    w = (((d * 31 + cls * 17 + 13) % 101).astype(np.float32) / 50.0 - 1.0).astype(np.float32)
    return np.argmax(rows @ w, axis=1)


@pytest.mark.parametrize("tq,tk,seed", [
    (2, 2053, 0xD3C0DE02), (3, 4105, 0xD3C0DE03), (4, 8207, 0xD3C0DE04), (5, 16399, 0xD3C0DE05),
    (4, 2063, 0x6A5A4B1E), (3, 65537, 0xCA55A1A5)])
def test_turbo4_fused_matches_dequant_route_reference_cases(tq, tk, seed):
    """The reference's own fused-versus-dequantize parity test
    (turbo_tests.rs:1166-1226, cases :1311-1324): seeded rotations, its value
    generator, q [6, tq, D] over K/V [2, tk, D], bottom-right causal; the fused
    verify pass and the dequantize-then-SDPA route (here: the general route
    with the causal mask given as an array, which expands the rotated rows) agree
    within RMS 5e-3, with the same fixed-projection argmax on every row. head_dim
    128 here (the reference test uses 64, below this build's Turbo4 head dims)."""
    import qw_amd

    HQ, HKV, D = 6, 2, 128
    q = _ref_synth(HQ * tq * D, (seed + 1) % (1 << 32)).reshape(HQ, tq, D).astype(np.float16)
    k = _ref_synth(HKV * tk * D, (seed + 2) % (1 << 32)).reshape(HKV, tk, D).astype(np.float16)
    v = _ref_synth(HKV * tk * D, (seed + 3) % (1 << 32)).reshape(HKV, tk, D).astype(np.float16)
    cache = qw_amd.KVCache("turbo4", HKV, D, turbo_seed=seed)
    cache.update(_gpu(k), _gpu(v))
    scale = 1.0 / np.sqrt(D)
    fused = _np(cache.attention(_gpu(q), scale, causal=True))[0].astype(np.float32)
    mask = np.arange(tk)[None, :] <= (tk - tq + np.arange(tq))[:, None]
    ref = _np(cache.attention_general(_gpu(q), scale, mask=_gpu(mask)))[0].astype(np.float32)
    rms = float(np.sqrt(np.mean((fused.astype(np.float64) - ref) ** 2)))
    print(f"fused vs dequant route tq={tq} tk={tk}: rms {rms:.3e}", flush=True)
    assert rms < 5e-3
    np.testing.assert_array_equal(_fixed_projection_argmax(fused, D),
                                  _fixed_projection_argmax(ref, D))
