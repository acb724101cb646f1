"""GPU parity of the fused q/k RoPE + append (MI355X, through the C ABI).

Reference: fused_rope_qk_append (crates/mlxcel-core/src/lib.rs:1462, kernel
crates/mlx-cpp/turbo/fused_rope_append.cpp:80-180) and its parity suite
(crates/mlxcel-core/src/fused_rope_parity_tests.rs:195-384).

Bars:
  - v, the unrotated tail and position 0 are bit-exact copies;
  - q and k within one fp16 ulp of the oracle's float64 rotation from its
    fp32 angles, plus the fp32 error of the angle and of cosf / sinf
    (2.5e-7 (2 + |theta|) (|x1| + |x2|) per element), and within the
    reference's own bar against MLX's RoPE (normalized rms 2e-3, normalized
    max 1.2e-2, fused_rope_parity_tests.rs:99-104);
  - layout 1 is layout 0 transposed, bit for bit;
  - the cache RoPE-append stores exactly what the standalone op followed by
    an ordinary update stores, in every cache mode, and its q is the op's q.
"""
import numpy as np
import pytest

import oracle
from conftest import rng

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


def _gpu(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0")


def _np(t):
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


def _rope_tol(x, rope_dims, traditional, base, scale, positions):
    """Per-element tolerance on the rotated prefix of x [..., T, D]."""
    th = np.abs(oracle.rope_theta(rope_dims, positions, base, scale).astype(np.float64))
    i1, i2 = oracle.rope_pairs(rope_dims, traditional)
    x = np.abs(np.asarray(x, np.float64))
    mag = x[..., i1] + x[..., i2]
    t = 2.5e-7 * (2.0 + th) * mag
    tol = np.zeros(x.shape[:-1] + (rope_dims,))
    tol[..., i1] = t
    tol[..., i2] = t
    return tol


def _check_rotated(got, ref, x, rope_dims, traditional, base, scale, positions, what):
    got = np.asarray(got, np.float64)
    ulp = np.spacing(np.abs(ref[..., :rope_dims]).astype(np.float16)).astype(np.float64)
    tol = ulp + _rope_tol(x, rope_dims, traditional, base, scale, positions)
    err = np.abs(got[..., :rope_dims] - ref[..., :rope_dims])
    worst = float((err / tol).max()) if err.size else 0.0
    rms = np.sqrt(np.mean((got - ref) ** 2)) / max(np.sqrt(np.mean(ref ** 2)), 1e-20)
    nmax = np.abs(got - ref).max() / max(np.sqrt(np.mean(ref ** 2)), 1e-20)
    print(f"{what}: worst err/tol {worst:.3f}, normalized rms {rms:.2e}, max {nmax:.2e}",
          flush=True)
    assert worst <= 1.0, (what, worst)
    assert rms <= 2e-3 and nmax <= 1.2e-2, (what, rms, nmax)
    # the unrotated tail is copied
    np.testing.assert_array_equal(got[..., rope_dims:], ref[..., rope_dims:])


CASES = [
    # B, L, hq, hkv, D, R, traditional, positions_base, base, scale
    (1, 7, 24, 4, 256, 256, False, 0, 10000.0, 1.0),
    (1, 33, 8, 2, 128, 128, True, 1000, 10000.0, 1.0),
    (2, 5, 4, 1, 256, 64, False, 4090, 1000000.0, 1.0),
    (1, 1, 24, 4, 256, 256, False, 32768, 10000000.0, 1.0),
    (3, 17, 6, 3, 64, 32, True, 12, 10000.0, 0.5),
    (1, 9, 5, 1, 96, 96, False, 77, 500000.0, 1.0),
    (1, 2, 2, 2, 256, 128, False, 131071, 1000000.0, 0.125),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "B{}L{}hq{}hkv{}D{}R{}{}p{}".format(
    *c[:6], "t" if c[6] else "h", c[7]))
def test_fused_rope_qk_append_matches_oracle(case):
    import qw_amd

    B, L, hq, hkv, D, R, trad, p0, base, scale = case
    r = rng(100 + D + L)
    qkv = r.standard_normal((B, L, (hq + 2 * hkv) * D)).astype(np.float16)
    print(f"case {case}", flush=True)
    x = _gpu(qkv)
    q, k, v = qw_amd.fused_rope_qk_append(x, hq, hkv, D, R, base, scale, trad, p0, 0)
    q1, k1, v1 = qw_amd.fused_rope_qk_append(x, hq, hkv, D, R, base, scale, trad, p0, 1)
    q, k, v, q1, k1, v1 = map(_np, (q, k, v, q1, k1, v1))
    rq, rk, rv = oracle.fused_rope_qk_append(qkv, hq, hkv, D, R, base, scale, trad, p0, 0)
    xs = qkv.reshape(B, L, hq + 2 * hkv, D).transpose(0, 2, 1, 3)
    pos = p0 + np.arange(L)
    _check_rotated(q, rq, xs[:, :hq], R, trad, base, scale, pos, "q")
    _check_rotated(k, rk, xs[:, hq:hq + hkv], R, trad, base, scale, pos, "k")
    np.testing.assert_array_equal(v, rv.astype(np.float16))
    np.testing.assert_array_equal(q1, q)
    np.testing.assert_array_equal(k1, k.transpose(0, 2, 1, 3))
    np.testing.assert_array_equal(v1, v.transpose(0, 2, 1, 3))
    if p0 == 0:
        # position 0 turns by nothing: an exact copy
        np.testing.assert_array_equal(q[:, :, 0], xs[:, :hq, 0])
        np.testing.assert_array_equal(k[:, :, 0], xs[:, hq:hq + hkv, 0])


def test_fused_rope_positions_are_absolute():
    """fused_rope_parity_tests.rs:218: token t of a window at base p turns as
    a single token at p + t does."""
    import qw_amd

    hq, hkv, D, R = 8, 2, 256, 256
    qkv = rng(7).standard_normal((1, 6, (hq + 2 * hkv) * D)).astype(np.float16)
    q, k, _ = map(_np, qw_amd.fused_rope_qk_append(_gpu(qkv), hq, hkv, D, R, 1e6, 1.0, False,
                                                   300, 0))
    for t in range(6):
        qt, kt, _ = map(_np, qw_amd.fused_rope_qk_append(_gpu(qkv[:, t:t + 1]), hq, hkv, D, R,
                                                         1e6, 1.0, False, 300 + t, 0))
        np.testing.assert_array_equal(qt[:, :, 0], q[:, :, t])
        np.testing.assert_array_equal(kt[:, :, 0], k[:, :, t])


@pytest.mark.parametrize("mode", ["fp16", "affine4", "affine8", "int8"])
@pytest.mark.parametrize("D,R,trad", [(256, 256, False), (128, 64, True)])
def test_rope_update_stores_what_rope_then_update_stores(mode, D, R, trad):
    import qw_amd

    hq, hkv = 24, 4
    base = 1e6
    print(f"mode {mode} D {D} R {R} traditional {trad}", flush=True)
    a = qw_amd.KVCache(mode, hkv, D)
    b = qw_amd.KVCache(mode, hkv, D)
    r = rng(11 + D)
    pos = 0
    for L in (37, 1, 1, 8, 3):  # prefill, decode rows, a verify block, ragged tail
        qkv = r.standard_normal((1, L, (hq + 2 * hkv) * D)).astype(np.float16)
        x = _gpu(qkv)
        qa = a.rope_update(x, hq, R, base, 1.0, trad)
        qr, kr, vr = qw_amd.fused_rope_qk_append(x, hq, hkv, D, R, base, 1.0, trad, pos, 0)
        b.update(kr, vr)
        pos += L
        assert a.offset == b.offset == pos
        np.testing.assert_array_equal(_np(qa), _np(qr))
    ka, va = map(_np, a.dequantize())
    kb, vb = map(_np, b.dequantize())
    np.testing.assert_array_equal(ka, kb)
    np.testing.assert_array_equal(va, vb)
    # the attention over the two caches is then the same computation
    q = _gpu(r.standard_normal((1, hq, 1, D)).astype(np.float16))
    np.testing.assert_array_equal(_np(a.attention(q, 1.0 / 16)), _np(b.attention(q, 1.0 / 16)))


def test_rope_update_affine4_matches_oracle_quantize():
    """The cache's K after the RoPE-append is the oracle's MLX quantize of the
    fp16-rounded rotation (bit-exact codes, scales and biases through the
    dequantized fetch), V the quantize of the copied rows."""
    import qw_amd

    hq, hkv, D, R = 24, 4, 256, 256
    L, p0 = 40, 0
    qkv = rng(21).standard_normal((1, L, (hq + 2 * hkv) * D)).astype(np.float16)
    cache = qw_amd.KVCache("affine4", hkv, D)
    cache.rope_update(_gpu(qkv), hq, R, 10000.0, 1.0, False, p0)
    _, k_rot, _ = qw_amd.fused_rope_qk_append(_gpu(qkv), hq, hkv, D, R, 10000.0, 1.0, False,
                                             p0, 0)
    k_rot = _np(k_rot)[0]
    v_new = qkv.reshape(L, hq + 2 * hkv, D)[:, hq + hkv:].transpose(1, 0, 2)
    ref = oracle.AffineCacheOracle(hkv, D, L, 4)
    ref.update(k_rot, np.ascontiguousarray(v_new))
    rk, rv = ref.fetch()
    k, v = map(_np, cache.dequantize())
    np.testing.assert_array_equal(k[0], rk)
    np.testing.assert_array_equal(v[0], rv)


# qw_kv_rope_update_and_attention: the served decode step from the projection
# (forward_fused_rope_append, then update_and_turbo4_attention) in one decode
# launch for decode-route shapes, the two calls otherwise.
@pytest.mark.parametrize("mode", ["affine4", "affine8", "int8", "turbo4"])
@pytest.mark.parametrize("D,R,trad,L,T0", [
    (256, 64, False, 1, 3000),   # the served Qwen3-Next shape: a quarter of the dims rotated
    (256, 256, True, 2, 700),    # a 2-row causal block, every dim rotated, adjacent pairs
    (128, 64, False, 1, 2500),
    (128, 128, True, 2, 40),
    (256, 64, False, 4, 3000),   # verify blocks: the block launch (Turbo4: the fused pass)
    (128, 128, True, 5, 2600),
])
def test_rope_update_and_attention_equals_the_two_reference_calls(mode, D, R, trad, L, T0):
    """Bit for bit against fused_rope_qk_append followed by
    update_and_attention on its q, k, v: the output, the rotated q, and the
    cache's rows afterwards (the same rotation arithmetic, rope_cs / rope_rot,
    and the same decode-launch arithmetic)."""
    import qw_amd

    hq, hkv, base = 24, 4, 1e7
    causal = L > 1
    print(f"mode {mode} D {D} R {R} traditional {trad} L {L} T0 {T0}", flush=True)
    r = rng(31 + D + L)
    k0 = _gpu(r.standard_normal((hkv, T0, D)).astype(np.float16))
    v0 = _gpu(r.standard_normal((hkv, T0, D)).astype(np.float16))
    a = qw_amd.KVCache(mode, hkv, D)
    b = qw_amd.KVCache(mode, hkv, D)
    a.update(k0, v0)
    b.update(k0, v0)
    for step in range(3):  # three consecutive steps: positions and appends chain
        qkv = _gpu(r.standard_normal((1, L, (hq + 2 * hkv) * D)).astype(np.float16))
        pos = a.offset
        out_a, q_a = a.rope_update_and_attention(qkv, hq, R, base, 1.0 / 16, 1.0, trad, pos,
                                                 causal)
        q_r, k_r, v_r = qw_amd.fused_rope_qk_append(qkv, hq, hkv, D, R, base, 1.0, trad, pos, 0)
        fn = b.update_and_causal_attention if causal else b.update_and_attention
        out_b = fn(q_r, k_r, v_r, 1.0 / 16)
        assert a.offset == b.offset == pos + L
        np.testing.assert_array_equal(_np(q_a), _np(q_r), err_msg=f"q, step {step}")
        np.testing.assert_array_equal(_np(out_a), _np(out_b), err_msg=f"out, step {step}")
    ka, va = map(_np, a.dequantize())
    kb, vb = map(_np, b.dequantize())
    np.testing.assert_array_equal(ka, kb)
    np.testing.assert_array_equal(va, vb)
    a.close()
    b.close()


@pytest.mark.parametrize("mode,R,L,T0", [
    ("affine4", 64, 4, 100),    # a verify block over fewer than 256 cached rows
    ("affine8", 24, 1, 1500),   # rope_dims not a multiple of 16
    ("fp16", 64, 1, 1500),      # an fp16 cache
    ("turbo4", 64, 4, 1500),    # a Turbo4 block under 2048 keys: no fused pass
])
def test_rope_update_and_attention_other_shapes_are_the_two_calls(mode, R, L, T0):
    """Shapes outside the one-launch routes run rope_update and attention."""
    import qw_amd

    hq, hkv, D, base = 24, 4, 256, 1e6
    print(f"mode {mode} R {R} L {L}", flush=True)
    r = rng(41 + L)
    k0 = _gpu(r.standard_normal((hkv, T0, D)).astype(np.float16))
    v0 = _gpu(r.standard_normal((hkv, T0, D)).astype(np.float16))
    a = qw_amd.KVCache(mode, hkv, D)
    b = qw_amd.KVCache(mode, hkv, D)
    a.update(k0, v0)
    b.update(k0, v0)
    qkv = _gpu(r.standard_normal((1, L, (hq + 2 * hkv) * D)).astype(np.float16))
    out_a, q_a = a.rope_update_and_attention(qkv, hq, R, base, 1.0 / 16, 1.0, False, T0, True)
    q_b = b.rope_update(qkv, hq, R, base, 1.0, False, T0)
    out_b = b.attention(q_b, 1.0 / 16, causal=True)
    np.testing.assert_array_equal(_np(q_a), _np(q_b))
    np.testing.assert_array_equal(_np(out_a), _np(out_b))
    a.close()
    b.close()


def test_rope_update_and_attention_contract_errors():
    import qw_amd

    c = qw_amd.KVCache("affine4", 4, 256)
    c.update(_gpu(np.zeros((4, 10, 256), np.float16)), _gpu(np.zeros((4, 10, 256), np.float16)))
    qkv = _gpu(np.zeros((1, 1, 32 * 256), np.float16))
    with pytest.raises(qw_amd.QwError):
        c.rope_update_and_attention(qkv, 24, 3, 1e6, 1.0 / 16)      # odd rope_dims
    with pytest.raises(qw_amd.QwError):
        c.rope_update_and_attention(qkv, 24, 64, -1.0, 1.0 / 16)    # base <= 0
    assert c.offset == 10                                           # nothing appended
    c.close()
