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
