"""GPU parity of the KV cache path through the C ABI (MI355X).

Codes, scales and biases of quantize-on-append must be bit-exact against the
oracle's restatement of MLX `quantize`; the dequantized fetch bit-exact
against MLX's composite dequantize; attention outputs within 2e-3 max-abs and
1e-3 relative-L2 of the oracle's MLX CPU-stream SDPA over the dequantized
cache (the stated tolerance; max-abs at unit output magnitude, see
assert_close), and no farther from the fp64 closed form than that reference.
"""
import numpy as np
import pytest

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


def _kv(r, H, T, D, jitter=True):
    s = r.uniform(0.5, 2.0, (H, 1, 1)) if jitter else 1.0
    return ((r.standard_normal((H, T, D)) * s).astype(np.float16),
            (r.standard_normal((H, T, D)) * s).astype(np.float16))


def assert_close(out, ref, what=""):
    """The stated bar: max-abs 2e-3 and rel-L2 1e-3. The max-abs bar is an
    absolute figure for outputs of magnitude <= 1 (the configs' N(0,1) data
    give |out| ~ 0.1); where a short, peaked softmax yields larger outputs
    (|out| = M > 1), MLX's own fp16 rounding of P moves its result by about
    M * 2^-11 from the exact value, so the max-abs bar scales with M there."""
    out = np.asarray(out, np.float64)
    ref = np.asarray(ref, np.float64)
    err = out - ref
    mx = np.abs(err).max()
    rel = np.linalg.norm(err) / max(np.linalg.norm(ref), 1e-30)
    mag = max(1.0, float(np.abs(ref).max()))
    print(f"{what}: max_abs={mx:.3e} rel_l2={rel:.3e} |ref|max={mag:.2f}", flush=True)
    assert mx <= MAX_ABS * mag and rel <= REL_L2, (what, mx, rel, mag)


def assert_as_exact_as_reference(out, ref, f64, what=""):
    """Distance to the fp64 closed form is no worse than the reference's own
    (MLX's fp16 roundings), within one fp16 ulp at the output's magnitude."""
    e_out = np.abs(np.asarray(out, np.float64) - f64).max()
    e_ref = np.abs(np.asarray(ref, np.float64) - f64).max()
    ulp = 2.0 ** -10 * max(1.0, float(np.abs(f64).max()))
    print(f"  vs fp64 closed form: ours {e_out:.3e}, reference {e_ref:.3e}", flush=True)
    assert e_out <= e_ref + ulp, (what, e_out, e_ref)


def _mode(bits):
    return {4: "affine4", 8: "affine8", 16: "fp16"}[bits]


@pytest.mark.parametrize("bits,D", [(4, 256), (8, 256), (4, 128), (8, 128)])
def test_append_codes_bit_exact(oracle_lib, bits, D):
    import qw_amd

    r = rng(bits * 1000 + D)
    H = 4
    sizes = [1, 7, 13, 256, 300, 1, 1, 37]
    T = sum(sizes)
    k, v = _kv(r, H, T, D)
    cache = qw_amd.KVCache(_mode(bits), H, D, capacity=64)
    t = 0
    for n in sizes:
        cache.update(_gpu(k[:, t:t + n])[None], _gpu(v[:, t:t + n])[None])
        t += n
    assert cache.offset == T and cache.capacity >= T
    snap = {name: _np(x) for name, x in cache.snapshot_tensors().items()}
    for side, src in (("k", k), ("v", v)):
        codes, scales, biases = oracle_lib.affine_quantize(src, bits)
        assert np.array_equal(snap[f"{side}_codes"].view(np.uint32), codes), side
        assert np.array_equal(snap[f"{side}_scales"].view(np.uint16), scales.view(np.uint16))
        assert np.array_equal(snap[f"{side}_biases"].view(np.uint16), biases.view(np.uint16))
    # dequantized fetch == MLX composite dequantize, bit for bit
    kd, vd = cache.dequantize()
    for side, src, got in (("k", k, kd), ("v", v, vd)):
        codes, scales, biases = oracle_lib.affine_quantize(src, bits)
        want = oracle_lib.affine_dequantize(codes, scales, biases, bits)
        assert np.array_equal(_np(got)[0].view(np.uint16), want.view(np.uint16)), side


@pytest.mark.parametrize("D", [256, 128])
def test_fp16_mode_fetch_is_identity(D):
    import qw_amd

    r = rng(D)
    k, v = _kv(r, 4, 333, D)
    cache = qw_amd.KVCache("fp16", 4, D, capacity=100)
    cache.update(_gpu(k[:, :300])[None], _gpu(v[:, :300])[None])
    kf, vf = cache.update_and_fetch(_gpu(k[:, 300:])[None], _gpu(v[:, 300:])[None])
    assert np.array_equal(_np(kf)[0], k) and np.array_equal(_np(vf)[0], v)


@pytest.mark.parametrize("bits", [4, 8])
def test_trim_then_reappend_equals_never_appended(bits):
    import qw_amd

    r = rng(50 + bits)
    k, v = _kv(r, 4, 120, 256)
    kx, vx = _kv(r, 4, 11, 256)
    a = qw_amd.KVCache(_mode(bits), 4, 256)
    a.update(_gpu(k[:, :100])[None], _gpu(v[:, :100])[None])
    a.update(_gpu(kx)[None], _gpu(vx)[None])           # rejected draft block
    assert a.trim(11) == 11 and a.offset == 100
    assert a.trim(0) == 0
    a.update(_gpu(k[:, 100:])[None], _gpu(v[:, 100:])[None])
    b = qw_amd.KVCache(_mode(bits), 4, 256)
    b.update(_gpu(k)[None], _gpu(v)[None])
    sa, sb = a.snapshot_tensors(), b.snapshot_tensors()
    for name in sa:
        assert torch.equal(sa[name], sb[name]), name
    assert a.trim(10_000) == 120 and a.offset == 0


@pytest.mark.parametrize("bits", [4, 8, 16])
def test_snapshot_round_trip(bits):
    import qw_amd

    r = rng(70 + bits)
    k, v = _kv(r, 4, 203, 256)
    a = qw_amd.KVCache(_mode(bits), 4, 256)
    a.update(_gpu(k)[None], _gpu(v)[None])
    snap = a.snapshot_tensors()
    b = qw_amd.KVCache(_mode(bits), 4, 256, capacity=16)
    b.restore_snapshot(snap)
    assert b.offset == 203
    ka, va = a.dequantize()
    kb, vb = b.dequantize()
    assert torch.equal(ka, kb) and torch.equal(va, vb)
    # and the restored cache keeps working: the same append gives the same state
    kn, vn = _kv(r, 4, 5, 256)
    a.update(_gpu(kn)[None], _gpu(vn)[None])
    b.update(_gpu(kn)[None], _gpu(vn)[None])
    for name, t in a.snapshot_tensors().items():
        assert torch.equal(t, b.snapshot_tensors()[name]), name


def _layer_call(oracle_lib, qw_amd, bits, T_prefix, L, causal, seed, D=256, hq=24, hkv=4,
                rows=None):
    """Prefill a cache with T_prefix rows, then one update_and_attention of L rows,
    on the GPU and in the oracle; returns (gpu_out, oracle_out, f64_out)."""
    r = rng(seed)
    k, v = _kv(r, hkv, T_prefix + L, D)
    q = r.standard_normal((hq, L, D)).astype(np.float16)
    cache = qw_amd.KVCache(_mode(bits), hkv, D, capacity=T_prefix + L)
    if T_prefix:
        cache.update(_gpu(k[:, :T_prefix])[None], _gpu(v[:, :T_prefix])[None])
    fn = cache.update_and_causal_attention if causal else cache.update_and_attention
    out = _np(fn(_gpu(q)[None], _gpu(k[:, T_prefix:])[None], _gpu(v[:, T_prefix:])[None],
                 1.0 / 16))[0]
    sel = np.arange(L) if rows is None else np.asarray(rows)
    out = out[:, sel]
    pos = oracle_lib.causal_positions(L, T_prefix + L) if causal else None
    pos_sel = None if pos is None else np.ascontiguousarray(pos[sel])
    q_sel = np.ascontiguousarray(q[:, sel])
    if bits == 16:
        ref = oracle_lib.sdpa_mlx_f16(q_sel, k, v, 1.0 / 16, q_pos=pos_sel)
        f64 = oracle_lib.sdpa_f64(q_sel, k, v, 1.0 / 16, q_pos=pos_sel)
        return out, ref, f64
    orc = oracle_lib.AffineCacheOracle(hkv, D, T_prefix + L, bits)
    if T_prefix:
        orc.update(k[:, :T_prefix], v[:, :T_prefix])
    ref = orc.update_and_attention(q, k[:, T_prefix:], v[:, T_prefix:], 1.0 / 16, causal,
                                   rows=None if rows is None else sel)
    kd, vd = orc.fetch()
    f64 = oracle_lib.sdpa_f64(q_sel, kd, vd, 1.0 / 16, q_pos=pos_sel)
    return out, ref, f64


@pytest.mark.parametrize("bits,T_prefix,L,causal", [
    (8, 4095, 1, False),     # config 1 geometry: 4096 keys, 8-bit
    (4, 32768, 1, False),    # config 2: decode at 32k + 1 appended, 4-bit
    (4, 1000, 2, True),      # 2-row verify block, bottom-right causal
    (8, 77, 1, False),       # ragged tail (77 + 1 keys)
    (4, 0, 1, False),        # first token: a single key
    (16, 5000, 1, False),    # fp16 cache
])
def test_update_and_attention_vs_oracle(oracle_lib, bits, T_prefix, L, causal):
    import qw_amd

    out, ref, f64 = _layer_call(oracle_lib, qw_amd, bits, T_prefix, L, causal,
                                seed=bits * 7 + T_prefix + L)
    assert np.isfinite(out).all()
    assert_close(out, ref, f"bits={bits} T={T_prefix}+{L} vs oracle")
    assert_as_exact_as_reference(out, ref, f64, f"bits={bits} T={T_prefix}+{L}")


@pytest.mark.parametrize("bits,T", [(4, 32769), (8, 4096)])
def test_headline_call_vs_oracle(oracle_lib, bits, T):
    """The call the headline roofline times, qw_kv_attention over a cache that
    already holds every key (the decode kernel without its append unit, with
    non-temporal loads at config 2's 37.8 MB), against the oracle at config 2
    (and config 1) size."""
    import qw_amd

    r = rng(300 + bits)
    hq, hkv, D = 24, 4, 256
    k, v = _kv(r, hkv, T, D)
    q = r.standard_normal((hq, 1, D)).astype(np.float16)
    cache = qw_amd.KVCache(_mode(bits), hkv, D)
    cache.update(_gpu(k)[None], _gpu(v)[None])
    out = _np(cache.attention(_gpu(q)[None], 1.0 / 16))[0]
    orc = oracle_lib.AffineCacheOracle(hkv, D, T, bits)
    orc.update(k, v)
    kd, vd = orc.fetch()
    ref = oracle_lib.sdpa_mlx_f16(q, kd, vd, 1.0 / 16)
    f64 = oracle_lib.sdpa_f64(q, kd, vd, 1.0 / 16)
    assert np.isfinite(out).all()
    assert_close(out, ref, f"headline call bits={bits} T={T} vs oracle")
    assert_as_exact_as_reference(out, ref, f64, f"headline call bits={bits} T={T}")


# The served verify blocks (MTP / DFlash2: 3..5 draft rows, the reference's
# fused-pass sizes, turbo4_attention.cpp:360, fused_attention.rs:70-100) on the
# affine codec at the config geometry: 18..30 rows a KV head (the block
# kernel, key-split), and G = 8 with 32 rows a KV head.
@pytest.mark.parametrize("bits,T_prefix,L,hq", [
    (4, 32768, 4, 24),      # 4-row verify at 32k
    (4, 65536, 5, 24),      # 5-row verify at 64k
    (4, 2049, 3, 24),       # 3 rows just past the reference's 2048-token gate
    (8, 5000, 5, 24),       # 8-bit
    (4, 3000, 4, 32),       # G = 8: exactly 32 rows a KV head
])
def test_served_verify_blocks_vs_oracle(oracle_lib, bits, T_prefix, L, hq):
    import qw_amd

    out, ref, f64 = _layer_call(oracle_lib, qw_amd, bits, T_prefix, L, True,
                                seed=bits * 13 + T_prefix + L + hq, hq=hq)
    assert np.isfinite(out).all()
    what = f"verify bits={bits} T={T_prefix}+{L} hq={hq}"
    assert_close(out, ref, what)
    assert_as_exact_as_reference(out, ref, f64, what)


# Many query rows per KV head (G * L > 16): the LDS-shared block kernel.
@pytest.mark.parametrize("bits,T_prefix,L,causal,D,hq,hkv,rows", [
    (4, 65536, 16, True, 256, 24, 4, None),     # config 4: 16-row verify at 64k, 4-bit
    (8, 16384, 2048, True, 256, 24, 4,           # config 3: 2048-row prefill chunk, 8-bit
     [0, 1, 2, 63, 64, 127, 500, 1023, 1024, 1500, 2000, 2046, 2047]),
    (4, 1000, 37, True, 256, 24, 4, None),      # ragged: 222 rows, 1000 + 37 keys
    (8, 300, 64, False, 256, 24, 4, None),      # no mask
    (16, 2000, 20, True, 256, 24, 4, None),     # fp16 cache
    (4, 0, 100, True, 256, 24, 4, None),        # prefill into an empty cache
    (4, 777, 5, True, 128, 32, 8, None),        # head_dim 128, G = 4
    (8, 4000, 17, True, 128, 8, 8, None),       # no GQA sharing (G = 1), 17 rows
    (4, 3000, 24, True, 128, 32, 8, None),      # 96 rows a KV head at head_dim 128: six row tiles, key-split
    (8, 2000, 13, True, 256, 24, 4, None),      # 78 rows a KV head: five row tiles, key-split
    # 3072+ rows a KV head: key tiles dequantized once into LDS images
    (4, 3000, 520, True, 256, 24, 4, [0, 1, 63, 64, 300, 519]),   # 3120 rows a KV head
    (4, 500, 400, False, 128, 16, 2, [0, 5, 128, 399]),           # head_dim 128, no mask
    (8, 0, 520, True, 256, 24, 4, [0, 1, 200, 519]),              # into an empty cache
    (16, 2000, 520, True, 256, 24, 4, [0, 1, 300, 519]),          # fp16 cache (layout images)
    # causal image launch of whole rounds with paired half tiles: 12144 rows a
    # KV head make 127 half tiles of 96 rows, so unit 63 holds half tile 63
    # alone and unit 0 pairs half tile 0 with the partial half tile 126
    (8, 1000, 2024, True, 256, 24, 4, [0, 15, 16, 1007, 1008, 1023, 1024, 2015, 2016, 2023]),
    # the same at head_dim 128, 8 KV heads: 6000 rows a KV head, 32 units a
    # head, 63 half tiles (the last one partial)
    (4, 200, 1500, True, 128, 32, 8, [0, 23, 24, 743, 744, 767, 768, 1487, 1488, 1499]),
])
def test_block_attention_vs_oracle(oracle_lib, bits, T_prefix, L, causal, D, hq, hkv, rows):
    import qw_amd

    out, ref, f64 = _layer_call(oracle_lib, qw_amd, bits, T_prefix, L, causal,
                                seed=bits * 11 + T_prefix + L + D, D=D, hq=hq, hkv=hkv, rows=rows)
    assert np.isfinite(out).all()
    what = f"block bits={bits} D={D} T={T_prefix}+{L} causal={causal}"
    assert_close(out, ref, what)
    assert_as_exact_as_reference(out, ref, f64, what)


# Every row of the paired-half-tile image launches, at full size: config 3
# (2048 rows, 8-bit, 16384 cached keys), the 2024-row chunk (an odd half-tile
# count, a lone middle half tile, a partial last one) and the 1500-row chunk
# at head_dim 128 with 8 KV heads. A half tile is 96 rows a KV head, i.e.
# 96 / G query rows; the launch pairs half tile j with half tile n - 1 - j.
#  - The first and last query row of every half tile (both members of every
#    pair) are checked against the oracle.
#  - All rows x heads are checked against the decode route row by row: the
#    cache is trimmed back to each row's last visible key and attended with
#    that row alone (bottom-right causal = all cached keys). The decode route
#    is a separate kernel whose config-2-size oracle test is green.
@pytest.mark.parametrize("bits,T_prefix,L,D,hq,hkv", [
    (8, 16384, 2048, 256, 24, 4),   # config 3
    (8, 1000, 2024, 256, 24, 4),    # 127 half tiles
    (4, 200, 1500, 128, 32, 8),     # head_dim 128, 63 half tiles
])
def test_paired_half_tiles_every_row(oracle_lib, bits, T_prefix, L, D, hq, hkv):
    import qw_amd

    G = hq // hkv
    per_half = 96 // G
    n_half = -(-L // per_half)
    sel = np.array(sorted({x for j in range(n_half)
                           for x in (j * per_half, min(L, (j + 1) * per_half) - 1)}))
    r = rng(7000 + bits + T_prefix + L + D)
    k, v = _kv(r, hkv, T_prefix + L, D)
    q = r.standard_normal((hq, L, D)).astype(np.float16)
    cache = qw_amd.KVCache(_mode(bits), hkv, D, capacity=T_prefix + L)
    cache.update(_gpu(k[:, :T_prefix])[None], _gpu(v[:, :T_prefix])[None])
    qg = _gpu(q)[None]
    out = _np(cache.update_and_causal_attention(qg, _gpu(k[:, T_prefix:])[None],
                                                _gpu(v[:, T_prefix:])[None], 1.0 / 16))[0]
    assert np.isfinite(out).all()
    what = f"paired half tiles bits={bits} D={D} T={T_prefix}+{L}"

    orc = oracle_lib.AffineCacheOracle(hkv, D, T_prefix + L, bits)
    orc.update(k[:, :T_prefix], v[:, :T_prefix])
    ref = orc.update_and_attention(q, k[:, T_prefix:], v[:, T_prefix:], 1.0 / 16, True, rows=sel)
    kd, vd = orc.fetch()
    pos = np.ascontiguousarray(oracle_lib.causal_positions(L, T_prefix + L)[sel])
    f64 = oracle_lib.sdpa_f64(np.ascontiguousarray(q[:, sel]), kd, vd, 1.0 / 16, q_pos=pos)
    assert_close(out[:, sel], ref, f"{what}: {len(sel)} half-tile edge rows vs oracle")
    assert_as_exact_as_reference(out[:, sel], ref, f64, what)

    rows = []
    for i in reversed(range(L)):
        rows.append(cache.attention(qg[:, :, i:i + 1], 1.0 / 16)[0])
        cache.trim(1)
    dec = _np(torch.cat(rows[::-1], dim=1))
    assert dec.shape == out.shape
    assert_close(out, dec, f"{what}: all {L} rows x {hq} heads vs the decode route")


def test_block_causal_rows_are_prefix_independent(oracle_lib):
    """Bottom-right causal: query row r of an L-row block sees exactly the keys
    a single-row call at the same position sees, so appending the block in one
    call equals appending it row by row (decode path) on the same cache."""
    import qw_amd

    r = rng(4242)
    hkv, hq, D, T0, L = 4, 24, 256, 3000, 8
    _rows_equal_decode(qw_amd, r, hkv, hq, D, T0, L)


def test_verify_rows_equal_row_by_row_decode():
    """The same for a served 5-row verify block (30 rows a KV head)."""
    import qw_amd

    _rows_equal_decode(qw_amd, rng(4343), 4, 24, 256, 5000, 5)


def _rows_equal_decode(qw_amd, r, hkv, hq, D, T0, L):
    k, v = _kv(r, hkv, T0 + L, D)
    q = r.standard_normal((hq, L, D)).astype(np.float16)
    a = qw_amd.KVCache("affine4", hkv, D)
    a.update(_gpu(k[:, :T0])[None], _gpu(v[:, :T0])[None])
    blk = _np(a.update_and_causal_attention(_gpu(q)[None], _gpu(k[:, T0:])[None],
                                            _gpu(v[:, T0:])[None], 1.0 / 16))[0]
    b = qw_amd.KVCache("affine4", hkv, D)
    b.update(_gpu(k[:, :T0])[None], _gpu(v[:, :T0])[None])
    for i in range(L):
        row = _np(b.update_and_attention(_gpu(q[:, i:i + 1])[None], _gpu(k[:, T0 + i:T0 + i + 1])[None],
                                         _gpu(v[:, T0 + i:T0 + i + 1])[None], 1.0 / 16))[0]
        assert_close(blk[:, i:i + 1], row, f"row {i}: block vs decode")


@pytest.mark.parametrize("bits", [4, 8])
def test_attention_without_append_equals_fused_call(oracle_lib, bits):
    """append-then-attend (the decode path folds the new token in during the
    split-K merge) equals attending a cache that already holds it: the same
    stored codes bit for bit, outputs within the stated tolerance."""
    import qw_amd

    r = rng(91 + bits)
    k, v = _kv(r, 4, 3000, 256)
    q = r.standard_normal((24, 1, 256)).astype(np.float16)
    a = qw_amd.KVCache(_mode(bits), 4, 256)
    a.update(_gpu(k)[None], _gpu(v)[None])
    o1 = _np(a.attention(_gpu(q)[None], 1.0 / 16))[0]
    b = qw_amd.KVCache(_mode(bits), 4, 256)
    b.update(_gpu(k[:, :2999])[None], _gpu(v[:, :2999])[None])
    o2 = _np(b.update_and_attention(_gpu(q)[None], _gpu(k[:, 2999:])[None],
                                    _gpu(v[:, 2999:])[None], 1.0 / 16))[0]
    for name, t in a.snapshot_tensors().items():
        assert torch.equal(t, b.snapshot_tensors()[name]), name
    assert_close(o2, o1, f"bits={bits} fused append vs cached")


@pytest.mark.parametrize("mode,D,T0,L,hq,causal,cap", [
    ("affine4", 256, 3000, 4, 24, True, 0),     # served 4-row verify
    ("affine8", 256, 2045, 5, 24, True, 0),     # new rows across an 8-key block and a 64-key tile
    ("int8", 256, 4093, 3, 24, True, 0),        # Int8 per-token rows
    ("affine4", 128, 1000, 16, 32, True, 0),    # head_dim 128, 128 rows a KV head
    ("affine4", 256, 700, 6, 24, False, 0),     # non-causal block: every row sees every new key
    ("affine8", 256, 512, 4, 24, True, 512),    # the call grows the capacity first
    # decode route (<= 16 rows a KV head): the decode launch's append unit
    ("affine4", 256, 3000, 2, 24, True, 0),     # 2-row verify (one draft), 12 rows a KV head
    ("affine8", 256, 2045, 2, 32, True, 0),     # 16 rows a KV head, across an 8-key block
    ("int8", 256, 1000, 2, 24, True, 0),
    ("affine4", 128, 500, 4, 16, True, 0),      # head_dim 128 (12-wave decode kernel)
    ("affine4", 256, 777, 3, 20, False, 0),     # non-causal, 15 rows a KV head
    ("affine8", 256, 256, 2, 24, True, 256),    # the call grows the capacity first
])
def test_verify_append_in_launch_equals_separate_append(oracle_lib, mode, D, T0, L, hq, causal, cap):
    """A verify block on an affine or Int8 cache appends its rows inside the
    attention launch (the block kernel's, or the decode kernel's append unit).
    The cache then holds exactly what one bulk update of the same rows stores
    (every snapshot tensor equal bit for bit), and the output equals attending
    the updated cache, within the stated tolerance."""
    import qw_amd

    r = rng(7000 + T0 + L + D)
    k, v = _kv(r, 4, T0 + L, D)
    q = r.standard_normal((hq, L, D)).astype(np.float16)
    a = qw_amd.KVCache(mode, 4, D, capacity=cap)
    a.update(_gpu(k[:, :T0])[None], _gpu(v[:, :T0])[None])
    fn = a.update_and_causal_attention if causal else a.update_and_attention
    o1 = _np(fn(_gpu(q)[None], _gpu(k[:, T0:])[None], _gpu(v[:, T0:])[None], 1.0 / 16))[0]
    b = qw_amd.KVCache(mode, 4, D)
    b.update(_gpu(k)[None], _gpu(v)[None])
    o2 = _np(b.attention(_gpu(q)[None], 1.0 / 16, causal))[0]
    assert a.offset == b.offset == T0 + L
    sa, sb = a.snapshot_tensors(), b.snapshot_tensors()
    for name, t in sa.items():
        assert torch.equal(t, sb[name]), name
    assert np.isfinite(o1).all()
    assert_close(o1, o2, f"{mode} D{D} T{T0}+{L} causal={causal}: append in launch vs cached")


@pytest.mark.parametrize("bits,D", [(4, 256), (8, 256), (4, 128), (8, 128)])
def test_decode_steps_store_the_same_codes_as_a_bulk_append(oracle_lib, bits, D):
    """Token-by-token decode (append fused into the attention call), across
    partly filled 8-key V blocks and a capacity growth, stores exactly the
    codes one bulk append of the same rows stores; each step's output matches
    the oracle."""
    import qw_amd

    r = rng(500 + bits + D)
    H, hq, T0, steps = 4, 16, 61, 23
    k, v = _kv(r, H, T0 + steps, D)
    q = r.standard_normal((hq, steps, D)).astype(np.float16)
    a = qw_amd.KVCache(_mode(bits), H, D, capacity=64)
    a.update(_gpu(k[:, :T0])[None], _gpu(v[:, :T0])[None])
    orc = oracle_lib.AffineCacheOracle(H, D, T0 + steps, bits)
    orc.update(k[:, :T0], v[:, :T0])
    for i in range(steps):
        t = T0 + i
        out = _np(a.update_and_attention(_gpu(q[:, i:i + 1])[None], _gpu(k[:, t:t + 1])[None],
                                         _gpu(v[:, t:t + 1])[None], 1.0 / 16))[0]
        ref = orc.update_and_attention(np.ascontiguousarray(q[:, i:i + 1]), k[:, t:t + 1],
                                       v[:, t:t + 1], 1.0 / 16, False)
        if i in (0, 1, steps - 1):
            assert_close(out, ref, f"step {i}")
    assert a.offset == T0 + steps
    b = qw_amd.KVCache(_mode(bits), H, D)
    b.update(_gpu(k)[None], _gpu(v)[None])
    for name, tt in b.snapshot_tensors().items():
        assert torch.equal(tt, a.snapshot_tensors()[name]), name


def test_invalid_calls_raise():
    import qw_amd

    c = qw_amd.KVCache("affine4", 4, 256)
    q = torch.zeros((1, 24, 1, 256), dtype=torch.float16, device="cuda:0")
    with pytest.raises(qw_amd.QwError):
        c.attention(q, 0.0625)               # empty cache: fewer keys than rows
    with pytest.raises(qw_amd.QwError):
        c.update(torch.zeros((1, 3, 1, 256), dtype=torch.float16, device="cuda:0"),
                 torch.zeros((1, 3, 1, 256), dtype=torch.float16, device="cuda:0"))
    q25 = torch.zeros((1, 25, 1, 256), dtype=torch.float16, device="cuda:0")
    k = torch.zeros((1, 4, 1, 256), dtype=torch.float16, device="cuda:0")
    with pytest.raises(qw_amd.QwError):
        c.update_and_attention(q25, k, k, 0.0625)  # 25 heads over 4 KV heads


@pytest.mark.parametrize("bits", [4, 8])
def test_extreme_scales_take_the_exact_slow_dequant(oracle_lib, bits):
    """Groups with |scale| < 2^-10 or >= 64 miss the 2-op dequant's exactness
    range; the kernel switches that sub-chunk to the separately rounded path,
    which must still match MLX's composite dequant."""
    import qw_amd

    r = rng(300 + bits)
    H, D, T = 4, 256, 700
    k, v = _kv(r, H, T + 1, D, jitter=False)
    k = k.astype(np.float32)
    v = v.astype(np.float32)
    k[:, 100:140, :64] *= 1e-3       # tiny scales
    k[:, 300:301, 64:128] *= 300.0   # |scale| >= 64 (4-bit) / 8-bit range
    v[:, 200:260, 128:192] *= 1e-3
    v[:, 500:510, :64] *= 100.0
    k, v = k.astype(np.float16), v.astype(np.float16)
    q = r.standard_normal((24, 1, D)).astype(np.float16)
    cache = qw_amd.KVCache(_mode(bits), H, D)
    cache.update(_gpu(k[:, :T])[None], _gpu(v[:, :T])[None])
    out = _np(cache.update_and_attention(_gpu(q)[None], _gpu(k[:, T:])[None],
                                         _gpu(v[:, T:])[None], 1.0 / 16))[0]
    orc = oracle_lib.AffineCacheOracle(H, D, T + 1, bits)
    orc.update(k[:, :T], v[:, :T])
    ref = orc.update_and_attention(q, k[:, T:], v[:, T:], 1.0 / 16, False).astype(np.float64)
    err = out.astype(np.float64) - ref
    rel = np.linalg.norm(err) / np.linalg.norm(ref)
    print(f"extreme bits={bits}: max_abs={np.abs(err).max():.3e} rel_l2={rel:.3e}")
    assert rel <= REL_L2 and np.abs(err).max() <= MAX_ABS * max(1.0, np.abs(ref).max())


@pytest.mark.gpu
@pytest.mark.parametrize("target,D,T", [("affine4", 256, 3001), ("affine8", 256, 777),
                                        ("affine4", 128, 65)])
def test_demote_equals_appending_the_rows_quantized(target, D, T):
    """cache.rs:3591 demote_fp16_to_turbo4, to an affine mode: the demoted
    cache holds exactly what appending the same rows in that mode stores
    (codes, scales, biases bit for bit), keeps its offset, and then behaves as
    that cache on further appends and attention."""
    import qw_amd

    r = rng(900 + T + D)
    H, hq = 4, 16
    k, v = _kv(r, H, T + 9, D)
    a = qw_amd.KVCache("fp16", H, D)
    a.update(_gpu(k[:, :T])[None], _gpu(v[:, :T])[None])
    assert a.demote_fp16_to_affine(target)
    assert a.mode == qw_amd.KVCacheMode.from_str(target) and a.offset == T
    b = qw_amd.KVCache(target, H, D)
    b.update(_gpu(k[:, :T])[None], _gpu(v[:, :T])[None])
    ta, tb = a.snapshot_tensors(), b.snapshot_tensors()
    assert set(ta) == set(tb)
    for name in tb:
        assert torch.equal(ta[name], tb[name]), name
    # both continue identically: append and attend in one call
    q = r.standard_normal((hq, 9, D)).astype(np.float16)
    oa = a.update_and_causal_attention(_gpu(q)[None], _gpu(k[:, T:])[None], _gpu(v[:, T:])[None],
                                       1.0 / 16)
    ob = b.update_and_causal_attention(_gpu(q)[None], _gpu(k[:, T:])[None], _gpu(v[:, T:])[None],
                                       1.0 / 16)
    assert torch.equal(oa, ob)
    assert a.offset == b.offset == T + 9


@pytest.mark.gpu
def test_demote_is_a_no_op_unless_a_populated_fp16_cache():
    import qw_amd

    empty = qw_amd.KVCache("fp16", 4, 256)
    assert not empty.demote_fp16_to_affine("affine4")
    assert empty.mode == qw_amd.KVCacheMode.FP16
    r = rng(77)
    k, v = _kv(r, 4, 40, 256)
    quant = qw_amd.KVCache("affine8", 4, 256)
    quant.update(_gpu(k)[None], _gpu(v)[None])
    before = quant.snapshot_tensors()
    assert not quant.demote_fp16_to_affine("affine4")
    for name, t in quant.snapshot_tensors().items():
        assert torch.equal(t, before[name]), name
    fp = qw_amd.KVCache("fp16", 4, 256)
    fp.update(_gpu(k)[None], _gpu(v)[None])
    with pytest.raises(qw_amd.QwError):
        fp.demote_fp16_to_affine("fp16")
    assert fp.mode == qw_amd.KVCacheMode.FP16 and fp.offset == 40


@pytest.mark.gpu
def test_policy_demotes_real_caches_past_the_threshold():
    """qwen3_5.rs:959 / :968 with real caches: a prefill past the threshold is
    quantized at its end; a short one is quantized before the forward that
    crosses the threshold, exactly once."""
    import qw_amd
    from qw_amd import policy

    r = rng(4096)
    thr = policy.QUANTIZE_THRESHOLD_TOKENS
    conf = qw_amd.KVCacheMode.AFFINE4
    mode0 = policy.initial_attention_cache_mode(conf)
    k, v = _kv(r, 4, thr + 1, 128)
    long_c = qw_amd.KVCache(mode0, 4, 128)
    long_c.update(_gpu(k)[None], _gpu(v)[None])
    assert policy.finish_initial_attention_prefill([long_c], conf) == 1
    assert long_c.mode == conf and long_c.offset == thr + 1
    short = qw_amd.KVCache(mode0, 4, 128)
    short.update(_gpu(k[:, :2])[None], _gpu(v[:, :2])[None])
    assert policy.finish_initial_attention_prefill([short], conf) == 0
    assert policy.prepare_attention_forward([short], conf, thr - 2, True) == 0
    assert short.mode == qw_amd.KVCacheMode.FP16
    assert policy.prepare_attention_forward([short], conf, thr - 1, True) == 1
    assert short.mode == conf
    assert policy.prepare_attention_forward([short], conf, thr - 1, True) == 0


# ------------------------------------------------------------- Int8 mode

def _int8_layer_call(oracle_lib, qw_amd, T_prefix, L, causal, seed, D=256, hq=24, hkv=4):
    r = rng(seed)
    k, v = _kv(r, hkv, T_prefix + L, D)
    q = r.standard_normal((hq, L, D)).astype(np.float16)
    cache = qw_amd.KVCache("int8", hkv, D, capacity=T_prefix + L)
    if T_prefix:
        cache.update(_gpu(k[:, :T_prefix])[None], _gpu(v[:, :T_prefix])[None])
    fn = cache.update_and_causal_attention if causal else cache.update_and_attention
    out = _np(fn(_gpu(q)[None], _gpu(k[:, T_prefix:])[None], _gpu(v[:, T_prefix:])[None],
                 1.0 / 16))[0]
    orc = oracle_lib.Int8CacheOracle(hkv, D, T_prefix + L)
    if T_prefix:
        orc.update(k[:, :T_prefix], v[:, :T_prefix])
    ref = orc.update_and_attention(q, k[:, T_prefix:], v[:, T_prefix:], 1.0 / 16, causal)
    kd, vd = orc.fetch()
    pos = oracle_lib.causal_positions(L, T_prefix + L) if causal else None
    f64 = oracle_lib.sdpa_f64(q, kd, vd, 1.0 / 16, q_pos=pos)
    return cache, orc, out, ref, f64


@pytest.mark.gpu
@pytest.mark.parametrize("D", [256, 128])
def test_int8_append_and_fetch_bit_exact(oracle_lib, D):
    """Int8 quantize-on-append (cache.rs:270-305, update_int8 :1042) stores the
    oracle's codes and scales exactly, across ragged appends that fill partial
    8-key blocks; the fetch is f16(code * scale) bit for bit (cache.rs:313)."""
    import qw_amd

    r = rng(8000 + D)
    H = 4
    k, v = _kv(r, H, 203, D)
    k[1, 17] = 0  # an all-zero token: scale 1, codes 0
    cache = qw_amd.KVCache("int8", H, D, capacity=64)
    orc = oracle_lib.Int8CacheOracle(H, D, 203)
    t = 0
    for n in (1, 6, 13, 40, 1, 142):
        cache.update(_gpu(k[:, t:t + n])[None], _gpu(v[:, t:t + n])[None])
        orc.update(k[:, t:t + n], v[:, t:t + n])
        t += n
    assert cache.offset == 203
    snap = cache.snapshot_tensors()
    assert np.array_equal(_np(snap["keys"]), orc.keys[:, :203])
    assert np.array_equal(_np(snap["values"]), orc.values[:, :203])
    assert np.array_equal(_np(snap["key_scales"])[..., 0].view(np.uint16),
                          orc.key_scales[:, :203].view(np.uint16))
    assert np.array_equal(_np(snap["val_scales"])[..., 0].view(np.uint16),
                          orc.val_scales[:, :203].view(np.uint16))
    kd, vd = cache.dequantize()
    ko, vo = orc.fetch()
    assert np.array_equal(_np(kd)[0].view(np.uint16), ko.view(np.uint16))
    assert np.array_equal(_np(vd)[0].view(np.uint16), vo.view(np.uint16))


@pytest.mark.gpu
@pytest.mark.parametrize("T_prefix,L,causal", [
    (4095, 1, False),    # decode over 4096 keys
    (1000, 2, True),     # 2-row verify block (decode kernel)
    (3000, 16, True),    # 16-row verify block (block kernel)
    (300, 64, False),    # block kernel, no mask
    (2000, 520, True),   # 3120 rows a KV head: key tiles dequantized once into LDS images
])
def test_int8_attention_vs_oracle(oracle_lib, T_prefix, L, causal):
    """Attention on an Int8 cache equals the reference's fetch-then-SDPA
    (a6 + a10) within the stated tolerance."""
    import qw_amd

    _, _, out, ref, f64 = _int8_layer_call(oracle_lib, qw_amd, T_prefix, L, causal,
                                           seed=31 + T_prefix + L)
    assert np.isfinite(out).all()
    assert_close(out, ref, f"int8 T={T_prefix}+{L}")
    assert_as_exact_as_reference(out, ref, f64, f"int8 T={T_prefix}+{L}")


@pytest.mark.gpu
def test_int8_snapshot_round_trip_and_trim():
    """Export -> import reproduces the cache (codes, scales, attention); trim
    then re-append equals never appended."""
    import qw_amd

    r = rng(1234)
    k, v = _kv(r, 4, 300, 256)
    a = qw_amd.KVCache("int8", 4, 256)
    a.update(_gpu(k[:, :290])[None], _gpu(v[:, :290])[None])
    snap = a.snapshot_tensors()
    b = qw_amd.KVCache("int8", 4, 256)
    b.restore_snapshot(snap)
    assert b.offset == 290
    for name, t in b.snapshot_tensors().items():
        assert torch.equal(t, snap[name]), name
    q = r.standard_normal((24, 1, 256)).astype(np.float16)
    oa = a.attention(_gpu(q)[None], 1.0 / 16)
    ob = b.attention(_gpu(q)[None], 1.0 / 16)
    assert torch.equal(oa, ob)
    # trim then re-append the same rows
    a.update(_gpu(k[:, 290:])[None], _gpu(v[:, 290:])[None])
    assert a.trim(10) == 10
    a.update(_gpu(k[:, 290:])[None], _gpu(v[:, 290:])[None])
    c = qw_amd.KVCache("int8", 4, 256)
    c.update(_gpu(k)[None], _gpu(v)[None])
    for name, t in c.snapshot_tensors().items():
        assert torch.equal(t, a.snapshot_tensors()[name]), name


@pytest.mark.gpu
@pytest.mark.parametrize("mode", ["affine4", "affine8", "int8"])
@pytest.mark.parametrize("D", [256, 128])
def test_decode_layer_call_stores_what_update_stores(mode, D):
    """A one-row update_and_attention appends in the decode launch's append
    unit; the cache it leaves equals update() of the same rows, codes, scales and biases
    (export bit for bit), over decode steps into a partly filled 8-key V block,
    and its output equals attention over the updated cache."""
    import qw_amd

    H, hq = 4, 24
    r = rng(77 + D)
    k, v = _kv(r, H, 700, D)
    a = qw_amd.KVCache(mode, H, D)
    b = qw_amd.KVCache(mode, H, D)
    a.update(_gpu(k[:, :697])[None], _gpu(v[:, :697])[None])
    b.update(_gpu(k[:, :697])[None], _gpu(v[:, :697])[None])
    for t in (697, 698, 699):
        q = _gpu(r.standard_normal((1, hq, 1, D)).astype(np.float16))
        out = _np(a.update_and_attention(q, _gpu(k[:, t:t + 1])[None], _gpu(v[:, t:t + 1])[None],
                                         1.0 / 16))
        b.update(_gpu(k[:, t:t + 1])[None], _gpu(v[:, t:t + 1])[None])
        ref = _np(b.attention(q, 1.0 / 16))
        assert_close(out, ref, f"{mode} D{D} t{t} fused vs separate")
    sa, sb = a.snapshot_tensors(), b.snapshot_tensors()
    for key in sa:
        np.testing.assert_array_equal(_np(sa[key]), _np(sb[key]), err_msg=f"{mode} {key}")
