"""GPU parity of the general attention options (qw_sdpa, qw_kv_attention_general,
qw_kv_update_and_attention_general, through the C ABI) against
oracle.sdpa_general: layers::attention's mask and softcap (layers.rs:4010),
causal_attention's sliding window (lib.rs:3185), the masked cache route
(update_and_fetch + attention, qwen3_next.rs:316-324) and the masked Turbo4
route (update_and_turbo4_attention, cache.rs:3495 -> sparse_v.rs:1051-1072).

Bar: 2e-3 max-abs and 1e-3 relative L2 (the attention tolerance); the cache
routes are checked against the oracle fed the cache's own dequantized rows
(whose bit-exactness the KV tests pin)."""
import numpy as np
import pytest

import oracle
from conftest import rng
from test_gpu_kv import _gpu, _np, assert_close

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


def _mask(r, kind, hq, L, T):
    """(numpy mask for the oracle, torch mask for the library)."""
    if kind is None:
        return None, None
    if kind == "bool":
        m = r.random((L, T)) < 0.7
        m[:, 0] = True
        return m, _gpu(m)
    if kind == "f32":
        m = (r.standard_normal((1, L, T)) * 2).astype(np.float32)
        m[0, :, 1::7] = -np.inf
        return m, _gpu(m)
    if kind == "f16_heads":
        m = (r.standard_normal((hq, L, T)) * 3).astype(np.float16)
        return m, _gpu(m)
    if kind == "bf16":
        m = (r.standard_normal((L, T)) * 2).astype(np.float32)
        t = _gpu(m).to(torch.bfloat16)
        return t.float().cpu().numpy(), t  # the values the device holds
    raise ValueError(kind)


CASES = [
    # hq, hkv, D, L, T, causal, window, softcap, mask
    (24, 4, 256, 1, 3000, False, 0, 0.0, None),
    (24, 4, 256, 5, 4100, True, 0, 0.0, "bool"),
    (24, 4, 256, 16, 2049, True, 512, 0.0, None),
    (8, 8, 128, 37, 700, True, 100, 30.0, None),
    (16, 2, 64, 64, 900, False, 0, 50.0, "f32"),
    (6, 1, 128, 3, 1000, False, 0, 0.0, "f16_heads"),
    (24, 4, 256, 200, 1500, True, 0, 0.0, "bf16"),
    (12, 4, 256, 1, 9000, True, 4096, 0.0, None),
    (24, 4, 256, 2048, 2048, True, 0, 0.0, None),
    (16, 2, 128, 2, 777, True, 0, 0.0, "bool"),      # 16 rows a KV head: one-wave launch
    (4, 4, 64, 1, 50, False, 0, 5.0, "f32"),         # shorter than a tile
]


@pytest.mark.parametrize("hq,hkv,D,L,T,causal,window,softcap,mkind", CASES)
def test_sdpa_matches_oracle(hq, hkv, D, L, T, causal, window, softcap, mkind):
    import qw_amd

    print(f"case hq={hq} hkv={hkv} D={D} L={L} T={T} causal={causal} window={window} "
          f"softcap={softcap} mask={mkind}", flush=True)
    r = rng(hq * 7 + D + L + T)
    q = r.standard_normal((hq, L, D)).astype(np.float16)
    k = r.standard_normal((hkv, T, D)).astype(np.float16)
    v = r.standard_normal((hkv, T, D)).astype(np.float16)
    m_np, m_t = _mask(r, mkind, hq, L, T)
    # K/V as views of larger buffers (head and row strides of a cache)
    kb = torch.zeros((hkv, T + 40, D + 64), dtype=torch.float16, device="cuda:0")
    vb = torch.zeros_like(kb)
    kb[:, :T, :D] = _gpu(k)
    vb[:, :T, :D] = _gpu(v)
    out = _np(qw_amd.attention(_gpu(q), kb[:, :T, :D], vb[:, :T, :D], D ** -0.5, m_t, softcap,
                               window, causal))[0]
    ref = oracle.sdpa_general(q, k, v, D ** -0.5, causal, window, softcap, m_np)
    assert np.isfinite(out).all()
    assert_close(out, ref, f"sdpa {mkind} sc={softcap} w={window}")


def test_causal_attention_and_plain_route_agree():
    """causal_attention with no softcap or window is the plain causal SDPA: the
    general kernel within the bar of the fused fp16-cache kernel."""
    import qw_amd

    r = rng(77)
    hq, hkv, D, L, T = 24, 4, 256, 4, 3000
    q = r.standard_normal((hq, L, D)).astype(np.float16)
    k = r.standard_normal((hkv, T, D)).astype(np.float16)
    v = r.standard_normal((hkv, T, D)).astype(np.float16)
    a = _np(qw_amd.causal_attention(_gpu(q), _gpu(k), _gpu(v), 1 / 16))[0]
    cache = qw_amd.KVCache("fp16", hkv, D)
    cache.update(_gpu(k), _gpu(v))
    b = _np(cache.attention(_gpu(q), 1 / 16, causal=True))[0]
    assert_close(a, b, "causal_attention vs fp16 cache")


def test_rows_without_visible_keys_are_zero():
    import qw_amd

    r = rng(78)
    hq, hkv, D, L, T = 4, 2, 128, 3, 500
    q = r.standard_normal((hq, L, D)).astype(np.float16)
    k = r.standard_normal((hkv, T, D)).astype(np.float16)
    v = r.standard_normal((hkv, T, D)).astype(np.float16)
    m = np.ones((L, T), bool)
    m[1] = False
    out = _np(qw_amd.attention(_gpu(q), _gpu(k), _gpu(v), 0.1, _gpu(m)))[0]
    assert np.all(out[:, 1] == 0)
    assert_close(out, oracle.sdpa_general(q, k, v, 0.1, mask=m), "empty row")


@pytest.mark.parametrize("mode", ["affine4", "affine8", "int8", "fp16"])
def test_cache_general_routes(mode):
    import qw_amd

    print(f"case cache {mode}", flush=True)
    r = rng(80 + len(mode))
    hq, hkv, D, T0, L = 24, 4, 256, 3000, 4
    k = r.standard_normal((hkv, T0 + L, D)).astype(np.float16)
    v = r.standard_normal((hkv, T0 + L, D)).astype(np.float16)
    q = r.standard_normal((hq, L, D)).astype(np.float16)
    cache = qw_amd.KVCache(mode, hkv, D)
    cache.update(_gpu(k[:, :T0]), _gpu(v[:, :T0]))
    m_np, m_t = _mask(r, "bool", hq, L, T0 + L)
    # update_and_turbo4_attention(q, k, v, scale, mask) form
    out = _np(cache.update_and_attention(_gpu(q), _gpu(k[:, T0:]), _gpu(v[:, T0:]), 1 / 16,
                                         mask=m_t))[0]
    assert cache.offset == T0 + L
    kd, vd = (_np(x)[0] for x in cache.dequantize())
    assert_close(out, oracle.sdpa_general(q, kd, vd, 1 / 16, mask=m_np), f"{mode} masked update")
    # window and softcap over the cache as it is
    out2 = _np(cache.attention_general(_gpu(q), 1 / 16, causal=True, window=300,
                                       softcap=20.0))[0]
    assert_close(out2, oracle.sdpa_general(q, kd, vd, 1 / 16, True, 300, 20.0),
                 f"{mode} window+softcap")
    # no options: the cache's own fused attention, exactly
    np.testing.assert_array_equal(_np(cache.attention_general(_gpu(q), 1 / 16, causal=True))[0],
                                  _np(cache.attention(_gpu(q), 1 / 16, causal=True))[0])


def test_turbo4_masked_route():
    """Turbo4 with a mask: q rotated into the K basis, the rotated expansion,
    SDPA with the mask, the output rotated back (the reference's
    attention_turbo4_dequant_sdpa with its mask argument)."""
    import qw_amd

    r = rng(90)
    hq, hkv, D, T0, L = 24, 4, 256, 2500, 3
    k = r.standard_normal((hkv, T0 + L, D)).astype(np.float16)
    v = r.standard_normal((hkv, T0 + L, D)).astype(np.float16)
    q = r.standard_normal((hq, L, D)).astype(np.float16)
    cache = qw_amd.KVCache("turbo4", hkv, D)
    cache.update(_gpu(k[:, :T0]), _gpu(v[:, :T0]))
    m = (r.standard_normal((L, T0 + L)) * 2).astype(np.float16)
    out = _np(cache.update_and_attention(_gpu(q), _gpu(k[:, T0:]), _gpu(v[:, T0:]), 1 / 16,
                                         mask=_gpu(m)))[0]
    t = cache.snapshot_tensors()
    snap = {n: _np(x) for n, x in t.items()}
    for n in ("k_rescale", "v_rescale"):
        snap[n] = snap[n][..., 0]
    tab = oracle.turbo4_tables(D)
    q_rot = oracle.turbo4_rotate(q.astype(np.float64), tab["k_s1"], tab["k_s2"]).astype(np.float16)
    k_rot = oracle.turbo4_expand_rotated(snap["k_packed"], snap["k_rescale"], tab)
    v_rot = oracle.turbo4_expand_rotated(snap["v_packed"], snap["v_rescale"], tab)
    o_rot = oracle.sdpa_general(q_rot, k_rot, v_rot, 1 / 16, mask=m)
    ref = oracle.turbo4_rotate(o_rot.astype(np.float64), tab["v_s2"], tab["v_s1"]).astype(np.float16)
    assert_close(out, ref, "turbo4 masked")


@pytest.mark.parametrize("mode", ["affine4", "int8", "turbo4"])
def test_cache_window_reads_only_the_window(mode):
    """A sliding window over a long cache: only the keys from the first row's
    window start are dequantized (Turbo4: expanded from the 256-key boundary
    below it), with the positions and an additive mask's columns shifted
    alike; the result is the windowed attention over the whole cache."""
    import qw_amd

    print(f"case window slice {mode}", flush=True)
    r = rng(95 + len(mode))
    hq, hkv, D, T0, L, W = 24, 4, 256, 5000, 3, 700
    T = T0 + L
    k = r.standard_normal((hkv, T, D)).astype(np.float16)
    v = r.standard_normal((hkv, T, D)).astype(np.float16)
    q = r.standard_normal((hq, L, D)).astype(np.float16)
    cache = qw_amd.KVCache(mode, hkv, D)
    cache.update(_gpu(k), _gpu(v))
    # an additive mask over all T keys whose finite columns below the window
    # would change the result if the shift were off by any amount
    m = (r.standard_normal((L, T)) * 2).astype(np.float16)
    m[:, T - W - L + 5::11] = -np.inf
    for softcap, mask in ((0.0, None), (0.0, m), (15.0, m)):
        out = _np(cache.attention_general(_gpu(q), 1 / 16, causal=True, window=W,
                                          softcap=softcap,
                                          mask=None if mask is None else _gpu(mask)))[0]
        if mode == "turbo4":
            t = cache.snapshot_tensors()
            snap = {n: _np(x) for n, x in t.items()}
            for n in ("k_rescale", "v_rescale"):
                snap[n] = snap[n][..., 0]
            tab = oracle.turbo4_tables(D)
            q_rot = oracle.turbo4_rotate(q.astype(np.float64), tab["k_s1"],
                                         tab["k_s2"]).astype(np.float16)
            k_rot = oracle.turbo4_expand_rotated(snap["k_packed"], snap["k_rescale"], tab)
            v_rot = oracle.turbo4_expand_rotated(snap["v_packed"], snap["v_rescale"], tab)
            o_rot = oracle.sdpa_general(q_rot, k_rot, v_rot, 1 / 16, True, W, softcap, mask)
            ref = oracle.turbo4_rotate(o_rot.astype(np.float64), tab["v_s2"],
                                       tab["v_s1"]).astype(np.float16)
        else:
            kd, vd = (_np(x)[0] for x in cache.dequantize())
            ref = oracle.sdpa_general(q, kd, vd, 1 / 16, True, W, softcap, mask)
        assert_close(out, ref, f"{mode} window {W} softcap {softcap} mask {mask is not None}")


WIN_CASES = [
    # mode, hq, hkv, D, T (after the rows), L, window
    ("affine4", 24, 4, 256, 32769, 1, 4096),   # a windowed decode step at the c2 geometry
    ("affine4", 24, 4, 256, 9000, 4, 1000),    # a verify block
    ("affine8", 24, 4, 256, 5000, 37, 300),    # 222 rows a KV head: two query tiles
    ("int8", 16, 2, 128, 3000, 5, 64),
    ("fp16", 8, 8, 128, 2500, 300, 700),       # a prefill chunk whose windows slide
    ("affine4", 6, 1, 128, 700, 3, 1),         # every row sees only its own key
    ("affine8", 24, 4, 256, 1200, 2, 5000),    # a window wider than the cache
]


@pytest.mark.parametrize("mode,hq,hkv,D,T,L,W", WIN_CASES)
def test_cache_window_fused_route(mode, hq, hkv, D, T, L, W):
    """A causal sliding window without mask or softcap over an affine, Int8 or
    fp16 cache runs the block kernel on the codes (a lower bound on each
    row's keys, splits over the keys the windows span): checked against the
    oracle on the cache's own dequantized rows."""
    import qw_amd

    print(f"case window fused {mode} hq={hq} hkv={hkv} D={D} T={T} L={L} W={W}", flush=True)
    r = rng(700 + L + W % 97)
    k = r.standard_normal((hkv, T, D)).astype(np.float16)
    v = r.standard_normal((hkv, T, D)).astype(np.float16)
    q = r.standard_normal((hq, L, D)).astype(np.float16)
    cache = qw_amd.KVCache(mode, hkv, D)
    cache.update(_gpu(k), _gpu(v))
    out = _np(cache.attention_general(_gpu(q), D ** -0.5, causal=True, window=W))[0]
    kd, vd = (_np(x)[0] for x in cache.dequantize())
    ref = oracle.sdpa_general(q, kd, vd, D ** -0.5, True, W)
    assert_close(out, ref, f"{mode} window {W} L {L}")
    if W == 1:
        # one visible key: the row is that key's V row, exactly
        G = hq // hkv
        for h in range(hq):
            np.testing.assert_array_equal(out[h], vd[h // G, T - L:T])
    cache.close()


def test_cache_window_long_prefill_rows():
    """A windowed prefill long enough that whole rounds of query tiles run
    unsplit and the rest split their keys (19200 rows a KV head: 128 unsplit
    tiles, 22 split), checked row by row: row r (position p) against the
    oracle on keys 0 .. p with the same window."""
    import qw_amd

    print("case window long prefill", flush=True)
    r = rng(905)
    hq, hkv, D, L, T0, W = 8, 2, 128, 4800, 1000, 700
    T = T0 + L
    G = hq // hkv
    k = r.standard_normal((hkv, T, D)).astype(np.float16)
    v = r.standard_normal((hkv, T, D)).astype(np.float16)
    q = r.standard_normal((hq, L, D)).astype(np.float16)
    cache = qw_amd.KVCache("affine4", hkv, D)
    cache.update(_gpu(k), _gpu(v))
    out = _np(cache.attention_general(_gpu(q), D ** -0.5, causal=True, window=W))[0]
    kd, vd = (_np(x)[0] for x in cache.dequantize())
    for row in (0, 1, 31, 32, 2000, 4095, 4096, 4500, 4799):  # rows 4096.. sit in split tiles
        p = T0 + row
        ref = oracle.sdpa_general(q[:, row:row + 1], kd[:, :p + 1], vd[:, :p + 1], D ** -0.5,
                                  True, W)
        assert_close(out[:, row:row + 1], ref, f"long window prefill row {row}")
    assert G * L == 19200
    cache.close()


CAP_CASES = [
    # mode, hq, hkv, D, T (after the rows), L, window, softcap, causal
    ("affine4", 24, 4, 256, 32769, 1, 0, 30.0, True),   # a softcapped decode step, c2 geometry
    ("affine8", 24, 4, 256, 5000, 37, 0, 50.0, True),
    ("int8", 16, 2, 128, 3000, 5, 0, 20.0, False),
    ("fp16", 8, 8, 128, 2500, 300, 700, 30.0, True),   # softcap and a sliding window
    ("affine4", 6, 1, 128, 700, 3, 0, 5.0, False),     # a cap that bends most scores
]


@pytest.mark.parametrize("mode,hq,hkv,D,T,L,W,cap,causal", CAP_CASES)
def test_cache_softcap_fused_route(mode, hq, hkv, D, T, L, W, cap, causal):
    """A logit softcap (with or without a causal window) and no mask over an
    affine, Int8 or fp16 cache runs the block kernel on the codes with the
    softcap composite's arithmetic (S = f16(q . k), tanh in fp32, fp32 P):
    checked against the oracle on the cache's own dequantized rows."""
    import qw_amd

    print(f"case softcap fused {mode} D={D} T={T} L={L} W={W} cap={cap} causal={causal}",
          flush=True)
    r = rng(800 + L + int(cap))
    k = (r.standard_normal((hkv, T, D)) * 2).astype(np.float16)
    v = r.standard_normal((hkv, T, D)).astype(np.float16)
    q = (r.standard_normal((hq, L, D)) * 2).astype(np.float16)
    cache = qw_amd.KVCache(mode, hkv, D)
    cache.update(_gpu(k), _gpu(v))
    out = _np(cache.attention_general(_gpu(q), D ** -0.5, causal=causal, window=W,
                                      softcap=cap))[0]
    kd, vd = (_np(x)[0] for x in cache.dequantize())
    ref = oracle.sdpa_general(q, kd, vd, D ** -0.5, causal, W, cap)
    assert_close(out, ref, f"{mode} softcap {cap} window {W}")
    cache.close()


@pytest.mark.parametrize("mode", ["affine4", "affine8"])
def test_fused_options_with_extreme_scales(mode):
    """Groups whose scales miss the 2-op dequant's exact range (|scale| < 2^-10
    or >= 64) send the fused window and softcap launches through their second,
    separately rounded pass, which must match the composite dequant the
    cache's own dequantize() returns."""
    import qw_amd

    print(f"case extreme fused options {mode}", flush=True)
    r = rng(860 + len(mode))
    hq, hkv, D, T, L = 24, 4, 256, 3000, 4
    k = r.standard_normal((hkv, T, D)).astype(np.float32)
    v = r.standard_normal((hkv, T, D)).astype(np.float32)
    k[:, 2500:2540, :64] *= 1e-3
    k[:, 2900:2901, 64:128] *= 300.0
    v[:, 2600:2660, 128:192] *= 1e-3
    v[:, 2950:2960, :64] *= 100.0
    k, v = k.astype(np.float16), v.astype(np.float16)
    q = r.standard_normal((hq, L, D)).astype(np.float16)
    cache = qw_amd.KVCache(mode, hkv, D)
    cache.update(_gpu(k), _gpu(v))
    kd, vd = (_np(x)[0] for x in cache.dequantize())
    for W, cap in ((600, 0.0), (0, 30.0), (600, 30.0)):
        out = _np(cache.attention_general(_gpu(q), 1 / 16, causal=True, window=W,
                                          softcap=cap))[0]
        ref = oracle.sdpa_general(q, kd, vd, 1 / 16, True, W, cap)
        assert_close(out, ref, f"{mode} extreme window {W} softcap {cap}")
    cache.close()


def test_general_contract_errors():
    import qw_amd

    q = torch.zeros((4, 2, 128), dtype=torch.float16, device="cuda:0")
    k = torch.zeros((2, 50, 128), dtype=torch.float16, device="cuda:0")
    m = torch.ones((2, 50), dtype=torch.bool, device="cuda:0")
    with pytest.raises(qw_amd.QwError) as e:  # bool mask with softcap
        qw_amd.attention(q, k, k, 0.1, m, 10.0)
    assert e.value.status == 2
    with pytest.raises(qw_amd.QwError):  # a window needs causal
        qw_amd.attention(q, k, k, 0.1, None, 0.0, 16, False)
    with pytest.raises(qw_amd.QwError):  # mask shape
        qw_amd.attention(q, k, k, 0.1, torch.ones((3, 50), dtype=torch.bool, device="cuda:0"))
    with pytest.raises(qw_amd.QwError):  # head dim 96
        qw_amd.attention(q[..., :96].contiguous(), k[..., :96].contiguous(),
                         k[..., :96].contiguous(), 0.1)
    # a rejected update leaves the cache as it was
    cache = qw_amd.KVCache("affine4", 2, 128)
    cache.update(k, k)
    with pytest.raises(qw_amd.QwError):
        cache.update_and_attention_general(q, k[:, :2], k[:, :2], 0.1, False, 8, 0.0, None)
    assert cache.offset == 50


def _torch_fp32_attention(q, k, v, scale, causal, window, softcap, mask):
    """Plain PyTorch fp32 attention of the same op (on the CPU): no fp16
    roundings of the scores or probabilities."""
    qf, kf, vf = (torch.from_numpy(np.asarray(x, np.float32)) for x in (q, k, v))
    hq, L, D = qf.shape
    hkv, T, _ = kf.shape
    G = hq // hkv
    kf = kf.repeat_interleave(G, dim=0)
    vf = vf.repeat_interleave(G, dim=0)
    s = torch.matmul(qf, kf.transpose(1, 2).contiguous()) * scale
    if softcap > 0:
        s = torch.tanh(s / softcap) * softcap
    t = torch.arange(T)[None, :]
    p = (T - L + torch.arange(L))[:, None]
    vis = torch.ones((L, T), dtype=torch.bool)
    if causal:
        vis &= t <= p
    if window > 0:
        vis &= t >= p - window + 1
    vis = vis[None].expand(hq, L, T).clone()
    if mask is not None:
        m = torch.from_numpy(np.ascontiguousarray(mask))
        m = m.reshape(-1, L, T).expand(hq, L, T)
        if m.dtype == torch.bool:
            vis &= m
        else:
            s = s + m.float()
    s = s.masked_fill(~vis, float("-inf"))
    return torch.matmul(torch.softmax(s, dim=-1), vf).numpy()


@pytest.mark.parametrize("causal,window,softcap,mkind", [
    (True, 0, 0.0, None), (True, 300, 0.0, "bool"), (False, 0, 25.0, "f32"), (True, 0, 40.0, None)])
def test_sdpa_against_torch_fp32(causal, window, softcap, mkind):
    """An independent check of the general kernel: PyTorch fp32 attention of
    the same op, which skips MLX's fp16 roundings of S (and of P without
    softcap), so the bar is the fp16 budget those roundings leave: 5e-3
    max-abs, 3e-3 relative L2."""
    import qw_amd

    r = rng(501 + int(softcap) + window)
    hq, hkv, D, L, T = 12, 2, 128, 6, 1500
    q = r.standard_normal((hq, L, D)).astype(np.float16)
    k = r.standard_normal((hkv, T, D)).astype(np.float16)
    v = r.standard_normal((hkv, T, D)).astype(np.float16)
    m_np, m_t = _mask(r, mkind, hq, L, T)
    if m_np is not None and m_np.dtype != np.bool_:
        m_np = m_np.astype(np.float16).astype(np.float32)  # the cast the reference applies
    out = _np(qw_amd.attention(_gpu(q), _gpu(k), _gpu(v), D ** -0.5, m_t, softcap, window,
                               causal))[0].astype(np.float64)
    ref = _torch_fp32_attention(q, k, v, D ** -0.5, causal, window, softcap, m_np)
    err = np.abs(out - ref)
    rel = np.linalg.norm(out - ref) / np.linalg.norm(ref)
    print(f"torch fp32 {mkind} sc={softcap} w={window}: max_abs={err.max():.3e} rel_l2={rel:.3e}",
          flush=True)
    assert err.max() < 5e-3 and rel < 3e-3
