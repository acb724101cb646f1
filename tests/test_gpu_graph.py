"""HIP-graph capture of the hot-path calls through the C ABI.

A captured decode / verify / D-LSA call must give the eager result on every
replay, with eager work and synchronizations between the replays, and a
split-K workspace that grows after the capture (a larger call on the same
cache or stream) must not break the captured graph: the old buffer is retired,
not freed, while a graph may still read it."""
import numpy as np
import pytest

from conftest import rng
from test_gpu_kv import _gpu, _np

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


def _cache(mode, r, H, T, D):
    import qw_amd

    k = r.standard_normal((H, T, D)).astype(np.float16)
    v = r.standard_normal((H, T, D)).astype(np.float16)
    c = qw_amd.KVCache(mode, H, D, capacity=T + 256)
    c.update(_gpu(k), _gpu(v))
    return c


@pytest.mark.parametrize("mode", ["affine4", "affine8"])
def test_graph_attention_replays_and_growth(mode):
    """Decode (1 row) and a 16-row verify block captured in one graph; replays
    equal the eager outputs, before and after a 2048-row prefill-sized call
    grows the cache's split-K workspace."""
    r = rng(11)
    H, G, D, T = 4, 6, 256, 9000
    c = _cache(mode, r, H, T, D)
    q1 = _gpu(r.standard_normal((H * G, 1, D)).astype(np.float16))
    q16 = _gpu(r.standard_normal((H * G, 16, D)).astype(np.float16))
    want1 = _np(c.attention(q1, 1 / 16))
    want16 = _np(c.attention(q16, 1 / 16, causal=True))
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):  # size the workspace on the capture stream
        o1 = c.attention(q1, 1 / 16)
        o16 = c.attention(q16, 1 / 16, causal=True)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        o1 = c.attention(q1, 1 / 16)
        o16 = c.attention(q16, 1 / 16, causal=True)
    for rep in range(3):
        o1.zero_()
        o16.zero_()
        g.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(_np(o1), want1, err_msg=f"replay {rep}")
        np.testing.assert_array_equal(_np(o16), want16, err_msg=f"replay {rep}")
        _ = (q1.float() * 2).sum().item()  # eager work between replays
    # a 2048-row causal call needs a larger split workspace: it grows
    q2k = _gpu(r.standard_normal((H * G, 2048, D)).astype(np.float16))
    big = _np(c.attention(q2k, 1 / 16, causal=True))
    assert np.isfinite(big).all()
    for rep in range(2):
        o1.zero_()
        o16.zero_()
        g.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(_np(o1), want1, err_msg=f"after growth, replay {rep}")
        np.testing.assert_array_equal(_np(o16), want16, err_msg=f"after growth, replay {rep}")
    del g
    c.close()


def test_graph_window_and_softcap_routes():
    """The fused window and softcap launches (the block kernel's WIN / CAP
    instances over the codes, split partials and their merge) captured in one
    graph: replays equal the eager outputs, with eager work between them, also
    after a larger call grows the cache's split-K workspace."""
    r = rng(13)
    H, G, D, T = 4, 6, 256, 9000
    c = _cache("affine4", r, H, T, D)
    q1 = _gpu(r.standard_normal((H * G, 1, D)).astype(np.float16))
    q4 = _gpu(r.standard_normal((H * G, 4, D)).astype(np.float16))
    want_w = _np(c.attention_general(q1, 1 / 16, causal=True, window=700))
    want_c = _np(c.attention_general(q4, 1 / 16, causal=True, softcap=30.0))
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):  # size the workspace on the capture stream
        c.attention_general(q1, 1 / 16, causal=True, window=700)
        c.attention_general(q4, 1 / 16, causal=True, softcap=30.0)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        o_w = c.attention_general(q1, 1 / 16, causal=True, window=700)
        o_c = c.attention_general(q4, 1 / 16, causal=True, softcap=30.0)
    for rep in range(3):
        o_w.zero_()
        o_c.zero_()
        g.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(_np(o_w), want_w, err_msg=f"window replay {rep}")
        np.testing.assert_array_equal(_np(o_c), want_c, err_msg=f"softcap replay {rep}")
        _ = (q1.float() * 2).sum().item()  # eager work between replays
    q2k = _gpu(r.standard_normal((H * G, 2048, D)).astype(np.float16))
    big = _np(c.attention(q2k, 1 / 16, causal=True))
    assert np.isfinite(big).all()
    for rep in range(2):
        o_w.zero_()
        o_c.zero_()
        g.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(_np(o_w), want_w, err_msg=f"after growth, window {rep}")
        np.testing.assert_array_equal(_np(o_c), want_c, err_msg=f"after growth, softcap {rep}")
    del g
    c.close()


def test_graph_dlsa_replays_and_growth():
    """A D-LSA read captured on its own stream: replays equal the eager
    output, also after a larger call grows that stream's workspace."""
    import qw_amd

    r = rng(12)
    T, H, G, D, W = 6000, 4, 6, 256, 900
    k = _gpu(r.standard_normal((H, T, D)).astype(np.float16))
    v = _gpu(r.standard_normal((H, T, D)).astype(np.float16))
    q = _gpu(r.standard_normal((H * G, 1, D)).astype(np.float16))
    lists = _gpu(r.choice(T, W, replace=False).astype(np.int32)[None])
    lens = _gpu(np.array([W], np.int32))
    want = _np(qw_amd.sparse_attention(q, k, v, lists, lens, D ** -0.5))
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        out = qw_amd.sparse_attention(q, k, v, lists, lens, D ** -0.5)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        out = qw_amd.sparse_attention(q, k, v, lists, lens, D ** -0.5)
    for rep in range(3):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(_np(out), want, err_msg=f"replay {rep}")
    # 8 rows x 128 parts on the same stream: a much larger workspace
    q8 = _gpu(r.standard_normal((H * G, 8, D)).astype(np.float16))
    l8 = _gpu(np.stack([r.choice(T, W, replace=False) for _ in range(8)]).astype(np.int32))
    n8 = _gpu(np.full(8, W, np.int32))
    with torch.cuda.stream(s):
        big = qw_amd.sparse_attention_with(q8, k, v, l8, n8, D ** -0.5, 128, 0)
    torch.cuda.synchronize()
    assert np.isfinite(_np(big)).all()
    for rep in range(2):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(_np(out), want, err_msg=f"after growth, replay {rep}")


def test_graph_dlsa_first_use_inside_capture():
    """A stream whose D-LSA workspace does not exist yet when the capture
    starts: HIP allows no allocation during the capture, so the call fails
    with QW_ERR_STATE and a message saying to run one call before capturing,
    without invalidating the capture; the same call then works eagerly and
    under a new capture on that stream."""
    import qw_amd

    r = rng(13)
    T, H, G, D, W = 4000, 4, 6, 256, 700
    k = _gpu(r.standard_normal((H, T, D)).astype(np.float16))
    v = _gpu(r.standard_normal((H, T, D)).astype(np.float16))
    q = _gpu(r.standard_normal((H * G, 1, D)).astype(np.float16))
    lists = _gpu(r.choice(T, W, replace=False).astype(np.int32)[None])
    lens = _gpu(np.array([W], np.int32))
    want = _np(qw_amd.sparse_attention(q, k, v, lists, lens, D ** -0.5))
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with pytest.raises(qw_amd.QwError) as ei:
        with torch.cuda.graph(g, stream=s):
            qw_amd.sparse_attention(q, k, v, lists, lens, D ** -0.5)
    assert ei.value.status == 5 and "before capturing" in str(ei.value)
    assert not torch.cuda.is_current_stream_capturing()
    del g
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        np.testing.assert_array_equal(_np(qw_amd.sparse_attention(q, k, v, lists, lens,
                                                                  D ** -0.5)), want)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        out = qw_amd.sparse_attention(q, k, v, lists, lens, D ** -0.5)
    for rep in range(2):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(_np(out), want, err_msg=f"replay {rep}")


def test_graph_turbo4_routes():
    """Turbo4 attention captured in a HIP graph: the decode route (one row)
    and the fused verify route (4 causal rows past 2048 tokens).
    The route's workspace is per stream, so both capture; replays equal the
    eager outputs, with eager work between the replays, also after a larger
    call grows the stream's workspace."""
    r = rng(14)
    H, G, D, T = 4, 6, 256, 3000
    c = _cache("turbo4", r, H, T, D)
    q1 = _gpu(r.standard_normal((H * G, 1, D)).astype(np.float16))
    q4 = _gpu(r.standard_normal((H * G, 4, D)).astype(np.float16))
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):  # size the stream's workspaces before capturing
        want1 = _np(c.attention(q1, 1 / 16))
        want4 = _np(c.attention(q4, 1 / 16, causal=True))
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        o1 = c.attention(q1, 1 / 16)
        o4 = c.attention(q4, 1 / 16, causal=True)
    for rep in range(3):
        o1.zero_()
        o4.zero_()
        g.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(_np(o1), want1, err_msg=f"decode replay {rep}")
        np.testing.assert_array_equal(_np(o4), want4, err_msg=f"verify replay {rep}")
        _ = (q1.float() * 2).sum().item()
    # a 64-row block on the same stream needs a larger workspace: it grows
    q64 = _gpu(r.standard_normal((H * G, 64, D)).astype(np.float16))
    with torch.cuda.stream(s):
        big = _np(c.attention(q64, 1 / 16, causal=True))
    torch.cuda.synchronize()
    assert np.isfinite(big).all()
    for rep in range(2):
        o1.zero_()
        o4.zero_()
        g.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(_np(o1), want1, err_msg=f"after growth, decode replay {rep}")
        np.testing.assert_array_equal(_np(o4), want4, err_msg=f"after growth, verify replay {rep}")
    del g
    c.close()


@pytest.mark.parametrize("mode,L", [("affine8", 600), ("turbo4", 200)])
def test_graph_tile_image_route(mode, L):
    """A long prefill call (the key tiles expanded once into LDS images, then
    copied into LDS by the attention launch) captured in a HIP graph: replays
    equal the eager output, with eager work between them, also after a larger
    call grows the stream's image workspace."""
    r = rng(21)
    H, G, D, T = 4, 6, 256, 1500
    c = _cache(mode, r, H, T, D)
    q = _gpu(r.standard_normal((H * G, L, D)).astype(np.float16))
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):  # size the stream's workspaces before capturing
        want = _np(c.attention(q, 1 / 16, causal=True))
    torch.cuda.synchronize()
    assert np.isfinite(want).all()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        o = c.attention(q, 1 / 16, causal=True)
    for rep in range(3):
        o.zero_()
        g.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(_np(o), want, err_msg=f"replay {rep}")
        _ = (q.float() * 2).sum().item()  # eager work between replays
    # more keys: a larger image workspace on the same stream
    k = _gpu(r.standard_normal((H, 2000, D)).astype(np.float16))
    big_c = _cache(mode, r, H, 1, D)
    big_c.update(k, k)
    with torch.cuda.stream(s):
        big = _np(big_c.attention(q, 1 / 16, causal=True))
    torch.cuda.synchronize()
    assert np.isfinite(big).all()
    for rep in range(2):
        o.zero_()
        g.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(_np(o), want, err_msg=f"after growth, replay {rep}")
    del g
    c.close()
    big_c.close()


def test_graph_general_options_replay():
    """The general options captured in a graph: a masked SDPA over K/V views,
    a softcap-and-window call, and a masked call over an affine cache (its
    rows dequantized into the stream's workspace inside the graph); every
    replay equals the eager output, with eager work between replays."""
    import qw_amd

    r = rng(13)
    H, G, D, T, L = 4, 6, 256, 3000, 5
    k = _gpu(r.standard_normal((H, T, D)).astype(np.float16))
    v = _gpu(r.standard_normal((H, T, D)).astype(np.float16))
    q = _gpu(r.standard_normal((H * G, L, D)).astype(np.float16))
    m = _gpu(r.random((L, T)) < 0.6)
    madd = _gpu((r.standard_normal((L, T)) * 2).astype(np.float16))
    c = _cache("affine4", r, H, T, D)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())

    def calls():
        return (qw_amd.attention(q, k, v, 1 / 16, m),
                qw_amd.causal_attention(q, k, v, 1 / 16, 30.0, 700),
                c.attention_general(q, 1 / 16, mask=madd))

    with torch.cuda.stream(s):  # size the stream's workspaces first
        want = [_np(x) for x in calls()]
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        outs = calls()
    for rep in range(3):
        for o in outs:
            o.zero_()
        g.replay()
        torch.cuda.synchronize()
        for o, w in zip(outs, want):
            np.testing.assert_array_equal(_np(o), w, err_msg=f"replay {rep}")
        _ = (q.float() * 3).sum().item()  # eager work between replays
    del g
    c.close()
