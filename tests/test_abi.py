"""The C ABI library loads and exports every entry point include/qwattn.h
declares; argument checks that run before any device call return the
documented status codes. CPU only: nothing here launches a kernel."""
import ctypes
import os
import re

import pytest

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "qwattn.h")


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(qw_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def qwlib():
    import qw_amd

    if not os.path.exists(qw_amd.LIB_PATH):
        from qw_amd import build

        build.build()
    return qw_amd.lib()


def test_header_declares_the_path():
    names = _declared()
    for n in ("qw_kv_create", "qw_kv_update", "qw_kv_update_and_attention", "qw_kv_trim",
              "qw_kv_export", "qw_kv_import", "qw_dlsa_sparse_attention"):
        assert n in names


def test_every_declared_symbol_is_exported(qwlib):
    missing = [n for n in _declared() if not hasattr(qwlib, n)]
    assert not missing, missing


def test_abi_version_matches_header(qwlib):
    m = re.search(r"#define QWATTN_ABI_VERSION (\d+)", open(HEADER).read())
    assert qwlib.qw_abi_version() == int(m.group(1))


def test_invalid_arguments_fail_before_device_work(qwlib):
    h = ctypes.c_void_p()
    assert qwlib.qw_kv_create(7, 64, 4, 256, 1024, 0, ctypes.byref(h)) == 1
    assert b"mode" in qwlib.qw_last_error()
    assert qwlib.qw_kv_create(2, 32, 4, 256, 1024, 0, ctypes.byref(h)) == 2  # group != 64
    assert qwlib.qw_kv_create(2, 64, 4, 96, 1024, 0, ctypes.byref(h)) == 2   # head_dim
    assert qwlib.qw_kv_create(2, 64, 0, 256, 1024, 0, ctypes.byref(h)) == 1
    assert qwlib.qw_kv_create(2, 64, 4, 256, 1024, 0, None) == 1
    assert not h.value
    # null handle
    off = ctypes.c_int()
    assert qwlib.qw_kv_offset(None, ctypes.byref(off)) == 1
    assert qwlib.qw_kv_trim(None, 1, None) == 1
    assert qwlib.qw_kv_destroy(None) == 0
    # D-LSA geometry checks
    f = qwlib.qw_dlsa_sparse_attention
    assert f(None, None, None, 0, 0, 0, 0, None, None, 1, 1, 24, 4, 256, 10, 0.1, None, None) == 1
    one = ctypes.c_void_p(16)
    args = [one, one, one, 0, 256, 0, 256, one, one, 1, 8, 24, 4, 256, 10, 0.1, one, None]
    args_bad_dim = list(args)
    args_bad_dim[13] = 96
    assert f(*args_bad_dim) == 1
    args_bad_g = list(args)
    args_bad_g[11], args_bad_g[12] = 68, 4  # 17 heads per KV head
    assert f(*args_bad_g) == 1
    args_bad_w = list(args)
    args_bad_w[10] = 0
    assert f(*args_bad_w) == 1


def test_fused_rope_contract_fails_before_device_work(qwlib):
    """fused_rope_append.cpp:394-418: the argument contract, checked before
    any launch (status 1, QW_ERR_INVALID_ARGUMENT)."""
    f = qwlib.qw_fused_rope_qk_append
    one = ctypes.c_void_p(16)

    def call(**kw):
        a = dict(batch=1, seq=4, hq=8, hkv=2, D=128, R=64, base=10000.0, scale=1.0, trad=0,
                 pos=0, layout=0)
        a.update(kw)
        return f(one, a["batch"], a["seq"], a["hq"], a["hkv"], a["D"], a["R"], a["base"],
                 a["scale"], a["trad"], a["pos"], a["layout"], one, one, one, None)

    assert call(R=0) == 1
    assert b"rope_dims" in qwlib.qw_last_error()
    assert call(R=63) == 1
    assert call(R=130) == 1
    assert call(D=127, R=64) == 1
    assert b"head_dim must be even" in qwlib.qw_last_error()
    assert call(hq=0) == 1
    assert call(hkv=-1) == 1
    assert call(layout=2) == 1
    assert b"dest_layout" in qwlib.qw_last_error()
    assert call(seq=-1) == 1
    assert call(seq=0) == 0  # nothing to do: no launch
    assert f(None, 1, 4, 8, 2, 128, 64, 10000.0, 1.0, 0, 0, 0, None, None, None, None) == 1
    assert qwlib.qw_kv_rope_update(None, one, 8, 4, 64, 0, 10000.0, 1.0, 0, one, None) == 1


def test_general_attention_contract_fails_before_device_work(qwlib):
    """qw_sdpa's argument contract (mask, softcap and window as the reference's
    layers::attention / causal_attention take them), checked before any HIP
    call."""
    f = qwlib.qw_sdpa
    one = ctypes.c_void_p(16)

    def call(**kw):
        a = dict(hq=8, L=4, hkv=2, T=100, D=128, causal=1, window=0, softcap=0.0, mask=None,
                 md=0, mhs=0, mrs=100)
        a.update(kw)
        return f(one, a["hq"], a["L"], one, one, a["hkv"], a["T"], a["D"], a["T"] * a["D"],
                 a["D"], a["T"] * a["D"], a["D"], 0.1, a["causal"], a["window"], a["softcap"],
                 a["mask"], a["md"], a["mhs"], a["mrs"], one, None)

    assert call(D=96) == 1
    assert call(hq=9) == 1                     # not a multiple of the KV heads
    assert call(T=3) == 1                      # causal with fewer keys than rows
    assert call(causal=0, window=8) == 1       # a window is the windowed causal mask
    assert b"window" in qwlib.qw_last_error()
    assert call(softcap=-1.0) == 1
    assert call(mask=one, md=7) == 1           # unknown mask dtype
    assert call(mask=one, md=3, softcap=5.0) == 2  # bool mask with softcap
    assert b"bool mask" in qwlib.qw_last_error()
    assert call(mask=one, md=0, mrs=-1) == 1
    assert f(None, 8, 4, one, one, 2, 100, 128, 0, 128, 0, 128, 0.1, 1, 0, 0.0, None, 0, 0, 0,
             one, None) == 1
