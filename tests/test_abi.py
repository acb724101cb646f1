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
