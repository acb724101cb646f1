"""The Rust binding recipe of the integration guide (DOC below) stays in step with the build and
the C header: build.rs compiles exactly qw_amd/build.py's SOURCES, and the
extern "C" block declares every entry point of include/qwattn.h with the same
number of arguments. CPU only (text checks)."""
import os
import re

from conftest import ROOT

DOC = os.path.join(ROOT, "INTEGRATION.md")
HEADER = os.path.join(ROOT, "include", "qwattn.h")


def _header_arity():
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    out = {}
    for name, args in re.findall(r"\b(qw_[a-z0-9_]+)\s*\(([^)]*)\)\s*;", text, re.S):
        args = " ".join(args.split())
        out[name] = 0 if args in ("", "void") else len(args.split(","))
    return out


def _ffi_arity():
    text = open(DOC).read()
    block = re.search(r'extern "C" \{(.*?)\n\}', text, re.S).group(1)
    out = {}
    for name, args in re.findall(r"pub fn (qw_[a-z0-9_]+)\(([^)]*)\)", block, re.S):
        args = " ".join(args.split())
        out[name] = 0 if not args else len(args.split(","))
    return out


def test_build_rs_compiles_every_source():
    from qw_amd.build import SOURCES

    text = open(DOC).read()
    m = re.search(r"let sources = \[(.*?)\];", text, re.S)
    assert m, "build.rs has no sources list"
    listed = re.findall(r'"([A-Za-z0-9_]+\.hip)"', m.group(1))
    assert listed == SOURCES


def test_extern_block_declares_the_header():
    hdr, ffi = _header_arity(), _ffi_arity()
    assert set(ffi) == set(hdr), (sorted(set(hdr) - set(ffi)), sorted(set(ffi) - set(hdr)))
    bad = {n: (hdr[n], ffi[n]) for n in hdr if hdr[n] != ffi[n]}
    assert not bad, bad
