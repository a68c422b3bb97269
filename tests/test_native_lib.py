"""The C-ABI library loads without a GPU and exports exactly what
include/ab_attention.h declares; its host-side validation answers without
touching the device."""
import ctypes
import os
import re

import pytest

from ab_attention import _lib

INCLUDE = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include")


def _declared(header):
    text = open(os.path.join(INCLUDE, header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ab_\w+)\s*\(", text)))


def test_every_declared_symbol_is_exported():
    lib = _lib.load()
    names = _declared("ab_attention.h")
    assert len(names) >= 9
    for name in names:
        assert hasattr(lib, name), name
    assert sorted(_lib.SIGNATURES) == names


def test_static_library_exports_its_header():
    static = _lib.load_static()
    names = _declared("ab_attention_static.h")
    assert names == ["ab_ibcs_sip_static"] == sorted(_lib.STATIC_SIGNATURES)
    for name in names:
        assert hasattr(static, name), name
    assert not hasattr(_lib.load(), "ab_ibcs_sip_static")  # the main library carries no static scratch


def test_prefill_launch_geometry():
    lib = _lib.load()
    # row slots per XCD and launch: whole generations of 64
    for bh, n, launches in ((80, 75600, 5), (24, 32760, 1), (24, 119056, 3), (2, 2048, 1), (1, 128, 1)):
        per = lib.ab_prefill_launch_slots(bh, n)
        slots = -(-(-(-n // 128)) // 8) * bh
        assert per > 0 and per % 64 == 0
        assert -(-slots // per) == launches, (bh, n, per)
    assert lib.ab_prefill_launch_slots(0, 100) == 0


def test_abi_version():
    assert _lib.load().ab_abi_version() == _lib.ABI_VERSION


def test_workspace_and_stride_queries():
    lib = _lib.load()
    assert lib.ab_ibcs_lse_stride(75600) == 18944  # 18,900 rounded up to 64
    assert lib.ab_ibcs_lse_stride(2048) == 512
    ws = lib.ab_ibcs_workspace_bytes(80, 75600)
    rows = 80 * 591
    assert ws >= rows * 8 * 18944 * 2 + rows * 8 * 128 * 2
    assert ws % 256 == 0
    assert lib.ab_ibcs_workspace_bytes(0, 100) == 0


@pytest.mark.parametrize("call,msg", [
    (lambda L: L.ab_sip(None, None, 4, 16, 16, None, None, None), b"inside the population"),
    (lambda L: L.ab_sip(None, None, 4, 16, 0, None, None, None), b"inside the population"),
    (lambda L: L.ab_ibcs(None, None, 1, 1022, None, 0, None, None), b"divisible by 4"),
    (lambda L: L.ab_ibcs(None, None, 1, 4 * 40000, None, 0, None, None), b"32768"),
    (lambda L: L.ab_paged_prefill(None, None, None, 1, 1024, None, None, 48, None, None, None), b"multiple of 32"),
    (lambda L: L.ab_paged_prefill(None, None, None, 1, 1024, None, None, 64, None, None, None), b"null pointer"),
    (lambda L: L.ab_dense_prefill(None, None, None, 1, 1024, 1022, None, None, None), b"divisible by 4"),
    (lambda L: L.ab_dense_prefill(None, None, None, 1, 1024, 1024, None, None, None), b"null pointer"),
    (lambda L: L.ab_ibcs_sip_exact_draws(None, None, None, 1, 1024, None, 300, None, 0, None, None, None),
     b"inside the population"),
])
def test_validation_before_launch(call, msg):
    lib = _lib.load()
    assert call(lib) == 1
    assert msg in lib.ab_last_error()


_A = 4096  # a 16-byte aligned stand-in address: every case is rejected before any runtime call


@pytest.mark.parametrize("args,msg", [
    ((_A, _A, None, 1, 1022, _A, 64, _A, _A, None), b"divisible by 4"),
    ((_A, _A, None, 1, 4 * 40000, _A, 64, _A, _A, None), b"32768"),
    ((_A, _A, None, 70000, 1024, _A, 64, _A, _A, None), b"grid too large"),
    ((_A, _A, None, 1, 1024, _A, 300, _A, _A, None), b"inside the population"),
    ((_A, _A, None, 1, 1024, _A, 0, _A, _A, None), b"inside the population"),
    ((_A, None, None, 1, 1024, _A, 64, _A, _A, None), b"null pointer"),
    ((_A, _A, None, 1, 1024, _A, 64, None, _A, None), b"null pointer"),
    ((_A + 8, _A, None, 1, 1024, _A, 64, _A, _A, None), b"16-byte aligned"),
    ((_A, _A, None, 1, 131072, _A, 2048, _A, _A, None), b"static scratch"),
])
def test_static_validation_before_launch(args, msg):
    static = _lib.load_static()
    assert static.ab_ibcs_sip_static(*args) == 1
    err = _lib.load().ab_last_error()
    assert msg in err and err.startswith(b"ibcs_sip_static:"), err
