"""The C-ABI library loads without a GPU and exports exactly what
include/ab_attention.h declares; its host-side validation answers without
touching the device."""
import ctypes
import os
import re

import pytest

from ab_attention import _lib

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "ab_attention.h")


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ab_\w+)\s*\(", text)))


def test_every_declared_symbol_is_exported():
    lib = _lib.load()
    names = _declared()
    assert len(names) >= 9
    for name in names:
        assert hasattr(lib, name), name
    assert sorted(_lib.SIGNATURES) == names


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
