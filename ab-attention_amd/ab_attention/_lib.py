"""ctypes binding of the gfx950 libraries.

``libab_attention_hip.so`` carries every entry point of
``include/ab_attention.h``. ``libab_attention_static.so`` carries only
``ab_ibcs_sip_static`` (``include/ab_attention_static.h``) and its static
512 MiB device scratch; it is loaded by ``load_static()`` on first use, so a
process that never asks for it holds no such array. torch is imported first
so that the library binds to the HIP runtime torch already loaded (both carry
the soname ``libamdhip64.so.7``), which makes torch's streams valid handles
for the library. There is no fallback: if the library is missing or fails to
load, every entry point raises.
"""
from __future__ import annotations

import ctypes
import os

import torch

LIB_NAME = "libab_attention_hip.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)
STATIC_LIB_NAME = "libab_attention_static.so"
STATIC_LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), STATIC_LIB_NAME)

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_SZ = ctypes.c_size_t

# name -> (restype, argtypes); mirrors include/ab_attention.h
SIGNATURES = {
    "ab_last_error": (ctypes.c_char_p, []),
    "ab_abi_version": (ctypes.c_int, []),
    "ab_ibcs_workspace_bytes": (_SZ, [_I64, _I64]),
    "ab_ibcs": (ctypes.c_int, [_P, _P, _I64, _I64, _P, _SZ, _P, _P]),
    "ab_ibcs_lse_stride": (_I64, [_I64]),
    "ab_ibcs_cluster_pool": (ctypes.c_int, [_P, _P, _I64, _I64, _P, _P, _P, _P]),
    "ab_ibcs_lse": (ctypes.c_int, [_P, _P, _I64, _I64, _P, _P, _P, _P]),
    "ab_ibcs_masses": (ctypes.c_int, [_P, _P, _P, _P, _I64, _I64, _P, _P]),
    "ab_sip": (ctypes.c_int, [_P, _P, _I64, _I64, _I64, _P, _P, _P]),
    "ab_paged_prefill": (ctypes.c_int, [_P, _P, _P, _I64, _I64, _P, _P, _I64, _P, _P, _P]),
    "ab_paged_prefill_kv": (ctypes.c_int, [_P, _P, _P, _I64, _I64, _I64, _P, _P, _I64, _P, _P, _P]),
    "ab_merge_states": (ctypes.c_int, [_P, _P, _P, _P, _I64, _P, _P, _P]),
    "ab_ibcs_ordered": (ctypes.c_int, [_P, _P, _P, _I64, _I64, _P, _SZ, _P, _P]),
    "ab_remap_ids": (ctypes.c_int, [_P, _I64, _P, _I64, _P, _P]),
    "ab_paged_prefill_ordered": (ctypes.c_int, [_P, _P, _P, _P, _I64, _I64, _P, _P, _I64, _P, _P, _P]),
    "ab_ibcs_sip_workspace_bytes": (_SZ, [_I64, _I64]),
    "ab_ibcs_sip": (ctypes.c_int, [_P, _P, _P, _I64, _I64, _P, _I64, _P, _SZ, _P, _P, _P]),
    "ab_ibcs_sip_exact_draws": (ctypes.c_int, [_P, _P, _P, _I64, _I64, _P, _I64, _P, _SZ, _P, _P, _P]),
    "ab_dense_prefill": (ctypes.c_int, [_P, _P, _P, _I64, _I64, _I64, _P, _P, _P]),
    "ab_prefill_launch_slots": (_I64, [_I64, _I64]),
}

# name -> (restype, argtypes); mirrors include/ab_attention_static.h
STATIC_SIGNATURES = {
    "ab_ibcs_sip_static": (ctypes.c_int, [_P, _P, _P, _I64, _I64, _P, _I64, _P, _P, _P]),
}

ABI_VERSION = 4
_lib = None
_static = None


class NativeLibraryError(RuntimeError):
    """The HIP library is missing, stale or failed to load."""


def load():
    """Load (once) and return the ctypes handle with typed entry points."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise NativeLibraryError(
            f"{LIB_NAME} is not built (expected at {LIB_PATH}); run __graft_entry__.build() "
            "or `make -C ab-attention_amd/csrc`")
    try:
        handle = ctypes.CDLL(LIB_PATH)
    except OSError as exc:  # pragma: no cover - depends on the runtime
        raise NativeLibraryError(f"failed to load {LIB_PATH}: {exc}") from exc
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(handle, name)
        fn.restype = restype
        fn.argtypes = argtypes
    if handle.ab_abi_version() != ABI_VERSION:
        raise NativeLibraryError(f"{LIB_NAME} ABI {handle.ab_abi_version()} != expected {ABI_VERSION}")
    _lib = handle
    return _lib


def load_static():
    """Load (once) ``libab_attention_static.so`` after the main library and
    return its handle; its failures are reported by the main library's
    ``ab_last_error``."""
    global _static
    if _static is not None:
        return _static
    load()
    if not os.path.exists(STATIC_LIB_PATH):
        raise NativeLibraryError(
            f"{STATIC_LIB_NAME} is not built (expected at {STATIC_LIB_PATH}); run __graft_entry__.build() "
            "or `make -C ab-attention_amd/csrc`")
    try:
        handle = ctypes.CDLL(STATIC_LIB_PATH)
    except OSError as exc:  # pragma: no cover - depends on the runtime
        raise NativeLibraryError(f"failed to load {STATIC_LIB_PATH}: {exc}") from exc
    for name, (restype, argtypes) in STATIC_SIGNATURES.items():
        fn = getattr(handle, name)
        fn.restype = restype
        fn.argtypes = argtypes
    _static = handle
    return _static


def check(rc: int) -> None:
    """Raise RuntimeError (as the reference's TORCH_CHECK does) on a nonzero status."""
    if rc != 0:
        raise RuntimeError(load().ab_last_error().decode(errors="replace"))


def ptr(t: torch.Tensor | None) -> ctypes.c_void_p:
    return ctypes.c_void_p(0 if t is None else t.data_ptr())


def stream(device: torch.device) -> ctypes.c_void_p:
    """The current torch stream of ``device`` as a hipStream_t."""
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)
