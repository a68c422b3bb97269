"""CPU oracle for AB-Attention's selection and weighted paged prefill.

TEST INFRASTRUCTURE ONLY: imported by tests/, ``__graft_entry__.smoke()`` and
the ``cpu_baseline`` leg of ``bench.py`` as the checker. The product path
(``ab_attention``) never imports it.

The arithmetic lives in ``ab_oracle.c`` (built by ``oracle/Makefile`` into
``liboracle.so``); this module converts torch/numpy arrays and calls it. Row
loops run on OpenMP threads (``OMP_NUM_THREADS``); every row is computed by
one thread in a fixed order, so results do not depend on the thread count.
Reference call sites restated (paths relative to the reference checkout):
``csrc/ibcs.cu:106-538`` (IBCS), ``csrc/sip.cu:33-167`` (SIP),
``ab_attention/flashinfer_backend.py:30-59`` (weighted prefill).
"""
from __future__ import annotations

import ctypes
import math
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

HEAD_DIM = 128
QUERY_BLOCK = 128
KV_BLOCK = 4
CENTROIDS = 8

# float(128 ** -0.5 * log2(e)), the centroid pre-scale of csrc/ibcs.cu:601-602.
QK_SCALE_LOG2 = float(np.float32(math.pow(128.0, -0.5) * 1.4426950408889634))

_P = ctypes.c_void_p
_I64 = ctypes.c_int64


def build(force: bool = False) -> str:
    """Compile ``liboracle.so`` with the committed Makefile."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        _lib.orc_cluster.argtypes = [_P, _I64, _I64, ctypes.c_float, _P, _P]
        _lib.orc_pool.argtypes = [_P, _I64, _I64, _P]
        _lib.orc_lse.argtypes = [_P, _P, _I64, _I64, _P, _P, _P]
        _lib.orc_lse_rows.argtypes = [_P, _I64, _P, _I64, _P, _P, _P]
        _lib.orc_masses.argtypes = [_P, _P, _P, _P, _I64, _I64, _P]
        _lib.orc_ibcs.argtypes = [_P, _P, _I64, _I64, ctypes.c_float, _P]
        _lib.orc_ibcs.restype = ctypes.c_int
        _lib.orc_sip.argtypes = [_P, _P, _I64, _I64, _I64, _P, _P]
        _lib.orc_sip.restype = ctypes.c_int
        _lib.orc_prefill.argtypes = [_P, _P, _P, _I64, _I64, _P, _P, _I64, _P, _I64, _P, _P]
        _lib.orc_prefill.restype = ctypes.c_int
        _lib.orc_prefill_kv.argtypes = [_P, _P, _P, _I64, _I64, _I64, _P, _P, _I64, _P, _I64, _P, _P]
        _lib.orc_prefill_kv.restype = ctypes.c_int
        _lib.orc_f32_to_f16.argtypes = [ctypes.c_float]
        _lib.orc_f32_to_f16.restype = ctypes.c_uint16
        _lib.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
        _lib.orc_f16_to_f32.restype = ctypes.c_float
        _lib.orc_f32_to_bf16.argtypes = [ctypes.c_float]
        _lib.orc_f32_to_bf16.restype = ctypes.c_uint16
        _lib.orc_num_threads.argtypes = []
        _lib.orc_num_threads.restype = ctypes.c_int
    return _lib


def num_threads() -> int:
    """Host threads the oracle's row loops run on (OpenMP)."""
    return int(lib().orc_num_threads())


def _ptr(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.c_void_p)


def bf16_bits(x) -> np.ndarray:
    """bfloat16 torch tensor (any device) -> contiguous uint16 numpy bits."""
    import torch

    t = x.detach()
    if t.dtype != torch.bfloat16:
        t = t.to(torch.bfloat16)
    return np.ascontiguousarray(t.cpu().contiguous().view(torch.int16).numpy().view(np.uint16))


def bits_to_f32(bits: np.ndarray) -> np.ndarray:
    """uint16 bfloat16 bits -> float32 (exact)."""
    return (bits.astype(np.uint32) << 16).view(np.float32)


def _dims(bh: int, n: int):
    qb = -(-n // QUERY_BLOCK)
    return qb, n // KV_BLOCK, bh * qb


def cluster(q_bits: np.ndarray, bh: int, n: int):
    """Scaled bf16 centroids [rows, 8, 128] (uint16 bits) and populations [rows, 8]."""
    qb, fb, rows = _dims(bh, n)
    cent = np.empty((rows, CENTROIDS, HEAD_DIM), np.uint16)
    pops = np.empty((rows, CENTROIDS), np.float32)
    lib().orc_cluster(_ptr(q_bits), bh, n, QK_SCALE_LOG2, _ptr(cent), _ptr(pops))
    return cent, pops


def pool(k_bits: np.ndarray, bh: int, n: int) -> np.ndarray:
    """Pooled bf16 key pairs [bh, n/4, 2, 128] (uint16 bits)."""
    out = np.empty((bh, n // KV_BLOCK, 2, HEAD_DIM), np.uint16)
    lib().orc_pool(_ptr(k_bits), bh, n, _ptr(out))
    return out


def lse(cent: np.ndarray, pooled: np.ndarray, bh: int, n: int):
    """fp16 pair-LSE bits [rows, 8, fb] and the (max, den) normalisers [rows, 8]."""
    qb, fb, rows = _dims(bh, n)
    out = np.empty((rows, CENTROIDS, fb), np.uint16)
    mx = np.empty((rows, CENTROIDS), np.float32)
    den = np.empty((rows, CENTROIDS), np.float32)
    lib().orc_lse(_ptr(np.ascontiguousarray(cent)), _ptr(np.ascontiguousarray(pooled)), bh, n,
                  _ptr(out), _ptr(mx), _ptr(den))
    return out, mx, den


def lse_rows(cent: np.ndarray, pooled_head: np.ndarray):
    """Pair-LSEs of centroid rows [r, 8, 128] against one head's pooled keys [fb, 2, 128]."""
    cent = np.ascontiguousarray(cent)
    pooled_head = np.ascontiguousarray(pooled_head)
    rows, fb = cent.shape[0], pooled_head.shape[0]
    out = np.empty((rows, CENTROIDS, fb), np.uint16)
    mx = np.empty((rows, CENTROIDS), np.float32)
    den = np.empty((rows, CENTROIDS), np.float32)
    lib().orc_lse_rows(_ptr(cent), rows, _ptr(pooled_head), fb, _ptr(out), _ptr(mx), _ptr(den))
    return out, mx, den


def masses(lse_bits, pops, mx, den, rows: int, fb: int) -> np.ndarray:
    out = np.empty((rows, fb), np.float32)
    lib().orc_masses(_ptr(np.ascontiguousarray(lse_bits)), _ptr(np.ascontiguousarray(pops)),
                     _ptr(np.ascontiguousarray(mx)), _ptr(np.ascontiguousarray(den)), rows, fb,
                     _ptr(out))
    return out


def ibcs(q_bits: np.ndarray, k_bits: np.ndarray, bh: int, n: int) -> np.ndarray:
    """Block masses [bh*qb, n/4] float32 for bf16 q/k bits [bh, n, 128]."""
    qb, fb, rows = _dims(bh, n)
    out = np.empty((rows, fb), np.float32)
    rc = lib().orc_ibcs(_ptr(np.ascontiguousarray(q_bits)), _ptr(np.ascontiguousarray(k_bits)),
                        bh, n, QK_SCALE_LOG2, _ptr(out))
    if rc:
        raise MemoryError("oracle ibcs allocation failed")
    return out


def sip(scores: np.ndarray, offsets: np.ndarray, samples: int):
    """SIP ids [rows, samples] int32 and log2(1/pi) weights [rows, samples] float32."""
    scores = np.ascontiguousarray(scores, np.float32)
    offsets = np.ascontiguousarray(offsets, np.float32)
    rows, pop = scores.shape
    ids = np.empty((rows, samples), np.int32)
    logw = np.empty((rows, samples), np.float32)
    rc = lib().orc_sip(_ptr(scores), _ptr(offsets), rows, pop, samples, _ptr(ids), _ptr(logw))
    if rc:
        raise ValueError("sample count must be inside the population")
    return ids, logw


def prefill(q: np.ndarray, k: np.ndarray, v: np.ndarray, ids: np.ndarray, logw: np.ndarray, rows=None):
    """Exact weighted sparse attention. q float32 [bh, n, 128]; k/v float32
    [bh, n_kv, 128] (n_kv may differ from n); ids/logw [rows, S], rows = bh*ceil(n/128).

    Returns (out float32 [bh, n, 128], lse float32 [bh, n], base 2). With
    ``rows`` (row indices) only those rows' queries are computed; the other
    outputs are NaN. A -inf weight removes its block."""
    bh, n, _ = q.shape
    n_kv = k.shape[1]
    q, k, v = (np.ascontiguousarray(t, np.float32) for t in (q, k, v))
    nrows = ids.shape[0]
    ids = np.ascontiguousarray(ids.reshape(nrows, -1), np.int32)
    logw = np.ascontiguousarray(logw.reshape(nrows, -1), np.float32)
    out = np.full_like(q, np.nan)
    lse_out = np.full((bh, n), np.nan, np.float32)
    row_arr = None if rows is None else np.ascontiguousarray(rows, np.int64)
    rc = lib().orc_prefill_kv(_ptr(q), _ptr(k), _ptr(v), bh, n, n_kv, _ptr(ids), _ptr(logw), ids.shape[1],
                              None if row_arr is None else _ptr(row_arr),
                              0 if row_arr is None else len(row_arr), _ptr(out), _ptr(lse_out))
    if rc:
        raise ValueError("plan id or row outside range")
    return out, lse_out


def merge_states(o_a: np.ndarray, s_a: np.ndarray, o_b: np.ndarray, s_b: np.ndarray):
    """Merge of two attention states over disjoint key sets, base-2 LSEs, in
    float64: FlashInfer's merge_state (flashinfer-python 0.6.12, used by
    ab_attention/video.py:31-40; not vendored under the reference):
        m = max(s_a, s_b), w = 2^(s - m), o = (o_a w_a + o_b w_b) / (w_a + w_b),
        s = m + log2(w_a + w_b).
    o_*: [..., 128], s_*: [...]. Returns (o float64, s float64)."""
    s_a = np.asarray(s_a, np.float64)
    s_b = np.asarray(s_b, np.float64)
    m = np.maximum(s_a, s_b)
    w_a, w_b = np.exp2(s_a - m), np.exp2(s_b - m)
    d = w_a + w_b
    o = (np.asarray(o_a, np.float64) * w_a[..., None] + np.asarray(o_b, np.float64) * w_b[..., None]) / d[..., None]
    return o, m + np.log2(d)


def f32_to_f16_bits(x: float) -> int:
    return int(lib().orc_f32_to_f16(x))


def f16_bits_to_f32(h: int) -> float:
    return float(lib().orc_f16_to_f32(h))


def f32_to_bf16_bits(x: float) -> int:
    return int(lib().orc_f32_to_bf16(x))
