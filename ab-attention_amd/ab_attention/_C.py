"""Native ops with the reference's ``ab_attention._C`` interface.

``ibcs(q, k) -> scores`` and ``sip(scores, offsets, ids, logs)`` keep the
argument meaning and the checks of the reference's pybind module
(csrc/bindings.cpp:3-8, csrc/ops.h:5-8); failed checks raise RuntimeError as
TORCH_CHECK does (csrc/ibcs.cu:550-568, csrc/sip.cu:172-192). Both run on the
current stream of the tensors' device through ``libab_attention_hip.so``.
"""
from __future__ import annotations

import torch

from . import _lib

HEAD_DIM = 128
QUERY_BLOCK = 128
KV_BLOCK = 4
MAX_KV_BLOCKS = 32768


def _require(cond: bool, message: str) -> None:
    if not cond:
        raise RuntimeError(message)


def ibcs(q: torch.Tensor, k: torch.Tensor) -> torch.Tensor:
    """IBCS block masses for q, k [batch, heads, tokens, 128] bf16 (csrc/ibcs.cu:549-617).

    Returns float32 scores [batch*heads*ceil(tokens/128), tokens/4]; each row
    is the population-weighted centroid-softmax mass of every KV4 block.
    """
    _require(q.is_cuda and k.is_cuda, "q and k must be CUDA tensors")
    _require(q.device == k.device, "q and k must use the same CUDA device")
    _require(q.is_contiguous() and k.is_contiguous(), "q and k must be contiguous")
    _require(q.shape == k.shape and q.dim() == 4,
             "q and k must have matching [batch, heads, tokens, 128] shapes")
    _require(q.dtype == torch.bfloat16 and k.dtype == torch.bfloat16, "IBCS requires bfloat16 q/k")
    _require(q.shape[3] == HEAD_DIM, "IBCS requires head_dim=128")
    _require(q.shape[2] % KV_BLOCK == 0, "sequence length must be divisible by 4")
    batch, heads, tokens, _ = q.shape
    fine_blocks = tokens // KV_BLOCK
    _require(0 < fine_blocks <= MAX_KV_BLOCKS, "KV4 block count must be in [1, 32768]")
    batch_heads = batch * heads
    rows = batch_heads * -(-tokens // QUERY_BLOCK)
    lib = _lib.load()
    with torch.cuda.device(q.device):
        ws_bytes = lib.ab_ibcs_workspace_bytes(batch_heads, tokens)
        workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device)
        scores = torch.empty((rows, fine_blocks), dtype=torch.float32, device=q.device)
        _lib.check(lib.ab_ibcs(_lib.ptr(q), _lib.ptr(k), batch_heads, tokens, _lib.ptr(workspace),
                               ws_bytes, _lib.ptr(scores), _lib.stream(q.device)))
    return scores


def ibcs_ordered(q: torch.Tensor, k: torch.Tensor, order: torch.Tensor) -> torch.Tensor:
    """ibcs of q, k with their tokens taken in the order ``order`` (int32 [tokens],
    a permutation: position t is stored token order[t]), without permuting them.
    Same checks and result layout as ``ibcs`` of the permuted tensors."""
    _require(q.is_contiguous() and k.is_contiguous(), "q and k must be contiguous")
    _require(q.is_cuda and k.is_cuda, "q and k must be CUDA tensors")
    _require(order.dtype == torch.int32 and order.is_contiguous() and order.device == q.device
             and order.shape == (q.shape[2],), "order must be int32 [tokens] on the q device")
    batch, heads, tokens = q.shape[0], q.shape[1], q.shape[2]
    batch_heads = batch * heads
    rows = batch_heads * -(-tokens // QUERY_BLOCK)
    lib = _lib.load()
    with torch.cuda.device(q.device):
        ws_bytes = lib.ab_ibcs_workspace_bytes(batch_heads, tokens)
        workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device)
        scores = torch.empty((rows, tokens // KV_BLOCK), dtype=torch.float32, device=q.device)
        _lib.check(lib.ab_ibcs_ordered(_lib.ptr(q), _lib.ptr(k), _lib.ptr(order), batch_heads, tokens,
                                       _lib.ptr(workspace), ws_bytes, _lib.ptr(scores), _lib.stream(q.device)))
    return scores


def sip(scores: torch.Tensor, offsets: torch.Tensor, ids: torch.Tensor, logs: torch.Tensor) -> None:
    """SIP sampling into the caller's ``ids``/``logs`` slices (csrc/sip.cu:170-199)."""
    _require(scores.is_cuda and offsets.device == scores.device and ids.device == scores.device
             and logs.device == scores.device, "all SIP tensors must share a CUDA device")
    _require(scores.dtype == torch.float32 and offsets.dtype == torch.float32
             and ids.dtype == torch.int32 and logs.dtype == torch.float32,
             "SIP requires float32 scores/offsets/weights and int32 ids")
    _require(scores.dim() == 2 and offsets.dim() == 1 and ids.dim() == 2 and ids.shape == logs.shape,
             "expected scores [rows,N], offsets [rows], ids/weights [rows,samples]")
    _require(scores.is_contiguous() and offsets.is_contiguous() and ids.is_contiguous()
             and logs.is_contiguous(), "SIP tensors must be contiguous")
    _require(scores.shape[0] == offsets.shape[0] and scores.shape[0] == ids.shape[0],
             "row counts must agree")
    samples = ids.shape[1]
    _require(0 < samples < scores.shape[1], "sample count must be inside the population")
    lib = _lib.load()
    with torch.cuda.device(scores.device):
        _lib.check(lib.ab_sip(_lib.ptr(scores), _lib.ptr(offsets), scores.shape[0], scores.shape[1],
                              samples, _lib.ptr(ids), _lib.ptr(logs), _lib.stream(scores.device)))


def ibcs_sip(q: torch.Tensor, k: torch.Tensor, offsets: torch.Tensor, ids: torch.Tensor, logs: torch.Tensor,
             order: torch.Tensor | None = None) -> None:
    """``sip(ibcs(q, k), offsets, ids, logs)`` in one native call (ab_ibcs_sip).

    The same ids and weights bit for bit, without materialising the scores:
    one kernel computes each row's masses into LDS and samples the row. With
    ``order`` (int32 [tokens]) the tokens are read through that permutation,
    as ``ibcs_ordered``. This is build_plan's per-chunk work
    (reference: attention.py:65-75).
    """
    _require(q.is_cuda and k.is_cuda, "q and k must be CUDA tensors")
    _require(q.device == k.device, "q and k must use the same CUDA device")
    _require(q.is_contiguous() and k.is_contiguous(), "q and k must be contiguous")
    _require(q.shape == k.shape and q.dim() == 4,
             "q and k must have matching [batch, heads, tokens, 128] shapes")
    _require(q.dtype == torch.bfloat16 and k.dtype == torch.bfloat16, "IBCS requires bfloat16 q/k")
    _require(q.shape[3] == HEAD_DIM, "IBCS requires head_dim=128")
    _require(q.shape[2] % KV_BLOCK == 0, "sequence length must be divisible by 4")
    batch, heads, tokens, _ = q.shape
    fine_blocks = tokens // KV_BLOCK
    _require(0 < fine_blocks <= MAX_KV_BLOCKS, "KV4 block count must be in [1, 32768]")
    batch_heads = batch * heads
    rows = batch_heads * -(-tokens // QUERY_BLOCK)
    _require(offsets.dtype == torch.float32 and ids.dtype == torch.int32 and logs.dtype == torch.float32,
             "SIP requires float32 offsets/weights and int32 ids")
    _require(offsets.shape == (rows,) and ids.dim() == 2 and ids.shape == logs.shape and ids.shape[0] == rows,
             "expected offsets [rows], ids/weights [rows,samples]")
    _require(all(t.device == q.device and t.is_contiguous() for t in (offsets, ids, logs)),
             "SIP tensors must be contiguous and on the q device")
    samples = ids.shape[1]
    _require(0 < samples < fine_blocks, "sample count must be inside the population")
    if order is not None:
        _require(order.dtype == torch.int32 and order.is_contiguous() and order.device == q.device
                 and order.shape == (tokens,), "order must be int32 [tokens] on the q device")
    lib = _lib.load()
    with torch.cuda.device(q.device):
        ws_bytes = lib.ab_ibcs_sip_workspace_bytes(batch_heads, tokens)
        workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device)
        _lib.check(lib.ab_ibcs_sip(_lib.ptr(q), _lib.ptr(k), _lib.ptr(order), batch_heads, tokens,
                                   _lib.ptr(offsets), samples, _lib.ptr(workspace), ws_bytes, _lib.ptr(ids),
                                   _lib.ptr(logs), _lib.stream(q.device)))
