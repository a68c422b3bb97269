"""Weighted paged sparse prefill on gfx950.

``paged_attention`` keeps the reference's signature, validation (ValueError)
and output/LSE layout (ab_attention/flashinfer_backend.py:164-242). The
arithmetic is ``ab_paged_prefill_kv`` in libab_attention_hip.so: a bf16 MFMA
flash-attention kernel that reads each row's KV4 blocks straight from K and
V by their per-head ids and adds the SIP weight of each block to its logits
(the reference's ABSipAttention variant, flashinfer_backend.py:30-59).
``_prefill_dense`` runs the library's dense attention kernel, which walks
every KV4 block of K/V at weight 0 with no page list in memory
(ab_dense_prefill; the same rings and pipeline on 16x16x32 MFMA tiles).

The reference translates per-head ids into a global page table and caches it
per descriptor (flashinfer_backend.py:62-74, :202-217); the kernel here
indexes K/V by (head, id) directly, so there is no table and no cache to keep
coherent. Queries are not padded either: the tail of the last query block is
simply not stored (the reference computes it on zero-padded queries and drops
it, flashinfer_backend.py:77-91, :236-242).
"""
from __future__ import annotations

import math

import torch

from . import _lib

_HEAD_DIM = 128
_QUERY_BLOCK = 128
_PAGE_SIZE = 4


def _prefill(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, ids: torch.Tensor, weights: torch.Tensor,
             order: torch.Tensor | None, return_lse: bool):
    """The weighted prefill of row-major q, k, v: ab_paged_prefill_kv, or
    ab_paged_prefill_ordered when a query token order is given; ids/weights
    [rows, S]. Shapes are checked by the callers."""
    batch, heads, tokens, _ = q.shape
    q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
    ids = ids.to(torch.int32).contiguous()
    weights = weights.to(torch.float32).contiguous()
    output = torch.empty_like(q)
    lse = torch.empty((batch, heads, tokens), dtype=torch.float32, device=q.device) if return_lse else None
    lib = _lib.load()
    with torch.cuda.device(q.device):
        if order is None:
            rc = lib.ab_paged_prefill_kv(
                _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), batch * heads, tokens, k.shape[2], _lib.ptr(ids),
                _lib.ptr(weights), ids.shape[-1], _lib.ptr(output), _lib.ptr(lse), _lib.stream(q.device))
        else:
            rc = lib.ab_paged_prefill_ordered(
                _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(order), batch * heads, tokens, _lib.ptr(ids),
                _lib.ptr(weights), ids.shape[-1], _lib.ptr(output), _lib.ptr(lse), _lib.stream(q.device))
        _lib.check(rc)
    return (output, lse) if return_lse else output


def check_prefill_inputs(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> None:
    """paged_attention's Q/K/V checks (reference: flashinfer_backend.py:176-186)."""
    if q.ndim != 4 or q.shape != k.shape or q.shape != v.shape:
        raise ValueError("Q/K/V must have the same [B,H,N,D] shape")
    if q.device != k.device or q.device != v.device:
        raise ValueError("Q/K/V must be on the same CUDA device")
    if q.device.type != "cuda":
        raise ValueError("paged attention requires GPU tensors")
    if q.dtype != torch.bfloat16 or k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError("paged attention requires BF16 Q/K/V")
    if q.shape[-1] != _HEAD_DIM or q.shape[2] % _PAGE_SIZE:
        raise ValueError("paged attention requires head_dim=128 and N divisible by 4")


@torch.no_grad()
def paged_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    descriptor: torch.Tensor,
    log_weights: torch.Tensor,
    *,
    return_lse: bool = False,
):
    """Weighted sparse attention over the plan's KV4 blocks; returns o (and base-2 lse)."""
    check_prefill_inputs(q, k, v)
    batch, heads, tokens, dim = q.shape
    batch_heads = batch * heads
    rows = batch_heads * math.ceil(tokens / _QUERY_BLOCK)
    if (descriptor.ndim != 3 or descriptor.shape != log_weights.shape
            or descriptor.shape[0] != rows or descriptor.shape[-1] != 32):
        raise ValueError(f"descriptor and log_weights must share [{rows}, pages, 32] shape")
    if descriptor.device != q.device or log_weights.device != q.device:
        raise ValueError("descriptor and log_weights must be on the Q device")

    samples = descriptor.shape[1] * 32
    return _prefill(q, k, v, descriptor.reshape(rows, samples), log_weights.reshape(rows, samples), None,
                    return_lse)


def _prefill_kv(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, ids: torch.Tensor, weights: torch.Tensor,
                *, return_lse: bool = False):
    """The weighted prefill with K/V of their own length.

    q bf16 [B,H,Nq,128], k/v bf16 [B,H,Nk,128] with Nk % 4 == 0, ids int32 /
    weights f32 [B*H*ceil(Nq/128), S] with S % 8 == 0 (per-head KV4 ids; a -inf
    weight removes its block). Shapes are checked by the callers.
    """
    return _prefill(q, k, v, ids, weights, None, return_lse)


def _prefill_dense(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, return_lse: bool = False):
    """Dense attention of q bf16 [B,H,Nq,128] over every key of k/v bf16
    [B,H,Nk,128] (Nk % 4 == 0) on the dense kernel (ab_dense_prefill); the
    page list is implicit, so nothing of size rows x blocks is built. Shapes
    are checked by the callers."""
    batch, heads, tokens, _ = q.shape
    q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
    output = torch.empty_like(q)
    lse = torch.empty((batch, heads, tokens), dtype=torch.float32, device=q.device) if return_lse else None
    lib = _lib.load()
    with torch.cuda.device(q.device):
        _lib.check(lib.ab_dense_prefill(_lib.ptr(q), _lib.ptr(k), _lib.ptr(v), batch * heads, tokens, k.shape[2],
                                        _lib.ptr(output), _lib.ptr(lse), _lib.stream(q.device)))
    return (output, lse) if return_lse else output


def _remap_ids(ids: torch.Tensor, page_map: torch.Tensor) -> torch.Tensor:
    """int32 ids -> page_map[ids] (ab_remap_ids; ids clamped into the map)."""
    ids = ids.to(torch.int32).contiguous()
    out = torch.empty_like(ids)
    lib = _lib.load()
    with torch.cuda.device(ids.device):
        _lib.check(lib.ab_remap_ids(_lib.ptr(ids), ids.numel(), _lib.ptr(page_map), page_map.numel(),
                                    _lib.ptr(out), _lib.stream(ids.device)))
    return out


def _prefill_ordered(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, order: torch.Tensor, ids: torch.Tensor,
                     weights: torch.Tensor, *, return_lse: bool = False):
    """The weighted prefill of the token-permuted q (query t is stored row
    order[t]) over stored-order k/v pages; output and lse in stored order.
    Shapes are checked by the callers."""
    return _prefill(q, k, v, ids, weights, order.to(torch.int32).contiguous(), return_lse)
