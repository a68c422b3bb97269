"""AB-Attention and explicit sampling-plan reuse (MI355X build).

Same public surface as the reference's ``ab_attention/attention.py``:
``SamplePlan``, ``build_plan``, ``apply_plan`` and ``ab_attention`` with the
same arguments, defaults, validation (ValueError) and plan layout.

Differences that do not change results:
  - the IBCS scratch budget per head chunk (``LSE_BUDGET_BYTES``) defaults
    to 16 GiB, sized for 288 GB of HBM, so the Wan2.1-14B 720p call runs as
    one chunk instead of nine; rows are independent and the offsets are
    drawn before chunking, so the plan does not depend on the chunking
    (attention.py:54-75 in the reference). A caller that shares the GPU can
    lower it: set ``ab_attention.attention.LSE_BUDGET_BYTES`` or the
    environment variable ``AB_ATTENTION_LSE_BUDGET_BYTES`` (read at import);
    the reference's value is 1.5 GiB;
  - ``apply_plan`` goes to the gfx950 paged prefill in ``paged.py``.
"""
import math
import os
from typing import NamedTuple

import torch

_BUDGET_ENV = "AB_ATTENTION_LSE_BUDGET_BYTES"


def _budget_from_env(default: int) -> int:
    """The pair-LSE budget from ``AB_ATTENTION_LSE_BUDGET_BYTES`` (an integer
    or a float such as ``1.5e9``, in bytes), or ``default`` when unset."""
    raw = os.environ.get(_BUDGET_ENV)
    if raw is None or not raw.strip():
        return default
    try:
        value = float(raw)
    except ValueError:
        raise ValueError(f"{_BUDGET_ENV}={raw!r} is not a byte count (an integer or a float like 1.5e9)") from None
    if not math.isfinite(value) or value <= 0:
        raise ValueError(f"{_BUDGET_ENV}={raw!r} must be a positive, finite byte count")
    return int(value)


# Budget for the [rows, 8, ~tokens/4] fp16 pair-LSEs of one head chunk; the
# whole IBCS workspace of a chunk is about 1.07 times this (plus pooled keys
# and centroids). At least one head is processed per chunk.
LSE_BUDGET_BYTES = _budget_from_env(16 * 1024 ** 3)


class SamplePlan(NamedTuple):
    """The sampled key blocks of every 128-query block and their weights.

    ``descriptor`` holds int32 KV4-block indices counted within the block's
    own (batch, head); ``log_weights`` holds the float32 logit shift of each
    entry, log2 of its inverse inclusion probability (0 for blocks SIP kept
    with certainty). Both are [rows, pages, 32]: one row per (batch, head,
    query block) in that order, ``pages`` = ``sample_pages``, 32 blocks per
    page. ``apply_plan`` only reads them, so one plan can serve several
    calls; a new selection needs a new plan. (Reference: attention.py:11-23.)
    """

    descriptor: torch.Tensor
    log_weights: torch.Tensor


def _heads_per_chunk(batch_heads: int, q_blocks: int, tokens: int) -> int:
    lse_bytes_per_head = q_blocks * 8 * (tokens // 4) * 2
    return max(1, min(batch_heads, int(LSE_BUDGET_BYTES) // lse_bytes_per_head))


@torch.no_grad()
def build_plan(q, k, *, sample_pages=64, seed=42):
    """Choose, for every block of 128 queries, the KV4 blocks it attends to.

    Inputs: bf16 tensors of shape [batch, heads, tokens, 128] on one GPU,
    with a token count that is a multiple of 4 and larger than the
    ``128 * sample_pages`` keys kept per query block. Each query block is
    reduced to 8 centroids, each KV4 block to 2 averaged key pairs; the
    centroids' softmax over the key pairs gives every KV4 block a mass, and
    systematic sampling proportional to those masses keeps
    ``32 * sample_pages`` distinct blocks per query block. Each kept block
    carries log2 of its inverse inclusion probability, added to its logits
    when the plan is applied. The result is a ``SamplePlan`` whose two
    tensors are [rows, sample_pages, 32]. (Reference: attention.py:26-82.)
    """
    return _build_plan(q, k, sample_pages, seed)


def _build_plan(q, k, sample_pages, seed, order=None):
    """build_plan, with the tokens read through ``order`` (int32 [tokens])
    when it is given (the cube layout on stored-order tensors)."""
    sample_pages = int(sample_pages)
    if q.ndim != 4 or q.shape != k.shape or q.shape[2] % 4:
        raise ValueError("Q/K must match [B,H,N,D] with N divisible by 4")
    if sample_pages <= 0:
        raise ValueError("sample_pages must be positive")
    if sample_pages * 128 >= q.shape[2]:
        raise ValueError("sampled key count must be smaller than the sequence length")
    from . import _C as ops

    batch_heads = q.shape[0] * q.shape[1]
    tokens, dim = q.shape[2:]
    q_blocks = math.ceil(tokens / 128)
    rows, samples = batch_heads * q_blocks, sample_pages * 32

    # All offsets are drawn before chunking, so chunking cannot change the plan.
    generator = torch.Generator(device=q.device).manual_seed(seed)
    offsets = torch.rand(rows, device=q.device, generator=generator)
    flat_q = q.reshape(batch_heads, tokens, dim)
    flat_k = k.reshape(batch_heads, tokens, dim)

    heads_per_chunk = _heads_per_chunk(batch_heads, q_blocks, tokens)
    sampled = torch.empty((rows, samples), dtype=torch.int32, device=q.device)
    log_weights = torch.empty((rows, samples), dtype=torch.float32, device=q.device)

    for start in range(0, batch_heads, heads_per_chunk):
        stop = min(batch_heads, start + heads_per_chunk)
        first, last = start * q_blocks, stop * q_blocks
        # IBCS scores and SIP sampling of the chunk (the reference's _C.ibcs
        # then _C.sip) in one native call that keeps the scores on chip.
        ops.ibcs_sip(
            flat_q[start:stop].unsqueeze(0).contiguous(),
            flat_k[start:stop].unsqueeze(0).contiguous(),
            offsets[first:last], sampled[first:last], log_weights[first:last], order,
        )

    return SamplePlan(
        sampled.reshape(rows, sample_pages, 32),
        log_weights.reshape(rows, sample_pages, 32),
    )


@torch.no_grad()
def apply_plan(q, k, v, plan, *, return_lse=False):
    """Weighted sparse attention of q over each row's sampled KV4 blocks.

    A plan can be reused across denoising steps while the tensor shape and
    device stay the same. With ``return_lse`` the base-2 softmax normaliser is
    also returned as float32 [batch, heads, tokens], for merging attention
    partitions. (Reference: attention.py:85-96.)
    """
    from .paged import paged_attention

    return paged_attention(q, k, v, *plan, return_lse=return_lse)


@torch.no_grad()
def ab_attention(q, k, v, *, sample_pages=64, seed=42):
    """``build_plan`` then ``apply_plan`` in one call: sparse attention over
    a freshly sampled plan, returned in q's shape and dtype
    (reference: attention.py:99-102)."""
    return apply_plan(q, k, v, build_plan(q, k, sample_pages=sample_pages, seed=seed))
