"""Video integration of the attention path: the cube token layout, exact
(dense) attention, attention-state merging, the per-layer plan schedule and
HunyuanVideo's text/video partition.

``cube_layout_order`` is the token permutation of the reference's
``use_cube_layout`` (ab_attention/video.py:90-126, order math :97-105): video
tokens grouped into 4x4x4 spatiotemporal cubes, cubes in (t, h, w) order,
tokens inside a cube in (t, h, w) order, and boundary cubes holding only their
valid tokens. The attention call itself sees ordinary [B, H, N, 128] tensors
in cube order, so the kernels need nothing special for it.

``exact_attention`` and ``merge_states`` stand for the reference's ``_exact``
(FA3 dense prefill with base-2 LSE, video.py:13-28) and ``_merge``
(FlashInfer merge_state, video.py:31-40); both run on this library's kernels.
``VideoAttention`` is the reference's denoising schedule (video.py:53-87) with
the plans kept on the GPU, or in pinned host memory (``offload=True``) as the
reference keeps them. ``hunyuan_attention`` is ``_hunyuan_attention``
(video.py:129-151): by default the video queries attend to their sampled pages
and to every text block (weight 0) in one prefill, which equals the
reference's sampled state merged with the exact text state.
"""
from __future__ import annotations

import math

import torch

from . import _lib
from .attention import SamplePlan, apply_plan, build_plan
from .paged import _prefill_dense, _prefill_kv, _prefill_ordered, _remap_ids

_QUERY_BLOCK = 128
_PAGE = 4


def cube_layout_order(num_frames: int, height: int, width: int):
    """(order, inverse) int64 permutations for a video of the given pixel size.

    The latent grid is (1 + (num_frames - 1) // 4, height // 16, width // 16),
    as in the reference. ``x.index_select(token_dim, order)`` moves raster
    tokens into cube order and ``index_select(token_dim, inverse)`` undoes it.
    """
    return cube_order((1 + (num_frames - 1) // 4, height // 16, width // 16))


def cube_order(grid):
    """(order, inverse) for a latent grid (T, H, W) in row-major token order.

    Tokens are sorted by the key (cube t, cube h, cube w, t % 4, h % 4, w % 4),
    which is unique per token; partial cubes at the grid edges keep only their
    real tokens.
    """
    t, h, w = (int(s) for s in grid)
    tt, hh, ww = torch.meshgrid(torch.arange(t), torch.arange(h), torch.arange(w), indexing="ij")
    cubes_h, cubes_w = -(-h // 4), -(-w // 4)
    cube = ((tt // 4) * cubes_h + hh // 4) * cubes_w + ww // 4
    inner = ((tt % 4) * 4 + hh % 4) * 4 + ww % 4
    order = torch.argsort((cube * 64 + inner).reshape(-1))
    return order, torch.argsort(order)


_CUBE_MAPS = {}


def _cube_maps(grid, device):
    """(order, page_map) of a latent grid (T, H, W) on ``device``, cached:
    order int32 [T*H*W] (cube position t is stored token order[t]) and
    page_map int32 [T*H*W/4] (cube-order KV4 block j is stored block
    page_map[j]). Every cube-order KV4 block must be 4 consecutive stored
    tokens starting at a multiple of 4, which holds when W % 4 == 0."""
    key = (tuple(int(s) for s in grid), str(device))
    if key not in _CUBE_MAPS:
        order, _ = cube_order(grid)
        if order.numel() % _PAGE:
            raise ValueError("the cube layout needs T*H*W divisible by 4")
        quads = order.reshape(-1, _PAGE)
        if not bool(torch.all(quads == quads[:, :1] + torch.arange(_PAGE))) or not bool(torch.all(quads[:, 0] % _PAGE == 0)):
            raise ValueError("the cube layout's KV4 blocks must be 4 consecutive stored tokens (latent width % 4 == 0)")
        _CUBE_MAPS[key] = (order.to(torch.int32).to(device), (quads[:, 0] // _PAGE).to(torch.int32).to(device))
    return _CUBE_MAPS[key]


def _check_cube(q: torch.Tensor, grid):
    t, h, w = (int(s) for s in grid)
    if q.ndim != 4 or q.shape[2] != t * h * w:
        raise ValueError("the cube layout needs [B,H,N,128] tensors with N = T*H*W of the latent grid")


@torch.no_grad()
def cube_plan(q: torch.Tensor, k: torch.Tensor, grid, *, sample_pages: int = 64, seed: int = 42) -> SamplePlan:
    """build_plan in the cube token layout (reference: use_cube_layout,
    video.py:90-126, which runs attention on cube-ordered tensors) for q, k
    kept in their stored (raster) order: equal to build_plan(q[:, :, order],
    k[:, :, order], ...) with ``order`` from cube_order(grid), without
    permuting q or k. The plan's ids are cube-order KV4 blocks."""
    from .attention import _build_plan

    _check_cube(q, grid)
    order, _ = _cube_maps(grid, q.device)
    return _build_plan(q, k, sample_pages, seed, order)


@torch.no_grad()
def apply_cube_plan(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, plan: SamplePlan, grid, *,
                    return_lse: bool = False):
    """apply_plan in the cube token layout on stored-order q, k, v: equal to
    apply_plan on the cube-ordered tensors with the output (and lse) scattered
    back to stored order. K/V pages are read in place (cube-order ids are
    remapped to stored pages) and queries are gathered and scattered by the
    prefill, so nothing is permuted in memory."""
    from .paged import check_prefill_inputs

    check_prefill_inputs(q, k, v)
    _check_cube(q, grid)
    batch, heads, tokens, _ = q.shape
    rows = batch * heads * math.ceil(tokens / _QUERY_BLOCK)
    descriptor, log_weights = plan
    if descriptor.ndim != 3 or descriptor.shape != log_weights.shape or descriptor.shape[0] != rows \
            or descriptor.shape[-1] != 32:
        raise ValueError(f"descriptor and log_weights must share [{rows}, pages, 32] shape")
    order, page_map = _cube_maps(grid, q.device)
    ids = _remap_ids(descriptor.reshape(rows, -1), page_map)
    return _prefill_ordered(q, k, v, order, ids, log_weights.reshape(rows, -1), return_lse=return_lse)


@torch.no_grad()
def cube_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, grid, *, sample_pages: int = 64,
                   seed: int = 42) -> torch.Tensor:
    """ab_attention in the cube token layout on stored-order tensors; the
    output is in stored order (the reference gathers the hidden states into
    cube order once and scatters them back after the last block,
    video.py:90-126)."""
    return apply_cube_plan(q, k, v, cube_plan(q, k, grid, sample_pages=sample_pages, seed=seed), grid)


def _check_qkv(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor):
    if q.ndim != 4 or k.ndim != 4 or k.shape != v.shape or q.shape[:2] != k.shape[:2]:
        raise ValueError("Q [B,H,Nq,128] and K/V [B,H,Nk,128] must share batch and heads")
    if q.shape[-1] != 128 or k.shape[-1] != 128:
        raise ValueError("attention requires head_dim=128")
    if q.device.type != "cuda" or k.device != q.device or v.device != q.device:
        raise ValueError("Q/K/V must be on the same CUDA device")
    if q.dtype != torch.bfloat16 or k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError("attention requires BF16 Q/K/V")
    if k.shape[2] % _PAGE:
        raise ValueError("the key/value length must be divisible by 4")


def _dense_pages(rows: int, blocks: int, device, offset: int = 0):
    """ids/weights listing KV4 blocks offset .. offset+blocks-1 at weight 0 for
    every row, padded to a multiple of 8 with -inf-weight repeats of the first."""
    samples = -(-blocks // 8) * 8
    ids = torch.full((samples,), offset, dtype=torch.int32, device=device)
    ids[:blocks] = torch.arange(offset, offset + blocks, dtype=torch.int32, device=device)
    weights = torch.full((samples,), float("-inf"), dtype=torch.float32, device=device)
    weights[:blocks] = 0.0
    return ids.expand(rows, samples).contiguous(), weights.expand(rows, samples).contiguous()


@torch.no_grad()
def exact_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, return_lse: bool = False):
    """Dense non-causal attention of q [B,H,Nq,128] over k/v [B,H,Nk,128]
    (bf16, Nk divisible by 4); returns o bf16 [B,H,Nq,128] (and the base-2
    lse f32 [B,H,Nq]). The reference's _exact (video.py:13-28) on this
    library's dense kernel, which walks every KV4 block of K/V at weight 0
    with no page list in memory (ab_dense_prefill)."""
    _check_qkv(q, k, v)
    return _prefill_dense(q, k, v, return_lse=return_lse)


@torch.no_grad()
def merge_states(state_a, state_b, *, return_lse: bool = False):
    """Merge two attention states over disjoint key sets: (o bf16 [B,H,N,128],
    lse f32 [B,H,N] base 2) each. Returns the merged o (and lse). The
    reference's _merge (video.py:31-40, FlashInfer merge_state)."""
    (o_a, s_a), (o_b, s_b) = state_a, state_b
    if o_a.shape != o_b.shape or o_a.shape[-1] != 128 or s_a.shape != o_a.shape[:-1] or s_b.shape != s_a.shape:
        raise ValueError("states must be o [..., 128] with lse [...] of matching shapes")
    if o_a.dtype != torch.bfloat16 or o_b.dtype != o_a.dtype:
        raise ValueError("merge_states requires BF16 outputs")
    if o_a.device.type != "cuda" or o_b.device != o_a.device or s_a.device != o_a.device or s_b.device != o_a.device:
        raise ValueError("states must be on the same CUDA device")
    o_a, o_b = o_a.contiguous(), o_b.contiguous()
    s_a, s_b = s_a.to(torch.float32).contiguous(), s_b.to(torch.float32).contiguous()
    out = torch.empty_like(o_a)
    lse = torch.empty_like(s_a) if return_lse else None
    lib = _lib.load()
    with torch.cuda.device(o_a.device):
        _lib.check(lib.ab_merge_states(_lib.ptr(o_a), _lib.ptr(s_a), _lib.ptr(o_b), _lib.ptr(s_b), s_a.numel(),
                                       _lib.ptr(out), _lib.ptr(lse), _lib.stream(o_a.device)))
    return (out, lse) if return_lse else out


def compact_plan(plan: SamplePlan) -> SamplePlan:
    """The plan with int16 block ids: exact, since a head has at most 32,768
    KV4 blocks (ids 0..32,767), and 6 bytes per entry instead of 8. The
    weights stay float32. ``expand_plan`` restores the int32 plan."""
    return SamplePlan(plan.descriptor.to(torch.int16), plan.log_weights)


def expand_plan(plan: SamplePlan, device=None) -> SamplePlan:
    """A plan from ``compact_plan`` (on any device) as the int32 plan
    ``apply_plan`` takes, on ``device`` (default: where it is)."""
    device = plan.descriptor.device if device is None else device
    return SamplePlan(plan.descriptor.to(device, non_blocking=True).to(torch.int32),
                      plan.log_weights.to(device, non_blocking=True))


def _store_plan(plan: SamplePlan, previous) -> SamplePlan:
    """Copy a plan into pinned host memory, reusing the previous buffers
    (reference: _store_plan, video.py:43-50)."""
    if previous is None or previous.descriptor.shape != plan.descriptor.shape \
            or previous.descriptor.dtype != plan.descriptor.dtype:
        previous = SamplePlan(*(torch.empty(t.shape, dtype=t.dtype, pin_memory=True) for t in plan))
    for storage, tensor in zip(previous, plan):
        storage.copy_(tensor)
    return previous


class VideoAttention:
    """One pipeline's denoising schedule and per-layer sample plans
    (reference: video.py:53-87). Steps 1-10 and layer 0 stay dense; other
    layers build a plan on steps 11, 15, ..., and reuse it in between.

    By default the plans stay on the GPU (two [rows, pages, 32] tensors per
    layer: 774 MB per layer at Wan2.1-14B 720p with B=2, which 288 GB of
    HBM holds for every layer). With ``offload=True`` they are kept in
    pinned host memory and copied back on each reuse, as the reference does
    for GPUs that cannot hold them. ``compact=True`` stores them with int16
    ids (``compact_plan``): the same plans in 3/4 of the memory and of the
    copy traffic.
    """

    def __init__(self, sample_pages: int, *, dense: bool = False, offload: bool = False,
                 compact: bool = False):
        self.sample_pages = sample_pages
        self.dense = dense
        self.offload = offload
        self.compact = compact
        self.reset()

    def reset(self):
        self.step = 1
        self.plans = {}

    def step_end(self, pipe, index, timestep, callback_kwargs):
        self.step = index + 2  # the pipeline counts from 0, the schedule from 1
        return callback_kwargs

    def is_sparse(self, layer: int) -> bool:
        return not self.dense and self.step > 10 and layer > 0

    def plan(self, layer: int, q: torch.Tensor, k: torch.Tensor) -> SamplePlan:
        """The layer's plan for the current step: built at each anchor step
        (seed 42 + layer*1000003 + anchor*97, as the reference), else reused."""
        anchor = 11 + (self.step - 11) // 4 * 4
        stored_anchor, stored = self.plans.get(layer, (None, None))
        stale = stored_anchor != anchor or (not self.offload and stored.descriptor.device != q.device)
        if stale:
            seed = 42 + layer * 1_000_003 + anchor * 97
            plan = build_plan(q, k, sample_pages=self.sample_pages, seed=seed)
            kept = compact_plan(plan) if self.compact else plan
            self.plans[layer] = (anchor, _store_plan(kept, stored) if self.offload else kept)
            return plan
        if self.compact:
            return expand_plan(stored, q.device)
        if self.offload:
            return SamplePlan(*(t.to(q.device, non_blocking=True) for t in stored))
        return stored

    def attend(self, layer: int, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, return_lse: bool = False):
        return apply_plan(q, k, v, self.plan(layer, q, k), return_lse=return_lse)


@torch.no_grad()
def hunyuan_attention(schedule: VideoAttention, layer: int, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                      video_tokens: int, prompt_tokens: int, *, fused: bool = True) -> torch.Tensor:
    """HunyuanVideo attention over [video | prompt | padding] tokens
    (reference: _hunyuan_attention, video.py:129-151). On sparse steps video
    queries use the sampled plan over video keys plus every prompt key; prompt
    queries attend densely to video and prompt keys; padding tokens attend
    among themselves. With ``fused`` (default) the video queries' sampled and
    prompt parts run as one prefill (the prompt blocks listed at weight 0);
    otherwise as the reference: sampled state, exact prompt state, merge."""
    _check_qkv(q, k, v)
    if q.shape != k.shape:
        raise ValueError("Q/K/V must have the same [B,H,N,D] shape")
    tokens = q.shape[2]
    prompt_end = video_tokens + prompt_tokens
    if video_tokens % _PAGE or prompt_tokens % _PAGE or (tokens - prompt_end) % _PAGE or prompt_end > tokens:
        raise ValueError("video, prompt and padding lengths must be divisible by 4 and fit in N")
    if not schedule.is_sparse(layer):
        outputs = [exact_attention(q[:, :, :prompt_end], k[:, :, :prompt_end], v[:, :, :prompt_end])]
    else:
        q_video = q[:, :, :video_tokens].contiguous()
        k_video = k[:, :, :video_tokens].contiguous()
        k_prompt, v_prompt = k[:, :, :prompt_end].contiguous(), v[:, :, :prompt_end].contiguous()
        if fused:
            plan = schedule.plan(layer, q_video, k_video)
            rows = plan.descriptor.shape[0]
            text_ids, text_w = _dense_pages(rows, prompt_tokens // _PAGE, q.device, offset=video_tokens // _PAGE)
            ids = torch.cat([plan.descriptor.reshape(rows, -1), text_ids], dim=1)
            weights = torch.cat([plan.log_weights.reshape(rows, -1), text_w], dim=1)
            video_out = _prefill_kv(q_video, k_prompt, v_prompt, ids, weights)
        else:
            video_state = schedule.attend(layer, q_video, k_video, v[:, :, :video_tokens].contiguous(),
                                          return_lse=True)
            text_state = exact_attention(q_video, k[:, :, video_tokens:prompt_end], v[:, :, video_tokens:prompt_end],
                                         return_lse=True)
            video_out = merge_states(video_state, text_state)
        outputs = [video_out, exact_attention(q[:, :, video_tokens:prompt_end], k_prompt, v_prompt)]
    if prompt_end < tokens:
        outputs.append(exact_attention(q[:, :, prompt_end:], k[:, :, prompt_end:], v[:, :, prompt_end:]))
    return torch.cat(outputs, dim=2)
