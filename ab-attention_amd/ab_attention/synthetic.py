"""Seeded synthetic self-attention inputs for the benchmark configurations.

Video tokens are in row-major (t, h, w) order. Per batch item a base field
F ~ N(0,1) over the latent grid is smoothed by a 3x3x3 box filter
(avg_pool3d, stride 1, padding 1, count_include_pad=False) and gets
0.5 * N(0,1) noise. Per head, Q = F @ Wq / sqrt(128) and K = F @ Wk / sqrt(128)
with Wq, Wk ~ N(0,1)^{128x128}, so attention is spatiotemporally local.
V ~ N(0,1). Text tokens (configuration 3) have i.i.d. N(0,1) Q/K/V and are
appended after the video tokens.

Random streams: generator(seed) draws F, the noise, then Wq and Wk for every
head; V and text tokens come from generator(seed + 1), head by head, so a
subset of heads is the same tensor slice as the full call.
"""
from __future__ import annotations

import dataclasses
import math

import torch
import torch.nn.functional as F


@dataclasses.dataclass(frozen=True)
class Config:
    name: str
    batch: int
    heads: int
    grid: tuple  # latent (T, H, W)
    sample_pages: int
    dtype: torch.dtype = torch.bfloat16
    text_tokens: int = 0
    cube_layout: bool = False
    seed: int = 0

    @property
    def video_tokens(self) -> int:
        return self.grid[0] * self.grid[1] * self.grid[2]

    @property
    def tokens(self) -> int:
        return self.video_tokens + self.text_tokens


CONFIGS = {
    0: Config("c0-cpu-plumbing", 1, 2, (4, 16, 32), 2, torch.float32, seed=1000),
    1: Config("wan2.1-1.3b-480p", 2, 12, (21, 30, 52), 64, seed=1001),
    2: Config("wan2.1-14b-720p", 2, 40, (21, 45, 80), 64, seed=1002),
    3: Config("hunyuanvideo-720p-129f", 1, 24, (33, 45, 80), 71, text_tokens=256, seed=1003),
    4: Config("wan2.1-14b-720p-cube", 2, 40, (21, 45, 80), 64, cube_layout=True, seed=1004),
}


def _gen(seed: int, device) -> torch.Generator:
    return torch.Generator(device=device).manual_seed(seed)


@torch.no_grad()
def make_qkv(cfg: Config, *, heads=None, device="cpu", dtype=None, seed=None):
    """Q, K, V of shape [batch, len(heads), tokens, 128] for the selected heads.

    ``heads`` defaults to all heads; the tensors for a head do not depend on
    which other heads are generated. Computation is float32 on ``device``; the
    result is cast to ``dtype`` (default: the configuration's dtype).
    """
    heads = list(range(cfg.heads)) if heads is None else list(heads)
    dtype = cfg.dtype if dtype is None else dtype
    seed = cfg.seed if seed is None else seed
    b, d = cfg.batch, 128
    t, h, w = cfg.grid
    n_video, n = cfg.video_tokens, cfg.tokens
    g = _gen(seed, device)
    base = torch.randn(b, d, t, h, w, generator=g, device=device)
    base = F.avg_pool3d(base, 3, stride=1, padding=1, count_include_pad=False)
    base = base + 0.5 * torch.randn(base.shape, generator=g, device=device)
    field = base.permute(0, 2, 3, 4, 1).reshape(b, n_video, d)
    wq = torch.randn(cfg.heads, d, d, generator=g, device=device)
    wk = torch.randn(cfg.heads, d, d, generator=g, device=device)
    g2 = _gen(seed + 1, device)
    q = torch.empty(b, len(heads), n, d, dtype=dtype, device=device)
    k = torch.empty_like(q)
    v = torch.empty_like(q)
    inv = 1.0 / math.sqrt(d)
    want = set(heads)
    slot = {hd: i for i, hd in enumerate(heads)}
    for hd in range(cfg.heads):
        # Every head consumes its draws so later heads see the same stream.
        vv = torch.randn(b, n_video, d, generator=g2, device=device)
        text = (torch.randn(3, b, cfg.text_tokens, d, generator=g2, device=device)
                if cfg.text_tokens else None)
        if hd not in want:
            continue
        i = slot[hd]
        q[:, i, :n_video] = (field @ wq[hd]).mul_(inv).to(dtype)
        k[:, i, :n_video] = (field @ wk[hd]).mul_(inv).to(dtype)
        v[:, i, :n_video] = vv.to(dtype)
        if text is not None:
            q[:, i, n_video:] = text[0].to(dtype)
            k[:, i, n_video:] = text[1].to(dtype)
            v[:, i, n_video:] = text[2].to(dtype)
    return q, k, v


def parity_offsets(rows: int, seed: int = 42) -> torch.Tensor:
    """Per-row uniforms for parity runs: torch.rand on a CPU generator."""
    return torch.rand(rows, generator=_gen(seed, "cpu"))
