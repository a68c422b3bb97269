"""Video-layout helpers of the attention path.

``cube_layout_order`` is the token permutation of the reference's
``use_cube_layout`` (ab_attention/video.py:90-126, order math :97-105): video
tokens grouped into 4x4x4 spatiotemporal cubes, cubes in (t, h, w) order,
tokens inside a cube in (t, h, w) order, and boundary cubes holding only their
valid tokens. The attention call itself sees ordinary [B, H, N, 128] tensors
in cube order, so the kernels need nothing special for it.
"""
from __future__ import annotations

import torch


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
