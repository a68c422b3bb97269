"""Seeded input generator and the cube-layout permutation (CPU)."""
import itertools

import pytest

import torch

from ab_attention.synthetic import CONFIGS, make_qkv
from ab_attention.video import cube_layout_order, cube_order


def test_shapes_and_determinism():
    cfg = CONFIGS[0]
    q, k, v = make_qkv(cfg)
    assert q.shape == (1, 2, 2048, 128) and q.dtype == torch.float32
    q2, _, _ = make_qkv(cfg)
    assert torch.equal(q, q2)


def test_head_subset_is_a_slice():
    cfg = CONFIGS[0]
    q, k, v = make_qkv(cfg, dtype=torch.bfloat16)
    q1, k1, v1 = make_qkv(cfg, heads=[1], dtype=torch.bfloat16)
    assert torch.equal(q[:, 1:2], q1) and torch.equal(k[:, 1:2], k1) and torch.equal(v[:, 1:2], v1)


def test_local_structure():
    """Neighbouring tokens' keys are more similar than distant ones. The box
    filter shares 18 of 27 cells between raster neighbours, so with the 0.5
    noise the expected correlation is (18/729) / (1/27 + 1/4) ~ 0.086."""
    q, k, _ = make_qkv(CONFIGS[0])
    kk = k[0, 0]
    near = torch.nn.functional.cosine_similarity(kk[:-1], kk[1:]).mean()
    far = torch.nn.functional.cosine_similarity(kk[:-700], kk[700:]).mean()  # no filter overlap
    assert near > far + 0.05 and abs(far) < 0.03


def _cube_order_bruteforce(t, h, w):
    order = []
    for ct, ch, cw in itertools.product(range(-(-t // 4)), range(-(-h // 4)), range(-(-w // 4))):
        for it, ih, iw in itertools.product(range(4), range(4), range(4)):
            tt, hh, ww = 4 * ct + it, 4 * ch + ih, 4 * cw + iw
            if tt < t and hh < h and ww < w:
                order.append((tt * h + hh) * w + ww)
    return torch.tensor(order)


def test_cube_order_matches_bruteforce():
    for grid in [(4, 16, 32), (5, 6, 7), (21, 45, 80)]:
        order, inverse = cube_order(grid)
        assert torch.equal(order, _cube_order_bruteforce(*grid))
        assert torch.equal(order[inverse], torch.arange(len(order)))


def test_cube_layout_order_pixel_shape():
    order, _ = cube_layout_order(num_frames=81, height=720, width=1280)
    assert len(order) == 21 * 45 * 80


def test_cube_page_map():
    """Every cube-order KV4 block is 4 consecutive raster tokens when W % 4 == 0;
    the page map sends cube block j to raster block order[4j] / 4."""
    from ab_attention.video import _cube_maps

    for grid in [(21, 45, 80), (6, 10, 12), (5, 7, 4)]:
        order, page_map = _cube_maps(grid, "cpu")
        quads = order.reshape(-1, 4).long()
        assert torch.equal(quads, 4 * page_map.long()[:, None] + torch.arange(4))
        assert torch.equal(torch.sort(order.long()).values, torch.arange(order.numel()))
    with pytest.raises(ValueError):
        _cube_maps((4, 6, 6), "cpu")
