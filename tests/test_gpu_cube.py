"""The cube token layout computed in place (GPU).

The reference's use_cube_layout (ab_attention/video.py:90-126) gathers the
hidden states into 4x4x4-cube order, so attention runs on permuted tensors.
cube_plan / apply_cube_plan / cube_attention compute the same attention on
tensors kept in raster order: Q and K tokens are read through the order,
cube-order KV4 ids are remapped to raster pages, and output rows are
scattered back. Only addressing differs, so the results must be bit-identical
to build_plan / apply_plan / ab_attention on explicitly permuted tensors
(whose own parity with the oracle is tested at c4 in test_gpu_configs.py).
"""
import pytest
import torch

from ab_attention import ab_attention, apply_plan, build_plan
from ab_attention.synthetic import CONFIGS, make_qkv
from ab_attention.video import apply_cube_plan, cube_attention, cube_order, cube_plan

pytestmark = pytest.mark.gpu


def _qkv(grid, heads, seed):
    torch.manual_seed(seed)
    n = grid[0] * grid[1] * grid[2]
    return (torch.randn(1, heads, n, 128, device="cuda").to(torch.bfloat16) for _ in range(3))


@pytest.mark.parametrize("grid,heads,pages", [((6, 10, 12), 2, 2), ((9, 14, 20), 3, 8)])
def test_cube_layout_in_place_small(grid, heads, pages):
    """Grids with partial cubes along T and H (and an odd query-block tail)."""
    print(f"cube in place grid={grid} heads={heads}", flush=True)
    q, k, v = _qkv(grid, heads, sum(grid))
    order, inverse = (t.cuda() for t in cube_order(grid))
    qc, kc, vc = (t.index_select(2, order) for t in (q, k, v))
    ref_plan = build_plan(qc, kc, sample_pages=pages, seed=3)
    plan = cube_plan(q, k, grid, sample_pages=pages, seed=3)
    assert torch.equal(plan.descriptor, ref_plan.descriptor)
    assert torch.equal(plan.log_weights.view(torch.int32), ref_plan.log_weights.view(torch.int32))
    ref_o, ref_l = apply_plan(qc, kc, vc, ref_plan, return_lse=True)
    out, lse = apply_cube_plan(q, k, v, plan, grid, return_lse=True)
    torch.cuda.synchronize()
    assert torch.equal(out, ref_o.index_select(2, inverse))
    assert torch.equal(lse, ref_l.index_select(2, inverse))


def test_cube_attention_c4_head():
    """One Wan2.1-14B 720p head (21x45x80 latent) end to end."""
    cfg = CONFIGS[4]
    print(f"cube attention c4 head, grid {cfg.grid}", flush=True)
    q, k, v = (t[:1].contiguous() for t in make_qkv(cfg, heads=[7], device="cuda", dtype=torch.bfloat16))
    order, inverse = (t.cuda() for t in cube_order(cfg.grid))
    qc, kc, vc = (t.index_select(2, order) for t in (q, k, v))
    ref = ab_attention(qc, kc, vc, sample_pages=cfg.sample_pages, seed=42).index_select(2, inverse)
    out = cube_attention(q, k, v, cfg.grid, sample_pages=cfg.sample_pages, seed=42)
    torch.cuda.synchronize()
    assert out.shape == q.shape and out.dtype == q.dtype
    assert torch.equal(out, ref)
