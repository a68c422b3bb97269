"""Whole calls of the other workloads on the GPU, checked the way the headline
call is (tests/test_gpu_c2.py::test_c2_full_call; reference:
ab_attention/attention.py:26-102, video.py:90-151):

  c1  Wan2.1-1.3B 480p: build_plan + apply_plan over B=2, H=12, 32,760 tokens
      (6,144 rows; the last query block of each head holds 120 queries);
  c3  HunyuanVideo 720p: hunyuan_attention on a sparse step over all 24 heads
      (plans over the 118,800 video tokens: 22,296 rows of 29,700 KV4 blocks,
      sampled with kept prefixes; every video row also attends to the 64
      prompt blocks, the prompt rows to every key; video rows of each of the
      fused prefill's 3 launches are compared with the oracle);
  c4  Wan2.1-14B 720p in cube layout, computed in place on the raster tensors
      (cube_plan + apply_cube_plan; plan ids are cube-order KV4 blocks).

For each: every row satisfies SIP's invariants (a row that breaks one must be
reproduced bit for bit by the oracle), 64 random rows across the heads are
bit-exact with the oracle's SIP on the GPU's scores and the call's uniforms,
the output is finite, and rows of a few heads (ragged last blocks included)
match the fp64 oracle prefill over the GPU plan: max-abs 2e-2, rel-L2 1e-2.
"""
import numpy as np
import pytest
import torch

from ab_attention import _C, apply_plan, build_plan
from ab_attention.synthetic import CONFIGS, make_qkv
from ab_attention.video import VideoAttention, apply_cube_plan, cube_order, cube_plan, hunyuan_attention
from test_gpu_c2 import _assert_sip_equal, _check_rows, _f32, _sip_invariants, check_rows_by_head, launch_check_rows

pytestmark = pytest.mark.gpu


def _plan_rows(oracle_mod, q_sel, k_sel, ids, w, fb, seed, tag):
    """SIP invariants on every row; 64 random rows (and any row that breaks
    an invariant) bit-exact with the oracle on the GPU's scores and the
    uniforms torch.rand(rows) draws from Generator(seed)."""
    rows, samples = ids.shape
    offsets = torch.rand(rows, device=ids.device, generator=torch.Generator(ids.device).manual_seed(seed))
    broken = _sip_invariants(ids, w, fb).cpu().numpy()
    print(f"{tag}: {broken.size} of {rows} rows break an invariant", flush=True)
    pick = np.sort(np.random.default_rng(5).choice(rows, size=64, replace=False))
    check = np.union1d(pick, broken)
    idx = torch.as_tensor(check, device=ids.device)
    scores = _C.ibcs(q_sel, k_sel)
    ids_o, w_o = oracle_mod.sip(scores[idx].cpu().numpy(), offsets[idx].cpu().numpy(), samples)
    del scores
    _assert_sip_equal(ids[idx].cpu().numpy(), w[idx].cpu().numpy(), ids_o, w_o)
    return pick


def test_c1_full_call(oracle_mod):
    cfg = CONFIGS[1]
    print("c1 full call: B=2 H=12 N=32,760", flush=True)
    q, k, v = make_qkv(cfg, device="cuda", dtype=torch.bfloat16)
    b, h, n, _ = q.shape
    qb, fb, samples = -(-n // 128), n // 4, cfg.sample_pages * 32
    rows, seed = b * h * qb, 42
    plan = build_plan(q, k, sample_pages=cfg.sample_pages, seed=seed)
    out = apply_plan(q, k, v, plan)
    torch.cuda.synchronize()
    assert plan.descriptor.shape == (rows, cfg.sample_pages, 32) and bool(torch.isfinite(out).all())
    ids, w = plan.descriptor.reshape(rows, samples), plan.log_weights.reshape(rows, samples)
    pick = _plan_rows(oracle_mod, q, k, ids, w, fb, seed, "c1 full call")
    assert len(np.unique(pick // qb)) > 16
    for bh_i in (0, 13, 23):
        bi, hi = divmod(bh_i, h)
        keep = np.array([0, qb // 2, qb - 1])
        head = slice(bh_i * qb, (bh_i + 1) * qb)
        ref, _ = oracle_mod.prefill(*(_f32(t[bi, hi]).reshape(1, n, 128) for t in (q, k, v)),
                                    ids[head].cpu().numpy(), w[head].cpu().numpy(), rows=keep)
        _check_rows(_f32(out[bi, hi]).reshape(n, 128), None, ref[0], None, keep, n)


def test_c3_full_call(oracle_mod):
    cfg = CONFIGS[3]
    video, prompt = cfg.video_tokens, cfg.text_tokens
    print(f"c3 full call: H=24, {video} video + {prompt} prompt tokens, P={cfg.sample_pages}", flush=True)
    q, k, v = make_qkv(cfg, device="cuda", dtype=torch.bfloat16)
    _, h, n, _ = q.shape
    sched = VideoAttention(cfg.sample_pages)
    sched.step = 11
    out = hunyuan_attention(sched, 1, q, k, v, video, prompt)
    torch.cuda.synchronize()
    assert out.shape == q.shape and bool(torch.isfinite(out).all())
    anchor, plan = sched.plans[1]
    seed = 42 + 1 * 1_000_003 + anchor * 97
    qb, fb, samples = -(-video // 128), video // 4, cfg.sample_pages * 32
    rows = h * qb
    assert plan.descriptor.shape == (rows, cfg.sample_pages, 32)
    ids, w = plan.descriptor.reshape(rows, samples), plan.log_weights.reshape(rows, samples)
    qv, kv = q[:, :, :video].contiguous(), k[:, :, :video].contiguous()
    pick = _plan_rows(oracle_mod, qv, kv, ids, w, fb, seed, "c3 full call")
    assert len(np.unique(pick // qb)) > 16
    del qv, kv
    text_ids = np.arange(video // 4, (video + prompt) // 4, dtype=np.int32)
    # Video rows over their plan plus the prompt blocks at weight 0: rows of
    # every launch of the fused prefill (3 at c3: its first and last row
    # slots and both sides of a generation boundary), and rows of heads 2
    # and 19; the prompt rows of those two heads over every key.
    per_launch = launch_check_rows(h, video)
    assert len(per_launch) == 3 and all(len(r) >= 2 for r in per_launch.values()), per_launch
    checked = [r for rs in per_launch.values() for r in rs] + [hi * qb + r for hi in (2, 19)
                                                               for r in (1, qb // 2, qb - 1)]
    checked = np.asarray(sorted(set(checked)))
    for hi in np.unique(checked // qb):
        keep = checked[checked // qb == hi] - hi * qb
        print(f"c3 full call: head {hi} rows {keep.tolist()}", flush=True)
        head = slice(hi * qb, (hi + 1) * qb)
        ids_h = np.concatenate([ids[head].cpu().numpy(), np.tile(text_ids, (qb, 1))], 1)
        w_h = np.concatenate([w[head].cpu().numpy(), np.zeros((qb, text_ids.size), np.float32)], 1)
        qf, kf, vf = (_f32(t[0, hi]).reshape(1, n, 128) for t in (q, k, v))
        ref, _ = oracle_mod.prefill(qf[:, :video], kf, vf, ids_h, w_h, rows=keep)
        got = _f32(out[0, hi]).reshape(n, 128)
        _check_rows(got[:video], None, ref[0], None, keep, video)
        if hi in (2, 19):
            all_ids = np.tile(np.arange((video + prompt) // 4, dtype=np.int32), (2, 1))
            ref_p, _ = oracle_mod.prefill(qf[:, video:], kf, vf, all_ids, np.zeros(all_ids.shape, np.float32))
            _check_rows(got[video:], None, ref_p[0], None, [0, 1], prompt)


def test_c4_full_call_in_place(oracle_mod):
    cfg = CONFIGS[4]
    print(f"c4 full call in place: B=2 H=40, grid {cfg.grid}", flush=True)
    q, k, v = make_qkv(cfg, device="cuda", dtype=torch.bfloat16)
    b, h, n, _ = q.shape
    qb, fb, samples = -(-n // 128), n // 4, cfg.sample_pages * 32
    rows, seed = b * h * qb, 42
    plan = cube_plan(q, k, cfg.grid, sample_pages=cfg.sample_pages, seed=seed)
    out = apply_cube_plan(q, k, v, plan, cfg.grid)
    torch.cuda.synchronize()
    assert plan.descriptor.shape == (rows, cfg.sample_pages, 32) and bool(torch.isfinite(out).all())
    ids, w = plan.descriptor.reshape(rows, samples), plan.log_weights.reshape(rows, samples)
    order, _ = cube_order(cfg.grid)
    order = order.cuda()
    qc, kc = q.index_select(2, order), k.index_select(2, order)
    pick = _plan_rows(oracle_mod, qc, kc, ids, w, fb, seed, "c4 full call")
    assert len(np.unique(pick // qb)) > 40
    del qc, kc
    # the oracle sees the cube-ordered tensors; the output is read back in
    # cube order. Rows of every prefill launch, and of heads 5 and 66.
    per_launch = launch_check_rows(b * h, n)
    assert len(per_launch) == 5 and all(len(r) >= 2 for r in per_launch.values()), per_launch
    extra = [bh_i * qb + r for bh_i in (5, 66) for r in (0, qb // 2, qb - 1)]
    check_rows_by_head(
        oracle_mod,
        lambda i: tuple(_f32(t[i // h, i % h].index_select(0, order)).reshape(1, n, 128) for t in (q, k, v)),
        lambda i: _f32(out[i // h, i % h].index_select(0, order)).reshape(n, 128), ids, w,
        [r for rs in per_launch.values() for r in rs] + extra, qb, n, "c4 full call")
