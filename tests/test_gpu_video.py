"""HunyuanVideo partition and its parts on the GPU (reference:
ab_attention/video.py:13-40 _exact/_merge, :129-151 _hunyuan_attention).

Against the exact (fp64) oracle: dense attention with a K/V length of its own
(bf16 max-abs 2e-2, rel-L2 1e-2, base-2 LSE within 1e-3), the state merge,
and the whole partition, fused (prompt blocks at weight 0 in the video
prefill) and as the reference structures it (sampled state, exact prompt
state, merge) -- the two must also agree with each other.
"""
import numpy as np
import pytest
import torch

from ab_attention.video import VideoAttention, exact_attention, hunyuan_attention, merge_states

pytestmark = pytest.mark.gpu

MAX_ABS, REL_L2, LSE_ABS = 2e-2, 1e-2, 1e-3


def _f32(t):
    return t.float().cpu().numpy()


def _close(got, ref):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    err = np.abs(got - ref).max()
    assert err <= MAX_ABS, err
    rel = np.linalg.norm(got - ref) / np.linalg.norm(ref)
    assert rel <= REL_L2, rel


def _dense_plan(rows, blocks, offset=0):
    ids = np.tile(np.arange(offset, offset + blocks, dtype=np.int32), (rows, 1))
    return ids, np.zeros(ids.shape, np.float32)


@pytest.mark.parametrize("nq,nk", [(300, 256), (256, 1000), (96, 4)])
def test_exact_attention(oracle_mod, nq, nk):
    torch.manual_seed(nq + nk)
    print(f"exact attention nq={nq} nk={nk}", flush=True)
    q = torch.randn(1, 2, nq, 128).to(torch.bfloat16)
    k = torch.randn(1, 2, nk, 128).to(torch.bfloat16)
    v = torch.randn(1, 2, nk, 128).to(torch.bfloat16)
    out, lse = exact_attention(q.cuda(), k.cuda(), v.cuda(), return_lse=True)
    torch.cuda.synchronize()
    rows = 2 * -(-nq // 128)
    ids, w = _dense_plan(rows, nk // 4)
    ref_o, ref_l = oracle_mod.prefill(_f32(q).reshape(2, nq, 128), _f32(k).reshape(2, nk, 128),
                                      _f32(v).reshape(2, nk, 128), ids, w)
    _close(_f32(out).reshape(2, nq, 128), ref_o)
    assert np.abs(_f32(lse).reshape(2, nq) - ref_l).max() <= LSE_ABS


def test_merge_states(oracle_mod):
    torch.manual_seed(7)
    n = 200
    print("merge states", flush=True)
    q = torch.randn(1, 3, n, 128).to(torch.bfloat16).cuda()
    ka, va = (torch.randn(1, 3, 64, 128).to(torch.bfloat16).cuda() for _ in range(2))
    kb = (torch.randn(1, 3, 128, 128) * 2).to(torch.bfloat16).cuda()  # sharper logits for the second part
    vb = torch.randn(1, 3, 128, 128).to(torch.bfloat16).cuda()
    sa = exact_attention(q, ka, va, return_lse=True)
    sb = exact_attention(q, kb, vb, return_lse=True)
    out, lse = merge_states(sa, sb, return_lse=True)
    torch.cuda.synchronize()
    ref_o, ref_l = oracle_mod.merge_states(_f32(sa[0]), _f32(sa[1]), _f32(sb[0]), _f32(sb[1]))
    # one bf16 rounding of the merged output: half an ulp, <= 2^-8 |o|
    assert np.all(np.abs(_f32(out) - ref_o) <= np.abs(ref_o) * 2.0 ** -8 * 1.01 + 1e-5)
    assert np.abs(_f32(lse) - ref_l).max() <= 1e-5
    # the merge of the two partitions is attention over the union
    union = exact_attention(q, torch.cat([ka, kb], 2), torch.cat([va, vb], 2))
    _close(_f32(out), _f32(union))


def _hunyuan_oracle(oracle_mod, q, k, v, plan, video, prompt, sparse):
    """Exact output of the partition: per-part oracle prefills (fp64)."""
    b, h, n, _ = q.shape
    bh, end = b * h, video + prompt
    f = lambda t, lo, hi: _f32(t[:, :, lo:hi]).reshape(bh, hi - lo, 128)
    out = np.empty((bh, n, 128))
    if sparse:
        rows = plan.descriptor.shape[0]
        t_ids, t_w = _dense_plan(rows, prompt // 4, offset=video // 4)
        ids = np.concatenate([plan.descriptor.cpu().numpy().reshape(rows, -1), t_ids], 1)
        w = np.concatenate([plan.log_weights.cpu().numpy().reshape(rows, -1), t_w], 1)
        out[:, :video] = oracle_mod.prefill(f(q, 0, video), f(k, 0, end), f(v, 0, end), ids, w)[0]
        ids, w = _dense_plan(bh * -(-prompt // 128), end // 4)
        out[:, video:end] = oracle_mod.prefill(f(q, video, end), f(k, 0, end), f(v, 0, end), ids, w)[0]
    else:
        ids, w = _dense_plan(bh * -(-end // 128), end // 4)
        out[:, :end] = oracle_mod.prefill(f(q, 0, end), f(k, 0, end), f(v, 0, end), ids, w)[0]
    if end < n:
        ids, w = _dense_plan(bh * -(-(n - end) // 128), (n - end) // 4)
        out[:, end:] = oracle_mod.prefill(f(q, end, n), f(k, end, n), f(v, end, n), ids, w)[0]
    return out


@pytest.mark.parametrize("step,pad", [(11, 64), (13, 0), (5, 64)])
def test_hunyuan_partition(oracle_mod, step, pad):
    """Video 4x16x16 = 1024 tokens, 256 prompt tokens, optional padding."""
    torch.manual_seed(step + pad)
    video, prompt = 1024, 256
    n = video + prompt + pad
    print(f"hunyuan step={step} pad={pad}", flush=True)
    q, k, v = (torch.randn(1, 2, n, 128).to(torch.bfloat16).cuda() for _ in range(3))
    sched = VideoAttention(2)
    sched.step = step
    fused = hunyuan_attention(sched, 1, q, k, v, video, prompt)
    split = hunyuan_attention(sched, 1, q, k, v, video, prompt, fused=False)
    torch.cuda.synchronize()
    assert fused.shape == q.shape and fused.dtype == torch.bfloat16
    sparse = sched.is_sparse(1)
    plan = sched.plans[1][1] if sparse else None
    ref = _hunyuan_oracle(oracle_mod, q.cpu(), k.cpu(), v.cpu(), plan, video, prompt, sparse)
    _close(_f32(fused).reshape(2, n, 128), ref)
    _close(_f32(split).reshape(2, n, 128), ref)
    _close(_f32(fused), _f32(split))
