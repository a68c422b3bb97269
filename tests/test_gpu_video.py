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


def test_exact_attention_wide_logits(oracle_mod):
    """Queries of magnitude ~60: the logits of a row span hundreds (base 2),
    so most rows' maxima lie far above their first tile's and the dense walk
    runs them with a moving reference; rows and LSEs still match the oracle."""
    torch.manual_seed(23)
    nq, nk = 512, 1024
    print(f"exact attention wide logits nq={nq} nk={nk}", flush=True)
    q = (torch.randn(1, 2, nq, 128) * 60).to(torch.bfloat16)
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


def test_exact_attention_largest_head(oracle_mod):
    """Dense attention over the longest head a plan can cover (131,072
    tokens: 32,768 KV4 blocks, 1,024 query blocks), one head; the first and
    last rows against the oracle over every block at weight 0."""
    torch.manual_seed(31)
    n = 131072
    print(f"exact attention largest head n={n}", flush=True)
    q, k, v = (torch.randn(1, 1, n, 128).to(torch.bfloat16) for _ in range(3))
    out, lse = exact_attention(q.cuda(), k.cuda(), v.cuda(), return_lse=True)
    torch.cuda.synchronize()
    got, got_l = _f32(out).reshape(n, 128), _f32(lse).reshape(n)
    assert np.isfinite(got).all() and np.isfinite(got_l).all()
    rows = n // 128
    keep = np.array([0, rows - 1])
    ids, w = _dense_plan(rows, n // 4)
    ref_o, ref_l = oracle_mod.prefill(_f32(q).reshape(1, n, 128), _f32(k).reshape(1, n, 128),
                                      _f32(v).reshape(1, n, 128), ids, w, rows=keep)
    for r in keep:
        sl = slice(int(r) * 128, int(r) * 128 + 128)
        _close(got[sl], ref_o[0, sl])
        assert np.abs(got_l[sl] - ref_l[0, sl]).max() <= LSE_ABS, r


def test_dense_launch_chunks(oracle_mod):
    """Dense attention of 91 heads x 128 query blocks = 11,648 rows runs as two
    launches of whole generations (the first covering heads 0-47), like the
    sparse prefill. Every row is written (the output starts as NaN), and rows
    at both ends of each launch match the oracle over all 4,096 blocks at
    weight 0."""
    from ab_attention import _lib

    torch.manual_seed(12)
    heads, n = 91, 128 * 128
    print(f"dense launch chunks heads={heads} n={n}", flush=True)
    q, k, v = (torch.randn(1, heads, n, 128).to(torch.bfloat16) for _ in range(3))
    qd, kd, vd = q.cuda(), k.cuda(), v.cuda()
    out = torch.full_like(qd, float("nan"))
    lse = torch.full((1, heads, n), float("nan"), device="cuda")
    lib = _lib.load()
    _lib.check(lib.ab_dense_prefill(_lib.ptr(qd), _lib.ptr(kd), _lib.ptr(vd), heads, n, n, _lib.ptr(out), _lib.ptr(lse),
                                    _lib.stream(qd.device)))
    torch.cuda.synchronize()
    assert bool(torch.isfinite(out).all()) and bool(torch.isfinite(lse).all())
    rows = heads * 128
    keep = np.array([0, 47 * 128 + 5, 48 * 128 - 1, 48 * 128, 48 * 128 + 77, rows - 1])
    ids, w = _dense_plan(rows, n // 4)
    ref_o, ref_l = oracle_mod.prefill(_f32(q).reshape(heads, n, 128), _f32(k).reshape(heads, n, 128),
                                      _f32(v).reshape(heads, n, 128), ids, w, rows=keep)
    got, got_l = _f32(out).reshape(heads, n, 128), _f32(lse).reshape(heads, n)
    for r in keep:
        h, b = divmod(int(r), 128)
        sl = slice(b * 128, b * 128 + 128)
        _close(got[h, sl], ref_o[h, sl])
        assert np.abs(got_l[h, sl] - ref_l[h, sl]).max() <= LSE_ABS, r


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


def test_dense_equals_listed_pages(oracle_mod):
    """exact_attention walks the blocks with no page list (ab_dense_prefill,
    the 16x16x32 dense kernel); the sparse kernel over an explicit list of
    every block at weight 0 (padded to a multiple of 8 with -inf) computes the
    same attention with other MFMA tiles: the two agree within bf16 rounding
    (max-abs 2e-3, LSE 1e-4) everywhere, and both are within the bf16 bars of
    the oracle on the first and last rows of each head."""
    from ab_attention.paged import _prefill_kv
    from ab_attention.video import _dense_pages

    torch.manual_seed(17)
    nq, nk = 4000, 4092
    print(f"dense vs listed nq={nq} nk={nk}", flush=True)
    q = torch.randn(1, 2, nq, 128).to(torch.bfloat16).cuda()
    k = torch.randn(1, 2, nk, 128).to(torch.bfloat16).cuda()
    v = torch.randn(1, 2, nk, 128).to(torch.bfloat16).cuda()
    out, lse = exact_attention(q, k, v, return_lse=True)
    rows = 2 * -(-nq // 128)
    ids, w = _dense_pages(rows, nk // 4, q.device)
    out_l, lse_l = _prefill_kv(q, k, v, ids, w, return_lse=True)
    torch.cuda.synchronize()
    assert float((out.float() - out_l.float()).abs().max()) <= 2e-3
    assert float((lse - lse_l).abs().max()) <= 1e-4
    keep = np.array([0, rows // 2 - 1, rows // 2, rows - 1])
    ids_o, w_o = _dense_plan(rows, nk // 4)
    ref_o, ref_l = oracle_mod.prefill(_f32(q).reshape(2, nq, 128), _f32(k).reshape(2, nk, 128),
                                      _f32(v).reshape(2, nk, 128), ids_o, w_o, rows=keep)
    for o_t, l_t in ((out, lse), (out_l, lse_l)):
        got, got_l = _f32(o_t).reshape(2, nq, 128), _f32(l_t).reshape(2, nq)
        for r in keep:
            bh, blk = divmod(int(r), rows // 2)
            lo, hi = blk * 128, min(nq, blk * 128 + 128)
            _close(got[bh, lo:hi], ref_o[bh, lo:hi])
            assert np.abs(got_l[bh, lo:hi] - ref_l[bh, lo:hi]).max() <= LSE_ABS


def test_video_attention_plan_schedule(oracle_mod):
    """The denoising schedule (reference: video.py:53-87): dense through step
    10 and on layer 0; a layer's plan is built at anchor steps 11, 15, ...
    with seed 42 + layer*1000003 + anchor*97, and reused in between, here
    across steps 11, 12, 14 and 15 with new activations at every step. Each
    plan equals build_plan with that seed; the rebuilt plan at step 15 is
    bit-exact with the oracle's SIP on the GPU's scores and uniforms, and
    every step's output is within the bf16 bars of the oracle given the plan
    in use."""
    from ab_attention import _C, apply_plan, build_plan

    torch.manual_seed(23)
    n, pages, layer = 2048, 2, 3
    sched = VideoAttention(pages)
    assert not sched.is_sparse(layer)
    sched.step_end(None, 9, None, {})  # index 9 ends step 10; next is step 11
    assert sched.step == 11 and sched.is_sparse(layer) and not sched.is_sparse(0)
    plans = {}
    for step in (11, 12, 14, 15):
        sched.step = step
        print(f"schedule step {step}", flush=True)
        q, k, v = (torch.randn(1, 2, n, 128).to(torch.bfloat16).cuda() for _ in range(3))
        out = sched.attend(layer, q, k, v)
        anchor, plan = sched.plans[layer]
        assert anchor == (11 if step < 15 else 15)
        plans[step] = plan
        seed = 42 + layer * 1_000_003 + anchor * 97
        if step in (11, 15):
            fresh = build_plan(q, k, sample_pages=pages, seed=seed)
            assert torch.equal(fresh.descriptor, plan.descriptor)
            assert torch.equal(fresh.log_weights.view(torch.int32), plan.log_weights.view(torch.int32))
        else:
            assert plan is plans[11]  # reused, not rebuilt
        assert torch.equal(out, apply_plan(q, k, v, plan))
        rows = plan.descriptor.shape[0]
        ids = plan.descriptor.reshape(rows, -1).cpu().numpy()
        w = plan.log_weights.reshape(rows, -1).cpu().numpy()
        if step == 15:
            offsets = torch.rand(rows, device=q.device, generator=torch.Generator(q.device).manual_seed(seed))
            ids_o, w_o = oracle_mod.sip(_C.ibcs(q, k).cpu().numpy(), offsets.cpu().numpy(), pages * 32)
            assert np.array_equal(ids, ids_o) and np.array_equal(w.view(np.uint32), w_o.view(np.uint32))
        ref, _ = oracle_mod.prefill(*(_f32(t).reshape(2, n, 128) for t in (q, k, v)), ids, w)
        _close(_f32(out).reshape(2, n, 128), ref)
    assert plans[15] is not plans[11] and not torch.equal(plans[15].descriptor, plans[11].descriptor)


def test_apply_plan_in_hip_graph():
    """apply_plan recorded into a HIP graph (the reference runs its prefill
    with CUDA-graph buffers, flashinfer_backend.py:132-143): every replay, with
    new Q/K/V copied into the captured inputs and eager work and
    synchronisations between replays, equals the eager call bit for bit."""
    from ab_attention import apply_plan, build_plan

    torch.manual_seed(29)
    n, pages = 4096, 4
    q, k, v = (torch.randn(1, 2, n, 128).to(torch.bfloat16).cuda() for _ in range(3))
    plan = build_plan(q, k, sample_pages=pages, seed=5)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        apply_plan(q, k, v, plan, return_lse=True)  # warm-up outside capture
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static_out, static_lse = apply_plan(q, k, v, plan, return_lse=True)
    for i in range(4):
        print(f"graph replay {i}", flush=True)
        for t in (q, k, v):
            t.copy_(torch.randn(t.shape, device=t.device).to(torch.bfloat16))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        want, want_lse = apply_plan(q, k, v, plan, return_lse=True)
        torch.cuda.synchronize()
        assert torch.equal(static_out, want)
        assert torch.equal(static_lse, want_lse)


@pytest.mark.parametrize("compact", [False, True])
def test_video_attention_offloaded_plans(compact):
    """offload=True keeps each layer's plan in pinned host memory (the
    reference's _store_plan, video.py:43-50) and copies it back on reuse,
    with int16 ids when compact=True; the outputs equal the device-resident
    schedule's at every step, and so do the compact plans kept on the GPU."""
    torch.manual_seed(31)
    n, pages, layer = 2048, 2, 2
    on_gpu = VideoAttention(pages)
    offloaded = VideoAttention(pages, offload=True, compact=compact)
    compact_gpu = VideoAttention(pages, compact=True)
    for step in (11, 13, 15, 16):
        print(f"offloaded schedule step {step} compact={compact}", flush=True)
        on_gpu.step = offloaded.step = compact_gpu.step = step
        q, k, v = (torch.randn(1, 2, n, 128).to(torch.bfloat16).cuda() for _ in range(3))
        a = on_gpu.attend(layer, q, k, v)
        b = offloaded.attend(layer, q, k, v)
        c = compact_gpu.attend(layer, q, k, v)
        torch.cuda.synchronize()
        assert torch.equal(a, b) and torch.equal(a, c)
        stored = offloaded.plans[layer][1]
        assert stored.descriptor.device.type == "cpu" and stored.descriptor.is_pinned()
        assert stored.descriptor.dtype == (torch.int16 if compact else torch.int32)
        assert torch.equal(stored.descriptor.to(torch.int32), on_gpu.plans[layer][1].descriptor.cpu())
