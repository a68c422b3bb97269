"""The headline workload, Wan2.1-14B 720p (B=2, H=40,
75,600 raster-order tokens, 64 sample pages), on the GPU against the CPU
oracle (reference: ab_attention/attention.py:26-102).

test_c2_raster_head -- one full-length head (591 query blocks, the last
holding 80 queries; 18,900 KV4 blocks; 2,048 sampled per row):
  - the fused plan (_C.ibcs_sip, what build_plan calls) on all 591 rows:
    ids and weights bit-exact with the oracle's SIP given the GPU's IBCS
    scores (_C.ibcs) and the same uniforms;
  - the IBCS scores against the oracle's IBCS: rows sum to 1 within 2e-5,
    99 % of entries within 1e-5 relative, none beyond 3e-2 (the MFMA dot
    products and hardware exp2/log2 flip a few fp16 pair-LSEs by one ulp);
  - the share of plan ids equal to the oracle's own plan (oracle IBCS, then
    oracle SIP) is at least 0.99;
  - the output over the GPU plan against the exact fp64 oracle prefill given
    that plan on 10 rows, the ragged last query block among them: max-abs
    2e-2 and rel-L2 1e-2 per row, base-2 LSE within 1e-3.

test_c2_full_call -- the whole call through build_plan and apply_plan:
  - every one of the 47,280 rows satisfies SIP's invariants: ids inside the
    head, weights finite and >= 0, the certain blocks (weight 0) first and
    strictly ascending, then non-decreasing draws, and no id twice; a row
    that breaks one must be reproduced bit for bit by the oracle (the
    reference's walk can repeat an id inside a few-ulp window of its prefix
    array);
  - 64 random rows across all 80 heads are bit-exact with the oracle's SIP on
    the GPU's scores and build_plan's uniforms;
  - the output is finite; rows of every one of the prefill's 5 launches
    (each launch's first and last row slots and the slots on both sides of
    a generation boundary, on the first and last XCD) and 8 rows across 4
    heads match the oracle prefill.
"""
import numpy as np
import pytest
import torch

from ab_attention import SamplePlan, _C, apply_plan, build_plan
from ab_attention.synthetic import CONFIGS, make_qkv, parity_offsets

pytestmark = pytest.mark.gpu

MAX_ABS, REL_L2, LSE_ABS = 2e-2, 1e-2, 1e-3


def _f32(t):
    return t.float().cpu().numpy()


def _bits(t):
    return np.ascontiguousarray(t.cpu().contiguous().view(torch.int16).numpy().view(np.uint16))


def _check_rows(got, got_lse, ref, ref_lse, rows, n):
    """got/ref [n, 128] and lse [n] of one head; compare the given rows."""
    for r in rows:
        lo, hi = r * 128, min(n, r * 128 + 128)
        g, e = np.asarray(got[lo:hi], np.float64), np.asarray(ref[lo:hi], np.float64)
        err = np.abs(g - e).max()
        assert err <= MAX_ABS, (r, err)
        rel = np.linalg.norm(g - e) / np.linalg.norm(e)
        assert rel <= REL_L2, (r, rel)
        if got_lse is not None:
            lerr = np.abs(got_lse[lo:hi] - ref_lse[lo:hi]).max()
            assert lerr <= LSE_ABS, (r, lerr)


def launch_check_rows(bh, n):
    """Rows to compare with the oracle in every prefill launch of a call of
    bh heads x n tokens, as {launch: [rows]}: the first and last row slot of
    the launch and the two slots on each side of a generation boundary in
    its middle, each on XCD 0 and on the last XCD whose query blocks reach
    that slot. The library deals the rows of head h, query block b to XCD
    group b // ceil(qb / 8) at slot h * ceil(qb / 8) + b % ceil(qb / 8); launch
    i covers the slots [i * S, (i + 1) * S) of every group, S =
    ab_prefill_launch_slots (whole generations of 64 slots)."""
    from ab_attention import _lib

    qb = -(-n // 128)
    per_xcd = -(-qb // 8)
    slots = per_xcd * bh
    per_launch = _lib.load().ab_prefill_launch_slots(bh, n)
    picks = {}
    for launch, s0 in enumerate(range(0, slots, per_launch)):
        s1 = min(s0 + per_launch, slots)
        mid = s0 + 64 * (-(-(s1 - s0) // 64) // 2)
        rows = set()
        for slot in sorted({s0, mid - 1, mid, s1 - 1}):
            if not s0 <= slot < s1:
                continue
            head, off = divmod(slot, per_xcd)
            rows.add(head * qb + off)  # XCD 0
            for xcd in range(7, 0, -1):
                if xcd * per_xcd + off < qb:
                    rows.add(head * qb + xcd * per_xcd + off)
                    break
        picks[launch] = sorted(rows)
    return picks


def check_rows_by_head(oracle_mod, head_tensors, out_head, ids, w, rows, qb, n, tag):
    """Compare the output rows `rows` (global plan rows) with the oracle
    prefill, one head at a time. head_tensors(bh) -> (q, k, v) f32 [1, n, 128]
    and out_head(bh) -> output f32 [n, 128] of that head, in the order the plan
    indexes its tokens."""
    rows = np.asarray(sorted(set(int(r) for r in rows)))
    for bh_i in np.unique(rows // qb):
        local = rows[rows // qb == bh_i] - bh_i * qb
        head = slice(bh_i * qb, (bh_i + 1) * qb)
        print(f"{tag}: head {bh_i} rows {local.tolist()}", flush=True)
        qh, kh, vh = head_tensors(int(bh_i))
        ref, _ = oracle_mod.prefill(qh, kh, vh, ids[head].cpu().numpy(), w[head].cpu().numpy(), rows=local)
        _check_rows(out_head(int(bh_i)), None, ref[0], None, local, n)


def _assert_sip_equal(ids_g, w_g, ids_o, w_o):
    bad = np.nonzero((ids_g != ids_o).any(axis=1) | (w_g.view(np.uint32) != w_o.view(np.uint32)).any(axis=1))[0]
    assert bad.size == 0, f"{bad.size} rows differ from the oracle's SIP, first {bad[:8]}"


def test_c2_raster_head(oracle_mod):
    cfg = CONFIGS[2]
    head = 17
    print(f"c2 raster head {head}: tokens {cfg.tokens}, P={cfg.sample_pages}", flush=True)
    q, k, v = (t[:1].contiguous() for t in make_qkv(cfg, heads=[head], dtype=torch.bfloat16))
    n = q.shape[2]
    rows, fb, samples = -(-n // 128), n // 4, cfg.sample_pages * 32
    assert (rows, fb, n - (rows - 1) * 128) == (591, 18900, 80)
    offsets = parity_offsets(rows, seed=11)
    qd, kd, vd = q.cuda(), k.cuda(), v.cuda()
    ids = torch.empty((rows, samples), dtype=torch.int32, device="cuda")
    w = torch.empty((rows, samples), dtype=torch.float32, device="cuda")
    _C.ibcs_sip(qd, kd, offsets.cuda(), ids, w)
    scores = _C.ibcs(qd, kd)
    plan = SamplePlan(ids.reshape(rows, cfg.sample_pages, 32), w.reshape(rows, cfg.sample_pages, 32))
    out, lse = apply_plan(qd, kd, vd, plan, return_lse=True)
    torch.cuda.synchronize()
    ids_g, w_g, scores_g = ids.cpu().numpy(), w.cpu().numpy(), scores.cpu().numpy()

    # SIP: every row bit-exact on the GPU's own scores and the same uniforms
    ids_o, w_o = oracle_mod.sip(scores_g, offsets.numpy(), samples)
    _assert_sip_equal(ids_g, w_g, ids_o, w_o)

    # IBCS scores within tolerance of the oracle's
    scores_o = oracle_mod.ibcs(_bits(q).reshape(1, n, 128), _bits(k).reshape(1, n, 128), 1, n)
    np.testing.assert_allclose(scores_g.sum(axis=1), 1.0, rtol=0, atol=2e-5)
    rel = np.abs(scores_g - scores_o) / np.maximum(scores_o, 1e-30)
    assert np.quantile(rel, 0.99) < 1e-5, np.quantile(rel, 0.99)
    assert rel.max() < 3e-2, rel.max()

    # the GPU plan against the oracle's own plan (oracle IBCS and SIP)
    ids_own, _ = oracle_mod.sip(scores_o, offsets.numpy(), samples)
    match = float(np.mean(ids_g == ids_own))
    print(f"c2 head {head}: plan ids equal to the oracle's own plan: {match:.5f}", flush=True)
    assert match >= 0.99, match

    # the output over the GPU plan, ragged last block included
    keep = np.array([0, 1, 2, 147, 295, 296, 443, 588, 589, 590])
    ref, ref_lse = oracle_mod.prefill(*(_f32(t).reshape(1, n, 128) for t in (q, k, v)), ids_g, w_g, rows=keep)
    _check_rows(_f32(out).reshape(n, 128), lse.cpu().numpy().reshape(n), ref[0], ref_lse[0], keep, n)


def _sip_invariants(ids, w, fb):
    """Rows [R, S] (device tensors) that break an invariant of SIP's output."""
    bad = ((ids < 0) | (ids >= fb)).any(dim=1)
    bad |= (~torch.isfinite(w) | (w < 0)).any(dim=1)
    certain = w == 0
    # the certain blocks form a prefix of the row ...
    bad |= (certain[:, 1:] & ~certain[:, :-1]).any(dim=1)
    step = ids[:, 1:] - ids[:, :-1]
    # ... strictly ascending among themselves, then draws non-decreasing
    both_certain = certain[:, 1:] & certain[:, :-1]
    both_drawn = ~certain[:, 1:] & ~certain[:, :-1]
    bad |= (both_certain & (step <= 0)).any(dim=1)
    bad |= (both_drawn & (step < 0)).any(dim=1)
    # no id twice
    srt = torch.sort(ids, dim=1).values
    bad |= (srt[:, 1:] == srt[:, :-1]).any(dim=1)
    return torch.nonzero(bad).flatten()


def test_c2_full_call(oracle_mod):
    cfg = CONFIGS[2]
    print("c2 full call: B=2 H=40 N=75,600", flush=True)
    q, k, v = make_qkv(cfg, device="cuda", dtype=torch.bfloat16)
    b, h, n, _ = q.shape
    bh, qb, fb, samples = b * h, -(-n // 128), n // 4, cfg.sample_pages * 32
    rows = bh * qb
    seed = 42
    plan = build_plan(q, k, sample_pages=cfg.sample_pages, seed=seed)
    out = apply_plan(q, k, v, plan)
    torch.cuda.synchronize()
    assert plan.descriptor.shape == (rows, cfg.sample_pages, 32) and out.shape == q.shape
    ids = plan.descriptor.reshape(rows, samples)
    w = plan.log_weights.reshape(rows, samples)
    assert bool(torch.isfinite(out).all())

    # build_plan's uniforms, drawn the same way
    offsets = torch.rand(rows, device=q.device, generator=torch.Generator(q.device).manual_seed(seed))
    scores = _C.ibcs(q, k)
    rng = np.random.default_rng(2)
    pick = np.sort(rng.choice(rows, size=64, replace=False))
    broken = _sip_invariants(ids, w, fb).cpu().numpy()
    print(f"c2 full call: {broken.size} of {rows} rows break an invariant", flush=True)
    check = np.union1d(pick, broken)
    idx = torch.as_tensor(check, device=q.device)
    ids_o, w_o = oracle_mod.sip(scores[idx].cpu().numpy(), offsets[idx].cpu().numpy(), samples)
    _assert_sip_equal(ids[idx].cpu().numpy(), w[idx].cpu().numpy(), ids_o, w_o)
    assert len(np.unique(pick // qb)) > 40  # the random rows span the heads
    del scores

    # the output against the oracle: rows in every prefill launch (its first
    # and last row slots and both sides of a generation boundary), plus rows
    # of four heads, the ragged last query block among them
    per_launch = launch_check_rows(bh, n)
    assert len(per_launch) == 5 and all(len(r) >= 2 for r in per_launch.values()), per_launch
    extra = [bh_i * qb + r for bh_i in (0, 23, 41, 79)
             for r in ((bh_i % qb, qb - 1) if bh_i % 2 else (qb // 2, 7))]
    check_rows_by_head(
        oracle_mod, lambda i: tuple(_f32(t[i // h, i % h]).reshape(1, n, 128) for t in (q, k, v)),
        lambda i: _f32(out[i // h, i % h]).reshape(n, 128), ids, w,
        [r for rs in per_launch.values() for r in rs] + extra, qb, n, "c2 full call")
