"""Weighted paged prefill on the GPU against the exact (fp64) oracle given one
fixed plan: bf16 output within max-abs 2e-2 and rel-L2 1e-2; base-2 LSE
within 1e-3 (ab_attention/flashinfer_backend.py:30-59, :164-242)."""
import numpy as np
import pytest
import torch

from ab_attention.flashinfer_backend import paged_attention
from ab_attention.synthetic import CONFIGS, make_qkv, parity_offsets

pytestmark = pytest.mark.gpu

MAX_ABS, REL_L2, LSE_ABS = 2e-2, 1e-2, 1e-3


def _plan_from_oracle(oracle_mod, q, k, sample_pages):
    bh, n = q.shape[0] * q.shape[1], q.shape[2]
    bits = lambda t: np.ascontiguousarray(t.contiguous().view(torch.int16).numpy().view(np.uint16))
    scores = oracle_mod.ibcs(bits(q).reshape(bh, n, 128), bits(k).reshape(bh, n, 128), bh, n)
    offsets = parity_offsets(scores.shape[0]).numpy()
    ids, logw = oracle_mod.sip(scores, offsets, sample_pages * 32)
    return ids, logw


def _check(q, k, v, ids, logw, oracle_mod, rows_subset=None):
    b, h, n, _ = q.shape
    bh = b * h
    rows = ids.shape[0]
    pages = ids.shape[1] // 32
    desc = torch.from_numpy(ids.reshape(rows, pages, 32)).cuda()
    w = torch.from_numpy(logw.reshape(rows, pages, 32)).cuda()
    out, lse = paged_attention(q.cuda(), k.cuda(), v.cuda(), desc, w, return_lse=True)
    torch.cuda.synchronize()
    f32 = lambda t: t.float().numpy().reshape(bh, n, 128)
    ref_o, ref_lse = oracle_mod.prefill(f32(q), f32(k), f32(v), ids, logw)
    got = out.float().cpu().numpy().reshape(bh, n, 128)
    err = np.abs(got - ref_o)
    assert err.max() <= MAX_ABS, err.max()
    rel = np.linalg.norm(got - ref_o) / np.linalg.norm(ref_o)
    assert rel <= REL_L2, rel
    lerr = np.abs(lse.cpu().numpy().reshape(bh, n) - ref_lse)
    assert lerr.max() <= LSE_ABS, lerr.max()


@pytest.mark.parametrize("n,pages", [(2048, 2), (2048, 1), (2000, 2)])
def test_prefill_c0_geometry(oracle_mod, n, pages):
    q, k, v = make_qkv(CONFIGS[0], dtype=torch.bfloat16)
    q, k, v = (t[:, :, :n].contiguous() for t in (q, k, v))
    print(f"prefill c0 n={n} pages={pages}", flush=True)
    ids, logw = _plan_from_oracle(oracle_mod, q, k, pages)
    _check(q, k, v, ids, logw, oracle_mod)


def test_prefill_dense_equals_softmax(oracle_mod):
    """All KV4 blocks with weight 0 (S = fb) is plain softmax attention."""
    torch.manual_seed(0)
    n = 512
    q, k, v = (torch.randn(1, 2, n, 128).to(torch.bfloat16) for _ in range(3))
    rows, fb = 2 * (n // 128), n // 4
    ids = np.tile(np.arange(fb, dtype=np.int32), (rows, 1))
    logw = np.zeros((rows, fb), np.float32)
    _check(q, k, v, ids, logw, oracle_mod)
    qf, kf, vf = (t.double() for t in (q, k, v))
    att = torch.softmax(qf @ kf.transpose(-1, -2) / np.sqrt(128.0), dim=-1) @ vf
    desc = torch.from_numpy(ids.reshape(rows, fb // 32, 32)).cuda()
    out = paged_attention(q.cuda(), k.cuda(), v.cuda(), desc, torch.zeros_like(desc, dtype=torch.float32))
    assert (out.double().cpu() - att).abs().max() <= MAX_ABS


def test_prefill_random_plan_with_duplicates(oracle_mod):
    """Arbitrary (unsorted, repeated) ids and weights: every listed block counts."""
    rng = np.random.default_rng(5)
    torch.manual_seed(1)
    n = 1024
    q, k, v = (torch.randn(2, 1, n, 128).to(torch.bfloat16) for _ in range(3))
    rows, fb = 2 * (n // 128), n // 4
    ids = rng.integers(0, fb, size=(rows, 64)).astype(np.int32)
    logw = (rng.random((rows, 64)) * 6).astype(np.float32)
    _check(q, k, v, ids, logw, oracle_mod)


def test_prefill_partial_id_batch(oracle_mod):
    """640 sampled blocks (80 tiles of 8): the kernel's second batch of page ids
    and weights is partial, so its tail is read clamped to the row's end."""
    rng = np.random.default_rng(12)
    torch.manual_seed(3)
    n = 4096
    q, k, v = (torch.randn(1, 1, n, 128).to(torch.bfloat16) for _ in range(3))
    print("prefill n=4096 samples=640", flush=True)
    rows, fb = n // 128, n // 4
    ids = np.sort(rng.choice(fb, size=(rows, 640), replace=True), axis=1).astype(np.int32)
    logw = (rng.random((rows, 640)) * 5).astype(np.float32)
    _check(q, k, v, ids, logw, oracle_mod)


def test_prefill_c1_head_subset(oracle_mod):
    """One Wan2.1-1.3B head at full length (32,760 tokens, partial last block),
    64 sample pages; the oracle checks the first and last three rows."""
    q, k, v = make_qkv(CONFIGS[1], heads=[2], dtype=torch.bfloat16)
    q, k, v = q[:1], k[:1], v[:1]
    print("prefill c1 head 2", flush=True)
    n = q.shape[2]
    rng = np.random.default_rng(9)
    rows, fb = -(-n // 128), n // 4
    ids = np.sort(rng.choice(fb, size=(rows, 2048), replace=True), axis=1).astype(np.int32)
    logw = (rng.random((rows, 2048)) * 4).astype(np.float32)
    desc = torch.from_numpy(ids.reshape(rows, 64, 32)).cuda()
    w = torch.from_numpy(logw.reshape(rows, 64, 32)).cuda()
    out, lse = paged_attention(q.cuda(), k.cuda(), v.cuda(), desc, w, return_lse=True)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy().reshape(n, 128)
    got_lse = lse.cpu().numpy().reshape(n)
    f32 = lambda t: t.float().numpy().reshape(1, n, 128)
    keep = np.r_[0:3, rows - 3:rows]
    ref_o, ref_lse = oracle_mod.prefill(f32(q), f32(k), f32(v), ids, logw, rows=keep)
    for r in keep:
        lo, hi = r * 128, min(n, r * 128 + 128)
        e = np.abs(got[lo:hi] - ref_o[0, lo:hi])
        assert e.max() <= MAX_ABS, (r, e.max())
        assert np.abs(got_lse[lo:hi] - ref_lse[0, lo:hi]).max() <= LSE_ABS


def test_prefill_largest_head(oracle_mod):
    """The longest head a plan can cover (build_plan's limit): 131,072
    tokens (32,768 KV4 blocks, 1,024 query blocks), 64 sample pages; every
    row lists the head's first and last KV4 blocks (page offsets up to
    32 MiB - 1 KiB into K and V). The oracle checks the first and last three
    rows and two in the middle."""
    rng = np.random.default_rng(33)
    torch.manual_seed(8)
    n, samples = 131072, 2048
    print(f"prefill largest head n={n}", flush=True)
    q, k, v = (torch.randn(1, 1, n, 128).to(torch.bfloat16) for _ in range(3))
    rows, fb = n // 128, n // 4
    ids = np.sort(rng.choice(fb, size=(rows, samples), replace=True), axis=1).astype(np.int32)
    ids[:, 0], ids[:, -1] = 0, fb - 1
    logw = (rng.random((rows, samples)) * 4).astype(np.float32)
    desc = torch.from_numpy(ids.reshape(rows, samples // 32, 32)).cuda()
    w = torch.from_numpy(logw.reshape(rows, samples // 32, 32)).cuda()
    out, lse = paged_attention(q.cuda(), k.cuda(), v.cuda(), desc, w, return_lse=True)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy().reshape(n, 128)
    got_lse = lse.cpu().numpy().reshape(n)
    assert np.isfinite(got).all() and np.isfinite(got_lse).all()
    f32 = lambda t: t.float().numpy().reshape(1, n, 128)
    keep = np.r_[0:3, 511:513, rows - 3:rows]
    ref_o, ref_lse = oracle_mod.prefill(f32(q), f32(k), f32(v), ids, logw, rows=keep)
    for r in keep:
        lo, hi = r * 128, r * 128 + 128
        e = np.abs(got[lo:hi] - ref_o[0, lo:hi])
        assert e.max() <= MAX_ABS, (r, e.max())
        rel = np.linalg.norm(got[lo:hi] - ref_o[0, lo:hi]) / np.linalg.norm(ref_o[0, lo:hi])
        assert rel <= REL_L2, (r, rel)
        assert np.abs(got_lse[lo:hi] - ref_lse[0, lo:hi]).max() <= LSE_ABS


def test_prefill_workgroup_generations(oracle_mod):
    """7 heads x 80 query blocks: each XCD runs 70 row slots, one full
    generation of 64 (where the two workgroups sharing a CU take adjacent
    query blocks) and a partial one. Every row must be computed once: the
    output starts as NaN and all rows are checked against the oracle."""
    rng = np.random.default_rng(21)
    torch.manual_seed(4)
    heads, n, samples = 7, 80 * 128, 32
    print(f"prefill generations heads={heads} n={n}", flush=True)
    q, k, v = (torch.randn(1, heads, n, 128).to(torch.bfloat16) for _ in range(3))
    rows, fb = heads * (n // 128), n // 4
    ids = np.sort(rng.choice(fb, size=(rows, samples), replace=True), axis=1).astype(np.int32)
    logw = (rng.random((rows, samples)) * 3).astype(np.float32)
    _check(q, k, v, ids, logw, oracle_mod)


def test_prefill_neg_inf_blocks(oracle_mod):
    """A -inf weight removes its block wherever it sits in the row: rows whose
    first tile (8 blocks), first 20 blocks or a middle tile are at -inf match
    the oracle over the remaining blocks; a row with every block at -inf
    gives o = 0 and lse = -inf, not NaN."""
    rng = np.random.default_rng(31)
    torch.manual_seed(6)
    n, samples = 1024, 64
    rows, fb = n // 128, n // 4
    q, k, v = (torch.randn(1, 1, n, 128).to(torch.bfloat16) for _ in range(3))
    ids = np.sort(rng.choice(fb, size=(rows, samples), replace=True), axis=1).astype(np.int32)
    logw = (rng.random((rows, samples)) * 3).astype(np.float32)
    logw[0, :8] = -np.inf
    logw[1, :20] = -np.inf
    logw[2, 8:16] = -np.inf
    logw[3, :] = -np.inf
    logw[4, -8:] = -np.inf
    print("prefill -inf blocks n=1024", flush=True)
    desc = torch.from_numpy(ids.reshape(rows, 2, 32)).cuda()
    w = torch.from_numpy(logw.reshape(rows, 2, 32)).cuda()
    out, lse = paged_attention(q.cuda(), k.cuda(), v.cuda(), desc, w, return_lse=True)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy().reshape(n, 128)
    got_lse = lse.cpu().numpy().reshape(n)
    f32 = lambda t: t.float().numpy().reshape(1, n, 128)
    ref_o, ref_lse = oracle_mod.prefill(f32(q), f32(k), f32(v), ids, logw)
    for r in range(rows):
        lo, hi = r * 128, r * 128 + 128
        if r == 3:  # every block at -inf: the oracle's empty softmax, exactly
            assert np.array_equal(got[lo:hi], ref_o[0, lo:hi]) and np.all(ref_o[0, lo:hi] == 0.0)
            assert np.all(np.isneginf(got_lse[lo:hi])) and np.all(np.isneginf(ref_lse[0, lo:hi]))
            continue
        assert np.abs(got[lo:hi] - ref_o[0, lo:hi]).max() <= MAX_ABS, r
        assert np.abs(got_lse[lo:hi] - ref_lse[0, lo:hi]).max() <= LSE_ABS, r


def test_prefill_logit_range(oracle_mod):
    """Weights far above the first tile's maximum. The kernel keeps each
    query's first-tile maximum as its reference while no logit exceeds it by
    more than 64 (base 2), and otherwise runs the row again with a moving
    reference. Rows: a later tile 50 above (kept), 90 above (run again), the
    last tile 200 above (run again), the first tile 100 above the rest (kept;
    every later term is 2^-100 of it), +12 per tile (run again once the ramp
    passes 64); all match the oracle."""
    rng = np.random.default_rng(77)
    torch.manual_seed(9)
    n, samples = 1024, 64
    rows, fb = n // 128, n // 4
    q, k, v = (torch.randn(1, 1, n, 128).to(torch.bfloat16) for _ in range(3))
    ids = np.sort(rng.choice(fb, size=(rows, samples), replace=True), axis=1).astype(np.int32)
    logw = (rng.random((rows, samples)) * 3).astype(np.float32)
    logw[0, 24:32] += 50.0
    logw[1, 24:32] += 90.0
    logw[2, 56:64] += 200.0
    logw[3, :8] += 100.0
    logw[4] += 12.0 * (np.arange(samples) // 8)
    print("prefill logit range n=1024", flush=True)
    _check(q, k, v, ids, logw, oracle_mod)


def test_prefill_launch_chunks(oracle_mod):
    """91 heads x 128 query blocks = 11,648 rows: the prefill runs as two
    launches of whole generations (64 row slots per XCD, 16 slots per head on
    each XCD), the first covering heads 0-47. Every row must be written once
    (the output starts as NaN) and rows of heads 47 and 48, the first and the
    last, match the oracle."""
    from ab_attention import _lib

    rng = np.random.default_rng(41)
    torch.manual_seed(8)
    heads, n, samples = 91, 128 * 128, 32
    print(f"prefill launch chunks heads={heads} n={n}", flush=True)
    q, k, v = (torch.randn(1, heads, n, 128).to(torch.bfloat16) for _ in range(3))
    rows, fb = heads * 128, n // 4
    ids = np.sort(rng.choice(fb, size=(rows, samples), replace=True), axis=1).astype(np.int32)
    logw = (rng.random((rows, samples)) * 3).astype(np.float32)
    qd, kd, vd = q.cuda(), k.cuda(), v.cuda()
    out = torch.full_like(qd, float("nan"))
    lse = torch.full((1, heads, n), float("nan"), device="cuda")
    ids_d, logw_d = torch.from_numpy(ids).cuda(), torch.from_numpy(logw).cuda()
    lib = _lib.load()
    _lib.check(lib.ab_paged_prefill_kv(_lib.ptr(qd), _lib.ptr(kd), _lib.ptr(vd), heads, n, n, _lib.ptr(ids_d),
                                       _lib.ptr(logw_d), samples, _lib.ptr(out), _lib.ptr(lse), _lib.stream(qd.device)))
    torch.cuda.synchronize()
    assert bool(torch.isfinite(out).all()) and bool(torch.isfinite(lse).all())
    keep = np.array([0, 47 * 128 + 5, 48 * 128 - 1, 48 * 128, 48 * 128 + 77, rows - 1])
    ref_o, ref_l = oracle_mod.prefill(q.float().numpy().reshape(heads, n, 128), k.float().numpy().reshape(heads, n, 128),
                                      v.float().numpy().reshape(heads, n, 128), ids, logw, rows=keep)
    got, got_l = out.float().cpu().numpy().reshape(heads, n, 128), lse.cpu().numpy().reshape(heads, n)
    for r in keep:
        h, b = divmod(int(r), 128)
        sl = slice(b * 128, b * 128 + 128)
        assert np.abs(got[h, sl] - ref_o[h, sl]).max() <= MAX_ABS, r
        assert np.abs(got_l[h, sl] - ref_l[h, sl]).max() <= LSE_ABS, r
