"""The prefill's KV4-transposed V layout.

ab_kv4_transpose must be an exact rearrangement (v[b, h, 4j + r, d] ->
vt[b, h, j, d, r]), and the prefill over that layout (ab_paged_prefill_kv4t,
used by paged_attention) must give results bit-identical to the row-major
entry points (ab_paged_prefill_kv, ab_paged_prefill_ordered) on the same
inputs: both compute the same MFMA products in the same order, only the LDS
read of the V operand differs.
"""
import numpy as np
import pytest
import torch

from ab_attention import _lib
from ab_attention.paged import kv4_transpose

pytestmark = pytest.mark.gpu


def _random_plan(rows, samples, fb, seed):
    g = np.random.default_rng(seed)
    ids = g.integers(0, fb, size=(rows, samples), dtype=np.int32)
    logw = g.uniform(0.0, 6.0, size=(rows, samples)).astype(np.float32)
    return torch.from_numpy(ids).cuda(), torch.from_numpy(logw).cuda()


def _run(entry, q, k, v, ids, w, *, order=None, kv4t=False):
    lib = _lib.load()
    b, h, n, _ = q.shape
    nk = k.shape[2]
    out = torch.full_like(q, float("nan"))
    lse = torch.empty((b, h, n), dtype=torch.float32, device=q.device)
    st = _lib.stream(q.device)
    if kv4t:
        rc = lib.ab_paged_prefill_kv4t(_lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(order), b * h, n, nk,
                                       _lib.ptr(ids), _lib.ptr(w), ids.shape[1], _lib.ptr(out), _lib.ptr(lse), st)
    elif order is not None:
        rc = lib.ab_paged_prefill_ordered(_lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(order), b * h, n,
                                          _lib.ptr(ids), _lib.ptr(w), ids.shape[1], _lib.ptr(out), _lib.ptr(lse), st)
    else:
        rc = lib.ab_paged_prefill_kv(_lib.ptr(q), _lib.ptr(k), _lib.ptr(v), b * h, n, nk, _lib.ptr(ids),
                                     _lib.ptr(w), ids.shape[1], _lib.ptr(out), _lib.ptr(lse), st)
    _lib.check(rc)
    torch.cuda.synchronize()
    return out, lse


@pytest.mark.parametrize("nk", [4, 256, 2052])
def test_kv4_transpose_exact(nk):
    print(f"kv4_transpose nk={nk}", flush=True)
    torch.manual_seed(nk)
    v = torch.randn(2, 3, nk, 128, device="cuda").to(torch.bfloat16)
    vt = kv4_transpose(v)
    ref = v.reshape(2, 3, nk // 4, 4, 128).permute(0, 1, 2, 4, 3).contiguous()
    assert vt.shape == ref.shape
    assert torch.equal(vt.view(torch.int16), ref.view(torch.int16))


@pytest.mark.parametrize("n,nk,samples", [(2048, 2048, 64), (1000, 2052, 24), (300, 64, 16)])
def test_kv4t_prefill_bit_identical(n, nk, samples):
    print(f"kv4t prefill n={n} nk={nk} samples={samples}", flush=True)
    torch.manual_seed(n + nk)
    q = torch.randn(1, 2, n, 128, device="cuda").to(torch.bfloat16)
    k = torch.randn(1, 2, nk, 128, device="cuda").to(torch.bfloat16)
    v = torch.randn(1, 2, nk, 128, device="cuda").to(torch.bfloat16)
    rows = 2 * ((n + 127) // 128)
    ids, w = _random_plan(rows, samples, nk // 4, seed=n)
    o_row, l_row = _run("kv", q, k, v, ids, w)
    o_t, l_t = _run("kv4t", q, k, kv4_transpose(v), ids, w, kv4t=True)
    assert torch.equal(o_row.view(torch.int16), o_t.view(torch.int16))
    assert torch.equal(l_row.view(torch.int32), l_t.view(torch.int32))
    assert torch.isfinite(o_t.float()).all()


def test_kv4t_prefill_ordered_bit_identical():
    print("kv4t prefill ordered n=1024", flush=True)
    torch.manual_seed(7)
    n = 1024
    q, k, v = (torch.randn(1, 2, n, 128, device="cuda").to(torch.bfloat16) for _ in range(3))
    order = torch.randperm(n, generator=torch.Generator().manual_seed(3)).to(torch.int32).cuda()
    rows = 2 * (n // 128)
    ids, w = _random_plan(rows, 64, n // 4, seed=11)
    o_row, l_row = _run("ordered", q, k, v, ids, w, order=order)
    o_t, l_t = _run("kv4t", q, k, kv4_transpose(v), ids, w, order=order, kv4t=True)
    assert torch.equal(o_row.view(torch.int16), o_t.view(torch.int16))
    assert torch.equal(l_row.view(torch.int32), l_t.view(torch.int32))
