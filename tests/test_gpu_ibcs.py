"""IBCS stages on the GPU against the oracle (csrc/ibcs.cu:106-538).

cluster/pool are bit-exact (same fp32 operation order, IEEE division).
The pair-LSE stage differs from the oracle only through the MFMA dot-product
accumulation order and the hardware exp2/log2, so fp16 LSEs may differ by one
fp16 ulp on a small fraction of entries; masses given identical LSEs differ
only by exp2 rounding.
"""
import numpy as np
import pytest
import torch

from ab_attention import _C, _lib
from ab_attention.synthetic import CONFIGS, make_qkv

pytestmark = pytest.mark.gpu


def _bits(t):
    return np.ascontiguousarray(t.cpu().contiguous().view(torch.int16).numpy().view(np.uint16))


def _ordered(bits16: np.ndarray) -> np.ndarray:
    """fp16 bit patterns -> integers whose differences count ulps across zero."""
    b = bits16.astype(np.int32)
    return np.where(b & 0x8000, -(b & 0x7FFF), b)


def _stages_gpu(native, q, k):
    bh, n = q.shape[0] * q.shape[1], q.shape[2]
    qb, fb = -(-n // 128), n // 4
    rows = bh * qb
    dev = q.device
    cent = torch.empty((rows, 8, 128), dtype=torch.bfloat16, device=dev)
    pops = torch.empty((rows, 8), dtype=torch.float32, device=dev)
    pooled = torch.empty((bh, fb, 2, 128), dtype=torch.bfloat16, device=dev)
    s = _lib.stream(dev)
    _lib.check(native.ab_ibcs_cluster_pool(_lib.ptr(q), _lib.ptr(k), bh, n, _lib.ptr(cent), _lib.ptr(pops),
                                           _lib.ptr(pooled), s))
    ld = native.ab_ibcs_lse_stride(n)
    lse = torch.empty((rows, 8, ld), dtype=torch.float16, device=dev)
    mx = torch.empty((rows, 8), dtype=torch.float32, device=dev)
    den = torch.empty((rows, 8), dtype=torch.float32, device=dev)
    _lib.check(native.ab_ibcs_lse(_lib.ptr(cent), _lib.ptr(pooled), bh, n, _lib.ptr(lse), _lib.ptr(mx),
                                  _lib.ptr(den), s))
    torch.cuda.synchronize()
    return cent, pops, pooled, lse[:, :, :fb], mx, den


def _inputs(cfg_id, heads, n=None):
    cfg = CONFIGS[cfg_id]
    q, k, _ = make_qkv(cfg, heads=heads, dtype=torch.bfloat16)
    if n is not None:
        q, k = q[:, :, :n].contiguous(), k[:, :, :n].contiguous()
    return q, k


# Last query blocks of 80 (n = 2000), 68, 64, 20 and 4 queries: the two
# 64-query halves of a block are staged and summed separately, so blocks whose
# second half is partly filled, empty, or whose first half is partial are
# each a case.
@pytest.mark.parametrize("cfg_id,heads,n", [(0, None, None), (0, None, 2000), (0, None, 1988), (0, None, 1984),
                                            (0, None, 1940), (0, None, 1924), (1, [0], None)])
def test_cluster_pool_bit_exact(native, oracle_mod, cfg_id, heads, n):
    q, k = _inputs(cfg_id, heads, n)
    print(f"cluster/pool cfg={cfg_id} shape={tuple(q.shape)}", flush=True)
    bh, n = q.shape[0] * q.shape[1], q.shape[2]
    cent, pops, pooled, *_ = _stages_gpu(native, q.cuda(), k.cuda())
    qbits = _bits(q).reshape(bh, n, 128)
    kbits = _bits(k).reshape(bh, n, 128)
    cent_o, pops_o = oracle_mod.cluster(qbits, bh, n)
    pooled_o = oracle_mod.pool(kbits, bh, n)
    np.testing.assert_array_equal(pops.cpu().numpy(), pops_o)
    np.testing.assert_array_equal(_bits(cent).reshape(cent_o.shape), cent_o)
    np.testing.assert_array_equal(_bits(pooled).reshape(pooled_o.shape), pooled_o)


@pytest.mark.parametrize("cfg_id,heads,n", [(0, None, None), (0, None, 2000), (1, [5], None)])
def test_lse_stage(native, oracle_mod, cfg_id, heads, n):
    q, k = _inputs(cfg_id, heads, n)
    print(f"lse cfg={cfg_id} shape={tuple(q.shape)}", flush=True)
    bh, n = q.shape[0] * q.shape[1], q.shape[2]
    cent, pops, pooled, lse, mx, den = _stages_gpu(native, q.cuda(), k.cuda())
    lse_o, mx_o, den_o = oracle_mod.lse(_bits(cent).reshape(-1, 8, 128), _bits(pooled).reshape(bh, -1, 2, 128),
                                        bh, n)
    ulps = np.abs(_ordered(_bits(lse).reshape(lse_o.shape)) - _ordered(lse_o))
    assert ulps.max() <= 1, f"pair-LSE off by {ulps.max()} fp16 ulps"
    assert (ulps > 0).mean() < 2e-3, f"{(ulps > 0).mean():.2e} of pair-LSEs differ"
    # the max of fp16 values is exact up to those one-ulp flips
    np.testing.assert_allclose(mx.cpu().numpy(), mx_o, rtol=1e-3, atol=2e-2)
    rel = np.abs(den.cpu().numpy() - den_o) / den_o
    assert np.median(rel) < 1e-5 and rel.max() < 2e-2, (np.median(rel), rel.max())


@pytest.mark.parametrize("cfg_id,heads", [(0, None), (1, [3])])
def test_masses_stage(native, oracle_mod, cfg_id, heads):
    """Given the oracle's LSEs and normalisers, masses differ only by exp2 rounding."""
    q, k = _inputs(cfg_id, heads)
    bh, n = q.shape[0] * q.shape[1], q.shape[2]
    qb, fb = -(-n // 128), n // 4
    rows = bh * qb
    qbits, kbits = _bits(q).reshape(bh, n, 128), _bits(k).reshape(bh, n, 128)
    cent_o, pops_o = oracle_mod.cluster(qbits, bh, n)
    lse_o, mx_o, den_o = oracle_mod.lse(cent_o, oracle_mod.pool(kbits, bh, n), bh, n)
    m_o = oracle_mod.masses(lse_o, pops_o, mx_o, den_o, rows, fb)
    ld = native.ab_ibcs_lse_stride(n)
    lse_pad = np.zeros((rows, 8, ld), np.uint16)
    lse_pad[:, :, :fb] = lse_o
    lse_d = torch.from_numpy(lse_pad.view(np.int16)).cuda()
    args = [torch.from_numpy(a).cuda() for a in (pops_o, mx_o, den_o)]
    scores = torch.empty((rows, fb), dtype=torch.float32, device="cuda")
    _lib.check(native.ab_ibcs_masses(_lib.ptr(lse_d), *(_lib.ptr(a) for a in args), rows, fb, _lib.ptr(scores),
                                     _lib.stream(scores.device)))
    torch.cuda.synchronize()
    np.testing.assert_allclose(scores.cpu().numpy(), m_o, rtol=2e-6, atol=1e-12)


@pytest.mark.parametrize("cfg_id,heads", [(0, None), (1, [0, 7])])
def test_ibcs_end_to_end(native, oracle_mod, cfg_id, heads):
    q, k = _inputs(cfg_id, heads)
    print(f"ibcs e2e cfg={cfg_id} shape={tuple(q.shape)}", flush=True)
    bh, n = q.shape[0] * q.shape[1], q.shape[2]
    scores = _C.ibcs(q.cuda(), k.cuda())
    torch.cuda.synchronize()
    g = scores.cpu().numpy()
    o = oracle_mod.ibcs(_bits(q).reshape(bh, n, 128), _bits(k).reshape(bh, n, 128), bh, n)
    np.testing.assert_allclose(g.sum(axis=1), 1.0, rtol=0, atol=2e-5)
    rel = np.abs(g - o) / np.maximum(o, 1e-30)
    assert np.quantile(rel, 0.99) < 1e-5, np.quantile(rel, 0.99)
    assert rel.max() < 3e-2, rel.max()
