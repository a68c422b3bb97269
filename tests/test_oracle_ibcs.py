"""Pins for the oracle's IBCS restatement (csrc/ibcs.cu:106-538), CPU only.

- Number formats: fp16 / bf16 round-to-nearest-even against numpy.
- Pooling: closed form bf16(0.5 * (k_2r + k_2r+1)).
- Clustering: populations sum to the block size; every centroid is the bf16
  mean of its members (rescaled); every query sits with its nearest centre;
  identical rows form one cluster; a brute-force fp64 farthest-first
  clustering of well-separated blocks gives the same partition.
- Masses: fp64 closed form of the population-weighted centroid softmax over
  fp16-rounded pair-LSEs; rows sum to 1; constant keys give 1/fb.
"""
import math

import numpy as np
import pytest
import torch

QK = float(np.float32(math.pow(128.0, -0.5) * 1.4426950408889634))


def _bf16_round(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 -> float32 with round to nearest even (torch's cast)."""
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(torch.bfloat16).float().numpy()


@pytest.mark.filterwarnings("ignore:overflow")
def test_fp16_conversion_matches_numpy(oracle_mod):
    rng = np.random.default_rng(0)
    vals = np.concatenate([
        rng.normal(0, 30, 2000), rng.normal(0, 1e-5, 500), rng.normal(0, 1e-7, 200),
        [0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e6, -1e6, 2 ** -24, 2 ** -25, 3 * 2 ** -26, 6.1e-5],
    ]).astype(np.float32)
    for v in vals:
        got = oracle_mod.f32_to_f16_bits(float(v))
        assert got == int(np.float16(v).view(np.uint16)), v
        assert oracle_mod.f16_bits_to_f32(got) == np.float32(np.float16(v)), v


def test_bf16_conversion_matches_torch(oracle_mod):
    rng = np.random.default_rng(1)
    vals = np.concatenate([rng.normal(0, 10, 3000), rng.normal(0, 1e-30, 100)]).astype(np.float32)
    ref = torch.from_numpy(vals).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    got = np.array([oracle_mod.f32_to_bf16_bits(float(v)) for v in vals], np.uint16)
    np.testing.assert_array_equal(got, ref)


def test_pool_closed_form(oracle_mod):
    torch.manual_seed(2)
    bh, n = 2, 64
    k = torch.randn(bh, n, 128).to(torch.bfloat16)
    out = oracle_mod.pool(oracle_mod.bf16_bits(k), bh, n)
    kf = k.float().numpy().reshape(bh, n // 2, 2, 128)
    expect = _bf16_round(np.float32(0.5) * (kf[:, :, 0] + kf[:, :, 1]))
    got = oracle_mod.bits_to_f32(out).reshape(bh, n // 2, 128)
    np.testing.assert_array_equal(got, expect)


@pytest.mark.parametrize("n", [2048, 2000])
def test_cluster_invariants(oracle_mod, n):
    """Populations cover the block (ragged last block included); empty
    clusters have zero centroids; every bf16 centroid lies inside the
    bounding box of the block scaled by 128^-0.5 * log2(e)."""
    torch.manual_seed(3)
    q = torch.randn(1, n, 128).to(torch.bfloat16)
    bits = oracle_mod.bf16_bits(q).reshape(1, n, 128)
    cent, pops = oracle_mod.cluster(bits, 1, n)
    xall = oracle_mod.bits_to_f32(bits[0])
    for blk in range(-(-n // 128)):
        x = xall[blk * 128:min(n, blk * 128 + 128)]
        assert pops[blk].sum() == x.shape[0]
        c = oracle_mod.bits_to_f32(cent[blk])
        assert np.all(c[pops[blk] == 0] == 0.0)
        lo, hi = x.min(0) * QK, x.max(0) * QK
        live = pops[blk] > 0
        assert np.all(c[live] >= lo - 1e-2) and np.all(c[live] <= hi + 1e-2)


def _farthest_first_fp64(x: np.ndarray, k: int = 8):
    """Brute-force farthest-first clustering in fp64 (ibcs.cu:130-197)."""
    mean = x.mean(0)
    d0 = ((x - mean) ** 2).sum(1)
    center = int(np.argmax(d0))
    mind = np.full(len(x), np.inf)
    assign = np.zeros(len(x), int)
    for s in range(k):
        dist = ((x - x[center]) ** 2).sum(1)
        better = dist < mind
        mind[better] = dist[better]
        assign[better] = s
        if s + 1 < k:
            center = int(np.argmax(mind))
    return assign


def test_cluster_matches_fp64_farthest_first(oracle_mod):
    """Eight well-separated blobs: the oracle's partition, populations and
    centroids equal the brute-force fp64 farthest-first result."""
    rng = np.random.default_rng(4)
    centers = rng.normal(0, 8, (8, 128))
    lab = rng.integers(0, 8, 128)
    x = centers[lab] + rng.normal(0, 0.05, (128, 128))
    xb = _bf16_round(x.astype(np.float32))
    bits = torch.from_numpy(xb).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16).reshape(1, 128, 128)
    cent, pops = oracle_mod.cluster(np.ascontiguousarray(bits), 1, 128)
    assign = _farthest_first_fp64(xb.astype(np.float64))
    np.testing.assert_array_equal(pops[0], np.bincount(assign, minlength=8).astype(np.float32))
    for s in range(8):
        members = xb[assign == s]
        acc = np.zeros(128, np.float32)
        for row in members:  # row-order fp32 sum, as the reference
            acc = (acc + row).astype(np.float32)
        mean = _bf16_round(acc / np.float32(len(members)))
        expect = _bf16_round(mean * np.float32(QK))
        np.testing.assert_array_equal(oracle_mod.bits_to_f32(cent[0, s]), expect)


def test_cluster_identical_rows(oracle_mod):
    row = _bf16_round(np.random.default_rng(5).normal(0, 1, 128).astype(np.float32))
    x = np.tile(row, (128, 1))
    bits = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16).reshape(1, 128, 128)
    cent, pops = oracle_mod.cluster(np.ascontiguousarray(bits), 1, 128)
    assert pops[0].tolist() == [128.0] + [0.0] * 7
    np.testing.assert_array_equal(oracle_mod.bits_to_f32(cent[0, 0]), _bf16_round(row * np.float32(QK)))
    assert np.all(oracle_mod.bits_to_f32(cent[0, 1:]) == 0)


def _masses_fp64(cent_bits, pops, pooled_bits, oracle_mod):
    """Closed form: m_j = sum_s n_s 2^{l_sj} / sum_j' 2^{l_sj'} / sum_s n_s with
    l_sj = fp16(log2(2^{t0+1} + 2^{t1+1})), t = centroid . pooled rep."""
    c = oracle_mod.bits_to_f32(cent_bits).astype(np.float64)  # [rows, 8, 128]
    r = oracle_mod.bits_to_f32(pooled_bits).astype(np.float64)  # [fb, 2, 128]
    t = np.einsum("rsd,jkd->rsjk", c, r).astype(np.float32)
    a = t[..., 0] + np.float32(1.0)
    b = t[..., 1] + np.float32(1.0)
    mx = np.maximum(a, b)
    lexact = mx.astype(np.float64) + np.log2(np.exp2((a - mx).astype(np.float64)) + np.exp2((b - mx).astype(np.float64)))
    l16 = lexact.astype(np.float32).astype(np.float16).astype(np.float64)
    p = np.exp2(l16 - l16.max(axis=2, keepdims=True))
    p /= p.sum(axis=2, keepdims=True)
    return (pops[:, :, None] * p).sum(1) / pops.sum(1, keepdims=True)


def test_masses_closed_form(oracle_mod):
    torch.manual_seed(6)
    n, bh = 512, 1
    q = (torch.randn(bh, n, 128) * 0.5).to(torch.bfloat16)
    k = (torch.randn(bh, n, 128) * 0.5).to(torch.bfloat16)
    qb, kb = oracle_mod.bf16_bits(q), oracle_mod.bf16_bits(k)
    cent, pops = oracle_mod.cluster(qb, bh, n)
    pooled = oracle_mod.pool(kb, bh, n)
    got = oracle_mod.ibcs(qb, kb, bh, n)
    expect = _masses_fp64(cent, pops, pooled[0], oracle_mod)
    np.testing.assert_allclose(got, expect, rtol=2e-5, atol=1e-12)
    np.testing.assert_allclose(got.sum(1), 1.0, atol=1e-5)


def test_constant_keys_uniform(oracle_mod):
    torch.manual_seed(7)
    n = 1024
    q = torch.randn(1, n, 128).to(torch.bfloat16)
    k = torch.full((1, n, 128), -0.75).to(torch.bfloat16)
    got = oracle_mod.ibcs(oracle_mod.bf16_bits(q), oracle_mod.bf16_bits(k), 1, n)
    assert np.all(got == np.float32(1.0 / (n // 4)))


def test_lse_rows_matches_per_head(oracle_mod):
    torch.manual_seed(8)
    n = 512
    q = torch.randn(1, n, 128).to(torch.bfloat16)
    k = torch.randn(1, n, 128).to(torch.bfloat16)
    cent, pops = oracle_mod.cluster(oracle_mod.bf16_bits(q), 1, n)
    pooled = oracle_mod.pool(oracle_mod.bf16_bits(k), 1, n)
    a = oracle_mod.lse(cent, pooled, 1, n)
    b = oracle_mod.lse_rows(cent[1:3], pooled[0])
    np.testing.assert_array_equal(a[0][1:3], b[0])
    np.testing.assert_array_equal(a[1][1:3], b[1])
    np.testing.assert_array_equal(a[2][1:3], b[2])
