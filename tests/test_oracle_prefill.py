"""Pins for the oracle's weighted prefill (ab_attention/flashinfer_backend.py:30-59), CPU only.

- equals softmax attention over the gathered keys with additive logit bias
  w * ln 2, computed independently in fp64 with numpy;
- every block with weight 0 (all KV4 blocks listed once) is dense attention;
- a uniform weight c leaves the output unchanged and shifts the base-2 LSE by c;
- repeated ids count once per listing.
"""
import numpy as np


def _reference(q, k, v, ids, logw):
    bh, n, d = q.shape
    qb = -(-n // 128)
    out = np.empty((bh, n, d))
    lse = np.empty((bh, n))
    for h in range(bh):
        for blk in range(qb):
            row = h * qb + blk
            keys = (4 * ids[row][:, None] + np.arange(4)[None]).ravel()
            bias = np.repeat(logw[row].astype(np.float64), 4) * np.log(2.0)
            qq = q[h, blk * 128:min(n, blk * 128 + 128)].astype(np.float64)
            z = qq @ k[h, keys].astype(np.float64).T / np.sqrt(d) + bias
            m = z.max(1, keepdims=True)
            p = np.exp(z - m)
            out[h, blk * 128:blk * 128 + len(qq)] = (p @ v[h, keys].astype(np.float64)) / p.sum(1, keepdims=True)
            lse[h, blk * 128:blk * 128 + len(qq)] = (m[:, 0] + np.log(p.sum(1))) / np.log(2.0)
    return out, lse


def _inputs(rng, bh, n):
    q = rng.normal(0, 1, (bh, n, 128)).astype(np.float32)
    k = rng.normal(0, 1, (bh, n, 128)).astype(np.float32)
    v = rng.normal(0, 1, (bh, n, 128)).astype(np.float32)
    return q, k, v


def test_matches_softmax_with_bias(oracle_mod):
    rng = np.random.default_rng(0)
    bh, n, S = 2, 520, 40
    q, k, v = _inputs(rng, bh, n)
    rows, fb = bh * -(-n // 128), n // 4
    ids = rng.integers(0, fb, (rows, S)).astype(np.int32)
    logw = (rng.random((rows, S)) * 5).astype(np.float32)
    o, l = oracle_mod.prefill(q, k, v, ids, logw)
    ro, rl = _reference(q, k, v, ids, logw)
    np.testing.assert_allclose(o, ro, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(l, rl, rtol=1e-6, atol=1e-5)


def test_all_blocks_zero_weight_is_dense(oracle_mod):
    rng = np.random.default_rng(1)
    n = 256
    q, k, v = _inputs(rng, 1, n)
    rows, fb = n // 128, n // 4
    ids = np.tile(np.arange(fb, dtype=np.int32), (rows, 1))
    o, l = oracle_mod.prefill(q, k, v, ids, np.zeros((rows, fb), np.float32))
    z = q[0].astype(np.float64) @ k[0].astype(np.float64).T / np.sqrt(128)
    p = np.exp(z - z.max(1, keepdims=True))
    dense = p @ v[0] / p.sum(1, keepdims=True)
    np.testing.assert_allclose(o[0], dense, rtol=1e-5, atol=1e-6)
    lse2 = (z.max(1) + np.log(p.sum(1))) / np.log(2)
    np.testing.assert_allclose(l[0], lse2, rtol=1e-6, atol=1e-5)


def test_uniform_weight_shift(oracle_mod):
    rng = np.random.default_rng(2)
    n, S = 384, 24
    q, k, v = _inputs(rng, 1, n)
    rows, fb = n // 128, n // 4
    ids = rng.integers(0, fb, (rows, S)).astype(np.int32)
    o0, l0 = oracle_mod.prefill(q, k, v, ids, np.zeros((rows, S), np.float32))
    o1, l1 = oracle_mod.prefill(q, k, v, ids, np.full((rows, S), 2.5, np.float32))
    np.testing.assert_allclose(o1, o0, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(l1, l0 + 2.5, rtol=0, atol=1e-5)


def test_duplicate_ids_count_twice(oracle_mod):
    rng = np.random.default_rng(3)
    n = 128
    q, k, v = _inputs(rng, 1, n)
    ids_dup = np.array([[5, 5, 9]], np.int32)
    ids_w = np.array([[5, 9]], np.int32)
    o_dup, l_dup = oracle_mod.prefill(q, k, v, ids_dup, np.zeros((1, 3), np.float32))
    o_w, l_w = oracle_mod.prefill(q, k, v, ids_w, np.array([[1.0, 0.0]], np.float32))  # 2^1 = twice
    np.testing.assert_allclose(o_dup, o_w, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(l_dup, l_w, rtol=1e-6, atol=1e-5)


def test_row_subset(oracle_mod):
    rng = np.random.default_rng(4)
    n, S = 512, 16
    q, k, v = _inputs(rng, 1, n)
    ids = rng.integers(0, n // 4, (4, S)).astype(np.int32)
    w = rng.random((4, S)).astype(np.float32)
    full, lf = oracle_mod.prefill(q, k, v, ids, w)
    sub, ls = oracle_mod.prefill(q, k, v, ids, w, rows=[2])
    np.testing.assert_array_equal(sub[0, 256:384], full[0, 256:384])
    assert np.isnan(sub[0, :256]).all()
