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


def test_separate_kv_length_matches_dense_softmax(oracle_mod):
    """K/V of their own length (the text partition of video.py:129-151): all
    blocks at weight 0 is dense softmax attention of Nq queries over Nk keys;
    a -inf weight removes its block."""
    rng = np.random.default_rng(4)
    nq, nk = 200, 96
    q = rng.normal(0, 1, (1, nq, 128)).astype(np.float32)
    k = rng.normal(0, 1, (1, nk, 128)).astype(np.float32)
    v = rng.normal(0, 1, (1, nk, 128)).astype(np.float32)
    rows, fb = -(-nq // 128), nk // 4
    ids = np.tile(np.r_[np.arange(fb), [0, 0]].astype(np.int32), (rows, 1))  # two removed repeats
    logw = np.tile(np.r_[np.zeros(fb), [-np.inf, -np.inf]].astype(np.float32), (rows, 1))
    o, l = oracle_mod.prefill(q, k, v, ids, logw)
    z = q[0].astype(np.float64) @ k[0].astype(np.float64).T / np.sqrt(128)
    p = np.exp(z - z.max(1, keepdims=True))
    np.testing.assert_allclose(o[0], p @ v[0] / p.sum(1, keepdims=True), rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(l[0], (z.max(1) + np.log(p.sum(1))) / np.log(2), rtol=1e-6, atol=1e-5)


def test_merge_of_disjoint_partitions_is_attention_over_union(oracle_mod):
    """FlashInfer merge_state restated: merging the states of two disjoint
    key sets equals attention over their union (the identity that lets the
    Hunyuan text keys ride in the video prefill at weight 0)."""
    rng = np.random.default_rng(5)
    n = 384
    q, k, v = _inputs(rng, 2, n)
    rows, fb = 2 * (n // 128), n // 4
    perm = np.stack([rng.permutation(fb) for _ in range(rows)]).astype(np.int32)
    a_ids, b_ids = perm[:, :40], perm[:, 40:72]
    a_w = (rng.random((rows, 40)) * 3).astype(np.float32)
    b_w = np.zeros((rows, 32), np.float32)
    oa, la = oracle_mod.prefill(q, k, v, a_ids, a_w)
    ob, lb = oracle_mod.prefill(q, k, v, b_ids, b_w)
    om, lm = oracle_mod.merge_states(oa, la, ob, lb)
    ou, lu = oracle_mod.prefill(q, k, v, np.concatenate([a_ids, b_ids], 1), np.concatenate([a_w, b_w], 1))
    np.testing.assert_allclose(om, ou, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(lm, lu, rtol=1e-6, atol=1e-5)
    # a state merged with an empty one (lse -inf) is unchanged
    o2, l2 = oracle_mod.merge_states(oa, la, ob, np.full_like(lb, -np.inf))
    np.testing.assert_allclose(o2, oa, rtol=1e-12, atol=0)
    np.testing.assert_allclose(l2, la, rtol=1e-12, atol=0)


def test_neg_inf_weights_remove_blocks(oracle_mod):
    """A block at weight -inf contributes nothing: the row equals attention
    over its other blocks (those blocks dropped from the list). A row whose
    every block is at -inf has an empty softmax: o = 0 and lse = -inf, with
    no NaN (the convention the GPU kernel follows; no reference fixture pins
    it)."""
    rng = np.random.default_rng(5)
    n, S = 512, 16
    q, k, v = _inputs(rng, 1, n)
    rows, fb = n // 128, n // 4
    ids = rng.integers(0, fb, (rows, S)).astype(np.int32)
    logw = (rng.random((rows, S)) * 2).astype(np.float32)
    logw[0, :5] = -np.inf
    logw[1, 3::4] = -np.inf
    logw[2, :] = -np.inf
    o, l = oracle_mod.prefill(q, k, v, ids, logw)
    for r in (0, 1):
        keep = np.isfinite(logw[r])
        sub_ids = np.tile(ids[r][keep], (rows, 1))
        sub_w = np.tile(logw[r][keep], (rows, 1))
        ro, rl = _reference(q, k, v, sub_ids, sub_w)
        sl = slice(r * 128, r * 128 + 128)
        np.testing.assert_allclose(o[0, sl], ro[0, sl], rtol=1e-5, atol=1e-6)
        np.testing.assert_allclose(l[0, sl], rl[0, sl], rtol=1e-6, atol=1e-5)
    assert np.all(o[0, 256:384] == 0.0) and np.all(np.isneginf(l[0, 256:384]))
    assert np.all(np.isfinite(o[0, 384:]))
