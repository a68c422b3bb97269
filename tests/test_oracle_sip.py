"""Pins for the oracle's SIP restatement (csrc/sip.cu:33-167), CPU only.

- K1/K2: hand-derived known answers from the reference algorithm.
- K3: constant keys at the c0 geometry make every block mass exactly 2^-9,
  which fixes the whole IBCS -> SIP chain in closed form.
- Madow's systematic sampling includes block j with probability pi_j: a fine
  sweep of the uniform u reproduces pi_j.
- Exact rational systematic sampling on small rows (away from rounding ties).
- An independent pure-Python restatement with CUB's association order agrees
  bit for bit with the C oracle on random rows, including certainty.
"""
from fractions import Fraction

import numpy as np
import pytest


def test_k1_uniform(oracle_mod):
    ids, w = oracle_mod.sip(np.ones((1, 8), np.float32), np.array([0.25], np.float32), 2)
    assert ids.tolist() == [[1, 5]]
    assert w.tolist() == [[2.0, 2.0]]


def test_k2_certainty(oracle_mod):
    scores = np.array([[10, 1, 1, 1, 1, 1, 1, 1]], np.float32)
    ids, w = oracle_mod.sip(scores, np.array([0.5], np.float32), 2)
    assert ids.tolist() == [[0, 4]]
    assert w[0, 0] == 0.0
    assert w[0, 1] == np.float32(np.log2(7.0))


def test_k3_constant_keys(oracle_mod):
    """Constant K: every pair-LSE equal -> m_j = 2^-9 (fb = 512), pi = 1/8,
    ids[s] = 8s + floor(8u), weights 3.0."""
    import torch

    torch.manual_seed(0)
    n, bh = 2048, 2
    q = torch.randn(bh, n, 128).to(torch.bfloat16)
    k = torch.full((bh, n, 128), 0.25).to(torch.bfloat16)
    scores = oracle_mod.ibcs(oracle_mod.bf16_bits(q), oracle_mod.bf16_bits(k), bh, n)
    assert np.all(scores == np.float32(2.0 ** -9))
    u = np.array([0.0, 0.1, 0.5, 0.99], np.float32).repeat(8)[: scores.shape[0]]
    ids, w = oracle_mod.sip(scores, u, 64)
    for r in range(scores.shape[0]):
        expect = [8 * s + int(np.floor(8 * np.float64(u[r]))) for s in range(64)]
        assert ids[r].tolist() == expect
    assert np.all(w == 3.0)


def _pi(x: np.ndarray, samples: int) -> np.ndarray:
    """Inclusion probabilities min(1, tau*m) with sum S (certainty iteration)."""
    x = np.maximum(x.astype(np.float64), 1e-30)
    cert = np.zeros(len(x), bool)
    while True:
        scale = (samples - cert.sum()) / x[~cert].sum()
        new = (~cert) & (x * scale >= 1)
        if not new.any():
            break
        cert |= new
    return np.where(cert, 1.0, x * scale)


@pytest.mark.parametrize("peaky", [False, True])
def test_madow_inclusion_frequencies(oracle_mod, peaky):
    rng = np.random.default_rng(3 + peaky)
    pop, samples, grid = 40, 7, 4000
    m = rng.gamma(0.8, size=pop)
    if peaky:
        m[[3, 17]] *= 40
    m = (m / m.sum()).astype(np.float32)
    pi = _pi(m, samples)
    assert abs(pi.sum() - samples) < 1e-9
    u = ((np.arange(grid) + 0.5) / grid).astype(np.float32)
    ids, w = oracle_mod.sip(np.tile(m, (grid, 1)), u, samples)
    freq = np.bincount(ids.ravel(), minlength=pop) / grid
    np.testing.assert_allclose(freq, pi, atol=2.0 / grid + 1e-6)
    # weight = log2(1/pi) for every sampled block
    np.testing.assert_allclose(w, -np.log2(pi[ids]), rtol=0, atol=2e-6)


def _exact_systematic(masses, u: Fraction, samples: int):
    """Madow systematic sampling in exact rationals (no certainty case)."""
    x = [Fraction(float(max(v, np.float32(1e-30)))) for v in masses]
    total = sum(x)
    scale = Fraction(samples) / total
    cum, out, j = Fraction(0), [], 0
    for s in range(samples):
        th = u + s
        while cum + x[j] * scale <= th:
            cum += x[j] * scale
            j += 1
        out.append(j)
    return out


def test_exact_rational_brute_force(oracle_mod):
    rng = np.random.default_rng(7)
    checked = 0
    for trial in range(60):
        pop = int(rng.integers(9, 70))
        samples = int(rng.integers(1, pop // 3 + 1))
        m = (rng.random(pop) + 0.05).astype(np.float32)
        if (m.astype(np.float64) * samples / m.astype(np.float64).sum()).max() >= 1:
            continue  # certainty: covered by the other tests
        u = np.float32(rng.random())
        ids, _ = oracle_mod.sip(m[None], np.array([u], np.float32), samples)
        exact = _exact_systematic(m, Fraction(float(u)), samples)
        assert ids[0].tolist() == exact, (trial, pop, samples)
        checked += 1
    assert checked > 30


def _tree32(p):
    p = list(p)
    off = 1
    while off < 32:
        for i in range(0, 32 - off, 2 * off):
            p[i] = p[i] + p[i + off]
        off *= 2
    return p[0]


def _python_sip(scores: np.ndarray, u: float, samples: int):
    """Second, independent restatement of sip.cu:33-167 (CUB order explicit)."""
    T = 256
    pop = len(scores)
    nb = (pop + 3) // 4
    vals = [float(np.maximum(np.float32(v), np.float32(1e-30))) for v in scores]
    cert = [False] * pop
    certainty = 0
    while True:
        part = [0.0] * T
        mx = 0.0
        for t in range(T):
            for i in range(t, pop, T):
                if not cert[i]:
                    part[t] = part[t] + vals[i]
                    mx = max(mx, vals[i])
        total = None
        for w in range(8):
            g = _tree32(part[32 * w:32 * w + 32])
            total = g if total is None else total + g
        scale = float(samples - certainty) / total
        added = 0
        if mx * scale >= 1.0:
            for i in range(pop):
                if not cert[i] and vals[i] * scale >= 1.0:
                    cert[i] = True
                    added += 1
        certainty += added
        if added == 0:
            break
    chunk = ((nb + T - 1) // T) * 4
    last = max(i for i in range(pop) if not cert[i])
    ids = [i for i in range(pop) if cert[i]]
    w = [0.0] * len(ids)
    cm = []
    for t in range(T):
        acc = 0.0
        for i in range(t * chunk, min(t * chunk + chunk, pop)):
            acc = acc + (0.0 if cert[i] else vals[i] * scale)
        cm.append(acc)
    raking = []
    for r in range(32):
        acc = cm[8 * r]
        for i in range(1, 8):
            acc = acc + cm[8 * r + i]
        raking.append(acc)
    inc = raking[:]
    off = 1
    while off < 32:
        inc = [inc[r - off] + inc[r] if r >= off else inc[r] for r in range(32)]
        off *= 2
    base = []
    for r in range(32):
        ex = 0.0 if r == 0 else 0.0 + inc[r - 1]
        for i in range(8):
            base.append(ex)
            ex = ex + cm[8 * r + i]
    residuals = samples - certainty
    prefix = [0.0] * (nb + 1)
    prefix[nb] = float(residuals)
    for t in range(T):
        c = base[t]
        for i in range(t * chunk, min(t * chunk + chunk, pop)):
            if i % 4 == 0:
                prefix[i // 4] = float(residuals) if i > last else c
            c = c + (0.0 if cert[i] else vals[i] * scale)
    for slot in range(residuals):
        th = float(np.float32(u)) + slot
        lo, hi = 0, nb
        while lo < hi:
            mid = (lo + hi + 1) // 2
            if prefix[mid] <= th:
                lo = mid
            else:
                hi = mid - 1
        b = min(lo, nb - 1)
        mass = prefix[b]
        sel = last
        for i in range(4 * b, min(4 * b + 4, pop)):
            if cert[i]:
                continue
            sel = i
            mass = float(np.fma(vals[i], scale, mass)) if hasattr(np, "fma") else _fma(vals[i], scale, mass)
            if mass > th:
                break
        ids.append(sel)
        w.append(float(np.float32(-np.log2(max(float(np.float32(scores[sel])), 1e-30) * scale))))
    return ids, w


def _fma(a: float, b: float, c: float) -> float:
    """Correctly rounded a*b+c via exact rationals."""
    return float(Fraction(a) * Fraction(b) + Fraction(c))


@pytest.mark.parametrize("seed,pop,samples,peak", [(0, 300, 40, 0.0), (1, 1030, 200, 30.0), (2, 517, 500, 0.0)])
def test_independent_python_restatement(oracle_mod, seed, pop, samples, peak):
    rng = np.random.default_rng(seed)
    m = rng.gamma(0.4, size=pop)
    if peak:
        m[rng.integers(0, pop, 6)] *= peak
    m = (m / m.sum()).astype(np.float32)
    u = np.float32(rng.random())
    ids_c, w_c = oracle_mod.sip(m[None], np.array([u], np.float32), samples)
    ids_p, w_p = _python_sip(m, float(u), samples)
    assert ids_c[0].tolist() == ids_p
    assert np.array_equal(w_c[0].view(np.uint32), np.array(w_p, np.float32).view(np.uint32))


def test_invariants(oracle_mod):
    rng = np.random.default_rng(11)
    pop, samples, rows = 2000, 256, 16
    m = rng.gamma(0.3, size=(rows, pop))
    m[:, rng.integers(0, pop, 10)] *= 50
    m = (m / m.sum(axis=1, keepdims=True)).astype(np.float32)
    u = rng.random(rows).astype(np.float32)
    ids, w = oracle_mod.sip(m, u, samples)
    for r in range(rows):
        pi = _pi(m[r], samples)
        cert = np.flatnonzero(pi >= 1.0)
        c = len(cert)
        assert ids[r, :c].tolist() == cert.tolist()  # certain first, ascending
        assert np.all(w[r, :c] == 0.0)
        assert len(set(ids[r].tolist())) == samples  # without replacement
        assert np.all(np.diff(ids[r, c:]) > 0)  # draws in increasing order
        assert np.all(w[r] >= 0.0)


def test_rejects_bad_sizes(oracle_mod):
    with pytest.raises(ValueError):
        oracle_mod.sip(np.ones((1, 8), np.float32), np.zeros(1, np.float32), 8)
