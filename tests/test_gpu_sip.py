"""SIP on the GPU is bit-exact with the oracle (csrc/sip.cu:33-167) given the
same scores and offsets: ids and weights compared as raw bits."""
import numpy as np
import pytest
import torch

from ab_attention import _C

pytestmark = pytest.mark.gpu


def _run_gpu(scores: np.ndarray, offsets: np.ndarray, samples: int):
    s = torch.from_numpy(scores).cuda()
    o = torch.from_numpy(offsets).cuda()
    ids = torch.empty((scores.shape[0], samples), dtype=torch.int32, device="cuda")
    logw = torch.empty((scores.shape[0], samples), dtype=torch.float32, device="cuda")
    _C.sip(s, o, ids, logw)
    torch.cuda.synchronize()
    return ids.cpu().numpy(), logw.cpu().numpy()


def _assert_bit_exact(scores, offsets, samples, oracle_mod):
    print(f"sip case rows={scores.shape[0]} pop={scores.shape[1]} samples={samples}", flush=True)
    ids_g, w_g = _run_gpu(scores, offsets, samples)
    ids_o, w_o = oracle_mod.sip(scores, offsets, samples)
    bad_ids = np.argwhere(ids_g != ids_o)
    assert bad_ids.size == 0, f"ids differ at {bad_ids[:5].tolist()}"
    bad_w = np.argwhere(w_g.view(np.uint32) != w_o.view(np.uint32))
    assert bad_w.size == 0, f"weights differ at {bad_w[:5].tolist()}"
    return ids_g, w_g


def _local_masses(rng, rows, pop, peak=0.0):
    """Smooth positive masses with optional spikes (to force certainty)."""
    x = rng.gamma(0.3, size=(rows, pop)).astype(np.float64)
    if peak > 0:
        hot = rng.integers(0, pop, size=(rows, max(1, pop // 64)))
        np.put_along_axis(x, hot, x.max(axis=1, keepdims=True) * peak, axis=1)
    x /= x.sum(axis=1, keepdims=True)
    return x.astype(np.float32)


def test_known_answers(oracle_mod):
    ids, w = _assert_bit_exact(np.ones((1, 8), np.float32), np.array([0.25], np.float32), 2, oracle_mod)
    assert ids.tolist() == [[1, 5]] and w.tolist() == [[2.0, 2.0]]
    ids, w = _assert_bit_exact(np.array([[10, 1, 1, 1, 1, 1, 1, 1]], np.float32),
                               np.array([0.5], np.float32), 2, oracle_mod)
    assert ids.tolist() == [[0, 4]]
    assert w[0, 0] == 0.0 and w[0, 1] == np.float32(np.log2(7.0))


@pytest.mark.parametrize("pop,samples,peak", [
    (512, 64, 0.0), (512, 64, 50.0), (513, 100, 0.0), (1001, 999, 0.0), (8190, 2048, 0.0),
    (8190, 2048, 20.0), (18900, 2048, 0.0), (18900, 2048, 200.0),
])
def test_random_rows(pop, samples, peak, oracle_mod):
    rng = np.random.default_rng(pop * 7 + samples)
    rows = 48
    scores = _local_masses(rng, rows, pop, peak)
    offsets = rng.random(rows, dtype=np.float32)
    _assert_bit_exact(scores, offsets, samples, oracle_mod)


def test_global_row_path(oracle_mod):
    """Hunyuan-size population (29,700 KV4 blocks) exceeds LDS for the
    in-LDS row copy and runs the global-memory row path."""
    rng = np.random.default_rng(3)
    scores = _local_masses(rng, 16, 29700, 30.0)
    offsets = rng.random(16, dtype=np.float32)
    _assert_bit_exact(scores, offsets, 2272, oracle_mod)


def test_degenerate_rows(oracle_mod):
    """Zeros (clamped to 1e-30), tiny and huge masses, one dominant block."""
    rng = np.random.default_rng(11)
    pop = 600
    rows = [np.zeros(pop), np.full(pop, 1e-38), rng.random(pop) * 1e-35,
            np.r_[1e6, np.ones(pop - 1)], np.r_[np.zeros(pop - 5), np.ones(5)]]
    scores = np.stack(rows).astype(np.float32)
    offsets = np.array([0.0, 0.999999, 0.5, 0.25, 0.75], np.float32)
    _assert_bit_exact(scores, offsets, 7, oracle_mod)
    _assert_bit_exact(scores, offsets, 599, oracle_mod)
