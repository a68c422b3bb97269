"""bench.py on the CPU: the work figures its roofline divides by, and the
one-GPU contract (no GPU is touched here)."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402


@pytest.mark.parametrize("bh, n, samples", [(80, 75600, 2048), (24, 32760, 2048), (24, 119056, 2272), (2, 2048, 64)])
def test_prefill_work_from_the_attention_definition(bh, n, samples):
    """F_pre counted query by query: each valid or padded query of a 128-query
    row attends to 4 keys per listed block, at 2*d FLOP for q.k and 2*d for
    p*v (d = 128)."""
    rows, fb, f_pre, _ = bench.work_figures(bh, n, samples)
    blocks_per_head = -(-n // 128)
    assert rows == bh * blocks_per_head and fb == n // 4
    queries = rows * 128
    keys_per_query = 4 * samples
    assert f_pre == queries * keys_per_query * (2 * 128 + 2 * 128)


def test_headline_figures():
    """c2 (Wan2.1-14B 720p, B=2, H=40): the figures the bench line and the
    committed profiles quote."""
    rows, fb, f_pre, b_sel = bench.work_figures(80, 75600, 2048)
    assert (rows, fb) == (47280, 18900)
    assert round(f_pre / 1e12, 3) == 25.383
    # The pair-LSEs dominate the reference dataflow: 8 centroids x fp16,
    # written once and read once, per (row, KV4 block).
    assert 2 * 16 * rows * fb / b_sel > 0.69
    assert round(b_sel / 1e9, 3) == 41.365


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""
