"""Writes tests/golden/c0_head0.npz: a small fixture at the reference geometry.

Inputs: head 0 of the configuration-0 synthetic generator (seed 1000), first
1,024 tokens (8 query blocks, 256 KV4 blocks), bf16 Q/K/V, plus the parity
uniforms torch.rand(8, generator=cpu_gen(42)) and sample_pages = 2 (64 KV4
blocks per row). Outputs: every stage of the CPU oracle (centroids,
populations, pooled keys, pair-LSEs, normalisers, masses, SIP ids/weights)
and the exact weighted prefill output and base-2 LSE.

Run from the repository root: python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path[:0] = [ROOT, os.path.join(ROOT, "ab-attention_amd")]

import oracle  # noqa: E402
from ab_attention.synthetic import CONFIGS, make_qkv, parity_offsets  # noqa: E402

N, PAGES = 1024, 2


def main():
    oracle.build()
    q, k, v = make_qkv(CONFIGS[0], heads=[0], dtype=torch.bfloat16)
    q, k, v = (t[0, :, :N].contiguous() for t in (q, k, v))  # [1, N, 128]
    qb, kb, vb = (oracle.bf16_bits(t) for t in (q, k, v))
    cent, pops = oracle.cluster(qb, 1, N)
    pooled = oracle.pool(kb, 1, N)
    lse, mx, den = oracle.lse(cent, pooled, 1, N)
    rows, fb = cent.shape[0], N // 4
    scores = oracle.masses(lse, pops, mx, den, rows, fb)
    assert np.array_equal(scores, oracle.ibcs(qb, kb, 1, N))
    offsets = parity_offsets(rows).numpy()
    ids, logw = oracle.sip(scores, offsets, PAGES * 32)
    f32 = lambda b: oracle.bits_to_f32(b).reshape(1, N, 128)
    out, lse2 = oracle.prefill(f32(qb), f32(kb), f32(vb), ids, logw)
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "c0_head0.npz")
    np.savez_compressed(path, q=qb, k=kb, v=vb, offsets=offsets, sample_pages=np.int32(PAGES),
                        centroids=cent, populations=pops, pooled=pooled, lse=lse, lse_max=mx, lse_den=den,
                        scores=scores, ids=ids, log_weights=logw, out=out, out_lse=lse2)
    print(path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
