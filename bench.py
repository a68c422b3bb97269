"""Benchmark: one AB-attention call (build_plan + apply_plan) per step.

Default workload: Wan2.1-14B 720p self-attention: bf16,
B=2 (CFG pair), H=40, 75,600 tokens, d=128, 64 sample pages (8,192 keys per
128-query block). Inputs are synthetic (seeded smooth-field Q/K, Gaussian V),
generated on the GPU and resident in HBM before timing starts.

Reported (one JSON line on stdout):
  value          effective TFLOP/s of the call = F_pre / call time, where
                 F_pre = 4*d*(128*rows)*(4*S) is the prefill work done;
  ms_per_step    ms per ab_attention call (mean over --steps);
  roofline       the prefill kernel (the dominant one): F_pre / its mean
                 duration (HIP events on the launch stream) vs the bf16 dense
                 MFMA peak; traffic from the committed rocprofv3 counter runs
                 (profiles/), or null;
  selection      build_plan time and the reference-dataflow byte count B_sel
                 divided by it, vs 8 TB/s;
  cpu_baseline   the CPU oracle (one thread) on a bounded sample of rows of
                 the same workload, extrapolated to a whole call.
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for p in (ROOT, os.path.join(ROOT, "ab-attention_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

PEAK_BF16_TFLOPS = 2516.6  # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0      # MI355X HBM3E

METRIC = "ms per AB-attn call + effective TFLOPS (MFMA %), Wan2.1-14B 720p 75.6k tokens"


def work_figures(bh: int, n: int, samples: int):
    qb, fb = -(-n // 128), n // 4
    rows = bh * qb
    f_pre = 262144.0 * rows * samples
    b_sel = (512.0 * bh * n + 256.0 * bh * n + 4096.0 * rows + 160.0 * rows + 40.0 * rows * fb
             + 4.0 * rows + 8.0 * rows * samples)
    return rows, fb, f_pre, b_sel


def _traffic_from_profiles():
    """HBM bytes per prefill launch from the committed counter summary, if any."""
    path = os.path.join(ROOT, "profiles", "prefill_traffic_c2.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f).get("traffic_bytes_per_launch")


def cpu_baseline(q, k, v, cfg, sample_rows: int):
    """Time the CPU oracle (single thread) on the first `sample_rows` query
    blocks of head 0 and extrapolate to the full call's rows."""
    import numpy as np
    import torch

    import oracle

    oracle.build()
    n = cfg.tokens
    samples = cfg.sample_pages * 32
    bits = lambda t: np.ascontiguousarray(t.contiguous().view(torch.int16).numpy().view(np.uint16))
    q0 = q[0, 0].cpu()
    k0 = k[0, 0].cpu()
    v0 = v[0, 0].cpu()
    toks = sample_rows * 128
    t0 = time.perf_counter()
    cent, pops = oracle.cluster(bits(q0[:toks]).reshape(1, toks, 128), 1, toks)
    pooled = oracle.pool(bits(k0).reshape(1, n, 128), 1, n)
    lse, mx, den = oracle.lse_rows(cent, pooled[0])
    scores = oracle.masses(lse, pops, mx, den, sample_rows, n // 4)
    offsets = np.random.default_rng(0).random(sample_rows).astype(np.float32)
    ids, logw = oracle.sip(scores, offsets, samples)
    qf = np.zeros((1, n, 128), np.float32)
    qf[0, :toks] = q0[:toks].float().numpy()
    full_ids = np.zeros((-(-n // 128), samples), np.int32)
    full_w = np.zeros_like(full_ids, dtype=np.float32)
    full_ids[:sample_rows], full_w[:sample_rows] = ids, logw
    oracle.prefill(qf, k0.float().numpy()[None], v0.float().numpy()[None], full_ids, full_w,
                   rows=np.arange(sample_rows))
    elapsed = time.perf_counter() - t0
    total_rows = cfg.batch * cfg.heads * -(-n // 128)
    return {
        "value": round(elapsed / sample_rows * total_rows * 1e3, 1),
        "unit": "ms per AB-attn call (extrapolated)",
        "cores": 1,
        "kind": "port",
        "sample": (f"{sample_rows} query blocks of head 0 (IBCS + SIP + weighted prefill, oracle C, fp64 "
                   f"prefill) in {elapsed:.1f} s, scaled by {total_rows} rows"),
        "cpu": platform.processor() or platform.machine(),
    }


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", type=int, default=2, help="BASELINE config index (default 2)")
    ap.add_argument("--heads", type=int, default=None, help="override head count (profiling only)")
    ap.add_argument("--cpu-sample-rows", type=int, default=80,
                    help="query blocks of head 0 timed on the CPU oracle (about 10 s on the GPU box host)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a 1 GiB device-to-device copy (HBM counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU only: every GPU box here has one GPU, and the path shards by "
              "heads with no communication (see DESIGN.md); run with --gpus 1", file=sys.stderr)
        return 2

    import torch

    if args.copy_calibration:
        src = torch.empty(1 << 28, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes_each_way": src.numel() * 4, "launches": 3}))
        return 0

    from ab_attention import apply_plan, build_plan
    from ab_attention.synthetic import CONFIGS, make_qkv

    cfg = CONFIGS[args.config]
    heads = None if args.heads is None else list(range(args.heads))
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    q, k, v = make_qkv(cfg, heads=heads, device=dev, dtype=torch.bfloat16)
    torch.cuda.synchronize()
    b, h, n, _ = q.shape
    bh = b * h
    samples = cfg.sample_pages * 32
    rows, fb, f_pre, b_sel = work_figures(bh, n, samples)

    def prefill_inputs(plan):
        """(ids, weights, order) that apply_plan hands to the prefill kernel."""
        return plan.descriptor.reshape(rows, samples), plan.log_weights.reshape(rows, samples), None

    if cfg.cube_layout:
        # c4: the cube token layout computed in place on raster-order tensors
        # (same results as permuting Q/K/V, attending and permuting back).
        from ab_attention.paged import _remap_ids
        from ab_attention.video import _cube_maps, apply_cube_plan, cube_plan

        build_plan = lambda q_, k_, **kw: cube_plan(q_, k_, cfg.grid, **kw)  # noqa: E731
        apply_plan = lambda q_, k_, v_, plan_: apply_cube_plan(q_, k_, v_, plan_, cfg.grid)  # noqa: E731

        def prefill_inputs(plan):  # noqa: F811
            order, page_map = _cube_maps(cfg.grid, q.device)
            return (_remap_ids(plan.descriptor.reshape(rows, samples), page_map),
                    plan.log_weights.reshape(rows, samples), order)

    def step():
        plan = build_plan(q, k, sample_pages=cfg.sample_pages, seed=42)
        return apply_plan(q, k, v, plan)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    ms_call = (time.perf_counter() - t0) * 1e3 / args.steps

    # Breakdown with HIP events on the launch stream (torch's current stream,
    # which every launch of the library uses): build_plan (selection) and the
    # prefill kernel alone (one launch).
    from ab_attention.paged import _prefill

    stream = torch.cuda.current_stream()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
    sel_ms, pre_ms = [], []
    for _ in range(max(3, args.steps)):
        ev[0].record(stream)
        plan = build_plan(q, k, sample_pages=cfg.sample_pages, seed=42)
        ev[1].record(stream)
        ids, weights, order = prefill_inputs(plan)
        ev[2].record(stream)
        _prefill(q, k, v, ids, weights, order, False)
        ev[3].record(stream)
        torch.cuda.synchronize()
        sel_ms.append(ev[0].elapsed_time(ev[1]))
        pre_ms.append(ev[2].elapsed_time(ev[3]))
    sel = sum(sel_ms) / len(sel_ms)
    pre = sum(pre_ms) / len(pre_ms)

    achieved = f_pre / (pre * 1e-3) / 1e12
    result = {
        "metric": METRIC,
        "value": round(f_pre / (ms_call * 1e-3) / 1e12, 2),
        "unit": "effective TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_call, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded smooth-field Q/K, Gaussian V), inputs resident in HBM",
        "config": {"workload": cfg.name, "batch": b, "heads": h, "tokens": n, "head_dim": 128,
                   "sample_pages": cfg.sample_pages, "keys_per_query_block": samples * 4,
                   "rows": rows, "parallelism": "none (1 GPU)"},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 1), "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
                     "traffic": _traffic_from_profiles(), "kernel": "prefill_kernel",
                     "ms": round(pre, 3), "work_tflop": round(f_pre / 1e12, 3)},
        "selection": {"ms": round(sel, 3), "bytes_gb": round(b_sel / 1e9, 3),
                      "effective_gbs": round(b_sel / (sel * 1e-3) / 1e9, 1),
                      "frac_of_hbm": round(b_sel / (sel * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)},
        "cpu_baseline": None,
    }
    if not args.no_cpu_baseline and args.heads is None:
        result["cpu_baseline"] = cpu_baseline(q, k, v, cfg, args.cpu_sample_rows)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
