"""Benchmark: one AB-attention call (build_plan + apply_plan) per step.

Default workload: Wan2.1-14B 720p self-attention: bf16,
B=2 (CFG pair), H=40, 75,600 tokens, d=128, 64 sample pages (8,192 keys per
128-query block). Inputs are synthetic (seeded smooth-field Q/K, Gaussian V),
generated on the GPU and resident in HBM before timing starts.

Reported (one JSON line on stdout):
  value          effective TFLOP/s of the call = F_pre / ms_per_step, where
                 F_pre = 4*d*(128*rows)*(4*S) is the prefill work done;
  ms_per_step    median over the --steps timed calls of the call's duration,
                 HIP events on the launch stream (torch's current stream,
                 which every launch of the library uses); wall_ms_per_step
                 is the host clock over the same steps, synchronised on both
                 sides, divided by --steps;
  roofline       the prefill kernel (the dominant one): F_pre / its median
                 duration (HIP events around its launches: the rows of a
                 call are launched in chunks of ~11,000, 5 at c2, so this
                 equals the per-launch work over the mean launch duration)
                 vs the bf16 dense MFMA peak; traffic = HBM bytes
                 per launch from the committed rocprofv3 counter runs
                 (profiles/), or null;
  selection      build_plan's median duration, and the reference-dataflow
                 byte count B_sel divided by it, vs 8 TB/s;
  dense          dense attention over the same Q/K/V (exact_attention: the
                 reference's dense steps and layer 0), median of 3 calls,
                 with its dense-equivalent work 4*d*N^2*B*H;
  cpu_baseline   the CPU oracle on all host threads (OpenMP) over one whole
                 head of the same workload, scaled by the head count.

--static-plan prints a different line instead: the plan through
ab_ibcs_sip_static (its workspace in the static array of
libab_attention_static.so, heads in chunks that fit it) against ab_ibcs_sip
with a caller workspace, median of --steps calls each, and whether the two
plans are the same bits.

--power prints a different line instead: socket power and graphics clock
(median over `amd-smi metric -p -c` readings, taken from a child process
every 0.2 s) while each part of the call runs back to back for
--power-seconds: the prefill on a fixed plan, build_plan, and dense
attention.
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import statistics
import subprocess
import sys
import threading
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


def prefill_launches(bh: int, n: int) -> int:
    """Launches the library splits one prefill call into (its own answer,
    ab_prefill_launch_slots: row slots per XCD per launch)."""
    from ab_attention import _lib

    per_launch = _lib.load().ab_prefill_launch_slots(bh, n)
    qb = -(-n // 128)
    slots = -(-qb // 8) * bh  # row slots per XCD
    return max(1, -(-slots // per_launch))


def _traffic_from_profiles(workload: str):
    """HBM bytes per prefill launch from the committed counter summary (c2 only)."""
    path = os.path.join(ROOT, "profiles", "prefill_traffic_c2.json")
    if not os.path.exists(path) or workload != "wan2.1-14b-720p":
        return None
    with open(path) as f:
        return json.load(f).get("traffic_bytes_per_launch")


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def cpu_baseline(q, k, v, cfg, head: int):
    """Time the CPU oracle (IBCS, SIP and the fp64 weighted prefill, row loops
    on every OpenMP thread) over all query blocks of one (batch 0, head) and
    scale by the call's head count."""
    import numpy as np
    import torch

    import oracle

    oracle.build()
    n = cfg.tokens
    samples = cfg.sample_pages * 32
    bits = lambda t: np.ascontiguousarray(t.contiguous().view(torch.int16).numpy().view(np.uint16))
    q0, k0, v0 = (t[0, head].cpu() for t in (q, k, v))
    qb = -(-n // 128)
    offsets = np.random.default_rng(0).random(qb).astype(np.float32)
    qf, kf, vf = (t.float().numpy()[None] for t in (q0, k0, v0))
    t0 = time.perf_counter()
    scores = oracle.ibcs(bits(q0).reshape(1, n, 128), bits(k0).reshape(1, n, 128), 1, n)
    ids, logw = oracle.sip(scores, offsets, samples)
    oracle.prefill(qf, kf, vf, ids, logw)
    elapsed = time.perf_counter() - t0
    heads = cfg.batch * cfg.heads
    return {
        "value": round(elapsed * heads * 1e3, 1),
        "unit": "ms per AB-attn call (one head timed, scaled by B*H)",
        "cores": oracle.num_threads(),
        "kind": "port",
        "sample": (f"all {qb} query blocks of one head (batch 0, head {head}): IBCS + SIP + weighted "
                   f"prefill (oracle C, fp64 prefill) in {elapsed:.1f} s on {oracle.num_threads()} threads, "
                   f"scaled by {heads} heads"),
        "cpu": _cpu_model(),
    }


def _smi_reading():
    """One amd-smi reading: (socket power in W, median graphics clock in MHz
    over the XCDs), or None where the tool or a value is unavailable."""
    try:
        out = subprocess.run(["amd-smi", "metric", "-p", "-c", "--json"], capture_output=True, text=True,
                             timeout=20).stdout
        gpu = json.loads(out)["gpu_data"][0]
        power = float(gpu["power"]["socket_power"]["value"])
        clocks = [float(c["clk"]["value"]) for name, c in gpu["clock"].items() if name.startswith("gfx_")]
        return power, statistics.median(clocks)
    except (OSError, subprocess.SubprocessError, ValueError, KeyError, IndexError, TypeError,
            statistics.StatisticsError):
        return None


def power_legs(legs, seconds: float):
    """Socket power and clock while each leg runs back to back for `seconds`
    (the first two readings of a leg are dropped as ramp-up)."""
    import torch

    out = {}
    for name, fn in legs:
        fn()
        torch.cuda.synchronize()
        readings, stop = [], threading.Event()

        def sample():
            while not stop.is_set():
                r = _smi_reading()
                if r is not None:
                    readings.append(r)
                stop.wait(0.2)

        th = threading.Thread(target=sample, daemon=True)
        th.start()
        t0, calls = time.perf_counter(), 0
        while time.perf_counter() - t0 < seconds:
            fn()
            torch.cuda.synchronize()
            calls += 1
        elapsed = time.perf_counter() - t0
        stop.set()
        th.join()
        steady = readings[2:] or readings
        out[name] = {"calls": calls, "ms_per_call": round(elapsed * 1e3 / calls, 3), "readings": len(steady),
                     "socket_w": statistics.median(r[0] for r in steady) if steady else None,
                     "gfx_mhz": statistics.median(r[1] for r in steady) if steady else None}
        print(f"power leg {name}: {out[name]}", file=sys.stderr, flush=True)
    return out


def static_plan_timing(q, k, rows: int, samples: int, steps: int, workload: str) -> dict:
    """Median ms of the plan through ab_ibcs_sip_static and through
    ab_ibcs_sip with a caller workspace (same inputs and uniforms)."""
    import torch

    from ab_attention import _lib

    lib, static = _lib.load(), _lib.load_static()
    bh, n = q.shape[0] * q.shape[1], q.shape[2]
    offsets = torch.rand(rows, device=q.device, generator=torch.Generator(q.device).manual_seed(42))
    out = {}
    plans = {}
    ws_bytes = lib.ab_ibcs_sip_workspace_bytes(bh, n)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device)
    st = _lib.stream(q.device)
    for name in ("workspace", "static"):
        ids = torch.empty(rows, samples, dtype=torch.int32, device=q.device)
        w = torch.empty(rows, samples, dtype=torch.float32, device=q.device)
        if name == "static":
            call = lambda: static.ab_ibcs_sip_static(_lib.ptr(q), _lib.ptr(k), None, bh, n, _lib.ptr(offsets),  # noqa: E731
                                                     samples, _lib.ptr(ids), _lib.ptr(w), st)
        else:
            call = lambda: lib.ab_ibcs_sip(_lib.ptr(q), _lib.ptr(k), None, bh, n, _lib.ptr(offsets), samples,  # noqa: E731
                                           _lib.ptr(ws), ws_bytes, _lib.ptr(ids), _lib.ptr(w), st)
        _lib.check(call())
        torch.cuda.synchronize()
        times = []
        for _ in range(max(steps, 1)):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            _lib.check(call())
            e1.record()
            torch.cuda.synchronize()
            times.append(e0.elapsed_time(e1))
        out[name + "_ms"] = round(statistics.median(times), 3)
        plans[name] = (ids, w)
    same = (torch.equal(plans["static"][0], plans["workspace"][0])
            and torch.equal(plans["static"][1].view(torch.int32), plans["workspace"][1].view(torch.int32)))
    head_bytes = lib.ab_ibcs_sip_workspace_bytes(1, n)
    chunk = min(bh, (512 << 20) // head_bytes) if head_bytes else 0
    while chunk > 1 and lib.ab_ibcs_sip_workspace_bytes(chunk, n) > (512 << 20):
        chunk -= 1
    return {"workload": workload, "static_plan": dict(out, bit_identical=same, heads_per_static_chunk=chunk,
                                                      workspace_bytes=ws_bytes)}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", type=int, default=2, help="BASELINE config index (default 2)")
    ap.add_argument("--heads", type=int, default=None, help="override head count (profiling only)")
    ap.add_argument("--cpu-head", type=int, default=0,
                    help="head (of batch item 0) timed on the CPU oracle, all its query blocks")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-dense", action="store_true", help="skip the dense-attention timing")
    ap.add_argument("--lse-budget-gib", type=float, default=None,
                    help="IBCS head-chunk budget (default: the library's 16 GiB; the reference uses 1.5)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a 1 GiB device-to-device copy (HBM counter calibration)")
    ap.add_argument("--power", action="store_true",
                    help="only report socket power and graphics clock per part of the call (amd-smi)")
    ap.add_argument("--power-seconds", type=float, default=10.0)
    ap.add_argument("--static-plan", action="store_true",
                    help="only time the no-allocation plan (ab_ibcs_sip_static) against ab_ibcs_sip")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU only: every GPU box here has one GPU, and the path shards by "
              "heads with no communication between GPUs; run with --gpus 1", file=sys.stderr)
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

    if args.lse_budget_gib is not None:
        from ab_attention import attention

        attention.LSE_BUDGET_BYTES = int(args.lse_budget_gib * 1024 ** 3)
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

    stream = torch.cuda.current_stream()

    if args.static_plan:
        print(json.dumps(static_plan_timing(q, k, rows, samples, args.steps, cfg.name)), flush=True)
        return 0

    if args.power:
        from ab_attention.paged import _prefill
        from ab_attention.video import exact_attention

        plan = build_plan(q, k, sample_pages=cfg.sample_pages, seed=42)
        ids, weights, order = prefill_inputs(plan)
        legs = [("prefill", lambda: _prefill(q, k, v, ids, weights, order, False)),
                ("selection", lambda: build_plan(q, k, sample_pages=cfg.sample_pages, seed=42))]
        if not cfg.text_tokens:
            legs.append(("dense", lambda: exact_attention(q, k, v)))
        print(json.dumps({"workload": cfg.name, "power": power_legs(legs, args.power_seconds)}), flush=True)
        return 0

    def step():
        plan = build_plan(q, k, sample_pages=cfg.sample_pages, seed=42)
        return apply_plan(q, k, v, plan)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    # The timed region: exactly --steps calls, synchronised on both sides,
    # with a HIP event pair around each call on the launch stream.
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
    t0 = time.perf_counter()
    for start, stop in ev:
        start.record(stream)
        step()
        stop.record(stream)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / args.steps
    ms_call = statistics.median(a.elapsed_time(b) for a, b in ev)

    # Breakdown with HIP events on the launch stream: build_plan (selection)
    # and the prefill kernel alone (one launch, recorded while build_plan's
    # kernels still run, so no host gap is timed).
    from ab_attention.paged import _prefill

    sel_ms, pre_ms = [], []
    for _ in range(max(3, args.steps)):
        e = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
        e[0].record(stream)
        plan = build_plan(q, k, sample_pages=cfg.sample_pages, seed=42)
        e[1].record(stream)
        ids, weights, order = prefill_inputs(plan)
        e[2].record(stream)
        _prefill(q, k, v, ids, weights, order, False)
        e[3].record(stream)
        torch.cuda.synchronize()
        sel_ms.append(e[0].elapsed_time(e[1]))
        pre_ms.append(e[2].elapsed_time(e[3]))
    sel = statistics.median(sel_ms)
    pre = statistics.median(pre_ms)

    # Per launch: the launches cover equal numbers of whole generations of
    # rows (the last may be smaller), so F_pre / launches over the mean launch
    # duration is F_pre over the prefill's total duration.
    launches = prefill_launches(bh, n)
    achieved = f_pre / (pre * 1e-3) / 1e12
    result = {
        "metric": METRIC,
        "value": round(f_pre / (ms_call * 1e-3) / 1e12, 2),
        "unit": "effective TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_call, 3),
        "wall_ms_per_step": round(wall_ms, 3),
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
                     "traffic": _traffic_from_profiles(cfg.name), "kernel": "prefill_kernel",
                     "launches": launches, "ms": round(pre, 3), "ms_per_launch": round(pre / launches, 3),
                     "work_tflop": round(f_pre / 1e12, 3),
                     "work_tflop_per_launch": round(f_pre / launches / 1e12, 3)},
        "selection": {"ms": round(sel, 3), "bytes_gb": round(b_sel / 1e9, 3),
                      "effective_gbs": round(b_sel / (sel * 1e-3) / 1e9, 1),
                      "frac_of_hbm": round(b_sel / (sel * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)},
        "dense": None,
        "cpu_baseline": None,
    }
    if not args.no_dense and not cfg.text_tokens:
        from ab_attention.video import exact_attention

        exact_attention(q, k, v)
        dense_ms = []
        for _ in range(3):
            e = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
            e[0].record(stream)
            exact_attention(q, k, v)
            e[1].record(stream)
            torch.cuda.synchronize()
            dense_ms.append(e[0].elapsed_time(e[1]))
        dms = statistics.median(dense_ms)
        f_dense = 4.0 * 128 * n * n * bh
        result["dense"] = {"ms": round(dms, 3), "work_tflop": round(f_dense / 1e12, 3),
                           "tflops": round(f_dense / (dms * 1e-3) / 1e12, 1),
                           "frac": round(f_dense / (dms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
                           "kernel": "dense_kernel"}
    if not args.no_cpu_baseline and args.heads is None:
        result["cpu_baseline"] = cpu_baseline(q, k, v, cfg, args.cpu_head)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
