"""Benchmark: MXFP4 dequant GB/s and MoE layer tokens/s, gpt-oss-120b shape, 1 GPU.

``python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload dequant]``

Prints ONE JSON line.  The headline workload is the MXFP4 dequantisation of
one gpt-oss-120b layer of expert weights (gate_up [128,5760,90,16] and down
[128,2880,90,16] packed bytes with their scales, to bfloat16), with inputs
resident in HBM.  A step is one dequantisation of the whole layer (both
projections).  ``value`` is the whole-job algorithmic bandwidth (bytes read
plus bytes written, 8,062,156,800 B per step) over the timed steps.

``roofline`` covers the dequant kernel, timed per launch with HIP events on
the launch stream; ``traffic`` is the measured HBM bytes per step from the
rocprofv3 FETCH_SIZE/WRITE_SIZE runs recorded in profiles/traffic.json (null
when absent).  ``cpu_baseline`` times the oracle's torch restatement of the
reference dequant on the host cores over a bounded sample of the same
workload.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

import torch

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0

GATE_UP = (128, 5760, 90)   # experts, rows (2 * intermediate), groups (hidden / 32)
DOWN = (128, 2880, 90)      # experts, rows (hidden), groups (intermediate / 32)


def dequant_bytes(E: int, R: int, G: int, out_elem: int = 2) -> int:
    """Algorithmic bytes: packed bytes + scale bytes read, dense output written."""
    return E * R * G * 16 + E * R * G + E * R * G * 32 * out_elem


def traffic_record(key: str):
    path = ROOT / "profiles" / "traffic.json"
    if not path.exists():
        return None
    try:
        return json.loads(path.read_text()).get(key)
    except (OSError, ValueError):
        return None


def cpu_baseline_dequant(experts: int = 16) -> dict:
    """Oracle torch restatement of the reference dequant on the host cores."""
    import oracle
    from blockstreamer_amd import synthetic

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    E, R, G = GATE_UP
    blocks, scales = synthetic.packed_weights(experts, R, G, seed=2, scale_lo=115, scale_hi=131)
    oracle.dequant_torch(blocks[:1], scales[:1], torch.bfloat16)  # warm-up
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        oracle.dequant_torch(blocks, scales, torch.bfloat16)
        times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    return {
        "value": round(dequant_bytes(experts, R, G) / t / 1e9, 3),
        "unit": "GB/s",
        "cores": cores,
        "kind": "port",
        "sample": f"{experts} of 128 gate_up experts [{experts},{R},{G},16] -> bf16, "
                  f"median of 3 runs ({t:.2f} s each)",
    }


def bench_dequant(args) -> dict:
    from blockstreamer_amd import kernels, synthetic

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    gu_b, gu_s = synthetic.packed_weights(*GATE_UP, seed=2, scale_lo=115, scale_hi=131, device=dev)
    dn_b, dn_s = synthetic.packed_weights(*DOWN, seed=3, scale_lo=115, scale_hi=131, device=dev)
    gu_out = torch.empty((GATE_UP[0], GATE_UP[2] * 32, GATE_UP[1]), dtype=torch.bfloat16, device=dev)
    dn_out = torch.empty((DOWN[0], DOWN[2] * 32, DOWN[1]), dtype=torch.bfloat16, device=dev)
    bytes_gu = dequant_bytes(*GATE_UP)
    bytes_dn = dequant_bytes(*DOWN)
    step_bytes = bytes_gu + bytes_dn

    def step(events=None):
        if events is not None:
            events[0].record()
        kernels.dequantize_mxfp4(gu_b, gu_s, torch.bfloat16, out=gu_out)
        if events is not None:
            events[1].record()
        kernels.dequantize_mxfp4(dn_b, dn_s, torch.bfloat16, out=dn_out)
        if events is not None:
            events[2].record()

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        step(evs[i])
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    gu_ms = [e[0].elapsed_time(e[1]) for e in evs]
    dn_ms = [e[1].elapsed_time(e[2]) for e in evs]
    kern_s = (sum(gu_ms) + sum(dn_ms)) / 1e3
    achieved = step_bytes * args.steps / kern_s / 1e9
    traffic = traffic_record("dequant_mxfp4_gptoss120b_layer")
    return {
        "metric": "MoE layer tokens/s + MXFP4 dequant GB/s, gpt-oss-120b shape, 1xMI355X",
        "value": round(step_bytes * args.steps / wall / 1e9, 2),
        "unit": "GB/s",
        "ms_per_step": round(wall / args.steps * 1e3, 4),
        "dtype": "bf16",
        "config": {
            "workload": "MXFP4 dequant of one gpt-oss-120b layer of experts: gate_up "
                        "[128,5760,90,16] + down [128,2880,90,16] uint8 with E8M0 scales "
                        "in [115,131] -> bf16 [128,2880,5760] + [128,2880,2880]",
            "bytes_per_step": step_bytes,
            "gate_up_ms": round(statistics.median(gu_ms), 4),
            "down_ms": round(statistics.median(dn_ms), 4),
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "kernel": "dequant_vec_kernel<bf16>",
        },
    }


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default="dequant", choices=["dequant"])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build runs the MoE expert path on a "
              "single MI355X (no multi-GPU path); run with --gpus 1", file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 2
    res = bench_dequant(args)
    line = {
        "metric": res["metric"],
        "value": res["value"],
        "unit": res["unit"],
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": res["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": res["dtype"],
        "data": "synthetic",
        "config": res["config"],
        "roofline": res["roofline"],
        "cpu_baseline": None if args.no_cpu_baseline else cpu_baseline_dequant(),
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
