"""Benchmark: MXFP4 dequant GB/s and MoE layer tokens/s, gpt-oss-120b shape, 1 GPU.

``python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload dequant]``

Prints ONE JSON line.  The headline workload is the MXFP4 dequantisation of
one gpt-oss-120b layer of expert weights (gate_up [128,5760,90,16] and down
[128,2880,90,16] packed bytes with their scales, to bfloat16), with inputs
resident in HBM.  A step is one dequantisation of the whole layer (both
projections).  ``value`` is the whole-job algorithmic bandwidth (bytes read
plus bytes written, 8,062,156,800 B per step) over the timed steps.

``roofline`` covers the one kernel of the step, dequant_vec_kernel<bf16>,
launched twice per step (gate_up: 5,374,771,200 algorithmic bytes; down:
2,687,385,600): ``achieved`` is the mean algorithmic bytes per launch over the
mean launch duration, timed with HIP events on the launch stream (the same
average rocprofv3 --stats reports for the kernel); ``traffic`` is the mean
measured HBM bytes per launch from the rocprofv3 FETCH_SIZE/WRITE_SIZE runs
recorded in profiles/traffic.json, each counter scaled by its plain-copy
calibration factor (null when absent).  ``cpu_baseline`` times the oracle's
torch restatement of the reference dequant on the host cores over the same
bytes (drawn on the CPU, copied to the GPU).

``moe_layer`` holds the MoE layer workloads (router, dispatch, expert GEMMs,
combine; inputs drawn on the CPU and copied to the GPU): the gpt-oss-120b
decode batches of 1, 8 and 64 tokens (HBM roofline of the weight stream),
the gpt-oss-20b layer at 2048 tokens and the gpt-oss-120b prefill at 8192
tokens (MFMA rooflines; forward plus the LoRA input-gradient backward), each
prefill on the two-term MX kernels and on the dequant-to-bf16 kernels, in
both blocks layouts, with the relative L2 distance to a float32 reference,
and CPU baselines of the oracle on token samples of the 64-, 2048- and
8192-token batches.
"""

from __future__ import annotations

import argparse
import functools
import json
import os
import statistics
import sys
import time
from pathlib import Path
from typing import NamedTuple

import torch

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0

GATE_UP = (128, 5760, 90)   # experts, rows (2 * intermediate), groups (hidden / 32)
DOWN = (128, 2880, 90)      # experts, rows (hidden), groups (intermediate / 32)


def dequant_bytes(E: int, R: int, G: int, out_elem: int = 2) -> int:
    """Algorithmic bytes: packed bytes + scale bytes read, dense output written."""
    return E * R * G * 16 + E * R * G + E * R * G * 32 * out_elem


def traffic_record(key: str, field: str):
    """Measured HBM bytes (calibrated FETCH_SIZE + WRITE_SIZE) from profiles/traffic.json."""
    path = ROOT / "profiles" / "traffic.json"
    if not path.exists():
        return None
    try:
        return json.loads(path.read_text()).get(key, {}).get(field)
    except (OSError, ValueError, AttributeError):
        return None


@functools.lru_cache(maxsize=1)
def cpu_packed() -> tuple:
    """Both projections' packed weights of one gpt-oss-120b layer, drawn on the
    CPU from seeded generators; the GPU run gets copies of these bytes."""
    from blockstreamer_amd import synthetic

    return (synthetic.packed_weights(*GATE_UP, seed=2, scale_lo=115, scale_hi=131),
            synthetic.packed_weights(*DOWN, seed=3, scale_lo=115, scale_hi=131))


def cpu_baseline_dequant() -> dict:
    """Oracle torch restatement of the reference dequant on the host cores.

    The sample is the whole workload: both projections of one gpt-oss-120b
    layer (all 128 experts), the same bytes the GPU dequantises, median of 3
    runs (about 10 s of CPU work).
    """
    import oracle

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    packed = cpu_packed()
    oracle.dequant_torch(packed[1][0][:1], packed[1][1][:1], torch.bfloat16)  # warm-up
    times = []
    for _ in range(3):
        t = 0.0
        for blocks, scales in packed:
            t0 = time.perf_counter()
            out = oracle.dequant_torch(blocks, scales, torch.bfloat16)
            t += time.perf_counter() - t0
            del out
        times.append(t)
    t = statistics.median(times)
    total = dequant_bytes(*GATE_UP) + dequant_bytes(*DOWN)
    return {
        "value": round(total / t / 1e9, 3),
        "unit": "GB/s",
        "cores": cores,
        "kind": "port",
        "cpu": cpu_model(),
        "sample": f"the whole workload (gate_up [128,5760,90,16] + down [128,2880,90,16] -> "
                  f"bf16), median of 3 runs ({t:.2f} s each)",
    }


def bench_dequant(args) -> dict:
    from blockstreamer_amd import kernels

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    (gu_b, gu_s), (dn_b, dn_s) = ((b.to(dev), sc.to(dev)) for b, sc in cpu_packed())
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
    launch_ms = statistics.mean(gu_ms + dn_ms)
    launch_bytes = step_bytes / 2
    achieved = launch_bytes / (launch_ms / 1e3) / 1e9
    step_traffic = traffic_record("dequant_mxfp4_gptoss120b_layer", "hbm_bytes_per_step")
    traffic = round(step_traffic / 2) if step_traffic else None
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
            "kernel": "dequant_vec_kernel<bf16> (gate_up and down launches)",
            "algorithmic_bytes": launch_bytes,
            "launch_ms": round(launch_ms, 4),
        },
    }


# ----------------------------------------------------------------------------- MoE layer

BF16_PEAK_TFLOPS = 2500.0
FP8_PEAK_TFLOPS = 5000.0
MXFP4_PEAK_TFLOPS = 10100.0


class Workload(NamedTuple):
    """A MoE layer workload: shape, seed and router bias std.  Expert scale
    bytes are uniform in [115, 131], activations N(0, 1) in bf16, router
    weights N(0, 0.02)."""
    E: int
    k: int
    H: int
    I: int
    seed: int
    bias_std: float


# the 120b decode batches route with a per-expert bias of std 0.5 (uneven
# expert load); the 20b layer uses 0.01; the 120b prefill 0
DECODE = Workload(128, 4, 2880, 2880, seed=4, bias_std=0.5)
LAYER_20B = Workload(32, 4, 2880, 2880, seed=3, bias_std=0.01)
PREFILL = Workload(128, 4, 2880, 2880, seed=5, bias_std=0.0)
EXPERT_KEYS = ("gate_up_proj_blocks", "gate_up_proj_scales", "gate_up_proj_bias",
               "down_proj_blocks", "down_proj_scales", "down_proj_bias")


@functools.lru_cache(maxsize=4)
def cpu_layer(wl: Workload, T: int) -> dict:
    """The layer's tensors drawn on the CPU from one seeded generator; the GPU
    runs get copies of these bytes, so the CPU baseline sees the same ones."""
    from blockstreamer_amd import synthetic

    return synthetic.moe_layer(synthetic.MoEShape(wl.E, wl.k, wl.H, wl.I, T), seed=wl.seed, scale_lo=115,
                               scale_hi=131, router_bias_std=wl.bias_std)


def expert_bytes(H: int, I: int) -> int:
    """Packed weights, scales and bf16 biases of one expert (both projections)."""
    gu = 2 * I * (H // 32) * 17 + 2 * I * 2
    dn = H * (I // 32) * 17 + H * 2
    return gu + dn


def moe_flops(T: int, k: int, H: int, I: int) -> int:
    return 2 * T * k * (H * 2 * I + I * H)


def _median_ms(pairs):
    return statistics.median([a.elapsed_time(b) for a, b in pairs])


def fp32_reference(x, idx, w, args, alpha=1.702, limit=7.0):
    """float32 torch reference of the experts on the GPU (block_streamer/
    gptoss.py:137-177): dense weights from the dequant kernel (bit-exact with
    the reference's dequant), float32 GEMMs and SwiGLU."""
    from blockstreamer_amd import kernels

    gub, gus, gubias, dnb, dns, dnbias = args
    h = x.float()
    out = torch.zeros_like(h)
    for e in torch.unique(idx).tolist():
        tok, pos = torch.where(idx == e)
        wgu = kernels.dequantize_mxfp4(gub[e:e + 1], gus[e:e + 1], torch.float32)[0]
        wdn = kernels.dequantize_mxfp4(dnb[e:e + 1], dns[e:e + 1], torch.float32)[0]
        gu = h[tok] @ wgu + gubias[e].float()
        gate, up = gu[:, 0::2].clamp(max=limit), gu[:, 1::2].clamp(min=-limit, max=limit)
        act = (up + 1) * (gate * torch.sigmoid(gate * alpha))
        o = act @ wdn + dnbias[e].float()
        out.index_add_(0, tok, o * w[tok, pos, None].float())
    return out


def _resolved_kernel(path: str, T: int, wl: Workload) -> str:
    """The expert GEMM kernels an inference forward runs for ``path`` (the
    library's rule: automatic selection takes the MX kernels above 16 rows
    per expert when H and I are multiples of 64 -- the bench's weights are
    aligned; a forward saving for the backward keeps the bf16 kernels)."""
    if path != "auto":
        return path
    if T * wl.k <= 16 * wl.E:
        return "stream"
    return "mx" if wl.H % 64 == 0 and wl.I % 64 == 0 else "tiled"


def _graph_ms(fn, reps: int) -> float:
    """Milliseconds per call of ``fn`` from ``reps`` calls captured in one
    HIP graph, replayed five times between two HIP events."""
    for _ in range(2):
        fn()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(reps):
            fn()
    graph.replay()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(5):
        graph.replay()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / (5 * reps)


def bench_moe(wl: Workload, T: int, steps: int, warmup: int, path: str = "auto", layout: str = "checkpoint",
              train: bool = False, fwd: bool = True, ref: bool = False) -> dict:
    """One MoE layer (router + dispatch + expert GEMMs + combine) of
    ``wl`` at T tokens.  ``train``: also the LoRA training use, a
    forward saving the SwiGLU's derivative factors followed by the
    input-gradient backward.  ``fwd=False``: only that (the profile of the training run).
    ``ref``: also the output's relative L2 distance to a float32 reference."""
    from blockstreamer_amd import kernels

    dev = torch.device("cuda", 0)
    E, k, H, I = wl.E, wl.k, wl.H, wl.I
    t = {n: v.to(dev) for n, v in cpu_layer(wl, T).items()}
    x = t["hidden"]
    args = tuple(t[n] for n in EXPERT_KEYS)
    if layout == "kpair":
        # the k-pair shard layout is an on-disk format: repacked once, before
        # anything is timed
        args = (kernels.to_kpair(args[0]),) + args[1:3] + (kernels.to_kpair(args[3]),) + args[4:]

    def route():
        # fused router kernel (logits, top-k, softmax over the top-k)
        _, scores, idx = kernels.router_forward(x, t["router_weight"], t["router_bias"], k)
        return idx, scores

    def step():
        idx, w = route()
        return kernels.moe_experts_forward(x, idx, w, *args, path=path)

    flops = moe_flops(T, k, H, I)
    kernel = _resolved_kernel(path, T, wl)
    res = {"tokens": T, "path": path, "kernel_path": kernel, "layout": layout}
    if fwd:
        for _ in range(warmup):
            step()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            step()
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0

        # per-stage HIP events on the launch stream (a separate pass, so the
        # events do not sit inside the timed layer steps above)
        idx, w = route()
        hit = int(torch.unique(idx).numel())
        st = kernels.MoEStages(x, idx, w, *args, path=path)
        names = ("route", "dispatch", "gate_up", "down", "combine")
        ev = {n: [] for n in names}
        for _ in range(max(steps, 5)):
            e = [torch.cuda.Event(enable_timing=True) for _ in range(len(names) + 1)]
            e[0].record()
            route()
            e[1].record()
            st.dispatch()
            e[2].record()
            st.gate_up()
            e[3].record()
            st.down()
            e[4].record()
            st.combine()
            e[5].record()
            for i, n in enumerate(names):
                ev[n].append((e[i], e[i + 1]))
        torch.cuda.synchronize()
        ms = {n: round(_median_ms(ev[n]), 4) for n in names}
        gemm_ms = ms["gate_up"] + ms["down"]
        wbytes = hit * expert_bytes(H, I)
        res.update({"tokens_per_s": round(T * steps / wall, 1), "ms_per_layer": round(wall / steps * 1e3, 4),
                    "stage_ms": ms, "hit_experts": hit})
        if kernel == "stream":
            # GPU time of the layer without the host: ten layer steps captured
            # in one HIP graph and replayed (how decode serving runs a layer)
            res["graph_ms_per_layer"] = round(_graph_ms(step, 10), 4)
        hbm = wbytes / (gemm_ms / 1e3) / 1e9
        tfl = flops / (gemm_ms / 1e3) / 1e12
        if kernel == "stream":
            res["roofline"] = {"bound": "hbm", "achieved": round(hbm, 1), "peak": HBM_PEAK_GBS,
                               "unit": "GB/s", "frac": round(hbm / HBM_PEAK_GBS, 4),
                               "kernel": "moe_stream_persist_kernel gate_up + down",
                               "algorithmic_bytes": wbytes}
            if T == 64 and layout == "checkpoint":
                gu_b = traffic_record("moe_layer_gptoss120b_decode_t64", "gate_up_hbm_bytes")
                dn_b = traffic_record("moe_layer_gptoss120b_decode_t64", "down_hbm_bytes")
                res["roofline"]["traffic"] = gu_b + dn_b if gu_b and dn_b else None
        elif kernel == "mx":
            # two f8f6f4 instructions (hi and lo activation terms) per 64-k
            # step, each at the FP8 rate: the path's own ceiling is half of it
            res["roofline"] = {"bound": "mfma", "achieved": round(tfl, 1), "peak": FP8_PEAK_TFLOPS,
                               "unit": "TFLOP/s", "frac": round(tfl / FP8_PEAK_TFLOPS, 4),
                               "path_ceiling": FP8_PEAK_TFLOPS / 2,
                               "frac_of_path_ceiling": round(tfl / (FP8_PEAK_TFLOPS / 2), 4),
                               "frac_of_mxfp4_peak": round(tfl / MXFP4_PEAK_TFLOPS, 4),
                               "kernel": "moe_mx_kernel (two-term MXFP8 x MXFP4) gate_up + down, "
                                         "with the split of the hidden rows",
                               "algorithmic_flops": flops}
        else:
            res["roofline"] = {"bound": "mfma", "achieved": round(tfl, 1), "peak": BF16_PEAK_TFLOPS,
                               "unit": "TFLOP/s", "frac": round(tfl / BF16_PEAK_TFLOPS, 4),
                               "frac_of_mxfp4_peak": round(tfl / MXFP4_PEAK_TFLOPS, 4),
                               "kernel": "moe_tiled2_kernel gate_up + down",
                               "algorithmic_flops": flops}
        if ref:
            want = fp32_reference(x, idx, w, args if layout == "checkpoint" else tuple(t[n] for n in EXPERT_KEYS))
            got = kernels.moe_experts_forward(x, idx, w, *args, path=path).float()
            res["rel_l2_vs_fp32"] = round(((got - want).norm() / want.norm()).item(), 6)
            # net of the output's own rounding: the same kernels with the
            # combine writing float32 (every bf16 output sits ~1.7e-3 from
            # float32 however exact its arithmetic), and the bf16 output
            # against the float32 reference rounded once to bf16
            got32 = kernels.moe_experts_forward(x, idx, w, *args, path=path, out_dtype=torch.float32)
            res["rel_l2_f32_out_vs_fp32"] = round(((got32 - want).norm() / want.norm()).item(), 6)
            want_r = want.to(torch.bfloat16).float()
            res["rel_l2_vs_fp32_rounded"] = round(((got - want_r).norm() / want_r.norm()).item(), 6)
    if train:
        # the LoRA training use: forward saving the SwiGLU's derivative
        # factors, then the input-gradient backward (expert weights frozen)
        idx, w = route()
        g = (torch.randn(T, H, generator=torch.Generator().manual_seed(7)) * 0.1).to(torch.bfloat16).to(dev)

        def timed_training(train_path):
            def fwd_only():
                return kernels.moe_experts_forward(x, idx, w, *args, path=train_path, save=True)

            def fwd_bwd():
                out, ws, pre = fwd_only()
                return kernels.moe_experts_backward(g, x, idx, w, args[0], args[1], args[3], args[4], ws, pre)

            for _ in range(2):
                fwd_bwd()
            torch.cuda.synchronize()
            pairs, fpairs = [], []
            for _ in range(max(steps // 2, 3)):
                a0, a1, a2 = (torch.cuda.Event(enable_timing=True) for _ in range(3))
                a0.record()
                fwd_only()
                a1.record()
                fwd_bwd()
                a2.record()
                fpairs.append((a0, a1))
                pairs.append((a1, a2))
            torch.cuda.synchronize()
            return _median_ms(pairs), _median_ms(fpairs)

        fb_ms, f_ms = timed_training(path)
        # a forward that saves for the backward keeps the bf16 kernels where
        # automatic selection would take the MX ones
        res["train_forward_kernel_path"] = "tiled" if path == "auto" and kernel == "mx" else kernel
        res["fwd_bwd_ms"] = round(fb_ms, 4)
        res["bwd_ms"] = round(fb_ms - f_ms, 4)
        res["bwd_TFLOP_per_s"] = round(flops / ((fb_ms - f_ms) / 1e3) / 1e12, 1)
        if path == "auto" and kernel == "mx":
            # the opt-in MX training forward (MXFP4Experts.mx_training)
            mfb, mf = timed_training("mx")
            res["mx_training"] = {"fwd_ms": round(mf, 4), "fwd_bwd_ms": round(mfb, 4)}
    return res


def cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline_moe(wl: Workload, T: int, sample: int, what: str) -> dict:
    """The oracle (float32 torch restatement of the reference path, router
    and per-expert dequant + GEMMs + SwiGLU + combine) on the host cores, over
    the first ``sample`` tokens of the same bytes the GPU runs; tokens/s of
    that sample, median of 3 runs."""
    import oracle

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    k = wl.k
    t = cpu_layer(wl, T)
    h = t["hidden"][:sample]
    args = tuple(t[n] for n in EXPERT_KEYS)
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        _, scores, idx = oracle.router_ref(h, t["router_weight"], t["router_bias"], k)
        oracle.experts_ref(h, idx, scores, *args)
        times.append(time.perf_counter() - t0)
    tm = statistics.median(times)
    return {"value": round(sample / tm, 3), "unit": "tokens/s", "cores": cores, "kind": "port",
            "cpu": cpu_model(),
            "sample": f"the first {sample} tokens of the {what} ({T} tokens), router + experts in "
                      f"float32 (per-expert dequant + GEMMs), median of 3 ({tm:.2f} s each)"}


def bench_norm(T: int, reps: int = 50) -> dict:
    """The post-attention RMSNorm of one gpt-oss layer (H = 2880, bf16
    activations, float32 weight as transformers loads it): the fused kernels
    against the eager transformers module.

    ``fused_*_gpu_us``: GPU time per call of the fused kernels, from ``reps``
    calls captured in one HIP graph and replayed between two HIP events (no
    host launch cost).  ``*_fwd_us`` / ``*_fwd_bwd_us``: the module's forward,
    and forward plus autograd input gradient, launched from the host as a
    model issues them (launch cost included), mean of ``reps`` calls.  The
    eager module stays out of graph capture (its reductions may record
    memset nodes)."""
    from blockstreamer_amd import gptoss, kernels

    dev = torch.device("cuda", 0)
    H, eps = PREFILL.H, 1e-5
    gen = torch.Generator().manual_seed(11)
    w = (torch.randn(H, generator=gen) * 0.3 + 1.0).to(dev)
    x = torch.randn(T, H, generator=gen).to(torch.bfloat16).to(dev)
    dy = (torch.randn(T, H, generator=gen) * 0.1).to(torch.bfloat16).to(dev)
    fused = gptoss.FusedRMSNorm(H, eps, torch.float32, dev)
    with torch.no_grad():
        fused.weight.copy_(w)
    fused.weight.requires_grad_(False)
    try:
        from transformers.models.gpt_oss.modeling_gpt_oss import GptOssRMSNorm
        eager = GptOssRMSNorm(H, eps=eps).to(dev)
        with torch.no_grad():
            eager.weight.copy_(w)
        eager.weight.requires_grad_(False)
    except ImportError:
        eager = None

    def graph_us(fn):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for _ in range(reps):
                fn()
        graph.replay()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        graph.replay()
        b.record()
        torch.cuda.synchronize()
        return round(a.elapsed_time(b) / reps * 1e3, 2)

    def host_us(fn):
        for _ in range(3):
            fn()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(reps):
            fn()
        b.record()
        torch.cuda.synchronize()
        return round(a.elapsed_time(b) / reps * 1e3, 2)

    def fwd_bwd(mod):
        xr = x.detach().requires_grad_(True)
        return lambda: torch.autograd.grad(mod(xr), [xr], dy)

    res = {"tokens": T, "hidden": H}
    with torch.no_grad():
        res["fused_fwd_gpu_us"] = graph_us(lambda: kernels.rmsnorm_forward(x, w, eps))
        res["fused_bwd_gpu_us"] = graph_us(lambda: kernels.rmsnorm_backward(dy, x, w, eps))
        res["fused_fwd_us"] = host_us(lambda: fused(x))
        if eager is not None:
            res["eager_fwd_us"] = host_us(lambda: eager(x))
    res["fused_fwd_bwd_us"] = host_us(fwd_bwd(fused))
    if eager is not None:
        res["eager_fwd_bwd_us"] = host_us(fwd_bwd(eager))
    # algorithmic HBM bytes: forward reads x and writes y, the input gradient
    # reads x and dy and writes dx; the weight is read once
    fwd_bytes, bwd_bytes = 2 * T * H * 2 + 4 * H, 3 * T * H * 2 + 4 * H
    res["fused_fwd_GB_per_s"] = round(fwd_bytes / (res["fused_fwd_gpu_us"] * 1e-6) / 1e9, 1)
    res["fused_bwd_GB_per_s"] = round(bwd_bytes / (res["fused_bwd_gpu_us"] * 1e-6) / 1e9, 1)
    return res


# gpt-oss attention (both sizes): 64 query heads, 8 key/value heads, head_dim
# 64, sliding window 128 on alternate layers (TF/models/gpt_oss/configuration_gpt_oss.py)
ATTN_HQ, ATTN_HKV, ATTN_D, ATTN_WINDOW = 64, 8, 64, 128


def attn_pairs(Tq: int, Tk: int, causal: bool, window: int) -> int:
    """Visible (query, key) pairs of one head."""
    if not causal:
        return Tq * Tk
    off = Tk - Tq
    return sum(off + t + 1 if window <= 0 else min(off + t + 1, window) for t in range(Tq))


def bench_attention(kind: str, steps: int, warmup: int, eager: bool = True, batch: int = 64) -> dict:
    """The attention core of a gpt-oss layer on the HIP kernels.

    prefill: one 8192-token sequence, causal (the full-attention layers) and
    causal with the 128-token window (the sliding layers), forward and the
    gradients of q, k, v.  decode: ``batch`` sequences (64 by default), one new
    token each, against 4096 cached keys; below 512 (row block, key head,
    sequence) workgroups the forward splits each sequence's keys over several
    workgroups (``single_launch_fwd_ms``: the unsplit launch beside it).  Inputs in the layout the projections produce
    ([B, T, H, 64] viewed [B, H, T, 64]), bf16, float32 sinks.

    Roofline: prefill against the bf16 MFMA peak with algorithmic flops
    (4 * 64 per visible (query, key, head) triple forward: q.k and p.v; 2.5x
    that backward: dP, dV, dK, dQ and the recomputed S); decode against HBM
    with its algorithmic bytes (each visible key and value row of every key
    head read once, q read and out written once); ``fwd_graph_us`` is the
    decode forward's GPU time from a replayed HIP graph (no host launch cost),
    ``graph_GB_per_s`` its rate.  ``eager_*``: transformers'
    eager_attention_forward on the same GPU, the reference's attention."""
    from blockstreamer_amd import attention as A

    dev = torch.device("cuda", 0)
    B, Tq, Tk = (1, 8192, 8192) if kind == "prefill" else (batch, 1, 4096)
    Hq, Hkv, D = ATTN_HQ, ATTN_HKV, ATTN_D
    scaling = D ** -0.5
    gen = torch.Generator().manual_seed(5)
    q = torch.randn(B, Tq, Hq, D, generator=gen).to(torch.bfloat16).to(dev).transpose(1, 2)
    k = torch.randn(B, Tk, Hkv, D, generator=gen).to(torch.bfloat16).to(dev).transpose(1, 2)
    v = torch.randn(B, Tk, Hkv, D, generator=gen).to(torch.bfloat16).to(dev).transpose(1, 2)
    sinks = (torch.randn(Hq, generator=gen) * 2).to(dev)
    dout = torch.randn(B, Tq, Hq, D, generator=gen).to(torch.bfloat16).to(dev)

    def timed(fn, n):
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(n):
            fn()
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) / n

    res = {"batch": B, "q_len": Tq, "kv_len": Tk, "heads": Hq, "kv_heads": Hkv, "head_dim": D}
    for name, window in (("full", 0), ("sliding", ATTN_WINDOW)):
        pairs = attn_pairs(Tq, Tk, True, window) * B * Hq
        out, lse = A.attention_forward(q, k, v, sinks, scaling, True, window, return_lse=True)
        ms = timed(lambda: A.attention_forward(q, k, v, sinks, scaling, True, window, return_lse=True), steps)
        r = {"fwd_ms": round(ms, 4)}
        if kind == "prefill":
            fl = 4 * D * pairs
            r["fwd_TFLOP_per_s"] = round(fl / (ms * 1e-3) / 1e12, 1)
            r["fwd_roofline"] = {"bound": "mfma", "achieved": r["fwd_TFLOP_per_s"], "peak": 2500.0,
                                 "unit": "TFLOP/s", "frac": round(r["fwd_TFLOP_per_s"] / 2500.0, 4)}
            bms = timed(lambda: A.attention_backward(dout, q, k, v, sinks, out, lse, scaling, True, window), steps)
            r["bwd_ms"] = round(bms, 4)
            r["bwd_TFLOP_per_s"] = round(2.5 * fl / (bms * 1e-3) / 1e12, 1)
            r["bwd_roofline_frac"] = round(r["bwd_TFLOP_per_s"] / 2500.0, 4)
        else:
            keys = min(Tk, window) if window else Tk
            byt = B * Hkv * keys * D * 2 * 2 + 2 * B * Tq * Hq * D * 2
            r["hbm_bytes"] = byt
            r["GB_per_s"] = round(byt / (ms * 1e-3) / 1e9, 1)
            r["roofline"] = {"bound": "hbm", "achieved": r["GB_per_s"], "peak": 8000.0, "unit": "GB/s",
                             "frac": round(r["GB_per_s"] / 8000.0, 4)}
            from blockstreamer_amd import _lib
            r["key_splits_workspace_bytes"] = int(_lib.lib().bsa_attention_split_workspace_bytes(
                B, Tq, Tk, Hq, Hkv, 1, window))
            if r["key_splits_workspace_bytes"]:
                o1 = torch.empty(B, Tq, Hq, D, dtype=torch.bfloat16, device=dev)
                s32 = sinks.float().contiguous()

                def single():
                    _lib.call("bsa_attention_fwd", q.data_ptr(), A._strides(q, 2, 1), k.data_ptr(),
                              A._strides(k, 2, 1), v.data_ptr(), A._strides(v, 2, 1), s32.data_ptr(), B, Tq, Tk,
                              Hq, Hkv, D, 1, window, scaling, o1.data_ptr(), A._strides(o1, 1, 2), None,
                              _lib.stream_handle(dev))
                r["single_launch_fwd_ms"] = round(timed(single, steps), 4)
            # GPU time without the host: ten calls captured in one HIP graph, replayed
            def graph_us(fn):
                fn()
                torch.cuda.synchronize()
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g):
                    for _ in range(10):
                        fn()
                g.replay()
                torch.cuda.synchronize()
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                for _ in range(5):
                    g.replay()
                e1.record()
                torch.cuda.synchronize()
                return e0.elapsed_time(e1) / 50 * 1e3
            gus = graph_us(lambda: A.attention_forward(q, k, v, sinks, scaling, True, window))
            r["fwd_graph_us"] = round(gus, 2)
            r["graph_GB_per_s"] = round(byt / (gus * 1e-6) / 1e9, 1)
            if r["key_splits_workspace_bytes"]:
                r["single_launch_graph_us"] = round(graph_us(single), 2)
        res[name] = r
    if eager and kind == "prefill":
        try:
            from transformers.masking_utils import causal_mask_function, eager_mask
            from transformers.models.gpt_oss.modeling_gpt_oss import eager_attention_forward

            class _M(torch.nn.Module):
                pass
            mod = _M()
            mod.sinks = sinks.to(torch.bfloat16)
            mod.num_key_value_groups = Hq // Hkv
            mask = eager_mask(B, Tq, Tk, mask_function=causal_mask_function, dtype=torch.bfloat16, device=dev)
            with torch.no_grad():
                ms = timed(lambda: eager_attention_forward(mod, q, k, v, mask, scaling=scaling), 2)
            res["eager_full_fwd_ms"] = round(ms, 3)
            del mask
            torch.cuda.empty_cache()
        except (ImportError, torch.OutOfMemoryError) as exc:  # noqa: PERF203
            res["eager_full_fwd_ms"] = f"not run: {type(exc).__name__}"
    return res


def bench_copy(steps: int, warmup: int) -> dict:
    """torch device-to-device copy of 2 GiB: 4 GiB of HBM traffic per step."""
    dev = torch.device("cuda", 0)
    src = torch.empty(2 << 30, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    for _ in range(warmup):
        dst.copy_(src)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        dst.copy_(src)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return {"bytes_per_step": 2 * src.numel(), "GB_per_s": round(2 * src.numel() * steps / wall / 1e9, 1),
            "ms_per_step": round(wall / steps * 1e3, 4)}


def focused(args) -> int:
    if args.workload == "copy":
        res = bench_copy(args.steps, args.warmup)
    elif args.workload == "attention":
        res = {"attention_prefill": bench_attention("prefill", args.steps, args.warmup),
               "attention_decode": bench_attention("decode", args.steps, args.warmup),
               "attention_decode_b1": bench_attention("decode", args.steps, args.warmup, batch=1),
               "attention_decode_b8": bench_attention("decode", args.steps, args.warmup, batch=8)}
    elif args.workload == "norm":
        res = {"norm": [bench_norm(t, reps=max(args.steps, 20)) for t in (64, 8192)]}
    elif args.workload == "moe_decode":
        res = bench_moe(DECODE, args.tokens, args.steps, args.warmup, path=args.path, layout=args.layout)
    elif args.workload == "moe_20b":
        res = bench_moe(LAYER_20B, 2048, args.steps, args.warmup, path=args.path, layout=args.layout)
    elif args.workload == "moe_prefill_train":
        res = bench_moe(PREFILL, 8192, args.steps, args.warmup, path=args.path, layout=args.layout,
                        train=True, fwd=False)
    else:
        res = bench_moe(PREFILL, 8192, args.steps, args.warmup, path=args.path, layout=args.layout)
    print(json.dumps({"workload": args.workload, "steps": args.steps, "warmup": args.warmup, **res}),
          flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default="dequant",
                    choices=["dequant", "moe_decode", "moe_20b", "moe_prefill", "moe_prefill_train", "copy",
                             "norm", "attention"],
                    help="dequant: the headline line (plus MoE layer results); moe_decode / moe_20b / "
                         "moe_prefill: one MoE layer forward alone; moe_prefill_train: the 8192-token "
                         "forward that saves for the backward plus the input-gradient backward; copy: a "
                         "plain 2 GiB device copy that calibrates the HBM byte counters; norm: the "
                         "post-attention RMSNorm, fused and eager; attention: the attention core "
                         "(prefill 8192 tokens and decode), against transformers' eager attention")
    ap.add_argument("--path", default="auto", choices=["auto", "stream", "tiled", "mx"],
                    help="expert GEMM kernels for the MoE workloads (auto: weight streaming for decode, "
                         "the two-term MX kernels for prefill)")
    ap.add_argument("--tokens", type=int, default=64, choices=[1, 8, 64],
                    help="token batch of the moe_decode workload (the decode batches 1, 8 and 64)")
    ap.add_argument("--layout", default="checkpoint", choices=["checkpoint", "kpair"],
                    help="layout of the packed blocks for the moe_decode / moe_prefill workloads")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-moe", action="store_true", help="skip the MoE layer measurements")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build runs the MoE expert path on a "
              "single MI355X (no multi-GPU path); run with --gpus 1", file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 2
    if args.workload != "dequant":
        return focused(args)
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
    if not args.no_moe:
        # the prefill lines take the full step count: with 5 timed steps they read
        # 5-8 % slower than in steady state (measured, same box)
        n_pre = max(args.steps, 10)
        moe = {
            "decode_t1": bench_moe(DECODE, 1, max(args.steps, 20), args.warmup),
            "decode_t8": bench_moe(DECODE, 8, max(args.steps, 20), args.warmup),
            "decode_t64": bench_moe(DECODE, 64, max(args.steps, 20), args.warmup),
            # gpt-oss-20b-shaped layer: 32 experts, top-4, 2048 tokens
            "layer_20b_t2048": bench_moe(LAYER_20B, 2048, max(args.steps, 10), args.warmup, ref=True),
            # the 8192-token prefill on the native block-scaled MX kernels
            # (auto), with the LoRA training use, beside the dequant-to-bf16
            # tiled kernels
            "prefill_t8192": bench_moe(PREFILL, 8192, n_pre, args.warmup, train=True, ref=True),
            "prefill_t8192_bf16": bench_moe(PREFILL, 8192, n_pre, args.warmup, path="tiled", ref=True),
            # the same workloads with the blocks in the k-pair shard layout
            "decode_t64_kpair": bench_moe(DECODE, 64, max(args.steps, 20), args.warmup, layout="kpair"),
            "prefill_t8192_kpair": bench_moe(PREFILL, 8192, n_pre, args.warmup, layout="kpair", ref=True),
            "prefill_t8192_bf16_kpair": bench_moe(PREFILL, 8192, n_pre, args.warmup, path="tiled",
                                                  layout="kpair", ref=True),
        }
        if not args.no_cpu_baseline:
            moe["decode_t64"]["cpu_baseline"] = cpu_baseline_moe(DECODE, 64, 64, "gpt-oss-120b decode batch")
            moe["layer_20b_t2048"]["cpu_baseline"] = cpu_baseline_moe(LAYER_20B, 2048, 256,
                                                                      "gpt-oss-20b layer batch")
            moe["prefill_t8192"]["cpu_baseline"] = cpu_baseline_moe(PREFILL, 8192, 64,
                                                                    "gpt-oss-120b prefill batch")
        line["moe_layer"] = moe
        line["post_attention_norm"] = {"t64": bench_norm(64), "t8192": bench_norm(8192)}
        line["attention"] = {"prefill_t8192": bench_attention("prefill", max(args.steps // 2, 5), args.warmup),
                             "decode_b64_kv4096": bench_attention("decode", max(args.steps, 20), args.warmup),
                             "decode_b1_kv4096": bench_attention("decode", max(args.steps, 20), args.warmup,
                                                                 batch=1)}
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
