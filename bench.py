"""Benchmark of the weight-quantized linear layer on one MI355X.

Default workload — the BASELINE.json metric, configs[1]'s up-projection: X bf16 [4096, 3072] ~ N(0,1),
W int8 [K=3072, N=12288] (the reference map's [K, N] layout) with codes uniform in [−127, 127],
per-output-channel fp32 scales U(1e−3, 2e−2), bias N(0, 0.02), fused GELU(tanh), bf16 output.
`--workload` selects the other configurations of the scope table (C0, C1 down, C2 fused QKV and
skinny, C3 fp8) with the same JSON line; the driver's line is the default one.

A step is one launch of the fused product on inputs already in HBM, the weight staged once by
sq8_pack_weight (`--layout packed`, the default) or read in place. Inputs are synthetic and seeded
(SplitMix64 + Box–Muller, the reference's generator, Sources/Verification/KernelStages.swift:553-567);
the seeds are in the JSON.

value = 2·M·N·K / (average kernel time), the kernel timed with HIP events on the stream it is
launched on, over the timed steps, after enough warm-up for the clocks to settle. roofline: the
dense bf16 MFMA peak (2.5 PFLOP/s) where the arithmetic intensity is above the HBM ridge
(2.5e15 / 8e12 = 312.5 FLOP/B), else the HBM peak (8 TB/s) on the algorithmic bytes.
cpu_baseline: the reference's CPU route restated (Widen.dequantize → fp32 GEMM → bias → activation,
WeightProducts.swift:698-709, Ops.swift:386-407) on a sample of the rows, run on the host cores of
the GPU box and scaled to the whole step.
"""
from __future__ import annotations

import argparse
import gc
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA, published
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E, published
RIDGE = PEAK_BF16_TFLOPS * 1e12 / (PEAK_HBM_GBS * 1e9)
# HBM bytes per launch of the product kernel (FETCH_SIZE × 2 + WRITE_SIZE × 1, the factors from a
# 512 MiB copy of the same session), by (workload, weight layout), with the profiles/ summary that records
# the rocprofv3 --pmc runs they come from; the line reports both, so a kernel change that leaves a figure
# stale is visible (take the runs again with the commands in that summary).
_TRAFFIC_SRC = "profiles/hbm_traffic_by_workload.md"
TRAFFIC = {
    ("c1_up", "packed"): (403.6e6, _TRAFFIC_SRC),
    ("c2_skinny", "packed"): (34.91e6, _TRAFFIC_SRC),
    ("c0", "packed"): (56.98e6, _TRAFFIC_SRC),
    ("skinny_m1", "packed"): (9.68e6, _TRAFFIC_SRC),
    ("skinny_m16", "packed"): (10.52e6, _TRAFFIC_SRC),
    ("skinny_m64", "packed"): (13.18e6, _TRAFFIC_SRC),
    ("c1_down", "packed"): (450.35e6, _TRAFFIC_SRC),
    ("c2_qkv", "packed"): (415.51e6, _TRAFFIC_SRC),
    ("c3_gate_up", "packed"): (715.93e6, _TRAFFIC_SRC),
    ("c3_down", "packed"): (367.51e6, _TRAFFIC_SRC),
    ("c3_plain", "packed"): (478.92e6, _TRAFFIC_SRC),
    ("c1_w8a8", "packed"): (472.42e6, _TRAFFIC_SRC),
    ("c1_q8", "packed"): (592.23e6, _TRAFFIC_SRC),
    ("c1_f32", "packed"): (1007.54e6, _TRAFFIC_SRC),
    ("c1_convrot", "packed"): (403.59e6, _TRAFFIC_SRC)}
GAMMA = np.uint64(0x9E3779B97F4A7C15)

# name: M, K, N, weight type, epilogue, activation distribution, description.
WORKLOADS = {
    "c1_up": (4096, 3072, 12288, "int8", "gelu_tanh", "normal",
              "C1 up-projection: int8 weight [K,N] per-channel fp32 scale, bf16 X, bias + fused GELU-tanh, bf16 out"),
    "c1_down": (4096, 12288, 3072, "int8", None, "gelu",
                "C1 down-projection on the GELU output: int8 weight, bias, bf16 out"),
    "c0": (1024, 3072, 3072, "int8", None, "normal",
           "C0: int8 weight [3072, 3072] per-channel scale, bias, bf16 out"),
    "c2_qkv": (4608, 3072, 9216, "int8", "qkv", "normal",
               "C2 fused QKV (4096 image + 512 text tokens): int8 weight [9216, 3072], bias, Q/K/V [4608, 3072] bf16"),
    "c2_skinny": (512, 3072, 3072, "int8", None, "normal",
                  "C2 skinny text stream: int8 weight [3072, 3072], bias, bf16 out"),
    # Short rows on C2's text-stream weight (3072 x 3072): the bandwidth-bound end of the skinny path.
    "skinny_m1": (1, 3072, 3072, "int8", None, "normal", "one row on an int8 weight [3072, 3072], bias, bf16 out"),
    "skinny_m16": (16, 3072, 3072, "int8", None, "normal", "16 rows on an int8 weight [3072, 3072], bias, bf16 out"),
    "skinny_m64": (64, 3072, 3072, "int8", None, "normal", "64 rows on an int8 weight [3072, 3072], bias, bf16 out"),
    "c3_gate_up": (4096, 3840, 20480, "fp8", "silu_glu", "normal",
                   "C3 fp8-e4m3 gate+up fused (2 x 10240) with SiLU-GLU, bf16 out [4096, 10240]"),
    "c3_down": (4096, 10240, 3840, "fp8", None, "silu",
                "C3 fp8-e4m3 down-projection [3840, 10240], bias, bf16 out"),
    "c3_plain": (4096, 3840, 12288, "fp8", None, "normal",
                 "C3 plain fp8-e4m3 linear W [12288, 3840], bias, bf16 out"),
    "c1_convrot": (4096, 3072, 12288, "int8", "gelu_tanh", "normal",
                   "C1 up-projection on a convrot int8 weight (groups of 256): fp32 X rotated and rounded to bf16, "
                   "then the product with bias + fused GELU-tanh, bf16 out"),
    "c1_w8a8": (4096, 3072, 12288, "int8", "gelu_tanh", "normal",
                "C1 up-projection on the W8A8 route (ComfyUI int8_linear): fp32 X rotated (groups of 256) and quantized "
                "per row to int8, int8 x int8 products summed in int32, float(acc)*(s_x*s_w) + bias, fused GELU-tanh, bf16 out"),
    "c1_q8": (4096, 3072, 12288, "q8_0", "gelu_tanh", "normal",
              "C1 up-projection on a GGUF Q8_0 weight: int8 codes [N,K] with one fp16 scale per 32 K of each output "
              "(sq8_linear_blocks), bf16 X, bias + fused GELU-tanh, bf16 out"),
    "c1_f32": (4096, 3072, 12288, "int8", "gelu_tanh", "normal",
               "C1 up-projection on the fp32 route: fp32 X used whole, not rounded (three exact bf16 parts along K, "
               "sq8_linear_f32), int8 weight, bias + fused GELU-tanh, bf16 out"),
}
Q8_BLOCK = 32
# Workloads on the fp32 route: the activation fp32, used whole; a step is the split pass and the
# product on its three parts (3K steps of K), both inside the one sq8_linear_f32 call.
EXACT = {"c1_f32"}
# Workloads whose weight is ComfyUI's convrot: the rotation group. Their activation is fp32 (the
# reference's rotate_groups reads fp32, TensorGEMM.swift:181-201) and a step is the rotation pass
# (fp32 → bf16, or fp32 → int8 codes and row scales on the W8A8 route) followed by the product —
# the two kernels sq8_linear_rotated / sq8_linear_quantized run.
ROTATED = {"c1_convrot": 256, "c1_w8a8": 256}
W8A8 = {"c1_w8a8"}
PEAK_INT8_TOPS = 5000.0     # MI355X dense int8 MFMA, published
SEEDS = {"x": 1, "w": 2, "scale": 3, "bias": 4}


def splitmix(seed: int, start: int, count: int) -> np.ndarray:
    """Outputs start+1 .. start+count of SplitMix64 from `seed` (state_i = seed + i·γ, then the mix)."""
    with np.errstate(over="ignore"):
        z = np.uint64(seed) + GAMMA * np.arange(start + 1, start + count + 1, dtype=np.uint64)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        return z ^ (z >> np.uint64(31))


def uniform(seed: int, count: int, start: int = 0) -> np.ndarray:
    return (splitmix(seed, start, count) >> np.uint64(11)).astype(np.float64) / 9007199254740992.0


def normal_f32(seed: int, count: int, chunk: int = 1 << 24) -> np.ndarray:
    """Box–Muller of consecutive uniform pairs, by chunks (bounded memory)."""
    out = np.empty(count, dtype=np.float32)
    for i in range(0, count, chunk):
        c = min(chunk, count - i)
        u = uniform(seed, 2 * c, start=2 * i)
        out[i:i + c] = np.sqrt(-2.0 * np.log(np.maximum(u[0::2], 1e-300))) * np.cos(2.0 * np.pi * u[1::2])
    return out


def inputs(workload: str):
    """X bf16 [M, K] (a torch tensor), codes [K, N] (numpy int8) or [N, K] (torch float8_e4m3fn; Q8_0:
    numpy int8), scales fp32 [N] (Q8_0: fp16 [N, K/32]), bias fp32 [N]."""
    import torch
    M, K, N, wt, epi, xdist, _ = WORKLOADS[workload]
    x = torch.from_numpy(normal_f32(SEEDS["x"], M * K).reshape(M, K))
    if xdist == "gelu":  # the up-projection's output
        x = torch.nn.functional.gelu(x, approximate="tanh")
    elif xdist == "silu":  # a SiLU-GLU output: silu(g)·u of two N(0,1)
        u = torch.from_numpy(normal_f32(SEEDS["x"] + 100, M * K).reshape(M, K))
        x = torch.nn.functional.silu(x) * u
    x = x.to(torch.bfloat16)
    b = (0.02 * normal_f32(SEEDS["bias"], N)).astype(np.float32)
    if wt == "int8":
        q = (np.floor(uniform(SEEDS["w"], K * N) * 255.0) - 127.0).clip(-127, 127).astype(np.int8).reshape(K, N)
        s = (1e-3 + (2e-2 - 1e-3) * uniform(SEEDS["scale"], N)).astype(np.float32)
        return x, q, s, b
    if wt == "q8_0":
        # GGUF Q8_0 as published: codes [N, K], one fp16 scale d per 32 consecutive K of an output.
        q = (np.floor(uniform(SEEDS["w"], K * N) * 255.0) - 127.0).clip(-127, 127).astype(np.int8).reshape(N, K)
        d = (1e-3 + (2e-2 - 1e-3) * uniform(SEEDS["scale"], N * (K // Q8_BLOCK))).astype(np.float16)
        return x, q, d.reshape(N, K // Q8_BLOCK), b
    # fp8: w ~ N(0, 0.02) [N, K], s_n = amax_n / 448, q = e4m3fn(RNE(w / s)) (|w / s| ≤ 448: no saturation)
    w = torch.from_numpy(normal_f32(SEEDS["w"], N * K).reshape(N, K)) * 0.02
    s = (w.abs().amax(dim=1) / 448.0).clamp_min(1e-30)
    q = (w / s[:, None]).to(torch.float8_e4m3fn)
    return x, q, s.numpy().astype(np.float32), b


def cpu_baseline(workload: str, x_bf16, q, s, b, budget_s: float = 12.0, x32=None):
    """The reference's CPU route on a sample of rows: the whole weight widened (oracle dequantiser,
    every core; a convrot weight with its rotation, Widen.dequantizeRotated), the sample's fp32 GEMM
    (numpy's BLAS, the cblas_sgemm of the reference) on the bf16 activation or, for a convrot weight,
    the fp32 one, bias + activation in fp32 (oracle). Repeated for about `budget_s`; scaled to all M
    rows."""
    from oracle import oracle
    M, K, N, wt, epi, _, _ = WORKLOADS[workload]
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    rows = min(512, M)
    group = ROTATED.get(workload)
    a32 = x32[:rows] if x32 is not None else oracle.bf16_to_f32(x_bf16[:rows].view(np.uint16))
    if wt == "int8":
        codes, kind = q.view(np.uint8), oracle.INT8            # [K, N], scales per column
    elif wt == "q8_0":
        codes, kind = np.ascontiguousarray(q.T).view(np.uint8), oracle.INT8   # [N, K] → [K, N], scales [K/32, N]
    else:
        codes, kind = np.ascontiguousarray(q.view(np.uint8).T), oracle.FP8_E4M3   # [N, K] → [K, N]
    e = {"gelu_tanh": oracle.EPI_GELU_TANH, "silu_glu": oracle.EPI_SILU_GLU}.get(epi, oracle.EPI_NONE)
    t_deq, t_gemm, reps = 0.0, 0.0, 0
    start = time.perf_counter()
    while time.perf_counter() - start < budget_s or reps < 2:
        t0 = time.perf_counter()
        if group:
            w = oracle.dequantize_rotated(q, group, s)
        elif wt == "q8_0":
            w = oracle.dequantize(codes, kind, np.ascontiguousarray(s.T).view(np.uint16), oracle.F16,
                                  oracle.SCALE_BLOCKS, columns=N, block_rows=Q8_BLOCK)
        else:
            w = oracle.dequantize(codes, kind, s, oracle.F32, oracle.SCALE_COLUMNS, columns=N)
        t1 = time.perf_counter()
        y = oracle.epilogue_f32(a32 @ w.reshape(K, N), bias=b, epilogue=e, threads=threads)
        t2 = time.perf_counter()
        t_deq += t1 - t0
        t_gemm += t2 - t1
        reps += 1
        del w, y
    t_step = t_deq / reps + (t_gemm / reps) * (M / rows)
    return {
        "value": round(2.0 * M * N * K / t_step / 1e12, 4),
        "unit": "TFLOP/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"{rows} of {M} rows × the whole weight, {reps} repetitions in {time.perf_counter() - start:.1f} s: "
                   f"widen {1e3 * t_deq / reps:.1f} ms + GEMM/bias/activation {1e3 * t_gemm / reps:.1f} ms per "
                   f"repetition; step = widen + GEMM×{M / rows:g}"),
        "ms_per_step": round(1e3 * t_step, 2),
    }


def derived_peak(cus: int) -> dict:
    """The dense bf16 MFMA peak re-derived on this box: CUs × max shader clock × 4096 FLOP per clock per
    CU (the clock from hipDeviceGetAttribute, hipDeviceAttributeClockRate = 5, in kHz). The roofline
    uses the published 2.5 PFLOP/s; this is printed beside it."""
    out = {"cus": cus}
    try:
        import ctypes
        lib = ctypes.CDLL("libamdhip64.so")
        khz = ctypes.c_int(0)
        if lib.hipDeviceGetAttribute(ctypes.byref(khz), 5, 0) == 0 and 100_000 <= khz.value <= 10_000_000:
            out.update({"max_sclk_mhz": khz.value / 1e3, "bf16_dense_tflops": round(cus * khz.value * 1e3 * 4096 / 1e12, 1)})
    except OSError:
        pass
    return out


def settle(step, settle_ms: float) -> dict:
    """The clock-settle phase: `step` launched back to back until `settle_ms` of wall time has passed
    (synchronizing every few launches so the time is the GPU's). The shader clock of this chip ramps
    over the first tens of milliseconds of sustained MFMA work and the power limit then sets it; a
    measurement that starts cold times the ramp. Returns what ran."""
    import torch
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    launches = 0
    while True:
        for _ in range(8):
            step()
        launches += 8
        torch.cuda.synchronize()
        if 1e3 * (time.perf_counter() - t0) >= settle_ms:
            break
    return {"settle_ms": round(1e3 * (time.perf_counter() - t0), 1), "settle_launches": launches}


def launch_stats(times_ms) -> dict:
    """Per-launch statistics of the timed steps (each bracketed by its own HIP events)."""
    t = sorted(times_ms)
    return {"min": round(t[0], 5), "median": round(float(np.median(t)), 5), "max": round(t[-1], 5)}


def c4_measure(route: str, steps: int, warmup: int, settle_ms: float) -> dict:
    """One synthetic single-stream DiT block forward (siliconed_amd.dit_block) on `route` ("bf16", or
    "w8a8" with convrot 256): hidden 3072, 24 heads of 128, 4096 image + 512 text tokens. Each timed
    forward is bracketed by its own HIP events; returns the median forward as `ms`, the mean beside it."""
    import torch
    from siliconed_amd.dit_block import DiTBlock
    S, d, heads = 4096 + 512, 3072, 24
    w8a8 = route == "w8a8"
    blk = DiTBlock(d=d, heads=heads, mlp=4, seed=SEEDS["w"], route=route, group=256 if w8a8 else 0)
    x = torch.from_numpy(normal_f32(SEEDS["x"], S * d).reshape(S, d)).cuda()
    temb = torch.from_numpy(normal_f32(SEEDS["bias"], d)).cuda()
    # The block updates its residual stream in place (as the reference's stream buffer): each step
    # gets its own copy of x, made before the timed region; the settle and warm-up forwards reuse one.
    streams = [x.clone() for _ in range(steps)]
    work = x.clone()
    gc.collect()
    st = settle(lambda: blk.forward_(work, temb), settle_ms)
    for _ in range(warmup):
        blk.forward_(work, temb)
    torch.cuda.synchronize()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    gc.disable()  # no collector pause while the timed forwards are queued
    try:
        t0 = time.perf_counter()
        ev[0].record()
        for i in range(steps):
            blk.forward_(streams[i], temb)
            ev[i + 1].record()
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
    finally:
        gc.enable()
    per = [ev[i].elapsed_time(ev[i + 1]) for i in range(steps)]
    mean = ev[0].elapsed_time(ev[steps]) / steps
    # The median forward: a host-side stall between two launches (the GPU then idles until the next one
    # is queued) lands in one forward's events and would move the mean, not the median.
    ms = float(np.median(per))
    flops = blk.flops(S)
    out = {"ms": round(ms, 4), "mean_ms": round(mean, 4), "per_forward_ms": launch_stats(per),
           "tflops": round(flops / (ms * 1e-3) / 1e12, 2), "flops": flops, "steps": steps, "warmup": warmup,
           "wall_ms_per_step": round(1e3 * wall / steps, 4), **st}
    del blk, streams, work, x
    torch.cuda.empty_cache()
    return out


def dit_block(args) -> int:
    """C4: one synthetic single-stream DiT block forward (siliconed_amd.dit_block): hidden 3072, 24
    heads of 128, 4096 image + 512 text tokens, int8 per-channel modulation / QKV / out / MLP-4×
    weights, bf16 attention, fp32 residual. value: the block's forward time in ms (HIP events over the
    timed forwards, the median forward); `tflops` beside it (linear + attention FLOPs over that time)."""
    S, d, heads = 4096 + 512, 3072, 24
    w8a8 = args.workload == "c4_block_w8a8"
    steps = max(args.steps // 2, 5)
    warm = max(args.warmup // 20, 2)
    r = c4_measure("w8a8" if w8a8 else "bf16", steps, warm, args.settle_ms)
    ms, flops, tflops = r["ms"], r["flops"], r["tflops"]
    result = {
        "metric": ("DiT block forward ms (hidden 3072, 24x128 heads, 4608 tokens, int8 weights"
                   + (", W8A8 route, convrot 256" if w8a8 else "") + ") on 1 MI355X"),
        "value": round(ms, 4), "unit": "ms", "tflops": round(tflops, 2), "n_gpus": 1, "steps": steps,
        "warmup": warm, "settle_ms": r["settle_ms"], "mean_ms": r["mean_ms"], "per_forward_ms": r["per_forward_ms"],
        "ms_per_step": r["wall_ms_per_step"], "higher_is_better": False,
        "scaling": "weak", "vs_baseline": None, "dtype": "int8" if w8a8 else "bf16",
        "data": f"synthetic, seeded: x, temb SplitMix64 + Box-Muller; weights torch generator seed {SEEDS['w']}",
        "config": {"workload": f"{args.workload}: one single-stream DiT block (modulation, modulated RMSNorm, fused QKV, "
                               "per-head RMSNorm, SDPA, Wo, GELU MLP 4x, gated residuals)"
                               + ("; products W8A8 (int8 activations quantized per row after a convrot rotation of 256, "
                                  "the norms writing the QKV and W_up codes)" if w8a8 else ""),
                   "tokens": S, "hidden": d, "heads": heads,
                   "flops": flops, "global_batch": S, "parallelism": "none (one GPU)"},
        "pct_bf16_peak": round(100.0 * tflops / PEAK_BF16_TFLOPS, 2),
    }
    print(json.dumps(result), flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=20)
    # The clocks reach their steady state only after ~50 ms of sustained work: a short warm-up counted
    # in steps leaves the first timed steps ~30 % slow (0.36 ms against 0.27 ms each on the default
    # workload). The settle phase runs the same step for a fixed time before the counted warm-up.
    ap.add_argument("--settle-ms", type=float, default=400.0,
                    help="wall time of back-to-back steps before the counted warm-up (clock settle)")
    ap.add_argument("--no-c4", action="store_true",
                    help="default workload only: skip the C4 block forwards reported beside the line")
    ap.add_argument("--workload", choices=sorted(WORKLOADS) + ["c4_block", "c4_block_w8a8"], default="c1_up")
    ap.add_argument("--layout", choices=["kn", "nk", "packed"], default="packed",
                    help="weight layout the product reads; packed = staged once by sq8_pack_weight")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--operands", choices=["synthetic", "zero-x", "ones-x", "zero-w"], default="synthetic",
                    help="diagnostic: the same launches on constant operands (all activations 0 or 1, or all codes 0), "
                         "which change the power the products draw and so the clock, not the work; the line says so")
    ap.add_argument("--shape", metavar="MxKxN", default=None,
                    help="the workload's product at another M, K, N (same weight type, epilogue and inputs' "
                         "distributions); the line then carries no measured traffic")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="instead of the product, copy MIB MiB device→device --steps times (the known-size kernel "
                         "that calibrates the FETCH_SIZE / WRITE_SIZE counters)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (run with --gpus 1).", file=sys.stderr)
        return 2

    import torch
    import siliconed_amd as sq

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.copy_probe:
        nbytes = args.copy_probe << 20
        src = torch.ones(nbytes // 4, dtype=torch.int32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(args.steps):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_probe_bytes": nbytes, "launches": args.steps}), flush=True)
        return 0

    if args.workload in ("c4_block", "c4_block_w8a8"):
        return dit_block(args)
    if args.shape:
        m_, k_, n_ = (int(v) for v in args.shape.lower().split("x"))
        w_ = list(WORKLOADS[args.workload])
        w_[0:3] = [m_, k_, n_]
        w_[6] = f"{w_[6]} (at {m_} x {k_} x {n_})"
        WORKLOADS[args.workload] = tuple(w_)
    M, K, N, wt, epi, _, desc = WORKLOADS[args.workload]
    fp8 = wt == "fp8"
    q8 = wt == "q8_0"
    glu = epi == "silu_glu"
    qkv = epi == "qkv"
    x, q, s, b = inputs(args.workload)
    if args.operands == "zero-x":
        x = torch.zeros_like(x)
    elif args.operands == "ones-x":
        x = torch.ones_like(x)
    elif args.operands == "zero-w":
        q = np.zeros_like(q) if isinstance(q, np.ndarray) else torch.zeros_like(q)
    xd = x.to(dev)
    sd = torch.from_numpy(s).to(dev)
    bd = torch.from_numpy(b).to(dev)
    ctx = sq.context(0)
    if q8:
        wd, lay = torch.from_numpy(q).to(dev), "nk"          # [N, K] int8 codes, scales [N, K/32] fp16
        sd = torch.from_numpy(s).to(dev)
        if args.layout == "kn":
            wd, sd, lay = wd.t().contiguous(), sd.t().contiguous(), "kn"
    elif fp8:
        wd, lay = q.to(dev), "nk"                           # [N, K] e4m3fn codes (packed from [N, K])
        if args.layout == "kn":
            wd, lay = wd.t().contiguous(), "kn"
    else:
        wd, lay = torch.from_numpy(q).to(dev), "kn"         # [K, N] int8 codes (packed from [K, N])
        if args.layout == "nk":
            wd, lay = wd.t().contiguous(), "nk"
    stage_ms = None
    if args.layout == "packed":
        torch.cuda.synchronize()
        t_stage = time.perf_counter()
        wd = ctx.pack_blocks(wd, sd, Q8_BLOCK, layout=lay, glu=glu) if q8 else ctx.pack(wd, layout=lay, glu=glu)
        torch.cuda.synchronize()
        stage_ms = 1e3 * (time.perf_counter() - t_stage)
    n_out = N // 2 if glu else N
    group = ROTATED.get(args.workload)
    x32 = None
    if group:
        x32 = normal_f32(SEEDS["x"], M * K).reshape(M, K)
        x32d = torch.from_numpy(x32).to(dev)
        xd = torch.empty((M, K), dtype=torch.bfloat16, device=dev)   # the rotated, rounded operand
        out = torch.empty((M, n_out), dtype=torch.bfloat16, device=dev)

        if args.workload in W8A8:
            codes = torch.empty((M, K), dtype=torch.int8, device=dev)
            sx = torch.empty(M, dtype=torch.float32, device=dev)

            def step(marks=None):
                if marks:
                    marks[0].record()
                ctx.quantize_rows(x32d, group, codes=codes, scales=sx)
                if marks:
                    marks[1].record()
                ctx.product_w8a8(codes, sx, wd, sd, layout=lay, bias=bd, epilogue=epi, out=out)
                if marks:
                    marks[2].record()
        else:
            def step(marks=None):
                if marks:
                    marks[0].record()
                ctx.rotate(x32d, group, out=xd)
                if marks:
                    marks[1].record()
                ctx.product(xd, wd, sd, layout=lay, bias=bd, epilogue=epi, out=out)
                if marks:
                    marks[2].record()
    elif args.workload in EXACT:
        x32 = normal_f32(SEEDS["x"], M * K).reshape(M, K)
        x32d = torch.from_numpy(x32).to(dev)
        out = torch.empty((M, n_out), dtype=torch.bfloat16, device=dev)

        def step():
            ctx.product(x32d, wd, sd, layout=lay, bias=bd, epilogue=epi, out=out, rounding=False)
    elif qkv:
        outs = tuple(torch.empty((M, N // 3), dtype=torch.bfloat16, device=dev) for _ in range(3))

        def step():
            ctx.product_qkv(xd, wd, sd, layout=lay, bias=bd, out=outs)
    elif q8:
        out = torch.empty((M, n_out), dtype=torch.bfloat16, device=dev)

        def step():
            ctx.product_blocks(xd, wd, sd, Q8_BLOCK, layout=lay, bias=bd, epilogue=epi, out=out)
    else:
        out = torch.empty((M, n_out), dtype=torch.bfloat16, device=dev)

        def step():
            ctx.product(xd, wd, sd, layout=lay, bias=bd, epilogue=epi, out=out)

    gc.collect()
    settled = settle(step, args.settle_ms)
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    gc.disable()  # no collector pause while the timed steps are queued (enabled again below)
    # Every timed step is bracketed by HIP events on torch's current stream, the stream the context
    # launches on: ev[i] before step i, ev[steps] after the last (rotated workloads: three marks a step,
    # around the activation pass and the product).
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps + 1)]
    marks = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(args.steps)] if group else None
    t0 = time.perf_counter()
    ev[0].record()
    for i in range(args.steps):
        if group:
            step(marks[i])
        else:
            step()
        ev[i + 1].record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    gc.enable()
    step_ms = ev[0].elapsed_time(ev[args.steps]) / args.steps
    per_step = [ev[i].elapsed_time(ev[i + 1]) for i in range(args.steps)]
    kernel_ms = step_ms
    per_kernel = per_step
    rotation = None
    if group:
        # The product kernel's own time (the roofline's), and the rotation pass's, from the marks
        # around each launch; the step (value) is both.
        per_kernel = [m[1].elapsed_time(m[2]) for m in marks]
        kernel_ms = sum(per_kernel) / args.steps
        rot_ms = sum(m[0].elapsed_time(m[1]) for m in marks) / args.steps
        rot_bytes = 4 * M * K + (1 if args.workload in W8A8 else 2) * M * K
        rotation = {"kind": "rotate + quantize to int8" if args.workload in W8A8 else "rotate + round to bf16",
                    "group": group, "ms": round(rot_ms, 5), "algorithmic_bytes": rot_bytes, "bound": "hbm",
                    "achieved": round(rot_bytes / (rot_ms * 1e-3) / 1e9, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                    "frac": round(rot_bytes / (rot_ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)}
    flops = 2.0 * M * N * K
    tflops = flops / (step_ms * 1e-3) / 1e12
    kernel_tflops = flops / (kernel_ms * 1e-3) / 1e12
    w8a8 = args.workload in W8A8
    # int8 codes + row scales, fp32 (the fp32 route), or bf16
    a_bytes = (1 * M * K + 4 * M) if w8a8 else 4 * M * K if args.workload in EXACT else 2 * M * K
    # Codes, their scales as published (fp32 per column, or Q8_0's fp16 per 32 K), bias, output.
    w_bytes = N * K + (2 * N * (K // Q8_BLOCK) if q8 else 4 * N)
    algo_bytes = a_bytes + w_bytes + 4 * N + 2 * M * n_out
    intensity = flops / algo_bytes
    gbs = algo_bytes / (kernel_ms * 1e-3) / 1e9
    peak_mfma = PEAK_INT8_TOPS if w8a8 else PEAK_BF16_TFLOPS
    if intensity >= peak_mfma * 1e12 / (PEAK_HBM_GBS * 1e9):
        roofline = {"bound": "mfma", "achieved": round(kernel_tflops, 2), "peak": peak_mfma,
                    "unit": "TOP/s" if w8a8 else "TFLOP/s", "frac": round(kernel_tflops / peak_mfma, 4)}
    else:
        roofline = {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                    "frac": round(gbs / PEAK_HBM_GBS, 4)}
    traffic, traffic_src = (None, None) if args.shape else TRAFFIC.get((args.workload, args.layout), (None, None))
    roofline.update({"traffic": traffic, "traffic_source": traffic_src,
                     "algorithmic_bytes": algo_bytes,
                     "flops": flops, "intensity_flop_per_byte": round(intensity, 1),
                     "hbm_bound_ms": round(algo_bytes / (PEAK_HBM_GBS * 1e9) * 1e3, 5),
                     "mfma_bound_ms": round(flops / (peak_mfma * 1e12) * 1e3, 5)})
    if args.workload in EXACT:
        # Three bf16 parts per fp32 value: the MFMAs do three times the product's FLOPs.
        roofline.update({"mfma_flops": 3 * flops, "mfma_bound_ms": round(3 * flops / (peak_mfma * 1e12) * 1e3, 5)})

    props = torch.cuda.get_device_properties(0)
    metric = ("TFLOP/s and % bf16 MFMA peak, int8-weight GEMM 4096x3072x12288 on 1 MI355X" if args.workload == "c1_up"
              else f"TOP/s and % int8 MFMA peak, W8A8 GEMM {M}x{K}x{N} on 1 MI355X" if w8a8
              else f"TFLOP/s and % bf16 MFMA peak, {wt}-weight GEMM {M}x{K}x{N} on 1 MI355X")
    result = {
        "metric": metric,
        "value": round(tflops, 2),
        "unit": "TOP/s" if w8a8 else "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(1e3 * wall / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8" if w8a8 else "f32" if args.workload in EXACT else "bf16",
        "data": f"synthetic, seeded (SplitMix64 + Box-Muller), seeds {SEEDS}"
                + ("" if args.operands == "synthetic" else f"; DIAGNOSTIC operands {args.operands}"),
        "config": {"workload": f"{args.workload}: {desc}", "M": M, "K": K, "N": N, "weight_type": wt,
                   "weight_layout": args.layout.upper(),
                   "staging_ms": None if stage_ms is None else round(stage_ms, 3), "global_batch": M,
                   "parallelism": "none (one GPU)"},
        "pct_bf16_peak": round(100.0 * tflops / PEAK_BF16_TFLOPS, 2),
        **({"pct_int8_peak": round(100.0 * tflops / PEAK_INT8_TOPS, 2)} if w8a8 else {}),
        "kernel_ms": round(kernel_ms, 5),
        "kernel_ms_per_launch": launch_stats(per_kernel),
        **settled,
        "roofline": roofline,
        **({"activation_pass": rotation} if rotation else {}),
        "device": {"name": props.name, "cus": props.multi_processor_count,
                   "peak_derived": derived_peak(props.multi_processor_count)},
    }
    if args.workload == "c1_up" and not args.no_c4:
        # C4 (a full DiT block forward, both product routes) beside the headline, so that the default
        # line records it; each route settles its clock first.
        del wd, xd, out
        torch.cuda.empty_cache()
        for route in ("bf16", "w8a8"):
            r = c4_measure(route, steps=10, warmup=2, settle_ms=min(args.settle_ms, 300.0))
            result[f"c4_block_{route}_ms"] = r["ms"]
            result[f"c4_block_{route}"] = {k: r[k] for k in ("mean_ms", "per_forward_ms", "tflops", "steps", "settle_ms")}
    if not args.no_cpu:
        xb = x.view(torch.int16).numpy()
        result["cpu_baseline"] = cpu_baseline(args.workload, xb, q.view(torch.uint8).numpy() if fp8 else q, s, b,
                                              x32=x32)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
