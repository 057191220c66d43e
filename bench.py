"""Benchmark of the weight-quantized linear layer on one MI355X (the BASELINE.json metric).

Workload (the up-projection the metric is quoted on): X bf16
[4096, 3072] ~ N(0,1), W int8 [K=3072, N=12288] (the reference map's [K, N] layout) with codes
uniform in [−127, 127], per-output-channel fp32 scales U(1e−3, 2e−2), bias N(0, 0.02), fused
GELU(tanh), bf16 output. A step is one launch of the fused product on inputs already in HBM.
Inputs are synthetic and seeded (SplitMix64 + Box–Muller, the reference's generator,
Sources/Verification/KernelStages.swift:553-567); the seeds are in the JSON.

value = 2·M·N·K / (average kernel time), the kernel timed with HIP events on the stream it is
launched on, over the timed steps. roofline.peak is MI355X's published dense bf16 MFMA rate.
cpu_baseline: the reference's CPU route restated (Widen.dequantize → fp32 GEMM → bias → GELU,
WeightProducts.swift:698-709, Ops.swift:386-407) on a sample of the rows, run on the host cores of
the GPU box and scaled to the whole step.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

M, K, N = 4096, 3072, 12288
SEEDS = {"x": 1, "w": 2, "scale": 3, "bias": 4}
PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA, published
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E, published
# HBM bytes per launch of the product kernel (FETCH_SIZE × 2 + WRITE_SIZE × 1, the factors from a 512 MiB copy),
# measured by the rocprofv3 --pmc runs in profiles/gemm_wd_kernel_c1_up_int8_packed_gelu.md, by weight layout.
TRAFFIC_BYTES = {"packed": 483.3e6}
GAMMA = np.uint64(0x9E3779B97F4A7C15)


def splitmix(seed: int, count: int) -> np.ndarray:
    """Outputs 1..count of SplitMix64 from `seed` (state_i = seed + i·γ, then the mix)."""
    with np.errstate(over="ignore"):
        z = np.uint64(seed) + GAMMA * np.arange(1, count + 1, dtype=np.uint64)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        return z ^ (z >> np.uint64(31))


def uniform(seed: int, count: int) -> np.ndarray:
    return (splitmix(seed, count) >> np.uint64(11)).astype(np.float64) / 9007199254740992.0


def normal(seed: int, count: int) -> np.ndarray:
    u = uniform(seed, 2 * count)
    u1, u2 = u[0::2], u[1::2]
    return np.sqrt(-2.0 * np.log(np.maximum(u1, 1e-300))) * np.cos(2.0 * np.pi * u2)


def inputs():
    import torch
    x = torch.from_numpy(normal(SEEDS["x"], M * K).astype(np.float32).reshape(M, K)).to(torch.bfloat16)
    q = (np.floor(uniform(SEEDS["w"], K * N) * 255.0) - 127.0).clip(-127, 127).astype(np.int8).reshape(K, N)
    s = (1e-3 + (2e-2 - 1e-3) * uniform(SEEDS["scale"], N)).astype(np.float32)
    b = (0.02 * normal(SEEDS["bias"], N)).astype(np.float32)
    return x, q, s, b


def cpu_baseline(x_bf16, q_kn, s, b, budget_s: float = 12.0):
    """The reference's CPU route on a sample of rows: the whole weight widened (oracle dequantiser,
    every core), the sample's fp32 GEMM (numpy's BLAS, the cblas_sgemm of the reference), bias +
    GELU in fp32 (oracle). Repeated for about `budget_s`; scaled to all M rows."""
    from oracle import oracle
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    rows = 512
    a = x_bf16[:rows].view(np.uint16)
    a32 = oracle.bf16_to_f32(a)
    t_deq, t_gemm, reps = 0.0, 0.0, 0
    start = time.perf_counter()
    while time.perf_counter() - start < budget_s or reps < 2:
        t0 = time.perf_counter()
        w = oracle.dequantize(q_kn.view(np.uint8), oracle.INT8, s, oracle.F32, oracle.SCALE_COLUMNS, columns=N)
        t1 = time.perf_counter()
        p = a32 @ w
        y = oracle.epilogue_f32(p, bias=b, epilogue=oracle.EPI_GELU_TANH, threads=threads)
        t2 = time.perf_counter()
        t_deq += t1 - t0
        t_gemm += t2 - t1
        reps += 1
        del w, p, y
    t_step = t_deq / reps + (t_gemm / reps) * (M / rows)
    return {
        "value": round(2.0 * M * N * K / t_step / 1e12, 4),
        "unit": "TFLOP/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"{rows} of {M} rows × the whole weight, {reps} repetitions in {time.perf_counter() - start:.1f} s: "
                   f"widen {1e3 * t_deq / reps:.1f} ms + GEMM/bias/GELU {1e3 * t_gemm / reps:.1f} ms per repetition; "
                   f"step = widen + GEMM×{M // rows}"),
        "ms_per_step": round(1e3 * t_step, 2),
    }


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    # The clocks reach their steady state only after ~50 ms of sustained work: 10 warm-up steps leave
    # the first timed steps 30 % slow (0.36 ms against 0.27 ms each).
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--layout", choices=["kn", "nk", "packed"], default="packed",
                    help="weight layout the product reads; packed = staged once from [K, N] by sq8_pack_weight")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
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
    x, q_kn, s, b = inputs()
    q = np.ascontiguousarray(q_kn.T) if args.layout == "nk" else q_kn
    xd = x.to(dev)
    wd = torch.from_numpy(q).to(dev)
    sd = torch.from_numpy(s).to(dev)
    bd = torch.from_numpy(b).to(dev)
    out = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    ctx = sq.context(0)
    stage_ms = None
    if args.layout == "packed":
        torch.cuda.synchronize()
        t_stage = time.perf_counter()
        wd = ctx.pack(wd, layout="kn")
        torch.cuda.synchronize()
        stage_ms = 1e3 * (time.perf_counter() - t_stage)
    layout = "nk" if args.layout == "nk" else "kn"

    def step():
        ctx.product(xd, wd, sd, layout=layout, bias=bd, epilogue="gelu_tanh", out=out)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record()
    for _ in range(args.steps):
        step()
    ev1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    # The events are recorded on torch's current stream, the stream the context launches on.
    kernel_ms = ev0.elapsed_time(ev1) / args.steps
    flops = 2.0 * M * N * K
    tflops = flops / (kernel_ms * 1e-3) / 1e12
    algo_bytes = 2 * M * K + N * K + 4 * N + 4 * N + 2 * M * N

    props = torch.cuda.get_device_properties(0)
    result = {
        "metric": "TFLOP/s and % bf16 MFMA peak, int8-weight GEMM 4096x3072x12288 on 1 MI355X",
        "value": round(tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(1e3 * wall / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": f"synthetic, seeded (SplitMix64 + Box-Muller), seeds {SEEDS}",
        "config": {"workload": "C1 up-projection: int8 weight [K,N] per-channel fp32 scale, bf16 X, bias + fused "
                               "GELU-tanh, bf16 out",
                   "M": M, "K": K, "N": N, "weight_layout": args.layout.upper(),
                   "staging_ms": None if stage_ms is None else round(stage_ms, 3), "global_batch": M,
                   "parallelism": "none (one GPU)"},
        "pct_bf16_peak": round(100.0 * tflops / PEAK_BF16_TFLOPS, 2),
        "kernel_ms": round(kernel_ms, 5),
        "roofline": {"bound": "mfma", "achieved": round(tflops, 2), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(tflops / PEAK_BF16_TFLOPS, 4),
                     "traffic": TRAFFIC_BYTES.get(args.layout),
                     "algorithmic_bytes": algo_bytes,
                     "hbm_bound_ms": round(algo_bytes / (PEAK_HBM_GBS * 1e9) * 1e3, 5)},
        "device": {"name": props.name, "cus": props.multi_processor_count},
    }
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(x.view(torch.int16).numpy(), q_kn, s, b)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
