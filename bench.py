"""Benchmark of the W4A4 SVDQuantLinear forward on one MI355X (BASELINE metric).

Workload (the shape the metric is quoted on): the ff.up linear of a
Krea-2 block, M=4096 tokens (1024x1024 latent), K=6144 -> N=16384, rank 32, group 64, W4A4.
Synthetic inputs: X bf16 ~ N(0,1) with 1% outlier channels x20; W fp32 ~ N(0, 0.02) quantized
on the GPU by the package converter (smoothing, rank-32 SVD, INT4 residual).

A step is one full layer forward (activation pass + W4A4 GEMM with the low-rank epilogue),
inputs resident in HBM.  ``value`` = effective TOPS = 2*M*N*K / step time.  ``roofline``
prices the dominant kernel (the W4A4 GEMM) against the INT8 dense MFMA peak, with its
average duration measured by HIP events on the stream the kernel runs on.  ``cpu_baseline``
times the oracle's restatement of the reference ``pytorch_sim`` forward on the host CPU on a
bounded row sample of the same layer.

    python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--no-cpu-baseline]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "W4A4 SVDQuantLinear eff. TOPS @M4096 K6144 N16384; ms/denoise step @1024px"
INT8_PEAK_TOPS = 5000.0   # MI355X dense INT8 MFMA, 5.0 POP/s
HBM_PEAK_GBS = 8000.0


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--m", type=int, default=4096)
    ap.add_argument("--k", type=int, default=6144)
    ap.add_argument("--n", type=int, default=16384)
    ap.add_argument("--rank", type=int, default=32)
    ap.add_argument("--group", type=int, default=64)
    ap.add_argument("--cpu-rows", type=int, default=256)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    return ap.parse_args()


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def time_loop(fn, iters: int) -> float:
    """Average ms per call of ``fn`` over ``iters`` calls, HIP events on the current stream."""
    import torch
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for _ in range(iters):
        fn()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / iters


def cpu_baseline(ds, x_dev, rows: int) -> dict:
    """The restated reference pytorch_sim forward (oracle) on the host CPU, bounded row sample."""
    import torch
    from oracle import sim

    f = lambda t: t.detach().float().cpu().numpy()  # noqa: E731
    st = sim.LayerState(smooth=f(ds.smooth_scale), qweight=ds.qweight.cpu().numpy(),
                        weight_scales=f(ds.weight_scales), l1=f(ds.l1), l2=f(ds.l2), bias=None,
                        group_size=ds.group_size, shape=tuple(ds.original_shape))
    x = x_dev[:rows].cpu()
    threads = torch.get_num_threads()
    sim.sim_forward_torch(x[:8], st)            # warm-up (allocations, thread pool)
    times = []
    for _ in range(2):
        t0 = time.perf_counter()
        sim.sim_forward_torch(x, st)
        times.append(time.perf_counter() - t0)
    t = min(times)
    m, k = x.shape
    n = st.shape[0]
    return {"value": round(2.0 * m * n * k / t / 1e12, 4), "unit": "TOPS", "cores": threads, "kind": "port",
            "sample": f"oracle sim_forward_torch (reference pytorch_sim, bf16 CPU torch) on {m} of the "
                      f"{x_dev.shape[0]} rows, K={k} N={n}; best of 2 after warm-up; {t:.2f} s per call"}


def main() -> int:
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: every GPU box of this build has a single MI355X, and the "
              "SVDQuantLinear path has no collective (a multi-GPU layout is described in DESIGN.md).",
              file=sys.stderr)
        return 2
    import torch
    from krea2_svdquant_amd.kernels.hip import backend, ops
    from krea2_svdquant_amd.quant.convert import convert_linear

    dev = torch.device("cuda:0")
    m, k, n, r, g = args.m, args.k, args.n, args.rank, args.group
    log(f"device {torch.cuda.get_device_name(dev)}; building state M={m} K={k} N={n} r={r} g={g}")
    gen = torch.Generator(device=dev).manual_seed(1)
    x = torch.randn(m, k, device=dev, generator=gen)
    outliers = torch.randperm(k, device=dev, generator=gen)[: round(0.01 * k)]
    x[:, outliers] *= 20.0
    x = x.to(torch.bfloat16)
    w = torch.randn(n, k, device=dev, generator=gen) * 0.02
    ds = convert_linear(w, None, x.float().abs().amax(0), rank=r, group_size=g, smooth_clamp=(None, None), seed=3)
    del w
    prep = backend.prepare_layer(ds, (), dev)
    torch.cuda.synchronize()

    def step():
        return backend.forward_prepared(x, prep, mode="w4a4")

    log(f"warmup {args.warmup}")
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    log(f"timing {args.steps} steps")
    ms = time_loop(step, args.steps)
    log(f"{ms:.4f} ms/step")

    # per-kernel averages, each kernel timed alone on the same (current) stream
    opc = ops.OPERAND_E4M3
    qa, sx, _, _, mid = ops.act_quant(x, prep.srs, prep.l2, None, None, g, prep.rtp, opc, False, False, False,
                                      True)
    ms_act = time_loop(lambda: ops.act_quant(x, prep.srs, prep.l2, None, None, g, prep.rtp, opc, False, False,
                                             False, True), args.steps)
    ms_gemm = time_loop(lambda: ops.w4a4_gemm(qa, sx, prep.weight_operand(opc), prep.weight_scale_pairs(opc), mid, prep.l1cat,
                                              None, g, opc, False), args.steps)
    log(f"act {ms_act:.4f} ms, gemm {ms_gemm:.4f} ms")
    flops = 2.0 * m * n * k
    act_bytes = 2 * m * k + 8 * k + 2 * r * k + m * k // 2 + 2 * m * (k // g) + 4 * m * prep.rtp
    gemm_tops = flops / (ms_gemm * 1e-3) / 1e12
    result = {
        "metric": METRIC,
        "value": round(flops / (ms * 1e-3) / 1e12, 2),
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (X ~ N(0,1) with 1% x20 outlier channels; random-init W ~ N(0,0.02) quantized on device)",
        "config": {"workload": "config1 ff.up: W4A4 SVDQuantLinear forward (act quant+pack+low-rank down, "
                               "INT8-MFMA GEMM + low-rank up epilogue), M=4096 K=6144 N=16384 rank 32 group 64",
                   "M": m, "K": k, "N": n, "rank": r, "group": g, "batch_tokens": m},
        "kernels": {"act_quant_ms": round(ms_act, 4), "w4a4_gemm_ms": round(ms_gemm, 4),
                    "act_quant_GBps": round(act_bytes / (ms_act * 1e-3) / 1e9, 1),
                    "act_quant_hbm_frac": round(act_bytes / (ms_act * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)},
        "roofline": {"bound": "mfma", "achieved": round(gemm_tops, 2), "peak": INT8_PEAK_TOPS, "unit": "TFLOP/s",
                     "frac": round(gemm_tops / INT8_PEAK_TOPS, 4), "traffic": None,
                     "kernel": "w4a4_kernel (INT8 MFMA)", "algorithmic_ops_per_launch": flops},
    }
    if not args.no_cpu_baseline:
        log(f"cpu baseline on {args.cpu_rows} rows")
        result["cpu_baseline"] = cpu_baseline(ds, x, args.cpu_rows)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
