"""Benchmark of the MI355X quantized-linear path.

``python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]``

Default workload (the headline metric): the FP8 linear at M=32760, K=5120,
N=13824 (the FFN up-projection shape) through the drop-in
``RowFP8Execution.linear``: per-token E4M3 quantization kernel + E4M3 MFMA GEMM
with the scale/bias epilogue.  Inputs are seeded synthetic tensors already in
HBM.  A step is one ``linear`` call; K timed steps are bracketed by
``torch.cuda.synchronize()``.  The dominant kernel (the GEMM) is timed with HIP
events recorded on the launch stream around each of its launches in the timed
region.  Prints one JSON line.

Other workloads (``qkv``, ``ffn``, ``skinny``, ``nvfp4``, ``small``) print the
same kind of line for the other shapes of this path.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
FP8_PEAK_TFLOPS = 5033.2  # MI355X dense FP8 MFMA (2.4 GHz)
BF16_PEAK_TFLOPS = 2516.6  # MI355X dense BF16 MFMA
HBM_PEAK_GBS = 8000.0


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument(
        "--workload", default="fp8_linear", choices=["fp8_linear", "qkv", "ffn", "skinny", "nvfp4", "small"]
    )
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--tile", type=int, default=0, help="force a GEMM tile configuration")
    p.add_argument("--group-m", type=int, default=0)
    return p.parse_args()


def seeded_linear(m, k, n, bias=True, seed=0):
    import torch

    from vflash_amd.prepare import quantize_weight_rows

    g = torch.Generator().manual_seed(seed)
    x = torch.randn((m, k), generator=g).to(torch.bfloat16)
    w = torch.randn((n, k), generator=g) * 0.02
    b = (torch.randn(n, generator=g) * 0.01).to(torch.bfloat16) if bias else None
    codes, scale = quantize_weight_rows(w)
    return x, codes, scale, b


def traffic_from_profiles(kernel: str):
    """HBM bytes per launch measured with rocprofv3 counters (committed summary)."""
    path = ROOT / "profiles" / f"traffic_{kernel}.txt"
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        if line.startswith("hbm_bytes_per_launch:"):
            return float(line.split(":", 1)[1])
    return None


def cpu_baseline_weight_only(x, codes, scale, b, flops_per_row):
    """The reference's CPU weight-only path on a bounded row sample."""
    import torch

    from oracle.baseline import weight_only_linear

    threads = torch.get_num_threads()
    rows = 128
    t0 = time.perf_counter()
    weight_only_linear(x[:rows], codes, scale, b)
    probe = time.perf_counter() - t0
    rows = int(min(x.shape[0], max(128, 128 * 4.0 / max(probe, 1e-3))) // 128 * 128)
    sample = x[:rows]
    weight_only_linear(sample, codes, scale, b)  # warm-up
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        weight_only_linear(sample, codes, scale, b)
        times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    return {
        "value": flops_per_row * rows / t / 1e12,
        "unit": "TFLOP/s",
        "cores": threads,
        "kind": "port",
        "sample": (
            f"weight-only dequant-matmul (restored bf16 W every call, F.linear + bias; "
            f"h3_fp8_linear.py:88-91) on {rows} of {x.shape[0]} rows, bf16 CPU torch, "
            f"median of 3 after 1 warm-up, {t * 1e3:.0f} ms per call"
        ),
    }


class EventTimer:
    """HIP events on the launch stream around each launch of one kernel."""

    def __init__(self):
        self.pairs = []

    def start(self):
        import torch

        s = torch.cuda.Event(enable_timing=True)
        e = torch.cuda.Event(enable_timing=True)
        s.record(torch.cuda.current_stream())
        self.pairs.append((s, e))

    def stop(self):
        import torch

        self.pairs[-1][1].record(torch.cuda.current_stream())

    def mean_ms(self):
        return statistics.mean(s.elapsed_time(e) for s, e in self.pairs)


def main():
    args = parse()
    if args.gpus != 1:
        print(
            "bench.py runs on one GPU: every box of this build has a single MI355X; "
            "the multi-GPU sharding of this path is a design note, not a measured mode",
            file=sys.stderr,
        )
        sys.exit(2)
    import torch

    from vflash_amd import _lib, kernels
    from vflash_amd.fp8_linear import RowFP8Execution

    dev = torch.device("cuda:0")
    if not _lib.is_gfx950(dev):
        raise SystemExit("bench.py needs a gfx950 (MI355X) device")
    _lib.library()
    if args.tile or args.group_m:
        _lib.set_gemm_tile(args.tile, args.group_m)

    wl = args.workload
    timer = EventTimer()
    cpu = None
    if wl in ("fp8_linear", "small", "qkv"):
        m, k, n = {"fp8_linear": (32760, 5120, 13824), "small": (4096, 3072, 3072),
                   "qkv": (32760, 5120, 15360)}[wl]
        x, codes, scale, b = seeded_linear(m, k, n, bias=True)
        xd, cd, sd, bd = x.to(dev), codes.to(dev), scale.to(dev), b.to(dev)
        ex = RowFP8Execution("w8a8", activation_quantizer="triton")

        def step(timed):
            a, sa = kernels.quantize_rows(xd)
            if timed:
                timer.start()
            if wl == "qkv":
                kernels.fp8_gemm_planes(a, sa, cd, sd, m, 3, bd)
            else:
                kernels.fp8_gemm(a, sa, cd, sd, m, bd)
            if timed:
                timer.stop()

        # The timed step is the same pair of launches RowFP8Execution.linear makes;
        # one call through the module API checks that path end to end first.
        ex.linear(xd[:16], cd, sd, bd)
        flops = 2.0 * m * n * k
        kernel = "fp8_gemm"
        peak = FP8_PEAK_TFLOPS
        config = {"workload": {"fp8_linear": "fp8_linear_ffn_up_shape", "small": "fp8_linear_small",
                               "qkv": "merged_qkv_planes"}[wl],
                  "m": m, "k": k, "n": n, "bias": True, "activation_quant": "per-token e4m3 (HIP)"}
        if not args.no_cpu_baseline:
            cpu = lambda: cpu_baseline_weight_only(x, codes, scale, b, 2.0 * n * k)
    elif wl == "ffn":
        from vflash_amd.fused import fp8_ffn

        m, h, f = 32760, 5120, 13824
        g = torch.Generator().manual_seed(0)
        x = torch.randn((m, h), generator=g).to(torch.bfloat16)
        from vflash_amd.prepare import quantize_weight_rows

        wu = torch.randn((f, h), generator=g) * 0.02
        bu = (torch.randn(f, generator=g) * 0.01).to(torch.bfloat16)
        wdn = torch.randn((h, f), generator=g) * 0.02
        bdn = (torch.randn(h, generator=g) * 0.01).to(torch.bfloat16)
        gate = torch.rand(h, generator=g).to(torch.bfloat16)
        res = torch.randn((m, h), generator=g).to(torch.bfloat16)
        cu, su = quantize_weight_rows(wu)
        cdn, sdn = quantize_weight_rows(wdn)
        t = [v.to(dev) for v in (x, cu, su, bu, cdn, sdn, bdn, gate, res)]
        ex = RowFP8Execution("w8a8", activation_quantizer="triton")

        def step(timed):
            a, sa = kernels.quantize_rows(t[0])
            if timed:
                timer.start()
            gg, amax = kernels.fp8_gemm_gelu(a, sa, t[1], t[2], m, t[3])
            if timed:
                timer.stop()
            hc, hs = kernels.requant_rows(gg, amax)
            kernels.fp8_gemm_gate_residual(hc, hs, t[4], t[5], m, t[7], t[8], t[6])

        fp8_ffn(ex, t[0][:64], t[1], t[2], t[3], t[4], t[5], t[6], t[7], t[8][:64])
        flops = 4.0 * m * h * f
        kernel = "fp8_gemm_gelu"
        peak = FP8_PEAK_TFLOPS
        config = {"workload": "fp8_ffn_gelu", "m": m, "hidden": h, "ffn": f}
        if not args.no_cpu_baseline:
            from oracle.baseline import gelu_ffn

            def cpu():
                rows = 64
                t0 = time.perf_counter()
                gelu_ffn(x[:rows], cu, su, bu, cdn, sdn, bdn, gate, res[:rows])
                dt = time.perf_counter() - t0
                return {"value": 4.0 * h * f * rows / dt / 1e12, "unit": "TFLOP/s",
                        "cores": torch.get_num_threads(), "kind": "port",
                        "sample": f"weight-only FFN chain on {rows} rows, one call"}
    elif wl == "skinny":
        from vflash_amd.fused import fp8_linear_lora

        m, k, n, r = 1024, 1536, 6144, 32
        x, codes, scale, b = seeded_linear(m, k, n, bias=True)
        g = torch.Generator().manual_seed(1)
        la = (torch.randn((r, k), generator=g) * 0.01).to(torch.bfloat16)
        lb = (torch.randn((n, r), generator=g) * 0.01).to(torch.bfloat16)
        xd, cd, sd, bd, ad, bbd = (v.to(dev) for v in (x, codes, scale, b, la, lb))
        ex = RowFP8Execution("w8a8", activation_quantizer="triton")

        def step(timed):
            if timed:
                timer.start()
            fp8_linear_lora(ex, xd, cd, sd, bd, ad, bbd)
            if timed:
                timer.stop()

        flops = 2.0 * m * n * k + 2.0 * m * r * (k + n)
        kernel = "fp8_linear_lora_call"
        peak = FP8_PEAK_TFLOPS
        config = {"workload": "skinny_lora", "m": m, "k": k, "n": n, "rank": r}
    elif wl == "nvfp4":
        from vflash_amd.nvfp4_linear import NVFP4Execution, NVFP4Weight
        from vflash_amd.prepare import quantize_nvfp4_weight

        m, k, n = 32760, 5120, 13824
        g = torch.Generator().manual_seed(0)
        x = torch.randn((m, k), generator=g).to(torch.bfloat16)
        w = torch.randn((n, k), generator=g) * 0.02
        packed, scales, alpha, ins = quantize_nvfp4_weight(w)
        weight = NVFP4Weight(packed.to(dev), scales.to(dev), alpha.to(dev), ins.to(dev))
        xd = x.to(dev)
        ex = NVFP4Execution()

        def step(timed):
            a, sa = kernels.quantize_rows(xd)
            if timed:
                timer.start()
            kernels.nvfp4_gemm(a, sa, weight.packed, weight.scales, weight.alpha, m)
            if timed:
                timer.stop()

        ex.linear(xd[:16], weight)
        flops = 2.0 * m * n * k
        kernel = "nvfp4_gemm"
        peak = BF16_PEAK_TFLOPS
        config = {"workload": "nvfp4_weight_linear", "m": m, "k": k, "n": n, "mfma": "bf16 (exact dequant)"}

    for _ in range(args.warmup):
        step(False)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step(True)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms_per_step = elapsed * 1e3 / args.steps
    kernel_ms = timer.mean_ms()
    kernel_tflops = flops / (kernel_ms * 1e-3) / 1e12
    line = {
        "metric": "FP8 linear TFLOP/s (M=32760,K=5120,N=13824) and % of gfx950 FP8 MFMA peak",
        "value": flops / (ms_per_step * 1e-3) / 1e12,
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8_e4m3" if wl != "nvfp4" else "fp8_e4m3 x e2m1 (bf16 mfma)",
        "data": "synthetic (seed 0, BASELINE recipe)",
        "config": config,
        "roofline": {
            "bound": "mfma",
            "achieved": kernel_tflops,
            "peak": peak,
            "unit": "TFLOP/s",
            "frac": kernel_tflops / peak,
            "traffic": traffic_from_profiles(kernel if wl != "ffn" else "fp8_gemm_gelu"),
            "kernel": kernel,
            "kernel_ms": kernel_ms,
        },
        "cpu_baseline": cpu() if cpu is not None else None,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
