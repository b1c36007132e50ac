"""Benchmark of the MI355X quantized-linear path.

``python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]``

Default workload (the headline metric): the FP8 linear at M=32760, K=5120,
N=13824 (the FFN up-projection shape) through the drop-in
``RowFP8Execution.linear``: per-token E4M3 quantization kernel + E4M3 MFMA GEMM
with the scale/bias epilogue.  Inputs are seeded synthetic tensors already in
HBM.  A step is one ``linear`` call; K timed steps are bracketed by
``torch.cuda.synchronize()``.  The dominant kernel (the GEMM) is timed with HIP
events recorded on the launch stream around each of its launches in the timed
region, placed by the execution's ``measure`` scope hook (the reference's
profiling interface), so the timed step is the drop-in call itself.  Prints one
JSON line.

Other workloads (``qkv``, ``ffn``, ``ffn_swiglu``, ``skinny``, ``nvfp4`` (W4A8, as configured),
``nvfp4_w4a4``, ``small``, ``norm_quant``) print the same kind of line for the other shapes of this path; ``copy`` times a plain
1 GiB device copy, the calibration kernel for the HBM byte counters.  For the
launch-bound shapes (``small``, ``skinny``) the line adds a device-side time
per step measured with the launch queue filled ahead; ``skinny`` also adds the
step rate when each step is replayed from a captured HIP graph.  The
``fp8_linear`` and ``small`` lines carry ``vendor_reference``: the reference's
own GEMM call (``torch._scaled_mm`` with row-wise scales, hipBLASLt, + bias) on
the same codes, timed the same way.
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
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument(
        "--workload",
        default="fp8_linear",
        choices=["fp8_linear", "qkv", "ffn", "ffn_swiglu", "skinny", "nvfp4", "nvfp4_w4a4", "small",
                 "norm_quant", "copy"],
    )
    p.add_argument("--skinny-m", type=int, default=1024)
    p.add_argument("--skinny-n", type=int, default=6144)
    p.add_argument("--skinny-k", type=int, default=1536,
                   help="skinny K: 1536 (the skinny configuration) or 5376 (the audio pass's Q/K/V)")
    p.add_argument("--skinny-rank", type=int, default=32,
                   help="adapter rank of the skinny step (32; 128 and 16 for the shipped adapters)")
    p.add_argument("--operand-sets", type=int, default=0,
                   help="rotating operand sets for the small shapes (0 = enough to exceed the last-level cache)")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--operands", default="bench", choices=["bench", "constant", "random"],
                   help="fp8_linear operands: the seeded configuration data (bench), constant codes "
                        "(activations 448, weights 0.5), or uniformly random E4M3 codes; the GEMM "
                        "does the same work on each, the board's power limit sets its clock")
    p.add_argument("--settle-ms", type=float, default=200.0,
                   help="untimed steps for this long before the warmup steps: a fresh process's "
                        "first ~25 launches of the metric GEMM (~50 ms) run 5-10 %% slower while "
                        "the GPU's clocks ramp up; 0 disables")
    p.add_argument("--board-power", action="store_true",
                   help="after the timed steps, keep running the step and read the board's socket "
                        "power and graphics clocks (amd-smi) while it runs")
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


def traffic_from_profiles(workload: str):
    """HBM bytes per launch of the dominant kernel, from the committed rocprofv3
    summary of this workload (FETCH_SIZE and WRITE_SIZE scaled by the copy
    calibration), or None when no counter run was summarised."""
    path = ROOT / "profiles" / f"{workload}.txt"
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        if line.startswith("hbm_bytes_per_launch:"):
            return float(line.split(":", 1)[1])
    return None


def host_threads() -> int:
    """Threads for the CPU baselines: every core this process may run on
    (os.cpu_count() narrowed by the CPU affinity), capped by OMP_NUM_THREADS
    when the host sets it (a GPU box's share of the host)."""
    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    env = os.environ.get("OMP_NUM_THREADS", "")
    if env.isdigit() and int(env) > 0:
        n = min(n, int(env))
    return max(1, n)


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform

    return platform.processor() or "unknown"


def use_host_threads() -> int:
    import torch

    threads = host_threads()
    torch.set_num_threads(threads)
    return threads


def cpu_oracle_linear(x, codes, scale, b, flops_per_row):
    """The CPU W8A8 emulation oracle (per-token E4M3 quantization, exact binary64
    sums, bf16(acc * sa * sw), bf16(+ bias)) timed on a row sample: the parity
    reference, reported beside the baseline but not the baseline."""
    from oracle import fp8 as O

    threads = use_host_threads()
    wc = codes.view(__import__("torch").uint8).numpy()
    sw = scale.reshape(-1).numpy()
    bias = None if b is None else b.float().numpy()
    rows = 16
    O.w8a8_linear(x[:rows].float().numpy(), wc, sw, bias)  # warm-up
    t0 = time.perf_counter()
    O.w8a8_linear(x[:rows].float().numpy(), wc, sw, bias)
    probe = time.perf_counter() - t0
    rows = int(min(x.shape[0], max(16, 16 * 3.0 / max(probe, 1e-3))) // 16 * 16)
    t0 = time.perf_counter()
    O.w8a8_linear(x[:rows].float().numpy(), wc, sw, bias)
    dt = time.perf_counter() - t0
    return {"value": flops_per_row * rows / dt / 1e12, "unit": "TFLOP/s", "threads": threads,
            "cpu_model": cpu_model(),
            "sample": (f"numpy W8A8 oracle (binary64 sums of decoded E4M3 products) on {rows} of "
                       f"{x.shape[0]} rows, {dt * 1e3:.0f} ms")}


def cpu_baseline_weight_only(x, codes, scale, b, flops_per_row):
    """The reference's CPU weight-only path: every row of the workload (the whole
    call, weight restore included, as the reference makes it), or a row sample
    when a probe predicts more than about 8 s per call on this host."""
    from oracle.baseline import weight_only_linear

    threads = use_host_threads()

    def timed(r):
        t0 = time.perf_counter()
        weight_only_linear(x[:r], codes, scale, b)
        return time.perf_counter() - t0

    # Two probes give the per-call cost (the weight restore) and the per-row cost.
    timed(128)
    t1, t2 = timed(128), timed(640)
    per_row = max((t2 - t1) / 512, 1e-9)
    if t1 + per_row * (x.shape[0] - 128) <= 8.0:
        rows = x.shape[0]
    else:
        rows = int(min(x.shape[0], max(128, 4.0 / per_row)) // 128 * 128)
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
        "threads": threads,
        "cpu_model": cpu_model(),
        "kind": "port",
        "sample": (
            f"weight-only dequant-matmul (restored bf16 W every call, F.linear + bias; "
            f"h3_fp8_linear.py:88-91) on {rows} of {x.shape[0]} rows, bf16 CPU torch, "
            f"median of 3 after 1 warm-up, {t * 1e3:.0f} ms per call"
        ),
    }


class EventTimer:
    """HIP events on the launch stream around each launch of one kernel.

    The kernels run on torch's current stream (the C-ABI is handed
    ``torch.cuda.current_stream()``), so events recorded on that stream bracket
    exactly one launch each.  The events are created before the timed steps
    (``n`` pairs, each recorded once, since torch creates the HIP event at its
    first record), so the timed region only records them again.
    """

    def __init__(self, n=0):
        import torch

        self.stream = torch.cuda.current_stream()
        self.pool = [self._pair() for _ in range(n)]
        for s, e in self.pool:
            s.record(self.stream)
            e.record(self.stream)
        self.used = 0

    @staticmethod
    def _pair():
        import torch

        return torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

    def start(self):
        if self.used == len(self.pool):
            self.pool.append(self._pair())
        self.pool[self.used][0].record(self.stream)

    def stop(self):
        self.pool[self.used][1].record(self.stream)
        self.used += 1

    def times_ms(self):
        return [s.elapsed_time(e) for s, e in self.pool[:self.used]]


class _NullScope:
    def __enter__(self):
        return None

    def __exit__(self, *exc):
        return False


class _TimedScope:
    __slots__ = ("timer",)

    def __init__(self, timer):
        self.timer = timer

    def __enter__(self):
        self.timer.start()

    def __exit__(self, *exc):
        self.timer.stop()
        return False


_NULL_SCOPE = _NullScope()


class ScopeTimer:
    """``measure`` hook of a RowFP8Execution that brackets the first
    ``linear.fp8_gemm`` scope of each armed step with the timer's events (the
    dominant GEMM launch of the drop-in call: the linear's GEMM, the FFN's up
    projection); every other scope is a no-op."""

    def __init__(self):
        self.timer = None

    def arm(self, timer):
        self.timer = timer

    def __call__(self, name):
        if name != "linear.fp8_gemm" or self.timer is None:
            return _NULL_SCOPE
        timer, self.timer = self.timer, None
        return _TimedScope(timer)


class Workload:
    """One shape of the path: its step, the dominant kernel and its roofline units."""

    def __init__(self, name, metric, unit, work, step, kernel, kernel_work, bound, peak, config,
                 dtype="fp8_e4m3", cpu=None, launch_bound=False):
        self.name = name
        self.metric = metric  # metric string of the JSON line
        self.unit = unit  # "TFLOP/s" or "GB/s"
        self.work = work  # algorithmic FLOPs (or bytes) of one step
        self.step = step  # step(i, timer or None)
        self.kernel = kernel  # dominant kernel, named as in the rocprof summaries
        self.kernel_work = kernel_work  # algorithmic FLOPs (or bytes) of one launch of it
        self.bound = bound  # "mfma" or "hbm"
        self.peak = peak
        self.config = config
        self.dtype = dtype
        self.cpu = cpu
        # Steps shorter than the host's launch cost: the GPU idles between
        # launches, so device time is also measured with the queue filled ahead.
        self.launch_bound = launch_bound
        self.extra = None  # optional comparison timing: () -> ms per step
        # Optional: () -> ms per step with the step replayed from captured HIP graphs.
        self.graph = None
        # Optional: () -> dict, the reference's own library call timed on the same inputs.
        self.vendor = None
        # Optional: () -> dict, the CPU W8A8 emulation oracle timed on a row sample.
        self.cpu_oracle = None
        # Also report the kernel's fraction of the FP8 MFMA peak (16-bit MFMA kernels).
        self.fp8_frac = False


def rate(work, ms, unit):
    return work / (ms * 1e-3) / (1e12 if unit == "TFLOP/s" else 1e9)


def linear_sets(m, k, n, count, dev):
    """``count`` independent operand sets (seeds 0..count-1) resident in HBM.

    Small shapes rotate over several sets so that the timed launches read HBM
    rather than the 256 MB last-level cache.
    """
    sets = []
    for seed in range(count):
        x, codes, scale, b = seeded_linear(m, k, n, bias=True, seed=seed)
        sets.append((x.to(dev), codes.to(dev), scale.to(dev), b.to(dev)))
        if seed == 0:
            host = (x, codes, scale, b)
    return host, sets


def operand_variant(kind, x, codes, scale, bias):
    """The same linear on other operand bits (same shapes, scales and bias):
    constant: every activation 1.0 (codes 448 after the per-token quantization)
    and every weight code 0.5; random: uniformly drawn finite E4M3 codes for both
    (each activation row holds 448, so its scale is 1 and its codes are the drawn
    ones)."""
    import torch

    if kind == "constant":
        return (torch.ones_like(x), torch.full_like(codes.view(torch.uint8), 0x30).view(codes.dtype),
                scale, bias)
    g = torch.Generator(device=x.device).manual_seed(7)

    def draw(shape):
        c = torch.randint(0, 254, shape, generator=g, device=x.device, dtype=torch.int32)
        c = c + (c >= 127).to(torch.int32)  # skip 0x7f (NaN); 0xff is never drawn
        return c.to(torch.uint8)

    xa = draw(x.shape).view(torch.float8_e4m3fn).to(torch.bfloat16)
    xa[:, 0] = 448.0
    return (xa, draw(codes.shape).view(codes.dtype), scale, bias)


def board_power(step, seconds=4.0):
    """Run the step back to back for a few seconds while amd-smi reads the
    socket power and the graphics clocks halfway through."""
    import subprocess
    import threading

    import torch

    result = {}

    def query():
        time.sleep(seconds / 2)
        try:
            r = subprocess.run(["amd-smi", "metric", "--power", "--clock"], capture_output=True,
                               text=True, timeout=30)
        except (OSError, subprocess.TimeoutExpired) as err:
            result["error"] = str(err)[:200]
            return
        clocks, power = [], None
        section = None
        for line in r.stdout.splitlines():
            t = line.strip()
            if t.startswith("GFX_"):
                section = "gfx"
            elif t.endswith(":") and not t.startswith("GFX_"):
                section = None if t != "POWER:" else "power"
            if t.startswith("SOCKET_POWER:"):
                power = t.split(":", 1)[1].strip()
            elif section == "gfx" and t.startswith("CLK:"):
                clocks.append(t.split(":", 1)[1].strip())
        result.update({"tool": "amd-smi metric --power --clock", "socket_power": power,
                       "gfx_clocks": clocks})

    th = threading.Thread(target=query)
    th.start()
    i = 0
    while th.is_alive():
        for _ in range(10):
            step(i, None)
            i += 1
        torch.cuda.synchronize()
    th.join()
    return result


def make_workload(args, dev):
    import torch

    from vflash_amd import kernels
    from vflash_amd.fp8_linear import RowFP8Execution

    wl = args.workload
    if wl in ("fp8_linear", "small", "qkv"):
        m, k, n = {"fp8_linear": (32760, 5120, 13824), "small": (4096, 3072, 3072),
                   "qkv": (32760, 5120, 15360)}[wl]
        host, sets = linear_sets(m, k, n, (args.operand_sets or 8) if wl == "small" else 1, dev)
        if args.operands != "bench":
            sets = [operand_variant(args.operands, *st) for st in sets]
        scope = ScopeTimer()
        ex = RowFP8Execution("w8a8", activation_quantizer="hip", measure=scope)
        from vflash_amd.fused import qkv_linear

        def step(i, timer):
            # The drop-in call: RowFP8Execution.linear, or the merged QKV linear
            # writing three planes.
            xd, cd, sd, bd = sets[i % len(sets)]
            scope.arm(timer)
            if wl == "qkv":
                qkv_linear(ex, xd, cd, sd, bd, planes=True)
            else:
                ex.linear(xd, cd, sd, bd)

        flops = 2.0 * m * n * k
        names = {"fp8_linear": "fp8_linear_m32760_k5120_n13824", "small": "fp8_linear_m4096_k3072_n3072",
                 "qkv": "merged_qkv_m32760_k5120_n15360_planes"}
        metric = (f"FP8 linear TFLOP/s (M={m},K={k},N={n}) and % of gfx950 FP8 MFMA peak"
                  if wl != "qkv" else "Merged QKV FP8 linear TFLOP/s (M=32760,K=5120,N=3x5120)")
        config = {"workload": names[wl], "m": m, "k": k, "n": n, "bias": True,
                  "activation_quant": "per-token e4m3 (HIP kernel)", "operand_sets": len(sets)}
        if args.operands != "bench":
            config["operands"] = args.operands
        if wl == "qkv":
            config["output"] = "3 planes [32760, 40 heads, 128]"
        cpu = None if args.no_cpu_baseline else (lambda: cpu_baseline_weight_only(*host, 2.0 * n * k))
        wlo = Workload(wl, metric, "TFLOP/s", flops, step, "fp8_gemm", flops, "mfma",
                       FP8_PEAK_TFLOPS, config, cpu=cpu, launch_bound=wl == "small")

        def vendor():
            # The reference's own GEMM call on the same codes and scales:
            # torch._scaled_mm with row-wise scales (hipBLASLt on ROCm) + bias
            # (h3_fp8_linear.py:109-121), timed like the GEMM above.
            xd, cd, sd, bd = sets[0]
            a, sa = kernels.quantize_rows(xd)

            def call():
                out = torch._scaled_mm(a, cd.t(), scale_a=sa, scale_b=sd.t(),
                                       out_dtype=torch.bfloat16, use_fast_accum=False)
                return out[:m] + bd

            for _ in range(5):
                call()
            timer = EventTimer()
            for _ in range(20):
                timer.start()
                call()
                timer.stop()
            torch.cuda.synchronize()
            ms = statistics.mean(timer.times_ms())
            return {"call": "torch._scaled_mm (row-wise scales, hipBLASLt) + bias", "ms": ms,
                    "tflops": flops / (ms * 1e-3) / 1e12}

        if wl != "qkv":
            wlo.vendor = vendor
        if not args.no_cpu_baseline and wl != "qkv":
            wlo.cpu_oracle = lambda: cpu_oracle_linear(*host, 2.0 * n * k)
        return wlo

    if wl in ("ffn", "ffn_swiglu"):
        from vflash_amd.fused import fp8_ffn
        from vflash_amd.prepare import quantize_weight_rows

        swiglu = wl == "ffn_swiglu"
        # GELU-tanh FFN at 5120 -> 13824; the H3 SwiGLU FFN at 5376 -> 2 x 14336.
        m, h, f = (32760, 5376, 14336) if swiglu else (32760, 5120, 13824)
        up_rows = 2 * f if swiglu else f
        g = torch.Generator().manual_seed(0)
        x = torch.randn((m, h), generator=g).to(torch.bfloat16)
        wu = torch.randn((up_rows, h), generator=g) * 0.02
        bu = (torch.randn(up_rows, generator=g) * 0.01).to(torch.bfloat16)
        wdn = torch.randn((h, f), generator=g) * 0.02
        bdn = (torch.randn(h, generator=g) * 0.01).to(torch.bfloat16)
        gate = torch.rand(h, generator=g).to(torch.bfloat16)
        res = torch.randn((m, h), generator=g).to(torch.bfloat16)
        cu, su = quantize_weight_rows(wu)
        cdn, sdn = quantize_weight_rows(wdn)
        t = [v.to(dev) for v in (x, cu, su, bu, cdn, sdn, bdn, gate, res)]
        scope = ScopeTimer()
        ex = RowFP8Execution("w8a8", activation_quantizer="hip", measure=scope)
        act = "swiglu" if swiglu else "gelu_tanh"

        def step(i, timer):
            # The drop-in call; the scope hook times its first GEMM (the up projection).
            scope.arm(timer)
            fp8_ffn(ex, t[0], t[1], t[2], t[3], t[4], t[5], t[6], t[7], t[8], activation=act)

        cpu = None
        if not args.no_cpu_baseline and not swiglu:
            from oracle.baseline import gelu_ffn

            def cpu():
                threads = use_host_threads()
                rows = 256
                gelu_ffn(x[:32], cu, su, bu, cdn, sdn, bdn, gate, res[:32])  # warm-up
                t0 = time.perf_counter()
                gelu_ffn(x[:rows], cu, su, bu, cdn, sdn, bdn, gate, res[:rows])
                dt = time.perf_counter() - t0
                return {"value": 4.0 * h * f * rows / dt / 1e12, "unit": "TFLOP/s",
                        "cores": threads, "threads": threads, "cpu_model": cpu_model(), "kind": "port",
                        "sample": (f"weight-only FFN chain (dequantized bf16 weights, GELU-tanh, "
                                   f"gate-residual) on {rows} of {m} rows, one call after a warm-up")}

        if swiglu:
            return Workload(
                wl, "H3 SwiGLU FP8 FFN TFLOP/s (M=32760, 5376 -> 2x14336 SwiGLU -> 5376, gate-residual)",
                "TFLOP/s", 2.0 * m * h * up_rows + 2.0 * m * f * h, step, "fp8_gemm_swiglu",
                2.0 * m * h * up_rows, "mfma", FP8_PEAK_TFLOPS,
                {"workload": "fp8_ffn_swiglu_m32760_h5376_f14336", "m": m, "hidden": h, "ffn": f,
                 "step": "quant, packed up GEMM + SwiGLU + row amax, requant, down GEMM + gate-residual"})
        return Workload(
            wl, "Fused FP8 FFN TFLOP/s (M=32760, 5120 -> 13824 GELU-tanh -> 5120, gate-residual)",
            "TFLOP/s", 4.0 * m * h * f, step, "fp8_gemm", 2.0 * m * h * f, "mfma", FP8_PEAK_TFLOPS,
            {"workload": "fp8_ffn_m32760_h5120_f13824", "m": m, "hidden": h, "ffn": f,
             "step": "quant, up GEMM, GELU-tanh + requant, down GEMM + gate-residual"},
            cpu=cpu)

    if wl == "skinny":
        m, k, n, r = args.skinny_m, args.skinny_k, args.skinny_n, args.skinny_rank
        per_set = m * k * 3 + n * k + 2 * m * n + 2 * r * (k + n) + 2 * m * r
        count = args.operand_sets or max(2, int(600e6 // per_set) + 1)  # > 2x the last-level cache
        sets = []
        for seed in range(count):
            x, codes, scale, b = seeded_linear(m, k, n, bias=True, seed=seed)
            g = torch.Generator().manual_seed(1000 + seed)
            la = (torch.randn((r, k), generator=g) * 0.01).to(torch.bfloat16)
            lb = (torch.randn((n, r), generator=g) * 0.01).to(torch.bfloat16)
            sets.append(tuple(v.to(dev) for v in (x, codes, scale, b, la, lb)))
        from vflash_amd.fused import fp8_linear_lora

        scope = ScopeTimer()
        ex = RowFP8Execution("w8a8", activation_quantizer="hip", measure=scope)

        def step(i, timer):
            # The drop-in call fused.fp8_linear_lora (host path included); the
            # scope hook times its GEMM with the adapter merge.
            scope.arm(timer)
            fp8_linear_lora(ex, *sets[i % len(sets)])

        # Algorithmic HBM bytes of the whole step: x read once (bf16), codes written
        # and read back (e4m3), row scales, weights (e4m3 + fp32 scale + bf16 bias),
        # LoRA A and B, t written and read, bf16 out.
        step_bytes = (2 * m * k + 2 * m * k + 8 * m + n * k + 6 * n
                      + 2 * r * (k + n) + 4 * m * r + 2 * m * n)
        gemm_bytes = m * k + 4 * m + n * k + 6 * n + 2 * m * r + 2 * n * r + 2 * m * n

        def graph_ms():
            # The same step (both launches) captured once per operand set into a
            # HIP graph and replayed: what a launch-bound caller does to skip the
            # per-call host path.
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                step(0, None)
            torch.cuda.current_stream().wait_stream(side)
            graphs = []
            for i in range(len(sets)):
                graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(graph):
                    step(i, None)
                graphs.append(graph)
            for i in range(2 * len(graphs)):
                graphs[i % len(graphs)].replay()
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for i in range(args.steps):
                graphs[i % len(graphs)].replay()
            torch.cuda.synchronize()
            return (time.perf_counter() - t0) * 1e3 / args.steps

        wlo = Workload(
            wl, f"Skinny-M FP8 linear + rank-{r} LoRA GB/s (M={m},K={k},N={n})", "GB/s", step_bytes, step,
            "fp8_gemm_lora", gemm_bytes, "hbm", HBM_PEAK_GBS,
            {"workload": f"skinny_lora_m{m}_k{k}_n{n}_r{r}", "m": m, "k": k, "n": n, "rank": r,
             "operand_sets": count, "flops_per_step": 2.0 * m * n * k + 2.0 * m * r * (k + n)},
            launch_bound=True)
        wlo.graph = graph_ms
        return wlo

    if wl in ("nvfp4", "nvfp4_w4a4"):
        from vflash_amd.nvfp4_linear import NVFP4Execution, NVFP4Weight
        from vflash_amd.prepare import quantize_nvfp4_weight

        # nvfp4: the NVFP4-weight linear as its benchmark configuration states it,
        # per-token E4M3 activations against E2M1 weights with E4M3 block scales
        # (W4A8).  nvfp4_w4a4: the reference module's arithmetic, NVFP4 activations
        # with a calibrated global input scale (448 * 6 / amax).
        w4a4 = wl == "nvfp4_w4a4"
        m, k, n = 32760, 5120, 13824
        g = torch.Generator().manual_seed(0)
        x = torch.randn((m, k), generator=g).to(torch.bfloat16)
        w = torch.randn((n, k), generator=g) * 0.02
        input_scale = 2688.0 / float(x.float().abs().max())
        packed, scales, alpha, ins = quantize_nvfp4_weight(w, input_scale)
        weight = NVFP4Weight(packed.to(dev), scales.to(dev), alpha.to(dev), ins.to(dev))
        xd = x.to(dev)
        NVFP4Execution("nvfp4" if w4a4 else "e4m3").linear(xd[:16], weight)
        out_scale = weight.alpha / weight.input_scale

        def step(i, timer):
            if w4a4:
                a, sa = kernels.nvfp4_quantize_rows(xd, weight.input_scale)
            else:
                a, sa = kernels.quantize_rows(xd)
            if timer:
                timer.start()
            if w4a4:
                kernels.nvfp4_w4a4_gemm(a, sa, weight.packed, weight.scales, out_scale, m)
            else:
                kernels.nvfp4_gemm(a, sa, weight.packed, weight.scales, weight.alpha, m)
            if timer:
                timer.stop()

        flops = 2.0 * m * n * k
        if w4a4:
            wlo = Workload(
                wl, "NVFP4 W4A4 linear TFLOP/s (M=32760,K=5120,N=13824)", "TFLOP/s", flops, step,
                "nvfp4_gemm_pipe<true>", flops, "mfma", BF16_PEAK_TFLOPS,
                {"workload": "nvfp4_w4a4_linear_m32760_k5120_n13824", "m": m, "k": k, "n": n,
                 "activations": "NVFP4 (e2m1 + e4m3 block-16 scales, global input scale)",
                 "mfma": "f16 on exactly dequantized e2m1 x e4m3 operands"},
                dtype="e2m1 x e2m1 with e4m3 block scales (f16 mfma, exact operands)")
        else:
            wlo = Workload(
                wl, "NVFP4-weight W4A8 linear TFLOP/s (M=32760,K=5120,N=13824)", "TFLOP/s", flops, step,
                "nvfp4_gemm_pipe<false>", flops, "mfma", BF16_PEAK_TFLOPS,
                {"workload": "nvfp4_weight_linear_m32760_k5120_n13824", "m": m, "k": k, "n": n,
                 "mfma": "f16 on exactly dequantized e4m3 activations and e2m1 x e4m3 weights"},
                dtype="e4m3 activations x e2m1 weights (f16 mfma, exact operands)")
        wlo.fp8_frac = True
        return wlo

    if wl == "norm_quant":
        from vflash_amd.producers import rmsnorm_modulate_quantize

        # The QKV/FFN-input producer: RMSNorm + adaLN modulation (rows of a
        # [24, 6, H] table gathered by per-token indices) + per-token E4M3
        # quantization, one pass over 32760 tokens of hidden 5120.  The indices
        # (timestep index * 3 + modality tag per token) are constant over runs
        # of consecutive tokens, as the packed sequence groups tokens by
        # modality and frame: here 24 runs of equal length in shuffled order.
        s_tok, h, r = 32760, 5120, 24
        g = torch.Generator().manual_seed(0)
        x = torch.randn((1, s_tok, h), generator=g).to(torch.bfloat16)
        w = (torch.rand(h, generator=g) * 2).to(torch.bfloat16)
        table = (torch.randn((r, 6, h), generator=g) * 0.5).to(torch.bfloat16)
        index = torch.randperm(r, generator=g)[torch.arange(s_tok) * r // s_tok]
        xd, wd, td, idd = x.to(dev), w.to(dev), table.to(dev), index.to(dev)
        sc, sh = td[:, 1, :], td[:, 0, :]
        rmsnorm_modulate_quantize(xd[:, :16], wd, sc, sh, eps=1e-6, index=idd[:16])

        def step(i, timer):
            if timer:
                timer.start()
            kernels.rmsnorm_modulate_quantize(xd.view(-1, h), wd, sc, sh, eps=1e-6, index=idd)
            if timer:
                timer.stop()

        # Algorithmic HBM bytes: x read once (bf16), codes written (e4m3), fp32 row
        # scales, the norm weight, the table rows and the indices read once.
        nbytes = 2.0 * s_tok * h + s_tok * h + 4.0 * s_tok + 2.0 * h + 2.0 * r * 2 * h + 8.0 * s_tok

        def unfused_ms():
            # The reference's unfused sequence on the same inputs, for comparison:
            # index_select gathers, F.rms_norm, eager bf16 modulation, HIP quantizer.
            def chain():
                scale = sc.index_select(0, idd)
                shift = sh.index_select(0, idd)
                n = torch.nn.functional.rms_norm(xd, (h,), wd, 1e-6)
                kernels.quantize_rows((n * (1.0 + scale) + shift).view(-1, h))
            for _ in range(3):
                chain()
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(10):
                chain()
            torch.cuda.synchronize()
            return (time.perf_counter() - t0) * 100.0

        cpu = None
        if not args.no_cpu_baseline:
            def cpu():
                from oracle import fp8 as O

                rows = 2048
                xs = x.view(-1, h)[:rows].float().numpy()
                idx = index.numpy()[:rows]
                tf = table.float().numpy()
                ws = w.float().numpy()
                times = []
                for _ in range(3):
                    t0 = time.perf_counter()
                    n = O.rms_norm(xs, ws, 1e-6)
                    O.quantize_rows(O.modulate(n, tf[idx, 1], tf[idx, 0]))
                    times.append(time.perf_counter() - t0)
                dt = statistics.median(times)
                return {"value": nbytes * rows / s_tok / dt / 1e9, "unit": "GB/s", "cores": 1,
                        "threads": 1, "cpu_model": cpu_model(), "kind": "port",
                        "sample": (f"numpy restatement of rms_norm + modulation + per-token quantization "
                                   f"on {rows} of {s_tok} rows, median of 3, {dt * 1e3:.0f} ms")}

        wlo = Workload(
            wl, "Fused RMSNorm + adaLN modulation + E4M3 quantization GB/s (32760 tokens, hidden 5120)",
            "GB/s", nbytes, step, "norm_mod_quant_rows", nbytes, "hbm", HBM_PEAK_GBS,
            {"workload": "norm_mod_quant_m32760_h5120", "m": s_tok, "hidden": h, "table_rows": r,
             "modulation": "adaLN table rows gathered in place by per-token int64 indices",
             "index_layout": "24 runs of consecutive tokens"},
            dtype="bf16 in, e4m3 out", cpu=cpu)
        wlo.extra = unfused_ms
        return wlo

    if wl == "copy":
        # A plain device copy of 1 GiB: the calibration kernel for the HBM
        # byte counters (FETCH_SIZE / WRITE_SIZE) of the rocprof summaries.
        src = torch.empty(1 << 30, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)

        def step(i, timer):
            if timer:
                timer.start()
            dst.copy_(src)
            if timer:
                timer.stop()

        nbytes = 2.0 * src.numel()
        return Workload(wl, "HBM copy GB/s (1 GiB read + 1 GiB write)", "GB/s", nbytes, step, "copy",
                        nbytes, "hbm", HBM_PEAK_GBS, {"workload": "hbm_copy_1GiB"}, dtype="u8")
    raise ValueError(wl)


def main():
    args = parse()
    if args.gpus != 1:
        print(
            "bench.py runs on one GPU only: this path is measured on a single MI355X; "
            "how it would shard over several GPUs is a design note, not a measured mode",
            file=sys.stderr,
        )
        sys.exit(2)
    import torch

    from vflash_amd import _lib

    dev = torch.device("cuda:0")
    if not _lib.is_gfx950(dev):
        raise SystemExit("bench.py needs a gfx950 (MI355X) device")
    _lib.library()

    w = make_workload(args, dev)
    timer = EventTimer(args.steps)
    # Settle: the step, untimed, until the device has run it for settle_ms (the
    # clocks of a fresh process ramp over its first tens of milliseconds).
    settled = 0.0
    if args.settle_ms > 0:
        t_settle = time.perf_counter()
        i = 0
        while (time.perf_counter() - t_settle) * 1e3 < args.settle_ms:
            w.step(i, None)
            i += 1
            if i % 8 == 0:
                torch.cuda.synchronize()
        torch.cuda.synchronize()
        settled = (time.perf_counter() - t_settle) * 1e3
    for i in range(args.warmup):
        w.step(i, None)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        w.step(i, timer)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms_per_step = elapsed * 1e3 / args.steps
    times = timer.times_ms()
    device = None
    if w.launch_bound:
        # Hold the stream with a spin kernel while the host enqueues every step,
        # then time the same steps on the device with events around the run.
        timer = EventTimer(args.steps)
        torch.cuda._sleep(100_000_000)
        first = torch.cuda.Event(enable_timing=True)
        last = torch.cuda.Event(enable_timing=True)
        first.record(torch.cuda.current_stream())
        for i in range(args.steps):
            w.step(i, timer)
        last.record(torch.cuda.current_stream())
        torch.cuda.synchronize()
        times = timer.times_ms()
        device = first.elapsed_time(last) / args.steps
    kernel_ms = statistics.mean(times)
    achieved = rate(w.kernel_work, kernel_ms, w.unit)
    line = {
        "metric": w.metric,
        "value": rate(w.work, ms_per_step, w.unit),
        "unit": w.unit,
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "settle_ms": round(settled, 1),
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": w.dtype,
        "data": "synthetic: seeded N(0,1) activations, N(0,0.02) weights quantized per row, N(0,0.01) bias",
        "config": w.config,
        "roofline": {
            "bound": w.bound,
            "achieved": achieved,
            "peak": w.peak,
            "unit": w.unit,
            "frac": achieved / w.peak,
            "traffic": traffic_from_profiles(w.config["workload"]),
            "kernel": w.kernel,
            "kernel_ms_mean": kernel_ms,
            "kernel_ms_median": statistics.median(times),
            "launches_timed": len(times),
        },
        "cpu_baseline": w.cpu() if w.cpu is not None else None,
    }
    if w.fp8_frac:
        line["roofline"]["frac_of_fp8_peak"] = achieved / FP8_PEAK_TFLOPS
    if w.cpu_oracle is not None:
        line["cpu_oracle"] = w.cpu_oracle()
    if w.extra is not None:
        line["unfused_reference_ms_per_step"] = w.extra()
    if w.vendor is not None:
        try:
            line["vendor_reference"] = w.vendor()
        except (RuntimeError, NotImplementedError) as err:  # a torch without row-wise FP8 GEMMs
            line["vendor_reference"] = {"error": str(err).splitlines()[0][:200]}
    if w.graph is not None:
        try:
            graph = w.graph()
            line["graph_ms_per_step"] = graph
            line["graph_rate"] = rate(w.work, graph, w.unit)
        except RuntimeError as err:  # a runtime that cannot capture the step
            line["graph_ms_per_step"] = {"error": str(err).splitlines()[0][:200]}
    if args.operands != "bench":
        line["data"] = {"constant": "synthetic: constant codes (activations 448 after quantization, "
                                    "weights 0.5), seeded scales and bias",
                        "random": "synthetic: uniformly random finite E4M3 codes for activations and "
                                  "weights, seeded weight scales and bias"}[args.operands]
    if args.board_power:
        line["board"] = board_power(w.step)
    if device is not None:
        line["device_ms_per_step"] = device
        line["device_rate"] = rate(w.work, device, w.unit)
        line["roofline"]["timing"] = "device queue filled ahead of the launches"
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
