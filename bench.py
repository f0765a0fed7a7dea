"""Benchmark of the MI355X Linear hot path.

Workload (one step): the decode-time W8A16 GEMVs of one token of a
Qwen2.5-0.5B-shaped model — 24 layers x the 7 Linear shapes (q 896x896,
k/v 128x896, o 896x896, gate/up 4864x896, down 896x4864), M = 1, no bias,
each layer with its own weights, so 168 GEMVs over 370.1 MB of distinct
int8 weights + BF16 scales (larger than the 256 MB last-level cache, so no
step is served from cache).  Weights q ~ U{-127..127}, scales
bf16(|N(0, 0.02)| / 127) per 64-column group, inputs bf16(N(0, 1)); seed 1;
all resident in HBM before timing.

Launch modes (--launch):
  plan   (default) all 168 independent GEMVs through one grouped plan: one
         kernel launch per step (infer_hip_w8a16_gemv_plan_launch).
  calls  168 separate infer_hip_gemv_w8a16 calls, the reference's per-Linear
         call pattern (src/qwen2.cpp:615-656).

Prints ONE JSON line (value = tokens/s, i.e. steps/s).  The roofline object
is for the dominant kernel: algorithmic bytes per launch / its average
duration from HIP events recorded around that launch on its stream inside
the timed region.  cpu_baseline is the CPU FP32 oracle (a C restatement of
the reference's cpu_ops.cpp linear_fp32) on the same dequantised weights,
timed on this host for a bounded sample.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PACKAGE = os.path.join(ROOT, "qwen2.5-jetson-inference_amd")
sys.path.insert(0, PACKAGE)

METRIC = "W8A16 decode tok/s + Linear GEMV HBM GB/s (% peak), Qwen2.5-0.5B b=1"
HBM_PEAK_GBS = 8000.0
LAYERS = 24
SHAPES = (("q_proj", 896, 896), ("k_proj", 128, 896), ("v_proj", 128, 896),
          ("o_proj", 896, 896), ("gate_proj", 4864, 896), ("up_proj", 4864, 896),
          ("down_proj", 896, 4864))


def gemv_bytes(n: int, k: int, bias: bool = False) -> int:
    """Compulsory bytes of one W8A16 GEMV: int8 weights, BF16 scales, BF16 x
    and y (and bias)."""
    return n * k + 2 * n * (-(-k // 64)) + 2 * k + 2 * n + (2 * n if bias else 0)


def parse():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--launch", choices=("plan", "calls"), default="plan")
    ap.add_argument("--workload", choices=("decode", "prefill"), default="decode",
                    help="decode: config 1 (the headline); prefill: config 3 GEMMs")
    ap.add_argument("--tokens", type=int, default=512, help="prefill M (config 3)")
    ap.add_argument("--dtype", choices=("w8a16", "bf16"), default="w8a16",
                    help="prefill weight type")
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="bounded CPU-baseline sample length (0 disables)")
    ap.add_argument("--detail", default="",
                    help="write per-shape and per-mode measurements to this JSON file")
    ap.add_argument("--traffic", default=os.path.join(ROOT, "profiles", "traffic.json"),
                    help="committed HBM traffic per launch measured with rocprofv3 --pmc")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="after timing, run one device-to-device copy of this many MiB "
                         "(the known-size reference for rocprofv3 --pmc byte counters)")
    return ap.parse_args()


class Layers:
    """24 layers x 7 W8A16 Linear weights, inputs and outputs on the GPU."""

    def __init__(self, dev, seed: int = 1):
        import torch
        g = torch.Generator(device=dev)
        g.manual_seed(seed)
        self.calls = []   # (weight, scales, 64, bias, x, y, n, k)
        self.names = []
        for layer in range(LAYERS):
            for name, n, k in SHAPES:
                q = torch.randint(-127, 128, (n, k), dtype=torch.int8, device=dev, generator=g)
                s = (torch.randn((n, k // 64), device=dev, generator=g) * 0.02).abs_() / 127.0
                x = torch.randn((k,), device=dev, generator=g).to(torch.bfloat16)
                y = torch.empty((n,), dtype=torch.bfloat16, device=dev)
                self.calls.append((q, s.to(torch.bfloat16), 64, None, x, y, n, k))
                self.names.append((layer, name))
        torch.cuda.synchronize()
        self.bytes = sum(gemv_bytes(c[6], c[7]) for c in self.calls)


def time_steps(step, steps: int, warmup: int):
    """Warm up, then time `steps` back-to-back calls of step() with events on
    the current stream, synchronised on both sides.  Returns (total ms, None)."""
    import torch
    for _ in range(warmup):
        step(None)
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        step(None)
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end), None


def cpu_baseline(layers, seconds: float):
    """The oracle's linear_fp32 (cpu_ops.cpp:23-30) over the same dequantised
    weights: whole 168-GEMV passes until `seconds` elapse."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import numpy as np
    import oracle  # test infrastructure: the CPU baseline leg only
    oracle.build()
    threads = len(os.sched_getaffinity(0))
    env = os.environ.get("OMP_NUM_THREADS")
    if env and env.isdigit():
        threads = min(threads, int(env))
    import torch
    host = []
    for (q, s, _, _, x, y, n, k) in layers.calls:
        qn = q.cpu().numpy()
        sn = s.view(torch.int16).cpu().numpy().view(np.uint16)
        xn = x.float().cpu().numpy()
        host.append((oracle.dequant_w8a16(qn, sn, 64, threads), xn))
    outs = [None] * len(host)
    passes = 0
    t0 = time.perf_counter()
    while True:
        for i, (w, xn) in enumerate(host):
            outs[i] = oracle.linear_fp32(w, None, xn, threads)
        passes += 1
        el = time.perf_counter() - t0
        if el >= seconds or passes >= 100000:
            break
    return {
        "value": passes / el,
        "unit": "tok/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"{passes} full passes (168 FP32 GEMVs each, 24 layers x 7 shapes, "
                   f"1.43 GB of dequantised FP32 weights) in {el:.1f} s; C/OpenMP "
                   f"restatement of cpu_ops.cpp linear_fp32"),
    }, outs


def check_outputs(layers, cpu_outs):
    """Every GPU output of the last step against the CPU FP32 result:
    |a - e| <= max(1e-2 |e|, 1e-3 rms(e)) per output."""
    import numpy as np
    worst = 0.0
    for (c, e) in zip(layers.calls, cpu_outs):
        a = c[5].float().cpu().numpy().astype(np.float64)
        e = e.astype(np.float64)
        tol = np.maximum(1e-2 * np.abs(e), 1e-3 * np.sqrt(np.mean(e * e)))
        err = np.abs(a - e)
        if np.any(err > tol):
            raise SystemExit(f"bench: GPU output outside tolerance ({np.max(err / tol):.3g}x)")
        worst = max(worst, float(np.max(err / tol)))
    return worst


def lm_head_detail(dev, hip):
    """Config 2: the fused LM head over two distinct 151936 x 896 BF16
    embedding copies (545 MB, alternated so no call is served from cache)."""
    import torch
    vocab, k = 151936, 896
    g = torch.Generator(device=dev)
    g.manual_seed(2)
    emb = [(torch.randn((vocab, k), device=dev, generator=g) * 0.02).to(torch.bfloat16)
           for _ in range(2)]
    h = torch.randn((k,), device=dev, generator=g).to(torch.bfloat16)
    logits = torch.empty((vocab,), dtype=torch.bfloat16, device=dev)
    bv = torch.empty(((vocab + 7) // 8,), dtype=torch.float32, device=dev)
    bi = torch.empty(((vocab + 7) // 8,), dtype=torch.int32, device=dev)
    am = torch.empty((1,), dtype=torch.int32, device=dev)
    calls = [0]

    def step(ev):
        e = emb[calls[0] & 1]
        calls[0] += 1
        hip.lm_head_bf16(e, None, h, logits, bv, bi, am, vocab, k)
    t, _ = time_steps(step, 100, 10)
    nbytes = 2 * vocab * k + 2 * k + 2 * vocab + 4
    us = t / 100 * 1e3
    return {"us_per_call": round(us, 2), "GBs": round(nbytes / (us * 1e-6) / 1e9, 1),
            "bytes": nbytes}


MFMA_PEAK_TFLOPS = 2500.0  # MI355X dense BF16


class PrefillLayers:
    """Config 3: `layers` layers x the 7 Linears at M tokens, each layer with
    its own weights (W8A16: q ~ U{-127..127}, s = bf16(|N(0,.02)|/127);
    BF16: bf16(N(0, .02))), inputs bf16(N(0,1)), seed 3; one grouped plan
    per layer (its 7 independent GEMMs in one launch)."""

    def __init__(self, dev, hip, m: int, w8: bool, layers: int = 4, seed: int = 3):
        import torch
        g = torch.Generator(device=dev)
        g.manual_seed(seed)
        self.calls = []   # per layer: list of call tuples
        self.plans = []
        for _ in range(layers):
            layer = []
            for name, n, k in SHAPES:
                x = torch.randn((m, k), device=dev, generator=g).to(torch.bfloat16)
                y = torch.empty((m, n), dtype=torch.bfloat16, device=dev)
                if w8:
                    q = torch.randint(-127, 128, (n, k), dtype=torch.int8, device=dev, generator=g)
                    sc = ((torch.randn((n, k // 64), device=dev, generator=g) * 0.02).abs_()
                          / 127.0).to(torch.bfloat16)
                    layer.append((q, sc, 64, None, x, y, m, n, k))
                else:
                    w = (torch.randn((n, k), device=dev, generator=g) * 0.02).to(torch.bfloat16)
                    layer.append((w, None, x, y, m, n, k))
            self.calls.append(layer)
            self.plans.append(hip.GemmPlan(layer))
        torch.cuda.synchronize()
        self.flops_per_layer = sum(2.0 * m * n * k for _, n, k in SHAPES)


def prefill_main(args, dev, hip) -> int:
    """Config 3: prefill GEMMs at M = --tokens.  One step = one layer's 7
    Linears as one grouped launch (value = GEMM TFLOP/s, i.e. the layer's
    FLOPs / the launch time); per-shape single calls in the roofline block."""
    import torch
    w8 = args.dtype == "w8a16"
    m = args.tokens
    pl = PrefillLayers(dev, hip, m, w8)
    nl = len(pl.plans)
    calls = [0]

    def step(ev):
        pl.plans[calls[0] % nl].launch()
        calls[0] += 1
    t, _ = time_steps(step, args.steps, args.warmup)
    ms = t / args.steps
    tflops = pl.flops_per_layer / (ms * 1e-3) / 1e12
    per_shape = {}
    for i, (name, n, k) in enumerate(SHAPES):
        def one(ev, i=i):
            c = pl.calls[calls[0] % nl][i]
            calls[0] += 1
            (hip.gemm_w8a16 if w8 else hip.gemm_bf16)(*c)
        tt, _ = time_steps(one, max(20, args.steps // 4), 5)
        us = tt / max(20, args.steps // 4) * 1e3
        per_shape[name] = {"us_per_call": round(us, 2),
                           "TFLOPs": round(2.0 * m * n * k / (us * 1e-6) / 1e12, 1)}
    line = {
        "metric": f"{'W8A16' if w8 else 'BF16'} prefill GEMM TFLOP/s (% of BF16 MFMA peak), "
                  f"Qwen2.5-0.5B Linears, M={m}",
        "value": round(tflops, 1),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8 x bf16 -> fp32" if w8 else "bf16 x bf16 -> fp32",
        "data": "synthetic",
        "config": {
            "workload": (f"config 3: one layer's 7 Qwen2.5-0.5B Linear GEMMs at M={m} as one "
                         f"grouped launch, {nl} layers of distinct weights rotated, seed 3"),
            "flops_per_step": pl.flops_per_layer,
            "parallelism": "single GPU",
        },
        "roofline": {
            "bound": "mfma",
            "kernel": "gemm_grouped_kernel (7 GEMMs of one layer)",
            "achieved": round(tflops, 1),
            "peak": MFMA_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(tflops / MFMA_PEAK_TFLOPS, 4),
            "traffic": None,
            "avg_launch_us": round(ms * 1e3, 2),
            "per_shape_single_calls": per_shape,
        },
        "cpu_baseline": None,
    }
    print(json.dumps(line))
    for p in pl.plans:
        p.close()
    return 0


def main() -> int:
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only; --gpus {args.gpus} is not "
              "supported (each GPU would serve its own model replica: value at N GPUs is "
              "N x the one-GPU figure, and no collective is on the path)", file=sys.stderr)
        return 2
    import torch
    import linear_hip as hip

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.workload == "prefill":
        return prefill_main(args, dev, hip)
    layers = Layers(dev)
    plan = hip.W8A16GemvPlan(layers.calls)
    assert abs(plan.bytes - layers.bytes) < 1, (plan.bytes, layers.bytes)

    def step_plan(ev):
        plan.launch()

    def step_calls(ev):
        for c in layers.calls:
            hip.gemv_w8a16(*c)

    step = step_plan if args.launch == "plan" else step_calls
    total_ms, _ = time_steps(step, args.steps, args.warmup)
    ms = total_ms / args.steps

    # The dominant kernel is the grouped GEMV (in plan mode the only one: one
    # launch per step, so the back-to-back step time IS its launch duration,
    # measured by events on the stream it runs on).
    if args.launch == "plan":
        launch_ms = ms
    else:
        t, _ = time_steps(step_plan, args.steps, args.warmup)
        launch_ms = t / args.steps
    achieved = plan.bytes / (launch_ms * 1e-3) / 1e9
    traffic = None
    if os.path.exists(args.traffic):
        with open(args.traffic) as f:
            traffic = json.load(f).get("w8a16_gemv_grouped_kernel")
    roofline = {
        "bound": "hbm",
        "kernel": "w8a16_gemv_grouped_kernel (168 GEMVs of one decode token)",
        "achieved": round(achieved, 1),
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(achieved / HBM_PEAK_GBS, 4),
        "traffic": traffic,
        "algorithmic_bytes_per_launch": int(plan.bytes),
        "avg_launch_us": round(launch_ms * 1e3, 2),
        "step_GBs": round(layers.bytes / (ms * 1e-3) / 1e9, 1),
    }

    detail = {"mode_ms": {}, "per_shape": {}}
    if args.detail:
        for mode, fn in (("plan", step_plan), ("calls", step_calls)):
            t, _ = time_steps(fn, max(20, args.steps // 4), 5)
            detail["mode_ms"][mode] = t / max(20, args.steps // 4)
        for name, n, k in SHAPES:
            sel = [c for c, (_, nm) in zip(layers.calls, layers.names) if nm == name]

            def one(ev, sel=sel):
                for c in sel:
                    hip.gemv_w8a16(*c)
            t, _ = time_steps(one, 20, 3)
            per_call = t / 20 / len(sel)
            detail["per_shape"][name] = {
                "us_per_call": round(per_call * 1e3, 2),
                "GBs": round(gemv_bytes(n, k) / (per_call * 1e-3) / 1e9, 1),
            }

    if args.detail:
        detail["lm_head"] = lm_head_detail(dev, hip)
    if args.copy_calibration > 0:
        src = torch.empty(args.copy_calibration << 20, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    cpu = None
    if args.cpu_seconds > 0:
        step(None)
        torch.cuda.synchronize()
        cpu, cpu_outs = cpu_baseline(layers, args.cpu_seconds)
        detail["max_err_over_tol"] = check_outputs(layers, cpu_outs)

    line = {
        "metric": METRIC,
        "value": round(1000.0 / ms, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8 x bf16 -> fp32",
        "data": "synthetic",
        "config": {
            "workload": ("config 1: W8A16 decode GEMV, M=1, 24 layers x 7 Qwen2.5-0.5B "
                         "Linear shapes = 168 GEMVs per step over 370.1 MB of distinct "
                         "int8 weights + bf16 scales, seed 1"),
            "launch": args.launch,
            "bytes_per_step": layers.bytes,
            "parallelism": "single GPU",
        },
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    if args.detail:
        with open(args.detail, "w") as f:
            json.dump({"line": line, "detail": detail}, f, indent=1)
    print(json.dumps(line))
    plan.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
