"""Benchmark of the MI355X Linear hot path and the decode step around it.

Workloads (--workload):

  e2e (default).  W8A16 greedy decode of a random-init
      Qwen2.5-0.5B-shaped model (24 layers, hidden 896, 14/2 heads, inter
      4864, vocab 151936, tied embedding; FP32 weights ~N(0, 0.02), norm
      weights 1, biases 0, seed 4, exported by the library's QWENBIN1
      exporter to group-64 int8 with BF16 scales and BF16 non-quantised
      tensors, and opened from that model directory) on the HIP decode
      runtime: prompt of 512 uniform-random tokens, prefilled once (not
      timed), max_seq 1024, BF16 KV cache.  One step = config 4's whole
      decode: the model is rewound to the end of the prompt (its KV cache
      kept) and runs the 511 greedy decode steps that follow the
      prefill's token (512 generated tokens, contexts 513-1023), each one
      graph replay, with no host sync inside the decode.  --steps such
      decodes are timed.  value = decode tokens/s.  The roofline object is
      for the decode step's dominant kernel (largest time per token), timed
      launch by launch with HIP events on the model's stream at the middle
      of the decoded context; `decode_linear` is the step's Linear launches
      combined, `linear_gemv_plan` config 1's figure (below),
      `prefill_m512` config 3's layer plan (W8A16 at M = 32/128/512, BF16 at
      512) against the MFMA peak and `lm_head` config 2's standalone LM
      head.  cpu_baseline is config 0: its own seed-0 model, the CPU FP32
      oracle model (a C restatement of the reference's cpu_ops.cpp +
      qwen2.cpp CPU path) on the same dequantised weights as the GPU's,
      prompt 32 + 128 greedy tokens, 3 timed samples (mean/p50/p95), the
      GPU's rate on the same workload beside it, and the first greedy
      divergence from the GPU checked by the near-tie rule;
      `other_configs` holds the CPU FP32 Linear path on configs 1, 2 and 3
      with the GPU time of the same work.  --detail FILE adds the reference's sweeps
      (canonical, prefill, decode context; W8A16 and W16A16), the
      per-Linear single calls and the LM head.

  gemv.  The decode-time W8A16 GEMVs of one token:
      24 layers x the 7 Linear shapes, 168 GEMVs over 370.1 MB of distinct
      int8 weights + BF16 scales (more than the 256 MB last-level cache);
      q ~ U{-127..127}, scales bf16(|N(0, 0.02)| / 127), x bf16(N(0, 1)),
      seed 1.  --launch plan: one grouped launch per step; calls: 168
      separate GEMV calls.  value = tokens/s of the Linear layers alone.

  prefill.  One layer's 7 GEMMs at M = --tokens as one
      grouped launch; value = TFLOP/s.

  ttft.  Config 4's model and prompt (--prompt tokens, seed 4, max_seq
      1024): one step = reset + the whole prefill of the prompt (embedding,
      24 layers with grouped MFMA GEMMs and the MFMA causal attention, final
      RMSNorm, LM head and argmax) and the host readback of the first token,
      timed on the host as the reference times TTFT.  value = median ms per
      prefill.  For kernel traces of the model's prefill.

Prints ONE JSON line.  All inputs are resident in HBM before timing.
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
    ap.add_argument("--steps", type=int, default=None,
                    help="timed steps (default: e2e 10 whole decodes, gemv 200, prefill 200)")
    ap.add_argument("--warmup", type=int, default=None,
                    help="untimed steps (default: e2e 2, else 20)")
    ap.add_argument("--launch", choices=("plan", "calls"), default="plan")
    ap.add_argument("--workload", choices=("e2e", "gemv", "prefill", "ttft", "tile"),
                    default="e2e",
                    help="e2e: config 4 decode (the headline); gemv: config 1; "
                         "prefill: config 3 GEMMs; ttft: config 4's prompt prefill; "
                         "tile: one GEMM on the prefill's wide MFMA tile")
    ap.add_argument("--shape", default="256,128,4864",
                    help="tile: M,N,K of the GEMM (256,128,K is one workgroup on one CU)")
    ap.add_argument("--prompt", type=int, default=512, help="e2e and ttft prompt length")
    ap.add_argument("--decode-tokens", type=int, default=0,
                    help="e2e: decode steps per bench step (default: to context 1023, the "
                         "whole of config 4's decode; fewer for counter runs)")
    ap.add_argument("--graph", choices=("on", "off"), default="on",
                    help="e2e: replay each decode step from a HIP graph (on) or launch its "
                         "kernels one by one (off; no per-kernel timing, for counter runs)")
    ap.add_argument("--tokens", type=int, default=512, help="prefill M (config 3)")
    ap.add_argument("--dtype", choices=("w8a16", "bf16"), default="w8a16",
                    help="prefill weight type")
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="bounded CPU-baseline sample length (0 disables)")
    ap.add_argument("--detail", default="",
                    help="write per-shape and per-mode measurements to this JSON file")
    ap.add_argument("--traffic", default=os.path.join(ROOT, "profiles", "traffic.json"),
                    help="committed HBM traffic per launch measured with rocprofv3 --pmc")
    args = ap.parse_args()
    if args.steps is None:
        args.steps = {"e2e": 10, "ttft": 20}.get(args.workload, 200)
    if args.warmup is None:
        args.warmup = {"e2e": 2, "ttft": 5}.get(args.workload, 20)
    return args


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


def progress(msg: str) -> None:
    """One line on stderr per long phase (stdout carries only the JSON line)."""
    print(f"bench.py: {msg}", file=sys.stderr, flush=True)


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
    threads = cpu_threads()
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
        "cpu_model": cpu_model(),
        "blas": "none: the oracle's own FP32 loops (OpenMP), no BLAS library",
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


def lm_head_detail(dev, hip, keep_inputs: bool = False):
    """Config 2: the fused LM head over two distinct 151936 x 896 BF16
    embedding copies (545 MB, alternated so no call is served from cache).
    keep_inputs returns the first copy and the hidden vector as well (keys
    "e" and "h", for the CPU baseline)."""
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
    out = {"us_per_call": round(us, 2), "GBs": round(nbytes / (us * 1e-6) / 1e9, 1),
           "bytes": nbytes}
    if keep_inputs:
        out["e"], out["h"] = emb[0], h
    return out


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


def prefill_roofline(dev, hip, steps: int = 100) -> tuple:
    """Config 3 for the default bench line: one layer's 7 Linear GEMMs as
    one grouped plan launch, 4 layers of distinct weights rotated, W8A16 at
    M = 32, 128 and 512 and BF16 at M = 512; TFLOP/s of the layer's FLOPs
    over the launch time, against the 2.5 PFLOP/s BF16 MFMA peak.  Also
    returns the W8A16 layers (the CPU baseline's inputs) and plan times."""
    out, sets = {}, {}
    for w8, m in ((True, 512), (False, 512), (True, 128), (True, 32)):
        pl = PrefillLayers(dev, hip, m, w8)
        nl = len(pl.plans)
        calls = [0]

        def step(ev):
            pl.plans[calls[0] % nl].launch()
            calls[0] += 1
        t, _ = time_steps(step, steps, 10)
        us = t / steps * 1e3
        tflops = pl.flops_per_layer / (us * 1e-6) / 1e12
        out[f"{'w8a16' if w8 else 'bf16'}_M{m}"] = {
            "us_per_layer_plan": round(us, 2), "TFLOPs": round(tflops, 1),
            "frac": round(tflops / MFMA_PEAK_TFLOPS, 4)}
        if w8:
            sets[m] = (pl.calls[0], round(us, 2))
        for plan in pl.plans:
            plan.close()
    return out, sets


WIDE_TILE = 5  # linear_hip.GEMM_TILES index of the 256 x 128 tile (8 waves)
UNIT_KINDS = {0: "whole_tile", 1: "split_part", 2: "gate_up_pair"}


def wide_timeline(plans, launches: int = 12) -> dict:
    """Where a wide-tile plan's launch spends its time: each workgroup's
    s_memrealtime stamps (entry, first stage loaded, epilogue start, end;
    100 MHz) and shader cycles from the plan's timeline launch
    (infer_hip_gemm_plan_timeline), over `launches` launches rotating the
    plans; medians over launches of per-kind medians, in microseconds."""
    import numpy as np
    import torch
    wg = plans[0].workgroups()
    words = plans[0].TIMELINE_WORDS
    stamps = torch.zeros(words * wg, dtype=torch.int64, device="cuda")
    per = []
    for i in range(launches + 2):
        for p in plans:  # warm: the plan's previous launch just ran
            p.launch()
        plans[i % len(plans)].launch_timeline(stamps)
        torch.cuda.synchronize()
        if i >= 2:
            per.append(stamps.cpu().numpy().reshape(wg, words).astype(np.int64))
    def summarize(a):
        entry, loop, epi, end = (a[:, j].astype(np.float64) for j in range(4))
        t0 = entry.min()
        unit = a[:, 6]
        stages = (unit >> 16) & 0xFF
        kind = (unit >> 24) & 0xFF
        us = 0.01  # one 100 MHz tick
        # workgroups are dealt to the XCDs round robin: every workgroup w of
        # one residue w mod 8 on one XCD, the 8 residues on 8 XCDs (the XCD
        # numbering itself may be rotated)
        xcc = a[:, 4] & 0xF
        per_residue = [set(xcc[np.arange(wg) % 8 == r].tolist()) for r in range(min(8, wg))]
        round_robin = (all(len(x) == 1 for x in per_residue) and
                       len(set().union(*per_residue)) == len(per_residue))
        res = {"kernel_span_us": (end.max() - t0) * us,
               "last_entry_us": (entry.max() - t0) * us,
               "xcd_by_workgroup_mod_8": float(round_robin),
               "xcc_of_workgroups_0_to_7": [int(v) for v in a[:8, 4]],
               "ghz_median": float(np.median(a[:, 7] / ((end - entry) * 10.0)))}
        for kcode, kname in UNIT_KINDS.items():
            sel = kind == kcode
            if not sel.any():
                continue
            res[kname] = {
                "units": int(sel.sum()),
                "stages": int(np.median(stages[sel])),
                "start_us": float(np.median(entry[sel] - t0) * us),
                "prologue_us": float(np.median(loop[sel] - entry[sel]) * us),
                "us_per_stage": float(np.median((epi[sel] - loop[sel]) / stages[sel]) * us),
                "epilogue_us": float(np.median(end[sel] - epi[sel]) * us),
                "end_us": float(np.median(end[sel] - t0) * us),
                "end_max_us": float((end[sel] - t0).max() * us),
            }
            if np.any(a[sel, 11] != 0):
                # the in-launch reduction by the XCD's workgroups: own unit
                # done -> first slice's parts arrived -> slices summed -> end
                hp = a[sel, 11].astype(np.float64)
                ar = np.where(a[sel, 9] != 0, a[sel, 9], a[sel, 11]).astype(np.float64)
                rd = a[sel, 10].astype(np.float64)
                res[kname]["help_start_us"] = float(np.median(hp - t0) * us)
                res[kname]["help_wait_us"] = float(np.median(ar - hp) * us)
                res[kname]["help_sum_us"] = float(np.median(rd - ar) * us)
                res[kname]["help_leave_us"] = float(np.median(end[sel] - rd) * us)
            elif kname == "split_part" and np.any(a[sel, 8] != 0):
                # the in-launch hand-off: partial stored, all parts arrived,
                # slices summed
                st, ar, rd = (a[sel, j].astype(np.float64) for j in (8, 9, 10))
                res[kname]["store_partial_us"] = float(np.median(st - epi[sel]) * us)
                res[kname]["wait_parts_us"] = float(np.median(ar - st) * us)
                res[kname]["sum_slices_us"] = float(np.median(rd - ar) * us)
        return res
    rows = [summarize(a) for a in per]
    def med(path):
        vals = []
        for r in rows:
            v = r
            for key in path:
                v = v.get(key) if isinstance(v, dict) else None
            if v is not None:
                vals.append(v)
        return round(float(np.median(vals)), 3) if vals else None
    out = {"workgroups": wg, "launches": len(rows),
           "xcc_of_workgroups_0_to_7": rows[-1]["xcc_of_workgroups_0_to_7"]}
    for key in ("kernel_span_us", "last_entry_us", "xcd_by_workgroup_mod_8", "ghz_median"):
        out[key] = med((key,))
    for kname in UNIT_KINDS.values():
        if kname in rows[0]:
            out[kname] = {f: med((kname, f)) for f in rows[0][kname]}
    return out


def wide_timeline_detail(dev, hip, m: int = 512) -> dict:
    """wide_timeline of the config-3 layer plans at M = 512, both dtypes."""
    out = {}
    for w8 in (True, False):
        pl = PrefillLayers(dev, hip, m, w8)
        out[f"{'w8a16' if w8 else 'bf16'}_M{m}"] = wide_timeline(pl.plans)
        for p in pl.plans:
            p.close()
    return out


def wide_tile_call(dev, hip, m: int, n: int, k: int, w8: bool, seed: int = 5):
    """One GEMM on the wide tile (synthetic config-3 distributions): returns
    a function that makes the call."""
    import torch
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    x = torch.randn((m, k), device=dev, generator=g).to(torch.bfloat16)
    y = torch.empty((m, n), dtype=torch.bfloat16, device=dev)
    if w8:
        q = torch.randint(-127, 128, (n, k), dtype=torch.int8, device=dev, generator=g)
        sc = ((torch.randn((n, k // 64), device=dev, generator=g) * 0.02).abs_()
              / 127.0).to(torch.bfloat16)
        return lambda: hip.gemm_w8a16_tile(q, sc, 64, None, x, y, m, n, k, WIDE_TILE)
    w = (torch.randn((n, k), device=dev, generator=g) * 0.02).to(torch.bfloat16)
    return lambda: hip.gemm_bf16_tile(w, None, x, y, m, n, k, WIDE_TILE)


def wide_tile_scaling(dev, hip, steps: int = 30) -> dict:
    """The wide tile alone and across the chip: one tile (one CU) at K = 896
    and 4864 separates the per-tile fixed cost from the per-stage cost, and
    64 / 128 / 152 tiles (K = 896) show the stage on many CUs at once (the
    clock under full load; rocprofv3 --pmc SQ_BUSY_CYCLES of `--workload
    tile` gives it)."""
    out = {}
    for w8 in (False, True):
        per = {}
        for (m, n, k) in ((256, 128, 896), (256, 128, 4864), (2048, 1024, 896),
                          (4096, 1024, 896), (512, 9728, 896)):
            call = wide_tile_call(dev, hip, m, n, k, w8)
            t, _ = time_steps(lambda ev: call(), steps, 5)
            per[f"{m}x{n}x{k}"] = {"us": round(t / steps * 1e3, 2),
                                   "tiles": ((m + 255) // 256) * ((n + 127) // 128),
                                   "stages": k // 64}
        a, b = per["256x128x896"]["us"], per["256x128x4864"]["us"]
        stage = (b - a) / (76 - 14)
        per["lone_tile_fixed_us"] = round(a - 14 * stage, 2)
        per["lone_tile_us_per_stage"] = round(stage, 3)
        for key in ("2048x1024x896", "4096x1024x896", "512x9728x896"):
            per[key]["us_per_stage_beyond_fixed"] = round(
                (per[key]["us"] - per["lone_tile_fixed_us"]) / 14, 3)
        out["w8a16" if w8 else "bf16"] = per
    return out


def tile_main(args, dev, hip) -> int:
    """One GEMM of --shape on the prefill's wide MFMA tile (256 x 128 of Y per
    workgroup of 8 waves, gemm_*_tile with the tile named): one step = one
    call; value = TFLOP/s.  For counter runs of the tile alone (one
    workgroup) and across the chip."""
    m, n, k = (int(v) for v in args.shape.split(","))
    w8 = args.dtype == "w8a16"
    call = wide_tile_call(dev, hip, m, n, k, w8)
    t, _ = time_steps(lambda ev: call(), args.steps, args.warmup)
    ms = t / args.steps
    tflops = 2.0 * m * n * k / (ms * 1e-3) / 1e12
    line = {
        "metric": f"{'W8A16' if w8 else 'BF16'} GEMM on the wide MFMA tile, M,N,K = {m},{n},{k}",
        "value": round(tflops, 2), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None,
        "dtype": "int8 x bf16 -> fp32" if w8 else "bf16 x bf16 -> fp32", "data": "synthetic",
        "config": {"workload": f"one gemm_{'w8a16' if w8 else 'bf16'}_tile call on the 256 x 128 "
                               f"tile: {((m + 255) // 256) * ((n + 127) // 128)} workgroups of "
                               f"{k // 64} stages", "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "kernel": "gemm_wide_kernel", "achieved": round(tflops, 2),
                     "peak": MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(tflops / MFMA_PEAK_TFLOPS, 4), "traffic": None,
                     "avg_launch_us": round(ms * 1e3, 2)},
        "cpu_baseline": None,
    }
    print(json.dumps(line))
    return 0


def committed_traffic(path: str, key: str):
    """HBM bytes per launch of `key` from the committed rocprofv3 --pmc
    summary (profiles/traffic.json), or None."""
    if not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f).get(key)


def prefill_cpu_baseline(pl, m: int, w8: bool, seconds: float, gpu_us: float) -> dict:
    """The reference's CPU FP32 prefill GEMMs (cpu_ops.cpp:108-123
    linear_fp32_batch, the oracle's C/OpenMP restatement) on the host cores,
    on the first layer's dequantised weights and inputs of this line: the 7
    GEMMs timed for about `seconds` (at least 3 layers); mean/p50/p95 per
    layer, TFLOP/s of the mean.  The GPU's BF16 outputs of the same layer
    (one plan launch) are compared with the CPU's FP32 ones."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import numpy as np
    import torch
    import oracle  # test infrastructure: the CPU baseline leg only
    oracle.build()
    threads = cpu_threads()
    host = []
    for c in pl.calls[0]:
        if w8:
            qn = c[0].cpu().numpy()
            sn = c[1].view(torch.int16).cpu().numpy().view(np.uint16)
            w = oracle.dequant_w8a16(qn, sn, 64, threads)
            x = c[4].float().cpu().numpy()
        else:
            w = c[0].float().cpu().numpy()
            x = c[2].float().cpu().numpy()
        host.append((w, x))
    outs = [None] * len(host)

    def layer():
        for i, (w, x) in enumerate(host):
            outs[i] = oracle.linear_fp32_batch(w, None, x, threads)
    t = repeat_for(layer, seconds)
    ms = stats_of([v * 1e3 for v in t])
    pl.plans[0].launch()
    torch.cuda.synchronize()
    worst = 0.0
    for c, ref in zip(pl.calls[0], outs):
        got = (c[5] if w8 else c[3]).float().cpu().numpy()
        scale = float(np.sqrt(np.mean(ref.astype(np.float64) ** 2))) or 1.0
        worst = max(worst, float(np.max(np.abs(got - ref))) / scale)
    tflops = pl.flops_per_layer / (ms["mean"] * 1e-3) / 1e12
    return {
        "value": round(tflops, 4), "unit": "TFLOP/s", "cores": threads, "kind": "port",
        "cpu_model": cpu_model(),
        "blas": "none: the oracle's own FP32 loops (OpenMP), no BLAS library",
        "sample": (f"{len(t)} layers of the 7 GEMMs at M={m} (layer 0's dequantised FP32 weights "
                   f"and inputs) in {sum(t):.1f} s; C/OpenMP restatement of cpu_ops.cpp "
                   f"linear_fp32_batch"),
        "ms_per_layer": ms, "gpu_us_same_work": round(gpu_us, 2),
        "gpu_speedup": round(ms["mean"] * 1e3 / gpu_us, 1),
        "gpu_max_abs_err_over_rms": round(worst, 5),
    }


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
            # (the plan's kernel: gemm_skinny_preferred for all 7 shapes, else tiles)
            "kernel": ("gemm_skinny_kernel (7 GEMMs of one layer; 32 weight rows per "
                       "workgroup, down_proj split over K)" if m <= (64 if w8 else 32) else
                       "gemm_wide_grouped_kernel + splitk_reduce_kernel (7 GEMMs of one layer; "
                       "256 x 128 tiles, down_proj split over K)" if m >= 256 else
                       "gemm_grouped_kernel (7 GEMMs of one layer; 64 x 64 tiles)"),
            "achieved": round(tflops, 1),
            "peak": MFMA_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(tflops / MFMA_PEAK_TFLOPS, 4),
            "traffic": None,
            "avg_launch_us": round(ms * 1e3, 2),
            "per_shape_single_calls": per_shape,
        },
        "cpu_baseline": (prefill_cpu_baseline(pl, m, w8, args.cpu_seconds, ms * 1e3)
                         if args.cpu_seconds > 0 else None),
    }
    if m == 512 and w8:
        line["roofline"]["traffic"] = committed_traffic(args.traffic, "gemm_wide_plan_w8a16_M512")
    if m >= 256:
        line["roofline"]["timeline"] = wide_timeline(pl.plans)
    print(json.dumps(line))
    for p in pl.plans:
        p.close()
    return 0


def near_tie_rule(gpu_logits, ref_logits, gpu_tok: int, ref_tok: int) -> dict:
    """The per-step rule of tests/test_gpu_model.py: a different argmax is a
    near-tie when the oracle's margin between the two tokens is within
    twice the step's largest logit error plus the BF16 rounding of the
    logits."""
    import numpy as np
    g = np.asarray(gpu_logits, dtype=np.float64)
    r = np.asarray(ref_logits, dtype=np.float64)
    err = float(np.max(np.abs(g - r)))
    margin = float(r[ref_tok] - r[gpu_tok])
    bound = 2 * err + 2.0 ** -8 * float(np.max(np.abs(r)))
    cos = float(g @ r / np.sqrt((g @ g) * (r @ r)))
    return {"gpu_token": int(gpu_tok), "oracle_token": int(ref_tok), "margin": margin,
            "bound": bound, "logits_cosine": round(cos, 6), "near_tie": margin <= bound}


def cpu_threads() -> int:
    """Threads for the CPU baselines: the process's affinity mask, capped by
    OMP_NUM_THREADS when it is set."""
    threads = len(os.sched_getaffinity(0))
    env = os.environ.get("OMP_NUM_THREADS")
    if env and env.isdigit():
        threads = min(threads, int(env))
    return threads


def cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo), for the CPU baselines."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def repeat_for(fn, seconds: float, min_reps: int = 3, max_reps: int = 10000):
    """Calls fn() at least min_reps times and until `seconds` have passed;
    returns the per-call times in seconds."""
    times = []
    t_end = time.perf_counter() + seconds
    while len(times) < min_reps or (time.perf_counter() < t_end and len(times) < max_reps):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return times


def linear_cpu_baselines(layers, lm, prefill_sets, seconds: float) -> dict:
    """The reference's CPU FP32 Linear path (cpu_ops.cpp:23-30, 108-123,
    175-177: the oracle's C/OpenMP restatement) on the host cores, on the
    same dequantised weights and inputs the GPU figures of this run use:
    config 1 (the 168 GEMVs of a token), config 2 (the tied LM head + argmax,
    qwen2.cpp:421-424) and config 3 (one layer's 7 GEMMs at M = 32/128/512).
    Each is timed for about `seconds` (at least 3 calls): mean/p50/p95 per
    call, beside the GPU's time for the same work."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import numpy as np
    import torch
    import oracle  # test infrastructure: the CPU baseline leg only
    oracle.build()
    threads = cpu_threads()
    out = {"cores": threads, "kind": "port", "cpu_model": cpu_model(),
           "blas": "none: the oracle's own FP32 loops (OpenMP), no BLAS library",
           "what": "FP32 C/OpenMP restatement of cpu_ops.cpp linear_fp32 / linear_fp32_batch / "
                   "argmax on the dequantised weights"}

    def host_w8(q, sc):
        qn = q.cpu().numpy()
        sn = sc.view(torch.int16).cpu().numpy().view(np.uint16)
        return oracle.dequant_w8a16(qn, sn, 64, threads)

    # config 1
    ws = [(host_w8(c[0], c[1]), c[4].float().cpu().numpy()) for c in layers["calls"]]
    wbytes = sum(w.nbytes for w, _ in ws)

    def one_token():
        for w, x in ws:
            oracle.linear_fp32(w, None, x, threads)
    t = repeat_for(one_token, seconds)
    ms = stats_of([v * 1e3 for v in t])
    out["config1_gemv_168"] = {
        "ms_per_token": ms, "fp32_weight_bytes": int(wbytes),
        "GBs": round(wbytes / (ms["mean"] * 1e-3) / 1e9, 1), "calls": len(t),
        "gpu_us_same_work": layers["gpu_us"],
        "gpu_speedup": round(ms["mean"] * 1e3 / layers["gpu_us"], 1)}
    del ws
    # config 2
    e32 = lm["e"].float().cpu().numpy()
    h32 = lm["h"].float().cpu().numpy()

    def head():
        oracle.argmax(oracle.linear_fp32(e32, None, h32, threads))
    t = repeat_for(head, seconds)
    ms = stats_of([v * 1e3 for v in t])
    out["config2_lm_head"] = {
        "ms_per_call": ms, "fp32_weight_bytes": int(e32.nbytes),
        "GBs": round(e32.nbytes / (ms["mean"] * 1e-3) / 1e9, 1), "calls": len(t),
        "gpu_us_same_work": lm["gpu_us"],
        "gpu_speedup": round(ms["mean"] * 1e3 / lm["gpu_us"], 1)}
    del e32
    # config 3
    c3 = {}
    for m, (calls, gpu_us) in prefill_sets.items():
        gw = [(host_w8(c[0], c[1]), c[4][:m].float().cpu().numpy()) for c in calls]
        flops = sum(2.0 * m * w.shape[0] * w.shape[1] for w, _ in gw)

        def layer():
            for w, x in gw:
                oracle.linear_fp32_batch(w, None, x, threads)
        t = repeat_for(layer, seconds / 2)
        ms = stats_of([v * 1e3 for v in t])
        c3[f"M{m}"] = {"ms_per_layer": ms, "GFLOPs": round(flops / (ms["mean"] * 1e-3) / 1e9, 1),
                       "calls": len(t), "gpu_us_same_work": gpu_us,
                       "gpu_speedup": round(ms["mean"] * 1e3 / gpu_us, 1)}
        del gw
    out["config3_gemm_layer_w8a16"] = c3
    return out


def config0_baseline(cfg, seconds: float, samples: int = 3):
    """Config 0: its own random-init model (seed 0, N(0, 0.02), norm weights
    1, biases 0) exported to W8A16 and opened on the GPU, and on the CPU the
    FP32 oracle model on the same dequantised weights (the FP32 work per
    token of config 0's model).  Workload: prompt of 32 uniform-random
    tokens (seed 0), 128 greedy tokens, max_seq 256.  The CPU decode is
    sampled `samples` times after one warm-up (mean/p50/p95 over the
    samples, per-token latency p50/p95 over all their steps); the GPU
    decodes the same workload (one graph replay a token).  Where the two
    greedy sequences first differ, both models are teacher-forced to the
    common prefix and that step is checked with the per-step near-tie rule;
    a difference that is not a near-tie fails the bench."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import shutil
    import tempfile
    import numpy as np
    import archive_hip
    import model_hip
    import oracle  # test infrastructure: the CPU baseline leg only
    import synthetic as S
    oracle.build()
    threads = cpu_threads()
    max_seq, prompt_len, out_len = 256, 32, 128
    workdir = tempfile.mkdtemp(prefix="qwen-config0-")
    try:
        checkpoint = S.random_checkpoint(cfg, seed=0, std=0.02, plain_init=True)
        export_model_dir(cfg, checkpoint, workdir, "w8a16")
        del checkpoint
        gpu = model_hip.Qwen2Model.open(workdir, "w8a16", max_sequence_length=max_seq)
        with archive_hip.ModelArchive(os.path.join(workdir, "model.w8a16.qbin")) as archive:
            tensors = {r.name: archive.data(r.name) for r in archive.records}
    finally:
        shutil.rmtree(workdir, ignore_errors=True)
    fp32 = S.dequantized_fp32(tensors, cfg)
    del tensors
    cpu = oracle.Model(fp32, cfg.num_layers, cfg.hidden_size, cfg.num_heads, cfg.num_kv_heads,
                       cfg.intermediate_size, cfg.vocab_size, max_seq, cfg.rms_norm_eps,
                       cfg.rope_theta, threads)
    del fp32
    prompt = [int(v) for v in np.random.default_rng(0).integers(0, cfg.vocab_size, prompt_len)]
    runs = []
    for r in range(samples + 1):  # the first run warms up
        t0 = time.perf_counter()
        tok = cpu.prefill(prompt)
        prefill_s = time.perf_counter() - t0
        toks, step_ms = [tok], []
        t0 = time.perf_counter()
        while len(toks) < out_len:
            t1 = time.perf_counter()
            toks.append(cpu.decode(toks[-1], prompt_len + len(toks) - 1))
            step_ms.append((time.perf_counter() - t1) * 1e3)
            if time.perf_counter() - t0 >= seconds:
                break
        decode_s = time.perf_counter() - t0
        if r > 0:
            runs.append((prefill_s, decode_s, step_ms, toks))
    cpu_tokens = runs[0][3]
    if any(rr[3] != cpu_tokens[:len(rr[3])] for rr in runs):
        raise SystemExit("bench: repeated CPU decodes of one prompt gave different tokens")
    rates = [len(rr[2]) / rr[1] for rr in runs]
    steps_all = [v for rr in runs for v in rr[2]]
    # the GPU on the same workload
    first = gpu.prefill(prompt)
    steps = len(cpu_tokens) - 1
    gpu_times = []
    for _ in range(4):
        gpu.rewind(prompt_len, first)
        t0 = time.perf_counter()
        gpu_tokens_tail = gpu.decode_steps(steps)
        gpu_times.append(time.perf_counter() - t0)
    gpu_tokens = [first] + list(gpu_tokens_tail)
    gpu_rate = steps / float(np.median(gpu_times[1:]))
    first_diff = next((i for i, (a, b) in enumerate(zip(gpu_tokens, cpu_tokens)) if a != b),
                      None)
    divergence = None
    if first_diff is not None:
        ref_tok, ref_logits = cpu.prefill(prompt, logits=True)
        gpu.reset()
        gpu_tok = gpu.prefill(prompt)
        for i in range(first_diff):
            ref_tok, ref_logits = cpu.decode(cpu_tokens[i], prompt_len + i, logits=True)
            gpu_tok = gpu.decode_next(cpu_tokens[i])
        divergence = near_tie_rule(gpu.last_logits_host(), ref_logits, gpu_tok, ref_tok)
        divergence["step"] = first_diff
    cpu.close()
    gpu.close()
    st = stats_of(rates)
    return {
        "value": st["mean"],
        "unit": "tok/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"config 0: seed-0 random-init model, prompt {prompt_len}, {steps} greedy "
                   f"decode steps, max_seq {max_seq}; {samples} timed decodes after one "
                   f"warm-up ({sum(len(rr[2]) for rr in runs)} steps, "
                   f"{sum(rr[1] for rr in runs):.1f} s); FP32 C/OpenMP restatement of "
                   f"cpu_ops.cpp + the qwen2.cpp CPU op order on the W8A16-dequantised weights"),
        "cpu_model": cpu_model(),
        "blas": "none: the oracle's own FP32 loops (OpenMP), no BLAS library",
        "decode_tok_s": st,
        "decode_ms_per_token": stats_of(steps_all),
        "prefill_tok_s": stats_of([prompt_len / rr[0] for rr in runs]),
        "ttft_ms": stats_of([rr[0] * 1e3 for rr in runs]),
        "gpu_same_workload_tok_s": round(gpu_rate, 1),
        "gpu_speedup": round(gpu_rate / st["mean"], 1),
        "greedy_tokens_compared": len(cpu_tokens),
        "first_divergence_vs_gpu": first_diff,
        "divergence_check": divergence,
    }


LINEAR_KINDS = ("qkv_gemv", "attn_o_gemv", "gate_up_gemv", "down_gemv")


def e2e_roofline(model, mid: int, ms_per_token: float, traffic_path: str):
    """The decode step's dominant kernel kind (largest time per token), from
    the model's per-kind graph replays timed with HIP events on its stream
    (infer_hip_model_kernel_times, which resets the model), and the decode
    Linear launches' combined rate (decode_linear)."""
    kt = model.kernel_times(mid, reps=20)
    per_token_us = {n: us * launches for n, (us, _, launches) in kt.items()}
    dominant = max(per_token_us, key=per_token_us.get)
    us, nbytes, launches = kt[dominant]
    achieved = nbytes / (us * 1e-6) / 1e9
    traffic = None
    if os.path.exists(traffic_path):
        with open(traffic_path) as f:
            traffic = json.load(f).get(dominant)
    step_bytes = sum(nb * ln for (_, nb, ln) in kt.values())
    breakdown = {n: {"us_per_launch": round(u, 2), "launches_per_token": ln,
                     "us_per_token": round(u * ln, 1), "GBs": round(nb / (u * 1e-6) / 1e9, 1)}
                 for n, (u, nb, ln) in kt.items()}
    lin = [kt[n] for n in LINEAR_KINDS if n in kt]
    lin_bytes = sum(nb * ln for (_, nb, ln) in lin)
    lin_us = sum(u * ln for (u, _, ln) in lin)
    lin_gbs = lin_bytes / (lin_us * 1e-6) / 1e9
    return {
        "bound": "hbm",
        "kernel": f"{dominant} (decode step, W8A16, context {mid + 1})",
        "achieved": round(achieved, 1),
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(achieved / HBM_PEAK_GBS, 4),
        "traffic": traffic,
        "algorithmic_bytes_per_launch": int(nbytes),
        "avg_launch_us": round(us, 2),
        "decode_linear": {
            "what": ("the decode step's Linear launches per token (q|k|v with the RMSNorm, "
                     "o with the attention merge and residual, gate|up with the RMSNorm and "
                     "SiLU-mul, down with the residual): their compulsory bytes over their "
                     "summed launch time"),
            "bytes_per_token": int(lin_bytes),
            "us_per_token": round(lin_us, 1),
            "achieved": round(lin_gbs, 1),
            "unit": "GB/s",
            "frac": round(lin_gbs / HBM_PEAK_GBS, 4),
        },
        "decode_step": {
            "compulsory_bytes_per_token": int(step_bytes),
            "step_GBs": round(step_bytes / (ms_per_token * 1e-3) / 1e9, 1),
            "kernels": breakdown,
        },
    }


def export_model_dir(cfg, checkpoint, workdir: str, precision: str):
    """The reference's export_model.py then Qwen2Model(dir): the FP32
    checkpoint through the library's QWENBIN1 exporter into workdir."""
    import archive_hip
    with open(os.path.join(workdir, "config.json"), "w") as f:
        json.dump({"model_type": "qwen2", "hidden_size": cfg.hidden_size,
                   "intermediate_size": cfg.intermediate_size,
                   "num_hidden_layers": cfg.num_layers,
                   "num_attention_heads": cfg.num_heads,
                   "num_key_value_heads": cfg.num_kv_heads, "vocab_size": cfg.vocab_size,
                   "max_position_embeddings": 32768, "eos_token_id": cfg.eos_token_id,
                   "rms_norm_eps": cfg.rms_norm_eps, "rope_theta": cfg.rope_theta,
                   "tie_word_embeddings": True}, f)
    return archive_hip.export(checkpoint, os.path.join(workdir, f"model.{precision}.qbin"),
                              precision, 64, source="random_checkpoint(seed=4)")


def stats_of(values):
    import numpy as np
    v = np.asarray(values, dtype=np.float64)
    return {"mean": round(float(v.mean()), 3), "p50": round(float(np.percentile(v, 50)), 3),
            "p95": round(float(np.percentile(v, 95)), 3)}


def e2e_detail(workdirs: dict, cfg, warmup: int = 5, repeat: int = 20) -> dict:
    """The reference's protocol (docs/performance.md:44-52) on the HIP path,
    W8A16 and W16A16, models opened from their exported model directories:
    canonical (32 prompt + 128 output, max_seq 256), prefill sweep (1/32/128/
    512 prompt + 1 output, max_seq 640), decode context sweep (32/128/512
    prompt + 128 output, max_seq 640; and 895 + 128 at max_seq 1024, contexts
    to 1023).  Each cell: warmup 5, repeat 20, prompt seed 0."""
    import numpy as np
    import model_hip
    out = {}
    for precision, wd in workdirs.items():
        res = {}

        def run(max_seq, prompt_len, new_tokens):
            progress(f"detail {precision}: prompt {prompt_len} + {new_tokens}, max_seq {max_seq}")
            prompt = [int(v) for v in
                      np.random.default_rng(0).integers(0, cfg.vocab_size, prompt_len)]
            m = model_hip.Qwen2Model.open(wd, precision, max_sequence_length=max_seq)
            for _ in range(warmup):
                m.generate(prompt, new_tokens, stop_on_eos=False)
            ttft, dec = [], []
            for _ in range(repeat):
                _, st = m.generate(prompt, new_tokens, stop_on_eos=False)
                ttft.append(st.ttft_ms)
                if new_tokens > 1:
                    dec.append(st.decode_tokens_per_second())
            m.close()
            cell = {"ttft_ms": stats_of(ttft),
                    "prefill_tok_s": round(prompt_len / (float(np.median(ttft)) * 1e-3), 1)}
            if dec:
                cell["decode_tok_s"] = stats_of(dec)
                cell["tpot_ms"] = round(1000.0 / float(np.median(dec)), 4)
            return cell

        res["canonical_32+128_max256"] = run(256, 32, 128)
        res["prefill_sweep_max640"] = {f"p{p}": run(640, p, 1) for p in (1, 32, 128, 512)}
        sweep = {f"context_{p}": run(640, p, 128) for p in (32, 128, 512)}
        sweep["context_895_to_1023_max1024"] = run(1024, 895, 128)
        res["decode_context_sweep"] = sweep
        out[precision] = res
    return out


def linear_calls_detail(dev) -> dict:
    """tools/linear_benchmark.cpp:230-550 on the HIP path: each of the seven
    Linears of a layer as its own call (the reference's per-Linear call
    pattern), M = 1 (GEMV) and M = 32 / 128 / 512 (GEMM), W8A16 and BF16,
    weights rotated over 4 layers' distinct tensors.  The calls of a shape
    are captured as one HIP graph of 24 calls and replayed, so a call's time
    is its kernel plus the gap to the next launch (no host overhead); per
    shape the mean over 10 replays after 3, and the layer's sum."""
    import torch
    import linear_hip as hip
    out = {}
    g = torch.Generator(device=dev)
    g.manual_seed(5)
    layers = 4
    for w8 in (True, False):
        for m in (1, 32, 128, 512):
            per = {}
            total_us = 0.0
            for name, n, k in SHAPES:
                calls = []
                for _ in range(layers):
                    x = torch.randn((m, k), device=dev, generator=g).to(torch.bfloat16)
                    y = torch.empty((m, n), dtype=torch.bfloat16, device=dev)
                    if w8:
                        q = torch.randint(-127, 128, (n, k), dtype=torch.int8, device=dev,
                                          generator=g)
                        sc = ((torch.randn((n, k // 64), device=dev, generator=g) * 0.02)
                              .abs_() / 127.0).to(torch.bfloat16)
                        calls.append((q, sc, 64, None, x, y, m, n, k) if m > 1 else
                                     (q, sc, 64, None, x, y, n, k))
                    else:
                        w = (torch.randn((n, k), device=dev, generator=g) * 0.02).to(
                            torch.bfloat16)
                        calls.append((w, None, x, y, m, n, k) if m > 1 else
                                     (w, None, x, y, n, k))
                fn = ({(True, True): hip.gemv_w8a16, (True, False): hip.gemm_w8a16,
                       (False, True): hip.gemv_bf16, (False, False): hip.gemm_bf16}
                      [(w8, m == 1)])
                per_graph = 24

                def timed(fn, calls):
                    for i in range(layers):  # eager once: argument checks, warm caches
                        fn(*calls[i])
                    torch.cuda.synchronize()
                    graph = torch.cuda.CUDAGraph()
                    with torch.cuda.graph(graph):
                        for i in range(per_graph):
                            fn(*calls[i % layers])

                    def one(ev, graph=graph):
                        graph.replay()
                    t, _ = time_steps(one, 10, 3)
                    return t / (10 * per_graph) * 1e3

                def cell_of(us):
                    if m == 1:
                        nbytes = (gemv_bytes(n, k) if w8 else 2 * n * k + 2 * k + 2 * n)
                        return {"us_per_call": round(us, 2),
                                "GBs": round(nbytes / (us * 1e-6) / 1e9, 1)}
                    return {"us_per_call": round(us, 2),
                            "TFLOPs": round(2.0 * m * n * k / (us * 1e-6) / 1e12, 2)}
                us = timed(fn, calls)
                total_us += us
                per[name] = cell_of(us)
                # A Linear whose lone call splits K with a workspace
                # (infer_hip_gemm_*_ws): the same call on a zeroed workspace.
                need = hip.gemm_workspace_bytes(m, n, k) if m > 1 else 0
                if need:
                    ws = torch.zeros(need // 4 + 1, dtype=torch.int32, device=dev)
                    wfn = hip.gemm_w8a16_ws if w8 else hip.gemm_bf16_ws
                    per[name + "_with_workspace"] = cell_of(
                        timed(wfn, [c + (ws,) for c in calls]))
                    del ws
            out[f"{'w8a16' if w8 else 'bf16'}_M{m}"] = {"per_shape": per,
                                                        "layer_us": round(total_us, 2)}
    return out


def torch_mm_detail(dev) -> dict:
    """The vendor library on the same GEMM shapes, for comparison: torch.mm
    (hipBLASLt) of BF16 X [M, K] by a contiguous BF16 W^T [K, N], each
    shape's 24 calls (4 layers' tensors rotated) captured as one HIP graph
    and replayed, as linear_calls_detail times this library's calls.  Not a
    Linear of the reference: plain BF16, no bias, no W8A16."""
    import torch
    out = {}
    g = torch.Generator(device=dev)
    g.manual_seed(6)
    layers, per_graph = 4, 24
    for m in (32, 128, 512):
        per = {}
        total_us = 0.0
        for name, n, k in SHAPES:
            calls = []
            for _ in range(layers):
                x = torch.randn((m, k), device=dev, generator=g).to(torch.bfloat16)
                wt = (torch.randn((k, n), device=dev, generator=g) * 0.02).to(torch.bfloat16)
                calls.append((x, wt, torch.empty((m, n), dtype=torch.bfloat16, device=dev)))
            for x, wt, y in calls:
                torch.mm(x, wt, out=y)
            torch.cuda.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                for i in range(per_graph):
                    x, wt, y = calls[i % layers]
                    torch.mm(x, wt, out=y)
            t, _ = time_steps(lambda ev: graph.replay(), 10, 3)
            us = t / (10 * per_graph) * 1e3
            total_us += us
            per[name] = {"us_per_call": round(us, 2),
                         "TFLOPs": round(2.0 * m * n * k / (us * 1e-6) / 1e12, 2)}
            del graph, calls
        out[f"bf16_M{m}"] = {"per_shape": per, "layer_us": round(total_us, 2)}
    return out


def torch_sum_read(dev) -> dict:
    """A library streaming read for comparison: torch's sum over 1 GiB of
    FP32 (more than the 256 MB last-level cache).  A reduction kernel, not a
    bandwidth ceiling: the Linear GEMV plan reads faster."""
    import torch
    x = torch.ones((1 << 28,), dtype=torch.float32, device=dev)
    t, _ = time_steps(lambda ev: x.sum(), 20, 3)
    ms = t / 20
    del x
    return {"kernel": "torch.sum over 1 GiB FP32", "us": round(ms * 1e3, 1),
            "GBs": round((1 << 30) / (ms * 1e-3) / 1e9, 1)}


def calibration_detail(dev) -> dict:
    """The floors the rooflines and the decode-step analysis are read against,
    measured with libinfer_calib.so (csrc/calibration.hip), every kernel
    replayed in a HIP graph:
    - hbm_read: a read-only 16-byte streaming kernel over 370,108,416 B (one
      decode token's Linear weights), 5 per graph, on 512 and on 65536
      workgroups (the two ends of a sweep over 512-65536, where both read
      fastest; 2048-4096 read ~15 % slower): the HBM read rate of a kernel
      that does nothing but read, the best of the two;
    - launch_floor: an empty kernel of 608 workgroups (the gate|up launch's
      grid), 48 per graph: the fixed cost of one launch in a replay; and the
      same for 1-4096 workgroups (`by_blocks`);
    - cold_read_gate_up: 48 reads of distinct 8,716,288-byte buffers (a
      layer's int8 gate and up weights; 418 MB together, more than the
      256 MB last-level cache) on the same 608-workgroup grid: the launch
      floor plus the weight stream of the decode step's gate|up launch,
      without its scales, activations or arithmetic."""
    import torch
    import calibration_hip as cal
    sink = torch.zeros(1, dtype=torch.int32, device=dev)
    out = {}

    def per_launch_us(fn, count, replays=10):
        fn(0)  # eager once
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for i in range(count):
                fn(i)
        t, _ = time_steps(lambda ev: graph.replay(), replays, 3)
        del graph
        return t / (replays * count) * 1e3

    nbytes = 370108416
    buf = torch.ones(nbytes // 4, dtype=torch.int32, device=dev)
    grids = {}
    for blocks in (512, 65536):
        us = per_launch_us(lambda i: cal.stream_read(buf, sink, blocks), 5)
        grids[str(blocks)] = {"us": round(us, 2), "GBs": round(nbytes / (us * 1e-6) / 1e9, 1)}
    out["hbm_read"] = {"bytes": nbytes, "by_grid": grids,
                       "GBs": max(g["GBs"] for g in grids.values())}
    del buf
    out["launch_floor"] = {
        "blocks": 608, "us_per_launch": round(per_launch_us(lambda i: cal.empty(608), 48), 2),
        "by_blocks": {str(b): round(per_launch_us(lambda i: cal.empty(b), 48), 2)
                      for b in (1, 64, 256, 1024, 2048, 4096)}}
    per = 8716288
    bufs = torch.ones((48, per // 4), dtype=torch.int32, device=dev)
    us = per_launch_us(lambda i: cal.stream_read(bufs[i], sink, 608), 48)
    out["cold_read_gate_up"] = {
        "bytes": per, "blocks": 608, "us_per_launch": round(us, 2),
        # the same bytes on other grids: 608 workgroups leave 96 CUs with a
        # third workgroup
        "by_blocks": {str(b): round(per_launch_us(
            lambda i: cal.stream_read(bufs[i], sink, b), 48), 2) for b in (256, 512, 1024, 2048)}}
    del bufs
    # XCD L2 contents across kernels: the same buffer read by 32 launches in
    # a row (a launch's workgroups land on the same XCDs as the previous
    # one's, whose L2s still hold the lines) against 32 distinct buffers.
    keep = {}
    for mb in (8, 16):
        nb = mb << 20
        bufs = torch.ones((32, nb // 4), dtype=torch.int32, device=dev)
        same = per_launch_us(lambda i: cal.stream_read(bufs[0], sink, 1024), 32)
        distinct = per_launch_us(lambda i: cal.stream_read(bufs[i], sink, 1024), 32)
        keep[f"{mb}MB"] = {"same_buffer_us": round(same, 2),
                           "distinct_buffers_us": round(distinct, 2)}
        del bufs
    out["l2_across_launches"] = keep
    if int(sink.item()) != 0:
        raise RuntimeError("calibration read wrote its sink")
    out["cu_rates"] = cu_rates(dev)
    return out


def cu_rates(dev, blocks: int = 256, iters: int = 2000) -> dict:
    """The compute-unit rates a GEMM stage is built from (csrc/calibration.hip
    cu_probe_kernel, one workgroup per CU, each timing its whole loop with
    the shader clock): LDS read and write bytes per clock per CU, cycles per
    v_mfma_f32_32x32x16_bf16 per SIMD alone and with the W8A16 fold (in
    blocks after each chain, with four partials in rotation, and pinned one
    MFMA then four FMAs), MFMAs beside LDS reads, and L2-to-LDS fills
    directly and through registers; at 4 and 8 waves per CU (1 and 2 per
    SIMD).  `GHz` is the shader clock over the 100 MHz clock."""
    import torch
    import calibration_hip as cal
    cycles = torch.zeros(2 * blocks, dtype=torch.int64, device=dev)
    sink = torch.zeros(1, dtype=torch.int32, device=dev)
    src = torch.ones(1 << 18, dtype=torch.int32, device=dev)
    out = {}
    for name, (_, lds_bytes, mfma, _) in cal.CU_PROBES.items():
        for threads in (256, 512):
            cal.cu_probe(name, blocks, threads, 10, cycles, sink, src)
            cal.cu_probe(name, blocks, threads, iters, cycles, sink, src)
            torch.cuda.synchronize()
            c = cycles.view(blocks, 2).cpu().double()
            shader, real = c[:, 0].median().item(), c[:, 1].median().item()
            waves = threads // 64
            line = {"GHz": round(shader / (real * 10.0), 3)}
            if lds_bytes:
                line["B_per_clk_per_CU"] = round(waves * iters * lds_bytes / shader, 1)
            if mfma:
                line["cycles_per_mfma_per_SIMD"] = round(shader / (waves / 4 * iters * mfma), 2)
            out[f"{name}/{waves}_waves"] = line
    return out


def e2e_main(args, dev):
    import numpy as np
    import torch
    import model_hip
    import synthetic as S
    cfg = S.QWEN25_0_5B
    max_seq = 1024
    prompt_len = args.prompt
    decode_len = max_seq - 1 - prompt_len   # config 4: 512 generated = 1 + 511 decode steps
    if args.decode_tokens > 0:
        decode_len = min(decode_len, args.decode_tokens)
    if decode_len < 1:
        print(f"bench.py: prompt {prompt_len} leaves no decode step at max_seq {max_seq}",
              file=sys.stderr)
        return 2
    # Config 4's model: the FP32 checkpoint exported to a W8A16 archive and
    # opened from its model directory (the reference's export_model.py then
    # Qwen2Model(dir, options)).
    import shutil
    import tempfile
    import archive_hip
    graph = args.graph == "on"
    workdirs = {p: tempfile.mkdtemp(prefix=f"qwen-{p}-") for p in ("w8a16", "w16a16")}
    try:
        t0 = time.perf_counter()
        progress("random FP32 checkpoint (seed 4)")
        checkpoint = S.random_checkpoint(cfg, seed=4, std=0.02, plain_init=True)
        t1 = time.perf_counter()
        progress("export to W8A16 QWENBIN1")
        report = export_model_dir(cfg, checkpoint, workdirs["w8a16"], "w8a16")
        t2 = time.perf_counter()
        if args.detail:
            export_model_dir(cfg, checkpoint, workdirs["w16a16"], "w16a16")
        del checkpoint
        t3 = time.perf_counter()
        progress("open the model directory")
        model = model_hip.Qwen2Model.open(workdirs["w8a16"], "w8a16",
                                          max_sequence_length=max_seq, use_graph=graph)
        t4 = time.perf_counter()
        archive_info = {"export_s": round(t2 - t1, 2), "open_s": round(t4 - t3, 2),
                        "archive_bytes": report["bytes"],
                        "max_groupwise_abs_error": report["max_groupwise_abs_error"],
                        "init_s": round(t1 - t0, 2)}
        prompt = [int(v) for v in
                  np.random.default_rng(4).integers(0, cfg.vocab_size, prompt_len)]
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        progress(f"prefill {prompt_len} tokens")
        first = model.prefill(prompt)
        ttft_ms = (time.perf_counter() - t0) * 1e3
        # One step = config 4's whole decode: back to the end of the prompt
        # (its KV cache is kept; no prefill inside the timed region), then
        # decode_len free-running greedy steps, one graph replay each.
        tokens = []

        def step():
            model.rewind(prompt_len, first)
            tokens.append(model.decode_steps(decode_len))
        progress(f"{args.warmup} + {args.steps} decodes of {decode_len} tokens")
        for _ in range(args.warmup):
            step()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            step()
        torch.cuda.synchronize()
        elapsed = time.perf_counter() - t0
        if any(t != tokens[0] for t in tokens):
            raise SystemExit("bench: repeated decodes of one prompt gave different tokens")
        ms_per_step = elapsed * 1e3 / args.steps
        ms_per_token = ms_per_step / decode_len
        mid = prompt_len + decode_len // 2
        roofline = None
        if graph:
            progress("per-kind launch timing")
            roofline = e2e_roofline(model, mid, ms_per_token, args.traffic)
        # Config 1 beside it: the 168 Linear GEMVs of a token as one grouped plan.
        import linear_hip as hip
        layers = Layers(dev)
        plan = hip.W8A16GemvPlan(layers.calls)
        t_plan, _ = time_steps(lambda ev: plan.launch(), 100, 10)
        plan_ms = t_plan / 100
        plan_gbs = plan.bytes / (plan_ms * 1e-3) / 1e9
        plan_line = {
            "workload": "config 1: 168 W8A16 GEMVs of one token (24 layers x 7 shapes), one "
                        "grouped launch",
            "achieved": round(plan_gbs, 1), "unit": "GB/s",
            "frac": round(plan_gbs / HBM_PEAK_GBS, 4), "avg_launch_us": round(plan_ms * 1e3, 2),
        }
        if roofline is not None:
            roofline["linear_gemv_plan"] = plan_line
        plan.close()
        model.close()
        # Configs 3 and 2 beside it: the prefill GEMM layer plan at M = 512
        # (MFMA-bound) and the standalone fused LM head (HBM-bound).
        progress("config 3 prefill GEMM layer plans")
        prefill, prefill_sets = prefill_roofline(dev, hip)
        progress("config 2 LM head")
        lm = lm_head_detail(dev, hip, keep_inputs=True)
        if roofline is not None:
            roofline["prefill_m512"] = {
                "bound": "mfma",
                "kernel": ("gemm_wide_grouped_kernel + splitk_reduce_kernel: one layer's 7 "
                           "Linear GEMMs at M = 512 as one grouped plan launch (config 3)"),
                "achieved": prefill["w8a16_M512"]["TFLOPs"], "peak": MFMA_PEAK_TFLOPS,
                "unit": "TFLOP/s", "frac": prefill["w8a16_M512"]["frac"],
                "avg_launch_us": prefill["w8a16_M512"]["us_per_layer_plan"],
                "traffic": committed_traffic(args.traffic, "gemm_wide_plan_w8a16_M512"),
                "north_star_target_frac": 0.40, "by_config": prefill}
            roofline["lm_head"] = {
                "bound": "hbm",
                "kernel": ("lm_head_bf16 (config 2: fused tied-embedding GEMV + FP32 argmax, "
                           "151936 x 896, two embedding copies alternated)"),
                "achieved": lm["GBs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(lm["GBs"] / HBM_PEAK_GBS, 4), "avg_launch_us": lm["us_per_call"],
                "algorithmic_bytes_per_launch": lm["bytes"]}
        cpu = None
        if args.cpu_seconds > 0:
            progress("CPU baseline: config 0 (seed-0 model)")
            cpu = config0_baseline(cfg, args.cpu_seconds)
            progress("CPU baselines: configs 1, 2, 3")
            cpu["other_configs"] = linear_cpu_baselines(
                {"calls": layers.calls, "gpu_us": plan_line["avg_launch_us"]},
                {"e": lm["e"], "h": lm["h"], "gpu_us": lm["us_per_call"]},
                prefill_sets, min(3.0, args.cpu_seconds))
        del layers, prefill_sets
        lm.pop("e", None)
        lm.pop("h", None)
        detail = None
        if args.detail:
            progress("detail sweeps")
            detail = {"e2e": e2e_detail(workdirs, cfg), "linear_calls": linear_calls_detail(dev),
                      "torch_mm_bf16": torch_mm_detail(dev),
                      "lm_head": lm_head_detail(dev, hip), "torch_sum_read": torch_sum_read(dev),
                      "gemm_wide_tile_scaling": wide_tile_scaling(dev, hip),
                      "gemm_wide_timeline": wide_timeline_detail(dev, hip),
                      "calibration": calibration_detail(dev)}
    finally:
        for wd in workdirs.values():
            shutil.rmtree(wd, ignore_errors=True)
    line = {
        "metric": METRIC,
        "value": round(args.steps * decode_len / elapsed, 1),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "w8a16: int8 weights x bf16 activations, fp32 accumulate",
        "data": "synthetic",
        "config": {
            "workload": (f"config 4: W8A16 greedy decode, random-init Qwen2.5-0.5B-shaped "
                         f"model (seed 4), prompt {prompt_len} (prefill once, untimed: "
                         f"{ttft_ms:.2f} ms), one step = the whole {decode_len}-token decode "
                         f"to context {prompt_len + decode_len} (max_seq {max_seq}), BF16 KV "
                         f"cache, batch 1, "
                         + ("one HIP graph replay per token" if graph
                            else "kernels launched one by one")),
            "decode_tokens_per_step": decode_len,
            "ms_per_token": round(ms_per_token, 5),
            "parallelism": "single GPU",
            "archive": archive_info,
            "first_token": first,
            "last_token": tokens[-1][-1],
        },
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    if args.detail:
        with open(args.detail, "w") as f:
            json.dump({"line": line, "detail": detail}, f, indent=1)
    print(json.dumps(line))
    div = (cpu or {}).get("divergence_check")
    if div is not None and not div["near_tie"]:
        print(f"bench.py: GPU and CPU greedy tokens differ at step {div['step']} by more "
              f"than a near-tie: {div}", file=sys.stderr)
        return 3
    return 0


def ttft_main(args, dev) -> int:
    """Config 4's prompt prefill on the HIP runtime, host-timed per prefill
    (the reference's TTFT, docs/performance.md:44-52): the model is reset,
    then Qwen2Model.prefill runs the prompt and reads back the first token."""
    import shutil
    import tempfile
    import numpy as np
    import model_hip
    import synthetic as S
    cfg = S.QWEN25_0_5B
    max_seq = 1024
    if not 1 <= args.prompt < max_seq:
        print(f"bench.py: prompt {args.prompt} does not fit max_seq {max_seq}", file=sys.stderr)
        return 2
    workdir = tempfile.mkdtemp(prefix="qwen-w8a16-")
    try:
        checkpoint = S.random_checkpoint(cfg, seed=4, std=0.02, plain_init=True)
        export_model_dir(cfg, checkpoint, workdir, "w8a16")
        del checkpoint
        model = model_hip.Qwen2Model.open(workdir, "w8a16", max_sequence_length=max_seq)
        prompt = [int(v) for v in
                  np.random.default_rng(4).integers(0, cfg.vocab_size, args.prompt)]
        firsts, times, all_ms = [], [], []
        for i in range(args.warmup + args.steps):
            model.reset()
            t0 = time.perf_counter()
            firsts.append(model.prefill(prompt))
            all_ms.append((time.perf_counter() - t0) * 1e3)
            if i >= args.warmup:
                times.append(all_ms[-1])
        model.close()
    finally:
        shutil.rmtree(workdir, ignore_errors=True)
    if any(f != firsts[0] for f in firsts):
        raise SystemExit("bench: repeated prefills of one prompt gave different tokens")
    line = {
        "metric": f"W8A16 prefill latency (TTFT) of a {args.prompt}-token prompt, "
                  "Qwen2.5-0.5B b=1",
        "value": round(float(np.median(times)), 4),
        "unit": "ms",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(float(np.mean(times)), 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "w8a16: int8 weights x bf16 activations, fp32 accumulate",
        "data": "synthetic",
        "config": {"workload": f"config 4's model (seed 4) and {args.prompt}-token prompt, "
                               f"max_seq {max_seq}: reset + prefill + first-token readback",
                   "prefill_ms": stats_of(times), "first_token": firsts[0],
                   # the first prefill of the model (cold) and the second
                   "first_prefill_ms": round(all_ms[0], 4),
                   "second_prefill_ms": round(all_ms[1], 4) if len(all_ms) > 1 else None,
                   "prefill_tok_s": round(args.prompt / float(np.median(times)) * 1e3, 1),
                   "parallelism": "single GPU"},
        "roofline": None,
        "cpu_baseline": None,
    }
    print(json.dumps(line))
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
    if args.workload == "e2e":
        return e2e_main(args, dev)
    if args.workload == "ttft":
        return ttft_main(args, dev)
    if args.workload == "tile":
        return tile_main(args, dev, hip)
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
