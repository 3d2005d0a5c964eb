#!/usr/bin/env python3
"""Benchmark of the W4A16 hot path on one MI355X: the Flux-style DiT MLP pair.

One step = fc1 3072->12288 (W4A16, bias, GELU-tanh fused into its epilogue) -> fc2 12288->3072
(W4A16, bias) over M = 4608 tokens (4096 image + 512 text), bf16 activations, int4 group-32
weights in the reference's packed layout, random init (seed 1 = config index), inputs resident in
HBM. Each linear is the engine's fp16 route: the exact row-scaled fp16 staging pass, then the
W4A16 GEMM (the 256 x 256-tile kernel at these shapes). Prints ONE JSON line (the driver's contract) with the whole-step TFLOP/s (2*M*N*K per
GEMM; GELU and staging not counted as flops), the GEMM kernel's MFMA roofline from HIP events
around its launches, the parity gate of this same run, and the CPU baseline (the oracle's fp32
dequant-then-matmul path on the host cores).

Usage: python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--no-cpu-baseline]

`--workload c1 | c3 | c4 | c5` instead measure the other BASELINE configurations (one JSON line
each, not the driver's line): C1 = the single linear x fp16 [4608, 3072] x W [3072, 3072] (W4A16,
and the reference's W4A4 numerics on the same shape); C3 = the W8A8 linear 3072 -> 21504 at
M = 4608 (per-token int8 quantize + int8 GEMM, bf16 out) against the int8 MFMA peak; C4 = the
skinny-M sweep (W4A16 at K = 4096, N = 10240 for M in {1, 4, 16, 64, 256}, plus 3072 -> 18432 at
M = 1) against the HBM peak, with 12 weight copies in rotation (more than the 256 MB last-level
cache) and the calls replayed back to back from a HIP graph; C5 = one denoise step of the 12B
Flux-style DiT with every Linear on the engine (ms/step).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16/fp16 MFMA, AMD spec
HERE = os.path.dirname(os.path.abspath(__file__))
M_TOKENS, HIDDEN, MLP = 4608, 3072, 12288
GATE = 2e-3


def parse():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-repeats", type=int, default=3)
    ap.add_argument("--workload", choices=["c1", "c2", "c3", "c4", "c5"], default="c2")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a plain 1 GiB device copy three times (reference kernel for the "
                         "FETCH_SIZE / WRITE_SIZE counters) and exit")
    return ap.parse_args()


def calibrate_copy():
    import torch
    n = 1 << 30
    src = torch.empty(n, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes": n, "launches": 3}), flush=True)


def host_cpu() -> dict:
    """The host CPU the cpu_baseline ran on: model name, logical CPUs visible to this process and
    the vector ISA extensions the kernel reports (from /proc/cpuinfo, as lscpu shows them)."""
    model, flags = "unknown", set()
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                k, _, v = line.partition(":")
                k = k.strip()
                if k == "model name" and model == "unknown":
                    model = v.strip()
                elif k == "flags" and not flags:
                    flags = set(v.split())
    except OSError:
        pass
    isa = [f for f in ("sse4_2", "avx", "avx2", "fma", "avx512f", "avx512bw", "avx512vl", "avx512_vnni", "avx512_bf16",
                       "avx_vnni", "amx_tile", "amx_bf16", "amx_int8") if f in flags]
    try:
        usable = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        usable = os.cpu_count() or 1
    return {"model": model, "logical_cpus": usable, "isa": isa}


def gelu_tanh_np(h):
    import numpy as np
    return 0.5 * h * (1.0 + np.tanh(np.float32(0.7978845608028654) * (h + np.float32(0.044715) * h * h * h)))


def cpu_baseline(x_bf16, w1, s1, b1, w2, s2, b2, repeats):
    """The oracle's CPU path (port of the reference's dequantize-then-matmul W4A16, nodes.py:43-52
    + stock matmul), fp32, timed on the whole C2 step: weights dequantized once (outside the
    timing, like Gfx906Int4Patch does at patch time), then per step matmul -> GELU -> matmul.
    Best of `repeats`."""
    import numpy as np
    sys.path.insert(0, HERE)
    from oracle import qlinear_oracle as orc
    try:
        from threadpoolctl import threadpool_info
        threads = max([p.get("num_threads", 1) for p in threadpool_info() if p.get("user_api") == "blas"] or [1])
    except Exception:
        threads = os.cpu_count() or 1
    x = orc.bf16_bits_to_f32(x_bf16)
    W1 = orc.dequant_int4(w1, s1)
    W2 = orc.dequant_int4(w2, s2)
    best = float("inf")
    for _ in range(repeats):
        t0 = time.perf_counter()
        h = x @ W1.T + b1
        h = gelu_tanh_np(h).astype(np.float32)
        y = h @ W2.T + b2
        best = min(best, time.perf_counter() - t0)
    flops = 2.0 * M_TOKENS * HIDDEN * MLP * 2
    return {"value": round(flops / best / 1e12, 4), "unit": "TFLOP/s", "cores": int(threads), "kind": "port",
            "sample": f"full C2 step on the host (M={M_TOKENS}, fp32 numpy BLAS, dequant outside the timing), "
                      f"best of {repeats}: {best:.2f} s/step", "cpu": host_cpu(), "_check": float(np.abs(y).max())}


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU: the W4A16 path is measured on a single MI355X "
                                   "and no multi-GPU sharding is launched",
                          "n_gpus": args.gpus}))
        sys.exit(2)
    if args.calibrate_copy:
        calibrate_copy()
        return
    if args.workload == "c3":
        bench_c3(args)
        return
    if args.workload == "c4":
        bench_c4(args)
        return
    if args.workload == "c5":
        bench_c5(args)
        return
    if args.workload == "c1":
        bench_c1(args)
        return
    import numpy as np
    import torch
    sys.path.insert(0, HERE)
    from comfy_ui_gfx906_tools_amd import _lib, ops

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    _lib.load_library()

    # ---- synthetic C2 inputs (seed 1 = config index), generated on the GPU -------------------
    g = torch.Generator(device=dev).manual_seed(1)
    x = torch.randn(M_TOKENS, HIDDEN, device=dev, generator=g).to(torch.bfloat16)
    w1f = torch.randn(MLP, HIDDEN, device=dev, generator=g) * 0.02
    w2f = torch.randn(HIDDEN, MLP, device=dev, generator=g) * 0.02
    b1 = (torch.randn(MLP, device=dev, generator=g) * 0.02).to(torch.bfloat16)
    b2 = (torch.randn(HIDDEN, device=dev, generator=g) * 0.02).to(torch.bfloat16)
    w1q, w1s = ops.quantize_pack_int4(w1f)  # the reference's quantizer rule, on the device
    w2q, w2s = ops.quantize_pack_int4(w2f)
    del w1f, w2f

    # HIP events around each GEMM call, recorded on the stream the library launches on (torch's
    # current stream, which _lib passes to every entry point)
    gemm_events = {"fc1": [], "fc2": []}

    def linear(a16, rs, wq, ws, bias, record, name, gelu=False, rowscaled=False):
        if record:
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record()
        # the fp16 dequant's column factors, the group-major scale copy and the output bound are
        # computed once per weight and kept with it (as the node's Linear does), not per call
        y = _lib.w4a16_gemm(a16, wq, ws, bias, out_dtype=torch.bfloat16, row_scale=rs, gelu=gelu,
                            col_scale=_lib.cached_col_scales(ws), scales_kn=_lib.cached_scales_kn(ws),
                            f16_rowscaled=rowscaled,
                            out_bound=_lib.cached_out_bound(wq, ws, bias) if rowscaled else None)
        if record:
            e1.record()
            gemm_events[name].append((e0, e1))
        return y

    def step(record=False):
        # x (bf16) staged once as the row-scaled fp16 operand; fc1 with GELU-tanh fused into its
        # epilogue writes the bf16 activation directly as fc2's row-scaled fp16 operand
        x16, rsx = _lib.rows_to_f16(x)
        h16, rsh = linear(x16, rsx, w1q, w1s, b1, record, "fc1", gelu=True, rowscaled=True)
        return linear(h16, rsh, w2q, w2s, b2, record, "fc2")

    # ---- parity gate of this run (fp32-dequant reference on the GPU, BASELINE tolerance) -----
    x16a, rsa = _lib.rows_to_f16(x)
    h32 = _lib.w4a16_gemm(x16a, w1q, w1s, b1.float(), out_dtype=torch.float32, row_scale=rsa)
    ref1 = x.float() @ dequant_fp32(w1q, w1s).t() + b1.float()
    err1 = ((h32 - ref1).abs().max() / ref1.abs().max()).item()
    hg = torch.nn.functional.gelu(h32.to(torch.bfloat16), approximate="tanh")
    x16, rs = _lib.rows_to_f16(hg)
    y32 = _lib.w4a16_gemm(x16, w2q, w2s, b2.float(), out_dtype=torch.float32, row_scale=rs)
    ref2 = hg.float() @ dequant_fp32(w2q, w2s).t() + b2.float()
    err2 = ((y32 - ref2).abs().max() / ref2.abs().max()).item()
    # the timed step itself (fused fc1 -> fc2 through the row-scaled fp16 activation) against the
    # fp32 reference chain with bf16 rounding between the ops: within 1 bf16 ulp + the gate
    ys = step().float()
    hb = torch.nn.functional.gelu((x.float() @ dequant_fp32(w1q, w1s).t() + b1.float()).to(torch.bfloat16),
                                  approximate="tanh")
    yr = (hb.float() @ dequant_fp32(w2q, w2s).t() + b2.float())
    yr_b = yr.to(torch.bfloat16).float()
    ulp = torch.exp2(torch.floor(torch.log2(yr_b.abs().clamp_min(2.0 ** -126))) - 7)
    step_excess = ((ys - yr_b).abs() - (ulp + GATE * yr.abs().max())).max().item()
    step_err = ((ys - yr).abs().max() / yr.abs().max()).item()
    del ref1, ref2, h32, y32, hg, x16, rs, x16a, rsa, ys, hb, yr, yr_b, ulp

    # ---- timing ---------------------------------------------------------------------------------
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step(record=True)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms_step = elapsed * 1e3 / args.steps
    flops_step = 2.0 * M_TOKENS * HIDDEN * MLP * 2
    value = flops_step / (elapsed / args.steps) / 1e12
    avg_ms = {k: sum(a.elapsed_time(b) for a, b in v) / len(v) for k, v in gemm_events.items()}
    flops_launch = 2.0 * M_TOKENS * HIDDEN * MLP  # fc1 and fc2 have the same 2*M*N*K
    # roofline of the dominant kernel: the fc1 GEMM call (w4a16_tile256_kernel: 768 whole 256 x 256
    # tiles, then the last 96 tiles as 192 halves of 128 x 256 in a second launch; HIP events around
    # both), the largest GEMM of the step
    achieved = flops_launch / (avg_ms["fc1"] * 1e-3) / 1e12

    traffic = None
    tpath = os.path.join(HERE, "profiles", "w4a16_tile256_c2_fc1_traffic.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            traffic = json.load(f).get("hbm_bytes_per_launch")

    out = {
        "metric": "W4A16 GEMM TFLOP/s + % MFMA peak at M=4608 Flux shapes; DiT step ms",
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (seeded random bf16 activations, random int4 group-32 weights in the reference layout)",
        "config": {"workload": "C2 Flux DiT MLP pair: W4A16 fc1 3072->12288 + GELU-tanh + W4A16 fc2 12288->3072",
                   "tokens": M_TOKENS, "hidden": HIDDEN, "mlp": MLP, "group": 32, "activations": "bf16",
                   "route": "row-scaled fp16 staging of x + fp16 MFMA, fp32 accumulate; fc1's bf16 GELU output "
                            "stored as fc2's row-scaled fp16 operand (no second staging pass)",
                   "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(achieved / PEAK_BF16_TFLOPS, 4), "traffic": traffic,
                     "kernel": "w4a16_tile256_kernel, fc1 GEMM call with fused GELU (M=4608 N=12288 K=3072, "
                               "347.9 GFLOP)",
                     "avg_launch_ms": round(avg_ms["fc1"], 4)},
        "gemm_ms": {k: round(v, 4) for k, v in avg_ms.items()},
        "parity": {"fc1_max_rel_err": err1, "fc2_max_rel_err": err2, "gate": GATE,
                   "step_max_rel_err_bf16_out": step_err, "step_excess_over_1ulp_plus_gate": step_excess,
                   "pass": bool(err1 <= GATE and err2 <= GATE and step_excess <= 0.0)},
    }
    if not args.no_cpu_baseline:
        cb = cpu_baseline(orc_bits(x), w1q.cpu().numpy(), w1s.cpu().numpy(), b1.float().cpu().numpy(),
                          w2q.cpu().numpy(), w2s.cpu().numpy(), b2.float().cpu().numpy(), args.cpu_repeats)
        cb.pop("_check", None)
        out["cpu_baseline"] = cb
    print(json.dumps(out), flush=True)


PEAK_INT8_TOPS = 5000.0  # MI355X dense int8 MFMA, AMD spec
PEAK_HBM_GBS = 8000.0    # MI355X HBM3E


def bench_c3(args):
    """C3: y = W8A8(x) for the fused single-stream linear 3072 -> 21504 at M = 4608. One step =
    per-token int8 quantize of the bf16 activations + the int8 GEMM with the per-token x
    per-channel epilogue, bf16 out. Parity: the int32 accumulators equal a float64 matmul of the
    same codes (exact), and the bf16 output equals torch's fp32 composition in the same order."""
    import numpy as np
    import torch
    sys.path.insert(0, HERE)
    from comfy_ui_gfx906_tools_amd import _lib
    M, K, N = 4608, 3072, 21504
    torch.cuda.set_device(0)
    _lib.load_library()
    g = torch.Generator(device="cuda").manual_seed(2)
    x = torch.randn(M, K, device="cuda", generator=g).to(torch.bfloat16)
    w = torch.randn(N, K, device="cuda", generator=g) * 0.02
    wq, sw = _lib.quantize_int8_per_token(w)  # per-output-channel weight rule (same kernel)
    del w
    xq, sx = _lib.quantize_int8_per_token(x)
    acc = _lib.w8a8_gemm(xq, None, wq, None, out_dtype=torch.int32)
    exact = bool(torch.equal(acc.double(), xq.double() @ wq.double().t()))
    y = _lib.w8a8_gemm(xq, sx, wq, sw, out_dtype=torch.bfloat16)
    same = bool(torch.equal(y, (acc.float() * (sx[:, None] * sw[None, :])).to(torch.bfloat16)))
    del acc
    ev = []

    def step(record):
        q, s = _lib.quantize_int8_per_token(x)
        if record:
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
        out = _lib.w8a8_gemm(q, s, wq, sw, out_dtype=torch.bfloat16)
        if record:
            e1.record()
            ev.append((e0, e1))
        return out

    for _ in range(args.warmup):
        step(False)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step(True)
    torch.cuda.synchronize()
    el = (time.perf_counter() - t0) / args.steps
    gemm_ms = sum(a.elapsed_time(b) for a, b in ev) / len(ev)
    ops = 2.0 * M * N * K
    out = {"metric": "W8A8 GEMM TOP/s at the C3 shape (quantize + GEMM per step)", "value": round(ops / el / 1e12, 2),
           "unit": "TOP/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(el * 1e3, 4),
           "higher_is_better": True, "dtype": "int8 (int32 accumulate)", "data": "synthetic",
           "config": {"workload": "C3 W8A8 linear 3072->21504, M=4608, per-token x per-channel, bf16 out"},
           "roofline": {"bound": "mfma", "achieved": round(ops / (gemm_ms * 1e-3) / 1e12, 2), "peak": PEAK_INT8_TOPS,
                        "unit": "TOP/s", "frac": round(ops / (gemm_ms * 1e-3) / 1e12 / PEAK_INT8_TOPS, 4),
                        "kernel": "w8a8_tile256_kernel", "avg_launch_ms": round(gemm_ms, 4)},
           "parity": {"int32_accumulators_exact": exact, "bf16_epilogue_exact": same, "pass": exact and same}}
    # the producer fusion: in the single-stream block this linear's input is the adaLN of the
    # residual stream; fused, the adaLN kernel writes the int8 operand and its scales itself
    shift = (torch.randn(K, device="cuda", generator=g) * 0.3).to(torch.bfloat16)
    scale = (torch.randn(K, device="cuda", generator=g) * 0.3).to(torch.bfloat16)

    def unfused():
        q, s = _lib.quantize_int8_per_token(_lib.adaln_modulate(x, shift, scale, out="plain"))
        return _lib.w8a8_gemm(q, s, wq, sw, out_dtype=torch.bfloat16)

    def fused():
        q, s = _lib.adaln_modulate(x, shift, scale, out="i8")
        return _lib.w8a8_gemm(q, s, wq, sw, out_dtype=torch.bfloat16)

    same_fused = bool(torch.equal(unfused(), fused()))
    times = {}
    for name, fn in (("unfused", unfused), ("fused", fused)):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(args.steps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        times[name] = e0.elapsed_time(e1) / args.steps
    out["producer_fusion"] = {"step": "adaLN(x) -> per-token int8 -> W8A8 GEMM (bf16 out)",
                              "unfused_ms": round(times["unfused"], 4), "fused_ms": round(times["fused"], 4),
                              "saved_ms": round(times["unfused"] - times["fused"], 4), "bit_identical": same_fused}
    if not args.no_cpu_baseline:
        # the oracle's exact integer matmul over the whole call: int8 codes in float64 (every
        # partial sum is an integer below 2^53, so the products and sums are exact), numpy BLAS
        # on all the host's cores, rows in chunks
        import numpy as np
        from oracle import qlinear_oracle as orc
        threads = torch.get_num_threads()
        a = xq.cpu().numpy()
        b = wq.cpu().numpy()
        t0 = time.perf_counter()
        acc64 = orc.int8_matmul_exact_f64(a, b)
        dt = time.perf_counter() - t0
        ok = bool(np.array_equal(acc64[:64], orc.int8_matmul_exact(a[:64], b)))
        out["cpu_baseline"] = {"value": round(ops / dt / 1e12, 5), "unit": "TOP/s", "cores": threads,
                               "kind": "port", "sample": f"oracle int8_matmul_exact_f64 over the whole call ({M} rows, "
                                                         f"float64 numpy BLAS, {threads} threads), {dt:.2f} s; "
                                                         f"equals the int64 oracle on the first 64 rows: {ok}",
                               "cpu": host_cpu()}
    print(json.dumps(out), flush=True)


def bench_c4(args):
    """C4: W4A16 at skinny M, HBM-bound. For each shape, 12 weight copies (> MALL) are rotated
    through 48 calls captured in one HIP graph, replayed back to back; the time per call is the
    replay time / 48 (median of 5 replays). Bytes = packed weights + fp32 scales + x + y."""
    import statistics
    import torch
    sys.path.insert(0, HERE)
    from comfy_ui_gfx906_tools_amd import _lib, ops
    torch.cuda.set_device(0)
    _lib.load_library()
    shapes = [(1, 4096, 10240), (4, 4096, 10240), (16, 4096, 10240), (64, 4096, 10240), (256, 4096, 10240),
              (1, 3072, 18432)]
    side = torch.cuda.Stream()
    res = []
    for M, K, N in shapes:
        g = torch.Generator(device="cuda").manual_seed(4)
        x = torch.randn(M, K, device="cuda", generator=g).to(torch.bfloat16)
        b = (torch.randn(N, device="cuda", generator=g) * 0.02).to(torch.bfloat16)
        ws = []
        for _ in range(12):
            w = torch.randn(N, K, device="cuda", generator=g) * 0.02
            q, s = ops.quantize_pack_int4(w)
            # column factors and group-major scales kept with the weight, as the node's Linear does
            ws.append((q, s, _lib.w4a16_col_scales(s), _lib.w4a16_scales_kn(s)))
        del w
        with torch.cuda.stream(side):
            for q, s, c, kn in ws:  # eager calls on the capture stream first: its workspace exists before capture
                y = _lib.w4a16_gemm(x, q, s, b, out_dtype=torch.bfloat16, col_scale=c, scales_kn=kn)
        side.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=side):
            for i in range(48):
                q, s, c, kn = ws[i % 12]
                y = _lib.w4a16_gemm(x, q, s, b, out_dtype=torch.bfloat16, col_scale=c, scales_kn=kn)
        graph.replay()
        torch.cuda.synchronize()
        times = []
        for _ in range(5):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            graph.replay()
            e1.record()
            torch.cuda.synchronize()
            times.append(e0.elapsed_time(e1) * 1e3 / 48)
        us = statistics.median(times)
        nbytes = N * K / 2 + N * (K // 32) * 4 + M * K * 2 + M * N * 2
        res.append({"M": M, "K": K, "N": N, "us_per_call": round(us, 2), "GB_s": round(nbytes / us / 1e3, 1),
                    "hbm_frac": round(nbytes / us / 1e3 / PEAK_HBM_GBS, 4)})
        del graph, ws, y
        torch.cuda.empty_cache()
    # the single-kernel read floor: the same weight + scale bytes read once per call by
    # qlinear_stream_read (no arithmetic), 12 buffers rotated through 48 graph-captured calls
    floors = {}
    for K, N in sorted({(K, N) for _, K, N in shapes}):
        nb = N * K // 2 + N * (K // 32) * 4
        bufs = [torch.empty(nb, dtype=torch.uint8, device="cuda").fill_(i + 1) for i in range(12)]
        out = torch.empty(torch.cuda.get_device_properties(0).multi_processor_count, dtype=torch.int32, device="cuda")
        with torch.cuda.stream(side):
            for bb in bufs:
                _lib.stream_read(bb, out)
        side.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=side):
            for i in range(48):
                _lib.stream_read(bufs[i % 12], out)
        graph.replay()
        torch.cuda.synchronize()
        times = []
        for _ in range(5):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            graph.replay()
            e1.record()
            torch.cuda.synchronize()
            times.append(e0.elapsed_time(e1) * 1e3 / 48)
        fus = statistics.median(times)
        floors[(K, N)] = {"bytes": nb, "us_per_call": round(fus, 2), "GB_s": round(nb / fus / 1e3, 1),
                          "hbm_frac": round(nb / fus / 1e3 / PEAK_HBM_GBS, 4)}
        del graph, bufs
        torch.cuda.empty_cache()
    for r in res:
        f = floors[(r["K"], r["N"])]
        r["read_floor_us"] = f["us_per_call"]
        r["frac_of_read_floor"] = round(f["us_per_call"] / r["us_per_call"], 4)
    print(json.dumps({"metric": "W4A16 skinny-M GB/s vs 8 TB/s HBM (C4)", "unit": "GB/s", "n_gpus": 1,
                      "dtype": "int4 weights, bf16 activations", "data": "synthetic",
                      "timing": "HIP graph of 48 calls over 12 weight copies, replayed back to back",
                      "results": res,
                      "read_floor": {f"K={k} N={n}": v for (k, n), v in floors.items()}}), flush=True)


def bench_c1(args):
    """C1: the single linear of BASELINE config 1 -- x fp16 [4608, 3072] ~ N(0, 1), W [3072, 3072]
    ~ N(0, 0.02) quantized to int4 group 32 with fp16-representable scales (amax / 7 rounded to
    fp16, stored in the fp32 scale layout), seed 0. Two GPU paths, each timed with HIP events over
    `steps` calls: the engine's W4A16 GEMM (fp16 x straight into fp16 MFMA), gated at 2e-3 against
    the fp32 dequant-then-matmul, and the reference's own W4A4 numerics (activation quantize_int4 +
    the W4A4 GEMM), checked bit-exact against the oracle on rows at both ends. CPU baseline: the
    oracle's fp32 dequant-then-matmul of the whole call on the host."""
    import numpy as np
    import torch
    sys.path.insert(0, HERE)
    from comfy_ui_gfx906_tools_amd import _lib, ext
    from oracle import qlinear_oracle as orc
    M, K, N = 4608, 3072, 3072
    torch.cuda.set_device(0)
    _lib.load_library()
    g = torch.Generator().manual_seed(0)
    x = torch.randn(M, K, generator=g).to(torch.float16)
    w = torch.randn(N, K, generator=g) * 0.02
    wb = w.numpy().reshape(N, K // 32, 32)
    s16 = (np.abs(wb).max(-1).clip(min=1e-8) / np.float32(7)).astype(np.float16).astype(np.float32)
    codes = np.clip(np.rint(wb / s16[..., None]), -8, 7).astype(np.int32).reshape(N, K)
    wq = ((codes[:, 0::2] & 0xF) | ((codes[:, 1::2] & 0xF) << 4)).astype(np.uint8).view(np.int8)
    xd, wqd, wsd = x.cuda(), torch.from_numpy(wq).cuda(), torch.from_numpy(s16).cuda()

    def timed(fn):
        for _ in range(args.warmup):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(args.steps):
            out = fn()
        e1.record()
        torch.cuda.synchronize()
        return out, e0.elapsed_time(e1) / args.steps

    # the fp16 dequant's column factors and the group-major scale copy, both kept with the weight
    # (as Gfx906Int4Ops.Linear keeps them)
    csd, knd = _lib.w4a16_col_scales(wsd), _lib.w4a16_scales_kn(wsd)
    y16, ms16 = timed(lambda: _lib.w4a16_gemm(xd, wqd, wsd, None, out_dtype=torch.float16, col_scale=csd,
                                              scales_kn=knd))
    y32 = _lib.w4a16_gemm(xd, wqd, wsd, None, out_dtype=torch.float32)
    ref = xd.float() @ dequant_fp32(wqd, wsd).t()
    err = ((y32 - ref).abs().max() / ref.abs().max()).item()
    (qa, sa), ms_q = timed(lambda: ext.quantize_int4(xd))
    y44, ms44 = timed(lambda: ext.gemm_int4(*ext.quantize_int4(xd), wqd, wsd, None, torch.float16))
    _, ms44g = timed(lambda: ext.gemm_int4(qa, sa, wqd, wsd, None, torch.float16))
    y44f = ext.gemm_int4(qa, sa, wqd, wsd, None, torch.float32).cpu().numpy()
    qa_np, sa_np = qa.cpu().numpy(), sa.cpu().numpy()
    exact = all(np.array_equal(y44f[r], orc.gemm_int4_w4a4(qa_np[r], sa_np[r], wq, s16)) for r in
                (slice(0, 32), slice(M - 32, M)))
    # a rotated layer (activation_rotation=True checkpoints): group-128 Hadamard rotation of x fused
    # into the fp16 staging pass, against the unfused sequence (fp32 rotation matmul, fp32 staging)
    from comfy_ui_gfx906_tools_amd import ops
    grp = ops.choose_rotation_group(K)
    _, ms_rot = timed(lambda: ops.int4_linear(xd, wqd, wsd, None, rotation_group=grp))
    R = ops.get_group_rotation(K, grp, xd.device)
    _, ms_rot_unfused = timed(lambda: _lib.w4a16_gemm(ops.apply_group_rotation(xd.float(), R, grp), wqd, wsd, None,
                                                      out_dtype=torch.float16, col_scale=csd, scales_kn=knd))
    flops = 2.0 * M * N * K
    out = {"metric": "W4A16 GEMM TFLOP/s at the C1 shape (x fp16 [4608, 3072], W [3072, 3072] int4 g32)",
           "value": round(flops / (ms16 * 1e-3) / 1e12, 2), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps,
           "warmup": args.warmup, "ms_per_step": round(ms16, 4), "higher_is_better": True, "dtype": "f16",
           "data": "synthetic, seed 0", "config": {"workload": "C1 single W4A16 linear, fp16 out"},
           "roofline": {"bound": "mfma", "achieved": round(flops / (ms16 * 1e-3) / 1e12, 2),
                        "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                        "frac": round(flops / (ms16 * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4)},
           "parity": {"w4a16_fp32_max_rel_err": err, "gate": GATE, "pass": bool(err <= GATE)},
           "w4a4_reference_numerics": {
               "tops_with_quantize": round(flops / (ms44 * 1e-3) / 1e12, 2),
               "tops_gemm_only": round(flops / (ms44g * 1e-3) / 1e12, 2), "ms_gemm": round(ms44g, 4),
               "ms_quantize": round(ms_q, 4),
               "int8_peak_frac_gemm": round(flops / (ms44g * 1e-3) / 1e12 / PEAK_INT8_TOPS, 4),
               "bit_exact_rows_vs_oracle": bool(exact)},
           "rotated_layer_group128": {"ms_fused": round(ms_rot, 4), "ms_unfused": round(ms_rot_unfused, 4),
                                      "tflops_fused": round(flops / (ms_rot * 1e-3) / 1e12, 2)}}
    if not args.no_cpu_baseline:
        threads = torch.get_num_threads()
        wd = orc.dequant_int4(wq, s16)
        xf = x.float().numpy()
        best = float("inf")
        for _ in range(max(1, args.cpu_repeats)):
            t0 = time.perf_counter()
            _ = xf @ wd.T
            best = min(best, time.perf_counter() - t0)
        out["cpu_baseline"] = {"value": round(flops / best / 1e12, 4), "unit": "TFLOP/s", "cores": threads,
                               "kind": "port", "sample": f"whole C1 call, fp32 numpy BLAS on the host, dequant outside "
                                                         f"the timing, best of {args.cpu_repeats}: {best:.3f} s",
                               "cpu": host_cpu()}
    print(json.dumps(out), flush=True)


def bench_c5(args):
    """C5: one denoise step of the 12B Flux-style DiT (19 double + 38 single blocks, hidden 3072,
    4096 image + 512 text tokens, batch 1), random init, every Linear on the W4A16 engine,
    attention on SDPA. Timed: `steps` whole forward steps after `warmup`, bracketed by
    synchronizations. Parity: double block 0 and single block 0 on the GPU against the same
    blocks in fp32 on the host (weights = the dequantized int4 codes, same input activations);
    the host time of those two blocks, scaled by the block counts, is the CPU baseline."""
    import numpy as np
    import torch
    sys.path.insert(0, HERE)
    from comfy_ui_gfx906_tools_amd import _lib, flux_dit as fd
    torch.cuda.set_device(0)
    _lib.load_library()
    cfg = fd.FluxDiTConfig.flux12b()
    n_side, n_txt = 64, 512
    t0 = time.perf_counter()
    with torch.no_grad():
        model = fd.FluxDiT(cfg, device="cuda", dtype=torch.bfloat16)
        fd.init_random_(model, seed=4)
        torch.cuda.synchronize()
        t_init = time.perf_counter() - t0
        inp = fd.synthetic_inputs(cfg, n_side, n_txt, seed=4, device="cuda")
        n_params = sum(b.numel() * (2 if b.dtype == torch.int8 and n.endswith("weight_q4") else 1)
                       for n, b in model.named_buffers()) + sum(p.numel() for p in model.parameters())
        for _ in range(args.warmup):
            y = model(*inp)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            y = model(*inp)
        torch.cuda.synchronize()
        step_s = (time.perf_counter() - t0) / args.steps
        finite = bool(torch.isfinite(y).all())

        # block-level parity + CPU baseline inputs: the activations entering block 0
        img, img_ids, txt, txt_ids, ts, yv, gd = inp
        dt = torch.bfloat16
        h_img = fd._linear(model.img_in, img)
        vec = fd._linear(model.time_in.in_layer, fd.timestep_embedding(ts, cfg.time_dim).to(dt))
        vec = fd._linear(model.time_in.out_layer, torch.nn.functional.silu(vec))
        vec = vec + model.guidance_in(fd.timestep_embedding(gd, cfg.time_dim).to(dt)) + model.vector_in(yv)
        h_txt = fd._linear(model.txt_in, txt)
        cos, sin = fd.rope_cos_sin(torch.cat([txt_ids, img_ids], 1), cfg.axes_dim, cfg.theta)
        dblk, sblk = model.double_blocks[0], model.single_blocks[0]
        g_img, g_txt = dblk(h_img, h_txt, vec, cos, sin)
        x_cat = torch.cat([g_txt, g_img], 1)
        g_single = sblk(x_cat, vec, cos, sin)
        torch.cuda.synchronize()

    def cpu_block(gpu_block, cls):
        blk = cls(cfg, torch.nn, dtype=torch.float32)
        sd = {}
        for name, mod in gpu_block.named_modules():
            if fd._is_engine_linear(mod):
                sd[f"{name}.weight"] = dequant_fp32(mod.weight_q4, mod.weight_scale).cpu()
                sd[f"{name}.bias"] = mod.bias.float().cpu()
        for name, p in gpu_block.named_parameters():
            if name.endswith(".scale"):
                sd[name] = p.float().cpu()
        blk.load_state_dict(sd)
        return blk

    threads = torch.get_num_threads()
    with torch.no_grad():
        c_cos, c_sin, c_vec = cos.cpu(), sin.cpu(), vec.float().cpu()
        cd = cpu_block(dblk, fd.DoubleStreamBlock)
        t0 = time.perf_counter()
        r_img, r_txt = cd(h_img.float().cpu(), h_txt.float().cpu(), c_vec, c_cos, c_sin)
        t_double = time.perf_counter() - t0
        del cd
        cs = cpu_block(sblk, fd.SingleStreamBlock)
        t0 = time.perf_counter()
        r_single = cs(x_cat.float().cpu(), c_vec, c_cos, c_sin)
        t_single = time.perf_counter() - t0
        del cs

    def rel(a, b):
        a, b = a.float().cpu().numpy().astype(np.float64), b.numpy().astype(np.float64)
        return float(np.abs(a - b).max() / np.abs(b).max())

    e_img, e_txt, e_single = rel(g_img, r_img), rel(g_txt, r_txt), rel(g_single, r_single)
    gate = 2e-2  # bf16 activations between the block's ops vs an all-fp32 host block
    lin_flops = cfg.linear_flops(n_side * n_side, n_txt)
    att_flops = cfg.attention_flops(n_side * n_side, n_txt)
    cpu_step = cfg.depth_double * t_double + cfg.depth_single * t_single
    out = {"metric": "DiT step ms (C5, 12B Flux-style, all linears W4A16)", "value": round(step_s * 1e3, 2),
           "unit": "ms/step", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
           "ms_per_step": round(step_s * 1e3, 2), "higher_is_better": False, "dtype": "bf16 activations, int4 weights",
           "data": "synthetic (random-init weights quantized on load, seeded N(0,1) inputs)",
           "config": {"workload": "C5 Flux-style DiT denoise step", "hidden": cfg.hidden, "heads": cfg.heads,
                      "double_blocks": cfg.depth_double, "single_blocks": cfg.depth_single,
                      "img_tokens": n_side * n_side, "txt_tokens": n_txt, "batch": 1,
                      "params": n_params, "attention": "torch SDPA (flash / mem-efficient)"},
           "linear_tflop_per_step": round(lin_flops / 1e12, 3), "sdpa_tflop_per_step": round(att_flops / 1e12, 3),
           "effective_tflops": round((lin_flops + att_flops) / step_s / 1e12, 1),
           "init_s": round(t_init, 1), "output_finite": finite,
           "parity": {"double_block0_img_rel_err": e_img, "double_block0_txt_rel_err": e_txt,
                      "single_block0_rel_err": e_single, "gate": gate,
                      "pass": bool(finite and max(e_img, e_txt, e_single) <= gate)},
           "cpu_baseline": {"value": round(cpu_step * 1e3, 1), "unit": "ms/step", "cores": threads, "kind": "port",
                            "sample": f"double block 0 ({t_double:.2f} s) and single block 0 ({t_single:.2f} s) in "
                                      f"fp32 torch on the host with the dequantized weights, extrapolated x"
                                      f"{cfg.depth_double} / x{cfg.depth_single} (embedders and final layer "
                                      f"left out)", "cpu": host_cpu()}}
    print(json.dumps(out), flush=True)


def dequant_fp32(w_q4, w_scale):
    """fp32 weights of the packed layout (low nibble first, two's complement) times the group
    scales, on the weights' device: the reference's dequant (nodes.py:43-52) in fp32."""
    import torch
    b = w_q4.view(torch.uint8).to(torch.int16)
    codes = torch.stack([b & 0xF, b >> 4], dim=-1).reshape(w_q4.shape[0], -1)
    codes = torch.where(codes > 7, codes - 16, codes).float()
    return codes * w_scale.float().repeat_interleave(32, dim=1)


def orc_bits(x):
    """bf16 tensor -> numpy uint16 bit patterns."""
    import torch
    return x.cpu().contiguous().view(torch.int16).numpy().view("uint16")


if __name__ == "__main__":
    main()
