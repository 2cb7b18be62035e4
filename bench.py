"""Benchmark of the MXFP4 MLP hot path on one MI355X (prints one JSON line).

Workload (the decode-shaped MLP the north star's
HBM target is quoted on): tokens=1, hidden=7168, intermediate=2048, x ~ f16
N(0,1), weights N(0,0.02) quantized to MXFP4 (E2M1 + E8M0 per 32 K), 77
distinct weight sets (1.8 GB) rotated inside the timed loop, as for MoE
experts.  Every configuration takes enough sets that a pass of one kernel
over one matrix per set streams at least 600 MB (over 2x the 256 MB
last-level cache); the sets the timed steps do not use run just before the
timed region, so the timed steps read from HBM.  One step = one full MLP
forward down(silu(gate(x)) * up(x)).

Secondary measurements (configs 0, 1 with T=8, 2, 3 and 4, and MoE grouped
experts at the C1 and C2 expert shapes) are reported in
the same JSON line under "secondary"; they are not the headline value.
Each carries a "roofline" block for its longest GEMM/GEMV step (HBM for the
decode GEMVs, the dequant kernels and the C3 weight-format GEMMs, the MFMA
peak of the row's arithmetic otherwise: f16 for fp16-MFMA rows and for the
scaled row, whose two FP8 x FP4 MFMAs per block take the time of one f16
MFMA; FP4 for W4A4), or for the whole pass where the library reports no
per-step times (MoE).

  value        effective TFLOP/s = 6*T*H*I / (time per step)
  roofline     the dominant kernel (fused gate/up GEMV): algorithmic bytes per
               launch / its average launch time from HIP events on the
               library stream, against 8 TB/s
  cpu_baseline the CPU oracle (a scalar C port of the reference's
               dequantize-then-accumulate MLP) on the host cores, same inputs

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-secondary]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "mpp-4.1-fp4-fp8-block_amd"))

HBM_PEAK = 8.0e12            # B/s
PEAK = {"fp4": 10.1e15, "fp8": 5.0e15, "f16": 2.5e15, "i8": 5.0e15}
METRIC = "MXFP4 MLP µs/iter + effective TFLOP/s (1×MI355X), % of MFMA/HBM roofline"
DEQUANT_NOTE = ("down GEMM takes the f32 mid as two f16 terms (hi + lo) on the fp16 MFMA, f32 x half "
                "as the reference's f_h_f")


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def roofline_block(bound, work, us, peak_key, kernel):
    """{bound, achieved, peak, unit, frac} for `work` algorithmic bytes
    (bound "hbm") or flops (bound "mfma") done in `us` microseconds."""
    rate = work / (us * 1e-6)
    if bound == "hbm":
        return {"bound": "hbm", "achieved": round(rate / 1e9, 1), "peak": HBM_PEAK / 1e9, "unit": "GB/s",
                "frac": round(rate / HBM_PEAK, 4), "kernel": kernel, "kernel_us": round(us, 3)}
    peak = PEAK[peak_key]
    return {"bound": "mfma", "achieved": round(rate / 1e12, 1), "peak": peak / 1e12, "unit": "TFLOP/s",
            "peak_dtype": peak_key, "frac": round(rate / peak, 4), "kernel": kernel, "kernel_us": round(us, 3)}


# The step kernels of the library's MLP forwards (mx_mlp_kernel_name /
# mx_fmt_mlp_kernel_name) that a roofline may be taken on, by what bounds
# them.  Anything else (quantize / split prologues, the byte-255 fix-up
# passes, the standalone SwiGLU) is never the roofline kernel.
GEMM_GATE_UP = {"gemm_q_mxfp4_gate_up_swiglu", "gemm_q_mxfp4_gate_up_swiglu_half", "gemm_h_mxfp4_gate_up_swiglu",
                "gemm_h_mxfp4_gate_up_swiglu_half", "gemm_q_scaled_gate_up_swiglu",
                "gemm_fp4_gate_up_swiglu_requant"}
GEMM_ONE = {"gemm_q_mxfp4_down", "gemm_q_mxfp4_down_f32", "gemm_h_mxfp4_down", "gemm_h_mxfp4_down_f32",
            "gemm_q_scaled_down", "gemm_fp4_down", "gemm_h_h_f_gate", "gemm_h_h_f_up", "gemm_f_h_down"}
FMT_GATE_UP = {"gemm_q_fmt_gate_up_swiglu", "gemm_h_fmt_gate_up_swiglu", "gemm_q_w8a8_gate_up_swiglu",
               "gemm_q_f8x2_fmt_gate_up_swiglu"}
FMT_DOWN = {"gemm_q_fmt_down", "gemm_h_fmt_down", "gemm_q_w8a8_down", "gemm_q_f8x2_fmt_down"}


def fmt_bytes(wfmt, n, k):
    """Bytes of one format weight matrix [n][k] with its scales."""
    if wfmt == 4:  # INT4: nibbles + f16 scale per 32
        return n * k // 2 + n * (k // 32) * 2
    return n * k + n * 4  # 8-bit codes + f32 row scale


def kernel_work(name, T, H, I, wfmt=0):
    """(bound, algorithmic flops or bytes) of one step kernel of an MLP row,
    from its name in the library's kernel table; (None, 0) for kernels that
    are not a GEMM / GEMV / dequant step."""
    if name == "gemv_mxfp4_gate_up_swiglu":  # decode GEMV: weights + activations in and out
        return "hbm", 2 * mxfp4_bytes(I, H) + T * H * 2 + T * I * 2
    if name == "gemv_mxfp4_down":
        return "hbm", mxfp4_bytes(H, I) + T * I * 2 + T * H * 2
    if name in ("dequant_gate", "dequant_up", "dequant_down"):  # MXFP4 in, f16 out
        return "hbm", mxfp4_bytes(I, H) + I * H * 2
    if name in FMT_GATE_UP:  # format rows are HBM-bound
        return "hbm", 2 * fmt_bytes(wfmt, I, H) + T * H * 2 + T * I * 2
    if name in FMT_DOWN:
        return "hbm", fmt_bytes(wfmt, H, I) + T * I * 2 + T * H * 2
    if name in GEMM_GATE_UP:
        return "mfma", 2 * T * H * 2 * I
    if name in GEMM_ONE:
        return "mfma", 2 * T * H * I
    return None, 0


def secondary_roofline(r, T, H, I, peak_key, wfmt=0):
    """Roofline of a secondary row's dominant (longest) GEMM/GEMV kernel."""
    best = None
    for name, us in (r.get("kernel_us") or {}).items():
        bound, work = kernel_work(name, T, H, I, wfmt)
        if bound and (best is None or us > best[3]):
            best = (name, bound, work, us)
    if best is None:
        return None
    name, bound, work, us = best
    return roofline_block(bound, work, us, peak_key, name)


def mxfp4_bytes(n, k):
    return n * k // 2 + n * k // 32


def sets_for(matrix_bytes, floor=600e6):
    """Weight sets so that a pass of one kernel over one matrix of each set
    streams at least `floor` bytes (over 2x the 256 MB last-level cache), so
    every per-kernel time is measured from HBM."""
    return int(-(-floor // matrix_bytes))


def make_sets(dev, M, T, H, I, n_sets, seed, wfmt=0):
    """x (f16) and n_sets weight sets, all generated and quantized on the GPU."""
    x = dev.alloc(T * H * 2)
    dev.fill_normal(x, M.DT_F16, T * H, seed, 0.0, 1.0)
    tmp = dev.alloc(max(I * H, H * I) * 4)
    sets, bufs = [], []
    for s in range(n_sets):
        mats = []
        for j, (n, k) in enumerate(((I, H), (I, H), (H, I))):
            dev.fill_normal(tmp, M.DT_F32, n * k, seed * 100 + s * 3 + j + 1, 0.0, 0.02)
            if wfmt == 0:
                q, sc = dev.alloc(n * k // 2), dev.alloc(n * k // 32)
                dev.mxfp4_quantize(tmp, M.DT_F32, n, k, q, sc)
            else:
                qb = n * k // 2 if wfmt == M.WFMT_INT4 else n * k
                sb = n * (k // 32) * 2 if wfmt == M.WFMT_INT4 else n * 4
                q, sc = dev.alloc(qb), dev.alloc(sb)
                dev.fmt_quantize(wfmt, tmp, n, k, q, sc)
            mats.append((q, sc))
            bufs += [q, sc]
        sets.append(M.Device.weights(*mats))
    tmp.free()
    dev.sync()
    return x, sets, bufs


SPINUP_S = 0.3  # untimed forwards before each row's timed region (wall-clock seconds)


def spin_up(call, iters, seconds=None):
    """Bring the GPU to steady state before a timed region: untimed
    stream-mode passes of the row's own forwards, in calls of at least ~50 ms
    of GPU work, for `seconds` of wall time.  `call(n)` runs n forwards and
    returns their seconds.  Measured on C3 FP8 (graph, 40 forwards per
    measurement, same process): 84.1, 74.5, 69.4, 69.3 us per forward for
    the first four measurements; stream-mode timing likewise settled at
    69-70 us.  A row measured first after process start or after the host
    work of a CPU baseline otherwise reports the GPU's ramp."""
    seconds = SPINUP_S if seconds is None else seconds
    if seconds <= 0:
        return
    t0 = time.time()
    per = call(iters) / iters
    n = max(iters, int(0.05 / max(per, 1e-7)))
    while time.time() - t0 < seconds:
        call(n)


def run_config(dev, M, name, variant, T, H, I, n_sets, iters, warmup, seed, wfmt=0, cpu=None, cpu_flop_cap=1e11):
    """Time `iters` forwards twice: replayed from one HIP graph, between
    timing events that are the graph's first and last nodes (the value; the
    reference likewise pre-encodes all iterations in one command buffer and
    reports its GPU start-to-end time, main.swift:2062-2133), and launched one
    by one on the stream (reported as stream_us_per_iter).
    cpu: None, or the token count of the CPU baseline sample run on this
    row's own inputs (weight set 0) before they are freed."""
    x, sets, bufs = make_sets(dev, M, T, H, I, n_sets, seed, wfmt)
    out = dev.alloc(T * H * 4)
    if wfmt:
        spin_up(lambda n: dev.fmt_mlp_benchmark(wfmt, T, H, I, x, sets, out, warmup=0, iterations=n, graph=False), iters)
    else:
        spin_up(lambda n: dev.mlp_benchmark(variant, T, H, I, x, sets, out, warmup=0, iterations=n,
                                            per_kernel=False, graph=False)[0], iters)
    if wfmt:
        secs, kern = dev.fmt_mlp_benchmark(wfmt, T, H, I, x, sets, out, warmup=warmup, iterations=iters,
                                           graph=True, per_kernel=True)
        ssecs = dev.fmt_mlp_benchmark(wfmt, T, H, I, x, sets, out, warmup=0, iterations=iters,
                                      graph=False)
    else:
        secs, kern = dev.mlp_benchmark(variant, T, H, I, x, sets, out, warmup=warmup,
                                       iterations=iters, graph=True)
        ssecs, _ = dev.mlp_benchmark(variant, T, H, I, x, sets, out, warmup=0,
                                     iterations=iters, per_kernel=False, graph=False)
    us = secs / iters * 1e6
    flops = 6.0 * T * H * I
    res = {"tokens": T, "hidden": H, "intermediate": I, "weight_sets": n_sets, "iters": iters,
           "us_per_iter": round(us, 3), "tflops": round(flops / (us * 1e-6) / 1e12, 3),
           "stream_us_per_iter": round(ssecs / iters * 1e6, 3),
           "kernel_us": {k: round(v, 3) for k, v in kern.items()}}
    if cpu:
        res["cpu_baseline"] = cpu_row(dev, M, variant, wfmt, T, H, I, x, bufs[:6], out, cpu, flop_cap=cpu_flop_cap)
    for b in bufs + [x, out]:
        b.free()
    log(f"[bench] {name}: {us:.2f} us/iter (stream {res['stream_us_per_iter']}), "
        f"{res['tflops']} TFLOP/s, kernels {res['kernel_us']}")
    return res, (x, sets)


def run_moe(dev, M, name, E, per_expert, H, I, iters, warmup, seed):
    """E experts of shape (H, I), per_expert tokens each, one grouped MoE pass
    per iteration (mx_moe_benchmark).  Expert weights N(0, 0.02), MXFP4."""
    counts = [per_expert] * E
    T = E * per_expert
    x = dev.alloc(T * H * 2)
    dev.fill_normal(x, M.DT_F16, T * H, seed, 0.0, 1.0)
    tmp = dev.alloc(E * I * H * 4)
    mats = []
    for j, (n, k) in enumerate(((E * I, H), (E * I, H), (E * H, I))):
        dev.fill_normal(tmp, M.DT_F32, n * k, seed * 100 + j + 1, 0.0, 0.02)
        q, sc = dev.alloc(n * k // 2), dev.alloc(n * k // 32)
        dev.mxfp4_quantize(tmp, M.DT_F32, n, k, q, sc)
        mats.append((q, sc))
    tmp.free()
    w = M.Device.weights(*mats)
    out = dev.alloc(T * H * 2)
    spin_up(lambda n: dev.moe_benchmark(H, I, counts, x, [w], out, warmup=0, iterations=n, graph=False), iters)
    secs = dev.moe_benchmark(H, I, counts, x, [w], out, warmup=warmup, iterations=iters, graph=True)
    us = secs / iters * 1e6
    wbytes = E * 3 * mxfp4_bytes(I, H)
    res = {"experts": E, "tokens_per_expert": per_expert, "hidden": H, "intermediate": I, "iters": iters,
           "us_per_iter": round(us, 3), "tflops": round(6.0 * T * H * I / (us * 1e-6) / 1e12, 3),
           "weight_bytes": wbytes, "hbm_gbps": round((wbytes + 2 * T * H * 2) / (us * 1e-6) / 1e9, 1)}
    res["hbm_frac"] = round(res["hbm_gbps"] * 1e9 / HBM_PEAK, 4)
    for q, sc in mats:
        q.free()
        sc.free()
    x.free()
    out.free()
    log(f"[bench] {name}: {us:.2f} us/iter, {res['tflops']} TFLOP/s, {res['hbm_gbps']} GB/s")
    return res


CPU_THREADS = 16  # the GPU box's CPU share for one GPU (its nproc may show more)


def cpu_row(dev, M, variant, wfmt, T, H, I, x, wbufs, out, tokens, budget_s=12.0, flop_cap=1e11):
    """The CPU baseline of one configuration, on that GPU row's own inputs:
    x and weight set 0 are downloaded, and the CPU port (oracle/mx_oracle.c,
    the reference's one-output-per-dot-product loop restated,
    PackedNumericKernels.metal:542-581 and 801-832, with BASELINE's
    dequantize-then-FP32-accumulate semantics) runs the first `tokens`
    tokens on CPU_THREADS host threads.  A sample smaller than T is scaled
    to the whole job and labelled extrapolated.  Its output is checked
    against the GPU's for the same tokens (max-abs / rms, cosine).  The
    sample stops at `budget_s` seconds or `flop_cap` flops, whichever
    comes first."""
    import numpy as np
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    threads = min(CPU_THREADS, os.cpu_count() or 1)
    xh = dev.download(x, np.float16, (T, H))[:tokens].copy()
    mats = []
    for j, (n, k) in enumerate(((I, H), (I, H), (H, I))):
        q, sc = wbufs[2 * j], wbufs[2 * j + 1]
        if not wfmt:
            mats += [dev.download(q, np.uint8, (n, k // 2)), dev.download(sc, np.uint8, (n, k // 32))]
        elif wfmt == M.WFMT_INT4:
            mats += [dev.download(q, np.uint8, (n, k // 2)), dev.download(sc, np.float16, (n, k // 32))]
        else:
            mats += [dev.download(q, np.uint8, (n, k)), dev.download(sc, np.float32, (n,))]
    w0 = M.Device.weights(*[(wbufs[2 * j], wbufs[2 * j + 1]) for j in range(3)])
    if wfmt:
        dev.fmt_mlp_forward(wfmt, T, H, I, x, w0, out)
        mode = None
    else:
        dev.mlp_forward(variant, T, H, I, x, w0, out)
        mode = {M.MLP_FUSED: O.MLP_F16, M.MLP_DEQUANT: O.MLP_F16, M.MLP_W4A4: O.MLP_W4A4}[variant]
    gpu = dev.download(out, np.float16, (T, H))[:tokens]

    def run():
        if wfmt:
            return O.mlp_format(wfmt, xh, *mats, H, I, threads=threads)
        return O.mlp_mxfp4(mode, xh, *mats, H, I, threads=threads)

    O.set_accum_f32(True)
    try:
        flops = 6.0 * tokens * H * I
        if flops < 5e9:
            run()  # one warm run where it is cheap
        n, t0 = 0, time.perf_counter()
        while True:
            ref = run()
            n += 1
            el = time.perf_counter() - t0
            if el >= budget_s or flops * (n + 1) > flop_cap:
                break
    finally:
        O.set_accum_f32(False)
    us = el / n * 1e6 * (T / tokens)
    rel, cos = O.mlp_error(gpu, ref)
    fmt = {0: "MXFP4", 1: "FP8 E4M3", 2: "FP8 E5M2", 3: "INT8", 4: "INT4 g32", 5: "W8A8"}[wfmt]
    what = f"{n} MLP forward(s) of {tokens} tokens" + (f", scaled x{T // tokens} (extrapolated)"
                                                        if tokens < T else "")
    return {"value": round(6.0 * T * H * I / (us * 1e-6) / 1e12, 6), "unit": "TFLOP/s",
            "us_per_iter": round(us, 1), "cores": threads, "kind": "port",
            "extrapolated": tokens < T,
            "gpu_vs_cpu": {"max_abs_over_rms": round(float(rel), 6), "cosine": round(float(cos), 7)},
            "sample": f"{what} at T={T} H={H} I={I}, {fmt} weights: this GPU row's own x and "
                      f"weight set 0, oracle/mx_oracle.c with float32 accumulation in K order, "
                      f"{threads} threads, {el:.1f} s"}


def copy_probe(nbytes=256 << 20, reps=3):
    """A plain copy kernel of known size, for calibrating the HBM traffic
    counters: every dispatch reads and writes exactly `nbytes`."""
    import torch
    a = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    b = torch.empty_like(a)
    a.fill_(1)
    for _ in range(reps):
        b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes_per_dispatch": nbytes, "dispatches": reps}), flush=True)


def traffic_file(kernel):
    return os.path.join(ROOT, "profiles", f"{kernel}_c1_t1_traffic.md")


def measured_traffic(kernel):
    """HBM bytes per launch of `kernel` at the headline shape, as recorded
    from two rocprofv3 --pmc passes (FETCH_SIZE, WRITE_SIZE) scaled by the
    copy kernel; None when no such record exists."""
    try:
        with open(traffic_file(kernel)) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":", 1)[1].strip())
    except OSError:
        pass
    return None


def main():
    global SPINUP_S
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=24)
    ap.add_argument("--no-secondary", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--spinup", type=float, default=SPINUP_S,
                    help="seconds of untimed forwards before each row's timed region (0: none; "
                         "profiler runs, whose tracer records every dispatch)")
    ap.add_argument("--only", default="",
                    help="comma-separated secondary configs to run (c1_t8,c4,c0,c2,c3,moe), or one variant "
                         "of a config (c0_fused, c2_dequant, c3_int8, ...); default all")
    ap.add_argument("--copy-probe", action="store_true",
                    help="run only a 256 MiB device-to-device copy x3 (the known-size kernel that "
                         "scales rocprofv3 FETCH_SIZE / WRITE_SIZE to bytes) and exit")
    args = ap.parse_args()
    if args.copy_probe:
        copy_probe()
        return
    SPINUP_S = args.spinup
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: --gpus {args.gpus} is not supported "
              "(the MXFP4 MLP hot path here is a single-GPU kernel; a multi-GPU run would shard "
              "the weight rows across GPUs).",
              file=sys.stderr)
        sys.exit(2)

    import mxfp4hip as M
    dev = M.Device(0)
    name, cus, clk = dev.info()
    log(f"[bench] device {name}, {cus} CUs, {clk} MHz")

    # ---- headline: config 1, T=1 ------------------------------------------
    T, H, I = 1, 7168, 2048
    n_sets = sets_for(mxfp4_bytes(H, I))  # 77: the down pass alone streams 600 MB
    prim, _ = run_config(dev, M, "C1 T=1 fused", M.MLP_FUSED, T, H, I, n_sets, args.steps,
                         args.warmup, seed=1, cpu=None if args.no_cpu else T,
                         cpu_flop_cap=4e11)  # about 12 s of host work for the headline sample
    us = prim["us_per_iter"]
    # algorithmic bytes per launch of each kernel the decode MLP may run:
    # weights + E8M0 scales + activations in + results out (for the whole
    # MLP: x in and out, the compulsory traffic BASELINE.md counts)
    mlp_bytes = 3 * mxfp4_bytes(I, H) + 2 * T * H * 2
    kernel_bytes = {"gemv_mxfp4_gate_up_swiglu": 2 * mxfp4_bytes(I, H) + T * H * 2 + T * I * 2,
                    "gemv_mxfp4_down": mxfp4_bytes(H, I) + T * I * 2 + T * H * 2}
    dom = max(prim["kernel_us"], key=prim["kernel_us"].get)   # the dominant kernel
    dom_us = prim["kernel_us"][dom]
    achieved = kernel_bytes[dom] / (dom_us * 1e-6)
    roofline = {"bound": "hbm", "achieved": round(achieved / 1e9, 1), "peak": HBM_PEAK / 1e9,
                "unit": "GB/s", "frac": round(achieved / HBM_PEAK, 4), "traffic": measured_traffic(dom),
                "kernel": dom, "algorithmic_bytes": kernel_bytes[dom],
                "kernel_us": round(dom_us, 3)}
    result = {
        "metric": METRIC, "value": prim["tflops"], "unit": "TFLOP/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "spinup_s": SPINUP_S, "ms_per_step": round(us / 1000.0, 6),
        "us_per_iter": us, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f16", "data": "synthetic",
        "config": {"workload": "BASELINE configs[1] decode MLP, tokens=1 hidden=7168 "
                               f"intermediate=2048, MXFP4 weights, {n_sets} rotated weight sets",
                   "tokens": T, "hidden": H, "intermediate": I, "weight_sets": n_sets,
                   "variant": "decode GEMV, two launches (gate/up + SwiGLU, then down), split-K "
                              "workgroups, in-register FP4 decode, fp16 MFMA"},
        "mlp_hbm_gbps": round(mlp_bytes / (us * 1e-6) / 1e9, 1),
        "mlp_hbm_frac": round(mlp_bytes / (us * 1e-6) / HBM_PEAK, 4),
        "kernel_us": prim["kernel_us"],
        "roofline": roofline,
    }

    if not args.no_secondary:
        sec = {}
        cpu = not args.no_cpu
        only = set(t for t in args.only.split(",") if t)
        want = lambda tag, variant="": not only or tag in only or f"{tag}_{variant}" in only
        if want("c1_t8"):
            r, _ = run_config(dev, M, "C1 T=8", M.MLP_FUSED, 8, 7168, 2048, sets_for(mxfp4_bytes(7168, 2048)),
                              200, 10, seed=2, cpu=cpu and 8)
            b = 3 * mxfp4_bytes(2048, 7168) + 2 * 8 * 7168 * 2
            r["hbm_frac"] = round(b / (r["us_per_iter"] * 1e-6) / HBM_PEAK, 4)
            r["roofline"] = secondary_roofline(r, 8, 7168, 2048, "f16")
            sec["c1_t8_fused"] = r
        if want("c4"):
            r, _ = run_config(dev, M, "C4 W4A4", M.MLP_W4A4, 4096, 8192, 28672, sets_for(mxfp4_bytes(8192, 28672)),
                              10, 2, seed=4, cpu=cpu and 64)
            r["fp4_mfma_frac"] = round(r["tflops"] * 1e12 / PEAK["fp4"], 4)
            r["roofline"] = secondary_roofline(r, 4096, 8192, 28672, "fp4")
            sec["c4_w4a4"] = r
        for v, tag in ((M.MLP_FUSED, "fused"), (M.MLP_DEQUANT, "dequant"), (M.MLP_W4A4, "w4a4"),
                       (M.MLP_SCALED, "scaled")):
            if not want("c0", tag):
                continue
            r, _ = run_config(dev, M, f"C0 {tag}", v, 128, 1024, 4096, sets_for(mxfp4_bytes(1024, 4096)), 100,
                              10, seed=5, cpu=cpu and tag == "fused" and 128)
            if v == M.MLP_DEQUANT:
                r["note"] = DEQUANT_NOTE
            r["roofline"] = secondary_roofline(r, 128, 1024, 4096, "fp4" if tag == "w4a4" else "f16")
            sec[f"c0_{tag}"] = r
        # the scaled row runs two FP8 x FP4 MFMAs per block (x split in two
        # E4M3 terms): the MFMA time of one f16 MFMA, so its useful FLOP/s are
        # held to the same f16 peak
        for v, tag in ((M.MLP_FUSED, "fused"), (M.MLP_DEQUANT, "dequant"), (M.MLP_SCALED, "scaled")):
            if not want("c2", tag):
                continue
            r, _ = run_config(dev, M, f"C2 {tag}", v, 512, 7168, 2048, sets_for(mxfp4_bytes(7168, 2048)), 100,
                              10, seed=6, cpu=cpu and tag == "fused" and 512)
            r["f16_mfma_frac"] = round(r["tflops"] * 1e12 / PEAK["f16"], 4)
            if v == M.MLP_DEQUANT:
                r["note"] = DEQUANT_NOTE
            r["roofline"] = secondary_roofline(r, 512, 7168, 2048, "f16")
            sec[f"c2_{tag}"] = r
        # the _f8x2 rows: the FP8 weights of the first two rows on the scaled
        # FP8 MFMA (x and mid as two E4M3 terms), against the widening rows;
        # their CPU baseline is the FP8 rows' (same weights and semantics)
        for wfmt, tag in ((M.WFMT_FP8_E4M3, "fp8_e4m3"), (M.WFMT_FP8_E5M2, "fp8_e5m2"),
                          (M.WFMT_FP8_E4M3_F8X2, "fp8_e4m3_f8x2"), (M.WFMT_FP8_E5M2_F8X2, "fp8_e5m2_f8x2"),
                          (M.WFMT_INT8, "int8"), (M.WFMT_INT4, "int4_g32"), (M.WFMT_W8A8, "w8a8")):
            if not want("c3", tag):
                continue
            fb = 4 if wfmt == M.WFMT_INT4 else 1  # fmt_bytes' format code (INT4 or 8-bit)
            wb = 3 * fmt_bytes(fb, 14336, 4096)
            r, _ = run_config(dev, M, f"C3 {tag}", None, 128, 4096, 14336, sets_for(fmt_bytes(fb, 4096, 14336)),
                              40, 4, seed=7, wfmt=wfmt, cpu=cpu and not tag.endswith("_f8x2") and 128)
            r["hbm_frac"] = round(wb / (r["us_per_iter"] * 1e-6) / HBM_PEAK, 4)
            # the longest format GEMM against HBM (weights + activations per launch)
            r["roofline"] = secondary_roofline(r, 128, 4096, 14336, None, wfmt=fb)
            sec[f"c3_{tag}"] = r
        if want("moe"):
            # MoE grouped launches at the C1 / C2 expert shapes: 64 experts x 4
            # tokens (1.5 GB of expert weights per pass) and 8 experts x 512
            r = run_moe(dev, M, "MoE C1 shape 64 experts x 4 tokens", 64, 4, 7168, 2048, 40, 4, seed=8)
            r["roofline"] = roofline_block("hbm", r["weight_bytes"] + 2 * 256 * 7168 * 2, r["us_per_iter"], None,
                                           "whole MoE pass (two grouped launches)")
            sec["moe_c1_64x4"] = r
            r = run_moe(dev, M, "MoE C2 shape 8 experts x 512 tokens", 8, 512, 7168, 2048, 20, 2, seed=9)
            r["f16_mfma_frac"] = round(r["tflops"] * 1e12 / PEAK["f16"], 4)
            r["roofline"] = roofline_block("mfma", 6.0 * 4096 * 7168 * 2048, r["us_per_iter"], "f16",
                                           "whole MoE pass (two grouped launches)")
            sec["moe_c2_8x512"] = r
        result["secondary"] = sec

    if not args.no_cpu:
        result["cpu_baseline"] = prim.pop("cpu_baseline")
    dev.close()
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
