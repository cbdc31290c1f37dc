#!/usr/bin/env python3
"""Benchmark of the MI355X vnpu backend on the reference's headline path.

Headline (the JSON line's `value`): BASELINE.json config 2, the int8 decode
GEMV - MATMUL_I8 with M=1, K=4096, N=32000 over packed int8 weights with
per-column scales, f32 output - reported as whole-job HBM GB/s with inputs
resident in HBM.  Bytes per call follow the reference's accounting
(src/core/scheduler.cpp:420-426): M*K + K*N + 4*(M+N) + 4*M*N.

Each step reads a different copy of the weights (rotation over > 768 MB) so
the 256 MB Infinity Cache cannot serve them.  The timed region is bracketed
by stream syncs (wall clock -> `value`) and by a hipEvent pair recorded on the
vnpu stream's own hipStream_t (GPU time / launches -> the average kernel
duration behind `roofline.achieved`).

Also printed (same line, key "extras"): the rest of config 2 (M in {1,4,8} x
N in {4096,11008,32000}) and the config-3 int8 prefill GEMM.  The CPU
baseline is the reference runtime built from its own sources, timed on this
host's cores on a bounded sample of the same GEMV.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "npuxl-improved_amd"))

from vnpu_mi355x import Session, abi, synth  # noqa: E402

HBM_PEAK_GBS = 8000.0
I8_PEAK_TOPS = 5000.0
F32_PEAK_TFLOPS = 157.3
ROTATE_BYTES = 800 << 20


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def i8_bytes(M, K, N):
    return M * K + K * N + 4 * (M + N) + 4 * M * N


class GemvCase:
    """One packed weight set replicated past the MALL, plus activations."""

    def __init__(self, s: Session, M: int, K: int, N: int, wq_dev, ws_dev, copies: int):
        self.s, self.M, self.K, self.N = s, M, K, N
        self.weights = [s.pack(wq_dev, K, N, scales=ws_dev) for _ in range(copies)]
        x = synth.normal(f"act_{M}x{K}", (M, K))
        bx = s.upload(x)
        self.a8, self.sa = s.alloc(M * K), s.alloc(4 * M)
        s.run(abi.OP_QUANTIZE_I8, X=bx, Y=self.a8, scales=self.sa, rows=M, cols=K, axis=abi.QUANT_PER_ROW)
        s.free(bx)
        self.c = s.alloc(4 * M * N)

    def cmd(self, i: int):
        return self.s.command(abi.OP_MATMUL_I8, id=i, A=self.a8, B=self.weights[i % len(self.weights)],
                              scale_a=self.sa, C=self.c, M=self.M, K=self.K, N=self.N)

    def release(self):
        for w in self.weights:
            self.s.release_packed(w)
        for b in (self.a8, self.sa, self.c):
            self.s.free(b)


class HipEvents:
    """hipEvent pair recorded on the vnpu stream's own hipStream_t (exported by
    the backend as vnpu_stream_hip_handle), i.e. on the stream the kernels run on."""

    def __init__(self, s: Session):
        self.hip = C.CDLL("libamdhip64.so")
        self.stream = C.c_void_p(s.lib.vnpu_stream_hip_handle(s.stream))
        self.e0, self.e1 = C.c_void_p(), C.c_void_p()
        for e in (self.e0, self.e1):
            assert self.hip.hipEventCreate(C.byref(e)) == 0

    def record(self, ev):
        assert self.hip.hipEventRecord(ev, self.stream) == 0

    def elapsed_ms(self) -> float:
        assert self.hip.hipEventSynchronize(self.e1) == 0
        ms = C.c_float()
        assert self.hip.hipEventElapsedTime(C.byref(ms), self.e0, self.e1) == 0
        return ms.value

    def close(self):
        self.hip.hipEventDestroy(self.e0)
        self.hip.hipEventDestroy(self.e1)


def timed(s: Session, make_cmd, steps: int, warmup: int):
    """Run warmup + steps commands.  Returns (wall seconds of the timed region,
    average GPU ns per command): the region is bracketed by stream syncs for the
    wall clock and by a hipEvent pair on the same stream for GPU time."""
    if warmup:
        s.check("submit", s.submit([make_cmd(i) for i in range(warmup)]))
        s.check("sync", s.sync())
    cmds = [make_cmd(i) for i in range(steps)]
    ev = HipEvents(s)
    s.check("sync", s.sync())
    t0 = time.perf_counter()
    ev.record(ev.e0)
    s.check("submit", s.submit(cmds))
    ev.record(ev.e1)
    s.check("sync", s.sync())
    wall = time.perf_counter() - t0
    gpu_ns = ev.elapsed_ms() * 1e6 / steps
    ev.close()
    return wall, gpu_ns


def weights_for(s: Session, K: int, N: int, name: str):
    w = synth.normal(name, (K, N), 0.02)
    bw = s.upload(w)
    del w
    wq, ws = s.alloc(K * N), s.alloc(4 * N)
    s.run(abi.OP_QUANTIZE_I8, X=bw, Y=wq, scales=ws, rows=K, cols=N, axis=abi.QUANT_PER_COLUMN)
    s.free(bw)
    return wq, ws


def bench_gemv(s: Session, M, K, N, steps, warmup, wq=None, ws=None):
    own = wq is None
    if own:
        wq, ws = weights_for(s, K, N, f"w_{K}x{N}")
    copies = max(2, -(-ROTATE_BYTES // (K * N)))
    case = GemvCase(s, M, K, N, wq, ws, copies)
    wall, gpu_ns = timed(s, case.cmd, steps, warmup)
    case.release()
    if own:
        s.free(wq)
        s.free(ws)
    b = i8_bytes(M, K, N)
    return {"M": M, "K": K, "N": N, "copies": copies, "gbs": b * steps / wall / 1e9,
            "kernel_us": gpu_ns / 1e3, "kernel_gbs": b / gpu_ns, "bytes": b}


def bench_gemm_i8(s: Session, M, K, N, steps, warmup):
    wq, ws = weights_for(s, K, N, f"w_{K}x{N}")
    w = s.pack(wq, K, N, scales=ws)
    s.free(wq)
    s.free(ws)
    x = synth.normal(f"act_{M}x{K}", (M, K))
    bx = s.upload(x)
    a8, sa, c = s.alloc(M * K), s.alloc(4 * M), s.alloc(4 * M * N)
    s.run(abi.OP_QUANTIZE_I8, X=bx, Y=a8, scales=sa, rows=M, cols=K, axis=abi.QUANT_PER_ROW)
    s.free(bx)
    mk = lambda i: s.command(abi.OP_MATMUL_I8, id=i, A=a8, B=w, scale_a=sa, C=c, M=M, K=K, N=N)
    wall, gpu_ns = timed(s, mk, steps, warmup)
    s.release_packed(w)
    for b in (a8, sa, c):
        s.free(b)
    ops = 2.0 * M * K * N
    return {"M": M, "K": K, "N": N, "tops": ops * steps / wall / 1e12, "kernel_us": gpu_ns / 1e3,
            "kernel_tops": ops / gpu_ns / 1e3, "frac_peak": ops / gpu_ns / 1e3 / I8_PEAK_TOPS}


def cpu_baseline(M, K, N, budget_s: float):
    """The reference runtime (built from its own sources) on this host."""
    import oracle  # checker/baseline infrastructure, used only here

    if not os.path.exists(oracle.REF_LIB_PATH):
        return None
    threads = min(16, os.cpu_count() or 1)
    cfg = abi.Config()
    cfg.abi_version = 1
    cfg.num_threads = threads
    with Session(oracle.REF_LIB_PATH, cfg) as r:
        info = r.info()
        w = synth.normal(f"w_{K}x{N}", (K, N), 0.02)
        wq, ws = oracle.quantize(w, abi.QUANT_PER_COLUMN)  # bit-identical to QUANTIZE_I8
        del w
        packed = r.pack(wq, K, N, scales=ws)
        del wq
        x = synth.normal(f"act_{M}x{K}", (M, K))
        xq, xs = oracle.quantize(x, abi.QUANT_PER_ROW)
        ba, bs, bc = r.upload(xq), r.upload(xs), r.alloc(4 * M * N)
        mk = lambda: r.command(abi.OP_MATMUL_I8, A=ba, B=packed, scale_a=bs, C=bc, M=M, K=K, N=N)
        for _ in range(2):  # the reference's own warm-up count (tools/vnpu_cli.cpp:438-453)
            r.run(abi.OP_MATMUL_I8, A=ba, B=packed, scale_a=bs, C=bc, M=M, K=K, N=N)
        times = []
        t_end = time.perf_counter() + budget_s
        while time.perf_counter() < t_end and len(times) < 2000:
            t0 = time.perf_counter()
            r.check("submit", r.submit([mk()]))
            r.check("sync", r.sync())
            times.append(time.perf_counter() - t0)
        med = float(np.median(times))
        return {"value": i8_bytes(M, K, N) / med / 1e9, "unit": "GB/s",
                "cores": int(info.num_threads), "kind": "reference",
                "sample": f"MATMUL_I8 M={M} K={K} N={N} decode GEMV, {len(times)} calls "
                          f"(median {med * 1e3:.3f} ms, best {min(times) * 1e3:.3f} ms), "
                          f"reference AVX2 path, {info.num_threads} threads"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extras", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=15.0)
    ap.add_argument("--only", choices=["gemm_i8"], default=None,
                    help="run one extra workload alone (for profiling)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this backend benchmarks one GPU only; multi-GPU sharding is "
                                   "design-only (see DESIGN.md)", "n_gpus": args.gpus}))
        sys.exit(2)

    M, K, N = 1, 4096, 32000
    s = Session()
    log("device", s.info().backend.decode())
    if args.only == "gemm_i8":
        for n in (4096, 14336):
            log("gemm_i8", bench_gemm_i8(s, 2048, 4096, n, args.steps, args.warmup))
        s.close()
        return
    wq, ws = weights_for(s, K, N, f"w_{K}x{N}")
    head = bench_gemv(s, M, K, N, args.steps, args.warmup, wq, ws)
    log("headline", head)
    extras = {}
    if not args.no_extras:
        gemv = []
        for n in (4096, 11008, 32000):
            if n == N:
                q, sc = wq, ws
            else:
                q, sc = weights_for(s, K, n, f"w_{K}x{n}")
            for m in (1, 4, 8):
                r = bench_gemv(s, m, K, n, max(50, args.steps // 2), 10, q, sc)
                gemv.append({k: (round(v, 3) if isinstance(v, float) else v) for k, v in r.items()})
                log("gemv", gemv[-1])
            if n != N:
                s.free(q)
                s.free(sc)
        extras["config2_gemv"] = gemv
        gemm = []
        for n in (4096, 14336):
            r = bench_gemm_i8(s, 2048, 4096, n, 20, 5)
            gemm.append({k: (round(v, 4) if isinstance(v, float) else v) for k, v in r.items()})
            log("gemm_i8", gemm[-1])
        extras["config3_gemm_i8"] = gemm
    s.free(wq)
    s.free(ws)
    s.close()

    cpu = None if args.no_cpu_baseline else cpu_baseline(M, K, N, args.cpu_budget)
    b = head["bytes"]
    line = {
        "metric": "int8 decode GEMV HBM GB/s (config 2, M=1 K=4096 N=32000)",
        "value": round(head["gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(b / head["gbs"] / 1e6, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic: seeded N(0,1) activations, N(0,0.02) weights quantized per column",
        "config": {"workload": "MATMUL_I8 decode GEMV M=1 K=4096 N=32000, weights rotated over "
                               f"{head['copies']} HBM copies", "M": M, "K": K, "N": N},
        "roofline": {"bound": "hbm", "achieved": round(head["kernel_gbs"], 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(head["kernel_gbs"] / HBM_PEAK_GBS, 4),
                     "traffic": None, "kernel": "gemv_i8_kernel", "kernel_us": round(head["kernel_us"], 3),
                     "algorithmic_bytes": b},
        "cpu_baseline": cpu,
        "extras": extras,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
