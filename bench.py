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
N in {4096,11008,32000}), config 1 (512^3 int8 and f32+SiLU), config 3 (int8
and f32 prefill GEMMs), config 4 (its attention calls alone, and one Llama-style
layer: prefill tokens/s at
batch 1 x 2048 and decode tokens/s at batch 8, context 4096) and config 5
(int8 GEMM over half-zero weight tiles, MTP head + softmax).  The CPU
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
# MATMUL_F32 prefill runs as three bf16 products per f32 product (hi*hi +
# hi*lo + lo*hi) on the bf16 matrix cores: its matrix bound is the dense bf16
# peak over three.
BF16_PEAK_TFLOPS = 2500.0
F32_SPLIT_BOUND_TFLOPS = BF16_PEAK_TFLOPS / 3
ROTATE_BYTES = 800 << 20
# HBM bytes per headline GEMV launch from two rocprofv3 PMC passes (FETCH_SIZE,
# WRITE_SIZE; KiB per dispatch), each scaled by what the counter reads for a
# copy kernel of known size (FETCH x2.000, WRITE x1.000):
# 64,112.2 KiB x 2 + 125 KiB.  Measured offline with the commands in
# profiles/gemv_i8_m1_k4096_n32000_traffic.md; re-measure when the kernel changes.
GEMV_TRAFFIC_BYTES = 131_417_766


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


def gpu_timed(s: Session, enqueue, steps: int, warmup: int):
    """Average GPU ms per step of an enqueue() that submits several commands:
    a hipEvent pair on the vnpu stream around `steps` enqueues."""
    for _ in range(warmup):
        enqueue()
    s.check("sync", s.sync())
    ev = HipEvents(s)
    t0 = time.perf_counter()
    ev.record(ev.e0)
    for _ in range(steps):
        enqueue()
    ev.record(ev.e1)
    s.check("sync", s.sync())
    wall = time.perf_counter() - t0
    ms = ev.elapsed_ms() / steps
    ev.close()
    return ms, wall * 1e3 / steps


def rounded(d, nd=4):
    return {k: (round(v, nd) if isinstance(v, float) else v) for k, v in d.items()}


def bench_config1(s: Session, steps: int):
    """512^3 int8 (QUANTIZE rows -> MATMUL_I8 with packed per-column weights)
    and MATMUL_F32 on the same A, B with bias, alpha 1, beta 0, SiLU."""
    M = K = N = 512
    a = synth.normal("c1/A", (M, K))
    b = synth.normal("c1/B", (K, N), 0.02)
    bias = synth.normal("c1/bias", (N,), 0.1)
    ba, bb, bbias, bc = s.upload(a), s.upload(b), s.upload(bias), s.alloc(4 * M * N)
    a8, sa, b8, sb = s.alloc(M * K), s.alloc(4 * M), s.alloc(K * N), s.alloc(4 * N)
    s.run(abi.OP_QUANTIZE_I8, X=bb, Y=b8, scales=sb, rows=K, cols=N, axis=abi.QUANT_PER_COLUMN)
    w = s.pack(b8, K, N, scales=sb)
    q = lambda: s.command(abi.OP_QUANTIZE_I8, X=ba, Y=a8, scales=sa, rows=M, cols=K,
                          axis=abi.QUANT_PER_ROW)
    g = lambda: s.command(abi.OP_MATMUL_I8, A=a8, B=w, scale_a=sa, C=bc, M=M, K=K, N=N)
    f = lambda: s.command(abi.OP_MATMUL_F32, A=ba, B=bb, bias=bbias, C=bc, M=M, K=K, N=N,
                          alpha=1.0, beta=0.0, epilogue=abi.EPI_SILU)
    # The command packets are built once and the same array is submitted
    # every step, so the host's per-step cost is one vnpu_stream_submit call.
    i8_cmds = (abi.Command * 2)(q(), g())
    f32_cmds = (abi.Command * 1)(f())
    i8_ms, _ = gpu_timed(s, lambda: s.check("submit", s.lib.vnpu_stream_submit(s.stream, i8_cmds, 2, None)),
                         steps, 5)
    f32_ms, _ = gpu_timed(s, lambda: s.check("submit", s.lib.vnpu_stream_submit(s.stream, f32_cmds, 1, None)),
                          steps, 5)
    s.release_packed(w)
    for x in (ba, bb, bbias, bc, a8, sa, b8, sb):
        s.free(x)
    ops = 2.0 * M * K * N
    return {"shape": "512x512x512", "i8_quantize_plus_matmul_us": i8_ms * 1e3,
            "i8_tops": ops / i8_ms / 1e9, "f32_silu_us": f32_ms * 1e3,
            "f32_tflops": ops / f32_ms / 1e9}


def bench_gemm_f32(s: Session, M, K, N, steps, warmup):
    """Config 3 f32: B stored [N][K] (trans_b), bias, alpha 1, beta 0.5 onto C, GELU."""
    a = synth.normal(f"c3/A_{M}x{K}", (M, K))
    bt = synth.normal(f"c3/Bt_{N}x{K}", (N, K), 0.02)
    bias = synth.normal(f"c3/bias_{N}", (N,), 0.1)
    c0 = synth.normal(f"c3/C_{M}x{N}", (M, N))
    ba, bb, bbias, bc = s.upload(a), s.upload(bt), s.upload(bias), s.upload(c0)
    del a, bt, c0
    mk = lambda i: s.command(abi.OP_MATMUL_F32, id=i, A=ba, B=bb, bias=bbias, C=bc, M=M, K=K, N=N,
                             trans_b=1, alpha=1.0, beta=0.5, epilogue=abi.EPI_GELU_TANH)
    wall, gpu_ns = timed(s, mk, steps, warmup)
    for x in (ba, bb, bbias, bc):
        s.free(x)
    flops = 2.0 * M * K * N
    tf = flops / gpu_ns / 1e3
    return {"M": M, "K": K, "N": N, "kernel_us": gpu_ns / 1e3, "kernel_tflops": tf,
            "arith": "f32 as 3 bf16 products, f32 accumulate",
            "frac_bound": tf / F32_SPLIT_BOUND_TFLOPS,
            "bound": f"{F32_SPLIT_BOUND_TFLOPS:.0f} TFLOP/s of f32 work (bf16 MFMA peak / 3 products)"}


def bench_attention(s: Session, steps: int, warmup: int, high_throughput: bool = False):
    """Config 4's ATTENTION_F32 calls alone: prefill B1 x 32 heads x 2048 causal
    and decode B8 x 32 heads x 1 query over a 4096-entry KV cache (D = 128).
    Prefill's matrix bound: the fp32 MFMA peak for the reference-order kernel
    (its products are fp32 rank-1 MFMA steps), the bf16 peak over three for
    the high-throughput kernel (three bf16 products per f32 product)."""
    bound = F32_SPLIT_BOUND_TFLOPS if high_throughput else F32_PEAK_TFLOPS
    out = {}
    h, d = 32, 128
    for name, b, sq, sk in (("prefill_b1_s2048", 1, 2048, 2048), ("decode_b8_ctx4096", 8, 1, 4096)):
        q = s.upload(synth.normal(f"c4att/{name}/q", (b, h, sq, d)))
        k = s.upload(synth.normal(f"c4att/{name}/k", (b, h, sk, d)))
        v = s.upload(synth.normal(f"c4att/{name}/v", (b, h, sk, d)))
        o = s.alloc(4 * b * h * sq * d)
        mk = lambda i: s.command(abi.OP_ATTENTION_F32, id=i, Q=q, K=k, V=v, O=o, batch=b, heads=h, seq_q=sq,
                                 seq_k=sk, head_dim=d, causal=1)
        wall, gpu_ns = timed(s, mk, steps, warmup)
        for x in (q, k, v, o):
            s.free(x)
        r = {"kernel_us": gpu_ns / 1e3}
        if sq > 1:
            r["tflops_causal"] = 4.0 * b * h * sq * sk * d / 2 / gpu_ns / 1e3
            r["frac_matrix_bound"] = r["tflops_causal"] / bound
        else:
            r["kv_gbs"] = 2.0 * b * h * sk * d * 4 / gpu_ns
        out[name] = r
    return out


def high_throughput_session() -> Session:
    """A session whose device is created with VNPU_CONFIG_HIGH_THROUGHPUT:
    split-bf16 matrix-core attention, within 2e-3 of the reference's
    attention but not of its block (int8 roundings flip downstream)."""
    cfg = abi.Config()
    cfg.abi_version = 1
    cfg.flags = abi.CONFIG_HIGH_THROUGHPUT
    return Session(None, cfg)


# The block on a high-throughput device, end to end against the reference's
# block output (tests/test_block.py, measured on MI355X).
HIGH_THROUGHPUT_BLOCK_NOTE = ("not tolerance-matched: end to end 9.9e-3 (decode) and 1.55e-2 (prefill) "
                              "max-rel > 2e-3; the default device's block is bit-exact")


def bench_copy(s: Session, steps: int):
    """A device-to-device COPY of 256 MiB, `steps` times: a plain copy kernel of
    known size that calibrates the FETCH_SIZE / WRITE_SIZE counters behind
    GEMV_TRAFFIC_BYTES (KiB per dispatch against 262,144 KiB read and written)."""
    n = 256 << 20
    a, b = s.alloc(n), s.alloc(n)
    s.run(abi.OP_MEMSET, dst=a, value=1, bytes=n)
    mk = lambda i: s.command(abi.OP_COPY, id=i, dst=b if i % 2 == 0 else a, src=a if i % 2 == 0 else b, bytes=n,
                             direction=abi.COPY_D2D)
    wall, gpu_ns = timed(s, mk, steps, 0)
    s.free(a)
    s.free(b)
    return {"bytes": n, "copies": steps, "kernel_us": gpu_ns / 1e3, "gbs": 2.0 * n / gpu_ns}


def bench_block(s: Session, steps: int):
    """Config 4: one Llama-style layer, prefill B1 S2048 and decode B8 @ ctx 4096."""
    from vnpu_mi355x.block import LLAMA_4096, Block, weights_f32

    sh = LLAMA_4096
    blk = Block(s, sh, weights_f32(sh, "config4"))
    out = {}
    try:
        blk.prepare(1, 2048)
        blk.set_input(synth.normal("config4/prefill/x", (2048, sh.d_model)))
        ms, wall = gpu_timed(s, lambda: blk.enqueue(True), max(3, steps // 4), 1)
        out["prefill_b1_s2048"] = {"ms": ms, "wall_ms": wall, "tok_s": 2048 / ms * 1e3}
        ctx = 4096
        blk.prepare(8, 1, past=ctx - 1, cache_len=ctx)
        kv = (8, sh.heads, ctx, sh.head_dim)
        blk.set_input(synth.normal("config4/decode/x", (8, sh.d_model)),
                      synth.normal("config4/decode/k_cache", kv), synth.normal("config4/decode/v_cache", kv))
        ms, wall = gpu_timed(s, lambda: blk.enqueue(True), steps, 3)
        out["decode_b8_ctx4096"] = {"ms": ms, "wall_ms": wall, "tok_s": 8 / ms * 1e3}
    finally:
        blk.close()
    return out


def bench_config5(s: Session, steps: int):
    """Config 5: int8 4096^3 with half of the 64x64 weight tiles zero (seeded
    Bernoulli), and the MTP head [4,4096] x [4096,32000] f32 + softmax."""
    M = K = N = 4096
    w = synth.normal("c5/W", (K, N), 0.02)
    keep = synth.bernoulli_mask("c5/tiles", (K // 64, N // 64), 0.5)

    # The dense weights quantized per column once; config 5's mask is passed
    # in at packing (vnpu_pack_weights_i8_masked), which packs the culled
    # tiles as zeros.  The unmasked packing is the dense baseline of the same
    # kernel family; beside config 5's half-zero tiles, a quarter-nonzero mask
    # of the same weights (below 40% nonzero tiles the strip kernel skips the
    # zero ones).
    keep25 = synth.bernoulli_mask("c5/tiles25", (K // 64, N // 64), 0.25)
    bw = s.upload(w)
    del w
    wq, ws = s.alloc(K * N), s.alloc(4 * N)
    s.run(abi.OP_QUANTIZE_I8, X=bw, Y=wq, scales=ws, rows=K, cols=N, axis=abi.QUANT_PER_COLUMN)
    s.free(bw)
    dense_w = s.pack(wq, K, N, scales=ws)
    packed = s.pack(wq, K, N, scales=ws, tile_mask=keep)
    sparse_w = s.pack(wq, K, N, scales=ws, tile_mask=keep25)
    s.free(wq)
    s.free(ws)
    x = synth.normal("c5/A", (M, K))
    bx = s.upload(x)
    a8, sa, c = s.alloc(M * K), s.alloc(4 * M), s.alloc(4 * M * N)
    s.run(abi.OP_QUANTIZE_I8, X=bx, Y=a8, scales=sa, rows=M, cols=K, axis=abi.QUANT_PER_ROW)
    s.free(bx)
    mk = lambda i: s.command(abi.OP_MATMUL_I8, id=i, A=a8, B=packed, scale_a=sa, C=c, M=M, K=K, N=N)
    mkd = lambda i: s.command(abi.OP_MATMUL_I8, id=i, A=a8, B=dense_w, scale_a=sa, C=c, M=M, K=K, N=N)
    # Culled and dense runs alternate (the chip's clock drifts with its
    # temperature over a run); each figure is the median of its rounds.
    mks = lambda i: s.command(abi.OP_MATMUL_I8, id=i, A=a8, B=sparse_w, scale_a=sa, C=c, M=M, K=K, N=N)
    cul, den, spa = [], [], []
    for _ in range(3):
        cul.append(timed(s, mk, max(1, steps // 3), 3)[1])
        den.append(timed(s, mkd, max(1, steps // 3), 3)[1])
        spa.append(timed(s, mks, max(1, steps // 3), 3)[1])
    gpu_ns, dense_ns, sparse_ns = float(np.median(cul)), float(np.median(den)), float(np.median(spa))
    s.release_packed(packed)
    s.release_packed(dense_w)
    s.release_packed(sparse_w)
    for b in (a8, sa, c):
        s.free(b)
    dense = 2.0 * M * K * N
    out = {"cull_i8_4096": {"kernel_us": gpu_ns / 1e3, "zero_tiles": int(keep.size - keep.sum()),
                            "dense_equiv_tops": dense / gpu_ns / 1e3,
                            "useful_tops": dense * keep.mean() / gpu_ns / 1e3,
                            "dense_weights_kernel_us": dense_ns / 1e3, "vs_dense": gpu_ns / dense_ns},
           "cull_i8_4096_quarter_nonzero": {"us": sparse_ns / 1e3, "nonzero_tiles": int(keep25.sum()),
                                            "useful_tops": dense * keep25.mean() / sparse_ns / 1e3,
                                            "vs_dense": sparse_ns / dense_ns}}
    G, H, V = 4, 4096, 32000
    hid = s.upload(synth.normal("c5/hidden", (G, H)))
    wm = synth.normal("c5/mtp_W", (H, V), 0.02)
    copies = [s.upload(wm) for _ in range(2)]   # 2 x 524 MB: past the 256 MB MALL
    del wm
    logits, probs = s.alloc(4 * G * V), s.alloc(4 * G * V)
    state = {"i": 0}

    def step():
        wcur = copies[state["i"] % 2]
        state["i"] += 1
        s.check("submit", s.submit([
            s.command(abi.OP_MTP_HEAD_F32, hidden=hid, W=wcur, logits=logits, gamma=G, hidden_dim=H,
                      vocab=V),
            s.command(abi.OP_SOFTMAX_F32, X=logits, Y=probs, rows=G, cols=V)]))

    ms, _ = gpu_timed(s, step, steps, 3)
    for b in copies + [hid, logits, probs]:
        s.free(b)
    mtp_bytes = 4.0 * (G * H + H * V + 2 * G * V) + 8.0 * G * V
    out["mtp_head_softmax"] = {"us": ms * 1e3, "gbs": mtp_bytes / ms / 1e6,
                               "frac_hbm": mtp_bytes / ms / 1e6 / HBM_PEAK_GBS}
    return out


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(M, K, N, budget_s: float):
    """The reference runtime (built from its own sources) on this host."""
    import oracle  # checker/baseline infrastructure, used only here

    if not os.path.exists(oracle.REF_LIB_PATH):
        return None
    # The reference's default thread count is the host's physical core count
    # (src/core/runtime.cpp:862-866): read it from the reference itself, then
    # run at that count unless it exceeds this process's CPU share (the GPU
    # box gives one GPU's job 16 CPUs).
    cfg = abi.Config()
    cfg.abi_version = 1
    with Session(oracle.REF_LIB_PATH, cfg) as probe:
        pinfo = probe.info()
        ref_default = int(pinfo.num_threads)
        physical = int(pinfo.physical_cores)
    share = min(16, len(os.sched_getaffinity(0)))
    threads = min(ref_default, share)
    cfg.num_threads = threads
    host = {"cpu_model": cpu_model(), "nproc": os.cpu_count(), "affinity": len(os.sched_getaffinity(0)),
            "physical_cores": physical, "reference_default_threads": ref_default}
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
        capped = "" if threads == ref_default else (
            f" (the reference default is {ref_default} threads, one per physical core; capped at "
            f"this job's CPU share of {share})")
        return {"value": i8_bytes(M, K, N) / med / 1e9, "unit": "GB/s",
                "cores": int(info.num_threads), "kind": "reference",
                "sample": f"MATMUL_I8 M={M} K={K} N={N} decode GEMV, {len(times)} calls "
                          f"(median {med * 1e3:.3f} ms, best {min(times) * 1e3:.3f} ms), "
                          f"reference AVX2 path, {info.num_threads} threads{capped}",
                "host": host}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extras", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=15.0)
    ap.add_argument("--only", choices=["gemm_i8", "gemm_f32", "attention", "block", "config1", "config5",
                                       "copy"],
                    default=None, help="run one extra workload alone (for profiling)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build benchmarks one GPU only: how the path shards across "
                                   "GPUs is a design, not a measured run", "n_gpus": args.gpus}))
        sys.exit(2)

    M, K, N = 1, 4096, 32000
    s = Session()
    log("device", s.info().backend.decode())
    if args.only:
        if args.only == "gemm_i8":
            for n in (4096, 14336):
                log("gemm_i8", bench_gemm_i8(s, 2048, 4096, n, args.steps, args.warmup))
        elif args.only == "gemm_f32":
            for n in (4096, 14336):
                log("gemm_f32", bench_gemm_f32(s, 2048, 4096, n, args.steps, args.warmup))
        elif args.only == "copy":
            log("copy", bench_copy(s, 5))
        elif args.only == "attention":
            log("attention", bench_attention(s, args.steps, args.warmup))
            x = high_throughput_session()
            log("attention high-throughput", bench_attention(x, args.steps, args.warmup, True))
            x.close()
        elif args.only == "block":
            log("block", bench_block(s, args.steps))
            x = high_throughput_session()
            log("block high-throughput", bench_block(x, args.steps))
            x.close()
        elif args.only == "config1":
            log("config1", bench_config1(s, args.steps))
        else:
            log("config5", bench_config5(s, args.steps))
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
        wq = ws = None
        extras["config1"] = rounded(bench_config1(s, 50), 3)
        log("config1", extras["config1"])
        extras["config3_gemm_f32"] = []
        for n in (4096, 14336):
            extras["config3_gemm_f32"].append(rounded(bench_gemm_f32(s, 2048, 4096, n, 5, 2)))
            log("gemm_f32", extras["config3_gemm_f32"][-1])
        # The default device: attention in the reference's order, so the
        # block is bit-exact with the reference's (the north-star parity bar).
        extras["config4_attention"] = {k: rounded(v, 3) for k, v in bench_attention(s, 20, 3).items()}
        log("attention", extras["config4_attention"])
        extras["config4_block"] = {k: rounded(v, 3) for k, v in bench_block(s, 20).items()}
        extras["config4_block"]["parity"] = "bit-exact with the reference's block output"
        log("block", extras["config4_block"])
        x = high_throughput_session()
        extras["config4_attention_high_throughput"] = {k: rounded(v, 3)
                                                       for k, v in bench_attention(x, 20, 3, True).items()}
        log("attention high-throughput", extras["config4_attention_high_throughput"])
        extras["config4_block_high_throughput"] = {k: rounded(v, 3) for k, v in bench_block(x, 20).items()}
        extras["config4_block_high_throughput"]["parity"] = HIGH_THROUGHPUT_BLOCK_NOTE
        log("block high-throughput", extras["config4_block_high_throughput"])
        x.close()
        extras["config5"] = {k: rounded(v, 3) for k, v in bench_config5(s, 10).items()}
        log("config5", extras["config5"])
    if wq is not None:
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
                     "traffic": GEMV_TRAFFIC_BYTES, "kernel": "gemv_i8_kernel", "kernel_us": round(head["kernel_us"], 3),
                     "algorithmic_bytes": b,
                     "traffic_source": "rocprofv3 FETCH_SIZE + WRITE_SIZE passes of this command, scaled by a copy "
                                       "kernel of known size: profiles/gemv_i8_m1_k4096_n32000_traffic.md"},
        "cpu_baseline": cpu,
        "extras": extras,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
