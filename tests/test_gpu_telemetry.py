"""GPU telemetry through the C ABI: device status counters, the trace summary,
the text and Chrome-JSON traces, MMIO registers and interrupts, autotune.

Semantics follow the reference runtime: status counters and the per-op byte /
flop accounting of src/core/scheduler.cpp (execute_*), the trace layout of
src/core/runtime.cpp:530-580, the register file and doorbell / batch-done
interrupts of src/core/runtime.cpp:1102-1138.  Where the reference build
(oracle/_ref, CPU) is present, the accounting is compared with it command by
command.
"""
import ctypes as C
import json

import numpy as np
import pytest

from vnpu_mi355x import abi

pytestmark = pytest.mark.gpu
RNG = np.random.default_rng(20261202)


def _reset(s):
    assert s.lib.vnpu_device_reset(s.dev) == abi.OK


def _commands(s):
    """One command per hot-path opcode on fresh buffers of session s.
    Returns (commands, keep-alive list)."""
    M, K, N = 48, 192, 80
    keep = []

    def up(a):
        b = s.upload(np.ascontiguousarray(a))
        keep.append(b)
        return b

    def out(nbytes):
        b = s.alloc(nbytes)
        keep.append(b)
        return b

    a8 = RNG.integers(-128, 128, (M, K)).astype(np.int8)
    b8 = RNG.integers(-128, 128, (K, N)).astype(np.int8)
    w = s.pack(b8, K, N, scales=(RNG.random(N).astype(np.float32) + 0.5) / 127)
    keep.append(("packed", w))
    af, bf = RNG.standard_normal((M, K)).astype(np.float32), RNG.standard_normal((K, N)).astype(np.float32)
    x = RNG.standard_normal((M, K)).astype(np.float32)
    q = RNG.standard_normal((1, 2, 24, 32)).astype(np.float32)
    cmds = [
        s.command(abi.OP_MATMUL_I8, id=1, A=up(a8), B=w, scale_a=up(np.full(M, 0.01, np.float32)).ptr,
                  C=out(4 * M * N), M=M, K=K, N=N),
        s.command(abi.OP_MATMUL_F32, id=2, A=up(af), B=up(bf), bias=up(np.ones(N, np.float32)).ptr,
                  C=up(np.ones((M, N), np.float32)), M=M, K=K, N=N, alpha=1.0, beta=0.5, epilogue=1),
        s.command(abi.OP_RMSNORM_F32, id=3, X=up(x), W=up(np.ones(K, np.float32)).ptr, Y=out(4 * M * K),
                  rows=M, cols=K, eps=1e-5),
        s.command(abi.OP_SOFTMAX_F32, id=4, X=up(x), Y=out(4 * M * K), rows=M, cols=K),
        s.command(abi.OP_SWIGLU_F32, id=5, gate=up(x), up=up(x), Y=out(4 * M * K), count=M * K),
        s.command(abi.OP_ADD_F32, id=6, A=up(x), B=up(x), Y=out(4 * M * K), count=M * K),
        s.command(abi.OP_QUANTIZE_I8, id=7, X=up(x), Y=out(M * K), scales=out(4 * M), rows=M, cols=K,
                  axis=abi.QUANT_PER_ROW),
        s.command(abi.OP_ROPE_F32, id=8, Q=up(q), K=up(q), batch=1, heads=2, q_seq=24, k_seq=24,
                  head_dim=32),
        s.command(abi.OP_ATTENTION_F32, id=9, Q=up(q), K=up(q), V=up(q), O=out(q.nbytes), batch=1,
                  heads=2, seq_q=24, seq_k=24, head_dim=32, causal=1),
    ]
    return cmds, keep


def _release(s, keep):
    for b in keep:
        if isinstance(b, tuple):
            s.release_packed(b[1])
        else:
            s.free(b)


def _status_after(s, cmds):
    _reset(s)
    assert s.submit(cmds) == abi.OK
    assert s.sync() == abi.OK
    return s.status()


def test_status_counters_follow_the_reference_accounting(gpu):
    M, K, N = 64, 256, 192
    A = RNG.integers(-128, 128, (M, K)).astype(np.int8)
    B = RNG.integers(-128, 128, (K, N)).astype(np.int8)
    w = gpu.pack(B, K, N)
    ba, bsa, bc = gpu.upload(A), gpu.upload(np.ones(M, np.float32)), gpu.alloc(4 * M * N)
    cmds = [gpu.command(abi.OP_MATMUL_I8, A=ba, B=w, scale_a=bsa.ptr, C=bc, M=M, K=K, N=N)
            for _ in range(3)]
    st = _status_after(gpu, cmds)
    assert st.commands_submitted == 3 and st.commands_completed == 3
    # execute_matmul_i8 (scheduler.cpp:420-426): MK + KN + 4(N + M) read, 4MN written
    assert st.flops == 3 * 2 * M * K * N
    assert st.bytes_read == 3 * (M * K + K * N + 4 * (N + M))
    assert st.bytes_written == 3 * 4 * M * N
    assert st.kernel_time_ns > 0 and st.dispatch_time_ns > 0
    assert st.busy == 0 and st.error == 0 and st.last_opcode == abi.OP_MATMUL_I8
    # the GPU time of the three launches is a plausible fraction of a second
    assert st.kernel_time_ns < 10**9
    for b in (ba, bsa, bc):
        gpu.free(b)
    gpu.release_packed(w)


def test_accounting_matches_the_reference_build(gpu, ref):
    """Same commands on the reference runtime (CPU, built from its sources)
    and on this backend: identical byte and flop counts per command."""
    for i in range(9):
        counts = []
        for s in (ref, gpu):
            cmds, keep = _commands(s)
            st = _status_after(s, [cmds[i]])
            counts.append((st.bytes_read, st.bytes_written, st.flops, st.commands_completed))
            _release(s, keep)
        assert counts[0] == counts[1], (int(cmds[i].opcode), counts)


def test_trace_summary_chrome_and_text(gpu, tmp_path):
    cmds, keep = _commands(gpu)
    lib = gpu.lib
    _reset(gpu)
    assert lib.vnpu_trace_enable(gpu.dev, 1) == abi.OK
    assert gpu.submit(cmds) == abi.OK and gpu.sync() == abi.OK
    st = gpu.status()
    summ = abi.TraceSummary()
    assert lib.vnpu_trace_get_summary(gpu.dev, C.byref(summ)) == abi.OK
    assert summ.events == len(cmds)
    assert summ.flops == st.flops and summ.bytes_read == st.bytes_read
    assert summ.bytes_written == st.bytes_written
    assert summ.total_time_ns > 0 and summ.compute_time_ns == summ.total_time_ns
    assert summ.hot_time_ns > 0 and summ.hot_opcode in (abi.OP_MATMUL_F32, abi.OP_MATMUL_I8,
                                                         abi.OP_ATTENTION_F32, abi.OP_QUANTIZE_I8,
                                                         abi.OP_RMSNORM_F32, abi.OP_SOFTMAX_F32,
                                                         abi.OP_SWIGLU_F32, abi.OP_ADD_F32,
                                                         abi.OP_ROPE_F32)
    assert summ.achieved_gflops > 0 and summ.achieved_gbytes_s > 0

    path = tmp_path / "trace.json"
    assert lib.vnpu_trace_write_chrome(gpu.dev, str(path).encode()) == abi.OK
    doc = json.loads(path.read_text())
    assert doc["displayTimeUnit"] == "ns" and "version" in doc["otherData"]
    ev = [e for e in doc["traceEvents"] if e["ph"] == "X"]
    names = ["MATMUL_I8#1", "MATMUL_F32#2", "RMSNORM_F32#3", "SOFTMAX_F32#4", "SWIGLU_F32#5",
             "ADD_F32#6", "QUANTIZE_I8#7", "ROPE_F32#8", "ATTENTION_F32#9"]
    assert [e["name"] for e in ev] == names
    assert all(e["cat"] == "compute" and e["dur"] > 0 for e in ev)
    assert ev[0]["ts"] == 0.0
    # one stream: GPU start times follow submission order and do not overlap
    for e0, e1 in zip(ev, ev[1:]):
        assert e1["ts"] >= e0["ts"] + e0["dur"] - 1e-3
    assert sum(e["args"]["flops"] for e in ev) == st.flops
    assert [e["args"]["op"] for e in ev] == [n.split("#")[0] for n in names]

    text = tmp_path / "trace.txt"
    assert lib.vnpu_trace_dump(gpu.dev, str(text).encode()) == abi.OK
    assert f"events {len(cmds)}" in text.read_text()

    assert lib.vnpu_trace_enable(gpu.dev, 0) == abi.OK
    lib.vnpu_trace_reset(gpu.dev)
    assert lib.vnpu_trace_get_summary(gpu.dev, C.byref(summ)) == abi.OK and summ.events == 0
    _release(gpu, keep)


def test_mmio_registers_and_interrupts(gpu):
    lib = gpu.lib
    dev = gpu.dev
    lib.vnpu_mmio_read32.restype = C.c_uint32
    lib.vnpu_mmio_write32.argtypes = [C.c_void_p, C.c_uint32, C.c_uint32]
    _reset(gpu)
    fired = []
    CB = C.CFUNCTYPE(None, C.c_void_p, C.c_uint32, C.c_void_p)
    cb = CB(lambda d, irq, user: fired.append(irq))
    lib.vnpu_device_set_interrupt_callback(dev, cb, None)
    try:
        assert lib.vnpu_mmio_read32(dev, 0x00) == 0x56504E55          # ID
        assert lib.vnpu_mmio_read32(dev, 0x0c) & 1                    # STATUS: ready
        lib.vnpu_mmio_write32(dev, 0x20, 0xffffffff)                  # clear IRQ_STATUS
        assert lib.vnpu_mmio_read32(dev, 0x20) == 0
        lib.vnpu_mmio_write32(dev, 0x1c, 1)                           # doorbell -> IRQ0
        assert lib.vnpu_mmio_read32(dev, 0x20) & 1
        nops = [gpu.command(abi.OP_NOP) for _ in range(5)]
        assert gpu.submit(nops) == abi.OK and gpu.sync() == abi.OK    # batch done -> IRQ1
        assert lib.vnpu_mmio_read32(dev, 0x20) & 2
        assert lib.vnpu_mmio_read32(dev, 0x18) == 5                   # CMD_TAIL = submitted
        assert lib.vnpu_mmio_read32(dev, 0x14) == 5                   # CMD_HEAD = completed
        # the callback gets the IRQ_STATUS bits: doorbell (bit 0), batch done (bit 1)
        assert any(v & 1 for v in fired) and any(v & 2 for v in fired)
        lib.vnpu_mmio_write32(dev, 0x08, 2)                           # CONTROL bit 1: reset
        assert gpu.status().commands_submitted == 0
        assert lib.vnpu_mmio_read32(dev, 0x20) == 0
        assert lib.vnpu_mmio_read32(dev, 0x40) == 0xffffffff          # past the register file
    finally:
        lib.vnpu_device_set_interrupt_callback(dev, None, None)


def test_set_tiles_and_autotune(gpu):
    lib = gpu.lib
    info0 = gpu.info()
    assert lib.vnpu_device_set_tiles(gpu.dev, 64, 32, 96) == abi.OK
    info = gpu.info()
    assert (info.tile_m, info.tile_k, info.tile_n) == (64, 32, 96)
    try:
        for dtype, shape in ((3, (512, 1024, 768)), (0, (256, 2048, 256))):  # VNPU_DTYPE_I8, _F32
            res = abi.TuneResult()
            assert lib.vnpu_autotune_gemm(gpu.dev, *shape, 3, dtype, C.byref(res)) == abi.OK
            assert res.best_ms > 0 and res.gflops > 0 and res.unit == abi.UNIT_GPU
            assert res.best_ms <= res.baseline_ms and res.speedup >= 1.0
            assert res.bytes_written == shape[0] * shape[2] * 4
            # the winner is left on the device
            info = gpu.info()
            assert (info.tile_m, info.tile_k, info.tile_n) == (res.tile_m, res.tile_k, res.tile_n)
    finally:
        assert lib.vnpu_device_set_tiles(gpu.dev, info0.tile_m, info0.tile_k, info0.tile_n) == abi.OK


@pytest.mark.parametrize("tiles", [(256, 128, 256), (256, 128, 192), (256, 128, 128), (256, 64, 128),
                                   (128, 64, 128), (128, 128, 64)])
def test_forced_int8_kernels_are_bit_exact(gpu, tiles):
    """Every int8 prefill kernel a tile triple can select gives the oracle's
    bits (the last triple is the automatic choice)."""
    import oracle
    M, K, N = 512, 384, 520
    A = RNG.integers(-128, 128, (M, K)).astype(np.int8)
    B = RNG.integers(-128, 128, (K, N)).astype(np.int8)
    sa = (RNG.random(M).astype(np.float32) + 0.5) / 127
    sb = (RNG.random(N).astype(np.float32) + 0.5) / 127
    w = gpu.pack(B, K, N, scales=sb)
    info0 = gpu.info()
    assert gpu.lib.vnpu_device_set_tiles(gpu.dev, *tiles) == abi.OK
    try:
        ba, bsa, bc = gpu.upload(A), gpu.upload(sa), gpu.alloc(4 * M * N)
        gpu.run(abi.OP_MATMUL_I8, A=ba, B=w, scale_a=bsa.ptr, C=bc, M=M, K=K, N=N)
        got = gpu.download(bc, np.float32, (M, N))
        for b in (ba, bsa, bc):
            gpu.free(b)
    finally:
        gpu.lib.vnpu_device_set_tiles(gpu.dev, info0.tile_m, info0.tile_k, info0.tile_n)
        gpu.release_packed(w)
    want = oracle.matmul_i8(A, B, sa, sb)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("depth", [64, 256, 1024])
def test_forced_f32_split_depths(gpu, depth):
    import oracle
    M, K, N = 256, 1024, 200
    A = RNG.standard_normal((M, K)).astype(np.float32)
    B = RNG.standard_normal((K, N)).astype(np.float32)
    bias = RNG.standard_normal(N).astype(np.float32)
    Cin = RNG.standard_normal((M, N)).astype(np.float32)
    info0 = gpu.info()
    assert gpu.lib.vnpu_device_set_tiles(gpu.dev, 128, depth, 128) == abi.OK
    try:
        ba, bb, bbias, bc = gpu.upload(A), gpu.upload(B), gpu.upload(bias), gpu.upload(Cin)
        gpu.run(abi.OP_MATMUL_F32, A=ba, B=bb, bias=bbias.ptr, C=bc, M=M, K=K, N=N, alpha=1.0,
                beta=0.5, epilogue=3)
        got = gpu.download(bc, np.float32, (M, N))
        for b in (ba, bb, bbias, bc):
            gpu.free(b)
    finally:
        gpu.lib.vnpu_device_set_tiles(gpu.dev, info0.tile_m, info0.tile_k, info0.tile_n)
    want = oracle.matmul_f32(A, B, Cin, bias, M, K, N, 0, 0, 1.0, 0.5, 3, acc64=True)
    assert oracle.rel_error(got, want) <= 1e-4


def test_autotune_leaves_the_other_dtype():
    """vnpu_autotune_gemm writes back only the tuned dtype's kernel choice.
    After an int8 tune (whatever tile triple it leaves on the device, e.g.
    128 x 64 x 128 for the generic int8 kernel) MATMUL_F32 still runs its
    automatic split-bf16 kernel: the same bits as on an untuned device (the
    fp32 split-K kernel a 128 x 64 x 128 f32 choice would force gives other
    bits) in about the same time; after an f32 tune the int8 GEMM keeps its
    time.  (vnpu_device_set_tiles, as in the reference, sets both.)"""
    import time
    from vnpu_mi355x import Session
    import gpu_ops as g
    s = Session()
    try:
        Mf, Kf, Nf = 2048, 512, 4096
        A = RNG.standard_normal((Mf, Kf)).astype(np.float32)
        B = RNG.standard_normal((Kf, Nf)).astype(np.float32)
        ba, bb, bc = s.upload(A), s.upload(B), s.alloc(4 * Mf * Nf)
        Mi, Ki, Ni = 2048, 4096, 4096
        A8 = RNG.integers(-128, 128, (Mi, Ki)).astype(np.int8)
        w = s.pack(RNG.integers(-128, 128, (Ki, Ni)).astype(np.int8), Ki, Ni)
        b8, bi = s.upload(A8), s.alloc(4 * Mi * Ni)
        f32_cmd = s.command(abi.OP_MATMUL_F32, A=ba, B=bb, C=bc, M=Mf, K=Kf, N=Nf, alpha=1.0)
        i8_cmd = s.command(abi.OP_MATMUL_I8, A=b8, B=w, C=bi, M=Mi, K=Ki, N=Ni)

        def timed(cmd, n=20):
            s.check("submit", s.submit([cmd] * 3))
            s.check("sync", s.sync())
            t0 = time.perf_counter()
            s.check("submit", s.submit([cmd] * n))
            s.check("sync", s.sync())
            return (time.perf_counter() - t0) / n

        t_f32, t_i8 = timed(f32_cmd), timed(i8_cmd)
        r0 = s.download(bc, np.float32, (Mf, Nf))
        res = abi.TuneResult()
        assert s.lib.vnpu_autotune_gemm(s.dev, 512, 1024, 768, 3, 3, C.byref(res)) == abi.OK   # int8
        s.check("submit", s.submit([f32_cmd]))
        s.check("sync", s.sync())
        r1 = s.download(bc, np.float32, (Mf, Nf))
        assert np.array_equal(r0.view(np.uint32), r1.view(np.uint32)), (res.tile_m, res.tile_k, res.tile_n)
        assert timed(f32_cmd) < 1.5 * t_f32
        assert s.lib.vnpu_autotune_gemm(s.dev, 256, 2048, 256, 3, 0, C.byref(res)) == abi.OK    # f32
        assert timed(i8_cmd) < 1.5 * t_i8
        s.release_packed(w)
    finally:
        s.close()
