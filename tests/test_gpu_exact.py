"""Bit-exact parity with the reference's AVX2 build for the block's f32 ops.

The oracle's *_avx2 restatements are pinned bit for bit against the
reference build in tests/test_oracle_vs_reference.py; here the GPU is held to
the same bits:
  * RMSNORM (every kernel: registers, chunked LDS, tails), SWIGLU, GELU, ADD
    and RoPE, always;
  * the row chains (ADD -> RMSNORM -> QUANTIZE_I8, SWIGLU -> QUANTIZE_I8);
  * ATTENTION_F32 on a device created with VNPU_CONFIG_REFERENCE_ORDER
    (decode and prefill tiles, other head sizes, masks, -inf, causal).
"""
import ctypes as C

import numpy as np
import pytest

import block_oracle
import gpu_ops as g
import oracle
from vnpu_mi355x import abi

pytestmark = pytest.mark.gpu
RNG = np.random.default_rng(777)


def bits(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


@pytest.mark.parametrize("rows,cols", [(2048, 4096), (8, 11008), (3, 12288), (3, 4099), (2, 20000), (5, 33),
                                       (4, 4100), (1, 7), (256, 7), (256, 13), (128, 12), (64, 4103),
                                       (3, 20005), (2, 12295)])
def test_rmsnorm_bit_exact(gpu, rows, cols):
    X = (RNG.standard_normal((rows, cols)) * 2).astype(np.float32)
    W = (1.0 + 0.1 * RNG.standard_normal(cols)).astype(np.float32)
    assert bits(g.unary_rows(gpu, abi.OP_RMSNORM_F32, X, W=W, eps=1e-5), oracle.rmsnorm_avx2(X, W, 1e-5))
    assert bits(g.unary_rows(gpu, abi.OP_RMSNORM_F32, X, eps=0.0), oracle.rmsnorm_avx2(X, None, 1e-5))


@pytest.mark.parametrize("n", [1, 7, 1001, 4096 * 8 + 4, 4103, 2048 * 11008])
def test_elementwise_bit_exact(gpu, n):
    """Vector kernel (n % 4 == 0) and scalar kernel, with the reference's
    scalar tail (last n % 8 elements) and exp's clamp edges in both parts."""
    a = (RNG.standard_normal(n) * 4).astype(np.float32)
    b = RNG.standard_normal(n).astype(np.float32)
    edges = np.array([90.0, -95.0, 0.0, -0.0, -80.5, -88.0], np.float32)   # outside exp's clamp, zeros
    a[: min(n, 3)] = edges[: min(n, 3)]
    a[-min(n, 3):] = edges[-min(n, 3):]
    for al, be in ((0.0, 0.0), (0.75, 0.25), (-1.5, 2.0)):
        assert bits(g.elementwise(gpu, abi.OP_SWIGLU_F32, a, b, alpha=al), oracle.swiglu_avx2(a, b, al or 1.0))
        assert bits(g.elementwise(gpu, abi.OP_ADD_F32, a, b, al, be), oracle.add_avx2(a, b, al, be))
        assert bits(g.elementwise(gpu, abi.OP_MUL_F32, a, b, al, be), oracle.mul_avx2(a, b, al or 1.0, be))
    assert bits(g.elementwise(gpu, abi.OP_GELU_F32, a), oracle.gelu_avx2(a))


@pytest.fixture(scope="module")
def gpu4():
    """A device created with num_threads = 4: the reference's elementwise
    ranges (max(4096, n / (4 * num_threads)) elements) follow the unit count."""
    from vnpu_mi355x import Session
    cfg = abi.Config()
    cfg.abi_version = 1
    cfg.num_threads = 4
    s = Session(None, cfg)
    yield s
    s.close()


@pytest.mark.parametrize("dev_name,n", [("gpu4", 70001), ("gpu4", 100004), ("gpu", 5_000_004),
                                        ("gpu", 5_000_003)])
def test_elementwise_reference_ranges(request, dev_name, n):
    """Above 16384 * num_threads elements the reference runs ranges whose
    length is not a multiple of 8, each ending in its own scalar tail: the
    GPU gives the same bits as the oracle split the same way (vector and
    scalar kernels), and not those of one range."""
    dev = request.getfixturevalue(dev_name)
    threads = dev.info().num_threads
    grain = oracle.ew_grain(n, threads)
    assert grain % 8 != 0 and n > grain, (threads, grain)
    a = (RNG.standard_normal(n) * 4).astype(np.float32)
    b = RNG.standard_normal(n).astype(np.float32)
    for end in list(range(grain, n, grain)) + [n]:
        a[end - 3:end] = (-90.0, -85.0, -81.0)     # exp's clamp edges in each range's tail
    for al, be in ((0.0, 0.0), (-1.5, 2.0)):
        sw = g.elementwise(dev, abi.OP_SWIGLU_F32, a, b, alpha=al)
        mu = g.elementwise(dev, abi.OP_MUL_F32, a, b, al, be)
        assert bits(sw, oracle.swiglu_avx2(a, b, al or 1.0, num_threads=threads))
        assert bits(mu, oracle.mul_avx2(a, b, al or 1.0, be, num_threads=threads))
        assert not bits(sw, oracle.swiglu_avx2(a, b, al or 1.0))
        assert bits(g.elementwise(dev, abi.OP_ADD_F32, a, b, al, be), oracle.add_avx2(a, b, al, be))
    assert bits(g.elementwise(dev, abi.OP_GELU_F32, a), oracle.gelu_avx2(a))


@pytest.mark.parametrize("interleaved", [0, 1])
@pytest.mark.parametrize("shape_q,shape_k,offset", [((1, 32, 2048, 128), (1, 32, 2048, 128), 0),
                                                    ((8, 32, 1, 128), (8, 32, 1, 128), 4095),
                                                    ((2, 3, 40, 64), (2, 3, 24, 64), 100),
                                                    ((1, 2, 10, 6), (1, 2, 10, 6), 70000)])
def test_rope_bit_exact(gpu, interleaved, shape_q, shape_k, offset):
    """Offset positions below 65536 come from the host table (the reference's
    libm); the last case, beyond it, is computed on the GPU (tolerance)."""
    Q = RNG.standard_normal(shape_q).astype(np.float32)
    K = RNG.standard_normal(shape_k).astype(np.float32)
    gq, gk = g.rope(gpu, Q, K, position_offset=offset, interleaved=interleaved)
    oq, ok = oracle.rope(Q, K, position_offset=offset, interleaved=interleaved)
    if offset + max(shape_q[2], shape_k[2]) <= 65536:
        assert bits(gq, oq) and bits(gk, ok)
    else:
        assert oracle.rel_error(gq, oq) <= 1e-4 and oracle.rel_error(gk, ok) <= 1e-4


@pytest.mark.parametrize("interleaved", [0, 1])
def test_rope_q_and_k_same_buffer(gpu, interleaved):
    """Q and K pointing at one buffer: the rows are rotated twice, K's pass
    starting from Q's result, as the reference's two passes over the same
    memory do."""
    X = RNG.standard_normal((2, 3, 5, 128)).astype(np.float32)
    bx = gpu.upload(X)
    b, h, t, d = X.shape
    gpu.run(abi.OP_ROPE_F32, Q=bx, K=bx, batch=b, heads=h, q_seq=t, k_seq=t, head_dim=d, position_offset=11,
            interleaved=interleaved)
    got = gpu.download(bx, np.float32, X.shape)
    gpu.free(bx)
    once, _ = oracle.rope(X, None, position_offset=11, interleaved=interleaved)
    twice, _ = oracle.rope(once, None, position_offset=11, interleaved=interleaved)
    assert np.array_equal(got.view(np.uint32), twice.view(np.uint32))


def test_rope_host_positions_bit_exact(gpu):
    """A host position array is scanned for the table rows it needs."""
    Q = RNG.standard_normal((1, 2, 6, 32)).astype(np.float32)
    pos = np.array([0, 5000, 2, 0, 9, 1], np.int32)
    bq = gpu.upload(Q)
    gpu.run(abi.OP_ROPE_F32, Q=bq.ptr, K=None, positions=pos.ctypes.data, batch=1, heads=2, q_seq=6, k_seq=0,
            head_dim=32, position_offset=0, interleaved=0, theta_base=0.0, scaling=0.0)
    got = gpu.download(bq, np.float32, Q.shape)
    gpu.free(bq)
    want, _ = oracle.rope(Q, None, positions=pos)
    assert bits(got, want)


def test_row_chain_add_norm_quant_bit_exact(gpu):
    """The block's ADD -> RMSNORM -> QUANTIZE_I8 batch (one row kernel) against
    the oracle's AVX2-order ops."""
    rows, cols = 300, 4096
    x = RNG.standard_normal((rows, cols)).astype(np.float32)
    y = RNG.standard_normal((rows, cols)).astype(np.float32)
    w = (1.0 + 0.1 * RNG.standard_normal(cols)).astype(np.float32)
    bx, by, bw = gpu.upload(x), gpu.upload(y), gpu.upload(w)
    bn, bq, bs = gpu.alloc(x.nbytes), gpu.alloc(rows * cols), gpu.alloc(4 * rows)
    gpu.check("submit", gpu.submit([
        gpu.command(abi.OP_ADD_F32, A=bx, B=by, Y=bx, count=rows * cols, alpha=1.0, beta=1.0),
        gpu.command(abi.OP_RMSNORM_F32, X=bx, W=bw, Y=bn, rows=rows, cols=cols, eps=1e-5),
        gpu.command(abi.OP_QUANTIZE_I8, X=bn, Y=bq, scales=bs, rows=rows, cols=cols, axis=0)]))
    gpu.check("sync", gpu.sync())
    s1 = gpu.download(bx, np.float32, x.shape)
    n1 = gpu.download(bn, np.float32, x.shape)
    q1 = gpu.download(bq, np.int8, x.shape)
    sc = gpu.download(bs, np.float32, (rows,))
    for b in (bx, by, bw, bn, bq, bs):
        gpu.free(b)
    ws = oracle.add(x, y, 1.0, 1.0)
    wn = oracle.rmsnorm_avx2(ws, w, 1e-5)
    wq, wsc = oracle.quantize(wn, 0)
    assert bits(s1, ws) and bits(n1, wn) and np.array_equal(q1, wq) and bits(sc, wsc)


@pytest.mark.parametrize("b,h,sq,sk,d,causal,mask", [
    (8, 32, 1, 4096, 128, 1, None),        # config-4 decode
    (1, 4, 256, 256, 128, 1, None),        # prefill tiles
    (1, 2, 300, 700, 64, 1, "inf"), (2, 2, 3, 500, 128, 0, "normal"), (1, 2, 17, 40, 64, 1, "row"),
    (1, 2, 37, 70, 20, 0, "normal"),       # other head sizes: the row-wise kernel
    (1, 2, 9, 40, 13, 1, None), (2, 2, 3, 50, 23, 0, None), (1, 2, 6, 30, 6, 1, None),
    (1, 1, 5, 64, 96, 1, None), (2, 3, 1, 1, 128, 0, None)])
def test_attention_reference_order_bit_exact(exact_gpu, b, h, sq, sk, d, causal, mask):
    Q = RNG.standard_normal((b, h, sq, d)).astype(np.float32)
    K = RNG.standard_normal((b, h, sk, d)).astype(np.float32)
    V = RNG.standard_normal((b, h, sk, d)).astype(np.float32)
    M = None
    if mask:
        M = RNG.standard_normal((b, h, sq, sk)).astype(np.float32)
        if mask == "inf":
            M[..., : sk // 3] = -np.inf
        if mask == "row":
            M[0, 0, 3, :] = -np.inf
    got = g.attention(exact_gpu, Q, K, V, M, causal)
    # per (batch, head) on threads: the same C restatement as one call
    want = block_oracle.attention_threaded(Q, K, V, causal, mask=M, avx2=True)
    assert bits(got, want)


def test_attention_reference_order_noalloc(exact_gpu):
    """The allocation-free entry point takes the reference-order kernels on
    such a device (no scratch needed)."""
    b, h, sq, sk, d = 2, 4, 1, 900, 128
    Q = RNG.standard_normal((b, h, sq, d)).astype(np.float32)
    K = RNG.standard_normal((b, h, sk, d)).astype(np.float32)
    V = RNG.standard_normal((b, h, sk, d)).astype(np.float32)
    s = exact_gpu
    bq, bk, bv, bo = s.upload(Q), s.upload(K), s.upload(V), s.alloc(Q.nbytes)
    a = abi.AttentionArgs()
    a.Q, a.K, a.V, a.O, a.mask = bq.ptr, bk.ptr, bv.ptr, bo.ptr, None
    a.batch, a.heads, a.seq_q, a.seq_k, a.head_dim, a.causal, a.scale = b, h, sq, sk, d, 1, 0.0
    assert s.lib.vnpu_attention_f32_noalloc(s.stream, C.byref(a)) == abi.OK
    assert s.sync() == abi.OK
    got = s.download(bo, np.float32, Q.shape)
    for x in (bq, bk, bv, bo):
        s.free(x)
    assert bits(got, oracle.attention_avx2(Q, K, V, None, 1))


def bits_or_nan(a, b):
    """Bit for bit, except that a NaN matches a NaN of any payload (x86's
    default NaN is 0xffc00000, the GPU's 0x7fc00000)."""
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    na, nb = np.isnan(a), np.isnan(b)
    return np.array_equal(na, nb) and np.array_equal(a[~na].view(np.uint32), b[~nb].view(np.uint32))


@pytest.mark.parametrize("b,h,sq,sk,d,causal,mask", [
    (2, 3, 200, 130, 128, 1, None),        # seq_k < seq_q, causal
    (1, 2, 129, 1000, 128, 0, "normal"),   # ragged row tiles, additive mask
    (1, 2, 100, 300, 64, 1, None)])        # seq_k > seq_q, causal offset
def test_attention_reference_order_prefill_shapes(exact_gpu, b, h, sq, sk, d, causal, mask):
    """The matrix-core prefill tiles (32 rows per wave, 128 per workgroup,
    64-key blocks) at ragged sizes and both causal offsets."""
    Q = RNG.standard_normal((b, h, sq, d)).astype(np.float32)
    K = RNG.standard_normal((b, h, sk, d)).astype(np.float32)
    V = RNG.standard_normal((b, h, sk, d)).astype(np.float32)
    M = RNG.standard_normal((b, h, sq, sk)).astype(np.float32) if mask else None
    got = g.attention(exact_gpu, Q, K, V, M, causal)
    assert bits(got, block_oracle.attention_threaded(Q, K, V, causal, mask=M, avx2=True))


def test_attention_reference_order_nonfinite_v_masked(exact_gpu):
    """Infinite and NaN values of V at keys some rows never weigh: the matrix
    core would turn v * 0 into NaN where the reference skips the key, so
    those waves take the exact vector-ALU recompute; rows that see the key
    are inf/NaN in both."""
    b, h, s, d = 1, 2, 70, 128
    Q = RNG.standard_normal((b, h, s, d)).astype(np.float32)
    K = RNG.standard_normal((b, h, s, d)).astype(np.float32)
    V = RNG.standard_normal((b, h, s, d)).astype(np.float32)
    V[0, 0, 50, :] = np.inf
    V[0, 1, 60, 3] = -np.inf
    V[0, 1, 20, 7] = np.nan
    got = g.attention(exact_gpu, Q, K, V, None, 1)
    want = block_oracle.attention_threaded(Q, K, V, 1, avx2=True)
    assert np.isfinite(want[0, 0, :50]).all() and not np.isfinite(want[0, 0, 50:]).all()
    assert bits_or_nan(got, want)


def test_attention_reference_order_denormal_v(exact_gpu):
    """V of denormal magnitude: products underflow to signed zeros, so the
    sign of a zero accumulator decides the output's bits; the waves with
    zero outputs take the exact recompute."""
    b, h, s, d = 1, 2, 40, 64
    Q = RNG.standard_normal((b, h, s, d)).astype(np.float32)
    K = RNG.standard_normal((b, h, s, d)).astype(np.float32)
    tiny = np.float32(1.4e-45)
    V = (RNG.choice([-1.0, 1.0], (b, h, s, d)) * RNG.integers(1, 4, (b, h, s, d))).astype(np.float32) * tiny
    got = g.attention(exact_gpu, Q, K, V, None, 1)
    want = block_oracle.attention_threaded(Q, K, V, 1, avx2=True)
    assert (want == 0).any() and np.signbit(want[want == 0]).any()
    assert bits(got, want)


def test_attention_reference_order_nan_scores(exact_gpu):
    """A NaN query row (every score NaN: the block max ignores them, the row
    is never live, output 0) and a NaN key (its weight is NaN in every row)."""
    b, h, s, d = 1, 2, 64, 128
    Q = RNG.standard_normal((b, h, s, d)).astype(np.float32)
    K = RNG.standard_normal((b, h, s, d)).astype(np.float32)
    V = RNG.standard_normal((b, h, s, d)).astype(np.float32)
    Q[0, 0, 5, 3] = np.nan
    K[0, 1, 9, :] = np.nan
    got = g.attention(exact_gpu, Q, K, V, None, 0)
    want = block_oracle.attention_threaded(Q, K, V, 0, avx2=True)
    assert (want[0, 0, 5] == 0).all() and np.isnan(want[0, 1]).all()
    assert bits_or_nan(got, want)


@pytest.mark.parametrize("flags", [0, abi.CONFIG_HIGH_THROUGHPUT | abi.CONFIG_REFERENCE_ORDER])
def test_attention_default_device_is_reference_order(flags):
    """ATTENTION_F32 is bit-exact on a device created without flags, and
    VNPU_CONFIG_REFERENCE_ORDER wins over VNPU_CONFIG_HIGH_THROUGHPUT."""
    from vnpu_mi355x import Session
    cfg = abi.Config()
    cfg.abi_version = 1
    cfg.flags = flags
    s = Session(None, cfg)
    try:
        for b, h, sq, sk, d in ((1, 2, 200, 200, 128), (2, 3, 1, 700, 64)):
            Q = RNG.standard_normal((b, h, sq, d)).astype(np.float32)
            K = RNG.standard_normal((b, h, sk, d)).astype(np.float32)
            V = RNG.standard_normal((b, h, sk, d)).astype(np.float32)
            got = g.attention(s, Q, K, V, None, 1)
            assert bits(got, block_oracle.attention_threaded(Q, K, V, 1, avx2=True))
    finally:
        s.close()


@pytest.mark.parametrize("rows,cols,temp", [(4, 32000, 1.0), (3, 50000, 0.7), (600, 300, 1.0), (5, 33, 2.0),
                                            (2, 4099, 0.0), (1, 7, 1.0)])
def test_softmax_avx2_elementwise(gpu, rows, cols, temp):
    """Every SOFTMAX_F32 kernel (one row per workgroup, the register kernel for
    few long rows, the three-pass chunked kernels) against the reference's
    AVX2 softmax, element by element with no element left out: each weight is
    the reference's bit for bit (exp256 with its clamp over the 8-wide part,
    the scalar exp in the tail, including weights exp(-80) * ... of logits
    more than 80 below the max and -inf logits); only the row sum's order
    differs."""
    X = (RNG.standard_normal((rows, cols)) * 4).astype(np.float32)
    X[0, 0] = 40.0
    X[0, 1] = -60.0
    X[0, cols - 1] = -60.0
    if rows > 1:
        X[1, 2] = -np.inf
    got = g.unary_rows(gpu, abi.OP_SOFTMAX_F32, X, temperature=temp)
    want = oracle.softmax_avx2(X, temp)
    zero = want == 0
    assert np.array_equal(got[zero], want[zero])
    rel = np.abs(got[~zero].astype(np.float64) - want[~zero]) / want[~zero]
    assert rel.max() <= 1e-5, f"max elementwise relative error {rel.max():.3g}"
