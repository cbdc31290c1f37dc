"""GPU parity: libvnpu.so (HIP, gfx950) against the C oracle, through the C ABI.

Bars (from the task's parity contract):
  * int8 tensors, scales and int32 accumulators bit-exact;
  * MATMUL_I8 f32 output bit-exact without bias (same (acc*sa)*sb order),
    rtol 1e-4 normalized with bias/epilogue;
  * f32 ops max|d| / max(1, max|ref|) <= 1e-4; attention <= 2e-3.
"""
import ctypes as C

import numpy as np
import pytest

import oracle
import gpu_ops as g
from vnpu_mi355x import abi

pytestmark = pytest.mark.gpu
RNG = np.random.default_rng(20261201)


def rel(a, b):
    return oracle.rel_error(a, b)


# ---------------------------------------------------------------- quantize
@pytest.mark.parametrize("shape", [(1, 1), (3, 7), (17, 300), (64, 512), (5, 4099), (2, 4096),
                                   (8, 11008), (3, 20000), (4096, 1000), (3000, 257), (33, 70000)])
@pytest.mark.parametrize("axis", [0, 1, 2])
def test_quantize_bit_exact(gpu, shape, axis):
    X = RNG.standard_normal(shape).astype(np.float32) * 3
    yg, sg = g.quantize(gpu, X, axis)
    yo, so = oracle.quantize(X, axis)
    assert np.array_equal(sg.view(np.uint32), so.view(np.uint32))
    assert np.array_equal(yg, yo)


@pytest.mark.parametrize("axis", [0, 1, 2])
def test_quantize_ties_zero_nonfinite(gpu, axis):
    X = RNG.integers(-100, 100, size=(8, 33)).astype(np.float32) + 0.5
    X[:, 0] = 127.0
    X[2] = 0.0
    X[3, 5] = np.inf
    X[4, 7] = np.nan
    X[5, 1] = -np.inf
    yg, sg = g.quantize(gpu, X, axis)
    yo, so = oracle.quantize(X, axis)
    assert np.array_equal(sg.view(np.uint32), so.view(np.uint32))
    assert np.array_equal(yg, yo)


def test_quantize_many_ties_full_row(gpu):
    # 2048 x 4096 activation row block: counts the exact-tie elements and
    # requires every byte to match (ties are where rint vs round differ).
    X = RNG.standard_normal((256, 4096)).astype(np.float32)
    yg, sg = g.quantize(gpu, X, 0)
    yo, so = oracle.quantize(X, 0)
    assert np.array_equal(sg.view(np.uint32), so.view(np.uint32))
    assert np.array_equal(yg, yo)


# ---------------------------------------------------------------- pack
@pytest.mark.parametrize("K,N,trans_b", [(37, 29, 0), (64, 16, 0), (100, 70, 1), (4096, 300, 0)])
def test_pack_info(gpu, K, N, trans_b):
    B = RNG.integers(-128, 128, size=(N, K) if trans_b else (K, N)).astype(np.int8)
    scales = RNG.random(N).astype(np.float32) + 0.1
    w = gpu.pack(B, K, N, scales=scales, trans_b=trans_b)
    k, n, nbytes, sc, cs = gpu.unpack_info(w)
    _, sums = oracle.pack_canonical(B, K, N, 0, trans_b)
    assert (k, n) == (K, N)
    assert nbytes == ((K + 63) // 64) * ((N + 15) // 16) * 1024
    assert np.array_equal(cs, sums)
    assert np.array_equal(sc, scales)
    gpu.release_packed(w)


# ---------------------------------------------------------------- matmul_i8
I8_SHAPES = [(1, 64, 16), (1, 4096, 4096), (1, 300, 1100), (2, 257, 33), (3, 1000, 513),
             (4, 4096, 11008), (5, 77, 19), (7, 129, 4000), (8, 4096, 1024),
             (9, 64, 16), (16, 300, 200), (64, 128, 96), (130, 257, 129), (257, 1000, 300),
             (512, 512, 512), (320, 4096, 700), (100, 1024, 2000), (513, 192, 130),
             # decode shapes of the config-4 block and long-K rows
             (8, 11008, 4096), (8, 4096, 12288), (1, 11008, 4096), (1, 40000, 48), (5, 9000, 33),
             # six or more rows over >= 1024 column strips: four strips per
             # workgroup (a ragged last group; K not a multiple of 64)
             (8, 1000, 16400), (6, 4096, 32000), (7, 130, 20000),
             # 512-1023 strips on the matrix core: two strips per workgroup, odd counts
             (8, 4096, 8200), (5, 2000, 9000),
             # one row over >= 512 strips: two strips per workgroup (513 and 1025
             # strips leave a last workgroup with one), and the headline shape
             (1, 4096, 8200), (1, 1000, 16400), (1, 4096, 32000)]


@pytest.mark.parametrize("M,K,N", I8_SHAPES)
def test_matmul_i8_bit_exact(gpu, M, K, N):
    A = RNG.integers(-128, 128, size=(M, K)).astype(np.int8)
    B = RNG.integers(-128, 128, size=(K, N)).astype(np.int8)
    sa = (RNG.random(M).astype(np.float32) + 0.5) / 127
    sb = (RNG.random(N).astype(np.float32) + 0.5) / 127
    w = gpu.pack(B, K, N, scales=sb)
    got = g.matmul_i8(gpu, A, w, M, K, N, scale_a=sa)
    want = oracle.matmul_i8(A, B, sa, sb)
    gpu.release_packed(w)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("M,K,N", [(8, 11008, 8200), (8, 20000, 4096), (6, 9000, 16400), (4, 11008, 8200),
                                   (2, 20000, 8200), (3, 50000, 300), (1, 140000, 48)])
def test_matmul_i8_gemv_multi_chunk(gpu, M, K, N):
    """Decode GEMVs whose activations are staged in two or three LDS chunks
    (up to 32 KiB per chunk from 512 column strips, 128 KiB below when the
    grid fits one workgroup per CU; a ragged last chunk): every GEMV kernel
    shape (matrix core <8,4,1>, <16,2,1>, <4,4,4>; v_dot4 for 1 to 4 rows),
    bit-exact against the float64 accumulator."""
    rng = np.random.default_rng(M * 100003 + K + N)
    A = rng.integers(-128, 128, size=(M, K)).astype(np.int8)
    B = rng.integers(-128, 128, size=(K, N)).astype(np.int8)
    sa = ((rng.random(M) + 0.5) / 127).astype(np.float32)
    sb = ((rng.random(N) + 0.5) / 127).astype(np.float32)
    w = gpu.pack(B, K, N, scales=sb)
    got = g.matmul_i8(gpu, A, w, M, K, N, scale_a=sa)
    gpu.release_packed(w)
    acc = np.zeros((M, N))
    for k0 in range(0, K, 4096):   # float64 BLAS in slices: exact, bounded memory
        acc += A[:, k0:k0 + 4096].astype(np.float64) @ B[k0:k0 + 4096].astype(np.float64)
    want = (acc.astype(np.float32) * sa[:, None]) * sb[None, :]
    assert np.array_equal(got.view(np.uint32), want.astype(np.float32).view(np.uint32))


@pytest.mark.parametrize("M,K,N", [(2048, 256, 12288), (2304, 384, 11000), (2048, 128, 12288),
                                   (4096, 256, 4096)])
def test_matmul_i8_wide_tile(gpu, M, K, N):
    """Whole 256-row tiles take the wide-tile kernels (256 x 256 for 4096 and
    11000 columns, 256 x 192 for 12288; 1, 2 and 3 k stages; a ragged last
    column tile).  Every output is
    checked: the float64 product of int8 matrices is the exact int32
    accumulator here, and C = ((float)acc * sa) * sb rounds each product
    once in float32, as the oracle's matmul_i8 does."""
    A = RNG.integers(-128, 128, size=(M, K)).astype(np.int8)
    B = RNG.integers(-128, 128, size=(K, N)).astype(np.int8)
    sa = (RNG.random(M).astype(np.float32) + 0.5) / 127
    sb = (RNG.random(N).astype(np.float32) + 0.5) / 127
    w = gpu.pack(B, K, N, scales=sb)
    got = g.matmul_i8(gpu, A, w, M, K, N, scale_a=sa)
    gpu.release_packed(w)
    acc = A.astype(np.float64) @ B.astype(np.float64)
    want = (acc.astype(np.float32) * sa[:, None]) * sb[None, :]
    assert np.array_equal(got.view(np.uint32), want.astype(np.float32).view(np.uint32))


@pytest.mark.parametrize("M,KS", [(321, 1), (300, 2), (321, 3), (300, 5), (321, 7), (300, 8), (321, 9),
                                  (300, 13), (321, 14), (300, 15)])
def test_matmul_i8_eight_wave_k_depths(gpu, M, KS):
    """Row tiles that are not whole 256-row tiles take the 8-wave kernel of
    128-deep stages; its loop runs six stages per trip and finishes the
    remaining one to seven stages separately, so each stage count from 1 to
    15 that ends in a different remainder is covered, with row clamping in
    the last row tile (M - 256 rows, not a multiple of 8).  Bit-exact
    against the exact float64 accumulator."""
    K, N = 128 * KS, 200
    A = RNG.integers(-128, 128, size=(M, K)).astype(np.int8)
    B = RNG.integers(-128, 128, size=(K, N)).astype(np.int8)
    sa = (RNG.random(M).astype(np.float32) + 0.5) / 127
    sb = (RNG.random(N).astype(np.float32) + 0.5) / 127
    w = gpu.pack(B, K, N, scales=sb)
    got = g.matmul_i8(gpu, A, w, M, K, N, scale_a=sa)
    gpu.release_packed(w)
    acc = A.astype(np.float64) @ B.astype(np.float64)
    want = (acc.astype(np.float32) * sa[:, None]) * sb[None, :]
    assert np.array_equal(got.view(np.uint32), want.astype(np.float32).view(np.uint32))


@pytest.mark.parametrize("K", [192, 320, 448, 576, 704, 832, 960, 4160])
def test_matmul_i8_pipe_odd_stage_counts(gpu, K):
    """K % 128 == 64 (an odd number of 64-deep stages) takes the 64-deep
    pipelined kernel; its loop issues two stages per trip and the drain copies
    the last one: 3 to 65 stages, bit-exact against the float64 accumulator
    (from 7 stages up the last stage used to be left uncopied)."""
    M, N = 300, 200
    A = RNG.integers(-128, 128, size=(M, K)).astype(np.int8)
    B = RNG.integers(-128, 128, size=(K, N)).astype(np.int8)
    sa = (RNG.random(M).astype(np.float32) + 0.5) / 127
    sb = (RNG.random(N).astype(np.float32) + 0.5) / 127
    w = gpu.pack(B, K, N, scales=sb)
    got = g.matmul_i8(gpu, A, w, M, K, N, scale_a=sa)
    gpu.release_packed(w)
    acc = A.astype(np.float64) @ B.astype(np.float64)
    want = (acc.astype(np.float32) * sa[:, None]) * sb[None, :]
    assert np.array_equal(got.view(np.uint32), want.astype(np.float32).view(np.uint32))


@pytest.mark.parametrize("tiles,K", [((256, 128, 256), 20480), ((256, 128, 192), 20480),
                                     ((256, 128, 128), 20480), ((256, 64, 128), 20544)])
def test_matmul_i8_long_k_every_kernel(gpu, tiles, K):
    """K above 16384 on the wide, 8-wave and 64-deep pipelined kernels
    (160 or 321 stages): the exact integer product, C = (float)acc."""
    rng = np.random.default_rng(K + tiles[2])
    M, N = 512, 520
    A = rng.integers(-128, 128, size=(M, K)).astype(np.int8)
    B = rng.integers(-128, 128, size=(K, N)).astype(np.int8)
    w = gpu.pack(B, K, N)
    info0 = gpu.info()
    assert gpu.lib.vnpu_device_set_tiles(gpu.dev, *tiles) == abi.OK
    try:
        got = g.matmul_i8(gpu, A, w, M, K, N)
    finally:
        gpu.lib.vnpu_device_set_tiles(gpu.dev, info0.tile_m, info0.tile_k, info0.tile_n)
        gpu.release_packed(w)
    acc = A.astype(np.float64) @ B.astype(np.float64)   # exact: |acc| < 2^53
    assert np.array_equal(got, acc.astype(np.float32))


@pytest.mark.parametrize("M,N0,N1,alias", [(512, 3000, 2000, False), (512, 11008, 11008, False),
                                           (6, 9000, 9000, False), (8, 8200, 9000, False),
                                           (512, 1000, 700, True), (8, 11008, 11008, False),
                                           (6, 3000, 2000, False), (8, 1000, 700, True),
                                           (8, 20000, 700, False), (5, 4096, 4096, False),
                                           (7, 1500, 1500, False)])
def test_matmul_i8_pair_in_one_batch(gpu, M, N0, N1, alias):
    """Two MATMUL_I8 commands in one batch with the same M (the block's gate
    and up projections) may share one launch (a wide-tile grid, or one
    matrix-core GEMV grid at M <= 8); both outputs must be the oracle's bits,
    with their own bias and epilogue.  With `alias` the second command reads
    the first one's output as its A (a dependency), which must keep them in
    order; 20000 and 700 columns take different GEMV variants (not paired)."""
    K = 256
    A = RNG.integers(-128, 128, size=(M, K)).astype(np.int8)
    B0 = RNG.integers(-128, 128, size=(K, N0)).astype(np.int8)
    B1 = RNG.integers(-128, 128, size=(K if not alias else 256, N1)).astype(np.int8)
    sa = (RNG.random(M).astype(np.float32) + 0.5) / 127
    sb0 = (RNG.random(N0).astype(np.float32) + 0.5) / 127
    sb1 = (RNG.random(N1).astype(np.float32) + 0.5) / 127
    bias1 = RNG.standard_normal(N1).astype(np.float32)
    w0, w1 = gpu.pack(B0, K, N0, scales=sb0), gpu.pack(B1, 256, N1, scales=sb1)
    ba, bsa = gpu.upload(A), gpu.upload(sa)
    bc0, bc1, bb1 = gpu.alloc(4 * M * N0), gpu.alloc(4 * M * N1), gpu.upload(bias1)
    # alias: the second GEMM's A is the first GEMM's output bytes (int8 view)
    a1 = bc0 if alias else ba
    cmds = [gpu.command(abi.OP_MATMUL_I8, A=ba, B=w0, scale_a=bsa.ptr, C=bc0, M=M, K=K, N=N0),
            gpu.command(abi.OP_MATMUL_I8, A=a1, B=w1, scale_a=bsa.ptr, bias=bb1.ptr, C=bc1, M=M, K=256,
                        N=N1, lda=4 * N0 if alias else 0, epilogue=2)]
    assert gpu.submit(cmds) == abi.OK and gpu.sync() == abi.OK
    c0 = gpu.download(bc0, np.float32, (M, N0))
    c1 = gpu.download(bc1, np.float32, (M, N1))
    for b in (ba, bsa, bc0, bc1, bb1):
        gpu.free(b)
    gpu.release_packed(w0)
    gpu.release_packed(w1)
    want0 = oracle.matmul_i8(A, B0, sa, sb0)
    assert np.array_equal(c0.view(np.uint32), want0.view(np.uint32))
    A1 = want0.view(np.int8).reshape(M, 4 * N0)[:, :256] if alias else A
    want1 = oracle.matmul_i8(A1, B1, sa, sb1, bias1, 2)
    assert rel(c1, want1) <= 1e-4


@pytest.mark.parametrize("M,N,mode", [(8, 4096, "in_place"), (1, 4096, "in_place"), (8, 1000, "c_first"),
                                        (5, 700, "y_is_c"), (8, 2000, "both0"), (3, 3000, "scaled"),
                                        (8, 1000, "count_mismatch"), (12, 1000, "in_place")])
def test_matmul_i8_then_add_in_one_batch(gpu, M, N, mode):
    """MATMUL_I8 at M <= 8 followed by an ADD_F32 of its output in the same
    batch (the block's down projection + residual at decode) may run as one
    GEMV launch whose store also writes the ADD's result.  Both outputs must
    be the bits of the same two commands submitted in separate batches (and C
    the oracle's within 1e-4 under its SiLU epilogue): the residual in place, C as the ADD's first operand, the
    ADD writing over C, alpha = beta = 0 (the defaults 1, 1), other scales;
    a count that is not M x N and M > 8 run unfused."""
    K = 512
    A = RNG.integers(-128, 128, size=(M, K)).astype(np.int8)
    B = RNG.integers(-128, 128, size=(K, N)).astype(np.int8)
    sa = (RNG.random(M).astype(np.float32) + 0.5) / 127
    sb = (RNG.random(N).astype(np.float32) + 0.5) / 127
    bias = RNG.standard_normal(N).astype(np.float32)
    x = RNG.standard_normal(M * N).astype(np.float32) * 100
    w = gpu.pack(B, K, N, scales=sb)
    ba, bsa, bb = gpu.upload(A), gpu.upload(sa), gpu.upload(bias)
    alpha, beta = {"both0": (0.0, 0.0), "scaled": (0.5, -2.0)}.get(mode, (1.0, 1.0))
    count = M * N - 4 if mode == "count_mismatch" else M * N

    def run(fused):
        bc, bx, by = gpu.alloc(4 * M * N), gpu.upload(x), gpu.alloc(4 * M * N)
        mm = gpu.command(abi.OP_MATMUL_I8, A=ba, B=w, scale_a=bsa.ptr, bias=bb.ptr, C=bc, M=M, K=K, N=N,
                         epilogue=2)
        a_, b_, y_ = (bc, bx, by) if mode == "c_first" else (bx, bc, bc if mode == "y_is_c" else
                                                             (bx if mode in ("in_place", "count_mismatch") else by))
        add = gpu.command(abi.OP_ADD_F32, A=a_, B=b_, Y=y_, count=count, alpha=alpha, beta=beta)
        batches = [[mm, add]] if fused else [[mm], [add]]
        for cmds in batches:
            assert gpu.submit(cmds) == abi.OK and gpu.sync() == abi.OK
        out = {n: gpu.download(b, np.float32, (M * N,)) for n, b in (("c", bc), ("x", bx), ("y", by))}
        for b in (bc, bx, by):
            gpu.free(b)
        return out

    got, want = run(True), run(False)
    for b in (ba, bsa, bb):
        gpu.free(b)
    gpu.release_packed(w)
    for n in ("c", "x", "y"):
        assert np.array_equal(got[n].view(np.uint32), want[n].view(np.uint32)), n
    if mode != "y_is_c":   # there the ADD overwrote C in both runs
        # SiLU epilogue: the same bar as the paired test's
        assert rel(got["c"], oracle.matmul_i8(A, B, sa, sb, bias, 2).reshape(-1)) <= 1e-4


@pytest.mark.parametrize("M", [9, 13, 16, 17, 31, 32, 33, 48, 64, 65])
@pytest.mark.parametrize("K,N", [(320, 4096), (4160, 9000), (192, 17600), (1000, 100)])
def test_matmul_i8_few_rows(gpu, M, K, N):
    """9..64 rows run the weight-streaming matrix-core kernel with a row
    capacity of 16, 32 or 64 (rows past M zero, not stored), in each of its
    three launch shapes (4096, 9000 and 17600 columns: 256, 563 and 1100
    strips); 65 rows take the GEMM kernels.  Bit-exact with scales, bias and
    a ReLU epilogue, and a ragged K (1000)."""
    A = RNG.integers(-128, 128, size=(M, K)).astype(np.int8)
    B = RNG.integers(-128, 128, size=(K, N)).astype(np.int8)
    sa = (RNG.random(M).astype(np.float32) + 0.5) / 127
    sb = (RNG.random(N).astype(np.float32) + 0.5) / 127
    bias = RNG.standard_normal(N).astype(np.float32)
    w = gpu.pack(B, K, N, scales=sb)
    ba, bsa, bb, bc = gpu.upload(A), gpu.upload(sa), gpu.upload(bias), gpu.alloc(4 * M * N)
    gpu.run(abi.OP_MATMUL_I8, A=ba, B=w, scale_a=bsa.ptr, bias=bb.ptr, C=bc, M=M, K=K, N=N, epilogue=1)
    got = gpu.download(bc, np.float32, (M, N))
    for b in (ba, bsa, bb, bc):
        gpu.free(b)
    gpu.release_packed(w)
    want = oracle.matmul_i8(A, B, sa, sb, bias, 1)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("M", [1, 6, 40])
def test_matmul_i8_accumulator_exact(gpu, M):
    # scale 1 everywhere: C == (float)acc exactly while |acc| < 2^24
    K, N = 1000, 257
    A = RNG.integers(-128, 128, size=(M, K)).astype(np.int8)
    B = RNG.integers(-128, 128, size=(K, N)).astype(np.int8)
    w = gpu.pack(B, K, N)
    got = g.matmul_i8(gpu, A, w, M, K, N)
    gpu.release_packed(w)
    acc = A.astype(np.int64) @ B.astype(np.int64)
    assert np.array_equal(got.astype(np.int64), acc)


@pytest.mark.parametrize("M", [1, 3, 8, 33])
@pytest.mark.parametrize("epi", [1, 2, 3, 4])
def test_matmul_i8_bias_epilogue(gpu, M, epi):
    K, N = 320, 200
    A = RNG.integers(-128, 128, size=(M, K)).astype(np.int8)
    B = RNG.integers(-128, 128, size=(K, N)).astype(np.int8)
    sa = RNG.random(M).astype(np.float32) / 127
    sb = RNG.random(N).astype(np.float32) / 127
    bias = RNG.standard_normal(N).astype(np.float32)
    w = gpu.pack(B, K, N, scales=sb)
    got = g.matmul_i8(gpu, A, w, M, K, N, scale_a=sa, bias=bias, epilogue=epi)
    gpu.release_packed(w)
    assert rel(got, oracle.matmul_i8(A, B, sa, sb, bias, epi)) <= 1e-4


@pytest.mark.parametrize("M", [2, 20])
def test_matmul_i8_strided_and_trans_b(gpu, M):
    K, N, lda, ldc = 200, 70, 256, 80
    A = RNG.integers(-128, 128, size=(M, lda)).astype(np.int8)
    Bt = RNG.integers(-128, 128, size=(N, K)).astype(np.int8)
    w = gpu.pack(Bt, K, N, trans_b=1)
    got = g.matmul_i8(gpu, A, w, M, K, N, lda=lda, ldc=ldc)
    gpu.release_packed(w)
    acc = A[:, :K].astype(np.int64) @ Bt.T.astype(np.int64)
    assert np.array_equal(got.astype(np.int64), acc)


@pytest.mark.parametrize("tiles,M,K", [((256, 128, 256), 512, 640), ((256, 128, 192), 512, 640),
                                        ((256, 128, 128), 320, 640), ((256, 64, 128), 320, 576)])
def test_matmul_i8_strided_a_every_kernel(gpu, tiles, M, K):
    """A with a row stride above K (lda = K + 48) and a padded C on each
    pipelined kernel: their copies address rows as a base plus lda steps."""
    rng = np.random.default_rng(K + M + tiles[2])
    N, lda, ldc = 300, K + 48, 312
    A = rng.integers(-128, 128, size=(M, lda)).astype(np.int8)
    B = rng.integers(-128, 128, size=(K, N)).astype(np.int8)
    w = gpu.pack(B, K, N)
    info0 = gpu.info()
    assert gpu.lib.vnpu_device_set_tiles(gpu.dev, *tiles) == abi.OK
    try:
        got = g.matmul_i8(gpu, A, w, M, K, N, lda=lda, ldc=ldc)
    finally:
        gpu.lib.vnpu_device_set_tiles(gpu.dev, info0.tile_m, info0.tile_k, info0.tile_n)
        gpu.release_packed(w)
    acc = A[:, :K].astype(np.float64) @ B.astype(np.float64)
    assert np.array_equal(got, acc.astype(np.float32))


def test_matmul_i8_zero_weight_blocks_exact(gpu):
    """Weights with zero 64 x 64 tiles (the config-5 pattern), on the GEMM
    (M = 64) and the GEMV (M = 4): the exact integer product."""
    M, K, N = 64, 512, 256
    A = RNG.integers(-128, 128, size=(M, K)).astype(np.int8)
    B = RNG.integers(-128, 128, size=(K, N)).astype(np.int8)
    keep = RNG.integers(0, 2, size=(K // 64, N // 64)).astype(bool)
    B *= np.kron(keep, np.ones((64, 64), bool)).astype(np.int8)
    for m in (M, 4):
        w = gpu.pack(B, K, N)
        got = g.matmul_i8(gpu, A[:m], w, m, K, N)
        gpu.release_packed(w)
        assert np.array_equal(got.astype(np.int64), A[:m].astype(np.int64) @ B.astype(np.int64))


def _zero_pattern(kind, K, N, rng):
    """A weight mask of zero 1 KiB blocks (64 deep x 16 columns) or larger."""
    if kind == "tiles64":        # the config-5 pattern: 64 x 64 tiles
        keep = rng.integers(0, 2, size=(K // 64, -(-N // 64))).astype(bool)
        return np.kron(keep, np.ones((64, 64), bool))[:, :N]
    if kind == "blocks16":       # single 16-column blocks: pairs half zero
        keep = rng.random((K // 64, -(-N // 16))) < 0.4
        return np.kron(keep, np.ones((64, 16), bool))[:, :N]
    keep = np.ones((K // 64, 1), bool)   # whole k blocks zero, every column
    keep[rng.random(K // 64) < 0.5] = False
    keep[0] = False
    return np.kron(keep, np.ones((64, N), bool))


@pytest.mark.parametrize("tiles", [(256, 128, 256), (256, 128, 192), (256, 128, 128)])
@pytest.mark.parametrize("epi", [abi.EPI_NONE, abi.EPI_RELU, abi.EPI_SILU, abi.EPI_GELU_TANH])
def test_matmul_i8_register_epilogue_padded_c(gpu, tiles, epi):
    """The wide and 8-wave kernels store C straight from the accumulator
    registers through a buffer whose range check drops rows past M and
    columns past N.  With a padded C (ldc > N) and sentinel rows after row
    M, the padding and the sentinel rows keep their contents, and the stored
    values follow the reference's store_i8_c order
    (src/kernels/kernels.cpp:526-535): bit for bit without an activation,
    within 1e-6 with one (the activations' exp is the backend's own)."""
    rng = np.random.default_rng(1000 + 10 * epi + tiles[2])
    M = 320 if tiles[2] == 128 else 512   # the 8-wave tile takes a ragged last row tile
    K, N, ldc, extra = 384, 520, 536, 8
    A = rng.integers(-128, 128, size=(M, K)).astype(np.int8)
    B = rng.integers(-128, 128, size=(K, N)).astype(np.int8)
    sa = ((rng.random(M) + 0.5) / 127).astype(np.float32)
    sb = ((rng.random(N) + 0.5) / 127).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    w = gpu.pack(B, K, N, scales=sb)
    sentinel = np.float32(7.25)
    ba, bsa, bb = gpu.upload(A), gpu.upload(sa), gpu.upload(bias)
    bc = gpu.upload(np.full((M + extra, ldc), sentinel, np.float32))
    info0 = gpu.info()
    assert gpu.lib.vnpu_device_set_tiles(gpu.dev, *tiles) == abi.OK
    try:
        gpu.run(abi.OP_MATMUL_I8, A=ba, B=w, scale_a=bsa.ptr, bias=bb.ptr, C=bc, M=M, K=K, N=N, ldc=ldc,
                epilogue=epi)
        out = gpu.download(bc, np.float32, (M + extra, ldc))
    finally:
        gpu.lib.vnpu_device_set_tiles(gpu.dev, info0.tile_m, info0.tile_k, info0.tile_n)
        gpu.release_packed(w)
        for b in (ba, bsa, bb, bc):
            gpu.free(b)
    assert np.all(out[:, N:] == sentinel) and np.all(out[M:] == sentinel)
    want = oracle.matmul_i8(A, B, sa, sb, bias, epi)
    if epi == abi.EPI_NONE:
        assert np.array_equal(out[:M, :N].view(np.uint32), want.view(np.uint32))
    else:
        assert rel(out[:M, :N], want) <= 1e-6


@pytest.mark.parametrize("tiles,K,M", [((256, 64, 128), 448, 320), ((128, 128, 64), 448, 320),
                                        ((256, 64, 128), 576, 64), ((128, 128, 64), 1000, 257)])
@pytest.mark.parametrize("epi", [abi.EPI_NONE, abi.EPI_RELU, abi.EPI_SILU, abi.EPI_GELU_TANH])
def test_matmul_i8_staged_epilogue_padded_c(gpu, tiles, K, M, epi):
    """The 64-deep pipelined kernel and the generic one store C from an LDS-
    staged tile (row scales, column scales, bias, epilogue): with a padded C
    and sentinel rows after row M the padding and those rows keep their
    contents, and the values follow store_i8_c's order
    (src/kernels/kernels.cpp:526-535)."""
    rng = np.random.default_rng(2000 + 10 * epi + K + M)
    N, ldc, extra = 520, 536, 8
    A = rng.integers(-128, 128, size=(M, K)).astype(np.int8)
    B = rng.integers(-128, 128, size=(K, N)).astype(np.int8)
    sa = ((rng.random(M) + 0.5) / 127).astype(np.float32)
    sb = ((rng.random(N) + 0.5) / 127).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    w = gpu.pack(B, K, N, scales=sb)
    sentinel = np.float32(-1.75)
    ba, bsa, bb = gpu.upload(A), gpu.upload(sa), gpu.upload(bias)
    bc = gpu.upload(np.full((M + extra, ldc), sentinel, np.float32))
    info0 = gpu.info()
    assert gpu.lib.vnpu_device_set_tiles(gpu.dev, *tiles) == abi.OK
    try:
        gpu.run(abi.OP_MATMUL_I8, A=ba, B=w, scale_a=bsa.ptr, bias=bb.ptr, C=bc, M=M, K=K, N=N, ldc=ldc,
                epilogue=epi)
        out = gpu.download(bc, np.float32, (M + extra, ldc))
    finally:
        gpu.lib.vnpu_device_set_tiles(gpu.dev, info0.tile_m, info0.tile_k, info0.tile_n)
        gpu.release_packed(w)
        for b in (ba, bsa, bb, bc):
            gpu.free(b)
    assert np.all(out[:, N:] == sentinel) and np.all(out[M:] == sentinel)
    want = oracle.matmul_i8(A, B, sa, sb, bias, epi)
    if epi == abi.EPI_NONE:
        assert np.array_equal(out[:M, :N].view(np.uint32), want.view(np.uint32))
    else:
        assert rel(out[:M, :N], want) <= 1e-6


@pytest.mark.parametrize("tiles", [(256, 128, 256), (256, 128, 192), (256, 128, 128), (128, 128, 64)])
@pytest.mark.parametrize("K", [128, 384, 1024])
@pytest.mark.parametrize("kind", ["tiles64", "blocks16", "kblocks"])
def test_matmul_i8_zero_weight_blocks_every_kernel(gpu, tiles, K, kind):
    """Weights with all-zero blocks (64 x 64 tiles, single 16-column
    blocks, whole k blocks) on every prefill kernel a tile triple can select
    (the last the automatic choice): one and several stages and a ragged last
    tile, exact."""
    rng = np.random.default_rng(K * 7 + len(kind))
    M, N = 512, 520
    A = rng.integers(-128, 128, size=(M, K)).astype(np.int8)
    B = rng.integers(-128, 128, size=(K, N)).astype(np.int8)
    B *= _zero_pattern(kind, K, N, rng).astype(np.int8)
    w = gpu.pack(B, K, N)
    info0 = gpu.info()
    assert gpu.lib.vnpu_device_set_tiles(gpu.dev, *tiles) == abi.OK
    try:
        got = g.matmul_i8(gpu, A, w, M, K, N)
    finally:
        gpu.lib.vnpu_device_set_tiles(gpu.dev, info0.tile_m, info0.tile_k, info0.tile_n)
        gpu.release_packed(w)
    assert np.array_equal(got.astype(np.int64), A.astype(np.int64) @ B.astype(np.int64))


# ---------------------------------------------------------------- matmul_f32
F32_CASES = [(37, 53, 29, 0, 0), (17, 41, 23, 0, 1), (9, 33, 18, 1, 0), (1, 512, 137, 0, 0),
             (4, 4096, 1000, 0, 0), (8, 300, 33, 0, 1), (64, 128, 64, 1, 1), (200, 300, 130, 0, 0),
             (256, 1024, 256, 0, 1)]


@pytest.mark.parametrize("M,K,N,ta,tb", F32_CASES)
@pytest.mark.parametrize("epi,beta,alpha", [(0, 0.0, 0.0), (2, 0.0, 1.0), (3, 0.5, 1.0), (1, 0.0, -2.0)])
def test_matmul_f32(gpu, M, K, N, ta, tb, epi, beta, alpha):
    A = RNG.standard_normal((K, M) if ta else (M, K)).astype(np.float32)
    B = RNG.standard_normal((N, K) if tb else (K, N)).astype(np.float32)
    bias = RNG.standard_normal(N).astype(np.float32)
    C0 = RNG.standard_normal((M, N)).astype(np.float32)
    got = g.matmul_f32(gpu, A, B, M, K, N, C_in=C0, bias=bias, trans_a=ta, trans_b=tb, beta=beta,
                       alpha=alpha, epilogue=epi)
    want = oracle.matmul_f32(A, B, C0, bias, M, K, N, ta, tb, alpha if alpha else 1.0, beta, epi,
                             acc64=True)
    assert rel(got, want) <= 1e-4


@pytest.mark.parametrize("M,K,N,ta,tb,epi,beta", [
    (1024, 1000, 2176, 0, 0, 2, 0.0), (1024, 1000, 2176, 0, 1, 3, 0.5), (1100, 520, 1920, 1, 0, 1, 0.0),
    (1100, 520, 1920, 1, 1, 0, 0.5), (2048, 4096, 1024, 0, 1, 3, 0.5), (1030, 37, 2050, 0, 0, 0, 0.0),
    (1100, 100, 6600, 0, 0, 2, 0.0), (1100, 37, 6600, 1, 1, 3, 0.5), (1300, 520, 6200, 0, 1, 3, 0.5),
    (1300, 520, 6200, 1, 0, 0, 0.0), (2048, 1000, 4096, 0, 1, 3, 0.5)])
def test_matmul_f32_split_bf16(gpu, M, K, N, ta, tb, epi, beta):
    """Grids of >= 128 tiles run the split-bf16 kernel (hi*hi + hi*lo + lo*hi
    on the bf16 matrix cores): every transpose combination, ragged M / N / K,
    the config-3 epilogue (bias, beta 0.5 onto C, GELU), to the f32 bar.  The
    last five have at least 256 tiles of 256 x 128, which take the eight-wave
    256 x 128 tile (the others the four-wave 128 x 128 one)."""
    A = RNG.standard_normal((K, M) if ta else (M, K)).astype(np.float32)
    B = RNG.standard_normal((N, K) if tb else (K, N)).astype(np.float32)
    bias = RNG.standard_normal(N).astype(np.float32)
    C0 = RNG.standard_normal((M, N)).astype(np.float32)
    got = g.matmul_f32(gpu, A, B, M, K, N, C_in=C0, bias=bias, trans_a=ta, trans_b=tb, beta=beta,
                       alpha=1.0, epilogue=epi)
    want = oracle.matmul_f32(A, B, C0, bias, M, K, N, ta, tb, 1.0, beta, epi, acc64=True)
    assert rel(got, want) <= 1e-4



@pytest.mark.parametrize("M,K,N,ta,tb", [(1100, 520, 6600, 0, 0), (1300, 520, 6200, 0, 1),
                                         (1100, 520, 1920, 1, 0), (512, 512, 512, 0, 1)])
def test_matmul_f32_strided_operands(gpu, M, K, N, ta, tb):
    """A and B with row strides above their widths on the split-bf16 paths:
    the warp-specialised kernel (B as K x N and as N x K), the four-wave tile
    with op(A) = A^T, and a K-split small grid; to the f32 bar."""
    rng = np.random.default_rng(M + K + N + 10 * ta + tb)
    a_rows, a_cols = (K, M) if ta else (M, K)
    b_rows, b_cols = (N, K) if tb else (K, N)
    lda, ldb = a_cols + 12, b_cols + 20
    A = rng.standard_normal((a_rows, lda)).astype(np.float32)
    B = rng.standard_normal((b_rows, ldb)).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    C0 = rng.standard_normal((M, N)).astype(np.float32)
    ba, bb, bbias, bc = gpu.upload(A), gpu.upload(B), gpu.upload(bias), gpu.upload(C0)
    try:
        gpu.run(abi.OP_MATMUL_F32, A=ba, B=bb, bias=bbias.ptr, C=bc, M=M, K=K, N=N, lda=lda, ldb=ldb,
                trans_a=ta, trans_b=tb, alpha=1.0, beta=0.5, epilogue=abi.EPI_SILU)
        got = gpu.download(bc, np.float32, (M, N))
    finally:
        for b in (ba, bb, bbias, bc):
            gpu.free(b)
    want = oracle.matmul_f32(np.ascontiguousarray(A[:, :a_cols]), np.ascontiguousarray(B[:, :b_cols]), C0, bias,
                             M, K, N, ta, tb, 1.0, 0.5, abi.EPI_SILU, acc64=True)
    assert rel(got, want) <= 1e-4


@pytest.mark.parametrize("M,K,N,pad", [(1, 4096, 32000, 0), (4, 1000, 25600, 0), (8, 300, 25602, 0),
                                       (3, 17, 26000, 6), (5, 1, 25600, 0), (2, 2000, 25601, 0),
                                       (7, 513, 25800, 3), (6, 4100, 25472, 0), (1, 12000, 25600, 0),
                                       (4, 8192, 25600, 0), (5, 4096, 25602, 2)])
def test_matmul_f32_gemv_wide_n(gpu, M, K, N, pad):
    """M <= 8 with at least 200 column blocks of 128 (the MTP head's width)
    runs the one-pass 16-wave GEMV when N and ldb are even: a partial last
    block, K below the wave count, a padded ldb, the largest K whose staged
    activations fit LDS (8192 at 4 rows, 4096 at 5-8), one row at a K past
    that (scalar activations), and the cases that fall back to the split-K
    GEMV (odd N, odd ldb, 199 blocks); bias, alpha (-2 at odd M), beta and
    GELU epilogue, to the f32 bar."""
    rng = np.random.default_rng(M * 7 + K + N + pad)
    ldb = N + pad
    A = rng.standard_normal((M, K)).astype(np.float32)
    B = rng.standard_normal((K, ldb)).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    C0 = rng.standard_normal((M, N)).astype(np.float32)
    alpha = -2.0 if M % 2 else 1.0
    ba, bb, bbias, bc = gpu.upload(A), gpu.upload(B), gpu.upload(bias), gpu.upload(C0)
    try:
        gpu.run(abi.OP_MATMUL_F32, A=ba, B=bb, bias=bbias.ptr, C=bc, M=M, K=K, N=N, ldb=ldb,
                alpha=alpha, beta=0.5, epilogue=abi.EPI_GELU_TANH)
        got = gpu.download(bc, np.float32, (M, N))
    finally:
        for b in (ba, bb, bbias, bc):
            gpu.free(b)
    want = oracle.matmul_f32(A, np.ascontiguousarray(B[:, :N]), C0, bias, M, K, N, 0, 0, alpha, 0.5,
                             abi.EPI_GELU_TANH, acc64=True)
    assert rel(got, want) <= 1e-4


@pytest.mark.parametrize("beta", [0.0, 0.5])
def test_matmul_f32_split_bf16_padded_c(gpu, beta):
    """The eight-wave split-bf16 tile stores C (and reads C_in for beta)
    straight from its accumulators through a buffer whose range check drops
    rows past M and columns past N: with ldc > N and sentinel rows after row
    M, the padding and the sentinel rows keep their contents and the rest is
    alpha * A B + bias + beta * C_in -> GELU to the f32 bar."""
    rng = np.random.default_rng(77 + int(beta * 10))
    M, K, N, ldc, extra = 1100, 96, 6600, 6616, 8       # 5 x 52 tiles of 256 x 128, ragged M and N
    A = rng.standard_normal((M, K)).astype(np.float32)
    B = rng.standard_normal((K, N)).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    sentinel = np.float32(-3.5)
    C0 = np.full((M + extra, ldc), sentinel, np.float32)
    C0[:M, :N] = rng.standard_normal((M, N)).astype(np.float32)
    ba, bb, bbias, bc = gpu.upload(A), gpu.upload(B), gpu.upload(bias), gpu.upload(C0)
    try:
        gpu.run(abi.OP_MATMUL_F32, A=ba, B=bb, bias=bbias.ptr, C=bc, M=M, K=K, N=N, ldc=ldc, alpha=1.0,
                beta=beta, epilogue=abi.EPI_GELU_TANH)
        out = gpu.download(bc, np.float32, (M + extra, ldc))
    finally:
        for b in (ba, bb, bbias, bc):
            gpu.free(b)
    assert np.all(out[:, N:] == sentinel) and np.all(out[M:] == sentinel)
    want = oracle.matmul_f32(A, B, C0[:M, :N], bias, M, K, N, 0, 0, 1.0, beta, abi.EPI_GELU_TANH, acc64=True)
    assert rel(out[:M, :N], want) <= 1e-4


@pytest.mark.parametrize("M,N,unit", [(256, 512, 2), (40, 96, 2), (128, 128, 1), (300, 200, 3),
                                      (4, 300, 0)])
def test_matmul_f32_wildcat_cull(gpu, M, N, unit):
    K = 24
    mask = RNG.integers(0, 2, size=(4, 6)).astype(np.uint8)
    A = RNG.standard_normal((M, K)).astype(np.float32)
    B = RNG.standard_normal((K, N)).astype(np.float32)
    got = g.matmul_f32(gpu, A, B, M, K, N, mask=mask, unit=unit)
    info = gpu.info()
    cull, _ = oracle.cull_map(M, N, unit, info.tile_m, info.tile_n, info.num_threads, 1, mask)
    assert np.array_equal(got == 0.0, cull.astype(bool))
    want = oracle.matmul_f32(A, B, None, None, M, K, N, 0, 0, 1.0, 0.0, 0, cull=cull, acc64=False)
    assert rel(got, want) <= 1e-4


@pytest.mark.parametrize("M,N,unit", [(256, 512, 2), (300, 200, 3), (1000, 1100, 2)])
def test_matmul_f32_cull_device_mask_matches_host_mask(gpu, M, N, unit):
    """A tile mask in device memory is sampled and classified on the GPU (no
    copy back in submit): the same outputs as the same mask in host memory,
    and the same culled-tile count in the device status."""
    K = 40
    mask = RNG.integers(0, 2, size=(5, 7)).astype(np.uint8)
    A = RNG.standard_normal((M, K)).astype(np.float32)
    B = RNG.standard_normal((K, N)).astype(np.float32)
    ba, bb, bm = gpu.upload(A), gpu.upload(B), gpu.upload(mask)
    outs, culled = [], []
    for mptr in (mask.ctypes.data, bm.ptr):
        bc = gpu.alloc(4 * M * N)
        before = gpu.status().tiles_culled
        gpu.run(abi.OP_MATMUL_F32, A=ba, B=bb, C=bc, M=M, K=K, N=N, unit=unit, tile_mask=mptr,
                mask_tile_m=mask.shape[0], mask_tile_n=mask.shape[1])
        assert gpu.sync() == abi.OK
        culled.append(gpu.status().tiles_culled - before)
        outs.append(gpu.download(bc, np.float32, (M, N)))
        gpu.free(bc)
    for b in (ba, bb, bm):
        gpu.free(b)
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    assert culled[0] == culled[1] > 0


# ---------------------------------------------------------------- row / elementwise ops
@pytest.mark.parametrize("rows,cols", [(1, 7), (7, 300), (64, 4096), (3, 32000), (5, 11008), (2, 12288),
                                       (3, 12292)])
def test_rmsnorm_softmax(gpu, rows, cols):
    X = RNG.standard_normal((rows, cols)).astype(np.float32)
    W = RNG.standard_normal(cols).astype(np.float32)
    assert rel(g.unary_rows(gpu, abi.OP_RMSNORM_F32, X, W=W, eps=1e-5), oracle.rmsnorm(X, W, 1e-5)) <= 1e-4
    assert rel(g.unary_rows(gpu, abi.OP_RMSNORM_F32, X, eps=0.0), oracle.rmsnorm(X, None, 1e-5)) <= 1e-4
    sm = g.unary_rows(gpu, abi.OP_SOFTMAX_F32, X * 4, temperature=0.0)
    assert rel(sm, oracle.softmax(X * 4, 1.0)) <= 1e-4
    assert np.allclose(sm.sum(axis=1), 1.0, atol=1e-4)


@pytest.mark.parametrize("rows,cols", [(4, 2049), (2, 300000), (511, 3000), (4, 32000)])
def test_softmax_split_rows(gpu, rows, cols):
    """Few long rows are split over workgroups; includes a temperature, a
    chunk that is -inf throughout (masked logits) and a ragged last chunk.

    The reference sums a row's exponentials one after another in float32;
    over 300000 columns that sum is itself off by more than 1e-4 (relative),
    so the bar is 1e-4 or twice the reference's own distance from the float64
    softmax, whichever is larger, and the GPU must be within 1e-4 of float64.
    The masked logits get what the reference's AVX2 build gives them: its
    8-wide exp clamps -inf to -80, so exp(-80) / sum (about 1e-35), not 0."""
    X = (RNG.standard_normal((rows, cols)) * 3).astype(np.float32)
    X[0, :1500] = -np.inf
    for t in (0.0, 0.7):
        sm = g.unary_rows(gpu, abi.OP_SOFTMAX_F32, X, temperature=t)
        want = oracle.softmax(X, 1.0 if t == 0.0 else t)
        x64 = X.astype(np.float64) * (1.0 if t == 0.0 else 1.0 / t)
        e = np.exp(x64 - x64.max(axis=1, keepdims=True))
        exact = e / e.sum(axis=1, keepdims=True)
        assert rel(sm, want) <= max(1e-4, 2 * rel(want, exact))
        assert rel(sm, exact) <= 1e-4
        masked = oracle.softmax_avx2(X[:1], 1.0 if t == 0.0 else t)[0, :1500]
        assert np.all(masked > 0.0) and np.all(masked < 1e-30)
        # the same weight over a row sum added in another order (3.6e-5 apart
        # at 300000 columns)
        np.testing.assert_allclose(sm[0, :1500], masked, rtol=1e-4, atol=0)
        assert np.allclose(sm.sum(axis=1), 1.0, atol=1e-4)


@pytest.mark.parametrize("n", [1, 1001, 4096 * 8 + 3, 2048 * 11008 // 64])
def test_elementwise(gpu, n):
    a = RNG.standard_normal(n).astype(np.float32)
    b = RNG.standard_normal(n).astype(np.float32)
    assert rel(g.elementwise(gpu, abi.OP_SWIGLU_F32, a, b, alpha=0.0), oracle.swiglu(a, b, 1.0)) <= 1e-4
    assert rel(g.elementwise(gpu, abi.OP_GELU_F32, a), oracle.gelu(a)) <= 1e-4
    assert rel(g.elementwise(gpu, abi.OP_ADD_F32, a, b, 0.0, 0.0), oracle.add(a, b, 1.0, 1.0)) <= 1e-6
    assert rel(g.elementwise(gpu, abi.OP_ADD_F32, a, b, 0.5, -2.0), oracle.add(a, b, 0.5, -2.0)) <= 1e-6
    assert rel(g.elementwise(gpu, abi.OP_MUL_F32, a, b, 0.0, 0.25), oracle.mul(a, b, 1.0, 0.25)) <= 1e-6


@pytest.mark.parametrize("interleaved", [0, 1])
@pytest.mark.parametrize("shape_q,shape_k,offset", [((2, 3, 40, 16), (2, 3, 24, 16), 100),
                                                    ((1, 4, 2048, 128), (1, 4, 2048, 128), 0),
                                                    ((8, 2, 1, 128), (8, 2, 1, 128), 4095),
                                                    ((1, 32, 2048, 128), (1, 32, 2048, 128), 0),
                                                    ((1, 13, 2600, 128), (1, 13, 2000, 128), 7)])
def test_rope(gpu, interleaved, shape_q, shape_k, offset):
    """Includes config 4's prefill shape (32 heads x 2048 tokens) and unequal
    Q / K lengths at scale."""
    Q = RNG.standard_normal(shape_q).astype(np.float32)
    K = RNG.standard_normal(shape_k).astype(np.float32)
    gq, gk = g.rope(gpu, Q, K, position_offset=offset, interleaved=interleaved, theta=0.0)
    oq, ok = oracle.rope(Q, K, position_offset=offset, interleaved=interleaved, theta=10000.0)
    assert rel(gq, oq) <= 1e-4 and rel(gk, ok) <= 1e-4


def test_rope_positions_and_identity(gpu):
    Q = RNG.standard_normal((1, 2, 6, 8)).astype(np.float32)
    pos = np.array([0, 5, 2, 0, 9, 1], np.int32)
    gq, _ = g.rope(gpu, Q, None, positions=pos)
    oq, _ = oracle.rope(Q, None, positions=pos)
    assert rel(gq, oq) <= 1e-5
    assert np.array_equal(gq[:, :, 0], Q[:, :, 0])  # position 0 is the identity
    # pair norms are preserved
    h = 4
    n0 = Q[..., :h] ** 2 + Q[..., h:] ** 2
    n1 = gq[..., :h] ** 2 + gq[..., h:] ** 2
    assert np.allclose(n0, n1, rtol=1e-5, atol=1e-6)


# ---------------------------------------------------------------- attention
@pytest.mark.parametrize("b,h,sq,sk,d,causal,use_mask", [
    (1, 2, 5, 5, 16, 1, False), (1, 2, 33, 70, 16, 1, False), (1, 2, 16, 100, 16, 0, True),
    (1, 2, 1, 130, 16, 1, False), (1, 4, 300, 300, 128, 1, False), (2, 2, 1, 4096, 128, 1, False),
    (8, 32, 1, 4096, 128, 1, False),   # config-4 decode: batch 8, 32 heads, context 4096
    # decode kernel (seq_q <= 4, head_dim % 32 == 0): query counts, widths, masks
    (2, 3, 1, 777, 64, 1, True), (1, 2, 3, 300, 96, 1, False), (1, 2, 4, 1000, 256, 1, True),
    (2, 2, 2, 64, 32, 0, False), (1, 1, 4, 3, 160, 1, False), (3, 1, 1, 1, 128, 1, False),
    # prefill kernel (f32 MFMA, head_dim 64/128): ragged lengths, masks, offsets
    (2, 3, 129, 200, 64, 0, True), (1, 2, 256, 256, 128, 1, True), (1, 2, 100, 1000, 128, 1, False),
    (1, 1, 5, 5, 128, 1, False), (1, 2, 300, 120, 64, 1, False), (1, 1, 640, 640, 128, 1, False),
    (1, 1, 17, 9, 64, 1, False), (1, 2, 40, 40, 80, 0, False)])
@pytest.mark.parametrize("dev", ["gpu", "fast_gpu"])
def test_attention(request, dev, b, h, sq, sk, d, causal, use_mask):
    """Both device modes: the default (reference order) and high throughput
    (split-bf16 prefill, split decode, generic and row-wise kernels)."""
    gpu = request.getfixturevalue(dev)
    Q = RNG.standard_normal((b, h, sq, d)).astype(np.float32)
    K = RNG.standard_normal((b, h, sk, d)).astype(np.float32)
    V = RNG.standard_normal((b, h, sk, d)).astype(np.float32)
    mask = RNG.standard_normal((b, h, sq, sk)).astype(np.float32) if use_mask else None
    got = g.attention(gpu, Q, K, V, mask, causal)
    want = oracle.attention(Q, K, V, mask, causal)
    assert rel(got, want) <= 2e-3


@pytest.mark.parametrize("b,h,sq,sk,d,causal", [
    (1, 4, 512, 512, 128, 1), (1, 2, 300, 700, 64, 1), (2, 2, 256, 384, 128, 0)])
def test_attention_prefill_split_precision(fast_gpu, b, h, sq, sk, d, causal):
    """The prefill kernel's three-term bf16 products (hi*hi + hi*lo + lo*hi)
    against float64 softmax attention: about 2^-16 relative per product, so
    the result sits far below the 2e-3 bar (checked at 1e-4 here; the
    kernel's hardware exp contributes ~1e-5 of it)."""
    Q = RNG.standard_normal((b, h, sq, d)).astype(np.float32)
    K = RNG.standard_normal((b, h, sk, d)).astype(np.float32)
    V = RNG.standard_normal((b, h, sk, d)).astype(np.float32)
    got = g.attention(fast_gpu, Q, K, V, None, causal)
    s = np.einsum("bhqd,bhkd->bhqk", Q.astype(np.float64), K.astype(np.float64)) / np.sqrt(d)
    if causal:
        qi = np.arange(sq)[:, None] + (sk - sq if sk > sq else 0)
        s = np.where(np.arange(sk)[None, :] > qi, -np.inf, s)
    p = np.exp(s - s.max(-1, keepdims=True))
    want = np.einsum("bhqk,bhkd->bhqd", p / p.sum(-1, keepdims=True), V.astype(np.float64))
    assert rel(got, want) <= 1e-4


def test_attention_prefill_invariants(fast_gpu):
    # Split-bf16 prefill kernel (head_dim 128): V constant -> O constant (0.75
    # is exact in bf16, so only the weights' split error remains); causal
    # row 0 = V[0].
    gpu = fast_gpu
    Q = RNG.standard_normal((1, 2, 200, 128)).astype(np.float32)
    K = RNG.standard_normal((1, 2, 200, 128)).astype(np.float32)
    V = np.full((1, 2, 200, 128), 0.75, np.float32)
    assert np.allclose(g.attention(gpu, Q, K, V, None, 1), 0.75, atol=3e-5)
    V = RNG.standard_normal((1, 2, 200, 128)).astype(np.float32)
    O = g.attention(gpu, Q, K, V, None, 1)
    assert np.allclose(O[:, :, 0], V[:, :, 0], atol=3e-5 * np.abs(V).max())


@pytest.mark.parametrize("dev", ["gpu", "fast_gpu"])
def test_attention_invariants(request, dev):
    # V constant -> O constant; causal row 0 attends only key 0 -> O[0] = V[0].
    gpu = request.getfixturevalue(dev)
    Q = RNG.standard_normal((1, 2, 20, 32)).astype(np.float32)
    K = RNG.standard_normal((1, 2, 20, 32)).astype(np.float32)
    V = np.full((1, 2, 20, 32), 0.75, np.float32)
    assert np.allclose(g.attention(gpu, Q, K, V, None, 1), 0.75, atol=1e-6)
    V = RNG.standard_normal((1, 2, 20, 32)).astype(np.float32)
    O = g.attention(gpu, Q, K, V, None, 1)
    assert np.allclose(O[:, :, 0], V[:, :, 0], atol=1e-6)


# ---------------------------------------------------------------- runtime semantics
def test_host_pointer_staging(gpu):
    # The reference's tools pass host pointers everywhere: they are staged.
    M, K, N = 3, 130, 70
    X = RNG.standard_normal((M, K)).astype(np.float32)
    A8 = np.empty((M, K), np.int8)
    sa = np.empty(M, np.float32)
    Bq = RNG.integers(-128, 128, size=(K, N)).astype(np.int8)
    w = gpu.pack(Bq, K, N)
    Cout = np.empty((M, N), np.float32)
    p = lambda a: a.ctypes.data
    gpu.run(abi.OP_QUANTIZE_I8, X=p(X), Y=p(A8), scales=p(sa), rows=M, cols=K, axis=0)
    gpu.run(abi.OP_MATMUL_I8, A=p(A8), B=w, scale_a=p(sa), C=p(Cout), M=M, K=K, N=N)
    yo, so = oracle.quantize(X, 0)
    assert np.array_equal(A8, yo) and np.array_equal(sa, so)
    assert np.array_equal(Cout.view(np.uint32), oracle.matmul_i8(yo, Bq, so, None).view(np.uint32))
    gpu.release_packed(w)


def test_batch_event_and_sticky_error():
    from vnpu_mi355x import Session
    s = Session()
    try:
        ev = C.c_void_p()
        assert s.lib.vnpu_event_create(C.byref(ev)) == abi.OK
        assert s.lib.vnpu_event_wait(ev, 0) == abi.ERR_TIMEOUT  # never submitted
        nops = [s.command(abi.OP_NOP) for _ in range(8)]
        assert s.submit(nops, ev) == abi.OK
        assert s.lib.vnpu_event_wait(ev, 10000) == abi.OK
        assert s.lib.vnpu_event_query(ev) == abi.OK
        # ones(16x16) . ones(16x16) = 16 (reference selftest known answer)
        ones = s.upload(np.ones((16, 16), np.float32))
        out = s.alloc(16 * 16 * 4)
        s.run(abi.OP_MATMUL_F32, A=ones, B=ones, C=out, M=16, K=16, N=16)
        assert np.all(s.download(out, np.float32, (16, 16)) == 16.0)
        # invalid command: submit still OK, event carries the failure, sync is sticky
        bad = s.command(abi.OP_MATMUL_F32, A=None, B=None, C=None, M=0, K=0, N=0)
        assert s.submit([bad], ev) == abi.OK
        assert s.lib.vnpu_event_wait(ev, 10000) == abi.ERR_INTERNAL
        assert s.sync() == abi.ERR_DEVICE_ERROR
        assert s.sync() == abi.ERR_DEVICE_ERROR
        assert s.submit([s.command(99)], None) == abi.OK
        st = s.status()
        assert st.error != 0
        s.lib.vnpu_event_destroy(ev)
    finally:
        s.close()


def test_two_streams_concurrent(gpu):
    M, K, N = 192, 256, 256
    A = RNG.standard_normal((M, K)).astype(np.float32)
    B = RNG.standard_normal((K, N)).astype(np.float32)
    want = oracle.matmul_f32(A, B, acc64=True)
    s2 = C.c_void_p()
    assert gpu.lib.vnpu_stream_create(gpu.dev, 0, C.byref(s2)) == abi.OK
    ba, bb = gpu.upload(A), gpu.upload(B)
    outs = [gpu.alloc(M * N * 4) for _ in range(8)]
    cmds = [gpu.command(abi.OP_MATMUL_F32, A=ba, B=bb, C=o, M=M, K=K, N=N) for o in outs]
    arr1 = (abi.Command * 4)(*cmds[:4])
    arr2 = (abi.Command * 4)(*cmds[4:])
    assert gpu.lib.vnpu_stream_submit(gpu.stream, arr1, 4, None) == abi.OK
    assert gpu.lib.vnpu_stream_submit(s2, arr2, 4, None) == abi.OK
    assert gpu.lib.vnpu_stream_sync(s2) == abi.OK and gpu.sync() == abi.OK
    for o in outs:
        assert rel(gpu.download(o, np.float32, (M, N)), want) <= 1e-4
    gpu.lib.vnpu_stream_destroy(s2)


def test_backend_table_and_info(gpu):
    tbl = gpu.lib.vnpu_get_backend_v1()
    raw = (C.c_uint32 * 2).from_address(tbl)
    assert raw[0] == 1 and raw[1] == 416
    info = gpu.info()
    assert info.num_compute_units >= 1 and info.total_memory_bytes > 0
    assert b"gfx950" in info.cpu_arch
    assert gpu.lib.vnpu_mmio_read32(gpu.dev, 0) == 0x56504E55


def test_f32_bounded_wait_timeout_is_reported(monkeypatch):
    """The warp-specialised MATMUL_F32 kernel's producer/consumer waits are
    bounded.  With the bound forced down to one poll from the host
    (VNPU_WS_MAX_SPIN=1 at device creation) the first waits give up while
    the operands are still in flight: every wave still finishes (the waits
    end, all accesses stay in the ring and the matrices), the result is
    wrong, and the stream's sync reports it as a device error, sticky on
    that stream, with the device error register set.  A device created
    without the bound computes the same call correctly."""
    from vnpu_mi355x import Session
    M, K, N = 2048, 256, 4096     # 8 x 32 = 256 tiles of 256 x 128: the warp-specialised kernel
    A = RNG.standard_normal((M, K)).astype(np.float32)
    B = RNG.standard_normal((K, N)).astype(np.float32)
    monkeypatch.setenv("VNPU_WS_MAX_SPIN", "1")
    s = Session()
    monkeypatch.delenv("VNPU_WS_MAX_SPIN")
    try:
        ba, bb, bc = s.upload(A), s.upload(B), s.alloc(4 * M * N)
        assert s.sync() == abi.OK
        cmd = s.command(abi.OP_MATMUL_F32, A=ba, B=bb, C=bc, M=M, K=K, N=N, alpha=1.0)
        assert s.submit([cmd]) == abi.OK
        assert s.sync() == abi.ERR_DEVICE_ERROR
        assert s.sync() == abi.ERR_DEVICE_ERROR          # sticky
        assert s.status().error == (-abi.ERR_INTERNAL) & 0xffffffff
    finally:
        s.close()
    ok = Session()
    try:
        got = g.matmul_f32(ok, A, B, M, K, N)
        assert ok.sync() == abi.OK
    finally:
        ok.close()
    assert rel(got, oracle.matmul_f32_blas(A, B)) <= 1e-4


@pytest.mark.parametrize("M,K,N,density,epi,use_bias", [
    (512, 1024, 512, 0.3, 0, False),      # whole 512 x 64 tiles
    (700, 1024, 520, 0.25, 2, True),      # rows past M clamped, a partial last column group, bias, SiLU
    (1100, 2048, 200, 0.35, 3, True),     # GELU, 200 columns: the last group has 8 of 64 columns
    (512, 640, 256, 0.0, 1, True),        # every tile zero: the epilogue of the bias alone
    (600, 16384, 192, 0.2, 0, False),     # 256 k blocks: all four list registers
    (300, 512, 384, 0.9, 0, False),       # above the strip kernel's density: the dense kernels
    (512, 1024, 512, 0.5, 1, True),       # config 5's density: the dense kernels
])
def test_int8_zero_tile_strip_kernel(gpu, M, K, N, density, epi, use_bias):
    """Weights whose 64 x 64 tiles are zero with probability 1 - density (the
    config-5 geometry; one column group and one k block are zeroed entirely):
    packing lists each 64-column group's nonzero k blocks and, at most 40%
    of the tiles nonzero, the strip kernel walks only those.  The int32 accumulators, hence C without an exp-based
    activation, bit-exact with the oracle; SiLU and GELU within 1e-6 (their
    exp, as in the dense kernels' epilogue tests)."""
    A = RNG.integers(-128, 128, (M, K)).astype(np.int8)
    B = RNG.integers(-128, 128, (K, N)).astype(np.int8)
    groups = (N + 63) // 64
    keep = (RNG.random((K // 64, groups)) < density).astype(np.int8)
    if density > 0:
        keep[:, 0] = 0          # a column group without any nonzero tile
        keep[K // 128, :] = 0   # a k block zero in every group
    B *= np.kron(keep, np.ones((64, 64), np.int8))[:, :N]
    sa = (RNG.random(M).astype(np.float32) + 0.5) / 127
    sb = (RNG.random(N).astype(np.float32) + 0.5) / 127
    bias = RNG.standard_normal(N).astype(np.float32) if use_bias else None
    w = gpu.pack(B, K, N, scales=sb)
    try:
        got = g.matmul_i8(gpu, A, w, M, K, N, scale_a=sa, bias=bias, epilogue=epi)
    finally:
        gpu.release_packed(w)
    want = oracle.matmul_i8_blas(A, B, sa, sb, bias, epi)
    if epi in (abi.EPI_NONE, abi.EPI_RELU):
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    else:
        assert rel(got, want) <= 1e-6


@pytest.mark.parametrize("M,K,N,density,trans_b,ldb,mask_ld,on_device", [
    (512, 1024, 512, 0.25, 0, 0, 0, False),      # strip kernel density, host mask
    (512, 1024, 512, 0.5, 0, 0, 0, True),        # config 5's density (dense kernels), device mask
    (300, 1000, 520, 0.3, 1, 1003, 11, False),   # ragged K and N (partial tiles), trans_b, ldb > K, mask_ld > groups
    (8, 4096, 4096, 0.5, 0, 0, 0, False),        # decode GEMV over culled weights
    (64, 640, 200, 0.0, 0, 0, 5, True),          # every tile culled
])
def test_pack_weights_i8_masked(gpu, M, K, N, density, trans_b, ldb, mask_ld, on_device):
    """vnpu_pack_weights_i8_masked: the weights are dense random int8, the
    Wildcat 64 x 64 weight-tile mask is passed in, and every MATMUL_I8 with
    the packed weights equals the oracle's on B with the culled tiles zeroed
    (bit-exact), with the culled weights' column sums, on whichever kernel
    the shape and density select."""
    Bl = RNG.integers(-128, 128, (K, N)).astype(np.int8)          # logical K x N
    A = RNG.integers(-128, 128, (M, K)).astype(np.int8)
    rows, groups = (K + 63) // 64, (N + 63) // 64
    ld_m = mask_ld or groups
    mask = np.full((rows, ld_m), 7, np.uint8)                     # bytes past the groups are ignored
    mask[:, :groups] = (RNG.random((rows, groups)) < density).astype(np.uint8) * 3
    culled = np.kron((mask[:, :groups] != 0).astype(np.int8), np.ones((64, 64), np.int8))[:K, :N]
    if trans_b:
        ld = ldb or K
        Bs = np.zeros((N, ld), np.int8)
        Bs[:, :K] = Bl.T
    else:
        ld = ldb or N
        Bs = np.zeros((K, ld), np.int8)
        Bs[:, :N] = Bl
    sa = (RNG.random(M).astype(np.float32) + 0.5) / 127
    sb = (RNG.random(N).astype(np.float32) + 0.5) / 127
    mbuf = gpu.upload(mask) if on_device else None
    w = gpu.pack(Bs, K, N, scales=sb, ldb=ldb, trans_b=trans_b,
                 tile_mask=mbuf if on_device else mask, mask_ld=ld_m)
    try:
        got = g.matmul_i8(gpu, A, w, M, K, N, scale_a=sa)
        _, _, _, _, sums = gpu.unpack_info(w)
    finally:
        gpu.release_packed(w)
        if mbuf is not None:
            gpu.free(mbuf)
    Bm = Bl * culled
    assert np.array_equal(sums, Bm.astype(np.int64).sum(axis=0).astype(np.int32))
    want = oracle.matmul_i8_blas(A, Bm, sa, sb, None, 0)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    if 0 < density < 1:
        assert not np.array_equal(want, oracle.matmul_i8_blas(A, Bl, sa, sb, None, 0))


def test_pack_weights_i8_masked_rejects_short_mask_ld(gpu):
    B = np.ones((128, 200), np.int8)
    mask = np.ones((2, 4), np.uint8)
    w = C.c_void_p()
    st = gpu.lib.vnpu_pack_weights_i8_masked(gpu.dev, B.ctypes.data_as(C.c_void_p), None, 128, 200, 0, 0,
                                             mask.ctypes.data_as(C.c_void_p), 3, C.byref(w))
    assert st == abi.ERR_INVALID_ARGUMENT and not w.value
    # NULL mask: vnpu_pack_weights_i8
    st = gpu.lib.vnpu_pack_weights_i8_masked(gpu.dev, B.ctypes.data_as(C.c_void_p), None, 128, 200, 0, 0,
                                             None, 0, C.byref(w))
    assert st == abi.OK and w.value
    gpu.lib.vnpu_packed_weights_destroy(w)
