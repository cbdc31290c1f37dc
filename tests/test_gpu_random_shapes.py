"""Seeded random shapes through the batch-level paths of the MI355X backend:
row chains (ADD -> RMSNORM -> QUANTIZE_I8, RMSNORM -> QUANTIZE_I8,
SWIGLU -> QUANTIZE_I8) at random rows, columns and aliasing must give the
bits of the same commands submitted one per batch, and pairs of MATMUL_I8
commands at M <= 8 with random K and N the oracle's bits (reference
src/kernels/kernels.cpp:922-978 accumulation and store_i8_c order)."""
import numpy as np
import pytest

import gpu_ops as g
import oracle
import test_gpu_rowchain as rc
from vnpu_mi355x import abi

pytestmark = pytest.mark.gpu


def test_random_row_chains(gpu):
    rng = np.random.default_rng(20261208)
    for _ in range(40):
        kind = rc.KINDS[rng.integers(4)]
        rows = int(rng.integers(1, 200))
        cols = 4 * int(rng.integers(1, 3200))   # past 12288 columns: commands one by one
        alias = bool(rng.integers(2))
        p = rc._params(kind, rows, cols)
        fused = rc._run(gpu, kind, rows, cols, alias, True, p)
        single = rc._run(gpu, kind, rows, cols, alias, False, p)
        for k in fused:
            assert np.array_equal(fused[k].view(np.uint8), single[k].view(np.uint8)), (kind, rows, cols, alias, k)


def test_random_matmul_i8_pairs_small_m(gpu):
    rng = np.random.default_rng(20261209)
    for _ in range(24):
        M, K = int(rng.integers(1, 9)), int(rng.integers(1, 3000))
        N0 = int(rng.integers(1, 20000))
        N1 = N0 if rng.integers(2) else int(rng.integers(1, 20000))
        A = rng.integers(-128, 128, size=(M, K)).astype(np.int8)
        Bs = [rng.integers(-128, 128, size=(K, n)).astype(np.int8) for n in (N0, N1)]
        sa = (rng.random(M).astype(np.float32) + 0.5) / 127
        ss = [(rng.random(n).astype(np.float32) + 0.5) / 127 for n in (N0, N1)]
        ws = [gpu.pack(B, K, n, scales=s) for B, n, s in zip(Bs, (N0, N1), ss)]
        ba, bsa = gpu.upload(A), gpu.upload(sa)
        cs = [gpu.alloc(4 * M * n) for n in (N0, N1)]
        cmds = [gpu.command(abi.OP_MATMUL_I8, A=ba, B=w, scale_a=bsa.ptr, C=c, M=M, K=K, N=n)
                for w, c, n in zip(ws, cs, (N0, N1))]
        assert gpu.submit(cmds) == abi.OK and gpu.sync() == abi.OK
        got = [gpu.download(c, np.float32, (M, n)) for c, n in zip(cs, (N0, N1))]
        for b in [ba, bsa] + cs:
            gpu.free(b)
        for w in ws:
            gpu.release_packed(w)
        for g_, B, s in zip(got, Bs, ss):
            want = oracle.matmul_i8(A, B, sa, s)
            assert np.array_equal(g_.view(np.uint32), want.view(np.uint32)), (M, K, N0, N1)


def test_random_attention_both_devices(gpu, fast_gpu):
    """Seeded random ATTENTION_F32 calls (reference src/kernels/llm.cpp:442-546):
    batch, heads, query and key lengths (decode and prefill paths, ragged
    64-key blocks and 128-row tiles), head sizes 64 and 128 (the tiled
    kernels) and others (the row-wise kernel), causal offsets, additive masks
    with -inf runs, explicit and default scales.  The default device must give
    the reference's bits (the oracle's AVX2-order restatement); the
    high-throughput device must be within the attention bar."""
    rng = np.random.default_rng(20261210)
    for case in range(24):
        b, h = int(rng.integers(1, 3)), int(rng.integers(1, 4))
        d = int(rng.choice([64, 128, 128, 64, 32, 80]))
        sq = int(rng.choice([1, 2, 4])) if rng.integers(3) == 0 else int(rng.integers(5, 300))
        sk = sq + int(rng.integers(0, 400))
        causal = int(rng.integers(2))
        scale = 0.0 if rng.integers(2) else float(rng.uniform(0.02, 0.3))
        Q = (rng.standard_normal((b, h, sq, d)) * rng.uniform(0.5, 3)).astype(np.float32)
        K = rng.standard_normal((b, h, sk, d)).astype(np.float32)
        V = rng.standard_normal((b, h, sk, d)).astype(np.float32)
        M = None
        if rng.integers(3) == 0:
            M = rng.standard_normal((b, h, sq, sk)).astype(np.float32)
            lo = int(rng.integers(0, sk))
            M[..., lo:lo + int(rng.integers(1, 80))] = -np.inf
        what = (case, b, h, sq, sk, d, causal, scale, M is not None)
        want = oracle.attention_avx2(Q, K, V, M, causal, scale)
        got = g.attention(gpu, Q, K, V, M, causal, scale)
        same = (got.view(np.uint32) == want.view(np.uint32)) | (np.isnan(got) & np.isnan(want))
        assert same.all(), what
        fast = g.attention(fast_gpu, Q, K, V, M, causal, scale)
        assert oracle.rel_error(fast, want) <= 2e-3, what



def test_random_reference_order_small_shapes(gpu):
    """Seeded random short rows and odd head sizes, where every rounding of
    the reference's AVX2 build shows: RMSNORM (reduction tails of any length),
    SWIGLU/MUL/ADD/GELU (scalar tails) and ATTENTION with head sizes 1..39
    (the row-wise kernel's dot tails), each bit-exact with the oracle's
    AVX2-order restatement."""
    rng = np.random.default_rng(20261211)

    def same(a, b):
        return np.array_equal(a.view(np.uint32), b.view(np.uint32))

    for _ in range(40):
        rows, cols = int(rng.integers(1, 300)), int(rng.integers(1, 80))
        X = (rng.standard_normal((rows, cols)) * rng.uniform(0.1, 10)).astype(np.float32)
        W = (1 + 0.1 * rng.standard_normal(cols)).astype(np.float32)
        assert same(g.unary_rows(gpu, abi.OP_RMSNORM_F32, X, W=W, eps=1e-5), oracle.rmsnorm_avx2(X, W, 1e-5)), \
            (rows, cols)
        n = int(rng.integers(1, 200))
        a = (rng.standard_normal(n) * rng.uniform(0.1, 30)).astype(np.float32)
        b = rng.standard_normal(n).astype(np.float32)
        al, be = float(rng.choice([0.0, 1.0, -1.5])), float(rng.choice([0.0, 2.5]))
        assert same(g.elementwise(gpu, abi.OP_SWIGLU_F32, a, b, alpha=al), oracle.swiglu_avx2(a, b, al or 1.0)), n
        assert same(g.elementwise(gpu, abi.OP_MUL_F32, a, b, al, be), oracle.mul_avx2(a, b, al or 1.0, be)), n
        assert same(g.elementwise(gpu, abi.OP_ADD_F32, a, b, al, be), oracle.add_avx2(a, b, al, be)), n
        assert same(g.elementwise(gpu, abi.OP_GELU_F32, a), oracle.gelu_avx2(a)), n
    for _ in range(24):
        h, d = int(rng.integers(1, 3)), int(rng.integers(1, 40))
        sq = int(rng.integers(1, 40))
        sk = sq + int(rng.integers(0, 140))
        causal = int(rng.integers(2))
        Q = (rng.standard_normal((1, h, sq, d)) * rng.uniform(0.5, 3)).astype(np.float32)
        K = rng.standard_normal((1, h, sk, d)).astype(np.float32)
        V = rng.standard_normal((1, h, sk, d)).astype(np.float32)
        assert same(g.attention(gpu, Q, K, V, None, causal), oracle.attention_avx2(Q, K, V, None, causal)), \
            (h, sq, sk, d, causal)


def test_random_masked_pack_matmul_i8(gpu):
    """Seeded random vnpu_pack_weights_i8_masked calls: random K, N, kept-tile
    density (from all tiles culled to none), trans_b and padded mask rows,
    then MATMUL_I8 at decode and prefill row counts (the GEMV, the dense
    GEMM kernels and, at low density, the kernel that walks only nonzero
    tiles): bit-exact with the oracle on the weights with the culled 64 x 64
    tiles zeroed, column sums included."""
    rng = np.random.default_rng(20261210)
    for it in range(16):
        M = int(rng.choice([1, 5, 8, 64, 300, 512]))
        K = int(64 * rng.integers(1, 48)) if rng.integers(2) else int(rng.integers(1, 3000))
        N = int(rng.integers(1, 3000))
        density = float(rng.choice([0.0, 0.1, 0.3, 0.5, 0.9, 1.0]))
        trans_b = int(rng.integers(2))
        rows, groups = (K + 63) // 64, (N + 63) // 64
        mask_ld = groups + int(rng.integers(0, 3))
        mask = np.zeros((rows, mask_ld), np.uint8)
        mask[:, :groups] = rng.random((rows, groups)) < density
        Bl = rng.integers(-128, 128, size=(K, N)).astype(np.int8)
        A = rng.integers(-128, 128, size=(M, K)).astype(np.int8)
        sa = (rng.random(M).astype(np.float32) + 0.5) / 127
        sb = (rng.random(N).astype(np.float32) + 0.5) / 127
        w = gpu.pack(np.ascontiguousarray(Bl.T) if trans_b else Bl, K, N, scales=sb, trans_b=trans_b,
                     tile_mask=mask, mask_ld=mask_ld)
        try:
            got = g.matmul_i8(gpu, A, w, M, K, N, scale_a=sa)
            sums = gpu.unpack_info(w)[4]
        finally:
            gpu.release_packed(w)
        Bm = Bl * np.kron(mask[:, :groups], np.ones((64, 64), np.uint8))[:K, :N].astype(np.int8)
        case = (it, M, K, N, density, trans_b, mask_ld)
        assert np.array_equal(sums, Bm.astype(np.int64).sum(axis=0).astype(np.int32)), case
        want = oracle.matmul_i8_blas(A, Bm, sa, sb, None, 0)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), case
