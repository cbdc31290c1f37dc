"""Pins the C oracle against the reference runtime built from its own sources.

The reference (oracle/_ref/libvnpu_ref.so, compiled by oracle/Makefile from
the reference tree with its own flags) is driven through its C ABI exactly
like the GPU backend.  Integer results must match bit for bit; float results
within the reference's own conformance metric (tools/conformance.cpp:95-103).
Skipped when the reference build is absent.
"""
import numpy as np
import pytest

import oracle
import gpu_ops as g
from vnpu_mi355x import abi

RNG = np.random.default_rng(1234)


def tie_matrix(rows, cols):
    """Rows whose quantized values hit exact .5 ties: max 127 -> scale 1."""
    X = RNG.integers(-100, 100, size=(rows, cols)).astype(np.float32) + 0.5
    X[:, 0] = 127.0
    return X


@pytest.mark.parametrize("shape", [(1, 1), (3, 7), (17, 300), (64, 512), (5, 4099)])
@pytest.mark.parametrize("axis", [0, 1, 2])
def test_quantize_bit_exact(ref, shape, axis):
    X = RNG.standard_normal(shape).astype(np.float32) * 3
    yr, sr = g.quantize(ref, X, axis)
    yo, so = oracle.quantize(X, axis)
    assert np.array_equal(yr, yo)
    assert np.array_equal(sr.view(np.uint32), so.view(np.uint32))


@pytest.mark.parametrize("axis", [0, 1, 2])
def test_quantize_ties_zero_and_nonfinite(ref, axis):
    X = tie_matrix(8, 33)
    X[2] = 0.0                       # zero row -> scale 1, all zero
    X[3, 5] = np.inf                 # inf -> scale 1, clamps to 127
    X[4, 7] = np.nan                 # NaN ignored by max, quantizes to 0
    X[5, 1] = -np.inf
    yr, sr = g.quantize(ref, X, axis)
    yo, so = oracle.quantize(X, axis)
    assert np.array_equal(yr, yo)
    assert np.array_equal(sr.view(np.uint32), so.view(np.uint32))


def test_quantize_ties_round_away_from_zero():
    # Closed form: scale exactly 1 (max 127) and x = k + 0.5 -> away from zero.
    X = np.array([[127.0, 0.5, -0.5, 1.5, -1.5, 2.5, -126.5]], np.float32)
    y, s = oracle.quantize(X, 0)
    assert s[0] == np.float32(1.0)
    assert y.tolist() == [[127, 1, -1, 2, -2, 3, -127]]


@pytest.mark.parametrize("K,N,trans_b", [(37, 29, 0), (64, 16, 0), (100, 70, 1), (5, 300, 0)])
def test_pack_column_sums_and_scales(ref, K, N, trans_b):
    B = RNG.integers(-128, 128, size=(N, K) if trans_b else (K, N)).astype(np.int8)
    scales = RNG.random(N).astype(np.float32) + 0.1
    w = ref.pack(B, K, N, scales=scales, trans_b=trans_b)
    k, n, _, sc, cs = ref.unpack_info(w)
    orig, sums = oracle.pack_canonical(B, K, N, 0, trans_b)
    assert (k, n) == (K, N)
    assert np.array_equal(cs, sums)
    assert np.array_equal(sc, scales)
    # closed form
    assert np.array_equal(sums, orig.astype(np.int64).sum(axis=0).astype(np.int32))


@pytest.mark.parametrize("M,K,N", [(1, 64, 32), (2, 300, 200), (3, 257, 1100), (8, 512, 64),
                                   (17, 300, 200), (64, 128, 96)])
def test_matmul_i8_bit_exact(ref, M, K, N):
    A = RNG.integers(-128, 128, size=(M, K)).astype(np.int8)
    B = RNG.integers(-128, 128, size=(K, N)).astype(np.int8)
    sa = (RNG.random(M).astype(np.float32) + 0.5) / 127
    sb = (RNG.random(N).astype(np.float32) + 0.5) / 127
    w = ref.pack(B, K, N, scales=sb)
    got = g.matmul_i8(ref, A, w, M, K, N, scale_a=sa)
    want = oracle.matmul_i8(A, B, sa, sb)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    # the integer core against brute force
    acc = oracle.gemm_i8_acc(A, B)
    assert np.array_equal(acc, (A.astype(np.int64) @ B.astype(np.int64)).astype(np.int32))


@pytest.mark.parametrize("epi", [0, 1, 2, 3, 4])
def test_matmul_i8_bias_epilogue(ref, epi):
    M, K, N = 5, 96, 40
    A = RNG.integers(-128, 128, size=(M, K)).astype(np.int8)
    B = RNG.integers(-128, 128, size=(K, N)).astype(np.int8)
    sa = RNG.random(M).astype(np.float32) / 127
    sb = RNG.random(N).astype(np.float32) / 127
    bias = RNG.standard_normal(N).astype(np.float32)
    w = ref.pack(B, K, N, scales=sb)
    got = g.matmul_i8(ref, A, w, M, K, N, scale_a=sa, bias=bias, epilogue=epi)
    want = oracle.matmul_i8(A, B, sa, sb, bias, epi)
    assert oracle.rel_error(got, want) <= 1e-6


@pytest.mark.parametrize("M,K,N,ta,tb", [(37, 53, 29, 0, 0), (17, 41, 23, 0, 1), (9, 33, 18, 1, 0),
                                         (1, 512, 137, 0, 0), (64, 128, 64, 0, 1)])
@pytest.mark.parametrize("epi,beta", [(0, 0.0), (2, 0.0), (3, 0.5), (1, 0.0)])
def test_matmul_f32(ref, M, K, N, ta, tb, epi, beta):
    A = RNG.standard_normal((K, M) if ta else (M, K)).astype(np.float32)
    B = RNG.standard_normal((N, K) if tb else (K, N)).astype(np.float32)
    bias = RNG.standard_normal(N).astype(np.float32)
    C0 = RNG.standard_normal((M, N)).astype(np.float32)
    got = g.matmul_f32(ref, A, B, M, K, N, C_in=C0, bias=bias, trans_a=ta, trans_b=tb, beta=beta,
                       epilogue=epi)
    want = oracle.matmul_f32(A, B, C0, bias, M, K, N, ta, tb, 1.0, beta, epi, acc64=True)
    # K <= 128 keeps the reference's packed path on its documented semantics
    assert oracle.rel_error(got, want) <= 1e-4


def test_rmsnorm_softmax_elementwise(ref):
    X = RNG.standard_normal((7, 300)).astype(np.float32)
    W = RNG.standard_normal(300).astype(np.float32)
    assert oracle.rel_error(g.unary_rows(ref, abi.OP_RMSNORM_F32, X, W=W, eps=1e-5),
                            oracle.rmsnorm(X, W, 1e-5)) <= 1e-5
    assert oracle.rel_error(g.unary_rows(ref, abi.OP_SOFTMAX_F32, X, temperature=0.7),
                            oracle.softmax(X, 0.7)) <= 1e-5
    a = RNG.standard_normal(1001).astype(np.float32)
    b = RNG.standard_normal(1001).astype(np.float32)
    assert oracle.rel_error(g.elementwise(ref, abi.OP_SWIGLU_F32, a, b, alpha=1.5),
                            oracle.swiglu(a, b, 1.5)) <= 1e-5
    assert oracle.rel_error(g.elementwise(ref, abi.OP_GELU_F32, a), oracle.gelu(a)) <= 1e-5
    assert oracle.rel_error(g.elementwise(ref, abi.OP_ADD_F32, a, b, 0.0, 0.0),
                            oracle.add(a, b, 1.0, 1.0)) <= 1e-6
    assert oracle.rel_error(g.elementwise(ref, abi.OP_MUL_F32, a, b, 2.0, 0.25),
                            oracle.mul(a, b, 2.0, 0.25)) <= 1e-6


@pytest.mark.parametrize("interleaved", [0, 1])
def test_rope(ref, interleaved):
    Q = RNG.standard_normal((2, 3, 40, 16)).astype(np.float32)
    K = RNG.standard_normal((2, 3, 24, 16)).astype(np.float32)
    gq, gk = g.rope(ref, Q, K, position_offset=100, interleaved=interleaved, theta=10000.0)
    oq, ok = oracle.rope(Q, K, position_offset=100, interleaved=interleaved, theta=10000.0)
    assert oracle.rel_error(gq, oq) <= 1e-5 and oracle.rel_error(gk, ok) <= 1e-5


@pytest.mark.parametrize("sq,sk,causal,use_mask", [(5, 5, 1, False), (33, 70, 1, False),
                                                   (16, 100, 0, True), (1, 130, 1, False)])
def test_attention(ref, sq, sk, causal, use_mask):
    Q = RNG.standard_normal((1, 2, sq, 16)).astype(np.float32)
    K = RNG.standard_normal((1, 2, sk, 16)).astype(np.float32)
    V = RNG.standard_normal((1, 2, sk, 16)).astype(np.float32)
    mask = RNG.standard_normal((1, 2, sq, sk)).astype(np.float32) if use_mask else None
    got = g.attention(ref, Q, K, V, mask, causal)
    want = oracle.attention(Q, K, V, mask, causal)
    assert oracle.rel_error(got, want) <= 2e-3


@pytest.mark.parametrize("M,N,unit", [(256, 512, 2), (40, 96, 2), (128, 128, 1), (300, 200, 3)])
def test_wildcat_cull_geometry(ref, M, N, unit):
    """The reference's culled region equals the oracle's restated geometry."""
    K = 8
    mask = oracle_mask = RNG.integers(0, 2, size=(4, 6)).astype(np.uint8)
    A = RNG.standard_normal((M, K)).astype(np.float32)
    B = RNG.standard_normal((K, N)).astype(np.float32)
    # No bias: a culled element is epi(0) = 0 exactly; a computed one is a
    # dot product of normals, never exactly 0 in practice.
    got = g.matmul_f32(ref, A, B, M, K, N, mask=mask, unit=unit)
    info = ref.info()
    cull, _ = oracle.cull_map(M, N, unit, info.tile_m, info.tile_n, info.num_threads, 1, oracle_mask)
    want = oracle.matmul_f32(A, B, None, None, M, K, N, 0, 0, 1.0, 0.0, 0, cull=cull)
    assert np.array_equal(got == 0.0, cull.astype(bool))
    assert oracle.rel_error(got, want) <= 1e-4


def _ref_session(env):
    """A reference device created under extra environment settings (read by
    the reference at device creation, src/core/runtime.cpp:889-903)."""
    import os
    from vnpu_mi355x import Session
    saved = {k: os.environ.get(k) for k in env}
    os.environ.update(env)
    try:
        cfg = abi.Config()
        cfg.abi_version = 1
        cfg.num_threads = 4
        return Session(oracle.REF_LIB_PATH, cfg)
    finally:
        for k, v in saved.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v


def test_matmul_f32_config1_epilogue_and_packed_defect(ref):
    """Config 1's MATMUL_F32 (512^3, bias, alpha 1, beta 0, SiLU).

    With VNPU_PACK=0 the reference computes the documented
    silu(A.B + bias), which the oracle restates.  Its default packed AVX2
    path (src/kernels/kernels.cpp:313-323) applies the epilogue after the
    first 128-deep K block only; this test records that the defect is real
    at this shape, and why the oracle does not follow the default path.
    """
    rng = np.random.default_rng(99)
    M = K = N = 512
    A = rng.standard_normal((M, K)).astype(np.float32)
    B = (0.02 * rng.standard_normal((K, N))).astype(np.float32)
    bias = (0.1 * rng.standard_normal(N)).astype(np.float32)
    want = oracle.matmul_f32(A, B, None, bias, M, K, N, 0, 0, 1.0, 0.0, abi.EPI_SILU)
    exact = oracle.matmul_f32(A, B, None, bias, M, K, N, 0, 0, 1.0, 0.0, abi.EPI_SILU,
                              acc64=True)
    assert oracle.rel_error(want, exact) <= 1e-5
    unpacked = _ref_session({"VNPU_PACK": "0"})
    try:
        got = g.matmul_f32(unpacked, A, B, M, K, N, bias=bias, epilogue=abi.EPI_SILU)
    finally:
        unpacked.close()
    assert oracle.rel_error(got, want) <= 1e-4
    packed = g.matmul_f32(ref, A, B, M, K, N, bias=bias, epilogue=abi.EPI_SILU)
    assert oracle.rel_error(packed, want) > 1e-2


# ---------------------------------------------------------------- AVX2 order
# The reference on an AVX2 host runs its AVX2 builds of these ops; the
# oracle's *_avx2 restatements follow their order of roundings and must
# equal the reference build bit for bit (the GPU kernels are then held to
# the same bits).

def _bits(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


@pytest.mark.parametrize("rows,cols", [(7, 4096), (3, 4099), (5, 33), (2, 11008), (2, 7), (1, 20000)])
def test_rmsnorm_avx2_order_bit_exact(ref, rows, cols):
    X = RNG.standard_normal((rows, cols)).astype(np.float32) * 2
    W = (1.0 + 0.1 * RNG.standard_normal(cols)).astype(np.float32)
    assert _bits(g.unary_rows(ref, abi.OP_RMSNORM_F32, X, W=W, eps=1e-5), oracle.rmsnorm_avx2(X, W, 1e-5))
    assert _bits(g.unary_rows(ref, abi.OP_RMSNORM_F32, X, eps=0.0), oracle.rmsnorm_avx2(X, None, 1e-5))


@pytest.mark.parametrize("cols", [1, 2, 3, 4, 5, 6, 7, 9, 11, 12, 13, 15, 20, 31, 4100, 4103])
def test_rmsnorm_avx2_tail_forms(ref, cols):
    """The sum of squares' scalar tail as the reference's build compiles it:
    with four or more tail elements the first four products are rounded (a
    4-wide vector epilogue) and added in order, the rest fused; a shorter
    tail is all fused.  Short rows make every rounding visible (many rows of
    7 differ between the all-fused form and the reference)."""
    X = (RNG.standard_normal((256 if cols < 100 else 16, cols)) * 2).astype(np.float32)
    W = (1.0 + 0.1 * RNG.standard_normal(cols)).astype(np.float32)
    assert _bits(g.unary_rows(ref, abi.OP_RMSNORM_F32, X, W=W, eps=1e-5), oracle.rmsnorm_avx2(X, W, 1e-5))
    assert _bits(g.unary_rows(ref, abi.OP_RMSNORM_F32, X, eps=0.0), oracle.rmsnorm_avx2(X, None, 1e-5))


@pytest.mark.parametrize("d", [3, 5, 6, 7, 12, 13, 15, 21, 23])
def test_attention_avx2_dot_tail_forms(ref, d):
    """dot_avx2's scalar tail, compiled like the sum of squares above (head
    sizes that leave 1..7 elements after the 8-wide steps)."""
    Q = (RNG.standard_normal((2, 2, 9, d)) * 2).astype(np.float32)
    K = RNG.standard_normal((2, 2, 40, d)).astype(np.float32)
    V = RNG.standard_normal((2, 2, 40, d)).astype(np.float32)
    got = g.attention(ref, Q, K, V, None, 1)
    assert _bits(got, oracle.attention_avx2(Q, K, V, None, 1))


@pytest.mark.parametrize("n", [3, 8, 1001, 4103, 16384, 2048 * 11008 // 32])
def test_elementwise_avx2_order_bit_exact(ref, n):
    """SWIGLU, GELU, ADD and MUL: 8-wide steps, then the last n % 8 elements in
    the scalar tail (MUL contracts differently there, SWIGLU's exp is not
    clamped there).  At these sizes the reference's ranges (max(4096, n / 16)
    elements at 4 threads) are multiples of 8, so only the last range has a
    tail."""
    a = (RNG.standard_normal(n) * 4).astype(np.float32)
    b = RNG.standard_normal(n).astype(np.float32)
    edges = np.array([90.0, -90.0, 80.0, -80.0, 80.5, -80.5, 0.0, -0.0, -88.0, -87.5], np.float32)   # exp's clamp
    a[: min(n, 8)] = edges[: min(n, 8)]
    a[-min(n, 3):] = edges[-min(n, 3):]   # the scalar tail too
    for al, be in ((0.0, 0.0), (0.5, 0.25), (-1.75, 3.0)):
        assert _bits(g.elementwise(ref, abi.OP_SWIGLU_F32, a, b, alpha=al), oracle.swiglu_avx2(a, b, al or 1.0))
        assert _bits(g.elementwise(ref, abi.OP_ADD_F32, a, b, al, be), oracle.add_avx2(a, b, al, be))
        assert _bits(g.elementwise(ref, abi.OP_MUL_F32, a, b, al, be), oracle.mul_avx2(a, b, al or 1.0, be))
    assert _bits(g.elementwise(ref, abi.OP_GELU_F32, a), oracle.gelu_avx2(a))


@pytest.mark.parametrize("n", [70001, 100004])
def test_elementwise_avx2_ranges_bit_exact(ref, n):
    """Above 16384 * num_threads elements the reference splits a command into
    ranges of max(4096, n / (4 * num_threads)) elements; at 4 threads these
    sizes give ranges that are not multiples of 8, so every range ends in a
    scalar tail of its own (SWIGLU's unclamped exp, MUL's other contraction)."""
    grain = oracle.ew_grain(n, 4)
    assert grain % 8 != 0 and n > grain
    a = (RNG.standard_normal(n) * 4).astype(np.float32)
    b = RNG.standard_normal(n).astype(np.float32)
    for end in list(range(grain, n, grain)) + [n]:
        a[end - 3:end] = (-90.0, -85.0, -81.0)     # exp's clamp edges in each range's tail
    for al, be in ((0.0, 0.0), (-1.75, 3.0)):
        sw = g.elementwise(ref, abi.OP_SWIGLU_F32, a, b, alpha=al)
        mu = g.elementwise(ref, abi.OP_MUL_F32, a, b, al, be)
        assert _bits(sw, oracle.swiglu_avx2(a, b, al or 1.0, num_threads=4))
        assert _bits(mu, oracle.mul_avx2(a, b, al or 1.0, be, num_threads=4))
        # one range (only the last n % 8 in a tail) is not the reference's result
        assert not _bits(sw, oracle.swiglu_avx2(a, b, al or 1.0))
        if al:   # alpha 1, beta 0: both of MUL's contractions are the exact product
            assert not _bits(mu, oracle.mul_avx2(a, b, al or 1.0, be))
        assert _bits(g.elementwise(ref, abi.OP_ADD_F32, a, b, al, be), oracle.add_avx2(a, b, al, be))
    assert _bits(g.elementwise(ref, abi.OP_GELU_F32, a), oracle.gelu_avx2(a))


def test_rope_bit_exact(ref):
    Q = RNG.standard_normal((2, 3, 50, 128)).astype(np.float32)
    K = RNG.standard_normal((2, 3, 40, 128)).astype(np.float32)
    for offset in (0, 4095):
        gq, gk = g.rope(ref, Q, K, position_offset=offset)
        oq, ok = oracle.rope(Q, K, position_offset=offset)
        assert _bits(gq, oq) and _bits(gk, ok)


@pytest.mark.parametrize("b,h,sq,sk,d,causal,mask", [
    (2, 2, 100, 300, 128, 1, None), (1, 3, 1, 4096, 128, 1, None), (2, 2, 37, 70, 20, 0, "normal"),
    (1, 2, 5, 130, 64, 1, "inf"), (1, 1, 16, 16, 64, 1, "row"), (1, 2, 3, 200, 96, 0, "inf")])
def test_attention_avx2_order_bit_exact(ref, b, h, sq, sk, d, causal, mask):
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
    got = g.attention(ref, Q, K, V, M, causal)
    assert _bits(got, oracle.attention_avx2(Q, K, V, M, causal))


@pytest.mark.parametrize("rows,cols,temp", [(4, 32000, 1.0), (3, 4099, 0.7), (5, 33, 1.0), (2, 7, 2.0),
                                            (1, 20000, 0.0), (6, 64, 1.5)])
def test_softmax_avx2_order_bit_exact(ref, rows, cols, temp):
    """SOFTMAX_F32 as the reference's AVX2 build computes it: per-lane maxima
    and sums over 8-wide steps, hsum256, the scalar tail, exp256's clamp to
    [-80, 80] (a logit 90 below the max keeps exp(-80), not 0, in the 8-wide
    part; the tail's scalar exp gives 0), -inf logits and a NaN row (a NaN
    element resets its lane's running max)."""
    X = (RNG.standard_normal((rows, cols)) * 4).astype(np.float32)
    X[0, 0] = 40.0
    X[0, 1] = -60.0             # 100 below the max: clamped in the 8-wide part
    X[0, cols - 1] = -60.0      # and in the tail (when cols % 8 != 0)
    if rows > 1:
        X[1, 3] = -np.inf
        X[1, cols - 1] = -np.inf
    if rows > 2 and cols > 16:
        X[2, 5] = np.nan        # lane 5's max restarts after it
        X[2, 13] = -3.0
    got = g.unary_rows(ref, abi.OP_SOFTMAX_F32, X, temperature=temp)
    want = oracle.softmax_avx2(X, temp)
    assert _bits(got, want)
    if rows > 1 and cols % 8 == 0:
        assert want[1, 3] > 0.0   # exp(-80) of the clamp, as the reference


def test_avx2_orders_random_sweep(ref):
    """Seeded random small shapes through every AVX2-order restatement at
    once (short rows, where every rounding of the reference's build shows):
    RMSNORM (eps defaults), SOFTMAX (temperatures), SWIGLU/MUL/ADD/GELU
    (alpha/beta defaults) and ATTENTION (head sizes 1..39 with any tail,
    causal offsets, masks, explicit scales)."""
    rng = np.random.default_rng(777)
    for _ in range(120):
        rows, cols = int(rng.integers(1, 6)), int(rng.integers(1, 80))
        X = (rng.standard_normal((rows, cols)) * rng.uniform(0.1, 10)).astype(np.float32)
        W = (1 + 0.1 * rng.standard_normal(cols)).astype(np.float32)
        eps = float(rng.choice([0.0, 1e-5, 1e-6, 0.1]))
        assert _bits(g.unary_rows(ref, abi.OP_RMSNORM_F32, X, W=W, eps=eps),
                     oracle.rmsnorm_avx2(X, W, eps if eps > 0 else 1e-5)), (rows, cols, eps)
        t = float(rng.choice([0.0, 0.5, 1.0, 2.0, 0.7]))
        assert _bits(g.unary_rows(ref, abi.OP_SOFTMAX_F32, X, temperature=t),
                     oracle.softmax_avx2(X, t if t > 0 else 1.0)), (rows, cols, t)
    for _ in range(120):
        n = int(rng.integers(1, 200))
        a = (rng.standard_normal(n) * rng.uniform(0.1, 30)).astype(np.float32)
        b = rng.standard_normal(n).astype(np.float32)
        al, be = float(rng.choice([0.0, 1.0, -1.5, 0.3])), float(rng.choice([0.0, 1.0, 2.5, -0.7]))
        assert _bits(g.elementwise(ref, abi.OP_SWIGLU_F32, a, b, alpha=al), oracle.swiglu_avx2(a, b, al or 1.0)), n
        assert _bits(g.elementwise(ref, abi.OP_MUL_F32, a, b, al, be), oracle.mul_avx2(a, b, al or 1.0, be)), n
        assert _bits(g.elementwise(ref, abi.OP_ADD_F32, a, b, al, be), oracle.add_avx2(a, b, al, be)), n
        assert _bits(g.elementwise(ref, abi.OP_GELU_F32, a), oracle.gelu_avx2(a)), n
    for _ in range(60):
        h, d = int(rng.integers(1, 3)), int(rng.integers(1, 40))
        sq = int(rng.integers(1, 40))
        sk = sq + int(rng.integers(0, 140))
        causal, scale = int(rng.integers(2)), (0.0 if rng.integers(2) else float(rng.uniform(0.05, 0.5)))
        Q = (rng.standard_normal((1, h, sq, d)) * rng.uniform(0.5, 3)).astype(np.float32)
        K = rng.standard_normal((1, h, sk, d)).astype(np.float32)
        V = rng.standard_normal((1, h, sk, d)).astype(np.float32)
        M = rng.standard_normal((1, h, sq, sk)).astype(np.float32) if rng.integers(3) == 0 else None
        assert _bits(g.attention(ref, Q, K, V, M, causal, scale),
                     oracle.attention_avx2(Q, K, V, M, causal, scale)), (h, sq, sk, d, causal, scale)
