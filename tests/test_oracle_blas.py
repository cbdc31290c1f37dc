"""The BLAS-backed oracle GEMMs used by the full-size GPU tests (CPU).

oracle.matmul_i8_blas takes the int32 accumulator from a float64 BLAS product
of the int8 operands (exact) and then runs the C store step; it must equal
the scalar C oracle oracle.matmul_i8 bit for bit.  oracle.matmul_f32_blas
must equal the float64-accumulator C oracle up to the order of the float64
sums (which moves (float)acc by at most one float32 ulp).
"""
import numpy as np
import pytest

import oracle

RNG = np.random.default_rng(314159)


@pytest.mark.parametrize("M,K,N", [(1, 64, 16), (7, 300, 33), (64, 1000, 130), (130, 4096, 70)])
@pytest.mark.parametrize("epi,use_bias,use_sa", [(0, False, True), (0, True, False), (2, True, True),
                                                 (3, False, True), (1, True, True)])
def test_matmul_i8_blas_bit_exact(M, K, N, epi, use_bias, use_sa):
    A = RNG.integers(-128, 128, (M, K)).astype(np.int8)
    B = RNG.integers(-128, 128, (K, N)).astype(np.int8)
    sa = (RNG.random(M).astype(np.float32) + 0.5) / 127 if use_sa else None
    sb = (RNG.random(N).astype(np.float32) + 0.5) / 127
    bias = RNG.standard_normal(N).astype(np.float32) if use_bias else None
    got = oracle.matmul_i8_blas(A, B, sa, sb, bias, epi)
    want = oracle.matmul_i8(A, B, sa, sb, bias, epi)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_matmul_i8_blas_extreme_accumulators():
    # |acc| up to K * 128 * 128 = 2^26 at K = 4096: still exact in float64.
    K = 4096
    A = np.full((3, K), -128, np.int8)
    B = np.full((K, 5), -128, np.int8)
    B[:, 1] = 127
    got = oracle.matmul_i8_blas(A, B)
    assert got[0, 0] == float(K * 128 * 128) and got[0, 1] == float(-K * 128 * 127)
    assert np.array_equal(got.view(np.uint32), oracle.matmul_i8(A, B).view(np.uint32))


@pytest.mark.parametrize("M,K,N,ta,tb", [(5, 64, 9, 0, 0), (33, 257, 70, 0, 1), (64, 600, 40, 1, 0),
                                         (17, 130, 17, 1, 1)])
@pytest.mark.parametrize("epi,alpha,beta", [(0, 1.0, 0.0), (3, 1.0, 0.5), (2, 0.0, -1.0)])
def test_matmul_f32_blas_matches_acc64(M, K, N, ta, tb, epi, alpha, beta):
    A = RNG.standard_normal((K, M) if ta else (M, K)).astype(np.float32)
    B = RNG.standard_normal((N, K) if tb else (K, N)).astype(np.float32)
    bias = RNG.standard_normal(N).astype(np.float32)
    Cin = RNG.standard_normal((M, N)).astype(np.float32)
    got = oracle.matmul_f32_blas(A, B, Cin, bias, ta, tb, alpha, beta, epi)
    want = oracle.matmul_f32(A, B, Cin, bias, M, K, N, ta, tb, alpha, beta, epi, acc64=True)
    assert oracle.rel_error(got, want) <= 1e-6
    # only the float64 summation order differs: nearly every element agrees
    assert np.mean(got == want) >= 0.99
