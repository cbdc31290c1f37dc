"""numpy front end of the C oracle (liboracle.so) - TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this package, and only as the checker.  Each wrapper calls the C
restatement in vnpu_oracle.c, which cites the reference routine it follows.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
REF_LIB_PATH = os.path.join(HERE, "_ref", "libvnpu_ref.so")

_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise FileNotFoundError("oracle not built: run `make -C oracle`")
        _lib = C.CDLL(LIB_PATH)
        f32p, i8p, u8p, i32p = (C.POINTER(C.c_float), C.POINTER(C.c_int8),
                                C.POINTER(C.c_uint8), C.POINTER(C.c_int32))
        u32, u64, f32 = C.c_uint32, C.c_uint64, C.c_float
        vp = C.c_void_p
        sig = {
            "vo_fast_expf": (f32, [f32]), "vo_silu": (f32, [f32]), "vo_gelu_tanh": (f32, [f32]),
            "vo_apply_epilogue": (f32, [f32, u32]),
            "vo_quantize_rows": (None, [vp, vp, vp, u64, u64]),
            "vo_quantize_columns": (None, [vp, vp, vp, u64, u64]),
            "vo_quantize_tensor": (None, [vp, vp, vp, u64, u64]),
            "vo_pack_canonical": (None, [vp, u32, u32, u32, u32, vp, vp]),
            "vo_gemm_i8_acc": (None, [vp, u32, vp, u32, u32, u32, vp]),
            "vo_matmul_i8": (None, [vp, u32, vp, vp, vp, vp, vp, u32, u32, u32, u32, u32]),
            "vo_store_i8": (None, [vp, vp, vp, vp, vp, u32, u32, u32]),
            "vo_store_f32": (None, [vp, vp, vp, u32, u32, f32, f32, u32]),
            "vo_matmul_f32": (None, [vp, vp, vp, vp, u32, u32, u32, u32, u32, u32, u32, u32,
                                     f32, f32, u32, vp]),
            "vo_matmul_f32_acc64": (None, [vp, vp, vp, vp, u32, u32, u32, u32, u32, u32, u32,
                                           u32, f32, f32, u32]),
            "vo_cull_map": (u64, [u32, u32, u32, u32, u32, u32, u32, vp, u32, u32, vp]),
            "vo_rmsnorm": (None, [vp, vp, vp, u32, u32, f32]),
            "vo_softmax": (None, [vp, vp, u32, u32, f32]),
            "vo_rope": (None, [vp, vp, vp, u32, u32, u32, u32, u32, u32, u32, f32, f32]),
            "vo_swiglu": (None, [vp, vp, vp, u64, f32]),
            "vo_add": (None, [vp, vp, vp, u64, f32, f32]),
            "vo_mul": (None, [vp, vp, vp, u64, f32, f32]),
            "vo_gelu": (None, [vp, vp, u64]),
            "vo_attention": (None, [vp, vp, vp, vp, vp, u32, u32, u32, u32, u32, u32, f32]),
            "vo_rmsnorm_avx2": (None, [vp, vp, vp, u32, u32, f32]),
            "vo_exp_avx2": (f32, [f32]),
            "vo_swiglu_avx2": (None, [vp, vp, vp, u64, f32, u64]),
            "vo_softmax_avx2": (None, [vp, vp, u32, u32, f32]),
            "vo_gelu_avx2": (None, [vp, vp, u64]),
            "vo_mul_avx2": (None, [vp, vp, vp, u64, f32, f32, u64]),
            "vo_add_avx2": (None, [vp, vp, vp, u64, f32, f32]),
            "vo_attention_avx2": (None, [vp, vp, vp, vp, vp, u32, u32, u32, u32, u32, u32, f32]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(_lib, name)
            fn.restype = res
            fn.argtypes = args
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def _c(a, dtype):
    return None if a is None else np.ascontiguousarray(a, dtype=dtype)


def fast_expf(x: float) -> float:
    return lib().vo_fast_expf(x)


def epilogue(x: np.ndarray, epi: int) -> np.ndarray:
    x = _c(x, np.float32)
    out = np.empty_like(x)
    f = lib().vo_apply_epilogue
    flat, of = x.reshape(-1), out.reshape(-1)
    for i in range(flat.size):
        of[i] = f(float(flat[i]), epi)
    return out


def quantize(X: np.ndarray, axis: int):
    """QUANTIZE_I8 -> (int8 tensor, float32 scales)."""
    X = _c(X, np.float32)
    rows, cols = X.shape
    Y = np.empty((rows, cols), np.int8)
    n = rows if axis == 0 else cols if axis == 1 else 1
    S = np.empty(n, np.float32)
    fn = [lib().vo_quantize_rows, lib().vo_quantize_columns, lib().vo_quantize_tensor][axis]
    fn(_p(X), _p(Y), _p(S), rows, cols)
    return Y, S


def pack_canonical(B: np.ndarray, K: int, N: int, ldb: int = 0, trans_b: int = 0):
    B = _c(B, np.int8)
    orig = np.empty((K, N), np.int8)
    sums = np.empty(N, np.int32)
    lib().vo_pack_canonical(_p(B), K, N, ldb, trans_b, _p(orig), _p(sums))
    return orig, sums


def gemm_i8_acc(A: np.ndarray, Bkn: np.ndarray) -> np.ndarray:
    A, Bkn = _c(A, np.int8), _c(Bkn, np.int8)
    M, K = A.shape
    N = Bkn.shape[1]
    acc = np.empty((M, N), np.int32)
    lib().vo_gemm_i8_acc(_p(A), K, _p(Bkn), M, K, N, _p(acc))
    return acc


def matmul_i8(A, Bkn, scale_a=None, scale_b=None, bias=None, epilogue: int = 0):
    A, Bkn = _c(A, np.int8), _c(Bkn, np.int8)
    M, K = A.shape
    N = Bkn.shape[1]
    C_ = np.empty((M, N), np.float32)
    lib().vo_matmul_i8(_p(A), K, _p(Bkn), _p(_c(scale_a, np.float32)), _p(_c(scale_b, np.float32)),
                       _p(_c(bias, np.float32)), _p(C_), N, M, K, N, epilogue)
    return C_


def matmul_i8_blas(A, Bkn, scale_a=None, scale_b=None, bias=None, epilogue: int = 0):
    """matmul_i8 for large shapes: the int32 accumulator is the float64 BLAS
    product of the int8 matrices (exact: every partial sum is an integer below
    2^53), then the C store step vo_store_i8 (the same rounding order as
    vo_matmul_i8; tests/test_oracle_blas.py checks the two agree bit for bit)."""
    A, Bkn = _c(A, np.int8), _c(Bkn, np.int8)
    M, N = A.shape[0], Bkn.shape[1]
    acc = np.ascontiguousarray((A.astype(np.float64) @ Bkn.astype(np.float64)).astype(np.int32))
    C_ = np.empty((M, N), np.float32)
    lib().vo_store_i8(_p(acc), _p(_c(scale_a, np.float32)), _p(_c(scale_b, np.float32)),
                      _p(_c(bias, np.float32)), _p(C_), M, N, epilogue)
    return C_


def matmul_f32_blas(A, B, C_in=None, bias=None, trans_a=0, trans_b=0, alpha=1.0, beta=0.0,
                    epilogue=0):
    """matmul_f32 with a float64 accumulator (vo_matmul_f32_acc64's semantics)
    for large shapes: the float64 BLAS product, then the C store step
    vo_store_f32."""
    A64 = np.asarray(A, np.float64)
    B64 = np.asarray(B, np.float64)
    acc = np.ascontiguousarray((A64.T if trans_a else A64) @ (B64.T if trans_b else B64))
    M, N = acc.shape
    out = np.zeros((M, N), np.float32) if C_in is None else np.array(C_in, np.float32, copy=True)
    lib().vo_store_f32(_p(acc), _p(_c(bias, np.float32)), _p(out), M, N, alpha, beta, epilogue)
    return out


def matmul_f32(A, B, C_in=None, bias=None, M=None, K=None, N=None, trans_a=0, trans_b=0,
               alpha=1.0, beta=0.0, epilogue=0, cull=None, acc64=False):
    A, B = _c(A, np.float32), _c(B, np.float32)
    if M is None:
        M, K = (A.shape[1], A.shape[0]) if trans_a else A.shape
        N = B.shape[0] if trans_b else B.shape[1]
    out = np.zeros((M, N), np.float32) if C_in is None else np.array(C_in, np.float32, copy=True)
    bias = _c(bias, np.float32)
    if acc64:
        lib().vo_matmul_f32_acc64(_p(A), _p(B), _p(bias), _p(out), M, K, N, 0, 0, 0, trans_a,
                                  trans_b, alpha, beta, epilogue)
    else:
        cull = _c(cull, np.uint8)
        lib().vo_matmul_f32(_p(A), _p(B), _p(bias), _p(out), M, K, N, 0, 0, 0, trans_a, trans_b,
                            alpha, beta, epilogue, _p(cull))
    return out


def cull_map(M, N, unit, tile_m, tile_n, threads, pack_b, mask):
    mask = _c(mask, np.uint8)
    out = np.empty((M, N), np.uint8)
    n = lib().vo_cull_map(M, N, unit, tile_m, tile_n, threads, pack_b, _p(mask),
                          mask.shape[0], mask.shape[1], _p(out))
    return out, int(n)


def rmsnorm(X, W=None, eps=1e-5):
    X = _c(X, np.float32)
    Y = np.empty_like(X)
    lib().vo_rmsnorm(_p(X), _p(_c(W, np.float32)), _p(Y), X.shape[0], X.shape[1], eps)
    return Y


def softmax(X, temperature=1.0):
    X = _c(X, np.float32)
    Y = np.empty_like(X)
    lib().vo_softmax(_p(X), _p(Y), X.shape[0], X.shape[1], temperature)
    return Y


def softmax_avx2(X, temperature=1.0):
    """The reference's AVX2 build of SOFTMAX_F32 (llm.cpp:137-180), bit for bit."""
    X = _c(X, np.float32)
    Y = np.empty_like(X)
    lib().vo_softmax_avx2(_p(X), _p(Y), X.shape[0], X.shape[1], temperature)
    return Y


def rope(Q, K, positions=None, position_offset=0, interleaved=0, theta=10000.0, scaling=1.0):
    """In-place rotation of copies of Q, K ([b, h, seq, d]); returns (Q', K')."""
    Q = None if Q is None else np.array(Q, np.float32, copy=True)
    K = None if K is None else np.array(K, np.float32, copy=True)
    ref = Q if Q is not None else K
    b, h, _, d = ref.shape
    qs = Q.shape[2] if Q is not None else 0
    ks = K.shape[2] if K is not None else 0
    lib().vo_rope(_p(Q), _p(K), _p(_c(positions, np.int32)), b, h, qs, ks, d, position_offset,
                  interleaved, theta, scaling)
    return Q, K


def swiglu(g, u, alpha=1.0):
    g, u = _c(g, np.float32), _c(u, np.float32)
    Y = np.empty_like(g)
    lib().vo_swiglu(_p(g), _p(u), _p(Y), g.size, alpha)
    return Y


def add(a, b, alpha=1.0, beta=1.0):
    a, b = _c(a, np.float32), _c(b, np.float32)
    Y = np.empty_like(a)
    lib().vo_add(_p(a), _p(b), _p(Y), a.size, alpha, beta)
    return Y


def mul(a, b, alpha=1.0, beta=0.0):
    a, b = _c(a, np.float32), _c(b, np.float32)
    Y = np.empty_like(a)
    lib().vo_mul(_p(a), _p(b), _p(Y), a.size, alpha, beta)
    return Y


def gelu(x):
    x = _c(x, np.float32)
    Y = np.empty_like(x)
    lib().vo_gelu(_p(x), _p(Y), x.size)
    return Y


def attention(Q, K, V, mask=None, causal=0, scale=0.0):
    Q, K, V = _c(Q, np.float32), _c(K, np.float32), _c(V, np.float32)
    b, h, sq, d = Q.shape
    sk = K.shape[2]
    O = np.empty_like(Q)
    lib().vo_attention(_p(Q), _p(K), _p(V), _p(_c(mask, np.float32)), _p(O), b, h, sq, sk, d,
                       causal, scale)
    return O


def rmsnorm_avx2(X, W=None, eps=1e-5):
    """RMSNORM in the order of the reference's AVX2 build (bit for bit)."""
    X = _c(X, np.float32)
    Y = np.empty_like(X)
    lib().vo_rmsnorm_avx2(_p(X), _p(_c(W, np.float32)), _p(Y), X.shape[0], X.shape[1], eps)
    return Y


def ew_grain(count, num_threads):
    """Range length of the reference's elementwise commands on a device of
    num_threads units (src/core/scheduler.cpp:541-543): max(4096, count /
    (4 num_threads)); None -> 0, one range."""
    return 0 if num_threads is None else max(4096, count // (4 * num_threads))


def swiglu_avx2(g, u, alpha=1.0, num_threads=None):
    """SWIGLU in the order of the reference's AVX2 build (bit for bit), split
    into the ranges the reference runs on a device of num_threads units (each
    range has its own scalar tail; None: one range)."""
    g, u = _c(g, np.float32), _c(u, np.float32)
    Y = np.empty_like(g)
    lib().vo_swiglu_avx2(_p(g), _p(u), _p(Y), g.size, alpha, ew_grain(g.size, num_threads))
    return Y


def gelu_avx2(x):
    """GELU in the order of the reference's AVX2 build (bit for bit)."""
    x = _c(x, np.float32)
    Y = np.empty_like(x)
    lib().vo_gelu_avx2(_p(x), _p(Y), x.size)
    return Y


def mul_avx2(a, b, alpha=1.0, beta=0.0, num_threads=None):
    """MUL in the order of the reference's AVX2 build (bit for bit), ranges as
    in swiglu_avx2."""
    a, b = _c(a, np.float32), _c(b, np.float32)
    Y = np.empty_like(a)
    lib().vo_mul_avx2(_p(a), _p(b), _p(Y), a.size, alpha, beta, ew_grain(a.size, num_threads))
    return Y


def add_avx2(a, b, alpha=1.0, beta=1.0):
    """ADD in the order of the reference's AVX2 build (bit for bit)."""
    a, b = _c(a, np.float32), _c(b, np.float32)
    Y = np.empty_like(a)
    lib().vo_add_avx2(_p(a), _p(b), _p(Y), a.size, alpha, beta)
    return Y


def attention_avx2(Q, K, V, mask=None, causal=0, scale=0.0):
    """ATTENTION_F32 in the order of the reference's AVX2 build (bit for bit)."""
    Q, K, V = _c(Q, np.float32), _c(K, np.float32), _c(V, np.float32)
    b, h, sq, d = Q.shape
    sk = K.shape[2]
    O = np.empty_like(Q)
    lib().vo_attention_avx2(_p(Q), _p(K), _p(V), _p(_c(mask, np.float32)), _p(O), b, h, sq, sk, d,
                            causal, scale)
    return O


def rel_error(got: np.ndarray, ref: np.ndarray) -> float:
    """max|got - ref| / max(1, max|ref|): the reference's conformance metric
    (tools/conformance.cpp:95-103)."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(got - ref)) / max(1.0, float(np.max(np.abs(ref)))))
