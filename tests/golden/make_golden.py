"""Writes tests/golden/vnpu_golden.npz from the reference runtime.

The reference's own tests hold no golden vectors (every expectation is
computed inline), so these fixtures are produced by the reference itself:
oracle/_ref/libvnpu_ref.so, compiled from the reference sources by
oracle/Makefile with the reference's own flags, driven through its C ABI.
Each case stores its inputs and the reference's outputs, nothing else.

    python tests/golden/make_golden.py      (needs oracle/_ref built)

Inputs are small and seeded; the file stays a few hundred KiB.  MATMUL_F32
cases keep K <= 128 or use trans_b, so the reference's default packed path
is on its documented semantics (its epilogue defect at
src/kernels/kernels.cpp:313-323 needs K > 128 with B not transposed).
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
for p in (ROOT, os.path.join(ROOT, "npuxl-improved_amd"), os.path.dirname(HERE)):
    if p not in sys.path:
        sys.path.insert(0, p)

OUT = os.path.join(HERE, "vnpu_golden.npz")


def quant_input(rng):
    X = rng.standard_normal((9, 77)).astype(np.float32)
    X[1] = 0.0                                          # zero row -> scale 1
    X[2, :] = rng.integers(-100, 100, 77).astype(np.float32) + 0.5
    X[2, 0] = 127.0                                     # exact .5 ties
    X[3, 5] = np.nan                                    # NaN ignored by max
    X[4, 9] = np.inf                                    # non-finite max -> scale 1
    X[5] *= 1e-30                                       # tiny values
    X[6, :] = -X[6, :] * 3.0
    return X


def generate():
    import gpu_ops as g
    import oracle
    from vnpu_mi355x import Session, abi

    if not os.path.exists(oracle.REF_LIB_PATH):
        raise SystemExit("oracle/_ref/libvnpu_ref.so is not built (make -C oracle)")
    cfg = abi.Config()
    cfg.abi_version = 1
    cfg.num_threads = 4
    ref = Session(oracle.REF_LIB_PATH, cfg)
    rng = np.random.default_rng(20261201)
    f = {}

    Xq = quant_input(rng)
    f["quant/X"] = Xq
    for axis, name in ((0, "row"), (1, "col"), (2, "tensor")):
        Y, S = g.quantize(ref, Xq, axis)
        f[f"quant/{name}/Y"], f[f"quant/{name}/scales"] = Y, S

    M, K, N = 6, 150, 37
    A = rng.integers(-128, 128, (M, K)).astype(np.int8)
    B = rng.integers(-128, 128, (K, N)).astype(np.int8)
    sa = (0.01 + rng.random(M)).astype(np.float32)
    sb = (0.001 + 0.02 * rng.random(N)).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    f.update({"i8/A": A, "i8/B": B, "i8/sa": sa, "i8/sb": sb, "i8/bias": bias})
    w = ref.pack(B, K, N, scales=sb)
    f["i8/column_sums"] = ref.unpack_info(w)[4].astype(np.int32)
    w1 = ref.pack(B, K, N)
    f["i8/acc"] = g.matmul_i8(ref, A, w1, M, K, N)      # scales 1: exact int32 sums
    ref.release_packed(w1)
    for epi in range(5):
        f[f"i8/C/epi{epi}"] = g.matmul_i8(ref, A, w, M, K, N, scale_a=sa, bias=bias, epilogue=epi)
    ref.release_packed(w)

    for name, (M, K, N, ta, tb, beta, epi) in {
            "nn_silu": (7, 100, 19, 0, 0, 0.0, abi.EPI_SILU),
            "nt_gelu_beta": (9, 300, 23, 0, 1, 0.5, abi.EPI_GELU_TANH),
            "tn_relu": (5, 64, 17, 1, 0, 0.0, abi.EPI_RELU),
            "row_gelu_erf": (1, 260, 40, 0, 0, 0.0, abi.EPI_GELU_ERF)}.items():
        A = rng.standard_normal((K, M) if ta else (M, K)).astype(np.float32)
        B = rng.standard_normal((N, K) if tb else (K, N)).astype(np.float32)
        bias = (0.1 * rng.standard_normal(N)).astype(np.float32)
        C0 = rng.standard_normal((M, N)).astype(np.float32)
        f[f"f32/{name}/A"], f[f"f32/{name}/B"] = A, B
        f[f"f32/{name}/bias"], f[f"f32/{name}/C0"] = bias, C0
        f[f"f32/{name}/args"] = np.array([M, K, N, ta, tb, epi], np.int64)
        f[f"f32/{name}/beta"] = np.array([beta], np.float32)
        f[f"f32/{name}/C"] = g.matmul_f32(ref, A, B, M, K, N, C_in=C0, bias=bias, trans_a=ta,
                                          trans_b=tb, beta=beta, epilogue=epi)

    X = rng.standard_normal((5, 133)).astype(np.float32)
    W = rng.standard_normal(133).astype(np.float32)
    f["rows/X"], f["rows/W"] = X, W
    f["rows/rmsnorm"] = g.unary_rows(ref, abi.OP_RMSNORM_F32, X, W=W, eps=1e-5)
    f["rows/softmax"] = g.unary_rows(ref, abi.OP_SOFTMAX_F32, 4.0 * X, temperature=0.7)
    f["rows/softmax_X"] = 4.0 * X

    a = rng.standard_normal(1001).astype(np.float32)
    b = rng.standard_normal(1001).astype(np.float32)
    f["ew/a"], f["ew/b"] = a, b
    f["ew/swiglu"] = g.elementwise(ref, abi.OP_SWIGLU_F32, a, b, alpha=0.5)
    f["ew/add"] = g.elementwise(ref, abi.OP_ADD_F32, a, b, alpha=0.25, beta=-2.0)
    f["ew/add_default"] = g.elementwise(ref, abi.OP_ADD_F32, a, b)
    f["ew/mul"] = g.elementwise(ref, abi.OP_MUL_F32, a, b, alpha=1.5, beta=0.0)
    f["ew/gelu"] = g.elementwise(ref, abi.OP_GELU_F32, 3.0 * a)
    f["ew/gelu_X"] = 3.0 * a

    Q = rng.standard_normal((2, 3, 5, 32)).astype(np.float32)
    Kr = rng.standard_normal((2, 3, 7, 32)).astype(np.float32)
    pos = rng.integers(0, 5000, 7).astype(np.int32)
    f["rope/Q"], f["rope/K"], f["rope/positions"] = Q, Kr, pos
    f["rope/half/Q"], f["rope/half/K"] = g.rope(ref, Q, Kr, position_offset=4090)
    f["rope/inter/Q"], f["rope/inter/K"] = g.rope(ref, Q, Kr, positions=pos, interleaved=1,
                                                  theta=500000.0, scaling=0.5)

    Qa = rng.standard_normal((1, 2, 19, 64)).astype(np.float32)
    Ka = rng.standard_normal((1, 2, 150, 64)).astype(np.float32)
    Va = rng.standard_normal((1, 2, 150, 64)).astype(np.float32)
    mask = rng.standard_normal((1, 2, 19, 150)).astype(np.float32)
    f["attn/Q"], f["attn/K"], f["attn/V"], f["attn/mask"] = Qa, Ka, Va, mask
    f["attn/causal"] = g.attention(ref, Qa, Ka, Va, None, 1)
    f["attn/masked"] = g.attention(ref, Qa, Ka, Va, mask, 0, scale=0.2)

    H = rng.standard_normal((4, 128)).astype(np.float32)
    Wm = (0.02 * rng.standard_normal((128, 600))).astype(np.float32)
    f["mtp/hidden"], f["mtp/W"] = H, Wm
    f["mtp/logits"] = g.mtp_head(ref, H, Wm)
    f["mtp/softmax"] = g.unary_rows(ref, abi.OP_SOFTMAX_F32, f["mtp/logits"])

    ref.close()
    np.savez_compressed(OUT, **f)
    print(f"wrote {OUT}: {len(f)} arrays, {os.path.getsize(OUT)} bytes")


if __name__ == "__main__":
    generate()
