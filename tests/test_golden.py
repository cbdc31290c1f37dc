"""Golden fixtures written by the reference runtime (tests/golden/make_golden.py).

The CPU half pins the C oracle against the reference's own outputs without
needing the reference build at test time; the GPU half runs the same inputs
through libvnpu.so on the MI355X.  Integer outputs are compared bit for bit,
float outputs with the reference's metric max|d| / max(1, max|ref|)
(tools/conformance.cpp:95-103): 1e-4 for ops, 2e-3 for attention.
"""
import os

import numpy as np
import pytest

import gpu_ops as g
import oracle
from vnpu_mi355x import abi

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "vnpu_golden.npz")


@pytest.fixture(scope="module")
def gold():
    with np.load(GOLDEN) as z:   # plain arrays only (allow_pickle stays False)
        return {k: z[k] for k in z.files}


F32_CASES = ["nn_silu", "nt_gelu_beta", "tn_relu", "row_gelu_erf"]


# --------------------------------------------------------------------------
# oracle vs the reference's outputs (CPU)
# --------------------------------------------------------------------------

@pytest.mark.parametrize("axis,name", [(0, "row"), (1, "col"), (2, "tensor")])
def test_oracle_quantize(gold, axis, name):
    Y, S = oracle.quantize(gold["quant/X"], axis)
    assert np.array_equal(Y, gold[f"quant/{name}/Y"])
    assert np.array_equal(S.view(np.uint32), gold[f"quant/{name}/scales"].view(np.uint32))


def test_oracle_matmul_i8(gold):
    A, B = gold["i8/A"], gold["i8/B"]
    assert np.array_equal(oracle.gemm_i8_acc(A, B).astype(np.float32), gold["i8/acc"])
    assert np.array_equal(oracle.pack_canonical(B, *B.shape)[1], gold["i8/column_sums"])
    for epi in range(5):
        got = oracle.matmul_i8(A, B, gold["i8/sa"], gold["i8/sb"], gold["i8/bias"], epi)
        # bit-exact only where the reference's epilogue math is also exact;
        # the transcendental epilogues use its fast_expf in both
        assert oracle.rel_error(got, gold[f"i8/C/epi{epi}"]) <= 1e-6, epi
    assert np.array_equal(oracle.matmul_i8(A, B, gold["i8/sa"], gold["i8/sb"], gold["i8/bias"], 0),
                          gold["i8/C/epi0"])


@pytest.mark.parametrize("name", F32_CASES)
def test_oracle_matmul_f32(gold, name):
    M, K, N, ta, tb, epi = (int(x) for x in gold[f"f32/{name}/args"])
    want = gold[f"f32/{name}/C"]
    got = oracle.matmul_f32(gold[f"f32/{name}/A"], gold[f"f32/{name}/B"], gold[f"f32/{name}/C0"],
                            gold[f"f32/{name}/bias"], M, K, N, ta, tb, 1.0,
                            float(gold[f"f32/{name}/beta"][0]), epi)
    assert oracle.rel_error(got, want) <= 1e-5


def test_oracle_rows_and_elementwise(gold):
    assert oracle.rel_error(oracle.rmsnorm(gold["rows/X"], gold["rows/W"], 1e-5),
                            gold["rows/rmsnorm"]) <= 1e-6
    assert oracle.rel_error(oracle.softmax(gold["rows/softmax_X"], 0.7), gold["rows/softmax"]) <= 1e-6
    a, b = gold["ew/a"], gold["ew/b"]
    assert oracle.rel_error(oracle.swiglu(a, b, 0.5), gold["ew/swiglu"]) <= 1e-6
    assert oracle.rel_error(oracle.add(a, b, 0.25, -2.0), gold["ew/add"]) <= 1e-6
    assert oracle.rel_error(oracle.add(a, b, 0.0, 0.0), gold["ew/add_default"]) <= 1e-6
    assert oracle.rel_error(oracle.mul(a, b, 1.5, 0.0), gold["ew/mul"]) <= 1e-6
    assert oracle.rel_error(oracle.gelu(gold["ew/gelu_X"]), gold["ew/gelu"]) <= 1e-6


def test_oracle_rope(gold):
    Q, K = gold["rope/Q"], gold["rope/K"]
    q, k = oracle.rope(Q, K, position_offset=4090)
    assert oracle.rel_error(q, gold["rope/half/Q"]) <= 1e-6
    assert oracle.rel_error(k, gold["rope/half/K"]) <= 1e-6
    q, k = oracle.rope(Q, K, positions=gold["rope/positions"], interleaved=1, theta=500000.0,
                       scaling=0.5)
    assert oracle.rel_error(q, gold["rope/inter/Q"]) <= 1e-6
    assert oracle.rel_error(k, gold["rope/inter/K"]) <= 1e-6


def test_oracle_attention_and_mtp(gold):
    Q, K, V = gold["attn/Q"], gold["attn/K"], gold["attn/V"]
    assert oracle.rel_error(oracle.attention(Q, K, V, None, 1), gold["attn/causal"]) <= 1e-5
    assert oracle.rel_error(oracle.attention(Q, K, V, gold["attn/mask"], 0, 0.2),
                            gold["attn/masked"]) <= 1e-5
    H, W = gold["mtp/hidden"], gold["mtp/W"]
    logits = oracle.matmul_f32(H, W, None, None, *H.shape, W.shape[1])
    assert oracle.rel_error(logits, gold["mtp/logits"]) <= 1e-5
    assert oracle.rel_error(oracle.softmax(gold["mtp/logits"]), gold["mtp/softmax"]) <= 1e-6


# --------------------------------------------------------------------------
# libvnpu.so on the MI355X vs the reference's outputs
# --------------------------------------------------------------------------

@pytest.mark.gpu
@pytest.mark.parametrize("axis,name", [(0, "row"), (1, "col"), (2, "tensor")])
def test_gpu_quantize(gpu, gold, axis, name):
    Y, S = g.quantize(gpu, gold["quant/X"], axis)
    assert np.array_equal(Y, gold[f"quant/{name}/Y"])
    assert np.array_equal(S.view(np.uint32), gold[f"quant/{name}/scales"].view(np.uint32))


@pytest.mark.gpu
def test_gpu_matmul_i8(gpu, gold):
    A, B = gold["i8/A"], gold["i8/B"]
    M, K = A.shape
    N = B.shape[1]
    w1 = gpu.pack(B, K, N)
    assert np.array_equal(gpu.unpack_info(w1)[4], gold["i8/column_sums"])
    assert np.array_equal(g.matmul_i8(gpu, A, w1, M, K, N), gold["i8/acc"])
    gpu.release_packed(w1)
    w = gpu.pack(B, K, N, scales=gold["i8/sb"])
    for epi in range(5):
        got = g.matmul_i8(gpu, A, w, M, K, N, scale_a=gold["i8/sa"], bias=gold["i8/bias"],
                          epilogue=epi)
        want = gold[f"i8/C/epi{epi}"]
        if epi <= 1:
            assert np.array_equal(got, want), epi
        else:
            assert oracle.rel_error(got, want) <= 1e-6, epi
    gpu.release_packed(w)


@pytest.mark.gpu
@pytest.mark.parametrize("name", F32_CASES)
def test_gpu_matmul_f32(gpu, gold, name):
    M, K, N, ta, tb, epi = (int(x) for x in gold[f"f32/{name}/args"])
    got = g.matmul_f32(gpu, gold[f"f32/{name}/A"], gold[f"f32/{name}/B"], M, K, N,
                       C_in=gold[f"f32/{name}/C0"], bias=gold[f"f32/{name}/bias"], trans_a=ta,
                       trans_b=tb, beta=float(gold[f"f32/{name}/beta"][0]), epilogue=epi)
    assert oracle.rel_error(got, gold[f"f32/{name}/C"]) <= 1e-4


@pytest.mark.gpu
def test_gpu_rows_elementwise_rope(gpu, gold):
    assert oracle.rel_error(g.unary_rows(gpu, abi.OP_RMSNORM_F32, gold["rows/X"], W=gold["rows/W"],
                                         eps=1e-5), gold["rows/rmsnorm"]) <= 1e-4
    assert oracle.rel_error(g.unary_rows(gpu, abi.OP_SOFTMAX_F32, gold["rows/softmax_X"],
                                         temperature=0.7), gold["rows/softmax"]) <= 1e-4
    a, b = gold["ew/a"], gold["ew/b"]
    assert oracle.rel_error(g.elementwise(gpu, abi.OP_SWIGLU_F32, a, b, alpha=0.5),
                            gold["ew/swiglu"]) <= 1e-4
    assert oracle.rel_error(g.elementwise(gpu, abi.OP_ADD_F32, a, b, alpha=0.25, beta=-2.0),
                            gold["ew/add"]) <= 1e-4
    assert oracle.rel_error(g.elementwise(gpu, abi.OP_ADD_F32, a, b), gold["ew/add_default"]) <= 1e-4
    assert oracle.rel_error(g.elementwise(gpu, abi.OP_MUL_F32, a, b, alpha=1.5),
                            gold["ew/mul"]) <= 1e-4
    assert oracle.rel_error(g.elementwise(gpu, abi.OP_GELU_F32, gold["ew/gelu_X"]),
                            gold["ew/gelu"]) <= 1e-4
    Q, K = gold["rope/Q"], gold["rope/K"]
    q, k = g.rope(gpu, Q, K, position_offset=4090)
    assert oracle.rel_error(q, gold["rope/half/Q"]) <= 1e-4
    assert oracle.rel_error(k, gold["rope/half/K"]) <= 1e-4
    q, k = g.rope(gpu, Q, K, positions=gold["rope/positions"], interleaved=1, theta=500000.0,
                  scaling=0.5)
    assert oracle.rel_error(q, gold["rope/inter/Q"]) <= 1e-4
    assert oracle.rel_error(k, gold["rope/inter/K"]) <= 1e-4


@pytest.mark.gpu
def test_gpu_attention_and_mtp(gpu, gold):
    Q, K, V = gold["attn/Q"], gold["attn/K"], gold["attn/V"]
    assert oracle.rel_error(g.attention(gpu, Q, K, V, None, 1), gold["attn/causal"]) <= 2e-3
    assert oracle.rel_error(g.attention(gpu, Q, K, V, gold["attn/mask"], 0, scale=0.2),
                            gold["attn/masked"]) <= 2e-3
    logits = g.mtp_head(gpu, gold["mtp/hidden"], gold["mtp/W"])
    assert oracle.rel_error(logits, gold["mtp/logits"]) <= 1e-4
    assert oracle.rel_error(g.unary_rows(gpu, abi.OP_SOFTMAX_F32, logits),
                            gold["mtp/softmax"]) <= 1e-4
