"""The Llama-style block restated with the C oracle (test infrastructure).

Same op sequence as npuxl-improved_amd/csrc/block_harness.hip and the
reference's block benchmark (tools/llm_bench.cpp:240-326): every vnpu op is
the oracle's restatement, the layout steps are numpy transposes.
"""
from __future__ import annotations

import numpy as np

import oracle


def gemm(x, wq, ws):
    a8, sa = oracle.quantize(x, 0)
    return oracle.matmul_i8(a8, wq, sa, ws)


def block(shape, wq, norm_attn, norm_ffn, x, batch, tokens, past=0, k_cache=None, v_cache=None,
          eps=1e-5, theta=10000.0):
    """wq: name -> (int8 [K][N], scales [N]).  Returns the new x [rows][d]."""
    d, H, D = shape.d_model, shape.heads, shape.head_dim
    B, T = batch, tokens
    x = np.array(x, np.float32, copy=True)
    xn = oracle.rmsnorm(x, norm_attn, eps)
    qkv = gemm(xn, *wq["qkv"])

    def heads(part):
        return np.ascontiguousarray(part.reshape(B, T, H, D).transpose(0, 2, 1, 3))

    q, k, v = heads(qkv[:, :d]), heads(qkv[:, d:2 * d]), heads(qkv[:, 2 * d:])
    q, k = oracle.rope(q, k, position_offset=past, theta=theta, scaling=1.0)
    if k_cache is not None:
        K = np.array(k_cache, np.float32, copy=True)
        V = np.array(v_cache, np.float32, copy=True)
        K[:, :, past:past + T] = k
        V[:, :, past:past + T] = v
    else:
        K, V = k, v
    o = oracle.attention(q, K, V, None, 1)
    att = np.ascontiguousarray(o.transpose(0, 2, 1, 3).reshape(B * T, d))
    x = oracle.add(x, gemm(att, *wq["o"]), 1.0, 1.0)
    xn = oracle.rmsnorm(x, norm_ffn, eps)
    a8, sa = oracle.quantize(xn, 0)
    gate = oracle.matmul_i8(a8, wq["gate"][0], sa, wq["gate"][1])
    up = oracle.matmul_i8(a8, wq["up"][0], sa, wq["up"][1])
    ff = oracle.swiglu(gate, up, 1.0)
    return oracle.add(x, gemm(ff, *wq["down"]), 1.0, 1.0)
