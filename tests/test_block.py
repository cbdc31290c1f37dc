"""The Llama-style decoder block through the block harness.

CPU: the harness driving the reference build (host layout steps) equals the
oracle's composition of the same ops.  GPU: the harness driving libvnpu.so
(layout kernels on the vnpu stream) equals the oracle at small and medium
shapes and the reference build at the full config-4 decode shape, within
the block tolerance 2e-3 (max|d| / max(1, max|ref|)).
"""
import os

import numpy as np
import pytest

import block_oracle
import oracle
from vnpu_mi355x import abi, synth
from vnpu_mi355x.block import LLAMA_4096, PROJECTIONS, Block, BlockShape, weights_f32

TINY = BlockShape(d_model=64, heads=2, head_dim=32, ffn=96)
SMALL = BlockShape(d_model=256, heads=2, head_dim=128, ffn=688)
TOL = 2e-3


def _ref_session():
    from vnpu_mi355x import Session
    if not os.path.exists(oracle.REF_LIB_PATH):
        pytest.skip("reference build oracle/_ref/libvnpu_ref.so not present")
    cfg = abi.Config()
    cfg.abi_version = 1
    cfg.num_threads = min(16, os.cpu_count() or 1)
    return Session(oracle.REF_LIB_PATH, cfg)


def _inputs(shape, batch, tokens, cache_len, tag):
    x = synth.normal(f"{tag}/x", (batch * tokens, shape.d_model))
    if not cache_len:
        return x, None, None
    kv = (batch, shape.heads, cache_len, shape.head_dim)
    return x, synth.normal(f"{tag}/k_cache", kv), synth.normal(f"{tag}/v_cache", kv)


def _run(s, gpu, shape, w32, batch, tokens, past, cache_len, tag, quantized=None):
    blk = Block(s, shape, w32, quantized=quantized)
    try:
        blk.prepare(batch, tokens, past=past, cache_len=cache_len)
        x, kc, vc = _inputs(shape, batch, tokens, cache_len, tag)
        blk.set_input(x, kc, vc)
        blk.run(gpu)
        wq = {n: blk.quantized_weights(n) for n in PROJECTIONS}
        return blk.output(), wq, (x, kc, vc)
    finally:
        blk.close()


def _oracle(shape, w32, wq, inputs, batch, tokens, past):
    x, kc, vc = inputs
    return block_oracle.block(shape, wq, w32["norm_attn"], w32["norm_ffn"], x, batch, tokens,
                              past=past, k_cache=kc, v_cache=vc)


CASES = [  # (shape, batch, tokens, past, cache_len)
    (TINY, 1, 37, 0, 0),          # prefill, odd length
    (TINY, 3, 1, 20, 21),         # decode after 20 cached positions
    (TINY, 2, 5, 11, 16),         # multi-token decode (speculative-style)
]


@pytest.mark.parametrize("shape,batch,tokens,past,cache_len", CASES)
def test_reference_block_matches_oracle(shape, batch, tokens, past, cache_len):
    s = _ref_session()
    try:
        w32 = weights_f32(shape, "test/tiny")
        got, wq, inputs = _run(s, False, shape, w32, batch, tokens, past, cache_len, "test/tiny")
    finally:
        s.close()
    want = _oracle(shape, w32, wq, inputs, batch, tokens, past)
    assert oracle.rel_error(got, want) <= TOL


@pytest.mark.gpu
@pytest.mark.parametrize("shape,batch,tokens,past,cache_len",
                         CASES + [(SMALL, 1, 300, 0, 0), (SMALL, 4, 1, 511, 512)])
def test_gpu_block_matches_oracle(gpu, shape, batch, tokens, past, cache_len):
    w32 = weights_f32(shape, "test/block")
    got, wq, inputs = _run(gpu, True, shape, w32, batch, tokens, past, cache_len, "test/block")
    want = _oracle(shape, w32, wq, inputs, batch, tokens, past)
    assert np.isfinite(got).all()
    assert oracle.rel_error(got, want) <= TOL


@pytest.mark.gpu
def test_gpu_block_full_decode_stagewise(gpu):
    """Config 4 decode at full size (batch 8, context 4096, new token at 4095),
    stage by stage: each op's GPU output against the oracle applied to the
    GPU's own input of that stage (integer stages bit-exact, f32 stages within
    their op tolerance).

    End to end the block is not compared at this size: it re-quantizes its
    activations to int8 four times, and f32 differences of ~1e-5 in the
    attention output (summation order) flip ~0.3% of the next int8 roundings;
    the flips compound through the O projection and the FFN until the input of
    the down projection differs in hundreds of +-1 steps per row, ~4e-2 on
    outputs of magnitude ~5.  The reference and the oracle agree end to end
    only because both are the same CPU f32 arithmetic.
    """
    shape, B, T, ctx = LLAMA_4096, 8, 1, 4096
    d, H, D, F = shape.d_model, shape.heads, shape.head_dim, shape.ffn
    w32 = weights_f32(shape, "config4")
    blk = Block(gpu, shape, w32)
    try:
        blk.prepare(B, T, past=ctx - 1, cache_len=ctx)
        x0, kc0, vc0 = _inputs(shape, B, T, ctx, "config4/decode")
        blk.set_input(x0, kc0, vc0)
        blk.run(True)
        get = lambda n, shp: gpu.download(blk.bufs[n], np.float32, shp)
        wq = {n: blk.quantized_weights(n) for n in PROJECTIONS}
        qkv, q, k, v = (get("qkv", (B, 3 * d)), get("q", (B, H, T, D)), get("k", (B, H, T, D)),
                        get("v", (B, H, T, D)))
        kv = (B, H, ctx, D)
        kc, vc, o, att = get("k_cache", kv), get("v_cache", kv), get("o", (B, H, T, D)), get("att", (B, d))
        gate, up, ff, down, x = (get("gate", (B, F)), get("up", (B, F)), get("ff", (B, F)),
                                 get("proj", (B, d)), get("x", (B, d)))
        xn2 = get("xn", (B, d))
    finally:
        blk.close()

    def gemm(a, name):
        a8, sa = oracle.quantize(a, 0)
        return oracle.matmul_i8(a8, wq[name][0], sa, wq[name][1])

    def heads(part):
        return np.ascontiguousarray(part.reshape(B, T, H, D).transpose(0, 2, 1, 3))

    xn1 = oracle.rmsnorm(x0, w32["norm_attn"], 1e-5)
    assert oracle.rel_error(qkv, gemm(xn1, "qkv")) <= 1e-4
    qr, kr = oracle.rope(heads(qkv[:, :d]), heads(qkv[:, d:2 * d]), position_offset=ctx - 1)
    assert oracle.rel_error(q, qr) <= 1e-4 and oracle.rel_error(k, kr) <= 1e-4
    assert np.array_equal(v, heads(qkv[:, 2 * d:]))
    assert np.array_equal(kc[:, :, ctx - 1:], k) and np.array_equal(vc[:, :, ctx - 1:], v)
    assert np.array_equal(kc[:, :, :ctx - 1], kc0[:, :, :ctx - 1])
    assert oracle.rel_error(o, oracle.attention(q, kc, vc, None, 1)) <= TOL
    assert np.array_equal(att, o.transpose(0, 2, 1, 3).reshape(B, d))
    # x after the attention residual is not kept by the harness: rebuild it
    # from the GPU's attention output (integer GEMM and exact add), then
    # check the FFN stages from the GPU's own normalized input.
    x1 = oracle.add(x0, gemm(att, "o"), 1.0, 1.0)
    assert oracle.rel_error(xn2, oracle.rmsnorm(x1, w32["norm_ffn"], 1e-5)) <= 1e-4
    a8, sa = oracle.quantize(xn2, 0)
    assert np.array_equal(gate, oracle.matmul_i8(a8, wq["gate"][0], sa, wq["gate"][1]))
    assert np.array_equal(up, oracle.matmul_i8(a8, wq["up"][0], sa, wq["up"][1]))
    assert oracle.rel_error(ff, oracle.swiglu(gate, up, 1.0)) <= 1e-4
    a8, sa = oracle.quantize(ff, 0)
    assert np.array_equal(down, oracle.matmul_i8(a8, wq["down"][0], sa, wq["down"][1]))
    assert np.isfinite(x).all()
