"""The Llama-style decoder block through the block harness.

CPU: the harness driving the reference build (host layout steps) equals the
oracle's composition of the same ops, and bit for bit the oracle's chain of
AVX2-order restatements.  GPU: the harness driving libvnpu.so (layout kernels
on the vnpu stream) equals the oracle at small and medium shapes within the
block tolerance 2e-3 (max|d| / max(1, max|ref|)); at the full config-4
decode and prefill shapes every stage is checked against the oracle on the
GPU's own stage input, and with VNPU_CONFIG_REFERENCE_ORDER the whole block
is bit-exact with the reference's output.
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


@pytest.mark.parametrize("shape,batch,tokens,past,cache_len",
                         CASES + [(SMALL, 1, 300, 0, 0), (SMALL, 4, 1, 511, 512)])
def test_reference_block_bit_exact_avx2_chain(shape, batch, tokens, past, cache_len):
    """The reference build's block (this host runs its AVX2 kernels) equals
    the oracle's chain of AVX2-order restatements bit for bit: the oracle
    the full-size GPU block tests compare with is the reference's output."""
    s = _ref_session()
    try:
        w32 = weights_f32(shape, "test/avx2")
        got, wq, (x, kc, vc) = _run(s, False, shape, w32, batch, tokens, past, cache_len, "test/avx2")
    finally:
        s.close()
    st = block_oracle.block_stages(shape, wq, w32["norm_attn"], w32["norm_ffn"], x, batch, tokens,
                                   past=past, k_cache=kc, v_cache=vc, avx2=True)
    assert np.array_equal(got.view(np.uint32), st["out"].view(np.uint32))


@pytest.mark.gpu
@pytest.mark.parametrize("shape,batch,tokens,past,cache_len",
                         CASES + [(SMALL, 1, 300, 0, 0), (SMALL, 4, 1, 511, 512)])
def test_gpu_block_matches_oracle(gpu, shape, batch, tokens, past, cache_len):
    w32 = weights_f32(shape, "test/block")
    got, wq, inputs = _run(gpu, True, shape, w32, batch, tokens, past, cache_len, "test/block")
    want = _oracle(shape, w32, wq, inputs, batch, tokens, past)
    assert np.isfinite(got).all()
    assert oracle.rel_error(got, want) <= TOL


def test_block_stages_equals_block():
    """The staged oracle the full-size tests use (BLAS int8 GEMMs, threaded
    attention) is bit-identical to the plain composition."""
    w32 = weights_f32(TINY, "test/stages")
    wq = {n: oracle.quantize(w32[n], 1) for n in PROJECTIONS}
    for batch, tokens, past, cache_len in ((1, 37, 0, 0), (3, 2, 20, 22)):
        x, kc, vc = _inputs(TINY, batch, tokens, cache_len, "test/stages")
        a = block_oracle.block(TINY, wq, w32["norm_attn"], w32["norm_ffn"], x, batch, tokens,
                               past=past, k_cache=kc, v_cache=vc)
        st = block_oracle.block_stages(TINY, wq, w32["norm_attn"], w32["norm_ffn"], x, batch, tokens,
                                       past=past, k_cache=kc, v_cache=vc)
        assert np.array_equal(a.view(np.uint32), st["out"].view(np.uint32))


# The north-star bar for the block: within 2e-3 max-rel of the reference's
# block output (the oracle's AVX2-order chain).  The default device computes
# ATTENTION_F32 in the reference's order, so its block is bit-exact.  A device
# created with VNPU_CONFIG_HIGH_THROUGHPUT runs the split-bf16 attention:
# every other stage is still bit-exact on its input, but attention's ~1e-7
# summation-order differences flip a few int8 roundings at the three quantize
# stages after it, and each flip moves later stages by a whole int8 step
# (measured on MI355X: decode 9.9e-3, prefill 1.55e-2 end to end), so that
# mode misses the bar and is reported as an expected failure.
NORTH_STAR_TOL = 2e-3


def _full_block(gpu, B, T, past, ctx, tag):
    shape = LLAMA_4096
    d, H, D, F = shape.d_model, shape.heads, shape.head_dim, shape.ffn
    w32 = weights_f32(shape, "config4")
    blk = Block(gpu, shape, w32)
    try:
        blk.prepare(B, T, past=past, cache_len=ctx)
        x0, kc0, vc0 = _inputs(shape, B, T, ctx, tag)
        blk.set_input(x0, kc0, vc0)
        blk.run(True)
        rows = B * T
        get = lambda n, shp: gpu.download(blk.bufs[n], np.float32, shp)
        wq = {n: blk.quantized_weights(n) for n in PROJECTIONS}
        out = {"qkv": get("qkv", (rows, 3 * d)), "q": get("q", (B, H, T, D)), "k": get("k", (B, H, T, D)),
               "v": get("v", (B, H, T, D)), "o": get("o", (B, H, T, D)),
               # one token per sequence: the harness feeds the O projection the
               # attention output itself ([B][H][1][D] is the [B][H*D] layout)
               "att": get("o" if T == 1 else "att", (rows, d)),
               "gate": get("gate", (rows, F)), "up": get("up", (rows, F)), "ff": get("ff", (rows, F)),
               "down": get("proj", (rows, d)), "x": get("x", (rows, d)), "xn2": get("xn", (rows, d))}
        if ctx:
            kv = (B, H, ctx, D)
            out["k_cache"], out["v_cache"] = get("k_cache", kv), get("v_cache", kv)
    finally:
        blk.close()
    # The first RMSNorm's output is overwritten by the second inside the
    # block: the same op alone on the GPU (its row kernel is the block's, bit
    # for bit, tests/test_gpu_rowchain.py) gives the GPU's first quantize input.
    import gpu_ops as g
    out["xn1"] = g.unary_rows(gpu, abi.OP_RMSNORM_F32, x0, W=w32["norm_attn"], eps=1e-5)
    return shape, w32, wq, (x0, kc0, vc0), out


def _check_stages(shape, w32, wq, inputs, gpu_out, B, T, past, ctx, exact):
    """Each op's GPU output against the oracle's restatement of the
    reference's AVX2 build applied to the GPU's own input of that stage:
    every stage bit-exact except attention on a high-throughput device
    (within 2e-3).
    Then the whole block against the oracle's chain from the same x, which is
    the reference's block output bit for bit
    (test_reference_block_bit_exact_avx2_chain).  Returns (end-to-end error,
    per-stage int8 flip counts, attention error)."""
    d, H, D = shape.d_model, shape.heads, shape.head_dim
    x0, kc0, vc0 = inputs
    G = gpu_out

    def gemm(a, name):
        a8, sa = oracle.quantize(a, 0)
        return oracle.matmul_i8_blas(a8, wq[name][0], sa, wq[name][1])

    def heads(part):
        return np.ascontiguousarray(part.reshape(B, T, H, D).transpose(0, 2, 1, 3))

    bits = lambda a, b: np.array_equal(a.view(np.uint32), b.view(np.uint32))
    assert bits(G["xn1"], oracle.rmsnorm_avx2(x0, w32["norm_attn"], 1e-5))
    assert bits(G["qkv"], gemm(G["xn1"], "qkv"))
    qr, kr = oracle.rope(heads(G["qkv"][:, :d]), heads(G["qkv"][:, d:2 * d]), position_offset=past)
    assert bits(G["q"], qr) and bits(G["k"], kr)
    assert np.array_equal(G["v"], heads(G["qkv"][:, 2 * d:]))
    if ctx:
        kc, vc = G["k_cache"], G["v_cache"]
        assert np.array_equal(kc[:, :, past:past + T], G["k"]) and np.array_equal(vc[:, :, past:past + T], G["v"])
        assert np.array_equal(kc[:, :, :past], kc0[:, :, :past])
    else:
        kc, vc = G["k"], G["v"]
    want_o = block_oracle.attention_threaded(G["q"], kc, vc, 1, avx2=True)
    att_err = oracle.rel_error(G["o"], want_o)
    assert bits(G["o"], want_o) if exact else att_err <= TOL
    assert np.array_equal(G["att"], G["o"].transpose(0, 2, 1, 3).reshape(B * T, d))
    # x after the attention residual is not kept by the harness: rebuild it
    # from the GPU's attention output (exact integer GEMM, the oracle's add).
    x1 = oracle.add(x0, gemm(G["att"], "o"), 1.0, 1.0)
    assert bits(G["xn2"], oracle.rmsnorm_avx2(x1, w32["norm_ffn"], 1e-5))
    assert bits(G["gate"], gemm(G["xn2"], "gate")) and bits(G["up"], gemm(G["xn2"], "up"))
    assert bits(G["ff"], oracle.swiglu_avx2(G["gate"], G["up"], 1.0))
    assert bits(G["down"], gemm(G["ff"], "down"))
    assert bits(G["x"], oracle.add(x1, G["down"], 1.0, 1.0))
    assert np.isfinite(G["x"]).all()

    st = block_oracle.block_stages(shape, wq, w32["norm_attn"], w32["norm_ffn"], x0, B, T, past=past,
                                   k_cache=kc0, v_cache=vc0, avx2=True)
    e2e = oracle.rel_error(G["x"], st["out"])
    fl = {n: block_oracle.flips(G[n], st[n]) for n in ("xn1", "att", "xn2", "ff")}
    if exact:
        assert bits(G["x"], st["out"])
    return e2e, fl, att_err


MODES = [pytest.param(False, id="high-throughput"), pytest.param(True, id="reference-order")]


def _e2e_bar(e2e, exact, what):
    if exact:
        assert e2e <= NORTH_STAR_TOL
    elif e2e > NORTH_STAR_TOL:
        pytest.xfail(f"{what} on a VNPU_CONFIG_HIGH_THROUGHPUT device: end to end {e2e:.3g} > 2e-3 "
                     "(split-bf16 attention flips int8 roundings downstream; the default device is bit-exact)")


@pytest.mark.gpu
@pytest.mark.parametrize("exact", MODES)
def test_gpu_block_full_decode_stagewise(request, exact):
    """Config 4 decode at full size (batch 8, context 4096, new token at 4095).

    Stage by stage, each op's GPU output against the oracle applied to the
    GPU's own input of that stage: bit-exact (attention within 2e-3 on a
    high-throughput device).  End to end the block is compared with the
    reference's block output (the oracle's AVX2-order chain) from the same
    input, and the number of int8 elements that differ at each of the four
    per-row quantize stages is printed.  On the default device the whole
    block is bit-exact.
    """
    gpu = request.getfixturevalue("gpu" if exact else "fast_gpu")
    B, T, ctx = 8, 1, 4096
    shape, w32, wq, inputs, G = _full_block(gpu, B, T, ctx - 1, ctx, "config4/decode")
    e2e, fl, att_err = _check_stages(shape, w32, wq, inputs, G, B, T, ctx - 1, ctx, exact)
    print(f"\n[block decode B8 ctx4096 {'reference-order' if exact else 'high-throughput'}] attention {att_err:.3g}, "
          f"end to end {e2e:.3g}, int8 flips per stage (elements, scales): {fl}", flush=True)
    _e2e_bar(e2e, exact, "block decode")


@pytest.mark.gpu
@pytest.mark.parametrize("exact", MODES)
def test_gpu_block_full_prefill_stagewise(request, exact):
    """Config 4 prefill at full size (batch 1, 2048 tokens, causal), with the
    same stage-by-stage bars and end-to-end report as the decode test."""
    gpu = request.getfixturevalue("gpu" if exact else "fast_gpu")
    B, T = 1, 2048
    shape, w32, wq, inputs, G = _full_block(gpu, B, T, 0, 0, "config4/prefill")
    e2e, fl, att_err = _check_stages(shape, w32, wq, inputs, G, B, T, 0, 0, exact)
    print(f"\n[block prefill B1 S2048 {'reference-order' if exact else 'high-throughput'}] attention {att_err:.3g}, "
          f"end to end {e2e:.3g}, int8 flips per stage (elements, scales): {fl}", flush=True)
    _e2e_bar(e2e, exact, "block prefill")
