"""GPU parity at the full sizes the bench times (configs 3 and 5), through the C ABI.

Inputs are the bench's own seeded tensors (vnpu_mi355x.synth, same names),
quantized and packed on the GPU exactly as bench.py does; the quantized
tensors are checked against the C oracle bit for bit, then the GEMM outputs
against the oracle's store step on exact float64 BLAS accumulators
(oracle.matmul_i8_blas / matmul_f32_blas, pinned to the scalar oracle in
tests/test_oracle_blas.py).

Bars: int8 tensors, scales and MATMUL_I8 outputs bit-exact; MATMUL_F32 and
the MTP head max|d| / max(1, max|ref|) <= 1e-4; softmax probabilities above
1e-6 within 1e-4 relative, element by element (the normalised metric alone
would accept large relative errors in a 32000-entry tail of ~3e-5 values).
"""
import numpy as np
import pytest

import oracle
from vnpu_mi355x import abi, synth

pytestmark = pytest.mark.gpu
RNG = np.random.default_rng(20261202)


def _quantized_weights(s, K, N, w):
    """Per-column QUANTIZE_I8 of f32 weights on the GPU (as bench.weights_for),
    checked against the oracle; returns (device int8, device scales, host int8,
    host scales)."""
    bw = s.upload(w)
    wq, ws = s.alloc(K * N), s.alloc(4 * N)
    s.run(abi.OP_QUANTIZE_I8, X=bw, Y=wq, scales=ws, rows=K, cols=N, axis=abi.QUANT_PER_COLUMN)
    s.free(bw)
    hq, hs = s.download(wq, np.int8, (K, N)), s.download(ws, np.float32, (N,))
    oq, os_ = oracle.quantize(w, abi.QUANT_PER_COLUMN)
    assert np.array_equal(hs.view(np.uint32), os_.view(np.uint32))
    assert np.array_equal(hq, oq)
    return wq, ws, hq, hs


def _quantized_rows(s, x):
    M, K = x.shape
    bx = s.upload(x)
    a8, sa = s.alloc(M * K), s.alloc(4 * M)
    s.run(abi.OP_QUANTIZE_I8, X=bx, Y=a8, scales=sa, rows=M, cols=K, axis=abi.QUANT_PER_ROW)
    s.free(bx)
    ha, hs = s.download(a8, np.int8, (M, K)), s.download(sa, np.float32, (M,))
    oq, os_ = oracle.quantize(x, abi.QUANT_PER_ROW)
    assert np.array_equal(hs.view(np.uint32), os_.view(np.uint32))
    assert np.array_equal(ha, oq)
    return a8, sa, ha, hs


def _bits_equal(got, want):
    return np.array_equal(np.asarray(got, np.float32).view(np.uint32),
                          np.asarray(want, np.float32).view(np.uint32))


@pytest.mark.parametrize("N", [4096, 14336])
def test_config3_int8_prefill_full(gpu, N):
    """Config 3 int8 at 2048 x 4096 x N on the kernels the bench times (the
    automatic choice: a 256-row wide tile over 32 k stages of 128)."""
    M, K = 2048, 4096
    w = synth.normal(f"w_{K}x{N}", (K, N), 0.02)
    wq, ws, hq, hs = _quantized_weights(gpu, K, N, w)
    del w
    packed = gpu.pack(wq, K, N, scales=ws)
    gpu.free(wq)
    gpu.free(ws)
    a8, sa, ha, has = _quantized_rows(gpu, synth.normal(f"act_{M}x{K}", (M, K)))
    c = gpu.alloc(4 * M * N)
    gpu.run(abi.OP_MATMUL_I8, A=a8, B=packed, scale_a=sa, C=c, M=M, K=K, N=N)
    got = gpu.download(c, np.float32, (M, N))
    gpu.release_packed(packed)
    for b in (a8, sa, c):
        gpu.free(b)
    assert _bits_equal(got, oracle.matmul_i8_blas(ha, hq, has, hs))


@pytest.mark.parametrize("N,epi", [(13000, 1), (14336, 0), (14336, 3)])
def test_int8_mixed_width_grid(gpu, N, epi):
    """2048-row problems whose columns split into whole rounds of 256-wide and
    192-wide tiles on 256 CUs (N in (12288, 14336]): the second range starts
    32 strips into the packed weights, with its own scales, bias and C
    columns; a ragged last tile; bias and activation epilogues (bit-exact up
    to ReLU; GELU within the int8 epilogue bar of 1e-6)."""
    M, K = 2048, 256
    A = RNG.integers(-128, 128, size=(M, K)).astype(np.int8)
    B = RNG.integers(-128, 128, size=(K, N)).astype(np.int8)
    sa = ((RNG.random(M) + 0.5) / 127).astype(np.float32)
    sb = ((RNG.random(N) + 0.5) / 127).astype(np.float32)
    bias = RNG.standard_normal(N).astype(np.float32)
    w = gpu.pack(B, K, N, scales=sb)
    ba, bsa, bb, bc = gpu.upload(A), gpu.upload(sa), gpu.upload(bias), gpu.alloc(4 * M * N)
    gpu.run(abi.OP_MATMUL_I8, A=ba, B=w, scale_a=bsa.ptr, bias=bb.ptr, C=bc, M=M, K=K, N=N, epilogue=epi)
    got = gpu.download(bc, np.float32, (M, N))
    for b in (ba, bsa, bb, bc):
        gpu.free(b)
    gpu.release_packed(w)
    want = oracle.matmul_i8_blas(A, B, sa, sb, bias, epi)
    if epi <= 1:
        assert _bits_equal(got, want)
    else:
        assert oracle.rel_error(got, want) <= 1e-6


def test_int8_pair_k4096_full(gpu):
    """The block's gate/up pair at prefill size (2048 x 4096 x 11008, twice,
    one batch): the paired wide-tile grid over 32 k stages, bit-exact."""
    M, K, N = 2048, 4096, 11008
    a8, sa, ha, has = _quantized_rows(gpu, RNG.standard_normal((M, K)).astype(np.float32))
    outs, wants, packs = [], [], []
    for i in range(2):
        B = RNG.integers(-128, 128, (K, N)).astype(np.int8)
        sb = (RNG.random(N).astype(np.float32) + 0.5) / 127
        packs.append(gpu.pack(B, K, N, scales=sb))
        wants.append(oracle.matmul_i8_blas(ha, B, has, sb))
        outs.append(gpu.alloc(4 * M * N))
    cmds = [gpu.command(abi.OP_MATMUL_I8, A=a8, B=packs[i], scale_a=sa, C=outs[i], M=M, K=K, N=N)
            for i in range(2)]
    gpu.check("submit", gpu.submit(cmds))
    gpu.check("sync", gpu.sync())
    for i in range(2):
        assert _bits_equal(gpu.download(outs[i], np.float32, (M, N)), wants[i]), f"command {i}"
        gpu.release_packed(packs[i])
        gpu.free(outs[i])
    gpu.free(a8)
    gpu.free(sa)


@pytest.mark.parametrize("N", [4096, 14336])
def test_config3_f32_prefill_full(gpu, N):
    """Config 3 f32: B stored [N][K] (trans_b), bias, alpha 1, beta 0.5 onto
    C, GELU - the bench's tensors, against a float64 accumulator."""
    M, K = 2048, 4096
    a = synth.normal(f"c3/A_{M}x{K}", (M, K))
    bt = synth.normal(f"c3/Bt_{N}x{K}", (N, K), 0.02)
    bias = synth.normal(f"c3/bias_{N}", (N,), 0.1)
    c0 = synth.normal(f"c3/C_{M}x{N}", (M, N))
    ba, bb, bbias, bc = gpu.upload(a), gpu.upload(bt), gpu.upload(bias), gpu.upload(c0)
    gpu.run(abi.OP_MATMUL_F32, A=ba, B=bb, bias=bbias, C=bc, M=M, K=K, N=N, trans_b=1, alpha=1.0,
            beta=0.5, epilogue=abi.EPI_GELU_TANH)
    got = gpu.download(bc, np.float32, (M, N))
    for b in (ba, bb, bbias, bc):
        gpu.free(b)
    want = oracle.matmul_f32_blas(a, bt, c0, bias, 0, 1, 1.0, 0.5, abi.EPI_GELU_TANH)
    assert np.isfinite(got).all()
    assert oracle.rel_error(got, want) <= 1e-4


@pytest.mark.parametrize("M,K,N", [(2000, 1000, 4100), (1700, 1000, 4700), (2048, 520, 14336), (1024, 4096, 2048),
                                   (1536, 4096, 1536), (1000, 3000, 1900), (2048, 2048, 2048)])
@pytest.mark.parametrize("tb", [0, 1])
def test_f32_last_round_k_split(gpu, M, K, N, tb):
    """Grids of 256 x 128 tiles whose last round fills at most half of the
    256 CUs (264, 259 and 896 tiles): those tiles run as two workgroups over
    half of K each, then a second pass adds the halves and applies alpha,
    bias, beta and the epilogue.  Grids of fewer tiles than CUs (64, 72, 60
    and 128 tiles) run every tile as 4, 3, 4 or 2 K slices the same way.
    Ragged M / N / K edges land in the split tiles; 259 and 60 tiles also
    skip the XCD remap (not a multiple of 8)."""
    a = RNG.standard_normal((M, K), dtype=np.float32)
    b = (RNG.standard_normal((N, K) if tb else (K, N), dtype=np.float32) * 0.05).astype(np.float32)
    bias = RNG.standard_normal(N, dtype=np.float32) * 0.1
    c0 = RNG.standard_normal((M, N), dtype=np.float32)
    ba, bb, bbias, bc = gpu.upload(a), gpu.upload(b), gpu.upload(bias), gpu.upload(c0)
    gpu.run(abi.OP_MATMUL_F32, A=ba, B=bb, bias=bbias, C=bc, M=M, K=K, N=N, trans_b=tb, alpha=0.75,
            beta=0.5, epilogue=abi.EPI_GELU_TANH)
    got = gpu.download(bc, np.float32, (M, N))
    for x in (ba, bb, bbias, bc):
        gpu.free(x)
    want = oracle.matmul_f32_blas(a, b, c0, bias, 0, tb, 0.75, 0.5, abi.EPI_GELU_TANH)
    assert np.isfinite(got).all()
    assert oracle.rel_error(got, want) <= 1e-4


def test_config5_cull_int8_4096_full(gpu):
    """Config 5: 4096^3 int8 with half of the 64 x 64 weight tiles zeroed by
    the seeded Bernoulli mask (the bench's tensors), bit-exact."""
    M = K = N = 4096
    w = synth.normal("c5/W", (K, N), 0.02)
    keep = synth.bernoulli_mask("c5/tiles", (K // 64, N // 64), 0.5)
    w *= np.kron(keep, np.ones((64, 64), np.uint8)).astype(np.float32)
    wq, ws, hq, hs = _quantized_weights(gpu, K, N, w)
    del w
    packed = gpu.pack(wq, K, N, scales=ws)
    gpu.free(wq)
    gpu.free(ws)
    a8, sa, ha, has = _quantized_rows(gpu, synth.normal("c5/A", (M, K)))
    c = gpu.alloc(4 * M * N)
    gpu.run(abi.OP_MATMUL_I8, A=a8, B=packed, scale_a=sa, C=c, M=M, K=K, N=N)
    got = gpu.download(c, np.float32, (M, N))
    gpu.release_packed(packed)
    for b in (a8, sa, c):
        gpu.free(b)
    assert 0.45 < keep.mean() < 0.55
    assert _bits_equal(got, oracle.matmul_i8_blas(ha, hq, has, hs))


def test_config5_cull_int8_4096_mask_passed_in(gpu):
    """Config 5 with the mask passed in: the dense weights quantized per
    column, the seeded Bernoulli 64 x 64 tile mask handed to
    vnpu_pack_weights_i8_masked, bit-exact with the oracle on the quantized
    weights with the culled tiles zeroed."""
    M = K = N = 4096
    w = synth.normal("c5/W", (K, N), 0.02)
    keep = synth.bernoulli_mask("c5/tiles", (K // 64, N // 64), 0.5)
    wq, ws, hq, hs = _quantized_weights(gpu, K, N, w)
    del w
    packed = gpu.pack(wq, K, N, scales=ws, tile_mask=keep)
    gpu.free(wq)
    gpu.free(ws)
    a8, sa, ha, has = _quantized_rows(gpu, synth.normal("c5/A", (M, K)))
    c = gpu.alloc(4 * M * N)
    gpu.run(abi.OP_MATMUL_I8, A=a8, B=packed, scale_a=sa, C=c, M=M, K=K, N=N)
    got = gpu.download(c, np.float32, (M, N))
    gpu.release_packed(packed)
    for b in (a8, sa, c):
        gpu.free(b)
    hq *= np.kron(keep, np.ones((64, 64), np.uint8)).astype(np.int8)
    assert _bits_equal(got, oracle.matmul_i8_blas(ha, hq, has, hs))


def test_config5_mtp_head_softmax_full(gpu):
    """Config 5: MTP head [4,4096] x [4096,32000] f32 then SOFTMAX over the
    vocabulary, one batch (the bench's tensors)."""
    G, H, V = 4, 4096, 32000
    hid = synth.normal("c5/hidden", (G, H))
    wm = synth.normal("c5/mtp_W", (H, V), 0.02)
    bh, bw = gpu.upload(hid), gpu.upload(wm)
    logits, probs = gpu.alloc(4 * G * V), gpu.alloc(4 * G * V)
    gpu.check("submit", gpu.submit([
        gpu.command(abi.OP_MTP_HEAD_F32, hidden=bh, W=bw, logits=logits, gamma=G, hidden_dim=H, vocab=V),
        gpu.command(abi.OP_SOFTMAX_F32, X=logits, Y=probs, rows=G, cols=V)]))
    gpu.check("sync", gpu.sync())
    gl = gpu.download(logits, np.float32, (G, V))
    gp = gpu.download(probs, np.float32, (G, V))
    for b in (bh, bw, logits, probs):
        gpu.free(b)
    want_l = oracle.matmul_f32_blas(hid, wm)
    assert oracle.rel_error(gl, want_l) <= 1e-4
    # the probabilities against the reference's AVX2 softmax of the float64
    # logits rounded to f32, every element (relative to each one)
    want_p = oracle.softmax_avx2(want_l, 1.0)
    assert (want_p > 0).all()
    relp = np.abs(gp.astype(np.float64) - want_p) / want_p
    assert relp.max() <= 1e-4, f"max relative probability error {relp.max():.3g}"
    assert np.allclose(gp.sum(axis=1), 1.0, atol=1e-5)
    # the softmax step alone, on the GPU's own logits: each weight is the
    # reference's bit for bit, only the order of the row sum differs
    own = oracle.softmax_avx2(gl, 1.0)
    relo = np.abs(gp.astype(np.float64) - own) / own
    print(f"\n[config5 softmax] elementwise vs the AVX2 softmax of the GPU's logits: {relo.max():.3g}", flush=True)
    assert relo.max() <= 1e-5


@pytest.mark.parametrize("b,h,sq,sk,d,causal", [
    (1, 2, 1, 100, 128, 0), (2, 3, 1, 5000, 128, 1), (1, 2, 4, 3000, 64, 0), (2, 2, 2, 40, 32, 1),
    (1, 2, 64, 200, 128, 1), (1, 2, 150, 700, 64, 0), (1, 2, 20, 50, 80, 0), (1, 1, 1, 1, 128, 0)])
@pytest.mark.parametrize("dev", ["gpu", "fast_gpu"])
def test_attention_neg_inf_mask(request, dev, b, h, sq, sk, d, causal):
    """Additive masks holding -inf (padding): leading keys masked, scattered
    -inf entries and one fully masked query row, on the decode kernel (one
    split and several), the prefill kernel and the generic kernel.  A fully
    masked row is 0, as in the reference (l = 0 -> inv 0).  Both device modes."""
    import gpu_ops as g
    gpu = request.getfixturevalue(dev)
    Q = RNG.standard_normal((b, h, sq, d)).astype(np.float32)
    K = RNG.standard_normal((b, h, sk, d)).astype(np.float32)
    V = RNG.standard_normal((b, h, sk, d)).astype(np.float32)
    mask = RNG.standard_normal((b, h, sq, sk)).astype(np.float32)
    mask[..., : max(1, sk // 3)] = -np.inf
    mask[RNG.random(mask.shape) < 0.2] = -np.inf
    mask[0, 0, sq - 1, :] = -np.inf
    if sk > 1:
        mask[..., -1] = 0.0   # every other row keeps at least one key
        mask[0, 0, sq - 1, -1] = -np.inf
    got = g.attention(gpu, Q, K, V, mask, causal)
    want = oracle.attention(Q, K, V, mask, causal)
    assert np.isfinite(got).all()
    assert np.all(got[0, 0, sq - 1] == 0.0)
    assert oracle.rel_error(got, want) <= 2e-3


def test_matmul_f32_infinite_and_huge_operands(gpu):
    """MATMUL_F32 on the split-bf16 path (>= 128 tiles) with infinite and
    near-FLT_MAX finite operands: a row holding +inf at k0 gives
    +-inf with the sign of B[k0, n] (the f32 product's), a near-FLT_MAX finite
    entry stays finite, and every other row keeps the 1e-4 bar."""
    import gpu_ops as g
    M, K, N = 1024, 512, 2048
    A = RNG.standard_normal((M, K)).astype(np.float32)
    B = (RNG.standard_normal((K, N)).astype(np.float32) + 3.0) * np.where(RNG.random((K, N)) < 0.5, 1, -1)
    B = B.astype(np.float32)   # |B| >= ~0 and away from zero in most entries
    A[5, 17] = np.inf
    A[9, 3] = -np.inf
    A[12, 40] = 3.4e38 / 4096
    B[100, :] *= 1e-3
    A[20, 100] = 3.4e38       # times 1e-3 * |B|: finite
    got = g.matmul_f32(gpu, A, B, M, K, N)
    inf_rows = {5: (17, 1.0), 9: (3, -1.0)}
    for r, (k0, sgn) in inf_rows.items():
        want = np.where(B[k0] > 0, sgn * np.inf, -sgn * np.inf)
        nz = B[k0] != 0
        assert np.array_equal(got[r][nz], want[nz]), f"row {r}"
    fin = np.setdiff1d(np.arange(M), list(inf_rows))
    assert np.isfinite(got[fin]).all()
    want = oracle.matmul_f32_blas(A[fin], B)
    huge = np.isin(fin, [12, 20])
    for r in np.nonzero(huge)[0]:   # each huge row on its own scale
        assert np.max(np.abs(got[fin[r]] - want[r])) <= 1e-4 * np.max(np.abs(want[r]))
    assert oracle.rel_error(got[fin[~huge]], want[~huge]) <= 1e-4


def test_forced_f32_depth_large_grid(gpu):
    """A 128 x 64 x 128 device tile triple forces a 64-deep f32 K split;
    on a 2048 x 4096 x 4096 grid its split-K workspace is capped (256 MiB),
    and the result keeps the f32 bar."""
    M, K, N = 2048, 4096, 4096
    A = RNG.standard_normal((M, K)).astype(np.float32)
    B = (RNG.standard_normal((K, N)) * 0.02).astype(np.float32)
    info0 = gpu.info()
    assert gpu.lib.vnpu_device_set_tiles(gpu.dev, 128, 64, 128) == abi.OK
    try:
        import gpu_ops as g
        got = g.matmul_f32(gpu, A, B, M, K, N)
    finally:
        gpu.lib.vnpu_device_set_tiles(gpu.dev, info0.tile_m, info0.tile_k, info0.tile_n)
    assert oracle.rel_error(got, oracle.matmul_f32_blas(A, B)) <= 1e-4


@pytest.mark.parametrize("b,h,sq,sk,d,causal,use_mask", [
    (1, 2, 5, 40, 320, 1, False), (2, 1, 3, 150, 1024, 0, True), (1, 2, 70, 70, 264, 1, True),
    (1, 70000, 1, 5, 8, 1, False), (2, 40000, 2, 3, 32, 0, True)])
@pytest.mark.parametrize("dev", ["gpu", "fast_gpu"])
def test_attention_wide_heads_and_many_heads(request, dev, b, h, sq, sk, d, causal, use_mask):
    """head_dim above 256 and more than 65535 (batch, head) pairs: the
    row-wise kernel (the reference takes any head_dim and any count)."""
    import gpu_ops as g
    gpu = request.getfixturevalue(dev)
    Q = RNG.standard_normal((b, h, sq, d)).astype(np.float32)
    K = RNG.standard_normal((b, h, sk, d)).astype(np.float32)
    V = RNG.standard_normal((b, h, sk, d)).astype(np.float32)
    mask = RNG.standard_normal((b, h, sq, sk)).astype(np.float32) if use_mask else None
    if use_mask:
        mask[..., 0] = -np.inf
    got = g.attention(gpu, Q, K, V, mask, causal)
    want = oracle.attention(Q, K, V, mask, causal)
    assert np.isfinite(got).all()
    assert oracle.rel_error(got, want) <= 2e-3


def test_config1_exact_calls(gpu):
    """Config 1 as the bench times it (the same seeded tensors): MATMUL_F32
    512^3 with B not transposed, bias ~ N(0, 0.1), alpha 1, beta 0 and SiLU
    against the documented semantics silu(A.B + bias) with float64 sums (the
    reference's VNPU_PACK=0 result; its default packed path applies the
    epilogue after the first K block, kernels.cpp:313-323), every element
    within 1e-4 of the output's scale, twice with identical bits; and the
    int8 half (per-row QUANTIZE_I8 of A, per-column of B, PACK, MATMUL_I8)
    bit for bit."""
    import gpu_ops as g
    M = K = N = 512
    a = synth.normal("c1/A", (M, K))
    b = synth.normal("c1/B", (K, N), 0.02)
    bias = synth.normal("c1/bias", (N,), 0.1)
    got = g.matmul_f32(gpu, a, b, M, K, N, bias=bias, alpha=1.0, beta=0.0, epilogue=abi.EPI_SILU)
    again = g.matmul_f32(gpu, a, b, M, K, N, bias=bias, alpha=1.0, beta=0.0, epilogue=abi.EPI_SILU)
    want = oracle.matmul_f32(a, b, None, bias, M, K, N, 0, 0, 1.0, 0.0, abi.EPI_SILU, acc64=True)
    assert np.array_equal(got.view(np.uint32), again.view(np.uint32))
    assert np.abs(got - want).max() <= 1e-4 * np.abs(want).max()
    assert oracle.rel_error(got, want) <= 1e-4
    a8, sa = g.quantize(gpu, a, abi.QUANT_PER_ROW)
    b8, sb = g.quantize(gpu, b, abi.QUANT_PER_COLUMN)
    oa8, osa = oracle.quantize(a, abi.QUANT_PER_ROW)
    ob8, osb = oracle.quantize(b, abi.QUANT_PER_COLUMN)
    assert np.array_equal(a8, oa8) and np.array_equal(b8, ob8)
    assert _bits_equal(sa, osa) and _bits_equal(sb, osb)
    w = gpu.pack(b8, K, N, scales=sb)
    try:
        c = g.matmul_i8(gpu, a8, w, M, K, N, scale_a=sa)
    finally:
        gpu.release_packed(w)
    assert _bits_equal(c, oracle.matmul_i8(oa8, ob8, osa, osb))
