"""Row chains on the MI355X backend: ADD -> RMSNORM [-> QUANTIZE_I8 per row],
RMSNORM -> QUANTIZE_I8 and SWIGLU -> QUANTIZE_I8 submitted in one batch run as
one row kernel.  Whatever the backend does with them, the outputs must be the
bits the same commands give when each is submitted in a batch of its own (the
single-op kernels), and those are held to the oracle (reference
src/kernels/llm.cpp:64-108 RMSNorm, 240-271 SwiGLU/add, 387-436 quantize).

The reference runs every command on its own (src/core/scheduler.cpp:430-581);
the chain is this backend's scheduling, so "fused == one by one, bit for bit"
is the parity property, with aliasing (in-place ADD as the transformer block
issues it, in-place RMSNORM, an output that overlaps another command's input)
covered because it decides whether the chain may run row by row."""
import numpy as np
import pytest

import oracle
from vnpu_mi355x import abi

pytestmark = pytest.mark.gpu

RNG = np.random.default_rng(20261207)
KINDS = ["add_norm_quant", "add_norm", "norm_quant", "swiglu_quant"]
# (rows, cols): the block's d_model and FFN rows, odd row counts, a short row,
# and 12300 columns (beyond the register-resident row length: single kernels);
# 256 rows or more take SWIGLU -> QUANTIZE's 256-thread kernels (4, 8 and 12
# float4 slots per thread by row length).
SHAPES = [(8, 4096), (64, 4096), (5, 11008), (3, 12288), (6, 100), (2, 12300), (1, 4), (300, 4096), (260, 6000),
          (256, 11008)]


def _inputs(kind, rows, cols):
    x = (RNG.standard_normal((rows, cols)) * 2).astype(np.float32)
    y = RNG.standard_normal((rows, cols)).astype(np.float32)
    w = (RNG.random(cols) + 0.5).astype(np.float32)
    return x, y, w


def _run(gpu, kind, rows, cols, alias, fused, params, overlap=False):
    """Builds the chain over fresh buffers; returns the named outputs."""
    x, y, w = params["x"], params["y"], params["w"]
    n = rows * cols
    bx, by, bw = gpu.upload(x), gpu.upload(y), gpu.upload(w)
    bo, bn = gpu.alloc(4 * n), gpu.alloc(4 * n)
    bq, bs = gpu.alloc(n), gpu.alloc(4 * rows)
    q_ptr = by.ptr if overlap else bq.ptr   # quantize output over the second input
    eps = params["eps"]
    cmds, outs = [], {}
    if kind.startswith("add"):
        first_out = bx if alias else bo    # in place: x = x + y, as the block issues it
        cmds.append(gpu.command(abi.OP_ADD_F32, A=bx, B=by, Y=first_out, count=n,
                                alpha=params["alpha"], beta=params["beta"]))
        norm_out = first_out if (alias and kind == "add_norm") else bn
        cmds.append(gpu.command(abi.OP_RMSNORM_F32, X=first_out, W=bw, Y=norm_out, rows=rows,
                                cols=cols, eps=eps))
        outs["sum"], outs["norm"], q_src = first_out, norm_out, norm_out
    elif kind == "norm_quant":
        norm_out = bx if alias else bn     # in-place RMSNORM
        cmds.append(gpu.command(abi.OP_RMSNORM_F32, X=bx, W=0 if params["no_w"] else bw,
                                Y=norm_out, rows=rows, cols=cols, eps=eps))
        outs["norm"], q_src = norm_out, norm_out
    else:
        ff = by if alias else bo           # SWIGLU writing over its up operand
        cmds.append(gpu.command(abi.OP_SWIGLU_F32, gate=bx, up=by, Y=ff, count=n,
                                alpha=params["alpha"]))
        outs["ff"], q_src = ff, ff
    if kind.endswith("quant"):
        cmds.append(gpu.command(abi.OP_QUANTIZE_I8, X=q_src, Y=q_ptr, scales=bs, rows=rows,
                                cols=cols, axis=abi.QUANT_PER_ROW))
    if fused:
        assert gpu.submit(cmds) == abi.OK
    else:
        for c in cmds:
            assert gpu.submit([c]) == abi.OK
    assert gpu.sync() == abi.OK
    got = {k: gpu.download(b, np.float32, (rows, cols)) for k, b in outs.items()}
    if kind.endswith("quant"):
        got["q"] = gpu.download(q_ptr, np.int8, (rows, cols))
        got["scales"] = gpu.download(bs, np.float32, (rows,))
    got["x"] = gpu.download(bx, np.float32, (rows, cols))
    got["y"] = gpu.download(by, np.float32, (rows, cols))
    for b in (bx, by, bw, bo, bn, bq, bs):
        gpu.free(b)
    return got


def _params(kind, rows, cols, **over):
    x, y, w = _inputs(kind, rows, cols)
    p = {"x": x, "y": y, "w": w, "eps": 1e-6, "alpha": 1.0, "beta": 1.0, "no_w": False}
    p.update(over)
    return p


def _same_bits(a, b):
    for k in a:
        assert a[k].dtype == b[k].dtype and a[k].shape == b[k].shape, k
        assert np.array_equal(a[k].view(np.uint8), b[k].view(np.uint8)), f"{k} differs"


@pytest.mark.parametrize("alias", [False, True])
@pytest.mark.parametrize("rows,cols", SHAPES)
@pytest.mark.parametrize("kind", KINDS)
def test_chain_equals_commands_one_by_one(gpu, kind, rows, cols, alias):
    p = _params(kind, rows, cols)
    fused = _run(gpu, kind, rows, cols, alias, True, p)
    single = _run(gpu, kind, rows, cols, alias, False, p)
    _same_bits(fused, single)
    # The single-op results against the oracle (the tolerances of the
    # single-op tests); the quantize stage bit-exact on the float rows the
    # backend produced (scale and every code).
    x, y, w = p["x"], p["y"], p["w"]
    if kind.startswith("add"):
        want_sum = oracle.add(x, y)
        if not (alias and kind == "add_norm"):  # else the norm overwrote the sum
            assert oracle.rel_error(fused["sum"], want_sum) <= 1e-6
        want_norm = oracle.rmsnorm(want_sum, w, 1e-6)
        assert oracle.rel_error(fused["norm"], want_norm) <= 1e-5
        src = fused["norm"]
    elif kind == "norm_quant":
        assert oracle.rel_error(fused["norm"], oracle.rmsnorm(x, w, 1e-6)) <= 1e-5
        src = fused["norm"]
    else:
        assert oracle.rel_error(fused["ff"], oracle.swiglu(x, y)) <= 1e-5
        src = fused["ff"]
    if kind.endswith("quant"):
        q, s = oracle.quantize(src, abi.QUANT_PER_ROW)
        assert np.array_equal(fused["q"], q)
        assert np.array_equal(fused["scales"].view(np.uint32), np.asarray(s, np.float32).view(np.uint32))


def test_swiglu_chain_reference_ranges(gpu):
    """SWIGLU -> QUANTIZE_I8 over 512 x 11004 elements: above 16384 *
    num_threads the reference's SWIGLU ranges (max(4096, n / (4 *
    num_threads))) are not multiples of 8 and each ends in a scalar tail; the
    chain and the commands one by one give the oracle's bits split that way."""
    rows, cols = 512, 11004
    threads = gpu.info().num_threads
    grain = oracle.ew_grain(rows * cols, threads)
    if grain % 8 == 0 or grain >= rows * cols:
        pytest.skip(f"num_threads {threads}: ranges of {grain} elements end on 8-element steps")
    p = _params("swiglu_quant", rows, cols)
    flat = p["x"].reshape(-1)
    for end in list(range(grain, rows * cols, grain)) + [rows * cols]:
        flat[end - 2:end] = (-90.0, -85.0)
    fused = _run(gpu, "swiglu_quant", rows, cols, False, True, p)
    single = _run(gpu, "swiglu_quant", rows, cols, False, False, p)
    _same_bits(fused, single)
    want = oracle.swiglu_avx2(p["x"], p["y"], 1.0, num_threads=threads).reshape(rows, cols)
    assert np.array_equal(fused["ff"].view(np.uint32), want.view(np.uint32))
    q, s = oracle.quantize(want, abi.QUANT_PER_ROW)
    assert np.array_equal(fused["q"], q)


@pytest.mark.parametrize("kind", ["add_norm_quant", "swiglu_quant"])
def test_chain_scalars(gpu, kind):
    """Non-default ADD alpha/beta and SWIGLU alpha, and ADD with alpha = beta
    = 0 (the reference's 'both zero means 1, 1', llm.cpp:226-227)."""
    rows, cols = 7, 4096
    for alpha, beta in [(0.5, -2.0), (0.0, 0.0), (1.5, 0.0)]:
        p = _params(kind, rows, cols, alpha=alpha, beta=beta)
        _same_bits(_run(gpu, kind, rows, cols, False, True, p), _run(gpu, kind, rows, cols, False, False, p))


def test_chain_without_norm_weight(gpu):
    p = _params("norm_quant", 9, 4096, no_w=True)
    _same_bits(_run(gpu, "norm_quant", 9, 4096, False, True, p), _run(gpu, "norm_quant", 9, 4096, False, False, p))


@pytest.mark.parametrize("kind", ["add_norm_quant", "swiglu_quant"])
def test_chain_output_over_an_input(gpu, kind):
    """The quantize output written over the ADD/SWIGLU second operand: a
    cross-row overlap, so the commands must take effect one after another."""
    rows, cols = 16, 4096
    p = _params(kind, rows, cols)
    _same_bits(_run(gpu, kind, rows, cols, False, True, p, overlap=True),
               _run(gpu, kind, rows, cols, False, False, p, overlap=True))


def test_chain_nan_and_zero_rows(gpu):
    """A zero row (scale 1, RMS eps only) and NaN/inf entries go through the
    chain exactly as through the single kernels."""
    rows, cols = 4, 4096
    p = _params("add_norm_quant", rows, cols)
    p["x"][1] = 0.0
    p["y"][1] = 0.0
    p["x"][2, 5] = np.nan
    p["y"][3, 7] = np.inf
    _same_bits(_run(gpu, "add_norm_quant", rows, cols, True, True, p),
               _run(gpu, "add_norm_quant", rows, cols, True, False, p))


@pytest.mark.parametrize("kind", KINDS)
def test_chain_counters_match_commands_one_by_one(gpu, kind):
    """Device counters (bytes, flops, commands) after a chained batch equal
    those after the same commands submitted one per batch: the reference's
    per-command accounting (scheduler.cpp:430-581) does not see the chain."""
    rows, cols = 32, 4096
    p = _params(kind, rows, cols)

    def delta(fused):
        s0 = gpu.status()
        before = (s0.bytes_read, s0.bytes_written, s0.flops, s0.commands_completed)
        _run(gpu, kind, rows, cols, False, fused, p)
        s1 = gpu.status()
        return tuple(a - b for a, b in zip((s1.bytes_read, s1.bytes_written, s1.flops, s1.commands_completed),
                                           before))

    assert delta(True) == delta(False)
