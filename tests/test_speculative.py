"""vnpu_speculative_step: the host logic of MTP-style speculative decoding.

Reference: src/cluster/cluster.cpp:552-646 (the step), :178-229 (argmax,
xorshift64, sampling) and tools/selftest.cpp:141-157,550-567 (the toy
logits callback and its checks).  The step runs on the host around the
caller's two logits callbacks, so the CPU tests below call it in
``libvnpu.so`` without a GPU and compare every output with the reference
runtime built from its own sources (``oracle/_ref``).  The GPU test backs both
callbacks with OP_MTP_HEAD_F32 on the MI355X and replays the logits it
produced through the reference step, token for token.

Pins that do not use the reference build: greedy steps follow the toy
callback's successor chain exactly; a vocabulary with one finite logit always
samples that token; sampled frequencies follow softmax(logits / T).
"""
import ctypes as C
import os

import numpy as np
import pytest

import oracle
from vnpu_mi355x import abi, load_backend


@pytest.fixture(scope="module")
def lib():
    return load_backend()


@pytest.fixture(scope="module")
def reflib():
    if not os.path.exists(oracle.REF_LIB_PATH):
        pytest.skip("reference build oracle/_ref/libvnpu_ref.so not present")
    return abi.bind(C.CDLL(oracle.REF_LIB_PATH))


def make_config(lib, **kw):
    cfg = abi.SpeculativeConfig()
    lib.vnpu_speculative_config_init(C.byref(cfg))
    for k, v in kw.items():
        setattr(cfg, k, v)
    return cfg


class Logits:
    """A vnpu_logits_fn_t backed by a Python function of (tokens, first, count).

    ``fn`` returns a (count, vocab) float32 array; every call is recorded so a
    test can check what the step asked for."""

    def __init__(self, fn):
        self.fn = fn
        self.calls = []
        self.status = abi.OK
        self.c = abi.LOGITS_FN(self._call)

    def _call(self, user, tokens, num_tokens, first, count, out, vocab):
        toks = np.ctypeslib.as_array(tokens, (num_tokens,)).copy() if num_tokens else np.zeros(0, np.int32)
        self.calls.append((toks, first, count))
        if self.status != abi.OK:
            return self.status
        vals = np.asarray(self.fn(toks, first, count, vocab), np.float32).reshape(count * vocab)
        np.ctypeslib.as_array(out, (count * vocab,))[:] = vals
        return abi.OK


def step(lib, cfg, context, draft, verify):
    ctx = np.ascontiguousarray(context, np.int32)
    res = abi.SpeculativeResult()
    rc = lib.vnpu_speculative_step(None, C.byref(cfg),
                                   ctx.ctypes.data if len(ctx) else None, len(ctx),
                                   draft.c, None, verify.c, None, C.byref(res))
    return rc, res


def outcome(rc, res):
    return rc, res.accepted, res.produced, res.eos, list(res.tokens[:res.produced])


def toy(tokens, first, count, vocab):
    """tools/selftest.cpp:141-157: logits peak at (token + 1) mod vocab."""
    out = np.empty((count, vocab), np.float32)
    v = np.arange(vocab)
    for p in range(count):
        t = int(tokens[min(len(tokens) - 1, p)])
        out[p] = -np.abs(v - (t + 1) % vocab).astype(np.float32)
    return out


def hashed(salt, scale=3.0, specials=False):
    """Deterministic pseudo-random logits for a position given its prefix.

    The value depends only on (salt, prefix tokens, position), so the draft and
    verify callbacks of two libraries see identical logits for identical
    requests.  ``specials`` plants -inf / NaN / +inf-free holes."""

    def fn(tokens, first, count, vocab):
        out = np.empty((count, vocab), np.float32)
        for p in range(count):
            pos = first + p
            key = hash((salt, tuple(int(t) for t in tokens[:pos]), pos)) & 0xFFFFFFFF
            rng = np.random.default_rng(key)
            row = (rng.standard_normal(vocab) * scale).astype(np.float32)
            if specials:
                row[rng.integers(0, vocab, vocab // 8)] = -np.inf
                row[rng.integers(0, vocab, vocab // 16)] = np.nan
            out[p] = row
        return out

    return fn


def test_selftest_toy_case(lib):
    """The reference selftest's case (tools/selftest.cpp:550-567).

    The toy callback reads token ``tokens[p]`` for the p-th requested
    position, so every one-position draft call peaks at tokens[0] + 1 = 4 and
    the verify rows peak at 3+1, 1+1, 4+1, 1+1, 5+1: draft 0 is accepted,
    draft 1 (4 against 2) is rejected and the bonus is row 1's argmax, 2."""
    cfg = make_config(lib, gamma=4, vocab=64, max_tokens=8, eos_token=999999, temperature=0.0)
    d, v = Logits(toy), Logits(toy)
    rc, res = step(lib, cfg, [3, 1, 4, 1, 5], d, v)
    assert rc == abi.OK and res.produced >= 1 and res.accepted <= cfg.gamma
    assert res.tokens_per_second > 0.0
    assert (res.accepted, res.produced, res.eos) == (1, 2, 0)
    assert list(res.tokens[:2]) == [4, 2]
    # gamma draft calls at positions ctx+j with one position each, then one
    # verify call over gamma + 1 positions starting at the context length
    assert [(len(t), f, n) for t, f, n in d.calls] == [(5 + j, 5 + j, 1) for j in range(4)]
    assert [(len(t), f, n) for t, f, n in v.calls] == [(9, 5, 5)]
    assert list(v.calls[0][0]) == [3, 1, 4, 1, 5, 4, 4, 4, 4]
    assert res.draft_time_ms >= 0 and res.verify_time_ms >= 0
    assert res.total_time_ms >= res.draft_time_ms
    assert res.theoretical_speedup > 0


def test_greedy_successor_chain(lib):
    """A callback whose logits peak at (previous token + 1) for every
    requested position: greedy drafts form the chain and are all accepted."""
    def chain(tokens, first, count, vocab):
        v = np.arange(vocab)
        return np.stack([-np.abs(v - (int(tokens[first + p - 1]) + 1) % vocab).astype(np.float32)
                         for p in range(count)])

    for max_tokens, want in ((0, 5), (8, 5), (3, 3)):
        cfg = make_config(lib, gamma=4, vocab=64, max_tokens=max_tokens, eos_token=999999,
                          temperature=0.0)
        rc, res = step(lib, cfg, [3, 1, 4, 1, 5], Logits(chain), Logits(chain))
        assert rc == abi.OK
        assert (res.accepted, res.produced, res.eos) == (min(4, want), want, 0)
        assert list(res.tokens[:want]) == [6, 7, 8, 9, 10][:want]


def test_config_defaults_match_reference(lib, reflib):
    a, b = make_config(lib), make_config(reflib)
    for f, _ in abi.SpeculativeConfig._fields_:
        assert getattr(a, f) == getattr(b, f), f


@pytest.mark.parametrize("kw, context", [
    (dict(gamma=0), [1]), (dict(gamma=abi.MAX_TOKENS), [1]), (dict(vocab=0), [1]),
])
def test_invalid_arguments(lib, reflib, kw, context):
    for L in (lib, reflib):
        cfg = make_config(L, **{"vocab": 16, **kw})
        rc, _ = step(L, cfg, context, Logits(toy), Logits(toy))
        assert rc == abi.ERR_INVALID_ARGUMENT
    res = abi.SpeculativeResult()
    cfg = make_config(lib, vocab=16)
    assert lib.vnpu_speculative_step(None, None, None, 0, Logits(toy).c, None, Logits(toy).c, None,
                                     C.byref(res)) == abi.ERR_INVALID_ARGUMENT
    assert lib.vnpu_speculative_step(None, C.byref(cfg), None, 3, Logits(toy).c, None,
                                     Logits(toy).c, None, C.byref(res)) == abi.ERR_INVALID_ARGUMENT
    assert lib.vnpu_speculative_step(None, C.byref(cfg), None, 0, Logits(toy).c, None,
                                     Logits(toy).c, None, None) == abi.ERR_INVALID_ARGUMENT


@pytest.mark.parametrize("which", ["draft", "verify"])
def test_callback_error_is_returned(lib, reflib, which):
    for L in (lib, reflib):
        d, v = Logits(toy), Logits(toy)
        (d if which == "draft" else v).status = abi.ERR_DEVICE_ERROR
        rc, _ = step(L, make_config(L, vocab=32), [1, 2], d, v)
        assert rc == abi.ERR_DEVICE_ERROR


CASES = [
    # gamma, vocab, temperature, seed, max_tokens, eos, context, draft salt, verify salt, specials
    (4, 64, 0.0, 1, 16, 999, [3, 1, 4], 1, 1, False),
    (4, 64, 0.8, 7, 16, 999, [3, 1, 4], 1, 1, False),
    (6, 97, 1.0, 3, 16, 999, [5], 2, 3, False),
    (8, 50, 0.5, 11, 3, 999, [1, 2, 3, 4], 4, 4, False),
    (5, 40, 1.3, 0, 0, 999, [9, 9], 5, 6, True),
    (3, 2000, 0.7, 123456789, 16, 999, [17, 42], 7, 8, False),
    (63, 32, 1.0, 5, 0, 999, [0], 9, 9, False),
    (63, 32, 0.0, 5, 10, 999, [0], 9, 10, True),
    (7, 32000, 0.9, 2024, 16, 2, [1, 2, 3], 11, 12, False),
    (2, 128, 2.0, 77, 16, 999, [], 13, 13, False),
]


@pytest.mark.parametrize("case", CASES, ids=[f"g{c[0]}v{c[1]}t{c[2]}s{c[3]}" for c in CASES])
def test_matches_reference_build(lib, reflib, case):
    gamma, vocab, temp, seed, max_tokens, eos, context, ds, vs, specials = case
    outs = []
    for L in (lib, reflib):
        cfg = make_config(L, gamma=gamma, vocab=vocab, temperature=temp, seed=seed,
                          max_tokens=max_tokens, eos_token=eos)
        d, v = Logits(hashed(ds, specials=specials)), Logits(hashed(vs, specials=specials))
        rc, res = step(L, cfg, context, d, v)
        outs.append((outcome(rc, res), [(list(t), f, n) for t, f, n in d.calls + v.calls]))
    assert outs[0] == outs[1]
    assert outs[0][0][0] == abi.OK


def test_eos_stops_and_is_reported(lib, reflib):
    """The first emitted EOS ends the step (cluster.cpp:624-632)."""
    def peaked(tokens, first, count, vocab):
        out = np.full((count, vocab), -5.0, np.float32)
        for p in range(count):
            out[p, 2 if first + p == 3 else 10 + first + p] = 5.0
        return out

    outs = []
    for L in (lib, reflib):
        cfg = make_config(L, gamma=6, vocab=64, temperature=0.0, eos_token=2, max_tokens=16)
        rc, res = step(L, cfg, [1], Logits(peaked), Logits(peaked))
        outs.append(outcome(rc, res))
    assert outs[0] == outs[1]
    assert outs[0] == (abi.OK, 3, 3, 1, [11, 12, 2])


def test_one_finite_logit_is_always_sampled(lib):
    """With every other logit -inf (or NaN) the sampler must return the one
    finite index, at any temperature and seed."""
    def single(tokens, first, count, vocab):
        out = np.full((count, vocab), -np.inf, np.float32)
        out[:, 1::3] = np.nan
        for p in range(count):
            out[p, ((first + p) * 7) % vocab] = -30.0
        return out

    for temp in (0.0, 0.3, 1.0, 5.0):
        for seed in (1, 2, 99):
            cfg = make_config(lib, gamma=5, vocab=91, temperature=temp, seed=seed, eos_token=1000)
            rc, res = step(lib, cfg, [4, 4], Logits(single), Logits(single))
            assert rc == abi.OK
            assert list(res.tokens[:6]) == [((2 + j) * 7) % 91 for j in range(6)]


def test_sampling_frequencies_follow_softmax(lib):
    """Drafts sampled at temperature T follow softmax(l / T): a flipped CDF
    comparison or a wrong temperature scale would fail the chi-square bar.

    The first draw of each step is left out: the state is a 32-bit seed XOR a
    fixed 64-bit constant, and one xorshift64 round (shifts 13, 7, 17) cannot
    carry seed bits up to bit 63, so the first u of every step falls in the
    same half of [0, 1) (the reference's generator, cluster.cpp:188-196,561)."""
    logits = np.array([0.0, 1.0, -1.0, 2.0, 0.5, -3.0, 1.5, 0.25], np.float32)
    T = 0.8
    fixed = lambda tokens, first, count, vocab: np.tile(logits, (count, 1))
    counts = np.zeros(len(logits))
    for seed in np.random.default_rng(0).integers(1, 2**32, 200):
        cfg = make_config(lib, gamma=63, vocab=len(logits), temperature=T, seed=int(seed),
                          max_tokens=0, eos_token=1000)
        v = Logits(fixed)
        rc, res = step(lib, cfg, [0], Logits(fixed), v)
        assert rc == abi.OK
        np.add.at(counts, v.calls[0][0][2:], 1)  # drafts after the first
    p = np.exp((logits - logits.max()) / T)
    p /= p.sum()
    expected = counts.sum() * p
    chi2 = float(((counts - expected) ** 2 / expected).sum())
    assert chi2 < 30.0, (chi2, counts, expected)  # 7 dof: P(chi2 > 30) < 1e-4


@pytest.mark.gpu
def test_mtp_head_backed_step_matches_reference(gpu, reflib):
    """Draft and verify logits from OP_MTP_HEAD_F32 on the MI355X.

    The verifier's head is W_v; the draft head is W_v plus a perturbation, so
    some drafts are rejected.  Each callback builds one hidden row per position
    from an embedding of the previous token and a position vector and runs the
    head on the GPU.  The logits every GPU call produced are then replayed
    through the reference build's step, which must ask for the same
    positions and produce the same tokens, acceptance and EOS."""
    rng = np.random.default_rng(5)
    hidden, vocab = 256, 4096
    emb = rng.standard_normal((vocab, hidden)).astype(np.float32)
    pos = rng.standard_normal((512, hidden)).astype(np.float32) * 0.5
    Wv = (rng.standard_normal((hidden, vocab)) / np.sqrt(hidden)).astype(np.float32) * 4
    Wd = Wv + (rng.standard_normal((hidden, vocab)) / np.sqrt(hidden)).astype(np.float32) * 1.5
    bufs = {k: gpu.upload(w) for k, w in (("v", Wv), ("d", Wd))}
    bh = gpu.alloc(4 * 65 * hidden)
    bl = gpu.alloc(4 * 65 * vocab)

    def head(which, record):
        def fn(tokens, first, count, voc):
            rows = np.stack([emb[int(tokens[first + p - 1])] + pos[first + p] for p in range(count)])
            gpu.write(bh, np.ascontiguousarray(rows, np.float32))
            gpu.run(abi.OP_MTP_HEAD_F32, hidden=bh, W=bufs[which], bias=None, logits=bl,
                    gamma=count, hidden_dim=hidden, vocab=voc, trans_w=0)
            out = gpu.download(bl, np.float32, (count, voc))
            record.append(out.copy())
            return out
        return fn

    def replay(record):
        it = iter(record)
        return lambda tokens, first, count, voc: next(it)

    try:
        total_acc = 0
        for trial, (temp, seed, gamma) in enumerate([(0.0, 1, 4), (0.7, 3, 6), (1.0, 9, 8),
                                                    (0.0, 4, 16), (0.5, 21, 3)]):
            context = list(rng.integers(0, vocab, 6))
            drec, vrec = [], []
            cfg = make_config(gpu.lib, gamma=gamma, vocab=vocab, temperature=temp, seed=seed,
                              max_tokens=0, eos_token=vocab + 1)
            d, v = Logits(head("d", drec)), Logits(head("v", vrec))
            rc, res = step(gpu.lib, cfg, context, d, v)
            assert rc == abi.OK, trial
            # the GPU head agrees with the float64 head on the same rows
            toks = v.calls[0][0]
            rows = np.stack([emb[int(toks[len(context) + p - 1])] + pos[len(context) + p]
                             for p in range(gamma + 1)]).astype(np.float64)
            want = rows @ Wv.astype(np.float64)
            err = np.abs(vrec[0] - want).max() / max(1.0, np.abs(want).max())
            assert err < 1e-4, (trial, err)
            rcfg = make_config(reflib, gamma=gamma, vocab=vocab, temperature=temp, seed=seed,
                               max_tokens=0, eos_token=vocab + 1)
            rd, rv = Logits(replay(drec)), Logits(replay(vrec))
            rrc, rres = step(reflib, rcfg, context, rd, rv)
            assert outcome(rc, res) == outcome(rrc, rres), trial
            assert [(list(t), f, n) for t, f, n in d.calls + v.calls] == \
                [(list(t), f, n) for t, f, n in rd.calls + rv.calls]
            total_acc += res.accepted
        assert total_acc > 0  # the perturbed draft head agrees some of the time
    finally:
        for b in (*bufs.values(), bh, bl):
            gpu.free(b)
