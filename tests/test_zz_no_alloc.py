"""vnpu_attention_f32_noalloc: ATTENTION_F32 with the per-GPU device scratch.

Through the C ABI, on device-resident tensors: two calls in a row, the
second with a smaller input, each compared with vnpu_attention_f32 (the
same kernels with the stream workspace) bit for bit and with the C oracle
within the attention bar; shapes above the 64 MiB scratch and host pointers
are refused without running anything.
"""
import ctypes as C

import numpy as np
import pytest

import block_oracle
import oracle
from vnpu_mi355x import abi

pytestmark = pytest.mark.gpu
RNG = np.random.default_rng(7707)


def _args(q, k, v, o, shape, sk, causal, mask=None):
    b, h, sq, d = shape
    a = abi.AttentionArgs()
    a.Q, a.K, a.V, a.O = q, k, v, o
    a.mask = mask
    a.batch, a.heads, a.seq_q, a.seq_k, a.head_dim, a.causal = b, h, sq, sk, d, causal
    a.scale = 0.0
    return a


def _case(gpu, b, h, sq, sk, d, causal, use_mask):
    Q = RNG.standard_normal((b, h, sq, d)).astype(np.float32)
    K = RNG.standard_normal((b, h, sk, d)).astype(np.float32)
    V = RNG.standard_normal((b, h, sk, d)).astype(np.float32)
    M = RNG.standard_normal((b, h, sq, sk)).astype(np.float32) if use_mask else None
    bufs = [gpu.upload(Q), gpu.upload(K), gpu.upload(V)]
    bm = gpu.upload(M) if use_mask else None
    o_ref, o_new = gpu.alloc(Q.nbytes), gpu.alloc(Q.nbytes)
    mp = bm.ptr if bm else None
    a_ref = _args(bufs[0].ptr, bufs[1].ptr, bufs[2].ptr, o_ref.ptr, Q.shape, sk, causal, mp)
    a_new = _args(bufs[0].ptr, bufs[1].ptr, bufs[2].ptr, o_new.ptr, Q.shape, sk, causal, mp)
    assert gpu.lib.vnpu_attention_f32(gpu.stream, C.byref(a_ref)) == abi.OK
    assert gpu.lib.vnpu_attention_f32_noalloc(gpu.stream, C.byref(a_new)) == abi.OK
    assert gpu.sync() == abi.OK
    want = gpu.download(o_ref, np.float32, Q.shape)
    got = gpu.download(o_new, np.float32, Q.shape)
    for x in bufs + [o_ref, o_new] + ([bm] if bm else []):
        gpu.free(x)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    want = block_oracle.attention_threaded(Q, K, V, causal, mask=M)
    assert oracle.rel_error(got, want) <= 2e-3


@pytest.mark.parametrize("dev,first,second", [
    # high-throughput device, split decode (partial triples in the scratch):
    # config-4 decode, then smaller
    ("fast_gpu", (8, 32, 1, 4096, 128, 1, False), (2, 4, 1, 1000, 128, 1, True)),
    # split-bf16 prefill (split K / V^T blocks in the scratch): 32 heads x
    # 2048 keys at head_dim 128 fills the 64 MiB exactly, then a smaller
    # masked call
    ("fast_gpu", (1, 32, 2048, 2048, 128, 1, False), (1, 2, 300, 300, 64, 0, True)),
    # the generic kernel (head_dim 80) with a split key range, then smaller
    ("fast_gpu", (1, 2, 20, 3000, 80, 1, False), (1, 1, 5, 700, 80, 0, True)),
    # default device, reference-order decode (the scores in the scratch):
    # config-4 decode, then three query rows at head_dim 64 with a mask
    ("gpu", (8, 32, 1, 4096, 128, 1, False), (2, 4, 3, 1000, 64, 1, True)),
])
def test_noalloc_matches_attention_two_calls(request, dev, first, second):
    gpu = request.getfixturevalue(dev)
    _case(gpu, *first)
    _case(gpu, *second)


def test_noalloc_refuses_oversize_and_host_pointers(fast_gpu):
    gpu = fast_gpu
    b, h, s, d = 1, 32, 2100, 128   # 66 split blocks per head: 66 MiB of scratch
    Q = gpu.alloc(b * h * s * d * 4)
    K = gpu.alloc(b * h * s * d * 4)
    V = gpu.alloc(b * h * s * d * 4)
    O = gpu.alloc(b * h * s * d * 4)
    a = _args(Q.ptr, K.ptr, V.ptr, O.ptr, (b, h, s, d), s, 1)
    assert gpu.lib.vnpu_attention_f32_noalloc(gpu.stream, C.byref(a)) == abi.ERR_INVALID_ARGUMENT
    host = np.zeros((1, 1, 4, 32), np.float32)
    a = _args(host.ctypes.data, K.ptr, V.ptr, O.ptr, (1, 1, 4, 32), 4, 0)
    assert gpu.lib.vnpu_attention_f32_noalloc(gpu.stream, C.byref(a)) == abi.ERR_INVALID_ARGUMENT
    assert gpu.lib.vnpu_attention_f32_noalloc(gpu.stream, None) == abi.ERR_INVALID_ARGUMENT
    assert gpu.sync() == abi.OK   # nothing was enqueued, no sticky error
    for x in (Q, K, V, O):
        gpu.free(x)
