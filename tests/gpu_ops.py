"""Helpers that run one vnpu command on a Session with numpy in/out.

Used by the GPU parity tests (against libvnpu.so) and by the reference
parity tests (against oracle/_ref/libvnpu_ref.so): the same call sequence
drives either library through the C ABI.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from vnpu_mi355x import abi


def quantize(s, X, axis):
    X = np.ascontiguousarray(X, np.float32)
    rows, cols = X.shape
    n = rows if axis == 0 else cols if axis == 1 else 1
    bx, by, bs = s.upload(X), s.alloc(rows * cols), s.alloc(4 * n)
    s.run(abi.OP_QUANTIZE_I8, X=bx, Y=by, scales=bs, rows=rows, cols=cols, axis=axis)
    out = s.download(by, np.int8, (rows, cols)), s.download(bs, np.float32, (n,))
    for b in (bx, by, bs):
        s.free(b)
    return out


def matmul_i8(s, A, w, M, K, N, scale_a=None, bias=None, epilogue=0, lda=0, ldc=0):
    A = np.ascontiguousarray(A, np.int8)
    ba = s.upload(A)
    bsa = s.upload(np.asarray(scale_a, np.float32)) if scale_a is not None else None
    bb = s.upload(np.asarray(bias, np.float32)) if bias is not None else None
    ldc_e = ldc or N
    bc = s.alloc(4 * M * ldc_e)
    s.run(abi.OP_MATMUL_I8, A=ba, B=w, scale_a=bsa.ptr if bsa else None,
          bias=bb.ptr if bb else None, C=bc, M=M, K=K, N=N, lda=lda, ldc=ldc, epilogue=epilogue)
    out = s.download(bc, np.float32, (M, ldc_e))[:, :N]
    for b in (ba, bsa, bb, bc):
        if b is not None:
            s.free(b)
    return out


def matmul_f32(s, A, B, M, K, N, C_in=None, bias=None, trans_a=0, trans_b=0, alpha=1.0,
               beta=0.0, epilogue=0, mask=None, unit=0, flags=0):
    ba, bb = s.upload(np.asarray(A, np.float32)), s.upload(np.asarray(B, np.float32))
    bbias = s.upload(np.asarray(bias, np.float32)) if bias is not None else None
    if C_in is not None:
        bc = s.upload(np.asarray(C_in, np.float32))
    else:
        bc = s.alloc(4 * M * N)
    bm = s.upload(np.asarray(mask, np.uint8)) if mask is not None else None
    s.run(abi.OP_MATMUL_F32, flags=flags, A=ba, B=bb, bias=bbias.ptr if bbias else None, C=bc,
          M=M, K=K, N=N, trans_a=trans_a, trans_b=trans_b, alpha=alpha, beta=beta,
          epilogue=epilogue, unit=unit, tile_mask=bm.ptr if bm else None,
          mask_tile_m=mask.shape[0] if mask is not None else 0,
          mask_tile_n=mask.shape[1] if mask is not None else 0)
    out = s.download(bc, np.float32, (M, N))
    for b in (ba, bb, bbias, bc, bm):
        if b is not None:
            s.free(b)
    return out


def unary_rows(s, op, X, **kw):
    X = np.ascontiguousarray(X, np.float32)
    bx, by = s.upload(X), s.alloc(X.nbytes)
    rows, cols = X.shape
    if op == abi.OP_RMSNORM_F32:
        W = kw.get("W")
        bw = s.upload(np.asarray(W, np.float32)) if W is not None else None
        s.run(op, X=bx, W=bw.ptr if bw else None, Y=by, rows=rows, cols=cols, eps=kw.get("eps", 0.0))
        if bw:
            s.free(bw)
    else:
        s.run(op, X=bx, Y=by, rows=rows, cols=cols, temperature=kw.get("temperature", 0.0))
    out = s.download(by, np.float32, X.shape)
    s.free(bx)
    s.free(by)
    return out


def elementwise(s, op, a, b=None, alpha=0.0, beta=0.0):
    a = np.ascontiguousarray(a, np.float32)
    ba = s.upload(a)
    bb = s.upload(np.asarray(b, np.float32)) if b is not None else None
    by = s.alloc(a.nbytes)
    if op == abi.OP_SWIGLU_F32:
        s.run(op, gate=ba, up=bb, Y=by, count=a.size, alpha=alpha)
    elif op == abi.OP_GELU_F32:
        s.run(op, X=ba, Y=by, count=a.size)
    else:
        s.run(op, A=ba, B=bb, Y=by, count=a.size, alpha=alpha, beta=beta)
    out = s.download(by, np.float32, a.shape)
    for x in (ba, bb, by):
        if x is not None:
            s.free(x)
    return out


def rope(s, Q, K, positions=None, position_offset=0, interleaved=0, theta=0.0, scaling=0.0):
    bq = s.upload(np.asarray(Q, np.float32)) if Q is not None else None
    bk = s.upload(np.asarray(K, np.float32)) if K is not None else None
    bp = s.upload(np.asarray(positions, np.int32)) if positions is not None else None
    ref = Q if Q is not None else K
    b, h, _, d = ref.shape
    s.run(abi.OP_ROPE_F32, Q=bq.ptr if bq else None, K=bk.ptr if bk else None,
          positions=bp.ptr if bp else None, batch=b, heads=h,
          q_seq=Q.shape[2] if Q is not None else 0, k_seq=K.shape[2] if K is not None else 0,
          head_dim=d, position_offset=position_offset, interleaved=interleaved,
          theta_base=theta, scaling=scaling)
    q = s.download(bq, np.float32, Q.shape) if bq else None
    k = s.download(bk, np.float32, K.shape) if bk else None
    for x in (bq, bk, bp):
        if x is not None:
            s.free(x)
    return q, k


def attention(s, Q, K, V, mask=None, causal=0, scale=0.0):
    bq, bk, bv = (s.upload(np.asarray(x, np.float32)) for x in (Q, K, V))
    bm = s.upload(np.asarray(mask, np.float32)) if mask is not None else None
    bo = s.alloc(np.asarray(Q).nbytes)
    b, h, sq, d = Q.shape
    s.run(abi.OP_ATTENTION_F32, Q=bq, K=bk, V=bv, mask=bm.ptr if bm else None, O=bo, batch=b,
          heads=h, seq_q=sq, seq_k=K.shape[2], head_dim=d, causal=causal, scale=scale)
    out = s.download(bo, np.float32, Q.shape)
    for x in (bq, bk, bv, bm, bo):
        if x is not None:
            s.free(x)
    return out


def mtp_head(s, hidden, W, bias=None, trans_w=0):
    hidden = np.ascontiguousarray(hidden, np.float32)
    gamma, hd = hidden.shape
    vocab = W.shape[0] if trans_w else W.shape[1]
    bh, bw = s.upload(hidden), s.upload(np.asarray(W, np.float32))
    bb = s.upload(np.asarray(bias, np.float32)) if bias is not None else None
    bl = s.alloc(4 * gamma * vocab)
    s.run(abi.OP_MTP_HEAD_F32, hidden=bh, W=bw, bias=bb.ptr if bb else None, logits=bl,
          gamma=gamma, hidden_dim=hd, vocab=vocab, trans_w=trans_w)
    out = s.download(bl, np.float32, (gamma, vocab))
    for x in (bh, bw, bb, bl):
        if x is not None:
            s.free(x)
    return out
