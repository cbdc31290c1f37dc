"""The synthetic Llama-style decoder block of the block benchmark, on any
vnpu library.

``Block`` quantizes and packs one layer's weights through the library's own
QUANTIZE_I8 (per column) and PACK_WEIGHTS_I8 - the reference's flow
(tools/llm_bench.cpp:115-130) - allocates the activations, and runs the
block with ``libvnpu_block.so`` (csrc/block_harness.hip), which submits the
op sequence through the library's vtable.  Against the MI355X backend the
layout steps run as HIP kernels on the vnpu stream; against the reference
build (host memory) they run on the host, as in the reference's llm_bench.

Weights follow the benchmark's recipe: every projection ~ N(0, 0.02) from
its own seeded stream; the two RMSNorm weight vectors are 1 + 0.1 N(0, 1)
(the reference's llm_bench uses all-ones; a non-trivial vector also checks
that the weights are applied).
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass

import numpy as np

from . import abi, synth
from .runtime import ROOT, Buffer, Session

BLOCK_LIB = os.path.join(ROOT, "lib", "libvnpu_block.so")


class BlockConfig(C.Structure):
    _fields_ = [("batch", C.c_uint32), ("tokens", C.c_uint32), ("d_model", C.c_uint32),
                ("heads", C.c_uint32), ("head_dim", C.c_uint32), ("ffn", C.c_uint32),
                ("past", C.c_uint32), ("cache_len", C.c_uint32), ("eps", C.c_float),
                ("theta", C.c_float)]


class BlockWeights(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in ("qkv", "o", "gate", "up", "down", "norm_attn",
                                           "norm_ffn")]


BUFFER_FIELDS = ("x", "xn", "a8", "scale_a", "qkv", "q", "k", "v", "o", "att", "proj", "gate",
                 "up", "ff", "k_cache", "v_cache")


class BlockBuffers(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in BUFFER_FIELDS]


_lib = None


def block_lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(BLOCK_LIB):
            raise FileNotFoundError(f"block harness not built: {BLOCK_LIB}")
        lib = C.CDLL(BLOCK_LIB, mode=C.RTLD_LOCAL)
        lib.vnpu_block_run.restype = C.c_int
        lib.vnpu_block_run.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.POINTER(BlockConfig),
                                       C.POINTER(BlockWeights), C.POINTER(BlockBuffers)]
        _lib = lib
    return _lib


@dataclass(frozen=True)
class BlockShape:
    d_model: int
    heads: int
    head_dim: int
    ffn: int


# d_model 4096, 32 heads x 128, FFN 11008.
LLAMA_4096 = BlockShape(4096, 32, 128, 11008)

PROJECTIONS = ("qkv", "o", "gate", "up", "down")


def projection_dims(shape: BlockShape, name: str) -> tuple[int, int]:
    d, f = shape.d_model, shape.ffn
    return {"qkv": (d, 3 * d), "o": (d, d), "gate": (d, f), "up": (d, f), "down": (f, d)}[name]


def weights_f32(shape: BlockShape, tag: str = "block") -> dict[str, np.ndarray]:
    """Seeded f32 weights of one layer (projections [K][N] row-major)."""
    w = {}
    for name in PROJECTIONS:
        K, N = projection_dims(shape, name)
        w[name] = synth.normal(f"{tag}/{name}", (K, N), 0.02)
    for name in ("norm_attn", "norm_ffn"):
        w[name] = (1.0 + 0.1 * synth.normal(f"{tag}/{name}", (shape.d_model,))).astype(np.float32)
    return w


class Block:
    """One layer resident on a Session: packed int8 projections + norm weights."""

    def __init__(self, s: Session, shape: BlockShape, w32: dict[str, np.ndarray],
                 quantized: dict[str, tuple[np.ndarray, np.ndarray]] | None = None):
        """w32: f32 weights (quantized here per column by the library), or
        quantized: name -> (int8 [K][N], scales [N]) already quantized (e.g.
        by another backend, to give two backends the same integer weights);
        w32 still supplies the norm weights."""
        self.s, self.shape = s, shape
        self.packed = {}
        self.quantized = {}   # name -> (int8 [K][N], scales [N]) buffers on this session
        for name in PROJECTIONS:
            K, N = projection_dims(shape, name)
            if quantized is not None:
                bq = s.upload(np.ascontiguousarray(quantized[name][0], np.int8))
                bs = s.upload(np.ascontiguousarray(quantized[name][1], np.float32))
            else:
                bw = s.upload(w32[name])
                bq, bs = s.alloc(K * N), s.alloc(4 * N)
                s.run(abi.OP_QUANTIZE_I8, X=bw, Y=bq, scales=bs, rows=K, cols=N,
                      axis=abi.QUANT_PER_COLUMN)
                s.free(bw)
            self.packed[name] = s.pack(bq, K, N, scales=bs)
            self.quantized[name] = (bq, bs)
        self.norm = {n: s.upload(w32[n]) for n in ("norm_attn", "norm_ffn")}
        self.weights = BlockWeights(*(self.packed[n].value for n in PROJECTIONS),
                                    self.norm["norm_attn"].ptr, self.norm["norm_ffn"].ptr)
        self.bufs: dict[str, Buffer] = {}
        self.cfg = None

    def quantized_weights(self, name: str) -> tuple[np.ndarray, np.ndarray]:
        K, N = projection_dims(self.shape, name)
        bq, bs = self.quantized[name]
        return self.s.download(bq, np.int8, (K, N)), self.s.download(bs, np.float32, (N,))

    def prepare(self, batch: int, tokens: int, past: int = 0, cache_len: int = 0,
                eps: float = 1e-5, theta: float = 10000.0) -> None:
        """Allocate activations for batch x tokens rows (and KV caches when
        cache_len > 0: decode of `tokens` new tokens after `past` cached)."""
        for b in self.bufs.values():
            self.s.free(b)
        sh = self.shape
        d, f = sh.d_model, sh.ffn
        rows = batch * tokens
        size = {"x": 4 * rows * d, "xn": 4 * rows * d, "a8": rows * max(d, f), "scale_a": 4 * rows,
                "qkv": 12 * rows * d, "q": 4 * rows * d, "k": 4 * rows * d, "v": 4 * rows * d,
                "o": 4 * rows * d, "att": 4 * rows * d, "proj": 4 * rows * d, "gate": 4 * rows * f,
                "up": 4 * rows * f, "ff": 4 * rows * f}
        if cache_len:
            size["k_cache"] = size["v_cache"] = 4 * batch * sh.heads * cache_len * sh.head_dim
        self.bufs = {n: self.s.alloc(sz) for n, sz in size.items()}
        self.buffers = BlockBuffers(*(self.bufs[n].ptr if n in self.bufs else None
                                      for n in BUFFER_FIELDS))
        self.cfg = BlockConfig(batch, tokens, d, sh.heads, sh.head_dim, f, past, cache_len, eps, theta)

    def set_input(self, x: np.ndarray, k_cache: np.ndarray | None = None,
                  v_cache: np.ndarray | None = None) -> None:
        self.s.write(self.bufs["x"], np.asarray(x, np.float32))
        if k_cache is not None:
            self.s.write(self.bufs["k_cache"], np.asarray(k_cache, np.float32))
            self.s.write(self.bufs["v_cache"], np.asarray(v_cache, np.float32))

    def output(self) -> np.ndarray:
        rows = self.cfg.batch * self.cfg.tokens
        return self.s.download(self.bufs["x"], np.float32, (rows, self.shape.d_model))

    def enqueue(self, gpu: bool) -> None:
        """Enqueue one block; gpu=True runs the layout kernels on the vnpu
        stream (MI355X backend), False on the host (reference build)."""
        lib = self.s.lib
        table = lib.vnpu_get_backend_v1()
        hip = lib.vnpu_stream_hip_handle(self.s.stream) if gpu else None
        rc = block_lib().vnpu_block_run(table, self.s.stream, hip, C.byref(self.cfg),
                                        C.byref(self.weights), C.byref(self.buffers))
        Session.check("vnpu_block_run", rc)

    def run(self, gpu: bool) -> None:
        self.enqueue(gpu)
        Session.check("vnpu_stream_sync", self.s.sync())

    def close(self) -> None:
        for b in self.bufs.values():
            self.s.free(b)
        self.bufs = {}
        for name in PROJECTIONS:
            self.s.release_packed(self.packed[name])
            for b in self.quantized[name]:
                self.s.free(b)
        for b in self.norm.values():
            self.s.free(b)
