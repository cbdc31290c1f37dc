"""ctypes mirror of the vnpu C ABI v1 (include/vnpu.h, include/vnpu_backend.h).

The same declarations drive two libraries with one ABI:

* ``libvnpu.so`` - this repository's MI355X backend (the product), and
* ``oracle/_ref/libvnpu_ref.so`` - the reference runtime built from its own
  sources (test and CPU-baseline infrastructure only).

Struct layouts follow the reference header (include/vnpu.h:186-468 of
riteshnair/npuxl-improved); ``check_layout`` asserts the LP64 sizes.
"""
from __future__ import annotations

import ctypes as C

c_f32_p = C.POINTER(C.c_float)
c_i8_p = C.POINTER(C.c_int8)
c_u8_p = C.POINTER(C.c_uint8)
c_i32_p = C.POINTER(C.c_int32)

# status codes (vnpu.h:102-117)
OK = 0
ERR_INVALID_ARGUMENT = -1
ERR_OUT_OF_MEMORY = -2
ERR_UNSUPPORTED = -3
ERR_INVALID_COMMAND = -4
ERR_DEVICE_BUSY = -5
ERR_DEVICE_ERROR = -6
ERR_TIMEOUT = -7
ERR_NETWORK = -8
ERR_AUTH = -9
ERR_PROTOCOL = -10
ERR_NOT_FOUND = -11
ERR_IO = -12
ERR_INTERNAL = -100

# opcodes (vnpu.h:164-184)
OP_NOP, OP_MATMUL_F32, OP_MATMUL_I8, OP_RMSNORM_F32, OP_SOFTMAX_F32 = 0, 1, 2, 3, 4
OP_ROPE_F32, OP_SWIGLU_F32, OP_GELU_F32, OP_ADD_F32, OP_MUL_F32 = 5, 6, 7, 8, 9
OP_ATTENTION_F32, OP_QUANTIZE_I8, OP_PACK_WEIGHTS_I8, OP_MTP_HEAD_F32 = 10, 11, 12, 13
OP_COPY, OP_MEMSET, OP_BARRIER, OP_COUNT = 14, 15, 16, 17

UNIT_AUTO, UNIT_VOODOO, UNIT_WILDCAT, UNIT_CELL, UNIT_GPU = 0, 1, 2, 3, 16
EPI_NONE, EPI_RELU, EPI_SILU, EPI_GELU_TANH, EPI_GELU_ERF = 0, 1, 2, 3, 4
QUANT_PER_ROW, QUANT_PER_COLUMN, QUANT_PER_TENSOR = 0, 1, 2
COPY_H2H, COPY_H2D, COPY_D2H, COPY_D2D = 0, 1, 2, 3

CMD_FLAG_ASYNC = 1 << 0
CMD_FLAG_PROFILE = 1 << 1
CMD_FLAG_WILDCAT_CULL = 1 << 2
CMD_FLAG_CELL_DMA = 1 << 3
CMD_FLAG_VOODOO_FIFO = 1 << 4

CONFIG_TRACE = 1 << 0
CONFIG_HIGH_THROUGHPUT = 1 << 6   # the faster split-bf16 attention (not the reference's bits)
CONFIG_REFERENCE_ORDER = 1 << 7   # attention in the reference's order (the default; include/vnpu.h)


class Config(C.Structure):
    _fields_ = [("abi_version", C.c_uint32), ("num_threads", C.c_uint32),
                ("num_compute_units", C.c_uint32), ("tile_m", C.c_uint32),
                ("tile_k", C.c_uint32), ("tile_n", C.c_uint32), ("flags", C.c_uint32),
                ("reserved0", C.c_uint32), ("trace_file", C.c_char_p),
                ("node_name", C.c_char_p)]


class DeviceInfo(C.Structure):
    _fields_ = [("abi_version", C.c_uint32), ("name", C.c_char * 64),
                ("vendor", C.c_char * 64), ("cpu_arch", C.c_char * 32),
                ("backend", C.c_char * 64), ("simd_bits", C.c_uint32),
                ("num_threads", C.c_uint32), ("num_compute_units", C.c_uint32),
                ("local_store_bytes", C.c_uint32), ("tile_m", C.c_uint32),
                ("tile_k", C.c_uint32), ("tile_n", C.c_uint32),
                ("physical_cores", C.c_uint32), ("features", C.c_uint64),
                ("l1d_bytes", C.c_uint64), ("l2_bytes", C.c_uint64),
                ("l3_bytes", C.c_uint64), ("total_memory_bytes", C.c_uint64)]


class DeviceStatus(C.Structure):
    _fields_ = [(n, C.c_uint64) for n in (
        "commands_submitted", "commands_completed", "kernel_time_ns", "dispatch_time_ns",
        "memory_time_ns", "sync_time_ns", "bytes_read", "bytes_written", "flops",
        "tiles_dispatched", "tiles_culled", "dma_bytes", "interrupts")] + [
        ("busy", C.c_uint32), ("error", C.c_uint32), ("last_opcode", C.c_uint32),
        ("active_workers", C.c_uint32), ("reserved", C.c_uint64 * 4)]


class TraceSummary(C.Structure):
    _fields_ = [(n, C.c_uint64) for n in (
        "events", "total_time_ns", "dispatch_time_ns", "memory_time_ns", "compute_time_ns",
        "sync_time_ns", "bytes_read", "bytes_written", "flops")] + [
        ("achieved_gflops", C.c_double), ("achieved_gbytes_s", C.c_double),
        ("hot_opcode", C.c_uint32), ("hot_time_ns", C.c_uint64),
        ("trace_overhead_ns", C.c_double)]


class TuneResult(C.Structure):
    _fields_ = [("tile_m", C.c_uint32), ("tile_k", C.c_uint32), ("tile_n", C.c_uint32),
                ("unit", C.c_uint32), ("threads", C.c_uint32), ("best_ms", C.c_double),
                ("baseline_ms", C.c_double), ("speedup", C.c_double), ("gflops", C.c_double),
                ("bytes_read", C.c_uint64), ("bytes_written", C.c_uint64)]


MAX_TOKENS = 64  # VNPU_MAX_TOKENS (vnpu.h)


class SpeculativeConfig(C.Structure):
    _fields_ = [("abi_version", C.c_uint32), ("gamma", C.c_uint32), ("vocab", C.c_uint32),
                ("max_tokens", C.c_uint32), ("eos_token", C.c_uint32), ("flags", C.c_uint32),
                ("temperature", C.c_float), ("seed", C.c_uint32)]


class SpeculativeResult(C.Structure):
    _fields_ = [("accepted", C.c_uint32), ("produced", C.c_uint32), ("eos", C.c_uint32),
                ("tokens", C.c_int32 * MAX_TOKENS), ("draft_time_ms", C.c_double),
                ("verify_time_ms", C.c_double), ("total_time_ms", C.c_double),
                ("tokens_per_second", C.c_double), ("theoretical_speedup", C.c_double)]


class ClusterConfig(C.Structure):
    _fields_ = [("abi_version", C.c_uint32), ("num_streams", C.c_uint32), ("flags", C.c_uint32),
                ("request_timeout_ms", C.c_uint32), ("auth_token", C.c_char_p), ("cluster_name", C.c_char_p)]


class RemoteNodeConfig(C.Structure):
    _fields_ = [("host", C.c_char_p), ("port", C.c_uint16), ("auth_token", C.c_char_p),
                ("weight", C.c_uint32), ("flags", C.c_uint32)]


class ClusterStats(C.Structure):
    _fields_ = [("local_jobs", C.c_uint64), ("remote_jobs", C.c_uint64), ("total_jobs", C.c_uint64),
                ("network_bytes_sent", C.c_uint64), ("network_bytes_received", C.c_uint64),
                ("failed_jobs", C.c_uint64), ("culled_tiles", C.c_uint64), ("local_time_ns", C.c_double),
                ("remote_time_ns", C.c_double), ("speedup_estimate", C.c_double)]


class NodeConfig(C.Structure):
    _fields_ = [("abi_version", C.c_uint32), ("port", C.c_uint16), ("reserved0", C.c_uint16),
                ("num_threads", C.c_uint32), ("flags", C.c_uint32), ("bind_address", C.c_char_p),
                ("auth_token", C.c_char_p), ("node_name", C.c_char_p)]


# vnpu_logits_fn_t(user, tokens, num_tokens, first_position, num_positions, logits, vocab)
LOGITS_FN = C.CFUNCTYPE(C.c_int, C.c_void_p, C.POINTER(C.c_int32), C.c_uint32, C.c_uint32,
                        C.c_uint32, C.POINTER(C.c_float), C.c_uint32)


class MatmulF32Args(C.Structure):
    _fields_ = [("A", C.c_void_p), ("B", C.c_void_p), ("bias", C.c_void_p), ("C", C.c_void_p),
                ("M", C.c_uint32), ("K", C.c_uint32), ("N", C.c_uint32),
                ("lda", C.c_uint32), ("ldb", C.c_uint32), ("ldc", C.c_uint32),
                ("trans_a", C.c_uint32), ("trans_b", C.c_uint32),
                ("alpha", C.c_float), ("beta", C.c_float), ("epilogue", C.c_uint32),
                ("unit", C.c_uint32), ("reserved0", C.c_uint32), ("tile_mask", C.c_void_p),
                ("mask_tile_m", C.c_uint32), ("mask_tile_n", C.c_uint32)]


class MatmulI8Args(C.Structure):
    _fields_ = [("A", C.c_void_p), ("B", C.c_void_p), ("scale_a", C.c_void_p),
                ("bias", C.c_void_p), ("C", C.c_void_p), ("M", C.c_uint32),
                ("K", C.c_uint32), ("N", C.c_uint32), ("lda", C.c_uint32),
                ("ldc", C.c_uint32), ("epilogue", C.c_uint32), ("unit", C.c_uint32)]


class RmsnormArgs(C.Structure):
    _fields_ = [("X", C.c_void_p), ("W", C.c_void_p), ("Y", C.c_void_p),
                ("rows", C.c_uint32), ("cols", C.c_uint32), ("eps", C.c_float),
                ("unit", C.c_uint32)]


class SoftmaxArgs(C.Structure):
    _fields_ = [("X", C.c_void_p), ("Y", C.c_void_p), ("rows", C.c_uint32),
                ("cols", C.c_uint32), ("temperature", C.c_float), ("unit", C.c_uint32)]


class RopeArgs(C.Structure):
    _fields_ = [("Q", C.c_void_p), ("K", C.c_void_p), ("positions", C.c_void_p),
                ("batch", C.c_uint32), ("heads", C.c_uint32), ("q_seq", C.c_uint32),
                ("k_seq", C.c_uint32), ("head_dim", C.c_uint32),
                ("position_offset", C.c_uint32), ("interleaved", C.c_uint32),
                ("theta_base", C.c_float), ("scaling", C.c_float)]


class BinaryArgs(C.Structure):
    _fields_ = [("A", C.c_void_p), ("B", C.c_void_p), ("Y", C.c_void_p),
                ("count", C.c_uint64), ("alpha", C.c_float), ("beta", C.c_float),
                ("unit", C.c_uint32), ("reserved0", C.c_uint32)]


class UnaryArgs(C.Structure):
    _fields_ = [("X", C.c_void_p), ("Y", C.c_void_p), ("count", C.c_uint64),
                ("param", C.c_float), ("unit", C.c_uint32), ("reserved0", C.c_uint32)]


class SwigluArgs(C.Structure):
    _fields_ = [("gate", C.c_void_p), ("up", C.c_void_p), ("Y", C.c_void_p),
                ("count", C.c_uint64), ("alpha", C.c_float), ("unit", C.c_uint32),
                ("reserved0", C.c_uint32)]


class AttentionArgs(C.Structure):
    _fields_ = [("Q", C.c_void_p), ("K", C.c_void_p), ("V", C.c_void_p),
                ("mask", C.c_void_p), ("O", C.c_void_p), ("workspace", C.c_void_p),
                ("workspace_bytes", C.c_uint64), ("batch", C.c_uint32),
                ("heads", C.c_uint32), ("seq_q", C.c_uint32), ("seq_k", C.c_uint32),
                ("head_dim", C.c_uint32), ("causal", C.c_uint32), ("scale", C.c_float),
                ("unit", C.c_uint32)]


class QuantizeArgs(C.Structure):
    _fields_ = [("X", C.c_void_p), ("Y", C.c_void_p), ("scales", C.c_void_p),
                ("rows", C.c_uint64), ("cols", C.c_uint64), ("axis", C.c_uint32),
                ("unit", C.c_uint32)]


class PackArgs(C.Structure):
    _fields_ = [("B", C.c_void_p), ("scales", C.c_void_p), ("out", C.c_void_p),
                ("K", C.c_uint32), ("N", C.c_uint32), ("ldb", C.c_uint32),
                ("trans_b", C.c_uint32), ("unit", C.c_uint32), ("reserved0", C.c_uint32)]


class MtpHeadArgs(C.Structure):
    _fields_ = [("hidden", C.c_void_p), ("W", C.c_void_p), ("bias", C.c_void_p),
                ("logits", C.c_void_p), ("gamma", C.c_uint32), ("hidden_dim", C.c_uint32),
                ("vocab", C.c_uint32), ("trans_w", C.c_uint32), ("unit", C.c_uint32),
                ("reserved0", C.c_uint32)]


class CopyArgs(C.Structure):
    _fields_ = [("dst", C.c_void_p), ("src", C.c_void_p), ("bytes", C.c_uint64),
                ("direction", C.c_uint32), ("reserved0", C.c_uint32)]


class MemsetArgs(C.Structure):
    _fields_ = [("dst", C.c_void_p), ("bytes", C.c_uint64), ("value", C.c_uint32),
                ("reserved0", C.c_uint32)]


class _CmdArgs(C.Union):
    _fields_ = [("matmul_f32", MatmulF32Args), ("matmul_i8", MatmulI8Args),
                ("rmsnorm", RmsnormArgs), ("softmax", SoftmaxArgs), ("rope", RopeArgs),
                ("binary", BinaryArgs), ("unary", UnaryArgs), ("swiglu", SwigluArgs),
                ("attention", AttentionArgs), ("quantize_i8", QuantizeArgs),
                ("pack_weights_i8", PackArgs), ("mtp_head", MtpHeadArgs),
                ("copy", CopyArgs), ("memset", MemsetArgs), ("raw", C.c_uint8 * 192)]


class Command(C.Structure):
    _fields_ = [("opcode", C.c_uint32), ("flags", C.c_uint32), ("id", C.c_uint64),
                ("args", _CmdArgs)]


# Opcode -> (union member, struct type) for building commands.
OP_FIELD = {
    OP_MATMUL_F32: ("matmul_f32", MatmulF32Args), OP_MATMUL_I8: ("matmul_i8", MatmulI8Args),
    OP_RMSNORM_F32: ("rmsnorm", RmsnormArgs), OP_SOFTMAX_F32: ("softmax", SoftmaxArgs),
    OP_ROPE_F32: ("rope", RopeArgs), OP_SWIGLU_F32: ("swiglu", SwigluArgs),
    OP_GELU_F32: ("unary", UnaryArgs), OP_ADD_F32: ("binary", BinaryArgs),
    OP_MUL_F32: ("binary", BinaryArgs), OP_ATTENTION_F32: ("attention", AttentionArgs),
    OP_QUANTIZE_I8: ("quantize_i8", QuantizeArgs), OP_PACK_WEIGHTS_I8: ("pack_weights_i8", PackArgs),
    OP_MTP_HEAD_F32: ("mtp_head", MtpHeadArgs), OP_COPY: ("copy", CopyArgs),
    OP_MEMSET: ("memset", MemsetArgs),
}

# Every function the C ABI exports (vnpu.h:474-751, vnpu_backend.h:150):
# name -> (restype, argtypes).  Pointer-typed handles are passed as c_void_p.
vp = C.c_void_p
u32, u64, i32, f32 = C.c_uint32, C.c_uint64, C.c_int, C.c_float
st = C.c_int  # vnpu_status_t
SIGNATURES = {
    "vnpu_config_init": (None, [vp]),
    "vnpu_status_string": (C.c_char_p, [st]),
    "vnpu_version_string": (C.c_char_p, []),
    "vnpu_abi_version": (u32, []),
    "vnpu_device_create": (st, [vp, vp]),
    "vnpu_device_destroy": (None, [vp]),
    "vnpu_device_get_info": (st, [vp, vp]),
    "vnpu_device_get_status": (st, [vp, vp]),
    "vnpu_device_reset": (st, [vp]),
    "vnpu_device_set_tiles": (st, [vp, u32, u32, u32]),
    "vnpu_mmio_read32": (u32, [vp, u32]),
    "vnpu_mmio_write32": (None, [vp, u32, u32]),
    "vnpu_device_set_interrupt_callback": (None, [vp, vp, vp]),
    "vnpu_stream_create": (st, [vp, i32, vp]),
    "vnpu_stream_destroy": (None, [vp]),
    "vnpu_stream_sync": (st, [vp]),
    "vnpu_stream_submit": (st, [vp, vp, u64, vp]),
    "vnpu_event_create": (st, [vp]),
    "vnpu_event_destroy": (None, [vp]),
    "vnpu_event_wait": (st, [vp, u32]),
    "vnpu_event_query": (st, [vp]),
    "vnpu_buffer_alloc": (st, [vp, u64, vp]),
    "vnpu_buffer_free": (None, [vp]),
    "vnpu_buffer_host_ptr": (vp, [vp]),
    "vnpu_buffer_size": (u64, [vp]),
    "vnpu_buffer_copy": (st, [vp, vp, vp, u64, u32]),
    "vnpu_buffer_memset": (st, [vp, vp, u32, u64]),
    "vnpu_pack_weights_i8": (st, [vp, vp, vp, u32, u32, u32, u32, vp]),
    "vnpu_pack_weights_i8_masked": (st, [vp, vp, vp, u32, u32, u32, u32, vp, u32, vp]),
    "vnpu_packed_weights_destroy": (None, [vp]),
    "vnpu_packed_weights_info": (st, [vp, vp, vp, vp, vp, vp]),
    "vnpu_matmul_f32": (st, [vp, vp]),
    "vnpu_matmul_i8": (st, [vp, vp]),
    "vnpu_quantize_i8": (st, [vp, vp]),
    "vnpu_rmsnorm_f32": (st, [vp, vp]),
    "vnpu_softmax_f32": (st, [vp, vp]),
    "vnpu_rope_f32": (st, [vp, vp]),
    "vnpu_swiglu_f32": (st, [vp, vp]),
    "vnpu_gelu_f32": (st, [vp, vp]),
    "vnpu_add_f32": (st, [vp, vp]),
    "vnpu_mul_f32": (st, [vp, vp]),
    "vnpu_attention_f32": (st, [vp, vp]),
    "vnpu_mtp_head_f32": (st, [vp, vp]),
    "vnpu_trace_enable": (st, [vp, i32]),
    "vnpu_trace_reset": (None, [vp]),
    "vnpu_trace_get_summary": (st, [vp, vp]),
    "vnpu_trace_dump": (st, [vp, C.c_char_p]),
    "vnpu_trace_write_chrome": (st, [vp, C.c_char_p]),
    "vnpu_autotune_gemm": (st, [vp, u32, u32, u32, u32, C.c_int, vp]),
    "vnpu_cluster_config_init": (None, [vp]),
    "vnpu_cluster_create": (st, [vp, vp]),
    "vnpu_cluster_destroy": (None, [vp]),
    "vnpu_cluster_add_device": (st, [vp, vp, u32]),
    "vnpu_cluster_add_remote": (st, [vp, vp, vp]),
    "vnpu_cluster_get_stats": (st, [vp, vp]),
    "vnpu_cluster_cache_weights_f32": (st, [vp, C.c_char_p, vp, u32, u32, u32, vp]),
    "vnpu_cluster_matmul_f32": (st, [vp, vp, vp, vp, u32, u32, u32, u32]),
    "vnpu_node_config_init": (None, [vp]),
    "vnpu_node_run": (st, [vp]),
    "vnpu_node_stop": (None, []),
    "vnpu_speculative_config_init": (None, [vp]),
    "vnpu_speculative_step": (st, [vp, vp, vp, u32, LOGITS_FN, vp, LOGITS_FN, vp, vp]),
    "vnpu_float_to_bf16": (C.c_uint16, [f32]),
    "vnpu_float_to_f16": (C.c_uint16, [f32]),
    "vnpu_bf16_to_float": (f32, [C.c_uint16]),
    "vnpu_f16_to_float": (f32, [C.c_uint16]),
    "vnpu_opcode_name": (C.c_char_p, [u32]),
    "vnpu_unit_name": (C.c_char_p, [u32]),
    "vnpu_get_backend_v1": (vp, []),
    "vnpu_stream_hip_handle": (vp, [vp]),  # MI355X additive extension
    "vnpu_attention_f32_noalloc": (st, [vp, vp]),  # MI355X additive extension
}

LAYOUT = {  # LP64 sizes measured on the reference header
    Command: 208, MatmulF32Args: 104, MatmulI8Args: 72, AttentionArgs: 88, RopeArgs: 64,
    QuantizeArgs: 48, Config: 48, DeviceInfo: 304, DeviceStatus: 152, TraceSummary: 112,
    TuneResult: 72, SpeculativeConfig: 32, SpeculativeResult: 312, ClusterConfig: 32,
    RemoteNodeConfig: 32, ClusterStats: 80, NodeConfig: 40,
}


def check_layout() -> None:
    for t, size in LAYOUT.items():
        assert C.sizeof(t) == size, (t.__name__, C.sizeof(t), size)
    assert Command.args.offset == 16
    assert MatmulF32Args.alpha.offset == 64 and MatmulF32Args.tile_mask.offset == 88
    assert MatmulI8Args.M.offset == 40


def bind(lib: C.CDLL) -> C.CDLL:
    """Attach restype/argtypes for every exported function present in ``lib``."""
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name, None)
        if fn is None:
            continue
        fn.restype = res
        fn.argtypes = args
    return lib
