"""CPU checks of the drop-in boundary: headers, layouts, exported symbols.

No compute call is made here (there is no GPU in the build container); the
library is loaded, its exports are checked against include/*.h, and
vnpu_device_create must refuse to run without a GPU instead of falling back.
"""
import ctypes as C
import os
import re
import subprocess

import pytest

from vnpu_mi355x import BACKEND_LIB, abi, load_backend

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INCLUDE = os.path.join(ROOT, "include")


def declared_symbols():
    names = set()
    for h in ("vnpu.h", "vnpu_backend.h"):
        text = open(os.path.join(INCLUDE, h)).read()
        for m in re.finditer(r"VNPU_API[^;{]*?\bVNPU_CALL\s+(vnpu_\w+)\s*\(", text, re.S):
            names.add(m.group(1))
    return names


def test_ctypes_layout_matches_reference_sizes():
    abi.check_layout()


def test_headers_compile_with_layout_asserts(tmp_path):
    src = tmp_path / "t.c"
    src.write_text('#include "vnpu_backend.h"\nint main(void){return (int)sizeof(vnpu_command_t)-208;}\n')
    exe = tmp_path / "t"
    subprocess.run(["gcc", "-std=c11", "-Wall", "-Werror", f"-I{INCLUDE}", str(src), "-o", str(exe)],
                   check=True)
    assert subprocess.run([str(exe)]).returncode == 0
    srcpp = tmp_path / "t.cpp"
    srcpp.write_text('#include "vnpu_backend.h"\nint main(){return 0;}\n')
    subprocess.run(["g++", "-std=c++17", "-Wall", "-Werror", f"-I{INCLUDE}", str(srcpp), "-o",
                    str(tmp_path / "tpp")], check=True)


@pytest.mark.skipif(not os.path.exists("/root/reference/include/vnpu.h"),
                    reason="reference headers not present")
def test_layout_identical_to_reference_header(tmp_path):
    probe = tmp_path / "probe.c"
    fields = {
        "vnpu_command_t": ["opcode", "flags", "id", "args"],
        "vnpu_matmul_f32_args_t": ["A", "B", "bias", "C", "M", "K", "N", "lda", "ldb", "ldc",
                                   "trans_a", "trans_b", "alpha", "beta", "epilogue", "unit",
                                   "tile_mask", "mask_tile_m", "mask_tile_n"],
        "vnpu_matmul_i8_args_t": ["A", "B", "scale_a", "bias", "C", "M", "K", "N", "lda", "ldc",
                                  "epilogue", "unit"],
        "vnpu_attention_f32_args_t": ["Q", "K", "V", "mask", "O", "workspace", "workspace_bytes",
                                      "batch", "heads", "seq_q", "seq_k", "head_dim", "causal",
                                      "scale", "unit"],
        "vnpu_rope_f32_args_t": ["Q", "K", "positions", "batch", "theta_base", "scaling"],
        "vnpu_quantize_i8_args_t": ["X", "Y", "scales", "rows", "cols", "axis", "unit"],
        "vnpu_device_info_t": ["name", "vendor", "cpu_arch", "backend", "physical_cores",
                               "features", "total_memory_bytes"],
        "vnpu_device_status_t": ["busy", "error", "reserved"],
        "vnpu_trace_summary_t": ["achieved_gflops", "hot_opcode", "hot_time_ns", "trace_overhead_ns"],
        "vnpu_backend_v1_t": ["backend_name", "device_create", "matmul_i8", "speculative_step",
                              "version_string", "reserved"],
        "vnpu_speculative_result_t": ["tokens", "draft_time_ms", "theoretical_speedup"],
    }
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "vnpu_backend.h"', "int main(void){"]
    for t, fs in fields.items():
        lines.append(f'printf("{t} %zu\\n", sizeof({t}));')
        for f in fs:
            lines.append(f'printf("{t}.{f} %zu\\n", offsetof({t}, {f}));')
    lines.append("return 0;}")
    probe.write_text("\n".join(lines))
    outs = []
    for inc in (INCLUDE, "/root/reference/include"):
        exe = tmp_path / ("p" + str(len(outs)))
        subprocess.run(["gcc", "-std=c11", f"-I{inc}", str(probe), "-o", str(exe)], check=True)
        outs.append(subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout)
    assert outs[0] == outs[1]


def test_library_exports_every_declared_symbol():
    assert os.path.exists(BACKEND_LIB), "run __graft_entry__.build() first"
    out = subprocess.run(["nm", "-D", "--defined-only", BACKEND_LIB], capture_output=True,
                         text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    missing = declared_symbols() - exported
    assert not missing, missing
    assert len(declared_symbols()) >= 68
    # and nothing beyond the ABI leaks out (hidden visibility)
    extra = {s for s in exported if not s.startswith("vnpu_")}
    assert not extra, sorted(extra)[:10]


def test_library_loads_and_binds_all_symbols():
    lib = load_backend()
    for name in abi.SIGNATURES:
        assert getattr(lib, name) is not None
    assert lib.vnpu_abi_version() == 1
    assert lib.vnpu_opcode_name(2) == b"MATMUL_I8"
    assert lib.vnpu_status_string(-6) == b"device error"
    assert lib.vnpu_bf16_to_float(lib.vnpu_float_to_bf16(1.5)) == 1.5
    assert lib.vnpu_f16_to_float(lib.vnpu_float_to_f16(-2.25)) == -2.25
    tbl = lib.vnpu_get_backend_v1()
    head = (C.c_uint32 * 2).from_address(tbl)
    assert head[0] == 1 and head[1] == 416
    fns = (C.c_void_p * 42).from_address(tbl + 16)
    assert all(fns), "every backend table entry is a function"


def test_f16_bf16_match_reference_helpers():
    import oracle
    if not os.path.exists(oracle.REF_LIB_PATH):
        pytest.skip("reference build absent")
    ours = load_backend()
    ref = abi.bind(C.CDLL(oracle.REF_LIB_PATH))
    import numpy as np
    vals = np.concatenate([np.random.default_rng(3).standard_normal(2000).astype(np.float32) * 1e3,
                           np.array([0.0, -0.0, 1e-8, 6e-5, 65504.0, 1e6, np.inf, -np.inf],
                                    np.float32)])
    for v in vals:
        v = float(v)
        assert ours.vnpu_float_to_f16(v) == ref.vnpu_float_to_f16(v)
        assert ours.vnpu_float_to_bf16(v) == ref.vnpu_float_to_bf16(v)
    for h in range(0, 65536, 7):
        a, b = ours.vnpu_f16_to_float(h), ref.vnpu_f16_to_float(h)
        assert a == b or (a != a and b != b)


def test_device_create_fails_loudly_without_gpu():
    if os.path.exists("/dev/kfd") and os.access("/dev/kfd", os.R_OK):
        pytest.skip("a GPU may be present")
    lib = load_backend()
    dev = C.c_void_p()
    assert lib.vnpu_device_create(None, C.byref(dev)) != abi.OK
    assert not dev.value
