"""The reference's own consumer programs, run unmodified against libvnpu.so.

oracle/Makefile compiles the reference's selftest (tools/selftest.cpp:161-572),
conformance tool (tools/conformance.cpp:169-371), shape fuzzer
(tests/fuzz_shapes.cpp:55-177) and dlopen example (examples/dynamic_load.c)
from their sources against the reference's public headers and links them
with this repository's library: the binary drop-in check.  Each must exit 0,
and the selftest must report every case passed (its local_cluster case uses
this library's cluster client on the GPU).
"""
import os
import re
import subprocess

import pytest

import oracle
from vnpu_mi355x.runtime import BACKEND_LIB

BIN = os.path.join(oracle.HERE, "_ref", "bin")


def _bin(name):
    path = os.path.join(BIN, name)
    if not os.path.exists(path):
        pytest.skip(f"{name} not built (oracle/Makefile consumers needs the reference sources)")
    return path


def _run(args, env=None, timeout=180):
    e = dict(os.environ)
    e.update(env or {})
    print("[consumer]", " ".join(args), flush=True)
    r = subprocess.run(args, capture_output=True, text=True, timeout=timeout, env=e)
    print(r.stdout[-4000:], r.stderr[-2000:], flush=True)
    return r


@pytest.mark.parametrize("name", ["vnpu-selftest", "vnpu-conformance", "vnpu-fuzz"])
def test_consumers_link_this_library(name):
    out = subprocess.run(["ldd", _bin(name)], capture_output=True, text=True, check=True).stdout
    line = next(l for l in out.splitlines() if "libvnpu.so" in l)
    assert os.path.realpath(line.split("=>")[1].split("(")[0].strip()) == os.path.realpath(BACKEND_LIB)


@pytest.mark.gpu
def test_reference_selftest():
    r = _run([_bin("vnpu-selftest")])
    cases = re.findall(r"^\[(PASS|FAIL)\] (\S+)", r.stdout, re.M)
    assert len(cases) >= 17, r.stdout
    failed = [n for s, n in cases if s == "FAIL"]
    assert not failed, failed
    assert r.returncode == 0 and re.search(r"(\d+) tests, 0 failures", r.stdout)


@pytest.mark.gpu
def test_reference_conformance():
    r = _run([_bin("vnpu-conformance")])
    assert r.returncode == 0, r.stdout[-2000:]


@pytest.mark.gpu
def test_reference_shape_fuzzer():
    r = _run([_bin("vnpu-fuzz"), "200"])
    assert r.returncode == 0, r.stderr[-2000:]


@pytest.mark.gpu
def test_reference_dynamic_load_example():
    r = _run([_bin("dynamic_load")], env={"VNPU_LIBRARY": os.path.realpath(BACKEND_LIB)})
    assert r.returncode == 0, r.stderr
    assert "gfx950" in r.stdout and "C[0]=32.0 C[last]=32.0 expected 32.0" in r.stdout
