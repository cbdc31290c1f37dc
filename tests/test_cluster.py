"""The vnpu-node wire protocol, the node server and the cluster client.

Reference: src/cluster/protocol.h:45-119 (wire format), src/cluster/node.cpp:81-270
(node), src/cluster/cluster.cpp:85-169, 240-546 (client).

A raw-socket client written here from the protocol header's layout pins the
wire format against the reference's own node (built from its sources into
oracle/_ref/libvnpu_ref.so, CPU) and then holds this library's node (GPU) to
the same replies.  Both directions of interoperation are checked: this
library's cluster client against the reference node (CPU only: a client with
remote workers only needs no GPU) and the reference's client against this
library's node (GPU), plus a local cluster on the GPU.  GEMM results are held
to the f32 bar against a float64 product.
"""
import ctypes as C
import os
import socket
import struct
import threading
import time

import numpy as np
import pytest

import oracle
from vnpu_mi355x import abi
from vnpu_mi355x.runtime import BACKEND_LIB, load_library

RNG = np.random.default_rng(90210)
MAGIC, VERSION = 0x314E5056, 1
OP_HELLO, OP_CAPS, OP_PING, OP_STORE, OP_MATMUL, OP_STATS, OP_SHUTDOWN = 1, 2, 3, 4, 5, 6, 7
HDR = struct.Struct("<8I")                 # 32 bytes
HELLO = struct.Struct("<64s64sII")         # 136
CAPS = struct.Struct("<4I64s64s")          # 144
STORE = struct.Struct("<Q4I64s")           # 88 + K*N floats
MATMUL = struct.Struct("<Q6I")             # 32 + M*K floats
STATS = struct.Struct("<7Q")               # 56
ERR = {"AUTH": 9, "INVALID_ARGUMENT": 1, "PROTOCOL": 10, "NOT_FOUND": 11, "UNSUPPORTED": 3}


def fnv1a64(s: str) -> int:
    h = 1469598103934665603
    for c in s.encode():
        h = ((h ^ c) * 1099511628211) & 0xFFFFFFFFFFFFFFFF
    return h


def free_port() -> int:
    with socket.socket() as s:
        s.bind(("127.0.0.1", 0))
        return s.getsockname()[1]


class Node:
    """vnpu_node_run of a library on a background thread, on 127.0.0.1."""

    def __init__(self, lib, token=b"", name=b"test-node", threads=2):
        self.lib, self.port = lib, free_port()
        cfg = abi.NodeConfig()
        lib.vnpu_node_config_init(C.byref(cfg))
        cfg.port, cfg.bind_address, cfg.auth_token, cfg.node_name = self.port, b"127.0.0.1", token, name
        cfg.num_threads = threads
        self.cfg, self.rc = cfg, None
        self.thread = threading.Thread(target=self._run, daemon=True)
        self.thread.start()
        deadline = time.time() + 60
        while time.time() < deadline:
            try:
                socket.create_connection(("127.0.0.1", self.port), timeout=1).close()
                return
            except OSError:
                if not self.thread.is_alive():
                    break
                time.sleep(0.05)
        raise RuntimeError(f"node did not start (rc {self.rc})")

    def _run(self):
        self.rc = self.lib.vnpu_node_run(C.byref(self.cfg))

    def stop(self):
        self.lib.vnpu_node_stop()
        self.thread.join(timeout=60)
        assert not self.thread.is_alive(), "node did not stop"
        assert self.rc == abi.OK


class Raw:
    """A client speaking the wire format directly."""

    def __init__(self, port):
        self.s = socket.create_connection(("127.0.0.1", port), timeout=30)
        self.rid = 100

    def request(self, op, payload=b""):
        self.rid += 1
        self.s.sendall(HDR.pack(MAGIC, VERSION, op, self.rid, len(payload), 0, 0, 0) + payload)
        h = self._recv(32)
        if h is None:
            return None, None
        magic, ver, rop, rid, size, status, _, _ = HDR.unpack(h)
        assert (magic, ver, rop, rid) == (MAGIC, VERSION, op, self.rid)
        return status, self._recv(size) if size else b""

    def _recv(self, n):
        buf = b""
        while len(buf) < n:
            chunk = self.s.recv(n - len(buf))
            if not chunk:
                return None
            buf += chunk
        return buf

    def closed(self):
        try:
            return self.s.recv(1) == b""
        except OSError:
            return True

    def close(self):
        self.s.close()


def hello(token):
    return HELLO.pack(token, b"pytest", 1, 0)


def exercise_node(port, token):
    """The protocol conversation whose replies both nodes must give."""
    bad = Raw(port)
    st, _ = bad.request(OP_PING)
    assert st == ERR["AUTH"] and bad.closed()            # nothing before HELLO
    bad.close()
    bad = Raw(port)
    st, _ = bad.request(OP_HELLO, hello(b"wrong"))
    assert st == ERR["AUTH"] and bad.closed()
    bad.close()

    c = Raw(port)
    assert c.request(OP_HELLO, hello(token))[0] == 0
    assert c.request(OP_PING) == (0, b"")
    st, caps = c.request(OP_CAPS)
    assert st == 0 and len(caps) == CAPS.size
    abi_v, threads, _, _, backend, name = CAPS.unpack(caps)
    assert abi_v == 1 and name.rstrip(b"\0") == b"test-node" and backend.rstrip(b"\0")

    M, K, N = 37, 300, 130
    B = RNG.standard_normal((K, N)).astype(np.float32)
    Bt = np.ascontiguousarray(B.T)
    A = RNG.standard_normal((M, K)).astype(np.float32)
    want = A.astype(np.float64) @ B.astype(np.float64)
    wid = fnv1a64(f"w:{K}x{N}")
    assert c.request(OP_STORE, STORE.pack(wid, K, N, 0, 0, b"w") + B.tobytes())[0] == 0
    st, out = c.request(OP_MATMUL, MATMUL.pack(wid, M, K, N, 0, 0, 0) + A.tobytes())
    assert st == 0 and len(out) == 4 * M * N
    assert oracle.rel_error(np.frombuffer(out, np.float32).reshape(M, N), want) <= 1e-4
    # weights sent transposed (N x K) give the same product
    wid_t = fnv1a64(f"wt:{K}x{N}")
    assert c.request(OP_STORE, STORE.pack(wid_t, K, N, 1, 0, b"wt") + Bt.tobytes())[0] == 0
    st, out = c.request(OP_MATMUL, MATMUL.pack(wid_t, M, K, N, 1, 0, 0) + A.tobytes())
    assert st == 0 and oracle.rel_error(np.frombuffer(out, np.float32).reshape(M, N), want) <= 1e-4
    # the replies the node gives to broken requests
    assert c.request(OP_MATMUL, MATMUL.pack(wid + 1, M, K, N, 0, 0, 0) + A.tobytes())[0] == ERR["NOT_FOUND"]
    assert c.request(OP_MATMUL, MATMUL.pack(wid, M, K + 1, N, 0, 0, 0) +
                     np.zeros(M * (K + 1), np.float32).tobytes())[0] == ERR["NOT_FOUND"]
    assert c.request(OP_MATMUL, MATMUL.pack(wid, 0, K, N, 0, 0, 0))[0] == ERR["INVALID_ARGUMENT"]
    assert c.request(OP_MATMUL, MATMUL.pack(wid, M, K, N, 0, 0, 0) + A.tobytes()[:100])[0] == ERR["PROTOCOL"]
    assert c.request(OP_STORE, STORE.pack(wid, 0, N, 0, 0, b"w"))[0] == ERR["INVALID_ARGUMENT"]
    assert c.request(OP_STORE, STORE.pack(wid, K, N, 0, 0, b"w") + B.tobytes()[:64])[0] == ERR["PROTOCOL"]
    assert c.request(OP_STORE, b"short")[0] == ERR["PROTOCOL"]
    assert c.request(99, b"xyz")[0] == ERR["UNSUPPORTED"]
    # the connection is still usable after every rejected request
    st, out = c.request(OP_MATMUL, MATMUL.pack(wid, M, K, N, 0, 0, 0) + A.tobytes())
    assert st == 0 and oracle.rel_error(np.frombuffer(out, np.float32).reshape(M, N), want) <= 1e-4
    st, stats = c.request(OP_STATS)
    assert st == 0 and len(stats) == STATS.size
    completed, _, flops, *_ = STATS.unpack(stats)
    assert flops >= 3 * 2 * M * K * N
    c.close()


def test_wire_layout_sizes():
    assert (HDR.size, HELLO.size, CAPS.size, STORE.size, MATMUL.size, STATS.size) == (32, 136, 144, 88, 32, 56)
    assert struct.pack("<I", MAGIC) == b"VPN1"


def _ref_lib():
    if not os.path.exists(oracle.REF_LIB_PATH):
        pytest.skip("reference build oracle/_ref/libvnpu_ref.so not present")
    return load_library(oracle.REF_LIB_PATH)


def test_reference_node_speaks_the_wire_format():
    """Pins the raw client (and so the replies expected below) on the
    reference's own node."""
    ref = _ref_lib()
    node = Node(ref, token=b"s3cret")
    try:
        exercise_node(node.port, b"s3cret")
    finally:
        node.stop()


def _cluster(lib, token=b"", streams=1):
    cfg = abi.ClusterConfig()
    lib.vnpu_cluster_config_init(C.byref(cfg))
    cfg.num_streams, cfg.auth_token, cfg.request_timeout_ms = streams, token, 30000
    cl = C.c_void_p()
    assert lib.vnpu_cluster_create(C.byref(cfg), C.byref(cl)) == abi.OK
    return cl, cfg


def _remote(lib, cl, port, token=b"", weight=1):
    rc = abi.RemoteNodeConfig()
    rc.host, rc.port, rc.auth_token, rc.weight = b"127.0.0.1", port, token, weight
    node = C.c_void_p()
    return lib.vnpu_cluster_add_remote(cl, C.byref(rc), C.byref(node))


def _cluster_matmul(lib, cl, M, K, N, trans_b=0):
    B = RNG.standard_normal((N, K) if trans_b else (K, N)).astype(np.float32)
    A = RNG.standard_normal((M, K)).astype(np.float32)
    h = C.c_void_p()
    assert lib.vnpu_cluster_cache_weights_f32(cl, b"layer0", B.ctypes.data, K, N, trans_b, C.byref(h)) == abi.OK
    Cout = np.zeros((M, N), np.float32)
    assert lib.vnpu_cluster_matmul_f32(cl, h, A.ctypes.data, Cout.ctypes.data, M, K, N, 0) == abi.OK
    Bkn = B.T if trans_b else B
    return Cout, A.astype(np.float64) @ Bkn.astype(np.float64)


def test_client_against_reference_node():
    """This library's cluster client (remote workers only: no GPU needed)
    against the reference node, two connections, trans_b weights."""
    ref = _ref_lib()
    ours = load_library(BACKEND_LIB)
    node = Node(ref, token=b"tok")
    try:
        cl, _ = _cluster(ours, token=b"tok", streams=2)
        try:
            assert _remote(ours, cl, node.port, b"tok") == abi.OK
            got, want = _cluster_matmul(ours, cl, 61, 200, 90, trans_b=1)
            assert oracle.rel_error(got, want) <= 1e-4
            st = abi.ClusterStats()
            assert ours.vnpu_cluster_get_stats(cl, C.byref(st)) == abi.OK
            assert st.remote_jobs == 2 and st.local_jobs == 0 and st.total_jobs == 1 and st.failed_jobs == 0
            assert st.network_bytes_sent > 4 * 200 * 90 and st.network_bytes_received >= 4 * 61 * 90
        finally:
            ours.vnpu_cluster_destroy(cl)
        cl, _ = _cluster(ours, token=b"nope")
        try:
            assert _remote(ours, cl, node.port, b"nope") == abi.ERR_NETWORK
        finally:
            ours.vnpu_cluster_destroy(cl)
    finally:
        node.stop()


@pytest.mark.gpu
def test_our_node_speaks_the_wire_format(gpu):
    node = Node(gpu.lib, token=b"s3cret")
    try:
        exercise_node(node.port, b"s3cret")
    finally:
        node.stop()


@pytest.mark.gpu
def test_reference_client_against_our_node(gpu):
    """The reference's cluster client (its own build) driving this library's
    node: weights stored in HBM, rows split over two connections."""
    ref = _ref_lib()
    node = Node(gpu.lib, token=b"k")
    try:
        cl, _ = _cluster(ref, token=b"k", streams=2)
        try:
            assert _remote(ref, cl, node.port, b"k") == abi.OK
            got, want = _cluster_matmul(ref, cl, 300, 512, 257)
            assert oracle.rel_error(got, want) <= 1e-4
            got, want = _cluster_matmul(ref, cl, 5, 64, 33, trans_b=1)
            assert oracle.rel_error(got, want) <= 1e-4
        finally:
            ref.vnpu_cluster_destroy(cl)
    finally:
        node.stop()


@pytest.mark.gpu
def test_local_and_remote_cluster_on_gpu(gpu):
    """Local GPU workers (two streams, weight 2) and one remote node of this
    library in one cluster: rows split 2:2:1:1 and every range correct."""
    node = Node(gpu.lib)
    try:
        cl, _ = _cluster(gpu.lib, streams=2)
        try:
            assert gpu.lib.vnpu_cluster_add_device(cl, gpu.dev, 2) == abi.OK
            assert _remote(gpu.lib, cl, node.port) == abi.OK
            got, want = _cluster_matmul(gpu.lib, cl, 203, 384, 300)
            assert oracle.rel_error(got, want) <= 1e-4
            st = abi.ClusterStats()
            assert gpu.lib.vnpu_cluster_get_stats(cl, C.byref(st)) == abi.OK
            assert st.local_jobs == 2 and st.remote_jobs == 2 and st.failed_jobs == 0
        finally:
            gpu.lib.vnpu_cluster_destroy(cl)
    finally:
        node.stop()


@pytest.mark.gpu
def test_node_shutdown_op(gpu):
    node = Node(gpu.lib)
    c = Raw(node.port)
    assert c.request(OP_HELLO, hello(b""))[0] == 0
    assert c.request(OP_SHUTDOWN)[0] == 0
    c.close()
    node.thread.join(timeout=60)
    assert not node.thread.is_alive() and node.rc == abi.OK


@pytest.mark.gpu
def test_node_frees_replaced_weights(gpu):
    """STORE over a weight id that a MATMUL on another connection may be
    using at that moment: the replaced weights are freed by whichever drops
    them last, so HBM does not grow over many replacements."""
    hip = C.CDLL("libamdhip64.so")

    def free_bytes():
        f, t = C.c_size_t(), C.c_size_t()
        assert hip.hipMemGetInfo(C.byref(f), C.byref(t)) == 0
        return f.value

    K, N, M = 2048, 4096, 256                       # 32 MiB of weights
    B = RNG.standard_normal((K, N)).astype(np.float32)
    A = RNG.standard_normal((M, K)).astype(np.float32)
    wid = fnv1a64("replaced")
    store = STORE.pack(wid, K, N, 0, 0, b"r") + B.tobytes()
    mm = MATMUL.pack(wid, M, K, N, 0, 0, 0) + A.tobytes()
    node = Node(gpu.lib)
    try:
        c1, c2 = Raw(node.port), Raw(node.port)
        assert c1.request(OP_HELLO, hello(b""))[0] == 0 and c2.request(OP_HELLO, hello(b""))[0] == 0
        for _ in range(2):                           # both connections' buffers at their size
            assert c1.request(OP_STORE, store)[0] == 0
            assert c2.request(OP_MATMUL, mm)[0] == 0
        base = free_bytes()
        stop, statuses = threading.Event(), []

        def matmuls():
            while not stop.is_set():
                st, out = c2.request(OP_MATMUL, mm)
                statuses.append(st)
                if st != 0 or len(out) != 4 * M * N:
                    break

        t = threading.Thread(target=matmuls)
        t.start()
        try:
            for _ in range(24):
                assert c1.request(OP_STORE, store)[0] == 0
        finally:
            stop.set()
            t.join(timeout=120)
        assert not t.is_alive() and statuses and all(s == 0 for s in statuses)
        lost = base - free_bytes()
        assert lost <= 2 * K * N * 4, f"{lost >> 20} MiB of HBM not returned after 24 replacements"
        c1.close()
        c2.close()
    finally:
        node.stop()
