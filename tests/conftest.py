import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "npuxl-improved_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libvnpu.so on HIP)")


@pytest.fixture(scope="session")
def gpu():
    """One MI355X session for all GPU tests (device + stream on libvnpu.so;
    the default device: ATTENTION_F32 in the reference's order)."""
    from vnpu_mi355x import Session
    s = Session()
    yield s
    s.close()


@pytest.fixture(scope="session")
def fast_gpu():
    """An MI355X session whose device is created with
    VNPU_CONFIG_HIGH_THROUGHPUT: ATTENTION_F32 on the split-bf16 matrix-core
    kernels (within tolerance of the reference, not its bits)."""
    from vnpu_mi355x import Session, abi
    cfg = abi.Config()
    cfg.abi_version = 1
    cfg.flags = abi.CONFIG_HIGH_THROUGHPUT
    s = Session(None, cfg)
    yield s
    s.close()


@pytest.fixture(scope="session")
def exact_gpu():
    """An MI355X session whose device is created with
    VNPU_CONFIG_REFERENCE_ORDER (the default order, asked for explicitly)."""
    from vnpu_mi355x import Session, abi
    cfg = abi.Config()
    cfg.abi_version = 1
    cfg.flags = abi.CONFIG_REFERENCE_ORDER
    s = Session(None, cfg)
    yield s
    s.close()


@pytest.fixture(scope="session")
def ref():
    """The reference runtime built from its own sources (CPU), if present."""
    import oracle
    if not os.path.exists(oracle.REF_LIB_PATH):
        pytest.skip("reference build oracle/_ref/libvnpu_ref.so not present")
    from vnpu_mi355x import Session, abi
    cfg = abi.Config()
    cfg.abi_version = 1
    cfg.num_threads = 4
    s = Session(oracle.REF_LIB_PATH, cfg)
    yield s
    s.close()
