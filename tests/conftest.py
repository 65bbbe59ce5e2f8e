import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X); run with -m gpu")


def load_golden(rel: str) -> np.ndarray:
    """Reference fixture: raw little-endian fp32 (testing/teeny-test/src/fixtures.rs:19-41)."""
    return np.fromfile(os.path.join(GOLDEN, rel), dtype="<f4")


@pytest.fixture(scope="session")
def dev():
    import teenygrad_amd as tg

    n = tg.device_count()
    if n == 0:
        pytest.fail("no HIP device visible: GPU tests need an MI355X")
    d = tg.open(0)
    info = d.info()
    print(f"\n[device] {info['name']} {info['arch']} CUs={info['compute_units']}", flush=True)
    return d


@pytest.fixture(scope="session")
def orc():
    """The CPU oracle, rebuilt for this host (-march=native, the same
    -ffp-contract=off arithmetic as the prebuilt library: identical results,
    faster) and spread over at most 16 threads (a GPU host's CPU share)."""
    import oracle

    oracle.use_native_build()
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    oracle.set_threads(max(1, min(16, n)))
    return oracle
