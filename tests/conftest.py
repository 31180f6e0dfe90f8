"""Shared test setup. `-m gpu` tests run the HIP kernels on a real MI355X; everything else runs on
the CPU (oracle pins, golden fixtures, host logic, the C-ABI exports)."""

import os
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent
if str(REPO) not in sys.path:
    sys.path.insert(0, str(REPO))

GOLDEN = REPO / "tests" / "golden"


def pytest_configure(config: pytest.Config) -> None:
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (gfx950) and the built HIP library")


@pytest.fixture(scope="session")
def oracle():
    from oracle.native import OracleGemm

    return OracleGemm()


@pytest.fixture(scope="session")
def ref():
    """The reference C kernels built from /root/reference (oracle/_ref); skipped where absent."""
    from oracle.native import RefGemm, ref_available

    if not ref_available():
        pytest.skip("oracle/_ref/libmx_ref.so not built (needs /root/reference)")
    return RefGemm()


@pytest.fixture(scope="session")
def ref_nofma():
    from oracle.native import REF_LIB_NOFMA, RefGemm, ref_available

    if not ref_available(nofma=True):
        pytest.skip("oracle/_ref/libmx_ref_nofma.so not built (needs /root/reference)")
    return RefGemm(REF_LIB_NOFMA)


@pytest.fixture(scope="session")
def gpu():
    """The HIP library on cuda:0; prints the case name before each use so a GPU failure names
    its test."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from matricxon_amd.gemm import HipGemm

    return HipGemm.get()


@pytest.fixture(autouse=True)
def _announce(request: pytest.FixtureRequest):
    if request.node.get_closest_marker("gpu") is not None:
        print(f"\n[gpu case] {request.node.nodeid}", flush=True)
    yield


def threads() -> int:
    return int(os.environ.get("OMP_NUM_THREADS", "0")) or len(os.sched_getaffinity(0))
