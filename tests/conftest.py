"""Shared fixtures.  GPU tests are marked ``gpu``; everything else runs on the
CPU (oracle, host algebra, the C ABI's host entry points and export list)."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

import __graft_entry__  # noqa: E402


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP) device")
    # Build what is missing (only then): the oracle is a few seconds of gcc,
    # the HIP library and its torch binding about two minutes.
    if not os.path.exists(os.path.join(ROOT, "oracle", "libec_oracle.so")):
        subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle")], check=True)
    if not all(os.path.exists(os.path.join(ROOT, "megatron-lm_amd", f))
               for f in ("libec_mi355.so", "_ec_shards.so")):
        subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "megatron-lm_amd")], check=True)


@pytest.fixture(scope="session")
def pkg():
    return __graft_entry__.load_package()


@pytest.fixture(scope="session")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a visible HIP device")
    return torch.device("cuda:0")


GOLDEN = os.path.join(ROOT, "tests", "golden")
