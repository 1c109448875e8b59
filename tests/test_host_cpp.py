"""The C++ host-side API (adapter-os_amd/host/aos_kernel_api.hpp) through its test program
tests/cpp/aos_host_test, built by __graft_entry__.build() (make -C tests/cpp)."""
import subprocess
from pathlib import Path

import pytest

EXE = Path(__file__).resolve().parent / "cpp" / "aos_host_test"


def _run(mode: str) -> None:
    if not EXE.exists():
        pytest.fail(f"{EXE} is not built: run make -C tests/cpp")
    r = subprocess.run([str(EXE), mode], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr


def test_host_api_cpu():
    """RouterRing / Decision / Router construction semantics (no device work)."""
    _run("cpu")


@pytest.mark.gpu
def test_host_api_gpu():
    """The reference's router and LoRA tests through the C++ API on the device, hot-swap included."""
    _run("gpu")
