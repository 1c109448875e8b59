"""The C++ host-side API (adapter-os_amd/host/aos_kernel_api.hpp) through its test program
tests/cpp/aos_host_test, built by __graft_entry__.build() (make -C tests/cpp)."""
import hashlib
import hmac
import json
import os
import subprocess
from pathlib import Path

import pytest

import oracle

# AOS_HOST_TEST selects another build of the program (the sanitizer build, aos_host_test_asan)
EXE = Path(os.environ.get("AOS_HOST_TEST") or Path(__file__).resolve().parent / "cpp" / "aos_host_test")


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


def _hkdf(ikm: bytes, info: bytes) -> bytes:
    prk = hmac.new(b"\x00" * 32, ikm, hashlib.sha256).digest()
    return hmac.new(prk, info + b"\x01", hashlib.sha256).digest()


@pytest.mark.parametrize("seed", [bytes(32), bytes([1] * 32), bytes(range(32))])
def test_determinism_context_seed_chain(seed):
    """DeterminismContext (adapteros-core/src/determinism.rs:138-176, seed.rs:986-1006) in C++
    against Python's hmac: router seed = hex(HKDF(request seed, "router")), with a manifest hash
    "router:<hex>", tie-break seed = HKDF(router seed, "router-tie"); a router seed that is not
    hex is hashed with BLAKE3 first."""
    if not EXE.exists():
        pytest.fail(f"{EXE} is not built: run make -C tests/cpp")
    r = subprocess.run([str(EXE), "seeds", seed.hex()], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stderr
    out = json.loads(r.stdout)
    router_seed = _hkdf(seed, b"router")
    assert out["router_seed_hex"] == router_seed.hex()
    assert out["tiebreak_seed"] == _hkdf(router_seed, b"router-tie").hex()
    manifest = oracle.blake3(b"manifest").hex()
    assert out["router_seed_with_manifest"] == _hkdf(seed, f"router:{manifest}".encode()).hex()
    assert out["low64"] == int.from_bytes(seed[:8], "little")
    r = subprocess.run([str(EXE), "seeds", seed.hex(), "not-a-hex-seed"], capture_output=True, text=True, timeout=60)
    out = json.loads(r.stdout)
    assert out["tiebreak_seed"] == _hkdf(oracle.blake3(b"not-a-hex-seed"), b"router-tie").hex()
