"""CPU checks of the C ABI (no GPU, no compute calls): the shared library loads, exports every
function include/aoship.h declares, and the 40-byte ring has the reference's layout."""
from __future__ import annotations

import ctypes
import shutil
import subprocess
from pathlib import Path

import numpy as np
import pytest

import aoship

ROOT = Path(__file__).resolve().parent.parent


def test_library_exports_every_header_symbol():
    syms = aoship.header_symbols()
    assert len(syms) >= 25
    L = ctypes.CDLL(str(aoship.LIB_PATH))
    missing = [s for s in syms if not hasattr(L, s)]
    assert not missing, missing


def test_binding_covers_header():
    """Every declared function has a ctypes signature in the binding."""
    assert set(aoship.header_symbols()) <= set(aoship._SIGS)


def test_version_and_error_convention():
    """Thread-local error text (mlx_get_last_error / mlx_clear_error, wrapper.h:199-200)."""
    L = aoship.lib()
    assert L.aoship_version().decode().startswith("aoship ")
    L.aoship_clear_error()
    assert L.aoship_get_last_error().decode() == ""
    # argument errors are reported before any device work
    assert not L.aoship_router_new(4, 9, 1.0, 0.02, 1.0, None)
    assert "exceeds maximum" in L.aoship_get_last_error().decode()
    L.aoship_clear_error()
    assert L.aoship_route(None, None, 1, None, None) == -1
    assert L.aoship_get_last_error().decode() != ""
    L.aoship_clear_error()


def test_ring_layout():
    """40 bytes, align 4, fields at 0 / 4 / 8 / 24 (MetalRingBufferLayout,
    crates/adapteros-lora-kernel-mtl/src/ring_buffer.rs:52-58; miri_safe_tests.rs:103-134)."""
    dt = aoship.RING_DTYPE
    assert dt.itemsize == 40
    assert [dt.fields[n][1] for n in ("top_k", "current_pos", "adapter_indices", "gates_q15")] == [0, 4, 8, 24]
    import oracle

    assert oracle.RING_DTYPE == dt


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_header_compiles_and_matches_layout(tmp_path):
    src = tmp_path / "lay.c"
    src.write_text(
        '#include <stdio.h>\n#include <stddef.h>\n#include "aoship.h"\n'
        "int main(void){printf(\"%zu %zu %zu %zu %zu %zu\\n\", sizeof(aoship_ring_t), _Alignof(aoship_ring_t),"
        " offsetof(aoship_ring_t, current_pos), offsetof(aoship_ring_t, adapter_indices),"
        " offsetof(aoship_ring_t, gates_q15), (size_t)AOSHIP_MAX_K); return 0;}\n")
    exe = tmp_path / "lay"
    subprocess.run(["gcc", "-std=c11", "-Wall", "-Werror", "-I", str(ROOT / "include"), str(src), "-o", str(exe)],
                   check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split()
    assert out == ["40", "4", "4", "8", "24", "8"]


def test_product_path_has_no_oracle_dependency():
    """The library and its binding never load the oracle: no reference to oracle/ or liborc in the
    package sources or the built library's dynamic dependencies."""
    pkg = ROOT / "adapter-os_amd"
    for p in list(pkg.glob("*.py")) + list((pkg / "csrc").glob("*")):
        text = p.read_text(errors="ignore")
        assert "liborc" not in text and "import oracle" not in text, p
    out = subprocess.run(["ldd", str(aoship.LIB_PATH)], capture_output=True, text=True).stdout
    assert "liborc" not in out


def test_binding_fails_loudly_without_library(tmp_path, monkeypatch):
    """No silent fallback: a missing library is an ImportError, not a CPU path."""
    monkeypatch.setattr(aoship, "_lib", None)
    monkeypatch.setattr(aoship, "LIB_PATH", tmp_path / "missing.so")
    with pytest.raises(ImportError):
        aoship.lib()


def test_ring_roundtrip_bytes():
    r = np.zeros(3, aoship.RING_DTYPE)
    r[1]["top_k"] = 2
    r[1]["adapter_indices"][:2] = [5, 9]
    r[1]["gates_q15"][:2] = [20000, 12767]
    back = aoship.rings_from_bytes(r.view(np.uint8))
    assert back.tobytes() == r.tobytes()


def test_attestation_is_a_valid_determinism_report():
    """aoship_attest_determinism (no device needed) serializes DeterminismReport's fields and
    passes the checks of DeterminismReport::validate (attestation.rs:160-214), restated."""
    import json

    import aoship

    r = json.loads(aoship.attest_determinism())
    for key in ("backend_type", "metallib_hash", "manifest", "rng_seed_method", "floating_point_mode",
                "determinism_level", "compiler_flags", "deterministic"):
        assert key in r, key
    assert r["backend_type"] == "Hip" and r["deterministic"] is True
    assert r["determinism_level"] in ("bit_exact", "bounded_tolerance")
    assert r["rng_seed_method"] == "HkdfSeeded" or "FixedSeed" in r["rng_seed_method"]
    assert r["floating_point_mode"] == "Deterministic"
    assert not any(f in flag for flag in r["compiler_flags"] for f in ("-ffast-math", "-funsafe-math-optimizations"))
