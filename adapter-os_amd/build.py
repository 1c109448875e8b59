"""Build the gfx950 library (libaoship.so), the synthetic-input helper (libaos_synth.so) and the
probes the bench reports beside the datasheet peaks (libaos_peak.so: the matrix-core peak and the
one-launch HBM stream).

Every HIP translation unit is compiled for gfx950 only, with IEEE float semantics: no fast-math,
no floating-point contraction, float32 denormals kept, and packed-FP32 instruction selection
disabled. Objects go to adapter-os_amd/_build/, the shared libraries next to this file.

Usage: python adapter-os_amd/build.py [--jobs N]
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libaoship.so"
SYNTH = PKG / "libaos_synth.so"
PEAK = PKG / "libaos_peak.so"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

HIP_FLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    f"--offload-arch={ARCH}",
    "-ffp-contract=off",
    "-fno-fast-math",
    "-fno-gpu-flush-denormals-to-zero",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-result",
    "-I", str(CSRC),
]

SOURCES = [
    "aoship_router.hip",
    "aoship_lora.hip",
    "aoship_gemv.hip",
    "aoship_gemm.hip",
    "aoship_model.hip",
    "aoship_liquid.hip",
    "aoship_mlp1.hip",
    "aoship_api.cpp",
]


# Kernels whose workgroups hand data to each other within the launch (the fused decode launches)
# must compile without a private stack: a non-inlined device function call in one of them (which
# forced a stack frame and one wave per SIMD) gave wrong one-token results even where the call
# was never taken. The build fails if one of them gets private memory.
NO_SCRATCH = ("aos_gemv_fused_kernel", "aos_route_gu_kernel", "aos_decode_mlp_kernel", "aos_mlp1_kernel")
RESOURCE_REMARKS = ["-Rpass-analysis=kernel-resource-usage"]


def _check_resources(src: str, text: str) -> None:
    kernel = None
    for line in text.splitlines():
        if "Function Name:" in line:
            kernel = line.split("Function Name:", 1)[1].split("[-Rpass", 1)[0].strip()
        elif "ScratchSize [bytes/lane]:" in line and kernel and any(k in kernel for k in NO_SCRATCH):
            size = int(line.split("ScratchSize [bytes/lane]:", 1)[1].split()[0])
            if size:
                raise SystemExit(f"build failed: {kernel} in {src} uses {size} bytes of private memory per lane")


def _run(cmd: list[str]) -> str:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(" ".join(cmd) + "\n" + proc.stdout + proc.stderr)
        raise SystemExit(f"build failed: {cmd[-1]}")
    # keep real warnings visible; drop the host pass's note about the GPU-only feature flag and
    # the resource-usage remarks (checked by _check_resources)
    noise = ("packed-fp32-ops", "warning generated", "warnings generated", "remark", "^", "|")
    for line in (proc.stdout + proc.stderr).splitlines():
        if line.strip() and not any(n in line for n in noise):
            sys.stderr.write(line + "\n")
    return proc.stdout + proc.stderr


def compile_one(src: str) -> Path:
    obj = BUILD / (Path(src).stem + ".o")
    lang = ["-x", "hip"]
    remarks = RESOURCE_REMARKS if src.endswith(".hip") else []
    out = _run([HIPCC, *lang, *HIP_FLAGS, *remarks, "-c", str(CSRC / src), "-o", str(obj)])
    _check_resources(src, out)
    return obj


def build(jobs: int = 4) -> None:
    if not Path(HIPCC).exists() and shutil.which("hipcc") is None:
        raise SystemExit("hipcc not found")
    BUILD.mkdir(exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(compile_one, SOURCES))
    tmp = LIB.with_suffix(".so.tmp")
    # no undefined symbols: a kernel whose host stub failed to instantiate must fail the build
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Wl,--no-undefined", "-o", str(tmp), *map(str, objs)])
    os.replace(tmp, LIB)
    tmp = SYNTH.with_suffix(".so.tmp")
    _run(["gcc", "-O2", "-std=c11", "-fPIC", "-shared", "-fopenmp", "-ffp-contract=off",
          "-o", str(tmp), str(PKG / "synth" / "aos_synth.c"), "-lm"])
    os.replace(tmp, SYNTH)
    tmp = PEAK.with_suffix(".so.tmp")
    _run([HIPCC, "-x", "hip", *HIP_FLAGS, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp),
          str(PKG / "probe" / "aos_mfma_peak.hip"), str(PKG / "probe" / "aos_hbm_stream.hip")])
    os.replace(tmp, PEAK)


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=4)
    a = ap.parse_args()
    build(a.jobs)
    print(f"built {LIB}, {SYNTH} and {PEAK}")
