"""CPU: the build's resource check refuses a private stack in the in-launch hand-off kernels."""
import importlib.util
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent


def _build_module():
    spec = importlib.util.spec_from_file_location("aos_build", ROOT / "adapter-os_amd" / "build.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _remarks(kernel: str, scratch: int) -> str:
    return (f"x.hip:1:1: remark: Function Name: {kernel} [-Rpass-analysis=kernel-resource-usage]\n"
            f"x.hip:1:1: remark:     VGPRs: 116 [-Rpass-analysis=kernel-resource-usage]\n"
            f"x.hip:1:1: remark:     ScratchSize [bytes/lane]: {scratch} [-Rpass-analysis=kernel-resource-usage]\n")


def test_guard_rejects_scratch_in_handoff_kernels():
    b = _build_module()
    for k in ("_ZN12_GLOBAL__N_119aos_route_gu_kernelILi1EEEv19aos_route_gu_params",
              "_ZN12_GLOBAL__N_121aos_gemv_fused_kernelILi1ELb1ELi4ELi4EEEv21aos_gemv_fused_params",
              "_ZN12_GLOBAL__N_121aos_decode_mlp_kernelILi1EEEv21aos_decode_mlp_params"):
        with pytest.raises(SystemExit):
            b._check_resources("x.hip", _remarks(k, 1736))
        b._check_resources("x.hip", _remarks(k, 0))


def test_guard_ignores_other_kernels():
    b = _build_module()
    b._check_resources("x.hip", _remarks("_ZN12_GLOBAL__N_116aos_route_kernelILb1EEEv16aos_route_params", 8))
