"""LiquidKernel::blend_and_forward through the C ABI (crates/adapteros-lora-kernel-api/src/
liquid.rs:147-257).

CPU: the descriptor layout the binding uses equals the header's, and the reference's argument
checks (liquid.rs:163-219) reject what it rejects, in its order, before any device work.
GPU: the reference's own known answer (liquid.rs:267-336: two adapters, one float32 and one
bfloat16, half weight each -> [2.0, 4.0]) and seeded cases against the oracle's restatement
(orc_liquid_blend): 1-3 adapters, float32 / bfloat16 / mixed, zero coefficients, up.rows below
the output length (the rest stays 0), ranks 1..64, long inputs. Tolerance: the north-star's
2e-2 relative rule (tests/cases.py tol_ratio); float outputs are also bit-identical run to run.
"""
import ctypes as C
import shutil
import subprocess
from pathlib import Path

import numpy as np
import pytest

import aoship
from cases import REL_TOL, tol_ratio

ROOT = Path(__file__).resolve().parents[1]


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_liquid_descriptor_layout(tmp_path):
    src = tmp_path / "liq.c"
    src.write_text(
        '#include <stdio.h>\n#include <stddef.h>\n#include "aoship.h"\n'
        "int main(void){printf(\"%zu %zu %zu %zu %zu %zu %zu\\n\", sizeof(aoship_liquid_tensor_t),"
        " offsetof(aoship_liquid_tensor_t, len), sizeof(aoship_liquid_adapter_t),"
        " offsetof(aoship_liquid_adapter_t, down), offsetof(aoship_liquid_adapter_t, up),"
        " offsetof(aoship_liquid_adapter_t, alpha), (size_t)AOSHIP_LIQUID_MAX_ADAPTERS); return 0;}\n")
    exe = tmp_path / "liq"
    subprocess.run(["gcc", "-std=c11", "-Wall", "-Werror", "-I", str(ROOT / "include"), str(src), "-o", str(exe)],
                   check=True)
    out = [int(v) for v in subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split()]
    T, A = aoship._LiquidTensor, aoship._LiquidAdapter
    assert out == [C.sizeof(T), T.len.offset, C.sizeof(A), A.down.offset, A.up.offset, A.alpha.offset, 3]


def _desc(rows, cols, n=None, bf16=0, ptr=0x1000):
    return aoship._LiquidTensor(ptr, bf16, rows, cols, rows * cols if n is None else n)


def _call(adapters, coefs, in_len, out_len, x=0x2000, y=0x3000):
    n = len(adapters)
    arr = (aoship._LiquidAdapter * max(n, 1))()
    for i, (d, u, al) in enumerate(adapters):
        arr[i].id, arr[i].down, arr[i].up, arr[i].alpha = i, d, u, al
    cf = (C.c_float * max(len(coefs), 1))(*coefs)
    L = aoship.lib()
    L.aoship_clear_error()
    rc = L.aoship_liquid_blend_and_forward(C.cast(arr, C.c_void_p), n, C.cast(cf, C.c_void_p), len(coefs), x,
                                           in_len, y, out_len, None, None)
    return rc, L.aoship_get_last_error().decode()


@pytest.mark.parametrize("case,message", [
    ("zero", "Liquid blend requested with zero adapters"),
    ("four", "Liquid blend exceeds max adapters (4 > 3)"),
    ("coefs", "Liquid blend coefficient mismatch: 2 adapters vs 1 coefficients"),
    ("down_shape", "Liquid tensor down has inconsistent shape: rows*cols=4 != len=3"),
    ("up_shape", "Liquid tensor up has inconsistent shape: rows*cols=4 != len=5"),
    ("input", "Liquid adapter 1 input mismatch: down.cols=3 vs input len=2"),
    ("output", "Liquid adapter 0 output mismatch: up.rows=3 vs output len=2"),
    ("rank", "Liquid adapter 0 rank mismatch: up.cols=1 vs down.rows=2"),
    ("rank_limit", "rank 1025 exceeds 1024"),
])
def test_liquid_rejects_like_the_reference(case, message):
    """The checks of blend_and_forward_reference (liquid.rs:163-219), with its messages, in its
    order: the first failing check is the one reported. No device is needed (they run first)."""
    ok = (_desc(2, 2), _desc(2, 2), 1.0)
    if case == "zero":
        rc, err = _call([], [], 2, 2)
    elif case == "four":
        rc, err = _call([ok] * 4, [1.0] * 4, 2, 2)
    elif case == "coefs":
        rc, err = _call([ok, ok], [1.0], 2, 2)
    elif case == "down_shape":
        rc, err = _call([(_desc(2, 2, n=3), _desc(2, 2, n=5), 1.0)], [1.0], 2, 2)
    elif case == "up_shape":
        rc, err = _call([(_desc(2, 2), _desc(2, 2, n=5), 1.0)], [1.0], 2, 2)
    elif case == "input":
        rc, err = _call([ok, (_desc(2, 3), _desc(2, 2), 1.0)], [1.0, 1.0], 2, 2)
    elif case == "output":
        rc, err = _call([(_desc(2, 2), _desc(3, 2), 1.0)], [1.0], 2, 2)
    elif case == "rank":
        rc, err = _call([(_desc(2, 2), _desc(2, 1), 1.0)], [1.0], 2, 2)
    else:
        rc, err = _call([(_desc(1025, 2), _desc(2, 1025), 1.0)], [1.0], 2, 2)
    assert rc == -1
    assert message in err


def _bf16(a):
    import workloads as W

    return W.f32_to_bf16_bits(np.asarray(a, np.float32).ravel()).reshape(np.shape(a))


def _dev(a):
    import torch

    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        a = a.view(np.int16)
    return torch.from_numpy(a).cuda()


@pytest.mark.gpu
def test_liquid_reference_known_answer(hip):
    """liquid.rs:267-336: adapter 1 float32 (A = identity, B = [[1, 2], [3, 4]], alpha 2), adapter 2
    bfloat16 (A = ones, B = 0.5, alpha 1), coefficients 0.5 / 0.5, input [1, 1] -> [2.0, 4.0] within
    1e-5, precision bfloat16."""
    import torch

    a1 = _dev(np.array([[1, 0], [0, 1]], np.float32))
    b1 = _dev(np.array([[1, 2], [3, 4]], np.float32))
    a2 = _dev(_bf16(np.ones((2, 2))))
    b2 = _dev(_bf16(np.full((2, 2), 0.5)))
    x = _dev(np.ones(2, np.float32))
    y = torch.full((2,), 7.0, dtype=torch.float32, device="cuda")
    prec = hip.liquid_blend_and_forward([(a1, b1, 2.0), (a2, b2, 1.0)], [0.5, 0.5], x, y)
    hip.sync()
    assert prec == 1
    out = y.cpu().numpy()
    assert abs(out[0] - 2.0) < 1e-5 and abs(out[1] - 4.0) < 1e-5, out


@pytest.mark.gpu
@pytest.mark.parametrize("seed", range(9))
def test_liquid_matches_oracle(hip, seed):
    import torch

    import oracle

    rng = np.random.default_rng(0xAD0511 + seed)
    n = 1 + seed % 3  # 1, 2 and 3 adapters
    din = int(rng.choice([64, 896, 3584, 5000]))
    dout = int(rng.choice([32, 1000, 4864, 18944]))
    As, Bs, ranks, alphas, coefs, ads = [], [], [], [], [], []
    for a in range(n):
        r = int(rng.choice([1, 8, 16, 40, 64]))
        rows = dout if a == 0 else int(rng.integers(1, dout + 1))  # up.rows <= out_len
        A = rng.normal(0, 1 / np.sqrt(din), (r, din)).astype(np.float32)
        B = rng.normal(0, 0.05, (rows, r)).astype(np.float32)
        down_bf, up_bf = bool(rng.integers(0, 2)), bool(rng.integers(0, 2))
        if down_bf:
            A = _to_f32(_bf16(A))
        if up_bf:
            B = _to_f32(_bf16(B))
        As.append(A)
        Bs.append(np.pad(B, ((0, dout - rows), (0, 0))))  # the oracle writes every row; rows past stay 0
        ranks.append(r)
        alphas.append(float(rng.choice([1.0, 16.0, 32.0])))
        coefs.append(0.0 if (seed in (4, 7) and a == n - 1) else float(rng.uniform(-1, 1)))
        ads.append((_dev(_bf16(A)) if down_bf else _dev(A), _dev(_bf16(B[:rows])) if up_bf else _dev(B[:rows]),
                    alphas[-1]))
    x = rng.normal(0, 1, din).astype(np.float32)
    ref = oracle.liquid_blend(As, Bs, ranks, alphas, coefs, x, dout)
    y = torch.full((dout,), float("nan"), dtype=torch.float32, device="cuda")
    xd = _dev(x)
    hip.liquid_blend_and_forward(ads, coefs, xd, y)
    y1 = y.cpu().numpy()
    hip.liquid_blend_and_forward(ads, coefs, xd, y)
    assert np.array_equal(y.cpu().numpy(), y1), "run-to-run outputs differ"
    assert np.all(np.isfinite(y1))
    if not np.any(ref):  # every coefficient 0: the output is exactly zero, as the reference's
        assert not np.any(y1)
        return
    ratio = tol_ratio(y1, ref)
    print(f"[parity] liquid seed {seed}: {n} adapters, in {din}, out {dout}, ranks {ranks}: tolerance ratio {ratio:.4g}")
    assert ratio <= REL_TOL


def _to_f32(bits):
    return (np.asarray(bits, np.uint32) << 16).view(np.float32)
