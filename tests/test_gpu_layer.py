"""GPU layer parity: the int4 + LoRA layer kernels against the CPU oracle.

Tolerance (from the workload definition): every output element within 2e-2 relative of the
oracle, |gpu - ref| <= 2e-2 * (|ref| + rms(ref)). Run-to-run results must be bit-identical.
"""
import numpy as np
import pytest

import workloads as W
from cases import REL_TOL, gpu_layer, oracle_mlp, oracle_proj, rings_for, tol_ratio

pytestmark = pytest.mark.gpu


def _dev(a, dtype=None):
    import torch

    t = torch.from_numpy(np.ascontiguousarray(a))
    return t.cuda()


def _run_mlp(hip, layer, xb, rings):
    import torch

    T, H = xb.shape
    x = _dev(xb.view(np.int16))
    r = _dev(rings.view(np.uint8))
    y = torch.empty((T, H), dtype=torch.int16, device="cuda")
    layer.mlp_forward(x, r, y)
    torch.cuda.synchronize()
    return y.cpu().numpy().view(np.uint16)


@pytest.mark.parametrize("cid,T", [(1, 1), (2, 1), (2, 8)])
def test_mlp_decode_parity(hip, cid, T):
    xb, xf = W.activations(W.CONFIGS[cid], T)
    rings, _ = rings_for(cid, T)
    layer, ads = gpu_layer(hip, cid)
    y1 = _run_mlp(hip, layer, xb, rings)
    y2 = _run_mlp(hip, layer, xb, rings)
    assert np.array_equal(y1, y2), "run-to-run outputs differ"
    ref = oracle_mlp(cid, xf, rings)
    ratio = tol_ratio(W.bf16_bits_to_f32(y1).reshape(ref.shape), ref)
    assert ratio <= REL_TOL, f"max tolerance ratio {ratio:.4g}"


def test_mlp_no_adapters_matches_base(hip):
    """Zero gates / empty rings: the layer is the plain int4 SwiGLU MLP."""
    cid, T = 1, 4
    xb, xf = W.activations(W.CONFIGS[cid], T)
    rings = np.zeros(T, dtype=hip.RING_DTYPE)
    layer, ads = gpu_layer(hip, cid)
    y = _run_mlp(hip, layer, xb, rings)
    ref = oracle_mlp(cid, xf, rings)
    assert tol_ratio(W.bf16_bits_to_f32(y).reshape(ref.shape), ref) <= REL_TOL


def test_mlp_prefill_shape_parity(hip):
    """2048-token prefill of the 7B-shaped layer, checked on a sample of tokens."""
    cid, T = 3, 2048
    xb, xf = W.activations(W.CONFIGS[cid], T)
    rings, _ = rings_for(cid, T)
    layer, ads = gpu_layer(hip, cid)
    y = _run_mlp(hip, layer, xb, rings)
    sample = np.array([0, 1, 2, 31, 32, 33, 511, 1024, 1500, 2046, 2047])
    ref = oracle_mlp(cid, xf[sample], rings[sample])
    got = W.bf16_bits_to_f32(y.reshape(T, -1)[sample])
    assert tol_ratio(got, ref) <= REL_TOL


def test_attention_projections_parity(hip):
    import torch

    cid, T = 4, 32
    cfg = W.CONFIGS[cid]
    xb, xf = W.activations(cfg, T)
    rings, _ = rings_for(cid, T)
    layer, ads = gpu_layer(hip, cid)
    x = _dev(xb.view(np.int16))
    r = _dev(rings.view(np.uint8))
    q = torch.empty((T, cfg.q_out), dtype=torch.int16, device="cuda")
    k = torch.empty((T, cfg.kv_out), dtype=torch.int16, device="cuda")
    v = torch.empty((T, cfg.kv_out), dtype=torch.int16, device="cuda")
    layer.qkv_forward(x, r, q, k, v)
    o = torch.empty((T, cfg.hidden), dtype=torch.int16, device="cuda")
    layer.proj_forward("o_proj", x, r, o)  # o's input: any [T, 3072] activation; reuse x
    torch.cuda.synchronize()
    for name, dev in (("q_proj", q), ("k_proj", k), ("v_proj", v), ("o_proj", o)):
        got = W.bf16_bits_to_f32(dev.cpu().numpy().view(np.uint16))
        ref = oracle_proj(cid, name, xf, rings)
        ratio = tol_ratio(got.reshape(ref.shape), ref)
        assert ratio <= REL_TOL, f"{name}: {ratio:.4g}"
