"""GPU: the decode GEMV's launch shapes give the same layer, within tolerance of the oracle.

The decode GEMV can run a workgroup's waves over one row block (K split across the waves) or over
several row blocks sharing one staged x slice; the geometry picks the row blocks per workgroup (wr)
and the K splits (ks) per shape. These tests pin other shapes through the diagnostic setter, among
them ones whose last workgroup holds row blocks past the matrix (the 0.5B layer's 28 down row blocks
at 8 per workgroup), and check each against the oracle (2e-2 rule) and run to run. A pinned shape
that does not fit the LDS budget falls back to one that does, which is checked all the same.
"""
import numpy as np
import pytest

import workloads as W
from cases import REL_TOL, assert_parity, gpu_layer, oracle_mlp, oracle_proj, rings_for, tol_ratio

pytestmark = pytest.mark.gpu


def _dev(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _mlp(layer, x, r, T, H):
    import torch

    y = torch.empty((T, H), dtype=torch.int16, device="cuda")
    layer.mlp_forward(x, r, y)
    torch.cuda.synchronize()
    return y.cpu().numpy().view(np.uint16)


# (gate/up pin, down pin) as (wr, ks); 0 = the geometry's own choice
MLP_PINS = [((1, 2), (1, 8)), ((2, 3), (2, 4)), ((4, 2), (8, 3)), ((4, 7), (4, 5)), ((2, 14), (8, 12))]


@pytest.mark.parametrize("cid,T", [(1, 3), (1, 8), (1, 32), (2, 3), (2, 8), (2, 32)])
def test_mlp_decode_pinned_geometries(hip, cid, T):
    cfg = W.CONFIGS[cid]
    xb, xf = W.activations(cfg, T)
    rings, _ = rings_for(cid, T)
    ref = oracle_mlp(cid, xf, rings)
    layer, ads = gpu_layer(hip, cid)
    x, r = _dev(xb.view(np.int16)), _dev(rings.view(np.uint8))
    for gu, dn in MLP_PINS:
        layer.set_gemv_geometry(0, *gu)
        layer.set_gemv_geometry(1, *dn)
        y1 = _mlp(layer, x, r, T, cfg.hidden)
        y2 = _mlp(layer, x, r, T, cfg.hidden)
        assert layer.wait_timeouts() == 0
        assert np.array_equal(y1, y2), f"gate/up {gu}, down {dn}: run-to-run outputs differ"
        ratio = assert_parity(f"test_mlp_decode_pinned_geometries cid={cid} T={T} gu={gu} dn={dn}", W.bf16_bits_to_f32(y1).reshape(ref.shape), ref)
        assert ratio <= REL_TOL, f"gate/up {gu}, down {dn}: tolerance ratio {ratio:.4g}"


@pytest.mark.parametrize("T", [5, 32])
def test_projections_pinned_geometries(hip, T):
    import torch

    cid = 4
    cfg = W.CONFIGS[cid]
    xb, xf = W.activations(cfg, T)
    rings, _ = rings_for(cid, T)
    refs = {m: oracle_proj(cid, m, xf, rings) for m in cfg.modules}
    layer, ads = gpu_layer(hip, cid)
    x, r = _dev(xb.view(np.int16)), _dev(rings.view(np.uint8))
    for wr, ks in [(1, 8), (2, 6), (4, 3), (4, 10), (4, 16)]:
        layer.set_gemv_geometry(2, wr, ks)
        outs = {}
        for rep in range(2):
            q = torch.empty((T, cfg.q_out), dtype=torch.int16, device="cuda")
            k = torch.empty((T, cfg.kv_out), dtype=torch.int16, device="cuda")
            v = torch.empty((T, cfg.kv_out), dtype=torch.int16, device="cuda")
            o = torch.empty((T, cfg.hidden), dtype=torch.int16, device="cuda")
            layer.qkv_forward(x, r, q, k, v)
            layer.proj_forward("o_proj", x, r, o)
            torch.cuda.synchronize()
            cur = {m: t.cpu().numpy().view(np.uint16) for m, t in zip(cfg.modules, (q, k, v, o))}
            if rep:
                for m in cfg.modules:
                    assert np.array_equal(outs[m], cur[m]), f"wr {wr} ks {ks} {m}: run-to-run outputs differ"
            outs = cur
        for m in cfg.modules:
            ratio = assert_parity(f"test_projections_pinned_geometries T={T} wr={wr} ks={ks} {m}", W.bf16_bits_to_f32(outs[m]).reshape(refs[m].shape), refs[m])
            assert ratio <= REL_TOL, f"wr {wr} ks {ks} {m}: tolerance ratio {ratio:.4g}"
