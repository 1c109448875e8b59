"""The allocation-free decode MLP forward (aoship_mlp_forward_noalloc) against aoship_mlp_forward,
through the C ABI: bit-identical outputs on two calls in a row, the second with fewer tokens (the
scratch keeps the first call's contents), then a call on another layer after the first layer's
regular forward, and the documented rejections. The regular forward's output is itself checked
against the oracle by the decode parity tests; here it is also checked at one size."""
import numpy as np
import pytest

import workloads as W
from cases import REL_TOL, gpu_layer, oracle_mlp, rings_for, tol_ratio

pytestmark = pytest.mark.gpu


def _io(hip, cid, T):
    import torch

    xb, xf = W.activations(W.CONFIGS[cid], T)
    rings, _ = rings_for(cid, T)
    x = torch.from_numpy(np.ascontiguousarray(xb.view(np.int16))).cuda()
    r = torch.from_numpy(rings.view(np.uint8).copy()).cuda()
    return x, r, xf, rings


def _fwd(layer, x, r, noalloc):
    import torch

    y = torch.empty((x.shape[0], x.shape[1]), dtype=torch.int16, device="cuda")
    (layer.mlp_forward_noalloc if noalloc else layer.mlp_forward)(x, r, y)
    torch.cuda.synchronize()
    return y.cpu().numpy().view(np.uint16)


def test_noalloc_equals_mlp_forward(hip):
    cid = 2
    layer, ads = gpu_layer(hip, cid)
    for T in (8, 1):  # the second call is smaller and finds the first call's contents
        x, r, xf, rings = _io(hip, cid, T)
        print(f"noalloc T={T}", flush=True)
        got = _fwd(layer, x, r, True)
        want = _fwd(layer, x, r, False)
        assert np.array_equal(got, want), f"T={T}: the allocation-free forward differs"
        assert layer.wait_timeouts() == 0
        if T == 1:
            ref = oracle_mlp(cid, xf, rings)
            assert tol_ratio(W.bf16_bits_to_f32(got).reshape(ref.shape), ref) <= REL_TOL
    # another layer (other shapes) on the same scratch, after regular forwards of the first
    other, ads1 = gpu_layer(hip, 1)
    x, r, _, _ = _io(hip, 1, 3)
    assert np.array_equal(_fwd(other, x, r, True), _fwd(other, x, r, False))
    x, r, _, _ = _io(hip, cid, 2)
    assert np.array_equal(_fwd(layer, x, r, True), _fwd(layer, x, r, False))


def test_noalloc_rejections(hip):
    import torch

    layer, ads = gpu_layer(hip, 1)
    x, r, _, _ = _io(hip, 1, 33)
    y = torch.empty((33, x.shape[1]), dtype=torch.int16, device="cuda")
    with pytest.raises(hip.AosError, match="decode batches"):
        layer.mlp_forward_noalloc(x, r, y)
    big, ads2 = gpu_layer(hip, 2)
    x, r, _, _ = _io(hip, 2, 32)
    y = torch.empty((32, x.shape[1]), dtype=torch.int16, device="cuda")
    try:
        big.mlp_forward_noalloc(x, r, y)
        torch.cuda.synchronize()
        fits = True
    except hip.AosError as e:
        assert "the scratch holds" in str(e)
        fits = False
    if fits:  # when it fits, it must equal the regular forward
        assert np.array_equal(y.cpu().numpy().view(np.uint16), _fwd(big, x, r, False))
