"""GPU: routing and the MLP of a layer in one call (aoship_route_mlp_forward) against the two
separate calls it replaces (aoship_route_features, then aoship_mlp_forward): the rings and
statuses equal bit for bit and the layer outputs equal bit for bit, at 1, 2 and 8 tokens (the
router inside the gate/up launch, the plan built by the router that finishes last), with more
adapters than that router split takes (the plan built by the launch's plan workgroup), at 40
tokens and with a router extra set (the calls in sequence), and repeated calls give the same
bits."""
import numpy as np
import pytest

import workloads as W
from cases import base, gpu_layer

pytestmark = pytest.mark.gpu


def _inputs(hip, cid, T):
    import torch

    cfg = W.CONFIGS[cid]
    f, w = W.router_inputs(cfg, T)
    xb, _ = W.activations(cfg, T)
    return cfg, torch.from_numpy(f).cuda(), torch.from_numpy(w).cuda(), torch.from_numpy(xb.view(np.int16)).cuda()


def _separate(router, layer, fd, wd, x):
    import torch

    T = x.shape[0]
    rings = torch.zeros(T * 40, dtype=torch.uint8, device="cuda")
    status = torch.full((T,), 7, dtype=torch.int32, device="cuda")
    y = torch.empty_like(x)
    router.route_features(fd, wd, rings, status=status)
    layer.mlp_forward(x, rings, y)
    torch.cuda.synchronize()
    return rings.cpu().numpy(), status.cpu().numpy(), y.cpu().numpy()


def _combined(router, layer, fd, wd, x):
    import torch

    T = x.shape[0]
    rings = torch.full((T * 40,), 0x5A, dtype=torch.uint8, device="cuda")
    status = torch.full((T,), 7, dtype=torch.int32, device="cuda")
    y = torch.empty_like(x)
    layer.route_mlp_forward(router, fd, wd, x, rings, y, status)
    torch.cuda.synchronize()
    return rings.cpu().numpy(), status.cpu().numpy(), y.cpu().numpy()


@pytest.mark.parametrize("cid,T", [(1, 1), (2, 1), (2, 2), (2, 8), (1, 40)])
def test_route_mlp_equals_separate_calls(hip, cid, T):
    cfg, fd, wd, x = _inputs(hip, cid, T)
    router = hip.Router(cfg.n_adapters, cfg.k, cfg.tau, cfg.eps, 1.0, np.arange(cfg.n_adapters, dtype=np.uint64))
    layer, ads = gpu_layer(hip, cid)
    ref = _separate(router, layer, fd, wd, x)
    got = _combined(router, layer, fd, wd, x)
    again = _combined(router, layer, fd, wd, x)
    assert layer.wait_timeouts() == 0
    for a, b, c, name in zip(ref, got, again, ("rings", "status", "y")):
        assert np.array_equal(a, b), f"{name} differs from the separate calls"
        assert np.array_equal(b, c), f"{name} differs run to run"


@pytest.mark.parametrize("T", [9, 16])
def test_route_mlp_many_adapters(hip, T):
    """72 adapters (over the 64 that the split router takes) at 9 and 16 tokens, where the x shrink
    covers every adapter and the router runs inside the gate/up launch: one router workgroup per
    token, and the plan workgroup waits for the routers' flag before it builds the plan."""
    import dataclasses

    import torch

    cfg = dataclasses.replace(W.CONFIGS[1], n_adapters=72)
    f, w = W.router_inputs(cfg, T)
    xb, _ = W.activations(cfg, T)
    fd, wd = torch.from_numpy(f).cuda(), torch.from_numpy(w).cuda()
    x = torch.from_numpy(xb.view(np.int16)).cuda()
    router = hip.Router(cfg.n_adapters, cfg.k, cfg.tau, cfg.eps, 1.0, np.arange(cfg.n_adapters, dtype=np.uint64))
    layer = hip.Layer(0)
    for m, (p, sc, b) in base(1).items():
        layer.set_base(m, p, sc, b)
    ads = []
    for a in range(cfg.n_adapters):
        ad = hip.LoraAdapter(a, 1, W.lora_scale(cfg))
        for m in cfg.modules:
            ad.set_module(0, m, *W.lora_weights(cfg, a, m))
        ads.append(ad)
    layer.set_adapters(ads)
    ref = _separate(router, layer, fd, wd, x)
    got = _combined(router, layer, fd, wd, x)
    again = _combined(router, layer, fd, wd, x)
    assert layer.wait_timeouts() == 0
    for a, b, c, name in zip(ref, got, again, ("rings", "status", "y")):
        assert np.array_equal(a, b), f"{name} differs from the separate calls"
        assert np.array_equal(b, c), f"{name} differs run to run"


def test_route_mlp_with_router_extras_runs_in_sequence(hip):
    """A scope hint set on the router: the call routes with the extras first, then runs the
    layer, and still equals the separate calls."""
    cid, T = 2, 4
    cfg, fd, wd, x = _inputs(hip, cid, T)
    router = hip.Router(cfg.n_adapters, cfg.k, cfg.tau, cfg.eps, 1.0, np.arange(cfg.n_adapters, dtype=np.uint64))
    scope = np.ones(cfg.n_adapters, np.uint8)
    scope[::3] = 0
    router.set_scope(scope)
    layer, ads = gpu_layer(hip, cid)
    ref = _separate(router, layer, fd, wd, x)
    got = _combined(router, layer, fd, wd, x)
    for a, b in zip(ref, got):
        assert np.array_equal(a, b)
