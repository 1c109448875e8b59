"""GPU: the give-up path of the in-launch hand-offs. With the wait bound set to 0 polls
(aoship_internal_set_spin_limit) every bounded wait of every launch gives up before its first poll,
so each kernel skips what it waited for and still runs to its end. For each fused path (the
two-launch decode MLP with per-producer lines and with the counted hand-off, the one-launch MLP of 1-2
tokens, the one-token launch with the down matrix in LDS (plain and routed), the router inside the
gate/up launch, the allocation-free MLP, the q/k/v projections, the prefill
GEMMs with their tile shrinks, and the stream-K prefill GEMMs): the forward that gave up is reported, the next forward on the layer
is refused (-1), aoship_layer_wait_timeouts reports 1 and resets the layer (then 0), and a forward
with the default bound equals the output from before the give-up bit for bit."""
import numpy as np
import pytest

import workloads as W
from cases import gpu_layer, rings_for

pytestmark = pytest.mark.gpu


def _dev_rings(hip, cid, T):
    import torch

    rings, _ = rings_for(cid, T)
    return torch.from_numpy(rings.view(np.uint8).copy()).cuda()


def _x(cid, T):
    import torch

    xb, _ = W.activations(W.CONFIGS[cid], T)
    return torch.from_numpy(xb.view(np.int16)).cuda()


def _give_up(hip, layer, run):
    """run() once with the default bound (reference), once with the bound at 0, then checks the
    report, the refusal, the reset and a clean run equal to the reference."""
    import torch

    ref = run()
    torch.cuda.synchronize()
    assert layer.wait_timeouts() == 0
    hip.set_spin_limit(0)
    try:
        run()
        torch.cuda.synchronize()
    finally:
        hip.set_spin_limit(hip.SPIN_LIMIT_DEFAULT)
    with pytest.raises(hip.AosError, match="gave up a bounded wait"):
        run()
    assert layer.wait_timeouts() == 1
    assert layer.wait_timeouts() == 0
    got = run()
    torch.cuda.synchronize()
    assert layer.wait_timeouts() == 0
    assert np.array_equal(ref, got), "output after the reset differs from the output before the give-up"


def _mlp_runner(layer, cid, T, noalloc=False):
    import torch

    x, rings = _x(cid, T), _dev_rings(None, cid, T)

    def run():
        y = torch.empty((T, W.CONFIGS[cid].hidden), dtype=torch.int16, device="cuda")
        (layer.mlp_forward_noalloc if noalloc else layer.mlp_forward)(x, rings, y)
        torch.cuda.synchronize()
        return y.cpu().numpy()

    return run


@pytest.mark.parametrize("T", [1, 2, 8])
def test_giveup_two_launch_decode(hip, T):
    layer, _ = gpu_layer(hip, 2)
    _give_up(hip, layer, _mlp_runner(layer, 2, T))


def test_giveup_counted_handoff(hip):
    layer, _ = gpu_layer(hip, 2)
    layer.set_decode_handoff(False, False)
    _give_up(hip, layer, _mlp_runner(layer, 2, 1))


@pytest.mark.parametrize("T", [1, 2])
def test_giveup_one_launch_mlp(hip, T):
    layer, _ = gpu_layer(hip, 2)
    layer.set_decode_handoff(True, True)
    _give_up(hip, layer, _mlp_runner(layer, 2, T))


def test_giveup_noalloc(hip):
    layer, _ = gpu_layer(hip, 2)
    _give_up(hip, layer, _mlp_runner(layer, 2, 1, noalloc=True))


@pytest.mark.parametrize("T", [40, 300])
def test_giveup_prefill(hip, T):
    layer, _ = gpu_layer(hip, 1)
    _give_up(hip, layer, _mlp_runner(layer, 1, T))


def test_giveup_prefill_stream_k(hip):
    """The stream-K prefill GEMMs (7B-shaped layer, 1100 tokens in 9 token tiles, shrinks in
    launches of their own): owners that give up waiting for the other pieces' partial sums still
    end."""
    layer, _ = gpu_layer(hip, 3)
    layer.set_prefill_shrink(False)
    run = _mlp_runner(layer, 3, 1100)
    run()
    assert layer.last_stream_k() == 3
    _give_up(hip, layer, run)


def _route_mlp_runner(hip, layer, cid, T):
    import torch

    cfg = W.CONFIGS[cid]
    f, w = W.router_inputs(cfg, T)
    fd, wd, x = torch.from_numpy(f).cuda(), torch.from_numpy(w).cuda(), _x(cid, T)
    router = hip.Router(cfg.n_adapters, cfg.k, cfg.tau, cfg.eps, 1.0, np.arange(cfg.n_adapters, dtype=np.uint64))

    def run():
        rings = torch.zeros(T * 40, dtype=torch.uint8, device="cuda")
        y = torch.empty((T, cfg.hidden), dtype=torch.int16, device="cuda")
        layer.route_mlp_forward(router, fd, wd, x, rings, y)
        torch.cuda.synchronize()
        return np.concatenate([rings.cpu().numpy().view(np.uint8), y.cpu().numpy().view(np.uint8).ravel()])

    return run


@pytest.mark.parametrize("T", [1, 8])
def test_giveup_route_mlp(hip, T):
    layer, _ = gpu_layer(hip, 2)
    _give_up(hip, layer, _route_mlp_runner(hip, layer, 2, T))


@pytest.mark.parametrize("routed", [False, True])
def test_giveup_mlp1(hip, routed):
    layer, _ = gpu_layer(hip, 2)
    layer.set_mlp1(True)
    _give_up(hip, layer, _route_mlp_runner(hip, layer, 2, 1) if routed else _mlp_runner(layer, 2, 1))


@pytest.mark.parametrize("T", [2, 32])
def test_giveup_qkv(hip, T):
    import torch

    cid = 4
    cfg = W.CONFIGS[cid]
    layer, _ = gpu_layer(hip, cid)
    x, rings = _x(cid, T), _dev_rings(hip, cid, T)

    def run():
        q = torch.empty((T, cfg.q_out), dtype=torch.int16, device="cuda")
        k = torch.empty((T, cfg.kv_out), dtype=torch.int16, device="cuda")
        v = torch.empty((T, cfg.kv_out), dtype=torch.int16, device="cuda")
        layer.qkv_forward(x, rings, q, k, v)
        torch.cuda.synchronize()
        return np.concatenate([q.cpu().numpy().ravel(), k.cpu().numpy().ravel(), v.cpu().numpy().ravel()])

    _give_up(hip, layer, run)
