"""GPU: the one-token MLP in one launch with the down matrix held in LDS (aoship_mlp1.hip), the path
aoship_mlp_forward and aoship_route_mlp_forward take for one token when the layer opts in
(aoship_internal_layer_set_mlp1).
Against the oracle within the tolerance (per element, and the norm-wise relative error), bit-identical
run to run, against the two-launch decode path within the tolerance, on hand-made rings (an adapter
named twice, zero and negative gates, an index past the table, an empty ring, eight slots), without
adapters, and with the routing in the same launch (rings bit-exact against the oracle, outputs equal
to the separate calls')."""
import numpy as np
import pytest

import workloads as W
from cases import REL_TOL, base, gpu_layer, norm_rel_err, oracle_mlp, report, rings_for

pytestmark = pytest.mark.gpu

NORM_TOL = 2e-2


def _run(layer, xb, rings):
    import torch

    T, H = xb.shape
    x = torch.from_numpy(np.ascontiguousarray(xb.view(np.int16))).cuda()
    r = torch.from_numpy(rings.view(np.uint8).copy()).cuda()
    y = torch.empty((T, H), dtype=torch.int16, device="cuda")
    layer.mlp_forward(x, r, y)
    torch.cuda.synchronize()
    return W.bf16_bits_to_f32(y.cpu().numpy().view(np.uint16))


def _check(name, got, ref):
    ratio = report(name, got, ref)
    assert ratio <= REL_TOL, f"{name}: worst tolerance ratio {ratio:.4g}"
    assert norm_rel_err(got, ref) <= NORM_TOL, f"{name}: norm-wise relative error"


@pytest.mark.parametrize("cid", [1, 2])
def test_mlp1_parity(hip, cid):
    print(f"mlp1 parity cid={cid}", flush=True)
    xb, xf = W.activations(W.CONFIGS[cid], 1)
    rings, _ = rings_for(cid, 1)
    layer, ads = gpu_layer(hip, cid)
    layer.set_mlp1(True)
    y1 = _run(layer, xb, rings)
    y2 = _run(layer, xb, rings)
    assert layer.wait_timeouts() == 0
    assert np.array_equal(y1, y2), "run-to-run outputs differ"
    ref = oracle_mlp(cid, xf, rings)
    _check(f"mlp1 cid {cid}", y1.reshape(ref.shape), ref)
    layer.set_mlp1(False)
    y_old = _run(layer, xb, rings)
    layer.set_mlp1(True)
    _check(f"two-launch cid {cid}", y_old.reshape(ref.shape), ref)
    assert np.array_equal(_run(layer, xb, rings), y1)


def _ring(idx, gates, k=None):
    import oracle

    r = np.zeros(1, dtype=oracle.RING_DTYPE)
    r["top_k"] = len(idx) if k is None else k
    r["adapter_indices"][0, : len(idx)] = idx
    r["gates_q15"][0, : len(gates)] = gates
    return r


@pytest.mark.parametrize("case", ["twice", "zero_negative", "past_table", "empty", "eight"])
def test_mlp1_ring_cases(hip, case):
    cid = 2
    n = W.CONFIGS[cid].n_adapters
    rings = {
        "twice": _ring([3, 3, 7, 1], [9000, 12000, 6000, 5767]),
        "zero_negative": _ring([2, 5, 9, 11], [20000, 0, -300, 12767]),
        "past_table": _ring([4, n + 3, 6, 0], [8000, 16000, 4000, 4767]),
        "empty": _ring([1, 2], [100, 200], k=0),
        "eight": _ring([0, 15, 3, 12, 8, 5, 10, 1], [6000, 5000, 4000, 3000, 2500, 2000, 1500, 767]),
    }[case]
    print(f"mlp1 ring case {case}", flush=True)
    xb, xf = W.activations(W.CONFIGS[cid], 1)
    layer, ads = gpu_layer(hip, cid)
    layer.set_mlp1(True)
    got = _run(layer, xb, rings)
    assert layer.wait_timeouts() == 0
    ref = oracle_mlp(cid, xf, rings)
    _check(f"mlp1 ring {case}", got.reshape(ref.shape), ref)


def test_mlp1_without_adapters(hip):
    cid = 2
    cfg = W.CONFIGS[cid]
    print("mlp1 without adapters", flush=True)
    layer = hip.Layer(0)
    layer.set_mlp1(True)
    for m, (p, s, b) in base(cid).items():
        layer.set_base(m, p, s, b)
    xb, xf = W.activations(cfg, 1)
    rings, _ = rings_for(cid, 1)
    got = _run(layer, xb, rings)
    assert layer.wait_timeouts() == 0
    empty = _ring([], [], k=0)
    ref = oracle_mlp(cid, xf, empty)
    _check("mlp1 no adapters", got.reshape(ref.shape), ref)


@pytest.mark.parametrize("cid", [1, 2])
def test_mlp1_with_routing(hip, cid):
    import torch

    print(f"mlp1 with routing cid={cid}", flush=True)
    cfg = W.CONFIGS[cid]
    f, w = W.router_inputs(cfg, 1)
    fd, wd = torch.from_numpy(f).cuda(), torch.from_numpy(w).cuda()
    xb, xf = W.activations(cfg, 1)
    x = torch.from_numpy(xb.view(np.int16)).cuda()
    router = hip.Router(cfg.n_adapters, cfg.k, cfg.tau, cfg.eps, 1.0, np.arange(cfg.n_adapters, dtype=np.uint64))
    layer, ads = gpu_layer(hip, cid)
    layer.set_mlp1(True)
    outs = []
    for _ in range(2):
        rings = torch.full((40,), 0x5A, dtype=torch.uint8, device="cuda")
        status = torch.full((1,), 7, dtype=torch.int32, device="cuda")
        y = torch.empty_like(x)
        layer.route_mlp_forward(router, fd, wd, x, rings, y, status)
        torch.cuda.synchronize()
        outs.append((rings.cpu().numpy(), status.cpu().numpy(), y.cpu().numpy()))
    assert layer.wait_timeouts() == 0
    for a, b in zip(*outs):
        assert np.array_equal(a, b), "run-to-run outputs differ"
    o_rings, _ = rings_for(cid, 1)
    assert outs[0][0].tobytes() == o_rings.tobytes(), "rings differ from the oracle"
    assert int(outs[0][1][0]) == 0
    y_sep = _run(layer, xb, o_rings)
    assert np.array_equal(W.bf16_bits_to_f32(outs[0][2].view(np.uint16)), y_sep), "differs from the separate calls"
    ref = oracle_mlp(cid, xf, o_rings)
    _check(f"route + mlp1 cid {cid}", y_sep.reshape(ref.shape), ref)
