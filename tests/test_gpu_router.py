"""GPU router parity: rings from the HIP router must equal the CPU oracle's bit for bit.

Covers the reference's router known answers (crates/adapteros-lora-router/tests/determinism.rs,
q15_edge_cases.rs), every workload's routing at full token counts (features -> priors on the
device for configs 1, 2, 4; prototype priors for 3; adversarial ties / signed zeros / Q15
boundaries / dominance with eps = 0 for 5), N above one wavefront, policy masks and the
non-finite error path.
"""
import json
from pathlib import Path

import numpy as np
import pytest

import workloads as W
from cases import rings_for

pytestmark = pytest.mark.gpu


def _gpu_route(hip, priors, k, tau=1.0, eps=0.02, bias=1.0, stable_ids=None, allowed=None):
    import torch

    pri = np.ascontiguousarray(priors, np.float32)
    T, n = pri.shape
    r = hip.Router(n, k, tau, eps, bias, stable_ids)
    if allowed is not None:
        r.set_policy_mask(allowed)
    dp = torch.from_numpy(pri).cuda()
    rings = torch.zeros(T * 40, dtype=torch.uint8, device="cuda")
    status = torch.full((T,), 7, dtype=torch.int32, device="cuda")
    r.route(dp, rings, status)
    torch.cuda.synchronize()
    return hip.rings_from_bytes(rings.cpu().numpy()), status.cpu().numpy()


def _oracle_rings(priors, k, tau=1.0, eps=0.02, bias=1.0, stable_ids=None, allowed=None):
    import oracle

    return oracle.route_batch(priors, k, tau, eps, bias, stable_ids, allowed)


def _assert_rings_equal(g, o):
    assert g.tobytes() == o.tobytes(), _first_diff(g, o)


def _first_diff(g, o):
    for t in range(len(g)):
        if g[t].tobytes() != o[t].tobytes():
            return f"token {t}: gpu {g[t]} oracle {o[t]}"
    return "equal"


GOLDEN = Path(__file__).resolve().parent / "golden"
KATS = json.loads((GOLDEN / "router_kats.json").read_text())["cases"]


@pytest.mark.parametrize("kat", KATS, ids=lambda c: c["name"])
def test_router_reference_kats(hip, kat):
    """The reference's router known answers (sources cited in the fixture), bit-exact with the
    oracle and equal to the asserted indices / gates."""
    pri = np.array([kat["priors"]], np.float32)
    ids = np.array(kat["stable_ids"], np.uint64)
    allowed = None if kat.get("allowed") is None else np.array(kat["allowed"], np.uint8)
    g, st = _gpu_route(hip, pri, kat["k"], kat["tau"], kat["eps"], 1.0, ids, allowed)
    o = _oracle_rings(pri, kat["k"], kat["tau"], kat["eps"], 1.0, ids, allowed)
    assert st[0] == 0
    _assert_rings_equal(g, o)
    kk = int(g[0]["top_k"])
    assert list(g[0]["adapter_indices"][:kk]) == kat["expect_indices"]
    if kat.get("expect_gates") is not None:
        assert list(g[0]["gates_q15"][:kk]) == kat["expect_gates"]


def test_router_adversarial_fixture(hip):
    """Committed 64-adapter adversarial vectors (ties, signed zeros, Q15 boundaries with eps = 0,
    a dominant adapter): the device rings equal the fixture byte for byte."""
    fx = np.load(GOLDEN / "router_adversarial.npz")
    pri = fx["priors"]
    sid = np.arange(pri.shape[1], dtype=np.uint64)
    g, st = _gpu_route(hip, pri, int(fx["k"]), float(fx["tau"]), float(fx["eps"]), 1.0, sid)
    assert (st == 0).all()
    assert g.tobytes() == fx["rings"].tobytes()


@pytest.mark.parametrize("cid,T", [(1, 1), (2, 1), (2, 8), (3, 2048), (4, 32), (5, 4096)])
def test_router_workloads_bit_exact(hip, cid, T):
    import torch

    cfg = W.CONFIGS[cid]
    o_rings, o_pri = rings_for(cid, T)
    sid = np.arange(cfg.n_adapters, dtype=np.uint64)
    if cfg.routing == "features":
        f, w = W.router_inputs(cfg, T)
        r = hip.Router(cfg.n_adapters, cfg.k, cfg.tau, cfg.eps, 1.0, sid)
        rings = torch.zeros(T * 40, dtype=torch.uint8, device="cuda")
        pri = torch.zeros((T, cfg.n_adapters), dtype=torch.float32, device="cuda")
        status = torch.full((T,), 7, dtype=torch.int32, device="cuda")
        r.route_features(torch.from_numpy(f).cuda(), torch.from_numpy(w).cuda(), rings, pri, status)
        torch.cuda.synchronize()
        assert np.array_equal(pri.cpu().numpy().view(np.uint32), o_pri.view(np.uint32)), "priors differ"
        g = hip.rings_from_bytes(rings.cpu().numpy())
        assert (status.cpu().numpy() == 0).all()
    else:
        g, st = _gpu_route(hip, o_pri, cfg.k, cfg.tau, cfg.eps, 1.0, sid)
        assert (st == 0).all()
    _assert_rings_equal(g, o_rings)


@pytest.mark.parametrize("n", [63, 64, 65, 200, 1000])
def test_router_many_adapters_with_ties(hip, n):
    rng = np.random.default_rng(n)
    T = 64
    pri = (np.floor(rng.normal(size=(T, n)) * 3) / 4).astype(np.float32)  # many exact ties
    ids = rng.permutation(n).astype(np.uint64)
    for k in (1, 3, 8):
        g, _ = _gpu_route(hip, pri, k, 1.0, 0.02, 1.2, ids)
        _assert_rings_equal(g, _oracle_rings(pri, k, 1.0, 0.02, 1.2, ids))


def test_router_policy_mask_and_nonfinite(hip):
    rng = np.random.default_rng(5)
    pri = rng.normal(size=(16, 24)).astype(np.float32)
    allowed = (rng.random(24) > 0.4).astype(np.uint8)
    g, st = _gpu_route(hip, pri, 4, allowed=allowed)
    _assert_rings_equal(g, _oracle_rings(pri, 4, allowed=allowed))
    bad = pri.copy()
    bad[3, 7] = np.nan
    bad[9, 0] = np.inf
    g, st = _gpu_route(hip, bad, 4)
    assert st[3] == -1 and st[9] == -1 and (np.delete(st, [3, 9]) == 0).all()
    assert g[3].tobytes() == bytes(40) and g[9].tobytes() == bytes(40)
    o = _oracle_rings(bad, 4)
    _assert_rings_equal(g, o)


def test_router_k_above_8_rejected(hip):
    with pytest.raises(hip.AosError):
        hip.Router(16, 9)
