"""GPU router parity: rings from the HIP router must equal the CPU oracle's bit for bit.

Covers the reference's router known answers (crates/adapteros-lora-router/tests/determinism.rs,
q15_edge_cases.rs), every workload's routing at full token counts (features -> priors on the
device for configs 1, 2, 4; prototype priors for 3; adversarial ties / signed zeros / Q15
boundaries / dominance with eps = 0 for 5), N above one wavefront, policy masks and the
non-finite error path.
"""
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


KATS = [
    # determinism.rs:38-87 -> [1, 2, 0]
    dict(priors=[0.5, 0.5, 0.5, 0.3, 0.2], ids=[300, 100, 200, 400, 500], k=3, eps=0.01, idx=[1, 2, 0]),
    # determinism.rs:537-574 -> [0, 2, 1]
    dict(priors=[0.9, 0.5, 0.5, 0.5, 0.1], ids=[10, 200, 100, 300, 400], k=3, eps=0.01, idx=[0, 2, 1]),
    # determinism.rs:908-1090: equal priors -> 0..K
    dict(priors=[0.25] * 8, ids=None, k=4, eps=0.02, idx=[0, 1, 2, 3]),
    # q15_edge_cases.rs:155-192: single adapter -> 32767
    dict(priors=[1.0], ids=None, k=1, eps=0.02, idx=[0], q=[32767]),
]


@pytest.mark.parametrize("kat", KATS)
def test_router_reference_kats(hip, kat):
    pri = np.array([kat["priors"]], np.float32)
    ids = None if kat["ids"] is None else np.array(kat["ids"], np.uint64)
    g, st = _gpu_route(hip, pri, kat["k"], 1.0, kat["eps"], 1.0, ids)
    o = _oracle_rings(pri, kat["k"], 1.0, kat["eps"], 1.0, ids)
    assert st[0] == 0
    _assert_rings_equal(g, o)
    kk = int(g[0]["top_k"])
    assert list(g[0]["adapter_indices"][:kk]) == kat["idx"]
    if "q" in kat:
        assert list(g[0]["gates_q15"][:kk]) == kat["q"]


def test_router_masked_single(hip):
    # q15_edge_cases.rs:74-135: the other adapter denied by policy -> one adapter, gate 32767
    pri = np.array([[1.0, 1.0]], np.float32)
    g, _ = _gpu_route(hip, pri, 2, allowed=np.array([1, 0], np.uint8))
    assert int(g[0]["top_k"]) == 1 and g[0]["adapter_indices"][0] == 0 and g[0]["gates_q15"][0] == 32767


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
