"""GPU: the Decision's entropy and candidates (aoship_router_set_decision_output) against the oracle
(oracle.route_one_detail): for every token the candidates' adapter indices, Q15 gates and raw scores
bit for bit, in decision order, and the entropy within float32 rounding (the device takes log2 in
double precision and rounds it to float; the oracle uses the C library's log2f, as the
reference's f32::log2 does). From priors and from router features, for adapter counts inside and
above one wavefront, with a scope hint and a routing bias, after a decision policy (the passing
candidates with their gates from before the renormalisation, the router's entropy), for tokens
without a decision (entropy 0, no candidates), and through aoship_route_mlp_forward."""
import numpy as np
import pytest

import oracle
import workloads as W
from cases import gpu_layer

pytestmark = pytest.mark.gpu

ENT_TOL = 2.0 ** -21  # relative: a few float32 ulps


def _route(hip, router, priors, T):
    import torch

    dec = torch.zeros(T * hip.DECISION_DTYPE.itemsize, dtype=torch.uint8, device="cuda")
    rings = torch.zeros(T * 40, dtype=torch.uint8, device="cuda")
    status = torch.full((T,), 7, dtype=torch.int32, device="cuda")
    router.set_decision_output(dec)
    router.route(torch.from_numpy(priors).cuda(), rings, status)
    torch.cuda.synchronize()
    router.set_decision_output(None)
    return dec.cpu().numpy().view(hip.DECISION_DTYPE), status.cpu().numpy()


def _check(d, idx, q, raw, h, what):
    n = len(idx)
    assert int(d["n_candidates"]) == n, what
    assert d["adapter_idx"][:n].tolist() == list(idx), what
    assert d["gate_q15"][:n].tolist() == list(q), what
    assert np.array_equal(d["raw_score"][:n].view(np.uint32), np.asarray(raw, np.float32).view(np.uint32)), what
    assert not d["adapter_idx"][n:].any() and not d["gate_q15"][n:].any() and not d["raw_score"][n:].any(), what
    e = float(d["entropy"])
    assert abs(e - float(h)) <= ENT_TOL * max(abs(float(h)), 1e-30), (what, e, float(h))


@pytest.mark.parametrize("n,k", [(16, 4), (64, 8), (150, 4), (5, 1)])
def test_decision_from_priors(hip, n, k):
    rng = np.random.default_rng(100 + n)
    T = 96
    p = rng.standard_normal((T, n)).astype(np.float32)
    p[3] = 0.25  # all equal: ties, uniform gates
    tau, eps = 1.5, 0.02
    router = hip.Router(n, k, tau, eps, 1.0, np.arange(n, dtype=np.uint64))
    dec, status = _route(hip, router, p, T)
    assert (status == 0).all()
    for t in range(T):
        idx, q, raw, h = oracle.route_one_detail(p[t], k, tau=tau, eps=eps, stable_ids=np.arange(n, dtype=np.uint64))
        _check(dec[t], idx, q, raw, h, f"token {t}")


def test_decision_with_scope_and_bias(hip):
    rng = np.random.default_rng(5)
    T, n, k = 64, 40, 4
    p = rng.standard_normal((T, n)).astype(np.float32)
    scope = (rng.random(n) < 0.5).astype(np.uint8)
    router = hip.Router(n, k, 1.0, 0.02, 2.0, np.arange(n, dtype=np.uint64))
    router.set_scope(scope)
    dec, status = _route(hip, router, p, T)
    for t in range(T):
        idx, q, raw, h = oracle.route_one_detail(p[t], k, routing_bias=2.0, scope=scope,
                                                 stable_ids=np.arange(n, dtype=np.uint64))
        _check(dec[t], idx, q, raw, h, f"token {t}")


def test_decision_after_policy(hip):
    """filter_decision_by_policy: the passing candidates in order (capped), gates as decided
    before the renormalisation of the ring's gates, entropy unchanged; none passing -> empty."""
    rng = np.random.default_rng(9)
    T, n, k = 64, 24, 6
    p = rng.standard_normal((T, n)).astype(np.float32)
    allowed = (rng.random(n) < 0.5).astype(np.uint8)
    router = hip.Router(n, k, 1.0, 0.02, 1.0, np.arange(n, dtype=np.uint64))
    router.set_decision_policy(allowed, 3)
    dec, status = _route(hip, router, p, T)
    for t in range(T):
        idx, q, raw, h = oracle.route_one_detail(p[t], k, stable_ids=np.arange(n, dtype=np.uint64))
        keep = [j for j in range(len(idx)) if allowed[idx[j]]][:3]
        if not keep:
            assert status[t] == -2
            _check(dec[t], [], [], [], 0.0, f"token {t} (denied)")
            continue
        _check(dec[t], [idx[j] for j in keep], [q[j] for j in keep], raw[keep], h, f"token {t}")


def test_tokens_without_a_decision(hip):
    n, k, T = 8, 3, 4
    p = np.zeros((T, n), np.float32)
    p[1, 2] = np.nan
    router = hip.Router(n, k, 1.0, 0.02, 1.0, np.arange(n, dtype=np.uint64))
    router.set_policy_mask(np.array([1, 1, 1, 1, 1, 1, 1, 1], np.uint8))
    dec, status = _route(hip, router, p, T)
    assert status[1] == -1
    _check(dec[1], [], [], [], 0.0, "non-finite prior")
    router.set_policy_mask(np.zeros(n, np.uint8))
    dec, status = _route(hip, router, p[:1], 1)
    _check(dec[0], [], [], [], 0.0, "nothing allowed")


def test_decision_from_features_and_route_mlp(hip):
    import torch

    cid = 2
    cfg = W.CONFIGS[cid]
    T = 8
    f, w = W.router_inputs(cfg, T)
    pri = oracle.priors(f, w)
    sid = np.arange(cfg.n_adapters, dtype=np.uint64)
    router = hip.Router(cfg.n_adapters, cfg.k, cfg.tau, cfg.eps, 1.0, sid)
    fd, wd = torch.from_numpy(f).cuda(), torch.from_numpy(w).cuda()
    dec = torch.zeros(T * hip.DECISION_DTYPE.itemsize, dtype=torch.uint8, device="cuda")
    router.set_decision_output(dec)
    rings = torch.zeros(T * 40, dtype=torch.uint8, device="cuda")
    router.route_features(fd, wd, rings)
    torch.cuda.synchronize()
    d1 = dec.cpu().numpy().view(hip.DECISION_DTYPE).copy()
    for t in range(T):
        idx, q, raw, h = oracle.route_one_detail(pri[t], cfg.k, tau=cfg.tau, eps=cfg.eps, stable_ids=sid)
        _check(d1[t], idx, q, raw, h, f"features token {t}")
    layer, _ = gpu_layer(hip, cid)
    xb, _ = W.activations(cfg, T)
    x = torch.from_numpy(xb.view(np.int16)).cuda()
    y = torch.empty_like(x)
    dec.zero_()
    layer.route_mlp_forward(router, fd, wd, x, rings, y)
    torch.cuda.synchronize()
    router.set_decision_output(None)
    assert dec.cpu().numpy().view(hip.DECISION_DTYPE).tobytes() == d1.tobytes()
