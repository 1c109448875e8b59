"""GPU parity of the router extras: the device rings and statuses equal the oracle's
(oracle.route_batch_ex) bit for bit with a scope hint, adaptive tie-breakers, a decision policy
(filter + Q15 renormalisation, cap, PolicyViolation) and the ring mapping (active ids,
strengths), alone and together, for adapter counts inside and above one wavefront, from priors
and from router features."""
import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu


def _tied_priors(rng, T, n):
    """Priors with many exact ties (a few levels) and some distinct values."""
    levels = rng.standard_normal(4).astype(np.float32)
    p = levels[rng.integers(0, 4, (T, n))]
    mix = rng.random((T, n)) < 0.3
    p[mix] = rng.standard_normal(int(mix.sum())).astype(np.float32)
    return p


def _extras(rng, n, which):
    e = {}
    if "scope" in which:
        e["scope"] = (rng.random(n) < 0.6).astype(np.uint8)
        e["scope"][0] = 1
    if "adaptive" in which:
        e["seed"] = rng.integers(0, 256, 32, dtype=np.uint8).tobytes()
    if "policy" in which:
        e["post_allowed"] = (rng.random(n) < 0.5).astype(np.uint8)
        e["post_max"] = int(rng.integers(-1, 5))
    if "mapping" in which:
        e["active_ids"] = rng.permutation(np.arange(1, n + 1, dtype=np.uint16) * 3)
        e["active_ids"][rng.integers(0, n)] = 65535 if n > 8 else e["active_ids"][0]
        s = rng.random(n).astype(np.float32) * 1.4 - 0.2
        s[rng.integers(0, n)] = np.nan
        e["strengths"] = s
    return e


def _run(hip, priors, k, sid, allowed, e, features=None, router_w=None, hashing=None):
    import torch

    T, n = priors.shape
    r = hip.Router(n, k, 1.0, 0.02, 1.0, sid)
    hashes = None
    if hashing is not None:
        hashes = torch.full((T * 96,), 0x5A, dtype=torch.uint8, device="cuda")
        r.set_decision_hashing(hashes, *hashing)
    r.set_policy_mask(allowed)
    r.set_scope(e.get("scope"))
    r.set_adaptive_seed(e.get("seed"))
    r.set_decision_policy(e.get("post_allowed"), e.get("post_max"))
    r.set_ring_mapping(e.get("active_ids"), e.get("strengths"))
    rings = torch.zeros(T * 40, dtype=torch.uint8, device="cuda")
    status = torch.full((T,), 7, dtype=torch.int32, device="cuda")
    if features is None:
        r.route(torch.from_numpy(priors).cuda(), rings, status)
    else:
        pout = torch.zeros((T, n), dtype=torch.float32, device="cuda")
        r.route_features(torch.from_numpy(features).cuda(), torch.from_numpy(router_w).cuda(), rings, pout, status)
    torch.cuda.synchronize()
    g_rings, g_status = hip.rings_from_bytes(rings.cpu().numpy()), status.cpu().numpy()
    br = None if "seed" not in e else oracle.tie_breakers(e["seed"], n)
    pm = e.get("post_max")
    o_rings, o_status = oracle.route_batch_ex(priors, k, 1.0, 0.02, 1.0, sid, allowed, e.get("scope"), br,
                                              e.get("post_allowed"), -1 if pm is None else pm,
                                              e.get("active_ids"), e.get("strengths"))
    if hashing is not None:
        return g_rings, g_status, o_rings, o_status, hashes.cpu().numpy().tobytes()
    return g_rings, g_status, o_rings, o_status


def _oracle_hashes(priors, k, sid, allowed, e, reasoning, backend):
    """Router::compute_decision_hash of each token's router decision (before the decision
    policy); 96 zero bytes where there is none."""
    n = priors.shape[1]
    br = None if "seed" not in e else oracle.tie_breakers(e["seed"], n)
    sc = e.get("scope")
    out = []
    for t in range(priors.shape[0]):
        try:
            idx, q = oracle.route_one_ex(priors[t], k, 1.0, 0.02, 1.0, sid, allowed, sc, br)
        except ValueError:
            idx = []
        if not idx:
            out.append(bytes(96))
            continue
        pr = priors[t].copy()
        if sc is not None:
            pr[np.asarray(sc) == 0] = np.float32(-1e9)
        out.append(oracle.decision_hash(pr, idx, q, reasoning, backend))
    return b"".join(out)


HASH_OPTS = [(None, None), (bytes(range(32)), None), (None, bytes(range(7, 39))), (bytes(32), bytes([255] * 32))]


@pytest.mark.parametrize("opts", range(len(HASH_OPTS)))
@pytest.mark.parametrize("n,T", [(5, 64), (64, 64), (300, 64), (4096, 12)])
def test_decision_hashes_bit_exact(hip, n, T, opts):
    """Device BLAKE3 decision hashes (one to seventeen chunks of priors) equal the oracle's, with
    scope, adaptive ties and a decision policy on; tokens with a non-finite prior or an empty
    decision get zeros."""
    rng = np.random.default_rng(n + 7 * opts)
    priors = _tied_priors(rng, T, n)
    priors[3, n // 2] = np.inf
    sid = rng.integers(0, 3, n).astype(np.uint64)
    allowed = (rng.random(n) < 0.9).astype(np.uint8)
    k = int(rng.integers(1, 9))
    e = _extras(rng, n, ("scope", "adaptive", "policy"))
    reasoning, backend = HASH_OPTS[opts]
    g_rings, g_status, o_rings, o_status, h = _run(hip, priors, k, sid, allowed, e, hashing=(reasoning, backend))
    _check(g_rings, g_status, o_rings, o_status)
    want = _oracle_hashes(priors, k, sid, allowed, e, reasoning, backend)
    for t in range(T):
        assert h[96 * t:96 * t + 96] == want[96 * t:96 * t + 96], f"token {t}"
    assert h[3 * 96:4 * 96] == bytes(96)


def test_decision_hashes_from_features_and_empty(hip):
    rng = np.random.default_rng(5)
    T, n, d = 32, 96, 128
    features = rng.standard_normal((T, d)).astype(np.float32)
    router_w = rng.standard_normal((n, d)).astype(np.float32)
    priors = oracle.priors(features, router_w)
    sid = np.arange(n, dtype=np.uint64)
    g_rings, g_status, o_rings, o_status, h = _run(hip, priors, 4, sid, None, {}, features, router_w,
                                                   hashing=(None, None))
    _check(g_rings, g_status, o_rings, o_status)
    assert h == _oracle_hashes(priors, 4, sid, None, {}, None, None)
    # every adapter masked: empty decisions, zero hashes
    none = np.zeros(n, np.uint8)
    _, _, _, _, h = _run(hip, priors, 4, sid, none, {}, hashing=(None, None))
    assert h == bytes(96 * T)


def _check(g_rings, g_status, o_rings, o_status):
    assert (g_status == o_status).all(), np.nonzero(g_status != o_status)[0][:5]
    for t in range(len(g_rings)):
        assert g_rings[t].tobytes() == o_rings[t].tobytes(), f"token {t}: gpu {g_rings[t]} oracle {o_rings[t]}"


WHICH = [("scope",), ("adaptive",), ("policy",), ("mapping",), ("scope", "adaptive", "policy", "mapping")]


@pytest.mark.parametrize("which", WHICH, ids=lambda w: "+".join(w))
@pytest.mark.parametrize("n", [5, 64, 200, 1000])
def test_router_extras_bit_exact(hip, n, which):
    rng = np.random.default_rng(1000 * n + len(which))
    T = 257
    priors = _tied_priors(rng, T, n)
    sid = rng.integers(0, 3, n).astype(np.uint64)  # stable_id collisions as well
    allowed = (rng.random(n) < 0.9).astype(np.uint8)
    k = int(rng.integers(1, 9))
    e = _extras(rng, n, which)
    g_rings, g_status, o_rings, o_status = _run(hip, priors, k, sid, allowed, e)
    _check(g_rings, g_status, o_rings, o_status)
    if "adaptive" in which and n >= 64:
        # on exact ties the seed decides: equal priors select other adapters than deterministic mode
        flat = np.full((4, n), 0.5, np.float32)
        ga, sa, oa, osa = _run(hip, flat, k, sid, allowed, e)
        _check(ga, sa, oa, osa)
        gd, _, _, _ = _run(hip, flat, k, sid, allowed, {})
        assert ga[0].tobytes() != gd[0].tobytes()


def test_router_extras_from_features(hip):
    """The same epilogue in the features -> priors kernel."""
    rng = np.random.default_rng(77)
    T, n, d = 64, 96, 256
    features = rng.standard_normal((T, d)).astype(np.float32)
    router_w = (rng.integers(-2, 3, (n, d)) * 0.25).astype(np.float32)  # coarse weights: ties
    priors = oracle.priors(features, router_w)
    e = _extras(rng, n, ("scope", "adaptive", "policy", "mapping"))
    sid = np.arange(n, dtype=np.uint64)[::-1].copy()
    g_rings, g_status, o_rings, o_status = _run(hip, priors, 6, sid, None, e, features, router_w)
    _check(g_rings, g_status, o_rings, o_status)


def test_policy_violation_and_reference_cases_on_device(hip):
    """worker_enforcement_tests.rs:127-215 through the device: denying one of two adapters leaves
    the other with gate 32767; denying every adapter reports status -2 with a zero ring."""
    pri = np.array([[0.9, 0.2], [0.1, 0.8]], np.float32)
    e = {"post_allowed": np.array([1, 0], np.uint8), "post_max": 2}
    g, s, o, os_ = _run(hip, pri, 2, np.zeros(2, np.uint64), None, e)
    _check(g, s, o, os_)
    assert (s == 0).all()
    assert [int(g[t]["top_k"]) for t in range(2)] == [1, 1]
    assert [int(g[t]["adapter_indices"][0]) for t in range(2)] == [0, 0]
    assert [int(g[t]["gates_q15"][0]) for t in range(2)] == [32767, 32767]
    e = {"post_allowed": np.array([0, 0], np.uint8)}
    g, s, o, os_ = _run(hip, pri, 2, np.zeros(2, np.uint64), None, e)
    _check(g, s, o, os_)
    assert (s == -2).all() and not g.tobytes().strip(b"\0")
