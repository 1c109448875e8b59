"""CPU pinning of the oracle's router (no GPU): the reference's own known answers, closed forms,
invariants and brute force over tie orders.

Each known-answer case names the reference test it restates; the inputs and expected outputs are
also kept as data in tests/golden/router_kats.json (checked here and by the GPU router tests).
"""
from __future__ import annotations

import itertools
import json
import math
from decimal import Decimal, getcontext
from pathlib import Path

import numpy as np
import pytest

import oracle

GOLDEN = Path(__file__).resolve().parent / "golden"


def kats():
    return json.loads((GOLDEN / "router_kats.json").read_text())["cases"]


@pytest.mark.parametrize("case", kats(), ids=lambda c: c["name"])
def test_reference_router_kats(case):
    """crates/adapteros-lora-router/tests/determinism.rs:38-87, :537-574, :908-1090 and
    tests/q15_edge_cases.rs:74-135, :155-192 (indices; gates where the test fixes them)."""
    idx, q = oracle.route_one(np.array(case["priors"], np.float32), case["k"], case["tau"], case["eps"],
                              1.0, np.array(case["stable_ids"], np.uint64),
                              None if case.get("allowed") is None else np.array(case["allowed"], np.uint8))
    assert idx == case["expect_indices"]
    if case.get("expect_gates") is not None:
        assert q == case["expect_gates"]
    if case.get("min_gate") is not None:
        g = [v / 32767.0 for v in q]
        assert min(g) >= case["min_gate"]
        assert abs(sum(g) - 1.0) < 0.01


def test_quantize_gate_known_answers():
    """crates/adapteros-lora-router/src/quantization.rs:239-252."""
    assert oracle.quantize_gate(-0.5) == 0
    assert oracle.quantize_gate(1.5) == 32767
    assert oracle.quantize_gate(0.0) == 0
    assert oracle.quantize_gate(0.5) == 16384
    assert oracle.quantize_gate(1.0) == 32767


def test_quantize_gate_roundtrip():
    """quantization.rs:213-228: encode/decode within 1e-4."""
    for g in (0.0, 0.25, 0.5, 0.75, 1.0):
        assert abs(g - oracle.quantize_gate(g) / 32767.0) < 1e-4


def test_quantize_gate_half_away_from_zero():
    """roundf semantics: values whose product with 32767 lands exactly on .5 round up."""
    for q in (0, 1, 2, 100, 16383):
        g = np.float32((q + 0.5) / 32767.0)
        prod = float(np.float32(g) * np.float32(32767.0))
        expect = math.floor(prod + 0.5) if prod >= 0 else 0
        assert oracle.quantize_gate(float(g)) == min(expect, 32767)


def test_total_cmp_key_order():
    """f32::total_cmp: -NaN < -inf < -x < -0 < +0 < x < inf < NaN; the key sorts descending."""
    vals = [float("-inf"), -1.0, -1e-30, -0.0, 0.0, 1e-30, 1.0, float("inf")]
    keys = [oracle.lib().orc_total_cmp_key_desc(v) for v in vals]
    assert keys == sorted(keys, reverse=True)
    assert len(set(keys)) == len(keys)


def test_single_adapter_full_gate():
    """K = 1 (or a single candidate) carries the whole gate: 32767."""
    for n in (1, 3, 9):
        pri = np.linspace(-1, 1, n).astype(np.float32)
        idx, q = oracle.route_one(pri, 1, 1.0, 0.02)
        assert q == [32767]
        assert idx == [int(np.argmax(pri))]


def test_two_equal_scores_eps_zero():
    """Two equal scores, eps = 0: g = 0.5 each; 0.5 * 32767 = 16383.5 rounds to 16384."""
    idx, q = oracle.route_one(np.array([0.3, 0.3, -5.0], np.float32), 2, 1.0, 0.0)
    assert q == [16384, 16384]
    assert idx == [0, 1]


def _round_f32(v: Decimal) -> np.float32:
    """Round an exact decimal to the nearest float32 (ties to even), with no intermediate
    float64 rounding."""
    c = np.float32(float(v))
    best = None
    for cand in (np.nextafter(c, np.float32(-np.inf)), c, np.nextafter(c, np.float32(np.inf))):
        dist = abs(Decimal(float(cand)) - v)
        even = (int(cand.view(np.uint32)) & 1) == 0
        key = (dist, not even)
        if best is None or key < best[0]:
            best = (key, cand)
    return np.float32(best[1])


def _softmax_exact(scores, tau):
    getcontext().prec = 60
    m = max(scores)
    es = [(Decimal(float(s)) - Decimal(float(m))) / Decimal(float(tau)) for s in scores]
    es = [e.exp() for e in es]
    tot = sum(es)
    return [float(e / tot) for e in es]


def test_softmax_against_exact_arithmetic():
    """Gates of random K=2..8 decisions against the softmax in 60-digit decimal arithmetic, the
    floor and renormalisation applied afterwards: every Q15 gate within one step of the exact
    value (f32 rounding of the renormalisation can move a boundary case by one)."""
    rng = np.random.default_rng(7)
    for trial in range(300):
        k = int(rng.integers(2, 9))
        n = k + int(rng.integers(0, 6))
        tau = float(rng.choice([0.5, 1.0, 2.0]))
        eps = float(rng.choice([0.0, 0.02, 0.1]))
        pri = rng.normal(0, 1.5, n).astype(np.float32)
        idx, q = oracle.route_one(pri, k, tau, eps)
        top = sorted(range(n), key=lambda i: (-pri[i], i))[:k]
        g = _softmax_exact([pri[i] for i in top], tau)
        g = [max(v, eps / k) for v in g]
        s = sum(g)
        exact = {top[j]: g[j] / s * 32767 for j in range(k)}
        for a, qa in zip(idx, q):
            assert abs(qa - exact[a]) <= 1.0, (trial, a, qa, exact[a])


def test_q15_sum_invariant():
    """router/src/tests.rs:1402-1450: Q15 gates sum to 32767 within K."""
    rng = np.random.default_rng(11)
    for _ in range(500):
        k = int(rng.integers(1, 9))
        n = int(rng.integers(1, 40))
        pri = rng.normal(0, 2, n).astype(np.float32)
        _, q = oracle.route_one(pri, k, 1.0, 0.02)
        assert abs(sum(q) - 32767) <= len(q)


def test_canonical_order():
    """Output order: Q15 descending, then score descending, stable_id and index ascending."""
    rng = np.random.default_rng(5)
    for _ in range(300):
        n = int(rng.integers(2, 20))
        pri = rng.choice(np.float32([0.1, 0.2, 0.5, 0.5, 1.0]), n).astype(np.float32)
        sid = rng.integers(0, 4, n).astype(np.uint64)
        idx, q = oracle.route_one(pri, 8, 1.0, 0.02, 1.0, sid)
        keys = [(-q[j], -float(pri[idx[j]]), int(sid[idx[j]]), idx[j]) for j in range(len(idx))]
        assert keys == sorted(keys)


def test_tie_order_permutation_brute_force():
    """Exhaustive over every permutation of N <= 6 adapters with tied scores: the decision,
    mapped back through the permutation, never changes (ties resolve by stable_id, never by
    position unless stable_ids tie too)."""
    pri = np.array([0.5, 0.5, 0.25, 0.5, 0.25, 0.1], np.float32)
    sid = np.array([40, 10, 30, 20, 5, 60], np.uint64)
    base_idx, base_q = oracle.route_one(pri, 4, 1.0, 0.02, 1.0, sid)
    for perm in itertools.permutations(range(6)):
        p = list(perm)
        idx, q = oracle.route_one(pri[p], 4, 1.0, 0.02, 1.0, sid[p])
        assert [p[i] for i in idx] == base_idx
        assert q == base_q


def test_policy_mask_excludes():
    """Denied adapters never appear; all denied -> empty decision (policy_mask.rs)."""
    pri = np.array([3.0, 2.0, 1.0, 0.0], np.float32)
    idx, _ = oracle.route_one(pri, 2, 1.0, 0.02, 1.0, None, np.array([0, 1, 0, 1], np.uint8))
    assert sorted(idx) == [1, 3]
    idx, q = oracle.route_one(pri, 2, 1.0, 0.02, 1.0, None, np.zeros(4, np.uint8))
    assert idx == [] and q == []


def test_non_finite_prior_rejected():
    """validate_router_inputs (router.rs:611-625): any non-finite prior is an error, masked or not."""
    for bad in (float("nan"), float("inf"), float("-inf")):
        pri = np.array([0.1, bad, 0.3], np.float32)
        with pytest.raises(ValueError):
            oracle.route_one(pri, 2)
        with pytest.raises(ValueError):
            oracle.route_one(pri, 2, allowed=np.array([1, 0, 1], np.uint8))


def test_k_limits_and_sanitisers():
    """k > 8 fails (router.rs:769-777); k = 0 acts as 1; tau <= 0 / non-finite -> 1.0 and eps
    outside [0, 1] -> 0.02 (router.rs:146-187)."""
    pri = np.array([0.4, 0.1, 0.9, 0.2], np.float32)
    with pytest.raises(ValueError):
        oracle.route_one(pri, 9)
    assert oracle.route_one(pri, 0) == oracle.route_one(pri, 1)
    assert oracle.route_one(pri, 3, tau=0.0) == oracle.route_one(pri, 3, tau=1.0)
    assert oracle.route_one(pri, 3, tau=float("nan")) == oracle.route_one(pri, 3, tau=1.0)
    assert oracle.route_one(pri, 3, eps=2.0) == oracle.route_one(pri, 3, eps=0.02)
    assert oracle.route_one(pri, 3, eps=-1.0) == oracle.route_one(pri, 3, eps=0.02)


def test_negative_zero_prior_is_plus_zero():
    """(prior + 0.0) maps -0.0 to +0.0 (router.rs:1664-1676), so -0.0 and +0.0 tie and fall back
    to stable_id."""
    pri = np.array([-0.0, 0.0, -1.0], np.float32)
    idx, q = oracle.route_one(pri, 2, 1.0, 0.0, 1.0, np.array([7, 3, 1], np.uint64))
    assert idx == [1, 0]
    assert q == [16384, 16384]


def test_floor_invariant():
    """determinism.rs:218-267: gates are floored at eps / K before the renormalisation; the floor
    adds at most eps to the sum, so every final gate is >= (eps / K) / (1 + eps), and the floor
    binds (some raw softmax gate below eps / K) in a good share of these cases."""
    rng = np.random.default_rng(3)
    for _ in range(200):
        k = int(rng.integers(2, 9))
        eps = float(rng.choice([0.01, 0.05, 0.2]))
        pri = (rng.normal(0, 4, 24)).astype(np.float32)
        _, q = oracle.route_one(pri, k, 1.0, eps)
        assert min(q) / 32767.0 >= (eps / k) / (1.0 + eps) - 1.0 / 32767.0
    _, q = oracle.route_one(np.array([10.0, 0.0, -3.0], np.float32), 3, 1.0, 0.3)
    floor = np.float32(0.3) / np.float32(3)
    g0 = np.float32(1.0 / (1.0 + np.exp(-10.0) + np.exp(-13.0)))
    s = np.float32(np.float32(np.float32(0.0) + g0) + floor) + floor
    assert q[1:] == [oracle.quantize_gate(float(np.float32(floor / s)))] * 2
    assert q[0] == oracle.quantize_gate(float(np.float32(g0 / s)))


def test_batch_matches_single_and_fills_rings():
    """Ring fill rules (kernel-api/src/lib.rs:122-193, 1442-1520): top_k, position = token,
    unused slots zero; a failing token leaves a zero ring."""
    rng = np.random.default_rng(9)
    pri = rng.normal(0, 1, (6, 12)).astype(np.float32)
    pri[4, 3] = np.nan
    rings = oracle.route_batch(pri, 3, 1.0, 0.02)
    for t in range(6):
        if t == 4:
            assert rings[t]["top_k"] == 0 and not rings[t]["adapter_indices"].any()
            continue
        idx, q = oracle.route_one(pri[t], 3)
        assert rings[t]["top_k"] == 3 and rings[t]["current_pos"] == t
        assert list(rings[t]["adapter_indices"][:3]) == idx
        assert list(rings[t]["gates_q15"][:3]) == q
        assert not rings[t]["adapter_indices"][3:].any() and not rings[t]["gates_q15"][3:].any()


def test_priors_float64():
    """The router-logit GEMV against a float64 evaluation."""
    rng = np.random.default_rng(1)
    f = rng.normal(0, 1, (3, 896)).astype(np.float32)
    w = rng.normal(0, 0.05, (8, 896)).astype(np.float32)
    p = oracle.priors(f, w)
    ref = f.astype(np.float64) @ w.astype(np.float64).T
    assert np.max(np.abs(p - ref)) < 1e-4


def test_priors_fixed_order():
    """The documented summation order, evaluated step by step in float32 on a small case: 64
    partial sums, partial l over elements 256k + 4l + e with fused multiply-adds, then a xor
    butterfly."""
    getcontext().prec = 80
    rng = np.random.default_rng(2)
    d = 512
    f = rng.normal(0, 1, (1, d)).astype(np.float32)
    w = rng.normal(0, 1, (1, d)).astype(np.float32)
    part = []
    for l in range(64):
        acc = np.float32(0.0)
        for k in range(d // 256):
            for e in range(4):
                i = 256 * k + 4 * l + e
                # fmaf: exact product plus accumulator, rounded once to float32
                exact = Decimal(float(w[0, i])) * Decimal(float(f[0, i])) + Decimal(float(acc))
                acc = _round_f32(exact)
        part.append(acc)
    off = 32
    while off >= 1:
        part = [np.float32(part[l] + part[l ^ off]) for l in range(64)]
        off //= 2
    assert oracle.priors(f, w)[0, 0] == part[0]


def test_exp_pinning():
    """The device router uses a correctly rounded exp; the oracle uses the host libm. On sampled
    softmax arguments the correctly rounded value matches 60-digit decimal arithmetic, and
    routing with it substituted into the oracle gives the same decisions on the synthetic
    workloads."""
    import ctypes

    import aoship

    getcontext().prec = 60
    rng = np.random.default_rng(4)
    xs = np.concatenate([-np.abs(rng.normal(0, 4, 2000)), -rng.uniform(0, 700, 200), [0.0, -1e-300, -745.0]])
    for x in xs:
        exact = Decimal(float(x)).exp()
        got = aoship.exp_cr(float(x))
        if got == 0.0:
            assert exact < Decimal(2.0) ** -1074
            continue
        lo, hi = np.nextafter(got, -np.inf), np.nextafter(got, np.inf)
        assert abs(Decimal(got) - exact) <= abs(Decimal(float(lo)) - exact)
        assert abs(Decimal(got) - exact) <= abs(Decimal(float(hi)) - exact)

    import workloads as W

    fn = ctypes.cast(aoship.lib().aoship_internal_exp_cr, ctypes.c_void_p).value
    for cid in (1, 2, 5):
        cfg = W.CONFIGS[cid]
        pri = W.priors(cfg, 64) if cfg.routing != "features" else oracle.priors(*W.router_inputs(cfg, 64))
        sid = np.arange(cfg.n_adapters, dtype=np.uint64)
        a = oracle.route_batch(pri, cfg.k, cfg.tau, cfg.eps, 1.0, sid)
        oracle.set_exp(fn)
        try:
            b = oracle.route_batch(pri, cfg.k, cfg.tau, cfg.eps, 1.0, sid)
        finally:
            oracle.set_exp(None)
        assert a.tobytes() == b.tobytes()


# ---- the Decision's entropy and candidates (router.rs:1287-1293, 1844-1860; types.rs:669-687) ----

def _softmax_entropy64(scores, tau=1.0):
    """Entropy (bits) of softmax(scores / tau) in float64: the closed form the float32 result must
    approach when the entropy floor is inactive."""
    s = np.asarray(scores, np.float64) / tau
    e = np.exp(s - s.max())
    g = e / e.sum()
    return float(-(g * np.log2(g)).sum())


def test_entropy_uniform_is_log2_k():
    for k in (1, 2, 4, 8):
        idx, q, raw, h = oracle.route_one_detail(np.ones(k, np.float32), k)
        assert len(idx) == k
        assert h == np.float32(np.log2(k)), (k, h)  # g = 1/k exactly for these k
        assert np.array_equal(raw, np.ones(k, np.float32))


def test_entropy_three_equal_within_rounding_of_log2_3():
    idx, q, raw, h = oracle.route_one_detail(np.zeros(3, np.float32), 3, eps=0.0)
    assert abs(float(h) - np.log2(3.0)) < 4e-7


def test_entropy_single_candidate_is_zero():
    idx, q, raw, h = oracle.route_one_detail(np.array([3.0, -1.0, 0.5], np.float32), 1)
    assert idx == [0] and q == [32767] and float(h) == 0.0 and raw.tolist() == [3.0]


@pytest.mark.parametrize("d", [0.1, 0.7, 2.5, 6.0])
def test_entropy_two_gates_matches_binary_entropy(d):
    idx, q, raw, h = oracle.route_one_detail(np.array([d, 0.0, -50.0], np.float32), 2, eps=1e-6)
    assert idx == [0, 1]
    assert abs(float(h) - _softmax_entropy64([d, 0.0])) < 2e-6


def test_entropy_random_softmax_matches_float64():
    rng = np.random.default_rng(7)
    for _ in range(50):
        n = int(rng.integers(8, 40))
        p = rng.standard_normal(n).astype(np.float32)
        k = int(rng.integers(2, 9))
        tau = float(rng.choice([0.5, 1.0, 2.0]))
        idx, q, raw, h = oracle.route_one_detail(p, k, tau=tau, eps=1e-7)
        top = np.sort(p)[::-1][:k]
        assert abs(float(h) - _softmax_entropy64(top, tau)) < 4e-6 * max(1.0, float(h))


def test_entropy_reference_uniform_above_skewed():
    """abstain_edge_cases.rs:121-162: uniform priors give a higher entropy than skewed ones."""
    _, _, _, h1 = oracle.route_one_detail(np.array([0.33, 0.33, 0.34], np.float32), 3, eps=0.01)
    _, _, _, h2 = oracle.route_one_detail(np.array([2.0, 0.1, 0.1], np.float32), 3, eps=0.01)
    assert h1 > h2


def test_empty_decision_has_zero_entropy_and_no_candidates():
    """abstain_edge_cases.rs:164-186 (and :60-76): no adapter, or none allowed."""
    idx, q, raw, h = oracle.route_one_detail(np.zeros(0, np.float32), 3)
    assert idx == [] and float(h) == 0.0 and raw.size == 0
    idx, q, raw, h = oracle.route_one_detail(np.ones(4, np.float32), 3, allowed=np.zeros(4, np.uint8))
    assert idx == [] and float(h) == 0.0


def test_candidates_are_the_decision_with_raw_scores():
    """router.rs:1848-1860: the candidates carry the top-K raw scores (scope and bias applied) in
    the decision's order; the decision's indices and gates are the candidates'."""
    rng = np.random.default_rng(3)
    for _ in range(30):
        n = int(rng.integers(4, 30))
        p = rng.standard_normal(n).astype(np.float32)
        scope = (rng.random(n) < 0.7).astype(np.uint8)
        bias = float(rng.choice([1.0, 2.0, 0.5]))
        idx, q, raw, h = oracle.route_one_detail(p, 4, routing_bias=bias, scope=scope)
        i2, q2 = oracle.route_one_ex(p, 4, routing_bias=bias, scope=scope)
        assert (idx, q) == (i2, q2)
        want = np.where(scope[idx] != 0, p[idx], np.float32(-1.0e9)) * np.float32(bias)
        assert np.array_equal(raw, want.astype(np.float32))
