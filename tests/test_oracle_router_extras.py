"""CPU pinning of the router extras (no GPU): scope hint, adaptive tie-breakers, the decision
policy filter with Q15 renormalisation, and the decision -> ring conversion with active ids and
strengths. Known answers restate the reference's own tests (each names its source); the ChaCha20
block function is pinned by the RFC 8439 test vectors; renormalisation by exact rational
arithmetic; adaptive selection by brute force over tie orders. The library's host-side
tie-breakers (aoship_adaptive_tie_breakers) are checked against the oracle here too. BLAKE3 and
the decision hash are pinned by the published BLAKE3 vectors (tests/golden/blake3_vectors.json),
hashes the reference holds, and byte layouts built here with struct."""
from __future__ import annotations

import hashlib
import hmac
import json
import struct
from fractions import Fraction
from pathlib import Path

import numpy as np
import pytest

import aoship
import oracle

SIGMA = [0x61707865, 0x3320646E, 0x79622D32, 0x6B206574]


def _words(b: bytes) -> list[int]:
    return list(struct.unpack(f"<{len(b) // 4}I", b))


def _bytes(words) -> bytes:
    return struct.pack(f"<{len(words)}I", *words)


# ---- ChaCha20 and the tie-breakers ---------------------------------------------------------------

CHACHA_VECTORS = [
    # (key, block counter, nonce (12 bytes), serialised block) -- RFC 8439 section 2.3.2 and A.1
    (bytes(range(32)), 1, bytes.fromhex("000000090000004a00000000"),
     "10f1e7e4d13b5915500fdd1fa32071c4c7d1f4c733c068030422aa9ac3d46c4e"
     "d2826446079faa0914c2d705d98b02a2b5129cd1de164eb9cbd083e8a2503c4e"),
    (bytes(32), 0, bytes(12),
     "76b8e0ada0f13d90405d6ae55386bd28bdd219b8a08ded1aa836efcc8b770dc7"
     "da41597c5157488d7724e03fb8d84a376a43b8f41518a11cc387b669b2ee6586"),
    (bytes(32), 1, bytes(12),
     "9f07e7be5551387a98ba977c732d080dcb0f29a048e3656912c6533e32ee7aed"
     "29b721769ce64e43d57133b074d839d531ed1f28510afb45ace10a1f4b794d6f"),
    (bytes(31) + b"\x01", 1, bytes(12),
     "3aeb5224ecf849929b9d828db1ced4dd832025e8018b8160b82284f3c949aa5a"
     "8eca00bbb4a73bdad192b5c42f73f2fd4e273644c8b36125a64addeb006c13a0"),
]


@pytest.mark.parametrize("key,counter,nonce,expect", CHACHA_VECTORS)
def test_chacha20_block_rfc8439(key, counter, nonce, expect):
    state = SIGMA + _words(key) + [counter] + _words(nonce)
    assert _bytes(oracle.chacha20_block(state)).hex() == expect


def test_tie_breakers_are_the_keystream_in_u64_steps():
    """rand_chacha's state (64-bit counter in words 12-13, stream 0) with the zero seed is RFC 8439
    A.1 vectors 1 and 2; gen::<u64>() joins words low first."""
    b = oracle.tie_breakers(bytes(32), 16)
    ks = bytes.fromhex(CHACHA_VECTORS[1][3] + CHACHA_VECTORS[2][3])
    assert b.tolist() == list(struct.unpack("<16Q", ks))
    assert int(b[0]) == 0x903DF1A0ADE0B876 and int(b[8]) == 0x7A385155BEE7079F
    # key bytes reach the key words little-endian (RFC A.1 vector 3 is block 1 of that key)
    b3 = oracle.tie_breakers(bytes(31) + b"\x01", 16)
    assert bytes(b3[8:].view(np.uint8)).hex() == CHACHA_VECTORS[3][3]


@pytest.mark.parametrize("n", [0, 1, 7, 8, 9, 63, 4096])
def test_library_tie_breakers_match_oracle(n):
    rng = np.random.default_rng(n)
    seed = rng.integers(0, 256, 32, dtype=np.uint8).tobytes()
    assert (aoship.adaptive_tie_breakers(seed, n) == oracle.tie_breakers(seed, n)).all()


def _hkdf_sha256(ikm: bytes, info: bytes, length: int = 32) -> bytes:
    prk = hmac.new(b"\x00" * 32, ikm, hashlib.sha256).digest()  # salt None = HashLen zeros
    okm, t, i = b"", b"", 1
    while len(okm) < length:
        t = hmac.new(prk, t + info + bytes([i]), hashlib.sha256).digest()
        okm += t
        i += 1
    return okm[:length]


def tiebreak_seed(request_seed: bytes) -> bytes:
    """DeterminismContext::router_tiebreak_seed for a request seed without manifest hash:
    derive_router_seed = hex(HKDF(request seed, "router")) (determinism.rs:142-150), then
    HKDF(from_hex(that), "router-tie") (determinism.rs:172-176, seed.rs:986-1006)."""
    return _hkdf_sha256(_hkdf_sha256(request_seed, b"router"), b"router-tie")


def test_adaptive_seeded_order_for_exact_ties():
    """tests.rs:856-925: 8 adapters with equal priors, stable_id i+1, K=3; request seeds [1;32]
    and [2;32] select the first three of (breaker, stable_id) order, and the two sets differ."""
    n, k = 8, 3
    sid = np.arange(1, n + 1, dtype=np.uint64)
    sel = []
    for s in (bytes([1] * 32), bytes([2] * 32)):
        br = oracle.tie_breakers(tiebreak_seed(s), n)
        order = sorted(range(n), key=lambda i: (int(br[i]), int(sid[i])))
        idx, q = oracle.route_one_ex(np.full(n, 0.5, np.float32), k, stable_ids=sid, breakers=br)
        assert sorted(idx) == sorted(order[:k])
        # canonical re-sort keeps stable_id: equal gates come out in stable_id order
        assert q == [10922, 10922, 10922] and idx == sorted(idx, key=lambda i: int(sid[i]))
        sel.append(sorted(idx))
    assert sel[0] != sel[1]


def test_adaptive_changes_nothing_without_ties():
    rng = np.random.default_rng(5)
    for _ in range(50):
        n = int(rng.integers(2, 40))
        p = rng.permutation(n).astype(np.float32) / n  # distinct scores
        br = oracle.tie_breakers(rng.integers(0, 256, 32, dtype=np.uint8).tobytes(), n)
        assert oracle.route_one_ex(p, 4, breakers=br) == oracle.route_one(p, 4)


def test_adaptive_brute_force_tie_orders():
    """Every tie pattern over 6 adapters with 3 score levels, breakers with collisions: the
    selection is the first K of (score desc, breaker, stable_id, index)."""
    rng = np.random.default_rng(9)
    levels = np.array([0.2, 0.5, 0.9], np.float32)
    for code in range(3 ** 6):
        lv = [(code // 3 ** i) % 3 for i in range(6)]
        p = levels[lv]
        br = rng.integers(0, 3, 6).astype(np.uint64)  # frequent breaker collisions
        sid = rng.integers(0, 2, 6).astype(np.uint64)  # and stable_id collisions
        k = int(rng.integers(1, 7))
        order = sorted(range(6), key=lambda i: (-float(p[i]), int(br[i]), int(sid[i]), i))
        idx, _ = oracle.route_one_ex(p, k, stable_ids=sid, breakers=br)
        assert sorted(idx) == sorted(order[:k]), (lv, br.tolist(), sid.tolist(), k)


# ---- scope hint --------------------------------------------------------------------------------------


def test_scope_hint_replaces_out_of_scope_priors():
    """router.rs:1587-1602: adapters outside the scope route as if their prior were -1e9."""
    p = np.array([0.9, 0.1, 0.5, 0.3], np.float32)
    assert oracle.route_one_ex(p, 1, scope=[0, 1, 1, 1])[0] == [2]
    idx, q = oracle.route_one_ex(p, 4, scope=[0, 1, 1, 1])
    assert idx[-1] == 0
    # adapter 0's exp underflows to 0, so its gate is the entropy floor eps / K renormalised
    floor = np.float32(0.02) / np.float32(4)
    assert q[-1] <= oracle.quantize_gate(floor) and q[-1] >= oracle.quantize_gate(floor) - 1
    # a non-finite prior is an error even outside the scope (validation precedes the hint)
    with pytest.raises(ValueError):
        oracle.route_one_ex(np.array([np.nan, 0.1], np.float32), 1, scope=[0, 1])


# ---- renormalize_gates_q15 ------------------------------------------------------------------------------


def _q(g: float) -> int:
    return oracle.quantize_gate(g)


def test_renormalize_reference_cases():
    """policy_mask.rs:501-563."""
    assert oracle.renormalize_q15([16384]) == [32767]
    r = oracle.renormalize_q15([_q(0.5), _q(0.5)])
    assert abs(sum(r) / 32767 - 1.0) < 0.001
    r = oracle.renormalize_q15([_q(0.6), _q(0.3)])
    assert abs(sum(r) / 32767 - 1.0) < 0.001 and abs(r[0] / r[1] - 2.0) < 0.05
    assert oracle.renormalize_q15([]) == []
    r = oracle.renormalize_q15([0, 0, 0])
    assert r[0] == r[1] == r[2] == _q(np.float32(1.0) / np.float32(3.0)) and abs(sum(r) / 32767 - 1) < 0.01
    g = [_q(0.4), _q(0.35), _q(0.15)]
    assert oracle.renormalize_q15(g) == oracle.renormalize_q15(g)


def _round_half_away(x: Fraction) -> int:
    f = x.numerator // x.denominator
    return f + 1 if x - f >= Fraction(1, 2) else f


def test_renormalize_exact_rationals():
    """q_i' = round(32767 q_i / sum q) exactly, away from rounding ties."""
    rng = np.random.default_rng(1)
    checked = 0
    for _ in range(2000):
        n = int(rng.integers(2, 9))
        q = rng.integers(0, 32768, n).tolist()
        if sum(q) == 0:
            continue
        got = oracle.renormalize_q15(q)
        for qi, gi in zip(q, got):
            exact = Fraction(32767 * qi, sum(q))
            frac = exact - (exact.numerator // exact.denominator)
            if abs(frac - Fraction(1, 2)) < Fraction(1, 1000):
                continue
            assert gi == min(_round_half_away(exact), 32767)
            checked += 1
    assert checked > 5000


# ---- filter_decision_by_policy ---------------------------------------------------------------------------


def test_filter_reference_cases():
    # policy_mask.rs:565-590: deny "c" of a, b, c -> two entries that sum to 1
    i, g = oracle.filter_decision([0, 1, 2], [_q(0.5), _q(0.3), _q(0.2)], [1, 1, 0])
    assert i == [0, 1] and abs(sum(g) / 32767 - 1) < 0.001
    assert g == [_round_half_away(Fraction(32767 * _q(0.5), _q(0.5) + _q(0.3))),
                 _round_half_away(Fraction(32767 * _q(0.3), _q(0.5) + _q(0.3)))]
    # policy_mask.rs:611-635: a policy that removes nothing keeps the gates bit for bit
    assert oracle.filter_decision([0, 1], [_q(0.7), _q(0.3)], [1, 1]) == ([0, 1], [_q(0.7), _q(0.3)])
    # worker_enforcement_tests.rs:127-172: deny adapter_b, max 2 -> [0] alone, gate 1.0
    assert oracle.filter_decision([0, 1], [20000, 12000], [1, 0], 2) == ([0], [32767])
    # worker_enforcement_tests.rs:174-215: all denied -> PolicyViolation
    with pytest.raises(PermissionError):
        oracle.filter_decision([0], [16000], [0])


def test_filter_cap_order_and_errors():
    # a cap that truncates counts as a removal: renormalised, decision order kept
    i, g = oracle.filter_decision([3, 1, 2], [16000, 10000, 6767], [1, 1, 1, 1], 2)
    assert i == [3, 1] and g == oracle.renormalize_q15([16000, 10000])
    # removal from the middle keeps order (no re-sort, even where gates now rise)
    i, g = oracle.filter_decision([0, 1, 2], [12000, 11000, 9767], [1, 0, 1])
    assert i == [0, 2]
    with pytest.raises(PermissionError):
        oracle.filter_decision([0, 1], [20000, 12767], [1, 1], 0)  # max_adapters_per_token = 0
    # a cap at least the length removes nothing
    assert oracle.filter_decision([0, 1], [20000, 12767], [1, 1], 5) == ([0, 1], [20000, 12767])


# ---- decision -> ring ----------------------------------------------------------------------------------------


def _ring(r):
    k = int(r["top_k"])
    return r["adapter_indices"][:k].tolist(), r["gates_q15"][:k].tolist(), int(r["current_pos"])


def test_ring_reference_cases():
    # router_bridge.rs:337-346: active ids map, position kept
    assert _ring(oracle.decision_to_ring([0, 1], [111, 222], active_ids=[42, 99], position=7)) == ([42, 99], [111, 222], 7)
    # :348-355: an index outside the active set is AosError::Routing
    with pytest.raises(LookupError):
        oracle.decision_to_ring([0, 1], [100, 200], active_ids=[7])
    # :328-335: the full signed Q15 range passes through
    assert _ring(oracle.decision_to_ring([0, 1, 2, 3], [-32767, -16383, 16383, 32767]))[1] == [-32767, -16383, 16383, 32767]


def test_ring_strengths_closed_forms():
    s = [1.0, 0.0, 0.5, float("nan"), 2.0, -1.0, 0.5, 1e-9]
    q = [20000, 20000, 3, 20000, 20000, 20000, 5, 32767]
    r = oracle.decision_to_ring(list(range(8)), q, strengths=s, n_active=8)
    # round half away from zero; NaN -> 0; clamp to [0, 1]
    assert _ring(r)[1] == [20000, 0, 2, 0, 20000, 0, 3, 0]
    # an active id of 65535 zero-fills the ring (set_with_max_adapter with u16::MAX)
    r = oracle.decision_to_ring([0, 1], [20000, 12767], active_ids=[5, 65535], position=3)
    assert int(r["top_k"]) == 0 and int(r["current_pos"]) == 3
    assert not r["adapter_indices"].any() and not r["gates_q15"].any()


# ---- BLAKE3 and the decision hash -----------------------------------------------------------------------
B3 = json.loads((Path(__file__).resolve().parent / "golden" / "blake3_vectors.json").read_text())


@pytest.mark.parametrize("case", B3["pattern"], ids=lambda c: str(c["len"]))
def test_blake3_published_vectors(case):
    """Oracle and library (host) BLAKE3 against the published vectors: one chunk, chunk
    boundaries, and trees up to 100 chunks."""
    data = bytes(i % 251 for i in range(case["len"]))
    assert oracle.blake3(data).hex() == case["hash"]
    assert aoship.blake3(data).hex() == case["hash"]


@pytest.mark.parametrize("case", B3["text"], ids=lambda c: c["input"] or "empty")
def test_blake3_reference_held_hashes(case):
    assert oracle.blake3(case["input"].encode()).hex() == case["hash"]
    assert aoship.blake3(case["input"].encode()).hex() == case["hash"]


def test_blake3_library_matches_oracle_random_lengths():
    rng = np.random.default_rng(3)
    for n in list(rng.integers(0, 40000, 60)) + [64, 128, 960, 17 * 1024]:
        data = rng.integers(0, 256, int(n), dtype=np.uint8).tobytes()
        assert aoship.blake3(data) == oracle.blake3(data), n


def test_decision_hash_layout():
    """compute_decision_hash (router.rs:1427-1484), features empty: input = priors f32 LE
    [+ reasoning], output = indices u16 LE then gates i16 LE [+ reasoning], combined = input ||
    output [|| reasoning] [|| backend]; the bytes built here with struct."""
    pri = [0.1, -0.0, 3.5, -1e9]
    idx, q = [2, 0, 1], [20000, 7000, 5767]
    r, b = bytes(range(32)), bytes(range(100, 132))
    for reasoning, backend in [(None, None), (r, None), (None, b), (r, b)]:
        got = oracle.decision_hash(pri, idx, q, reasoning, backend)
        h_in = oracle.blake3(struct.pack("<4f", *pri) + (reasoning or b""))
        h_out = oracle.blake3(struct.pack("<3H", *idx) + struct.pack("<3h", *q) + (reasoning or b""))
        h_comb = oracle.blake3(h_in + h_out + (reasoning or b"") + (backend or b""))
        assert got == h_in + h_out + h_comb
