"""CPU pinning of the oracle's layer functions (no GPU): int4 dequant, linear, LoRA delta,
SwiGLU MLP and projections against the reference's known answers, closed forms and independent
float64 evaluations in numpy."""
from __future__ import annotations

import numpy as np
import pytest

import oracle
import workloads as W
from cases import REL_TOL, tol_ratio


def pack_nibbles(q: np.ndarray) -> np.ndarray:
    """[out, in] nibble values -> MLX packing, 8 per uint32, element i at bits 4 * (i % 8)."""
    out, n = q.shape
    words = np.zeros((out, n // 8), np.uint32)
    for j in range(8):
        words |= q[:, j::8].astype(np.uint32) << np.uint32(4 * j)
    return words


def f16(a) -> np.ndarray:
    return np.asarray(a, np.float16)


def test_dequant_every_nibble_every_lane():
    """w[o, i] = scale[o, i/64] * q + bias[o, i/64] for every nibble value 0..15 in every one of
    the 8 positions of a word, across group boundaries, with negative, zero and large scales."""
    rng = np.random.default_rng(0)
    out, n = 16, 256
    q = np.zeros((out, n), np.uint8)
    for o in range(out):
        for i in range(n):
            q[o, i] = (o + i * 3 + (i // 8)) % 16
    assert all(len(set(q[:, i])) == 16 for i in range(8))
    s = f16(rng.choice([-0.5, -0.0, 0.0, 1e-3, 0.25, 3.0, 65504.0 / 16], (out, n // 64)))
    b = f16(rng.normal(0, 1, (out, n // 64)))
    w = oracle.dequant(pack_nibbles(q), s, b)
    sf = np.repeat(s.astype(np.float32), 64, axis=1)
    bf = np.repeat(b.astype(np.float32), 64, axis=1)
    expect = sf * q.astype(np.float32) + bf
    np.testing.assert_array_equal(w, expect)


def test_linear_against_float64():
    """x . dequant(W)^T in float32 (mode 0) and float64 (mode 1) against numpy float64."""
    rng = np.random.default_rng(1)
    out, n, T = 96, 512, 3
    q = rng.integers(0, 16, (out, n)).astype(np.uint8)
    s = f16(rng.normal(0, 0.02, (out, n // 64)))
    b = f16(rng.normal(0, 0.01, (out, n // 64)))
    x = rng.normal(0, 1, (T, n)).astype(np.float32)
    wd = np.repeat(s.astype(np.float64), 64, 1) * q + np.repeat(b.astype(np.float64), 64, 1)
    ref = x.astype(np.float64) @ wd.T
    y0 = oracle.linear_q4(x, pack_nibbles(q), s, b, mode=0)
    y1 = oracle.linear_q4(x, pack_nibbles(q), s, b, mode=1)
    assert np.max(np.abs(y1 - ref)) <= 1e-6 * np.max(np.abs(ref))
    assert tol_ratio(y0, ref) < 1e-4


def test_liquid_blend_known_answer():
    """crates/adapteros-lora-kernel-api/src/liquid.rs:267-336 (also lora-worker
    src/kernel_wrapper.rs:86-134): A1 = I, B1 = [[1,2],[3,4]], alpha 2, rank 2; A2 = ones, B2 =
    0.5s (bf16-exact), alpha 1; coefficients 0.5 / 0.5; x = [1, 1] -> [2.0, 4.0]."""
    A1 = np.eye(2, dtype=np.float32)
    B1 = np.array([[1, 2], [3, 4]], np.float32)
    A2 = np.ones((2, 2), np.float32)
    B2 = np.full((2, 2), 0.5, np.float32)
    out = oracle.liquid_blend([A1, A2], [B1, B2], [2, 2], [2.0, 1.0], [0.5, 0.5], np.ones(2, np.float32), 2)
    assert abs(out[0] - 2.0) < 1e-5 and abs(out[1] - 4.0) < 1e-5
    with pytest.raises(ValueError):
        oracle.liquid_blend([A1] * 4, [B1] * 4, [2] * 4, [1.0] * 4, [1.0] * 4, np.ones(2, np.float32), 2)


def _identity_q4(out: int, n: int):
    """int4 weights equal to the identity on the first `out` inputs: q = 1, scale 1, bias 0."""
    q = np.zeros((out, n), np.uint8)
    for o in range(out):
        q[o, o] = 1
    s = f16(np.ones((out, n // 64)))
    b = f16(np.zeros((out, n // 64)))
    return pack_nibbles(q), s, b


def test_lora_projection_known_answer():
    """crates/adapteros-lora-mlx-ffi/src/lora_cpp_tests.rs:57-119: W = I, x = [2, 3], A = [[1, 1]],
    B = [[1], [2]], scale 1, gate q = 16384 -> [2 + 5g, 3 + 10g] with g = 16384 / 32767 (the
    2x2 case embedded in a 32 x 64 int4 layer)."""
    out, n = 32, 64
    w = _identity_q4(out, n)
    x = np.zeros((1, n), np.float32)
    x[0, :2] = [2, 3]
    A = np.zeros((1, n), np.float32)
    A[0, :2] = 1
    B = np.zeros((out, 1), np.float32)
    B[:2, 0] = [1, 2]
    ring = np.zeros(1, oracle.RING_DTYPE)
    ring[0]["top_k"] = 1
    ring[0]["adapter_indices"][0] = 0
    ring[0]["gates_q15"][0] = 16384
    y = oracle.proj_forward(x, w, "foo", ["foo"], [{"foo": (A, B)}], [1.0], 1, ring)
    g = np.float32(16384) / np.float32(32767)
    assert abs(y[0, 0] - (2 + 5 * g)) < 1e-3 and abs(y[0, 1] - (3 + 10 * g)) < 1e-3
    assert np.all(y[0, 2:] == 0)


def _rand_layer(rng, H, I, n_ad, r):
    def q4(out, n):
        q = rng.integers(0, 16, (out, n)).astype(np.uint8)
        return pack_nibbles(q), f16(rng.normal(0, 0.02, (out, n // 64))), f16(rng.normal(0, 0.01, (out, n // 64))), q

    mats = {"gate_proj": q4(I, H), "up_proj": q4(I, H), "down_proj": q4(H, I)}
    lora = []
    for _ in range(n_ad):
        lora.append({m: (rng.normal(0, 1 / np.sqrt(H if m != "down_proj" else I), (r, H if m != "down_proj" else I)).astype(np.float32),
                         rng.normal(0, 0.05, (I if m != "down_proj" else H, r)).astype(np.float32))
                     for m in mats})
    return mats, lora


def _dense(m):
    p, s, b, q = m
    return np.repeat(s.astype(np.float64), 64, 1) * q + np.repeat(b.astype(np.float64), 64, 1)


def test_mlp_against_numpy_float64():
    """SwiGLU MLP with per-token rings (mlx_cpp_wrapper_real.cpp:3509-3527): each token's
    active slots (q > 0, bound adapter) add (x A^T) B^T * scale * q / 32767 to gate, up and down
    (down's LoRA input is h); checked against an independent numpy float64 evaluation."""
    rng = np.random.default_rng(2)
    H, I, n_ad, r, T = 128, 320, 5, 4, 4
    mats, lora = _rand_layer(rng, H, I, n_ad, r)
    scales = np.array([1.0, 0.5, 2.0, 1.0, 0.25], np.float32)
    rings = np.zeros(T, oracle.RING_DTYPE)
    slots = [[(0, 20000), (3, 12767)], [(1, 32767)], [(2, 0), (4, 9000), (7, 5000)], []]
    for t, sl in enumerate(slots):
        rings[t]["top_k"] = len(sl)
        for j, (a, q) in enumerate(sl):
            rings[t]["adapter_indices"][j] = a
            rings[t]["gates_q15"][j] = q
    x = rng.normal(0, 1, (T, H)).astype(np.float32)
    y = oracle.mlp_forward(x, mats["gate_proj"][:3], mats["up_proj"][:3], mats["down_proj"][:3], lora, scales, r, rings)
    y1 = oracle.mlp_forward(x, mats["gate_proj"][:3], mats["up_proj"][:3], mats["down_proj"][:3], lora, scales, r, rings,
                            mode=1)
    Wg, Wu, Wd = _dense(mats["gate_proj"]), _dense(mats["up_proj"]), _dense(mats["down_proj"])
    ref = np.zeros((T, H))
    for t in range(T):
        xt = x[t].astype(np.float64)
        act = [(a, q) for a, q in slots[t] if q > 0 and a < n_ad]
        g = Wg @ xt + sum(scales[a] * (q / 32767) * (lora[a]["gate_proj"][1] @ (lora[a]["gate_proj"][0] @ xt)) for a, q in act)
        u = Wu @ xt + sum(scales[a] * (q / 32767) * (lora[a]["up_proj"][1] @ (lora[a]["up_proj"][0] @ xt)) for a, q in act)
        h = g / (1 + np.exp(-g)) * u
        ref[t] = Wd @ h + sum(scales[a] * (q / 32767) * (lora[a]["down_proj"][1] @ (lora[a]["down_proj"][0] @ h)) for a, q in act)
    assert tol_ratio(y, ref) < 1e-4
    assert tol_ratio(y1, ref) < 1e-6


def test_zero_gate_and_unbound_contribute_nothing():
    """Slots with q <= 0 or an adapter index outside the table add nothing (backend.rs:409-425);
    a token with an empty ring gets the base layer."""
    rng = np.random.default_rng(3)
    H, I, r = 64, 128, 4
    mats, lora = _rand_layer(rng, H, I, 2, r)
    x = rng.normal(0, 1, (2, H)).astype(np.float32)
    empty = np.zeros(2, oracle.RING_DTYPE)
    inert = np.zeros(2, oracle.RING_DTYPE)
    for t in range(2):
        inert[t]["top_k"] = 3
        inert[t]["adapter_indices"][:3] = [0, 1, 9]
        inert[t]["gates_q15"][:3] = [0, -5, 30000]
    args = (mats["gate_proj"][:3], mats["up_proj"][:3], mats["down_proj"][:3], lora, np.ones(2, np.float32), r)
    np.testing.assert_array_equal(oracle.mlp_forward(x, *args[:3], *args[3:], empty),
                                  oracle.mlp_forward(x, *args[:3], *args[3:], inert))


def test_lora_linearity_in_gate():
    """The delta is linear in scale * blend: two slots of one adapter with gates q1, q2 equal one
    slot with q1 + q2 (to float32 rounding)."""
    rng = np.random.default_rng(4)
    n, out, r = 128, 64, 8
    w = _identity_q4(out, n)
    A = rng.normal(0, 0.1, (r, n)).astype(np.float32)
    B = rng.normal(0, 0.1, (out, r)).astype(np.float32)
    x = rng.normal(0, 1, (1, n)).astype(np.float32)

    def run(slots):
        ring = np.zeros(1, oracle.RING_DTYPE)
        ring[0]["top_k"] = len(slots)
        for j, q in enumerate(slots):
            ring[0]["adapter_indices"][j] = 0
            ring[0]["gates_q15"][j] = q
        return oracle.proj_forward(x, w, "m", ["m"], [{"m": (A, B)}], [1.0], r, ring)

    base = run([])
    d1 = run([10000, 6000]) - base
    d2 = run([16000]) - base
    assert np.max(np.abs(d1 - d2)) < 1e-5


def test_swiglu_special_values():
    """silu(g) * u: g = 0 gives 0; large positive g gives g * u; large negative g gives 0."""
    H, I = 64, 64
    rng = np.random.default_rng(5)
    w_id = _identity_q4(I, H)
    zero = (np.zeros((H, I // 8), np.uint32), f16(np.zeros((H, I // 64))), f16(np.zeros((H, I // 64))))
    x = np.zeros((3, H), np.float32)
    x[0, 0] = 0.0
    x[1, 0] = 30.0
    x[2, 0] = -30.0
    _, h = oracle.mlp_forward(x, w_id, w_id, zero, [], np.zeros(0, np.float32), 1, np.zeros(3, oracle.RING_DTYPE),
                              return_h=True)
    assert h[0, 0] == 0.0
    assert abs(h[1, 0] - 900.0) < 1e-3
    assert abs(h[2, 0]) < 1e-9
    del rng


def test_priors_match_synthetic_workload_digest():
    """The 0.5B-shaped fixture: synthetic tensors reproduce their SHA-256 digests, and the oracle
    reproduces the committed rings and MLP outputs bit for bit (a regression guard: the
    reference's own answers pin the functions above; this pins the generator and the whole
    oracle path together)."""
    import hashlib
    from pathlib import Path

    fx = np.load(Path(__file__).resolve().parent / "golden" / "c1_layer.npz")
    digests = dict(zip(fx["digest_names"].tolist(), fx["digests"].tolist()))
    cfg = W.CONFIGS[1]
    for m in cfg.modules:
        for name, arr in zip(("packed", "scales", "biases"), W.base_weights(cfg, m)):
            assert hashlib.sha256(np.ascontiguousarray(arr).tobytes()).hexdigest() == digests[f"{m}.{name}"]
    T = fx["y"].shape[0]
    f, w = W.router_inputs(cfg, T)
    pri = oracle.priors(f, w)
    np.testing.assert_array_equal(pri, fx["priors"])
    rings = oracle.route_batch(pri, cfg.k, cfg.tau, cfg.eps, 1.0, np.arange(cfg.n_adapters, dtype=np.uint64))
    assert rings.view(np.uint8).tobytes() == fx["rings"].tobytes()
    from cases import oracle_mlp

    _, xf = W.activations(cfg, T)
    y = oracle_mlp(1, xf, rings)
    np.testing.assert_array_equal(y, fx["y"])
    assert REL_TOL == 2e-2
