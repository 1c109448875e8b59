"""CPU pinning of the oracle's decoder-step pieces (RMSNorm, the fused forward's RoPE, causal GQA
attention) and of its full forward's KV cache: the reference's RoPE tests
(crates/adapteros-lora-mlx-ffi/src/attention.rs:893-980), closed forms, and float64 evaluation."""
import math

import numpy as np

import oracle


def test_rope_reference_cases():
    """attention.rs:893-980 at dim 2, theta 10000: position 0 is the identity; positions 1 and 5
    rotate [1, 0] to [cos p, sin p] and [0, 1] to [-sin p, cos p]."""
    x = np.array([[[1.0, 0.0], [0.0, 1.0]]], np.float32)  # one token, two rows (heads) of hd 2
    assert np.allclose(oracle.rope(x, 0, 10000.0)[0], [[1.0, 0.0], [0.0, 1.0]], atol=1e-6)
    one = np.array([[[1.0, 0.0]]], np.float32)
    for p in (1, 5):
        r = oracle.rope(one, p, 10000.0)[0, 0]
        assert abs(r[0] - math.cos(p)) < 1e-5 and abs(r[1] - math.sin(p)) < 1e-5
    r = oracle.rope(np.array([[[0.0, 1.0]]], np.float32), 1, 10000.0)[0, 0]
    assert abs(r[0] + math.sin(1.0)) < 1e-5 and abs(r[1] - math.cos(1.0)) < 1e-5


def test_rope_fused_forward_frequencies_and_halves():
    """The fused forward's rotation (mlx_cpp_wrapper_real.cpp:3249-3279) pairs element i with
    element i + hd/2 and uses inv_freq_i = 1 / theta^(-2i/hd): for hd 4 and theta 10000 the
    second pair turns 100 radians per position. Rotations preserve each pair's norm and compose
    additively in the position."""
    x = np.array([[[0.3, -1.2, 0.7, 0.4]]], np.float32)
    r = oracle.rope(x, 1, 10000.0)[0, 0]
    a = np.array([1.0, 100.0])
    c, s = np.cos(a), np.sin(a)
    want = [0.3 * c[0] - 0.7 * s[0], -1.2 * c[1] - 0.4 * s[1], 0.3 * s[0] + 0.7 * c[0], -1.2 * s[1] + 0.4 * c[1]]
    assert np.allclose(r, want, atol=2e-5)
    rng = np.random.default_rng(0)
    y = rng.standard_normal((3, 2, 16)).astype(np.float32)
    r = oracle.rope(y, 7, 500.0)
    assert np.allclose(np.hypot(r[..., :8], r[..., 8:]), np.hypot(y[..., :8], y[..., 8:]), rtol=1e-5)
    # rotating at position 3 then treating the result as position-0 data rotated by 4 == position 7
    # (angles are products of the position and a fixed frequency)
    assert np.allclose(oracle.rope(oracle.rope(y[:1], 3, 500.0), 4, 500.0), oracle.rope(y[:1], 7, 500.0), atol=2e-3)


def test_rmsnorm_closed_forms():
    w = np.linspace(0.5, 1.5, 64).astype(np.float32)
    x = np.full((1, 64), -3.0, np.float32)
    y = oracle.rmsnorm(x, w, 0.0)
    assert np.allclose(y[0], -w, rtol=1e-6)
    rng = np.random.default_rng(1)
    x = rng.standard_normal((5, 256)).astype(np.float32) * 4
    y32, y64 = oracle.rmsnorm(x, w.repeat(4), 1e-5), oracle.rmsnorm(x, w.repeat(4), 1e-5, mode=1)
    assert np.allclose(y32, y64, rtol=2e-6, atol=1e-6)
    # scale invariance up to eps
    assert np.allclose(oracle.rmsnorm(x * 8, w.repeat(4), 0.0), oracle.rmsnorm(x, w.repeat(4), 0.0), rtol=1e-5)


def test_attention_closed_forms():
    rng = np.random.default_rng(2)
    nh, nkv, hd = 4, 2, 16
    # one visible position: the output is that position's value (per kv head of the group)
    q = rng.standard_normal((1, nh, hd)).astype(np.float32)
    k = rng.standard_normal((1, nkv, hd)).astype(np.float32)
    v = rng.standard_normal((1, nkv, hd)).astype(np.float32)
    out = oracle.attention(q, k, v, 0)
    for h in range(nh):
        assert np.allclose(out[0, h], v[0, h // (nh // nkv)], atol=1e-6)
    # q = 0: equal scores, the mean of the visible values
    L, T = 9, 3
    k = rng.standard_normal((L, nkv, hd)).astype(np.float32)
    v = rng.standard_normal((L, nkv, hd)).astype(np.float32)
    out = oracle.attention(np.zeros((T, nh, hd), np.float32), k, v, L - T)
    for t in range(T):
        vis = L - T + t + 1
        for h in range(nh):
            assert np.allclose(out[t, h], v[:vis, h // 2].mean(0), atol=1e-5)
    # causality: changing keys and values after token t's position leaves token t unchanged
    q = rng.standard_normal((T, nh, hd)).astype(np.float32)
    a = oracle.attention(q, k, v, L - T)
    k2, v2 = k.copy(), v.copy()
    k2[L - 1] += 5.0
    v2[L - 1] -= 3.0
    b = oracle.attention(q, k2, v2, L - T)
    assert np.array_equal(a[:T - 1], b[:T - 1]) and not np.allclose(a[T - 1], b[T - 1])
    # float32 against float64
    assert np.allclose(a, oracle.attention(q, k, v, L - T, mode=1), atol=1e-5)
    # a dominant score selects its value (softmax of [1, 2, 3] grows with the score, attention.rs:990-1008)
    kk = np.zeros((3, 1, 2), np.float32)
    kk[:, 0, 0] = [1.0, 2.0, 3.0]
    vv = np.array([[0.0, 0.0], [1.0, 0.0], [0.0, 1.0]], np.float32)[:, None, :]
    qq = np.array([[[math.sqrt(2.0), 0.0]]], np.float32)  # scores 1, 2, 3 after the 1/sqrt(2) scale
    o = oracle.attention(qq, kk, vv, 2)[0, 0]
    p = np.exp([1.0, 2.0, 3.0])
    p /= p.sum()
    assert np.allclose(o, [p[1], p[2]], atol=1e-6)


def tiny_model(seed=0, L=2, H=128, I=256, nh=4, nkv=2, hd=32, vocab=256, n_adapters=3, rank=8, bias=True):
    """Random 4-bit weights (MLX layout), norms, q/k/v biases and rank-`rank` adapters on every
    module of every layer."""
    rng = np.random.default_rng(seed)

    def q4(out, inp):
        packed = rng.integers(0, 2 ** 32, (out, inp // 8), dtype=np.uint32)
        s = rng.uniform(0.01, 0.02, (out, inp // 64)).astype(np.float16)
        b = (-8.0 * s.astype(np.float32)).astype(np.float16)
        return packed, s, b

    shapes = {"q_proj": (nh * hd, H), "k_proj": (nkv * hd, H), "v_proj": (nkv * hd, H), "o_proj": (H, nh * hd),
              "gate_proj": (I, H), "up_proj": (I, H), "down_proj": (H, I)}
    layers, lora = [], []
    for _ in range(L):
        lw = {m: q4(*shapes[m]) for m in shapes}
        lw["input_norm"] = rng.uniform(0.8, 1.2, H).astype(np.float32)
        lw["post_norm"] = rng.uniform(0.8, 1.2, H).astype(np.float32)
        lw["bias"] = {m: (rng.standard_normal(shapes[m][0]) * 0.1).astype(np.float32) if bias else None
                      for m in ("q_proj", "k_proj", "v_proj")}
        layers.append(lw)
        lora.append([{m: ((rng.standard_normal((rank, shapes[m][1])) * 0.05).astype(np.float32),
                          (rng.standard_normal((shapes[m][0], rank)) * 0.05).astype(np.float32))
                      for m in shapes} for _ in range(n_adapters)])
    w = {"embed": q4(vocab, H), "lm_head": q4(vocab, H), "norm": rng.uniform(0.8, 1.2, H).astype(np.float32),
         "layers": layers}
    cfg = dict(num_layers=L, hidden=H, intermediate=I, num_heads=nh, num_kv_heads=nkv, head_dim=hd, vocab=vocab,
               rope_theta=10000.0, rms_eps=1e-6)
    scales = np.full(n_adapters, 2.0, np.float32)
    return cfg, w, lora, scales, rank


def rings(rng, T, n_adapters):
    r = np.zeros(T, oracle.RING_DTYPE)
    for t in range(T):
        k = int(rng.integers(0, 3))
        idx = rng.choice(n_adapters, k, replace=False)
        r[t]["top_k"] = k
        r[t]["current_pos"] = t
        r[t]["adapter_indices"][:k] = idx
        r[t]["gates_q15"][:k] = rng.integers(1, 32768, k)
    return r


def test_model_oracle_cache_equals_full_prefill():
    """Prefill then decode from the KV cache gives the logits of one prefill over the whole
    sequence (the cache holds exactly the rotated keys and values)."""
    cfg, w, lora, scales, rank = tiny_model()
    rng = np.random.default_rng(5)
    ids = rng.integers(0, cfg["vocab"], 9)
    rg = rings(rng, 9, len(scales))
    m = oracle.ModelOracle(cfg, w, lora, scales, rank)
    m.forward(ids[:6], rg[:6])
    m.forward(ids[6:8], rg[6:8])
    inc = m.forward(ids[8:], rg[8:])
    m.reset()
    full = m.forward(ids, rg)
    assert np.allclose(inc, full, rtol=1e-5, atol=1e-5)
    assert np.isfinite(full).all() and full.std() > 0.1


def test_model_oracle_fast_path_equals_c_loops():
    """ModelOracle(fast=True) (dequantised weights, float32 BLAS, per-adapter LoRA coefficients)
    against the C loops on the same model: a prefill, decode steps and a continuation, rings
    naming an adapter twice included; float32 with other summation orders."""
    cfg, w, lora, scales, rank = tiny_model(seed=5, n_adapters=3)
    rng = np.random.default_rng(11)
    n = 30
    ids = rng.integers(0, cfg["vocab"], n)
    rg = rings(rng, n, len(scales))
    rg[4]["top_k"] = 3
    rg[4]["adapter_indices"][:3] = [1, 1, 2]
    rg[4]["gates_q15"][:3] = [9000, 12000, 3000]
    slow = oracle.ModelOracle(cfg, w, lora, scales, rank)
    fast = oracle.ModelOracle(cfg, w, lora, scales, rank, fast=True)
    for a, b in [(0, 9), (9, 10), (10, 11), (11, 30)]:
        r0 = slow.forward(ids[a:b], rg[a:b])
        r1 = fast.forward(ids[a:b], rg[a:b])
        err = np.max(np.abs(r1 - r0)) / np.max(np.abs(r0))
        assert err < 2e-5, (a, b, err)
