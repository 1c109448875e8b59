"""ctypes wrapper of the CPU oracle (oracle/liborc.so).

TEST INFRASTRUCTURE ONLY: the oracle the HIP path is tested against. Only tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg use it. See aos_oracle.h for the reference file:line each function
restates and how each is pinned.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
# AOS_ORACLE_LIB selects another build of the same source (the sanitizer build, oracle/_asan)
LIB = Path(os.environ["AOS_ORACLE_LIB"]) if os.environ.get("AOS_ORACLE_LIB") else HERE / "liborc.so"

RING_DTYPE = np.dtype(
    [("top_k", "<u4"), ("current_pos", "<u4"), ("adapter_indices", "<u2", (8,)), ("gates_q15", "<i2", (8,))]
)

_lib = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)


class _Q4(C.Structure):
    _fields_ = [("wp", C.c_void_p), ("scales", C.c_void_p), ("biases", C.c_void_p)]


class _Mod(C.Structure):
    _fields_ = [("A", C.c_void_p), ("B", C.c_void_p)]


def lib():
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        L = C.CDLL(str(LIB))
        P = C.c_void_p
        L.orc_quantize_gate.restype = C.c_int16
        L.orc_quantize_gate.argtypes = [C.c_float]
        L.orc_total_cmp_key_desc.restype = C.c_uint64
        L.orc_total_cmp_key_desc.argtypes = [C.c_float]
        L.orc_route_one.restype = C.c_int
        L.orc_route_one.argtypes = [P, C.c_int, P, P, C.c_int, C.c_float, C.c_float, C.c_float, P, P]
        L.orc_route_batch.restype = C.c_int
        L.orc_route_batch.argtypes = [P, C.c_int, C.c_int, P, P, C.c_int, C.c_float, C.c_float, C.c_float, P, P]
        L.orc_route_one_ex.restype = C.c_int
        L.orc_route_one_ex.argtypes = [P, C.c_int, P, P, P, P, C.c_int, C.c_float, C.c_float, C.c_float, P, P]
        L.orc_route_one_detail.restype = C.c_int
        L.orc_route_one_detail.argtypes = [P, C.c_int, P, P, P, P, C.c_int, C.c_float, C.c_float, C.c_float, P, P,
                                           P, P]
        L.orc_renormalize_q15.restype = None
        L.orc_renormalize_q15.argtypes = [P, C.c_int, P]
        L.orc_filter_decision.restype = C.c_int
        L.orc_filter_decision.argtypes = [P, P, C.c_int, P, C.c_int, P, P]
        L.orc_decision_to_ring.restype = C.c_int
        L.orc_decision_to_ring.argtypes = [P, P, C.c_int, P, P, C.c_int, C.c_int, P]
        L.orc_route_batch_ex.restype = None
        L.orc_route_batch_ex.argtypes = [P, C.c_int, C.c_int, P, P, P, P, C.c_int, C.c_float, C.c_float,
                                         C.c_float, P, C.c_int, P, P, P, P]
        L.orc_chacha20_block.restype = None
        L.orc_chacha20_block.argtypes = [P, P]
        L.orc_tie_breakers.restype = None
        L.orc_tie_breakers.argtypes = [P, C.c_int, P]
        L.orc_blake3.restype = None
        L.orc_blake3.argtypes = [P, C.c_size_t, P]
        L.orc_decision_hash.restype = None
        L.orc_decision_hash.argtypes = [P, C.c_int, P, P, C.c_int, P, P, P]
        L.orc_rmsnorm.restype = None
        L.orc_rmsnorm.argtypes = [P, C.c_int, C.c_int, P, C.c_float, P, C.c_int]
        L.orc_rope.restype = None
        L.orc_rope.argtypes = [P, C.c_int, C.c_int, C.c_int, C.c_int, C.c_float]
        L.orc_attention.restype = None
        L.orc_attention.argtypes = [P, P, P, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, P, C.c_int]
        L.orc_priors.restype = None
        L.orc_priors.argtypes = [P, P, C.c_int, C.c_int, C.c_int, P]
        L.orc_dequant_q4.restype = None
        L.orc_dequant_q4.argtypes = [P, P, P, C.c_int, C.c_int, P]
        L.orc_linear_q4.restype = None
        L.orc_linear_q4.argtypes = [P, C.c_int, P, P, P, C.c_int, C.c_int, P, C.c_int]
        L.orc_lora_delta.restype = None
        L.orc_lora_delta.argtypes = [P, P, P, C.c_int, C.c_int, C.c_int, C.c_float, P, C.c_int, C.c_int]
        L.orc_liquid_blend.restype = C.c_int
        L.orc_liquid_blend.argtypes = [C.c_int, P, P, P, P, P, P, C.c_int, P, C.c_int]
        L.orc_mlp_forward.restype = None
        L.orc_mlp_forward.argtypes = [P, C.c_int, C.c_int, C.c_int, P, P, P, P, P, C.c_int, C.c_int, P, P,
                                      C.c_int, P]
        L.orc_proj_forward.restype = None
        L.orc_proj_forward.argtypes = [P, C.c_int, C.c_int, C.c_int, P, P, C.c_int, C.c_int, P, C.c_int,
                                       C.c_int, P, P, C.c_int]
        L.orc_exp.restype = C.c_double
        L.orc_exp.argtypes = [C.c_double]
        L.orc_set_exp.restype = None
        L.orc_set_exp.argtypes = [C.c_void_p]
        L.orc_f32_to_f16.restype = C.c_uint16
        L.orc_f32_to_f16.argtypes = [C.c_float]
        L.orc_f16_to_f32.restype = C.c_float
        L.orc_f16_to_f32.argtypes = [C.c_uint16]
        L.orc_num_threads.restype = C.c_int
        L.orc_set_num_threads.argtypes = [C.c_int]
        _lib = L
    return _lib


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


def quantize_gate(g: float) -> int:
    return int(lib().orc_quantize_gate(float(g)))


def route_one(priors, k, tau=1.0, eps=0.02, routing_bias=1.0, stable_ids=None, allowed=None):
    """Returns (indices, gates) lists, or raises ValueError for the reference's error cases."""
    p = _c(priors, np.float32)
    n = p.shape[0]
    sid = None if stable_ids is None else _c(stable_ids, np.uint64)
    al = None if allowed is None else _c(allowed, np.uint8)
    idx = np.zeros(8, np.uint16)
    q = np.zeros(8, np.int16)
    kk = lib().orc_route_one(p.ctypes.data, n, sid.ctypes.data if sid is not None else None,
                             al.ctypes.data if al is not None else None, k, tau, eps, routing_bias,
                             idx.ctypes.data, q.ctypes.data)
    if kk < 0:
        raise ValueError("routing error (non-finite prior/score or k > 8)")
    return idx[:kk].tolist(), q[:kk].tolist()


def route_batch(priors, k, tau=1.0, eps=0.02, routing_bias=1.0, stable_ids=None, allowed=None):
    """Rings for every token (a token whose routing fails gets an all-zero ring)."""
    p = _c(priors, np.float32)
    T, n = p.shape
    sid = None if stable_ids is None else _c(stable_ids, np.uint64)
    al = None if allowed is None else _c(allowed, np.uint8)
    rings = np.zeros(T, RING_DTYPE)
    bad = C.c_int(-1)
    lib().orc_route_batch(p.ctypes.data, T, n, sid.ctypes.data if sid is not None else None,
                          al.ctypes.data if al is not None else None, k, tau, eps, routing_bias,
                          rings.ctypes.data, C.byref(bad))
    return rings


def _opt(a, dtype):
    return None if a is None else _c(a, dtype)


def _ptr(a):
    return None if a is None else a.ctypes.data


def route_one_ex(priors, k, tau=1.0, eps=0.02, routing_bias=1.0, stable_ids=None, allowed=None,
                 scope=None, breakers=None):
    """route_one with a scope hint (bytes per adapter) and adaptive tie-breakers (u64 per adapter)."""
    p = _c(priors, np.float32)
    arrs = [_opt(stable_ids, np.uint64), _opt(allowed, np.uint8), _opt(scope, np.uint8), _opt(breakers, np.uint64)]
    idx = np.zeros(8, np.uint16)
    q = np.zeros(8, np.int16)
    kk = lib().orc_route_one_ex(p.ctypes.data, p.shape[0], *[_ptr(a) for a in arrs], k, tau, eps, routing_bias,
                                idx.ctypes.data, q.ctypes.data)
    if kk < 0:
        raise ValueError("routing error (non-finite prior/score or k > 8)")
    return idx[:kk].tolist(), q[:kk].tolist()


def route_one_detail(priors, k, tau=1.0, eps=0.02, routing_bias=1.0, stable_ids=None, allowed=None,
                     scope=None, breakers=None):
    """route_one_ex with the Decision's entropy and candidates: (indices, gates, raw_scores,
    entropy), the candidates in decision order (aos_oracle.c: orc_route_one_detail)."""
    p = _c(priors, np.float32)
    arrs = [_opt(stable_ids, np.uint64), _opt(allowed, np.uint8), _opt(scope, np.uint8), _opt(breakers, np.uint64)]
    idx = np.zeros(8, np.uint16)
    q = np.zeros(8, np.int16)
    raw = np.zeros(8, np.float32)
    ent = np.zeros(1, np.float32)
    kk = lib().orc_route_one_detail(p.ctypes.data, p.shape[0], *[_ptr(a) for a in arrs], k, tau, eps, routing_bias,
                                    idx.ctypes.data, q.ctypes.data, ent.ctypes.data, raw.ctypes.data)
    if kk < 0:
        raise ValueError("routing error (non-finite prior/score or k > 8)")
    return idx[:kk].tolist(), q[:kk].tolist(), raw[:kk].copy(), np.float32(ent[0])


def renormalize_q15(gates) -> list[int]:
    g = _c(gates, np.int16)
    out = np.zeros(max(len(g), 1), np.int16)
    lib().orc_renormalize_q15(g.ctypes.data, len(g), out.ctypes.data)
    return out[:len(g)].tolist()


def filter_decision(indices, gates, allowed, max_per_token=-1):
    """(indices, gates) after the policy filter; raises PermissionError for a PolicyViolation."""
    i = _c(indices, np.uint16)
    g = _c(gates, np.int16)
    al = _c(allowed, np.uint8)
    oi = np.zeros(8, np.uint16)
    og = np.zeros(8, np.int16)
    m = lib().orc_filter_decision(i.ctypes.data, g.ctypes.data, len(i), al.ctypes.data, max_per_token,
                                  oi.ctypes.data, og.ctypes.data)
    if m < 0:
        raise PermissionError("PolicyViolation: routing policy denied all adapters")
    return oi[:m].tolist(), og[:m].tolist()


def decision_to_ring(indices, gates, active_ids=None, strengths=None, n_active=None, position=0):
    i = _c(indices, np.uint16)
    g = _c(gates, np.int16)
    a = _opt(active_ids, np.uint16)
    s = _opt(strengths, np.float32)
    n = n_active if n_active is not None else (len(a) if a is not None else (len(s) if s is not None else 65536))
    ring = np.zeros(1, RING_DTYPE)
    rc = lib().orc_decision_to_ring(i.ctypes.data, g.ctypes.data, len(i), _ptr(a), _ptr(s), n, position,
                                    ring.ctypes.data)
    if rc < 0:
        raise LookupError("Routing: decision index not in active set")
    return ring[0]


def route_batch_ex(priors, k, tau=1.0, eps=0.02, routing_bias=1.0, stable_ids=None, allowed=None, scope=None,
                   breakers=None, post_allowed=None, post_max=-1, active_ids=None, strengths=None):
    """(rings, status) of one device routing call with the router extras."""
    p = _c(priors, np.float32)
    T, n = p.shape
    arrs = [_opt(stable_ids, np.uint64), _opt(allowed, np.uint8), _opt(scope, np.uint8), _opt(breakers, np.uint64)]
    post = [_opt(post_allowed, np.uint8)]
    tail = [_opt(active_ids, np.uint16), _opt(strengths, np.float32)]
    rings = np.zeros(T, RING_DTYPE)
    status = np.zeros(T, np.int32)
    lib().orc_route_batch_ex(p.ctypes.data, T, n, *[_ptr(a) for a in arrs], k, tau, eps, routing_bias,
                             _ptr(post[0]), post_max, *[_ptr(a) for a in tail], rings.ctypes.data,
                             status.ctypes.data)
    return rings, status


def chacha20_block(words) -> list[int]:
    w = _c(words, np.uint32)
    out = np.zeros(16, np.uint32)
    lib().orc_chacha20_block(w.ctypes.data, out.ctypes.data)
    return out.tolist()


def tie_breakers(seed: bytes, n: int) -> np.ndarray:
    sd = np.frombuffer(bytes(seed), dtype=np.uint8).copy()
    assert sd.size == 32
    out = np.zeros(max(n, 1), np.uint64)
    lib().orc_tie_breakers(sd.ctypes.data, n, out.ctypes.data)
    return out[:n]


def blake3(data: bytes) -> bytes:
    buf = np.frombuffer(bytes(data), dtype=np.uint8).copy() if len(data) else np.zeros(1, np.uint8)
    out = np.zeros(32, np.uint8)
    lib().orc_blake3(buf.ctypes.data, len(data), out.ctypes.data)
    return out.tobytes()


def decision_hash(priors, indices, gates, reasoning: bytes | None = None, backend: bytes | None = None) -> bytes:
    """96 bytes: the input, output and combined hashes of Router::compute_decision_hash."""
    p = _c(priors, np.float32)
    i = _c(indices, np.uint16) if len(indices) else np.zeros(1, np.uint16)
    g = _c(gates, np.int16) if len(gates) else np.zeros(1, np.int16)
    r = None if reasoning is None else np.frombuffer(reasoning, np.uint8).copy()
    b = None if backend is None else np.frombuffer(backend, np.uint8).copy()
    out = np.zeros(96, np.uint8)
    lib().orc_decision_hash(p.ctypes.data, p.shape[0], i.ctypes.data, g.ctypes.data, len(indices), _ptr(r), _ptr(b),
                            out.ctypes.data)
    return out.tobytes()


def priors(features, router_w):
    f = _c(features, np.float32)
    w = _c(router_w, np.float32)
    T, d = f.shape
    n = w.shape[0]
    out = np.empty((T, n), np.float32)
    lib().orc_priors(f.ctypes.data, w.ctypes.data, T, n, d, out.ctypes.data)
    return out


def dequant(packed, scales, biases):
    wp = _c(packed, np.uint32)
    out, w = wp.shape
    s = np.ascontiguousarray(scales).view(np.uint16)
    b = np.ascontiguousarray(biases).view(np.uint16)
    dst = np.empty((out, w * 8), np.float32)
    lib().orc_dequant_q4(wp.ctypes.data, s.ctypes.data, b.ctypes.data, out, w * 8, dst.ctypes.data)
    return dst


def linear_q4(x, packed, scales, biases, mode=0):
    x = _c(x, np.float32)
    wp = _c(packed, np.uint32)
    out, w = wp.shape
    s = np.ascontiguousarray(scales).view(np.uint16)
    b = np.ascontiguousarray(biases).view(np.uint16)
    y = np.empty((x.shape[0], out), np.float32)
    lib().orc_linear_q4(x.ctypes.data, x.shape[0], wp.ctypes.data, s.ctypes.data, b.ctypes.data, out, w * 8,
                        y.ctypes.data, mode)
    return y


def lora_delta(x, A, B, coef, mode=0):
    x = _c(x, np.float32)
    A = _c(A, np.float32)
    B = _c(B, np.float32)
    r, din = A.shape
    dout = B.shape[0]
    d = np.zeros(dout, np.float32)
    lib().orc_lora_delta(x.ctypes.data, A.ctypes.data, B.ctypes.data, r, din, dout, coef, d.ctypes.data, 1, mode)
    return d


def liquid_blend(As, Bs, ranks, alphas, coefs, x, out_len):
    n = len(As)
    As = [_c(a, np.float32) for a in As]
    Bs = [_c(b, np.float32) for b in Bs]
    Ap = (C.c_void_p * n)(*[a.ctypes.data for a in As])
    Bp = (C.c_void_p * n)(*[b.ctypes.data for b in Bs])
    rk = _c(ranks, np.int32)
    al = _c(alphas, np.float32)
    cf = _c(coefs, np.float32)
    x = _c(x, np.float32)
    out = np.zeros(out_len, np.float32)
    rc = lib().orc_liquid_blend(n, Ap, Bp, rk.ctypes.data, al.ctypes.data, cf.ctypes.data, x.ctypes.data,
                                x.shape[0], out.ctypes.data, out_len)
    if rc != 0:
        raise ValueError("liquid blend rejected")
    return out


class _Keep:
    """Keeps numpy buffers alive while C pointers to them are in use."""

    def __init__(self):
        self.items = []

    def __call__(self, a):
        self.items.append(a)
        return a


def _q4(keep, w):
    packed, scales, biases = w
    p = keep(_c(packed, np.uint32))
    s = keep(np.ascontiguousarray(scales).view(np.uint16))
    b = keep(np.ascontiguousarray(biases).view(np.uint16))
    return _Q4(p.ctypes.data, s.ctypes.data, b.ctypes.data)


def _mods(keep, lora, n_adapters, modules):
    """lora[a][module] = (A, B) or None -> flat [n_adapters * n_modules] array."""
    arr = (_Mod * (n_adapters * len(modules)))()
    for a in range(n_adapters):
        for mi, m in enumerate(modules):
            ab = lora[a].get(m) if lora[a] is not None else None
            if ab is None:
                continue
            A = keep(_c(ab[0], np.float32))
            B = keep(_c(ab[1], np.float32))
            arr[a * len(modules) + mi] = _Mod(A.ctypes.data, B.ctypes.data)
    return arr


def mlp_forward(x, gate, up, down, lora, scales, rank, rings, mode=0, return_h=False):
    """SwiGLU MLP with per-token rings; lora[a] = {"gate_proj": (A, B), ...}."""
    keep = _Keep()
    x = keep(_c(x, np.float32))
    T, H = x.shape
    I = gate[0].shape[0]
    g, u, d = _q4(keep, gate), _q4(keep, up), _q4(keep, down)
    n = len(lora)
    mods = _mods(keep, lora, n, ("gate_proj", "up_proj", "down_proj"))
    sc = keep(_c(scales, np.float32))
    rg = keep(np.ascontiguousarray(rings, dtype=RING_DTYPE))
    y = np.empty((T, H), np.float32)
    h = np.empty((T, I), np.float32) if return_h else None
    lib().orc_mlp_forward(x.ctypes.data, T, H, I, C.byref(g), C.byref(u), C.byref(d), mods, sc.ctypes.data, n,
                          rank, rg.ctypes.data, y.ctypes.data, mode, h.ctypes.data if h is not None else None)
    return (y, h) if return_h else y


def proj_forward(x, w, module, modules, lora, scales, rank, rings, mode=0):
    keep = _Keep()
    x = keep(_c(x, np.float32))
    T, din = x.shape
    dout = w[0].shape[0]
    q = _q4(keep, w)
    n = len(lora)
    mods = _mods(keep, lora, n, modules)
    sc = keep(_c(scales, np.float32))
    rg = keep(np.ascontiguousarray(rings, dtype=RING_DTYPE))
    y = np.empty((T, dout), np.float32)
    lib().orc_proj_forward(x.ctypes.data, T, din, dout, C.byref(q), mods, len(modules), modules.index(module),
                           sc.ctypes.data, n, rank, rg.ctypes.data, y.ctypes.data, mode)
    return y


def rmsnorm(x, w, eps, mode=0):
    x = _c(x, np.float32)
    T, H = x.shape
    w = _c(w, np.float32)
    y = np.empty_like(x)
    lib().orc_rmsnorm(x.ctypes.data, T, H, w.ctypes.data, eps, y.ctypes.data, mode)
    return y


def rope(x, offset, theta):
    """x[T][heads][hd] rotated (a copy)."""
    x = np.array(x, dtype=np.float32, order="C", copy=True)
    T, heads, hd = x.shape
    lib().orc_rope(x.ctypes.data, T, heads, hd, offset, theta)
    return x


def attention(q, k, v, offset, mode=0):
    """q[T][nh][hd]; k, v[L][nkv][hd] with L = offset + T -> out[T][nh][hd]."""
    q = _c(q, np.float32)
    k = _c(k, np.float32)
    v = _c(v, np.float32)
    T, nh, hd = q.shape
    nkv = k.shape[1]
    assert k.shape[0] == offset + T and v.shape == k.shape
    out = np.empty_like(q)
    lib().orc_attention(q.ctypes.data, k.ctypes.data, v.ctypes.data, T, offset, nh, nkv, hd, out.ctypes.data, mode)
    return out


def _lora_coefs(rings, n_adapters, has):
    """coef[t][a] = sum over token t's ring slots s < top_k naming adapter a (q > 0, a < n, the
    module present) of q / 32767: add_lora_for_ring's rule (aos_oracle.c) as one matrix."""
    rg = np.ascontiguousarray(rings, dtype=RING_DTYPE)
    T = rg.shape[0]
    coef = np.zeros((T, n_adapters), np.float32)
    for t in range(T):
        kk = min(int(rg[t]["top_k"]), 8)
        for sl in range(kk):
            q = int(rg[t]["gates_q15"][sl])
            a = int(rg[t]["adapter_indices"][sl])
            if q > 0 and a < n_adapters and has[a]:
                coef[t, a] += np.float32(q) / np.float32(32767.0)
    return coef


def proj_forward_fast(x, w_deq, module, lora, scales, rings):
    """proj_forward in float32 BLAS: x @ W^T with W dequantised once, plus each token's LoRA delta
    scale[a] * coef[t][a] * B_a (A_a x_t) summed over the adapters. The same arithmetic as the C
    oracle's, in another summation order (pinned against it by the oracle's own tests)."""
    x = _c(x, np.float32)
    y = x @ w_deq.T
    n = len(lora)
    has = [lora[a] is not None and lora[a].get(module) is not None for a in range(n)]
    coef = _lora_coefs(rings, n, has)
    for a in range(n):
        if not has[a] or not coef[:, a].any():
            continue
        A, B = lora[a][module]
        c = coef[:, a] * np.float32(scales[a])
        y += ((x @ np.asarray(A, np.float32).T) @ np.asarray(B, np.float32).T) * c[:, None]
    return y


class ModelOracle:
    """mlx_model_forward_with_cache_and_lora (mlx_cpp_wrapper_real.cpp:3339-3527) on the CPU with its
    KV cache: embedding, per layer RMSNorm -> q/k/v (+bias, +LoRA) -> RoPE -> cache -> causal GQA
    attention -> o_proj (+LoRA) -> residual -> RMSNorm -> SwiGLU MLP (+LoRA) -> residual, final
    RMSNorm, LM head on the last token. float32 activations throughout (MLX promotes to float32
    after RoPE).

    cfg: dict of num_layers, hidden, intermediate, num_heads, num_kv_heads, head_dim, vocab,
    rope_theta, rms_eps. w: {"embed": (packed, scales, biases) or "embed_bf16": uint16 rows,
    "lm_head": (packed, scales, biases), "norm": [H], "layers": [{"input_norm", "post_norm",
    "q_proj" .. "down_proj": (packed, scales, biases), "bias": {"q_proj": [out] or None, ..}}]}.
    lora[layer][a] = {module: (A, B)} for n adapters of one rank; scales[a] = alpha / rank.

    fast=True computes the projections and the MLP with the weights dequantised once and float32
    BLAS products (proj_forward_fast) instead of the C loops; the rest (norms, RoPE, attention,
    the LM head) is the same code. For model shapes where the C loops would take minutes."""

    ATTN = ("q_proj", "k_proj", "v_proj", "o_proj")
    MODS = ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")

    def __init__(self, cfg, w, lora, scales, rank, fast=False):
        self.cfg, self.w, self.lora, self.scales, self.rank = cfg, w, lora, scales, rank
        self.fast = fast
        self.deq = [{m: dequant(*lw[m]) for m in self.MODS} for lw in w["layers"]] if fast else None
        if "embed" in w:
            self.embed = dequant(*w["embed"])
        else:
            self.embed = (np.ascontiguousarray(w["embed_bf16"], np.uint16).astype(np.uint32) << 16).view(np.float32)
        self.reset()

    def reset(self):
        L, nkv, hd = self.cfg["num_layers"], self.cfg["num_kv_heads"], self.cfg["head_dim"]
        self.kc = [np.zeros((0, nkv, hd), np.float32) for _ in range(L)]
        self.vc = [np.zeros((0, nkv, hd), np.float32) for _ in range(L)]

    def forward(self, ids, rings, mode=0):
        c, w = self.cfg, self.w
        T = len(ids)
        nh, nkv, hd, eps = c["num_heads"], c["num_kv_heads"], c["head_dim"], c["rms_eps"]
        offset = self.kc[0].shape[0]
        x = self.embed[np.asarray(ids)].astype(np.float32)
        for li, lw in enumerate(w["layers"]):
            lo = self.lora[li]
            normed = rmsnorm(x, lw["input_norm"], eps, mode)
            qkv = []
            for m in ("q_proj", "k_proj", "v_proj"):
                y = (proj_forward_fast(normed, self.deq[li][m], m, lo, self.scales, rings) if self.fast else
                     proj_forward(normed, lw[m], m, self.ATTN, lo, self.scales, self.rank, rings, mode))
                b = lw.get("bias", {}).get(m)
                qkv.append(y + np.asarray(b, np.float32) if b is not None else y)
            q = rope(qkv[0].reshape(T, nh, hd), offset, c["rope_theta"])
            k = rope(qkv[1].reshape(T, nkv, hd), offset, c["rope_theta"])
            v = qkv[2].reshape(T, nkv, hd)
            self.kc[li] = np.concatenate([self.kc[li], k])
            self.vc[li] = np.concatenate([self.vc[li], v])
            a = attention(q, self.kc[li], self.vc[li], offset, mode).reshape(T, nh * hd)
            if self.fast:
                x = x + proj_forward_fast(a, self.deq[li]["o_proj"], "o_proj", lo, self.scales, rings)
                normed = rmsnorm(x, lw["post_norm"], eps, mode)
                g = proj_forward_fast(normed, self.deq[li]["gate_proj"], "gate_proj", lo, self.scales, rings)
                u = proj_forward_fast(normed, self.deq[li]["up_proj"], "up_proj", lo, self.scales, rings)
                h = (g * (np.float32(1.0) / (np.float32(1.0) + np.exp(-g)))) * u
                x = x + proj_forward_fast(h, self.deq[li]["down_proj"], "down_proj", lo, self.scales, rings)
                continue
            x = x + proj_forward(a, lw["o_proj"], "o_proj", self.ATTN, lo, self.scales, self.rank, rings, mode)
            normed = rmsnorm(x, lw["post_norm"], eps, mode)
            x = x + mlp_forward(normed, lw["gate_proj"], lw["up_proj"], lw["down_proj"], lo, self.scales,
                                self.rank, rings, mode)
        final = rmsnorm(x[-1:], w["norm"], eps, mode)
        return linear_q4(final, *w["lm_head"], mode=mode)[0]


def exp(x: float) -> float:
    return lib().orc_exp(x)


def set_exp(fn_ptr) -> None:
    """Install a C function pointer (double -> double) as the router's exp; None restores libm."""
    lib().orc_set_exp(fn_ptr)


def set_threads(n: int) -> None:
    lib().orc_set_num_threads(n)


def num_threads() -> int:
    return lib().orc_num_threads()
