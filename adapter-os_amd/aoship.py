"""ctypes binding of libaoship.so (include/aoship.h) for tests and the benchmark.

Device buffers are torch tensors on the HIP device; their data pointers cross the C ABI as plain
pointers. The library must be built (adapter-os_amd/build.py); loading fails loudly otherwise —
there is no CPU fallback.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

import numpy as np

PKG = Path(__file__).resolve().parent
LIB_PATH = PKG / "libaoship.so"

RING_DTYPE = np.dtype(
    [("top_k", "<u4"), ("current_pos", "<u4"), ("adapter_indices", "<u2", (8,)), ("gates_q15", "<i2", (8,))]
)
assert RING_DTYPE.itemsize == 40

# aoship_decision_t: a Decision's entropy and candidates (decision order)
DECISION_DTYPE = np.dtype(
    [("entropy", "<f4"), ("n_candidates", "<u4"), ("adapter_idx", "<u2", (8,)), ("gate_q15", "<i2", (8,)),
     ("raw_score", "<f4", (8,))]
)
assert DECISION_DTYPE.itemsize == 72

MODULES = ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")

# name -> (restype, argtypes)
_P = C.c_void_p
_SIGS = {
    "aoship_get_last_error": (C.c_char_p, []),
    "aoship_clear_error": (None, []),
    "aoship_version": (C.c_char_p, []),
    "aoship_init": (C.c_int, [C.c_int]),
    "aoship_device_name": (C.c_int, [C.c_char_p, C.c_int]),
    "aoship_sync": (C.c_int, []),
    "aoship_attest_determinism": (C.c_int, [C.c_char_p, C.c_int]),
    "aoship_router_new": (_P, [C.c_int, C.c_int, C.c_float, C.c_float, C.c_float, _P]),
    "aoship_router_set_policy_mask": (C.c_int, [_P, _P]),
    "aoship_router_set_stream": (C.c_int, [_P, _P]),
    "aoship_router_set_scope": (C.c_int, [_P, _P]),
    "aoship_router_set_adaptive_seed": (C.c_int, [_P, _P]),
    "aoship_adaptive_tie_breakers": (C.c_int, [_P, C.c_int, _P]),
    "aoship_router_set_decision_policy": (C.c_int, [_P, _P, C.c_int]),
    "aoship_router_set_ring_mapping": (C.c_int, [_P, _P, _P]),
    "aoship_router_set_decision_hashing": (C.c_int, [_P, _P, C.c_int, _P, _P]),
    "aoship_router_set_decision_output": (C.c_int, [_P, _P, C.c_int]),
    "aoship_blake3": (C.c_int, [_P, C.c_size_t, _P]),
    "aoship_router_free": (None, [_P]),
    "aoship_route": (C.c_int, [_P, _P, C.c_int, _P, _P]),
    "aoship_route_features": (C.c_int, [_P, _P, _P, C.c_int, C.c_int, _P, _P, _P]),
    "aoship_lora_adapter_new": (_P, [C.c_int, C.c_int, C.c_float]),
    "aoship_lora_adapter_set_module": (C.c_int, [_P, C.c_int, C.c_char_p, C.c_int, C.c_int, C.c_int, _P, _P]),
    "aoship_lora_adapter_free": (None, [_P]),
    "aoship_layer_new": (_P, [C.c_int, C.c_int, C.c_int]),
    "aoship_layer_set_base": (C.c_int, [_P, C.c_char_p, C.c_int, C.c_int, _P, _P, _P]),
    "aoship_layer_set_adapters": (C.c_int, [_P, _P, C.c_int]),
    "aoship_layer_reserve": (C.c_int, [_P, C.c_int]),
    "aoship_layer_set_stream": (C.c_int, [_P, _P]),
    "aoship_layer_set_profiling": (C.c_int, [_P, C.c_int]),
    "aoship_layer_kernel_stats": (C.c_int, [_P, C.c_int, C.POINTER(C.c_char_p), C.POINTER(C.c_double), C.POINTER(C.c_int64)]),
    "aoship_layer_wait_timeouts": (C.c_int, [_P]),
    "aoship_layer_free": (None, [_P]),
    "aoship_mlp_forward": (C.c_int, [_P, _P, C.c_int, _P, _P]),
    "aoship_liquid_blend_and_forward": (C.c_int, [_P, C.c_int, _P, C.c_int, _P, C.c_int, _P, C.c_int, _P, _P]),
    "aoship_mlp_forward_noalloc": (C.c_int, [_P, _P, C.c_int, _P, _P]),
    "aoship_route_mlp_forward": (C.c_int, [_P, _P, _P, C.c_int, _P, _P, C.c_int, _P, _P, _P]),
    "aoship_proj_forward": (C.c_int, [_P, C.c_char_p, _P, C.c_int, _P, _P]),
    "aoship_qkv_forward": (C.c_int, [_P, _P, C.c_int, _P, _P, _P, _P]),
    "aoship_model_new": (_P, [_P]),
    "aoship_model_free": (None, [_P]),
    "aoship_model_layer": (_P, [_P, C.c_int]),
    "aoship_model_set_embedding": (C.c_int, [_P, _P, _P, _P, _P]),
    "aoship_model_set_lm_head": (C.c_int, [_P, _P, _P, _P]),
    "aoship_model_set_norm": (C.c_int, [_P, C.c_int, C.c_int, _P]),
    "aoship_model_set_bias": (C.c_int, [_P, C.c_int, C.c_char_p, _P]),
    "aoship_model_set_adapters": (C.c_int, [_P, _P, C.c_int]),
    "aoship_model_set_stream": (C.c_int, [_P, _P]),
    "aoship_model_reserve": (C.c_int, [_P, C.c_int]),
    "aoship_model_reset_cache": (C.c_int, [_P]),
    "aoship_model_cache_len": (C.c_int, [_P]),
    "aoship_model_forward": (C.c_int, [_P, _P, C.c_int, C.c_int, _P, _P]),
}


class ModelConfig(C.Structure):
    """aoship_model_config_t"""
    _fields_ = [("num_layers", C.c_int), ("hidden", C.c_int), ("intermediate", C.c_int), ("num_heads", C.c_int),
                ("num_kv_heads", C.c_int), ("head_dim", C.c_int), ("vocab", C.c_int), ("max_seq", C.c_int),
                ("rope_theta", C.c_float), ("rms_eps", C.c_float)]

_lib = None


class AosError(RuntimeError):
    """A C-ABI call returned -1 / NULL; the message is the library's thread-local error text."""


def header_symbols() -> list[str]:
    """Function names declared in include/aoship.h."""
    import re

    text = (PKG.parent / "include" / "aoship.h").read_text()
    return sorted(set(re.findall(r"\b(aoship_[a-z0-9_]+)\s*\(", text)))


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise ImportError(f"{LIB_PATH} is not built: run python adapter-os_amd/build.py")
        L = C.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIGS.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        L.aoship_internal_exp_cr.restype = C.c_double
        L.aoship_internal_exp_cr.argtypes = [C.c_double]
        L.aoship_internal_layer_set_separate_shrinks.restype = C.c_int
        L.aoship_internal_layer_set_separate_shrinks.argtypes = [_P, C.c_int]
        L.aoship_internal_layer_set_decode_handoff.restype = C.c_int
        L.aoship_internal_layer_set_decode_handoff.argtypes = [_P, C.c_int, C.c_int]
        L.aoship_internal_layer_set_plan_pointers.restype = C.c_int
        L.aoship_internal_layer_set_plan_pointers.argtypes = [_P, C.c_int]
        L.aoship_internal_layer_set_prefill_shrink.restype = C.c_int
        L.aoship_internal_layer_set_prefill_shrink.argtypes = [_P, C.c_int]
        L.aoship_internal_layer_set_prefill_sk.restype = C.c_int
        L.aoship_internal_layer_set_prefill_sk.argtypes = [_P, C.c_int]
        L.aoship_internal_layer_last_stream_k.restype = C.c_int
        L.aoship_internal_layer_last_stream_k.argtypes = [_P]
        L.aoship_internal_layer_set_prefill_expand.restype = C.c_int
        L.aoship_internal_layer_set_prefill_expand.argtypes = [_P, C.c_int]
        L.aoship_internal_layer_last_expand.restype = C.c_int
        L.aoship_internal_layer_last_expand.argtypes = [_P]
        L.aoship_internal_layer_set_prefill_adapter_major.restype = C.c_int
        L.aoship_internal_layer_set_prefill_adapter_major.argtypes = [_P, C.c_int]
        L.aoship_internal_layer_set_prefill_expand_adapter_major.restype = C.c_int
        L.aoship_internal_layer_set_prefill_expand_adapter_major.argtypes = [_P, C.c_int]
        L.aoship_internal_layer_last_adapter_major.restype = C.c_int
        L.aoship_internal_layer_last_adapter_major.argtypes = [_P]
        L.aoship_internal_layer_last_perm.restype = C.c_int
        L.aoship_internal_layer_last_perm.argtypes = [_P, _P, C.c_int]
        L.aoship_internal_decode_geometry.restype = C.c_int
        L.aoship_internal_decode_geometry.argtypes = [C.c_int, C.c_int, C.c_int, C.c_int, C.POINTER(C.c_int),
                                                      C.POINTER(C.c_int), C.POINTER(C.c_int), C.POINTER(C.c_int)]
        L.aoship_internal_decode_geometry_pinned.restype = C.c_int
        L.aoship_internal_decode_geometry_pinned.argtypes = [C.c_int] * 6 + [C.POINTER(C.c_int)] * 4
        L.aoship_internal_layer_set_gemv_geometry.restype = C.c_int
        L.aoship_internal_layer_set_gemv_geometry.argtypes = [_P, C.c_int, C.c_int, C.c_int]
        L.aoship_internal_layer_set_mlp1.restype = C.c_int
        L.aoship_internal_layer_set_mlp1.argtypes = [_P, C.c_int]
        L.aoship_internal_set_spin_limit.restype = C.c_int
        L.aoship_internal_set_spin_limit.argtypes = [C.c_uint32]
        _lib = L
    return _lib


def decode_geometry(kind: int, out: int, inp: int, T: int, wr_pin: int = 0, ks_pin: int = 0) -> tuple[int, int, int, int]:
    """(waves, K splits, row blocks per workgroup, fewest K groups of any wave) of a decode launch
    shape (see aoship_internal_decode_geometry), optionally with a GEMV shape pinned as
    Layer.set_gemv_geometry pins it."""
    w, k, r, g = C.c_int(), C.c_int(), C.c_int(), C.c_int()
    _check(lib().aoship_internal_decode_geometry_pinned(kind, out, inp, T, wr_pin, ks_pin, C.byref(w), C.byref(k),
                                                        C.byref(r), C.byref(g)),
           "aoship_internal_decode_geometry")
    return w.value, k.value, r.value, g.value


SPIN_LIMIT_DEFAULT = 1 << 24


def set_spin_limit(polls: int) -> None:
    """Diagnostic: the bound (in polls) of every in-launch wait on the current device; 0 makes every
    wait give up at once (each kernel still ends normally and the layer reports the timeout)."""
    _check(lib().aoship_internal_set_spin_limit(polls), "aoship_internal_set_spin_limit")


def last_error() -> str:
    return lib().aoship_get_last_error().decode()


def _check(rc: int, what: str) -> None:
    if rc != 0:
        raise AosError(f"{what}: {last_error()}")


def _ptr(t) -> int | None:
    if t is None:
        return None
    return t.data_ptr()


_initialised = None


def init(device: int = 0) -> None:
    global _initialised
    if _initialised == device:
        return
    _check(lib().aoship_init(device), "aoship_init")
    _initialised = device


def sync() -> None:
    _check(lib().aoship_sync(), "aoship_sync")


def device_name() -> str:
    buf = C.create_string_buffer(256)
    _check(lib().aoship_device_name(buf, 256), "aoship_device_name")
    return buf.value.decode()


def attest_determinism() -> str:
    n = lib().aoship_attest_determinism(None, 0)
    buf = C.create_string_buffer(n + 1)
    lib().aoship_attest_determinism(buf, n + 1)
    return buf.value.decode()


def _host(a, dtype, n: int):
    if a is None:
        return None
    a = np.ascontiguousarray(np.asarray(a, dtype=dtype))
    if a.shape != (n,):
        raise ValueError(f"expected {n} entries, got shape {a.shape}")
    return a


def _hptr(a):
    return None if a is None else a.ctypes.data


def adaptive_tie_breakers(seed: bytes, n: int) -> np.ndarray:
    """ChaCha20Rng::from_seed(seed).gen::<u64>() x n, computed by the library on the host."""
    sd = np.frombuffer(bytes(seed), dtype=np.uint8).copy()
    if sd.size != 32:
        raise ValueError("the tie-break seed has 32 bytes")
    out = np.zeros(max(n, 1), np.uint64)
    _check(lib().aoship_adaptive_tie_breakers(sd.ctypes.data, n, out.ctypes.data), "aoship_adaptive_tie_breakers")
    return out[:n]


def blake3(data: bytes) -> bytes:
    """B3Hash::hash through the library (host)."""
    buf = C.create_string_buffer(bytes(data), max(len(data), 1))
    out = (C.c_uint8 * 32)()
    _check(lib().aoship_blake3(buf, len(data), out), "aoship_blake3")
    return bytes(out)


def rings_from_bytes(raw: np.ndarray) -> np.ndarray:
    return np.frombuffer(np.ascontiguousarray(raw).tobytes(), dtype=RING_DTYPE)


class Router:
    """Router::new_with_weights + route_with_adapter_info in deterministic mode (C ABI)."""

    def __init__(self, n_adapters: int, k: int, tau: float = 1.0, eps: float = 0.02,
                 routing_bias: float = 1.0, stable_ids=None):
        ids = None
        if stable_ids is not None:
            ids = np.ascontiguousarray(np.asarray(stable_ids, dtype=np.uint64))
        h = lib().aoship_router_new(n_adapters, k, tau, eps, routing_bias,
                                    ids.ctypes.data if ids is not None else None)
        if not h:
            raise AosError(f"aoship_router_new: {last_error()}")
        self.h = h
        self.n = n_adapters

    def set_policy_mask(self, allowed) -> None:
        a = None if allowed is None else np.ascontiguousarray(np.asarray(allowed, dtype=np.uint8))
        _check(lib().aoship_router_set_policy_mask(self.h, a.ctypes.data if a is not None else None),
               "aoship_router_set_policy_mask")

    def set_stream(self, stream_ptr: int | None) -> None:
        _check(lib().aoship_router_set_stream(self.h, stream_ptr), "aoship_router_set_stream")

    def set_scope(self, in_scope) -> None:
        """Scope hint: 1 where the adapter's scope_path equals the hint (None = no hint)."""
        a = _host(in_scope, np.uint8, self.n)
        _check(lib().aoship_router_set_scope(self.h, _hptr(a)), "aoship_router_set_scope")

    def set_adaptive_seed(self, seed: bytes | None) -> None:
        """Adaptive mode with the 32-byte tie-break seed (None = deterministic mode)."""
        a = None if seed is None else np.frombuffer(bytes(seed), dtype=np.uint8).copy()
        if a is not None and a.size != 32:
            raise ValueError("the tie-break seed has 32 bytes")
        _check(lib().aoship_router_set_adaptive_seed(self.h, _hptr(a)), "aoship_router_set_adaptive_seed")

    def set_decision_policy(self, allowed, max_adapters_per_token: int | None = None) -> None:
        """filter_decision_by_policy on every decision (allowed None = no policy)."""
        a = _host(allowed, np.uint8, self.n)
        cap = -1 if max_adapters_per_token is None else int(max_adapters_per_token)
        _check(lib().aoship_router_set_decision_policy(self.h, _hptr(a), cap), "aoship_router_set_decision_policy")

    def set_ring_mapping(self, active_ids=None, strengths=None) -> None:
        """Ring index = active_ids[decision index]; gates scaled by strengths[decision index]."""
        a = _host(active_ids, np.uint16, self.n)
        s = _host(strengths, np.float32, self.n)
        _check(lib().aoship_router_set_ring_mapping(self.h, _hptr(a), _hptr(s)), "aoship_router_set_ring_mapping")

    def set_decision_hashing(self, hashes, reasoning_hash: bytes | None = None,
                             backend_identity_hash: bytes | None = None) -> None:
        """Decision hashes into hashes (a device uint8 tensor of 96 bytes per token; None = off)."""
        cap = 0 if hashes is None else hashes.numel() // 96
        r = None if reasoning_hash is None else np.frombuffer(bytes(reasoning_hash), np.uint8).copy()
        b = None if backend_identity_hash is None else np.frombuffer(bytes(backend_identity_hash), np.uint8).copy()
        for a in (r, b):
            if a is not None and a.size != 32:
                raise ValueError("reasoning / backend identity hashes have 32 bytes")
        self._hashes = hashes  # keep the buffer alive while the router may write it
        _check(lib().aoship_router_set_decision_hashing(self.h, _ptr(hashes), cap, _hptr(r), _hptr(b)),
               "aoship_router_set_decision_hashing")

    def set_decision_output(self, decisions) -> None:
        """Each token's Decision entropy and candidates into decisions (a device uint8 tensor of
        DECISION_DTYPE.itemsize bytes per token, read back with .view(DECISION_DTYPE); None = off)."""
        cap = 0 if decisions is None else decisions.numel() * decisions.element_size() // DECISION_DTYPE.itemsize
        self._decisions = decisions  # keep the buffer alive while the router may write it
        _check(lib().aoship_router_set_decision_output(self.h, _ptr(decisions), cap),
               "aoship_router_set_decision_output")

    def route(self, priors, rings, status=None) -> None:
        T = priors.shape[0]
        _check(lib().aoship_route(self.h, _ptr(priors), T, _ptr(rings), _ptr(status)), "aoship_route")

    def route_features(self, features, router_w, rings, priors_out=None, status=None) -> None:
        T, d = features.shape
        _check(lib().aoship_route_features(self.h, _ptr(features), _ptr(router_w), d, T, _ptr(rings),
                                           _ptr(priors_out), _ptr(status)), "aoship_route_features")

    def __del__(self):
        if getattr(self, "h", None) and _lib is not None:
            _lib.aoship_router_free(self.h)
            self.h = None


class LoraAdapter:
    """mlx_lora_adapter_t counterpart (wrapper.h:375-420)."""

    def __init__(self, adapter_id: int, num_layers: int, scale: float):
        h = lib().aoship_lora_adapter_new(adapter_id, num_layers, scale)
        if not h:
            raise AosError(f"aoship_lora_adapter_new: {last_error()}")
        self.h = h

    def set_module(self, layer_idx: int, module: str, A: np.ndarray, B: np.ndarray) -> None:
        A = np.ascontiguousarray(A, dtype=np.float32)
        B = np.ascontiguousarray(B, dtype=np.float32)
        r, din = A.shape
        dout, r2 = B.shape
        if r2 != r:
            raise ValueError("rank mismatch between A and B")
        _check(lib().aoship_lora_adapter_set_module(self.h, layer_idx, module.encode(), r, din, dout,
                                                    A.ctypes.data, B.ctypes.data),
               "aoship_lora_adapter_set_module")

    def free(self) -> None:
        if getattr(self, "h", None) and _lib is not None:
            _lib.aoship_lora_adapter_free(self.h)
            self.h = None

    def __del__(self):
        self.free()


class Layer:
    """aoship_layer_t: int4 base projections + bound adapter table."""

    def __init__(self, layer_idx: int = 0, handle=None):
        self.owned = handle is None
        h = lib().aoship_layer_new(layer_idx, 64, 4) if handle is None else handle
        if not h:
            raise AosError(f"aoship_layer_new: {last_error()}")
        self.h = h
        self._adapters = []

    def set_base(self, module: str, packed: np.ndarray, scales_f16: np.ndarray, biases_f16=None) -> None:
        packed = np.ascontiguousarray(packed, dtype=np.uint32)
        out, w = packed.shape
        s = np.ascontiguousarray(scales_f16).view(np.uint16)
        b = None if biases_f16 is None else np.ascontiguousarray(biases_f16).view(np.uint16)
        _check(lib().aoship_layer_set_base(self.h, module.encode(), out, w * 8, packed.ctypes.data,
                                           s.ctypes.data, b.ctypes.data if b is not None else None),
               "aoship_layer_set_base")

    def set_adapters(self, adapters) -> None:
        arr = (C.c_void_p * max(1, len(adapters)))(*[a.h if a is not None else None for a in adapters])
        _check(lib().aoship_layer_set_adapters(self.h, arr, len(adapters)), "aoship_layer_set_adapters")
        self._adapters = list(adapters)

    def reserve(self, max_tokens: int) -> None:
        _check(lib().aoship_layer_reserve(self.h, max_tokens), "aoship_layer_reserve")

    def set_stream(self, stream_ptr) -> None:
        _check(lib().aoship_layer_set_stream(self.h, stream_ptr), "aoship_layer_set_stream")

    def set_profiling(self, on: bool) -> None:
        _check(lib().aoship_layer_set_profiling(self.h, 1 if on else 0), "aoship_layer_set_profiling")

    def set_separate_shrinks(self, on: bool) -> None:
        """Diagnostic: each decode LoRA shrink in a launch of its own (default: inside the GEMV
        launch that reads it)."""
        _check(lib().aoship_internal_layer_set_separate_shrinks(self.h, 1 if on else 0),
               "aoship_internal_layer_set_separate_shrinks")

    def set_decode_handoff(self, one_launch: bool, lines: bool) -> None:
        """Diagnostic: the 1-2 token MLP as one launch (default two), and per-producer lines in the
        fused launches (default) instead of an arrival count with one flag per consumer."""
        _check(lib().aoship_internal_layer_set_decode_handoff(self.h, 1 if one_launch else 0, 1 if lines else 0),
               "aoship_internal_layer_set_decode_handoff")

    def set_plan_pointers(self, on: bool) -> None:
        """Diagnostic: decode plans list the LoRA tables' row pointers for their readers (default)
        or the readers look them up through the plan's list; outputs are identical."""
        _check(lib().aoship_internal_layer_set_plan_pointers(self.h, 1 if on else 0),
               "aoship_internal_layer_set_plan_pointers")

    def set_gemv_geometry(self, kind: int, wr: int = 0, ks: int = 0) -> None:
        """Diagnostic: pin the decode GEMV geometry of launch kind 0 (gate/up), 1 (down) or 2
        (projections) to wr row blocks per workgroup and ks K splits (0: automatic)."""
        _check(lib().aoship_internal_layer_set_gemv_geometry(self.h, kind, wr, ks),
               "aoship_internal_layer_set_gemv_geometry")

    def set_mlp1(self, on: bool) -> None:
        """Diagnostic: one token's MLP (and its routing) in one launch with the down matrix held in
        LDS, where the layer's shape fits (off by default: the two-launch decode path is faster so
        far)."""
        _check(lib().aoship_internal_layer_set_mlp1(self.h, 1 if on else 0), "aoship_internal_layer_set_mlp1")

    def set_prefill_sk(self, mask) -> None:
        """Diagnostic: which prefill GEMMs may run as stream-K over the device's resident
        workgroups (bit 0 gate/up, bit 1 down; True = both, the default) where the plan finds it
        pays (no shrink workgroups in the launch, an idle tail in the plain grid), instead of one
        workgroup per task."""
        m = 3 if mask is True else (0 if mask is False else int(mask))
        _check(lib().aoship_internal_layer_set_prefill_sk(self.h, m), "aoship_internal_layer_set_prefill_sk")

    def last_stream_k(self) -> int:
        """Diagnostic: the prefill GEMMs that ran as stream-K in the last prefill MLP (bit 0
        gate/up, bit 1 down)."""
        r = lib().aoship_internal_layer_last_stream_k(self.h)
        if r < 0:
            raise AosError(last_error())
        return r

    def set_prefill_expand(self, cols: int = -1) -> None:
        """Diagnostic: the union width (columns of a tile's wider module) from which the prefill
        MLP's gate/up LoRA expand of a tile runs in an expand launch of its own instead of in the
        SwiGLU GEMM (0: never; negative: the default, 512)."""
        _check(lib().aoship_internal_layer_set_prefill_expand(self.h, int(cols)),
               "aoship_internal_layer_set_prefill_expand")

    def last_expand(self) -> int:
        """Diagnostic: 1 when the last prefill MLP ran the gate/up expand launch."""
        r = lib().aoship_internal_layer_last_expand(self.h)
        if r < 0:
            raise AosError(last_error())
        return r

    def set_prefill_adapter_major(self, tu: int = -1) -> None:
        """Diagnostic: the union size (adapters) from which a prefill tile's LoRA shrinks run
        adapter-major, each adapter's users gathered into tiles of their own (0: never; negative:
        the default)."""
        _check(lib().aoship_internal_layer_set_prefill_adapter_major(self.h, int(tu)),
               "aoship_internal_layer_set_prefill_adapter_major")

    def set_prefill_expand_adapter_major(self, tu: int = -1) -> None:
        """Diagnostic: the union size (adapters) from which a prefill tile's gate/up LoRA expand runs
        adapter-major, its sums added in LDS in adapter order (0: never; negative: the default)."""
        _check(lib().aoship_internal_layer_set_prefill_expand_adapter_major(self.h, int(tu)),
               "aoship_internal_layer_set_prefill_expand_adapter_major")

    def last_adapter_major(self) -> int:
        """Diagnostic: the last prefill MLP's adapter-major launches (bit 0 the x shrink, bit 1 the
        h shrink, bit 2 the gate/up expand)."""
        r = lib().aoship_internal_layer_last_adapter_major(self.h)
        if r < 0:
            raise AosError(last_error())
        return r

    def set_prefill_shrink(self, fused: bool) -> None:
        """Diagnostic: the prefill MLP's LoRA shrinks in the GEMM launches that consume them
        (default) or in launches of their own."""
        _check(lib().aoship_internal_layer_set_prefill_shrink(self.h, 1 if fused else 0),
               "aoship_internal_layer_set_prefill_shrink")

    def last_perm(self):
        """Token order (sorted position -> token) of the last grouped MLP prefill chunk, or None."""
        buf = np.zeros(4096, dtype=np.uint16)
        n = lib().aoship_internal_layer_last_perm(self.h, buf.ctypes.data, buf.size)
        if n < 0:
            raise AosError(last_error())
        return buf[:n].copy() if n else None

    def wait_timeouts(self) -> int:
        """1 if a fused decode launch's bounded wait gave up since the last call (the layer's
        counters and flags are then reset)."""
        r = lib().aoship_layer_wait_timeouts(self.h)
        if r < 0:
            raise AosError(last_error())
        return r

    def kernel_stats(self) -> dict:
        out = {}
        name = C.c_char_p()
        ms = C.c_double()
        n = C.c_int64()
        cnt = lib().aoship_layer_kernel_stats(self.h, -1, None, None, None)
        if cnt < 0:
            raise AosError(last_error())
        for i in range(cnt):
            lib().aoship_layer_kernel_stats(self.h, i, C.byref(name), C.byref(ms), C.byref(n))
            out[name.value.decode()] = (ms.value, n.value)
        return out

    def mlp_forward(self, x, rings, y) -> None:
        _check(lib().aoship_mlp_forward(self.h, _ptr(x), x.shape[0], _ptr(rings), _ptr(y)), "aoship_mlp_forward")

    def mlp_forward_noalloc(self, x, rings, y) -> None:
        """The decode MLP with its workspace in the device's static scratch (no allocation)."""
        _check(lib().aoship_mlp_forward_noalloc(self.h, _ptr(x), x.shape[0], _ptr(rings), _ptr(y)),
               "aoship_mlp_forward_noalloc")

    def route_mlp_forward(self, router, features, router_w, x, rings, y, status=None) -> None:
        """Route the tokens from features (device float32 [T, d]) and run the MLP on them in one
        call; rings (device uint8 [T * 40]) receive the decisions."""
        T, d = features.shape
        _check(lib().aoship_route_mlp_forward(router.h, _ptr(features), _ptr(router_w), d, self.h, _ptr(x), T,
                                              _ptr(rings), None if status is None else _ptr(status), _ptr(y)),
               "aoship_route_mlp_forward")

    def proj_forward(self, module: str, x, rings, y) -> None:
        _check(lib().aoship_proj_forward(self.h, module.encode(), _ptr(x), x.shape[0], _ptr(rings), _ptr(y)),
               "aoship_proj_forward")

    def qkv_forward(self, x, rings, q, k, v) -> None:
        _check(lib().aoship_qkv_forward(self.h, _ptr(x), x.shape[0], _ptr(rings), _ptr(q), _ptr(k), _ptr(v)),
               "aoship_qkv_forward")

    def __del__(self):
        if getattr(self, "h", None) and _lib is not None and getattr(self, "owned", True):
            _lib.aoship_layer_free(self.h)
        self.h = None


class _LiquidTensor(C.Structure):
    _fields_ = [("data", C.c_void_p), ("bf16", C.c_int), ("rows", C.c_int), ("cols", C.c_int), ("len", C.c_size_t)]


class _LiquidAdapter(C.Structure):
    _fields_ = [("id", C.c_uint16), ("down", _LiquidTensor), ("up", _LiquidTensor), ("alpha", C.c_float)]


def _liquid_tensor(t, rows: int | None = None, cols: int | None = None) -> _LiquidTensor:
    """A device tensor (float32, or int16/uint16 holding bfloat16 bits) as a LiquidTensor; rows and
    cols default to its 2-D shape (pass them to describe a buffer whose shape does not match)."""
    import torch

    bf16 = t.dtype in (torch.int16, torch.uint16, torch.bfloat16)
    r = rows if rows is not None else t.shape[0]
    c = cols if cols is not None else (t.shape[1] if t.dim() > 1 else 1)
    return _LiquidTensor(t.data_ptr() if t.numel() else None, 1 if bf16 else 0, r, c, t.numel())


def liquid_blend_and_forward(adapters, coefficients, x, out, stream=None) -> int:
    """LiquidKernel::blend_and_forward: adapters is a list of (down, up, alpha[, id]) with down / up
    device tensors (float32, or bfloat16 bits) or already-built (down, up) LiquidTensor pairs;
    coefficients a host sequence; x and out device float32 vectors. Returns the precision (0 =
    float32, 1 = bfloat16)."""
    n = len(adapters)
    arr = (_LiquidAdapter * max(n, 1))()
    for i, a in enumerate(adapters):
        down, up, alpha = a[0], a[1], a[2]
        aid = a[3] if len(a) > 3 else i
        arr[i].id = aid
        arr[i].down = down if isinstance(down, _LiquidTensor) else _liquid_tensor(down)
        arr[i].up = up if isinstance(up, _LiquidTensor) else _liquid_tensor(up)
        arr[i].alpha = alpha
    cf = np.ascontiguousarray(np.asarray(coefficients, dtype=np.float32))
    prec = C.c_int(-1)
    _check(lib().aoship_liquid_blend_and_forward(C.cast(arr, C.c_void_p), n, cf.ctypes.data if cf.size else None,
                                                 cf.size, _ptr(x), x.numel(), _ptr(out), out.numel(),
                                                 C.byref(prec), stream),
           "aoship_liquid_blend_and_forward")
    return prec.value


def exp_cr(x: float) -> float:
    """Host build of the router's correctly rounded float64 exp (for its pinning test)."""
    return lib().aoship_internal_exp_cr(x)


def _u16(a):
    return None if a is None else np.ascontiguousarray(a).view(np.uint16)


class Model:
    """aoship_model_t: a decoder model over the adapter-augmented layers, with its KV cache
    (mlx_model_forward_with_cache_and_lora)."""

    def __init__(self, num_layers, hidden, intermediate, num_heads, num_kv_heads, head_dim, vocab, max_seq,
                 rope_theta=10000.0, rms_eps=1e-6):
        self.cfg = ModelConfig(num_layers, hidden, intermediate, num_heads, num_kv_heads, head_dim, vocab, max_seq,
                               rope_theta, rms_eps)
        h = lib().aoship_model_new(C.byref(self.cfg))
        if not h:
            raise AosError(f"aoship_model_new: {last_error()}")
        self.h = h
        self.layers = [Layer(i, handle=lib().aoship_model_layer(h, i)) for i in range(num_layers)]
        self._adapters = []

    def set_embedding(self, packed=None, scales_f16=None, biases_f16=None, rows_bf16=None) -> None:
        p = None if packed is None else np.ascontiguousarray(packed, dtype=np.uint32)
        s, b, r = _u16(scales_f16), _u16(biases_f16), _u16(rows_bf16)
        _check(lib().aoship_model_set_embedding(self.h, *[None if a is None else a.ctypes.data for a in (p, s, b, r)]),
               "aoship_model_set_embedding")

    def set_lm_head(self, packed, scales_f16, biases_f16=None) -> None:
        p = np.ascontiguousarray(packed, dtype=np.uint32)
        s, b = _u16(scales_f16), _u16(biases_f16)
        _check(lib().aoship_model_set_lm_head(self.h, p.ctypes.data, s.ctypes.data, None if b is None else b.ctypes.data),
               "aoship_model_set_lm_head")

    def set_norm(self, layer_idx: int, which: int, weight) -> None:
        w = np.ascontiguousarray(weight, dtype=np.float32)
        _check(lib().aoship_model_set_norm(self.h, layer_idx, which, w.ctypes.data), "aoship_model_set_norm")

    def set_bias(self, layer_idx: int, module: str, bias) -> None:
        b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
        _check(lib().aoship_model_set_bias(self.h, layer_idx, module.encode(), None if b is None else b.ctypes.data),
               "aoship_model_set_bias")

    def set_adapters(self, adapters) -> None:
        arr = (C.c_void_p * max(1, len(adapters)))(*[a.h if a is not None else None for a in adapters])
        _check(lib().aoship_model_set_adapters(self.h, arr, len(adapters)), "aoship_model_set_adapters")
        self._adapters = list(adapters)

    def set_stream(self, stream_ptr) -> None:
        _check(lib().aoship_model_set_stream(self.h, stream_ptr), "aoship_model_set_stream")

    def reserve(self, max_tokens: int) -> None:
        _check(lib().aoship_model_reserve(self.h, max_tokens), "aoship_model_reserve")

    def reset_cache(self) -> None:
        _check(lib().aoship_model_reset_cache(self.h), "aoship_model_reset_cache")

    def cache_len(self) -> int:
        return lib().aoship_model_cache_len(self.h)

    def forward(self, ids, rings, logits, position_offset: int | None = None) -> None:
        """ids: device int32 [T]; rings: device uint8 [T * 40]; logits: device float32 [vocab]."""
        T = ids.numel()
        off = self.cache_len() if position_offset is None else position_offset
        _check(lib().aoship_model_forward(self.h, _ptr(ids), T, off, _ptr(rings), _ptr(logits)),
               "aoship_model_forward")

    def __del__(self):
        if getattr(self, "h", None) and _lib is not None:
            for layer in getattr(self, "layers", []):
                layer.h = None
            _lib.aoship_model_free(self.h)
            self.h = None
