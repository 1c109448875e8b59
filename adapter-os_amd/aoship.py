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
    "aoship_layer_free": (None, [_P]),
    "aoship_mlp_forward": (C.c_int, [_P, _P, C.c_int, _P, _P]),
    "aoship_proj_forward": (C.c_int, [_P, C.c_char_p, _P, C.c_int, _P, _P]),
    "aoship_qkv_forward": (C.c_int, [_P, _P, C.c_int, _P, _P, _P, _P]),
}

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
        _lib = L
    return _lib


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

    def __init__(self, layer_idx: int = 0):
        h = lib().aoship_layer_new(layer_idx, 64, 4)
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

    def proj_forward(self, module: str, x, rings, y) -> None:
        _check(lib().aoship_proj_forward(self.h, module.encode(), _ptr(x), x.shape[0], _ptr(rings), _ptr(y)),
               "aoship_proj_forward")

    def qkv_forward(self, x, rings, q, k, v) -> None:
        _check(lib().aoship_qkv_forward(self.h, _ptr(x), x.shape[0], _ptr(rings), _ptr(q), _ptr(k), _ptr(v)),
               "aoship_qkv_forward")

    def __del__(self):
        if getattr(self, "h", None) and _lib is not None:
            _lib.aoship_layer_free(self.h)
            self.h = None


def exp_cr(x: float) -> float:
    """Host build of the router's correctly rounded float64 exp (for its pinning test)."""
    return lib().aoship_internal_exp_cr(x)
