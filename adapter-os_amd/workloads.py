"""Seeded synthetic workloads for the adapter-augmented layer (five shapes).

  1  Qwen2.5-0.5B-shaped SwiGLU MLP, hidden 896 / intermediate 4864, 8 adapters of rank 8 on
     gate/up/down, K=2 gates from router features (896-dim) through a router weight; 1 token.
  2  Qwen2.5-7B-shaped MLP, 3584 / 18944, 16 adapters of rank 16, K=4, router over 3584-dim
     features; decode batches of 1 and 8 tokens.
  3  The same layer at a 2048-token prefill; per-token priors put each token on one of 6
     prototype adapter sets (boost 2.0 plus N(0, 0.1) noise), so tokens cluster by adapter set.
  4  Llama-3.2-3B-shaped attention projections, hidden 3072, 24 query / 8 KV heads of 128:
     q 3072->3072, k/v 3072->1024, o 3072->3072; 32 adapters of rank 16 on all four; 32 decode
     streams with their own K=4 rings.
  5  Qwen2.5-32B-shaped MLP, 5120 / 27648, 64 adapters of rank 64, K=8, 4096-token prefill with
     adversarial priors (exact ties, signed zeros, gates near Q15 rounding boundaries with a zero
     entropy floor, one dominant adapter).

Base weights use the MLX 4-bit layout (8 nibbles per uint32, low nibble first, group 64): uniform
nibbles, float16 scales ~ N(0, 0.02) and biases ~ N(0, 0.01). LoRA A ~ N(0, 1/sqrt(in)),
B ~ N(0, 0.01), float32, alpha = rank (scale 1). Activations ~ N(0, 1), rounded to bfloat16.
Every tensor is drawn from its own counter-based stream of libaos_synth.so, seeded with
0xAD0500 + config id, so any prefix of a token range is reproducible on its own.
"""
from __future__ import annotations

import ctypes as C
import math
from dataclasses import dataclass, field
from pathlib import Path

import numpy as np

PKG = Path(__file__).resolve().parent
SYNTH_PATH = PKG / "libaos_synth.so"

_synth = None


def synth():
    global _synth
    if _synth is None:
        if not SYNTH_PATH.exists():
            raise ImportError(f"{SYNTH_PATH} is not built: run python adapter-os_amd/build.py")
        L = C.CDLL(str(SYNTH_PATH))
        L.aos_synth_u32.argtypes = [C.c_uint64, C.c_uint64, C.c_int64, C.c_void_p]
        L.aos_synth_normal.argtypes = [C.c_uint64, C.c_uint64, C.c_int64, C.c_double, C.c_double, C.c_void_p]
        L.aos_synth_randint.argtypes = [C.c_uint64, C.c_uint64, C.c_int64, C.c_uint32, C.c_void_p]
        _synth = L
    return _synth


def u32(seed: int, stream: int, n: int) -> np.ndarray:
    out = np.empty(n, dtype=np.uint32)
    synth().aos_synth_u32(seed, stream, n, out.ctypes.data)
    return out


def normal(seed: int, stream: int, n: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    synth().aos_synth_normal(seed, stream, n, mean, std, out.ctypes.data)
    return out


def randint(seed: int, stream: int, n: int, m: int) -> np.ndarray:
    out = np.empty(n, dtype=np.uint32)
    synth().aos_synth_randint(seed, stream, n, m, out.ctypes.data)
    return out


def f32_to_bf16_bits(a: np.ndarray) -> np.ndarray:
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


MODULE_ID = {"q_proj": 0, "k_proj": 1, "v_proj": 2, "o_proj": 3, "gate_proj": 4, "up_proj": 5, "down_proj": 6}


@dataclass
class Config:
    cid: int
    name: str
    kind: str                     # "mlp" or "attn"
    hidden: int
    inter: int = 0                # mlp intermediate
    q_out: int = 0                # attn
    kv_out: int = 0
    n_adapters: int = 8
    rank: int = 8
    k: int = 2
    tokens: tuple = (1,)
    routing: str = "features"     # features | prototypes | adversarial
    eps: float = 0.02
    tau: float = 1.0
    modules: tuple = field(default=("gate_proj", "up_proj", "down_proj"))

    @property
    def seed(self) -> int:
        return 0xAD0500 + self.cid

    def shape(self, module: str) -> tuple[int, int]:
        """(out_features, in_features) of a module."""
        H = self.hidden
        if self.kind == "mlp":
            return {"gate_proj": (self.inter, H), "up_proj": (self.inter, H), "down_proj": (H, self.inter)}[module]
        return {"q_proj": (self.q_out, H), "k_proj": (self.kv_out, H), "v_proj": (self.kv_out, H),
                "o_proj": (H, self.q_out)}[module]


CONFIGS = {
    1: Config(1, "qwen0.5b-mlp-cpu", "mlp", 896, inter=4864, n_adapters=8, rank=8, k=2, tokens=(1,)),
    2: Config(2, "qwen7b-mlp-decode", "mlp", 3584, inter=18944, n_adapters=16, rank=16, k=4, tokens=(1, 8)),
    3: Config(3, "qwen7b-mlp-prefill", "mlp", 3584, inter=18944, n_adapters=16, rank=16, k=4, tokens=(2048,),
              routing="prototypes"),
    4: Config(4, "llama3b-attn-proj-decode", "attn", 3072, q_out=3072, kv_out=1024, n_adapters=32, rank=16, k=4,
              tokens=(32,), modules=("q_proj", "k_proj", "v_proj", "o_proj")),
    5: Config(5, "qwen32b-mlp-stress", "mlp", 5120, inter=27648, n_adapters=64, rank=64, k=8, tokens=(4096,),
              routing="adversarial", eps=0.0),
}

# stream numbering
S_PACKED, S_SCALE, S_BIAS = 100, 200, 300
S_ROUTER_W, S_FEATURES, S_X, S_PROTO_SETS, S_PROTO_PICK, S_PRIOR_NOISE, S_ADV = 400, 401, 402, 403, 404, 405, 406
S_LORA_A, S_LORA_B = 10000, 20000


def base_weights(cfg: Config, module: str):
    """MLX 4-bit base projection: (packed u32 [out, in/8], scales f16 [out, in/64], biases f16)."""
    out, inp = cfg.shape(module)
    m = MODULE_ID[module]
    packed = u32(cfg.seed, S_PACKED + m, out * inp // 8).reshape(out, inp // 8)
    scales = normal(cfg.seed, S_SCALE + m, out * inp // 64, 0.0, 0.02).astype(np.float16).reshape(out, inp // 64)
    biases = normal(cfg.seed, S_BIAS + m, out * inp // 64, 0.0, 0.01).astype(np.float16).reshape(out, inp // 64)
    return packed, scales, biases


def lora_weights(cfg: Config, adapter: int, module: str):
    """LoRA A [rank, in] and B [out, rank] float32 (MLX shapes)."""
    out, inp = cfg.shape(module)
    m = MODULE_ID[module]
    r = cfg.rank
    A = normal(cfg.seed, S_LORA_A + adapter * 8 + m, r * inp, 0.0, 1.0 / math.sqrt(inp)).reshape(r, inp)
    B = normal(cfg.seed, S_LORA_B + adapter * 8 + m, out * r, 0.0, 0.01).reshape(out, r)
    return A, B


def lora_scale(cfg: Config) -> float:
    return float(np.float32(cfg.rank) / np.float32(cfg.rank))  # alpha / rank with alpha = rank


def activations(cfg: Config, T: int, features_in: int | None = None):
    """x [T, in] as bfloat16 bits and as float32 values (identical numbers)."""
    din = features_in or cfg.hidden
    x = normal(cfg.seed, S_X, T * din, 0.0, 1.0).reshape(T, din)
    bits = f32_to_bf16_bits(x).reshape(T, din)
    return bits, bf16_bits_to_f32(bits).reshape(T, din)


def router_inputs(cfg: Config, T: int):
    """Router features [T, D] and weight [N, D] (routing == "features")."""
    D = cfg.hidden
    f = normal(cfg.seed, S_FEATURES, T * D, 0.0, 1.0).reshape(T, D)
    w = normal(cfg.seed, S_ROUTER_W, cfg.n_adapters * D, 0.0, 0.05).reshape(cfg.n_adapters, D)
    return f, w


def prototype_priors(cfg: Config, T: int, n_sets: int = 6, boost: float = 2.0):
    """Priors that route token t onto one of n_sets prototype K-adapter sets."""
    N, K = cfg.n_adapters, cfg.k
    keys = u32(cfg.seed, S_PROTO_SETS, n_sets * N).reshape(n_sets, N)
    sets = np.argsort(keys, axis=1, kind="stable")[:, :K]
    pick = randint(cfg.seed, S_PROTO_PICK, T, n_sets)
    noise = normal(cfg.seed, S_PRIOR_NOISE, T * N, 0.0, 0.1).reshape(T, N)
    pri = noise.copy()
    for t in range(T):
        pri[t, sets[pick[t]]] += np.float32(boost)
    return pri.astype(np.float32), sets, pick


def adversarial_priors(cfg: Config, T: int):
    """Priors exercising tie-breaks, signed zeros, Q15 rounding boundaries and dominance."""
    N, K = cfg.n_adapters, cfg.k
    base = normal(cfg.seed, S_ADV, T * N, 0.0, 1.0).reshape(T, N)
    pri = np.empty((T, N), dtype=np.float32)
    targets = np.array([0.49, 0.5, 0.5000001, 1.5, 2.5, 1.4999, 3.5], dtype=np.float64)
    for t in range(T):
        kind = t % 4
        b = base[t]
        if kind == 0:  # blocks of exactly equal scores
            pri[t] = np.floor(b * 2.0).astype(np.float32) / np.float32(4.0)
        elif kind == 1:  # signed zeros at the top, everything else negative
            p = -np.abs(b) - np.float32(0.5)
            zs = np.arange(t % 7, N, 5)[: K + 2]
            p[zs[0::2]] = np.float32(-0.0)
            p[zs[1::2]] = np.float32(0.0)
            pri[t] = p
        elif kind == 2:  # gates near Q15 rounding boundaries (eps = 0)
            p = np.full(N, -60.0, dtype=np.float32) + b.astype(np.float32) * np.float32(0.01)
            lead = (t * 7) % N
            p[lead] = np.float32(10.0)
            others = [(lead + 1 + j * 3) % N for j in range(K - 1)]
            for j, a in enumerate(others):
                tg = targets[j % len(targets)] * (1.0 + 1e-7 * (t % 5))
                p[a] = np.float32(10.0 + math.log(tg / 32767.0))
            pri[t] = p
        else:  # one dominant adapter
            p = b.astype(np.float32)
            p[(t * 13) % N] = np.float32(50.0)
            pri[t] = p
    return pri


def priors(cfg: Config, T: int):
    """Priors for the non-feature routings (prototypes / adversarial)."""
    if cfg.routing == "prototypes":
        return prototype_priors(cfg, T)[0]
    if cfg.routing == "adversarial":
        return adversarial_priors(cfg, T)
    raise ValueError("config routes from features")


def algorithmic_bytes(cfg: Config, T: int, distinct_adapters: int) -> int:
    """HBM bytes one layer call must move: int4 base + f16 scale/bias, bf16 LoRA of the distinct
    adapters, bf16 activations in and out."""
    total = 0
    for m in cfg.modules:
        out, inp = cfg.shape(m)
        total += out * inp // 2 + 2 * 2 * out * (inp // 64)
        total += distinct_adapters * cfg.rank * (inp + out) * 2
    if cfg.kind == "mlp":
        total += 2 * T * cfg.hidden * 2
    else:
        total += T * cfg.hidden * 2 * 2 + T * (cfg.q_out + 2 * cfg.kv_out) * 2
    return total


def algorithmic_flops(cfg: Config, T: int) -> int:
    """Multiply-adds counted as 2 FLOP: base GEMM + the K active adapters' shrink and expand."""
    total = 0
    for m in cfg.modules:
        out, inp = cfg.shape(m)
        total += 2 * T * out * inp + 2 * T * cfg.k * cfg.rank * (inp + out)
    return total
