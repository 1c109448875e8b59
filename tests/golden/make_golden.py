"""Writes the small fixtures under tests/golden/.

  router_kats.json     the reference's router known answers, as data (each case cites the test it
                       comes from); expected outputs are the reference's own asserted values.
  router_adversarial.npz
                       64 tokens of the 64-adapter adversarial prior set (exact ties, signed
                       zeros, Q15 rounding boundaries with eps = 0, a dominant adapter) and the
                       oracle's rings for them: a regression vector for the device router.
  c1_layer.npz         the 0.5B-shaped layer (hidden 896, intermediate 4864, 8 rank-8 adapters,
                       K = 2): SHA-256 digests of every generated tensor (pins the synthetic
                       generator), the oracle's rings and float32 MLP outputs for 4 tokens.

Run:  python tests/golden/make_golden.py   (needs oracle/liborc.so and libaos_synth.so built)
"""
from __future__ import annotations

import hashlib
import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
sys.path.insert(0, str(ROOT / "adapter-os_amd"))
sys.path.insert(0, str(ROOT / "oracle"))

ROUTER_KATS = [
    {
        "name": "determinism_rs_38_87_ties_by_stable_id",
        "source": "crates/adapteros-lora-router/tests/determinism.rs:38-87",
        "priors": [0.5, 0.5, 0.5, 0.3, 0.2], "stable_ids": [300, 100, 200, 400, 500],
        "k": 3, "tau": 1.0, "eps": 0.01, "expect_indices": [1, 2, 0], "expect_gates": None,
    },
    {
        "name": "determinism_rs_537_574_score_then_stable_id",
        "source": "crates/adapteros-lora-router/tests/determinism.rs:537-574",
        "priors": [0.9, 0.5, 0.5, 0.5, 0.1], "stable_ids": [10, 200, 100, 300, 400],
        "k": 3, "tau": 1.0, "eps": 0.01, "expect_indices": [0, 2, 1], "expect_gates": None,
    },
    {
        "name": "determinism_rs_908_1090_equal_scores_lowest_index",
        "source": "crates/adapteros-lora-router/tests/determinism.rs:908-966",
        "priors": [0.5] * 8, "stable_ids": [0] * 8,
        "k": 4, "tau": 1.0, "eps": 0.01, "expect_indices": [0, 1, 2, 3], "expect_gates": None,
    },
    {
        "name": "determinism_rs_218_267_floor_and_normalisation",
        "source": "crates/adapteros-lora-router/tests/determinism.rs:218-267",
        "priors": [0.9, 0.8, 0.1, 0.05, 0.02], "stable_ids": [0] * 5,
        "k": 3, "tau": 1.0, "eps": 0.01, "expect_indices": [0, 1, 2], "expect_gates": None,
        "min_gate": 0.01 / 3.0,
    },
    {
        "name": "q15_edge_cases_rs_74_135_masked_single",
        "source": "crates/adapteros-lora-router/tests/q15_edge_cases.rs:74-135",
        "priors": [1.0, 1.0], "stable_ids": [0, 0], "allowed": [1, 0],
        "k": 2, "tau": 1.0, "eps": 0.02, "expect_indices": [0], "expect_gates": [32767],
    },
    {
        "name": "q15_edge_cases_rs_155_192_single_adapter",
        "source": "crates/adapteros-lora-router/tests/q15_edge_cases.rs:155-192",
        "priors": [1.0], "stable_ids": [0],
        "k": 1, "tau": 1.0, "eps": 0.02, "expect_indices": [0], "expect_gates": [32767],
    },
]


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def main() -> None:
    import oracle
    import workloads as W

    (HERE / "router_kats.json").write_text(json.dumps({"cases": ROUTER_KATS}, indent=1) + "\n")

    cfg5 = W.CONFIGS[5]
    pri = W.adversarial_priors(cfg5, 64)
    sid = np.arange(cfg5.n_adapters, dtype=np.uint64)
    rings = oracle.route_batch(pri, cfg5.k, cfg5.tau, cfg5.eps, 1.0, sid)
    np.savez_compressed(HERE / "router_adversarial.npz", priors=pri, rings=rings.view(np.uint8).reshape(64, 40),
                        k=np.int32(cfg5.k), tau=np.float32(cfg5.tau), eps=np.float32(cfg5.eps))

    cfg1 = W.CONFIGS[1]
    T = 4
    digests = {}
    for m in cfg1.modules:
        p, s, b = W.base_weights(cfg1, m)
        digests[f"{m}.packed"] = sha(p)
        digests[f"{m}.scales"] = sha(s)
        digests[f"{m}.biases"] = sha(b)
    for a in range(cfg1.n_adapters):
        for m in cfg1.modules:
            A, B = W.lora_weights(cfg1, a, m)
            digests[f"lora{a}.{m}.A"] = sha(A)
            digests[f"lora{a}.{m}.B"] = sha(B)
    f, w = W.router_inputs(cfg1, T)
    xb, xf = W.activations(cfg1, T)
    digests["router.features"] = sha(f)
    digests["router.weight"] = sha(w)
    digests["x.bf16"] = sha(xb)
    pri1 = oracle.priors(f, w)
    sid1 = np.arange(cfg1.n_adapters, dtype=np.uint64)
    rings1 = oracle.route_batch(pri1, cfg1.k, cfg1.tau, cfg1.eps, 1.0, sid1)
    bw = {m: W.base_weights(cfg1, m) for m in cfg1.modules}
    lora = [{m: W.lora_weights(cfg1, a, m) for m in cfg1.modules} for a in range(cfg1.n_adapters)]
    scales = np.full(cfg1.n_adapters, W.lora_scale(cfg1), np.float32)
    y = oracle.mlp_forward(xf, bw["gate_proj"], bw["up_proj"], bw["down_proj"], lora, scales, cfg1.rank, rings1)
    names = sorted(digests)
    np.savez_compressed(HERE / "c1_layer.npz", digest_names=np.array(names), digests=np.array([digests[n] for n in names]),
                        priors=pri1, rings=rings1.view(np.uint8).reshape(T, 40), y=y)
    print("wrote", [p.name for p in sorted(HERE.iterdir()) if p.suffix in (".json", ".npz")])


if __name__ == "__main__":
    main()
