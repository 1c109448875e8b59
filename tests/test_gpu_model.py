"""GPU parity of the decoder step (aoship_model_forward, the counterpart of
mlx_model_forward_with_cache_and_lora, mlx_cpp_wrapper_real.cpp:3339-3527) against the oracle's
float32 forward (oracle.ModelOracle): a two-layer model with q/k/v biases, GQA and LoRA adapters on
every module, through a prefill, single-token decode steps from the KV cache and a continuation of
more than 32 tokens (the prefill GEMM path), logits within 2e-2 (|ref| + rms(ref)) and within 2e-2
norm-wise, both printed per call; the same calls give bit-identical logits; cache errors are
reported. The Qwen2.5-7B head layout (28 query and 4 key/value heads of 128, hidden 3584,
intermediate 18944, vocabulary 152064) runs through a 512-token prefill and decode past it."""
import numpy as np
import pytest

import oracle
from cases import assert_parity
from test_oracle_model import rings, tiny_model

pytestmark = pytest.mark.gpu

TOL = 2e-2


def _device_model(hip, cfg, w, lora, scales, rank, max_seq):
    m = hip.Model(cfg["num_layers"], cfg["hidden"], cfg["intermediate"], cfg["num_heads"], cfg["num_kv_heads"],
                  cfg["head_dim"], cfg["vocab"], max_seq, cfg["rope_theta"], cfg["rms_eps"])
    m.set_embedding(*w["embed"])
    m.set_lm_head(*w["lm_head"])
    m.set_norm(-1, 0, w["norm"])
    adapters = []
    for a in range(len(scales)):
        ad = hip.LoraAdapter(a, cfg["num_layers"], float(scales[a]))
        for li in range(cfg["num_layers"]):
            for mod, (A, B) in lora[li][a].items():
                ad.set_module(li, mod, A, B)
        adapters.append(ad)
    for li, lw in enumerate(w["layers"]):
        for mod in ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj"):
            m.layers[li].set_base(mod, *lw[mod])
        m.set_norm(li, 0, lw["input_norm"])
        m.set_norm(li, 1, lw["post_norm"])
        for mod, b in lw["bias"].items():
            m.set_bias(li, mod, b)
    m.set_adapters(adapters)
    m._keep = adapters
    return m


def _run(hip, m, ids, rg):
    import torch

    d_ids = torch.from_numpy(np.asarray(ids, np.int32)).cuda()
    d_rings = torch.from_numpy(rg.view(np.uint8).copy()).cuda()
    logits = torch.full((m.cfg.vocab,), float("nan"), dtype=torch.float32, device="cuda")
    m.forward(d_ids, d_rings, logits)
    torch.cuda.synchronize()
    return logits.cpu().numpy()


def test_model_forward_prefill_decode_continuation(hip):
    cfg, w, lora, scales, rank = tiny_model()
    rng = np.random.default_rng(7)
    n = 7 + 3 + 40
    ids = rng.integers(0, cfg["vocab"], n)
    rg = rings(rng, n, len(scales))
    dm = _device_model(hip, cfg, w, lora, scales, rank, max_seq=64)
    om = oracle.ModelOracle(cfg, w, lora, scales, rank)
    spans = [(0, 7), (7, 8), (8, 9), (9, 10), (10, 50)]
    for a, b in spans:
        print(f"span {a}:{b}", flush=True)
        g = _run(hip, dm, ids[a:b], rg[a:b])
        r = om.forward(ids[a:b], rg[a:b])
        assert_parity(f"model span {a}:{b}", g, r, rel_tol=TOL)
        assert dm.cache_len() == b
    # determinism: a fresh cache and the same calls give the same bits
    dm.reset_cache()
    again = [_run(hip, dm, ids[a:b], rg[a:b]) for a, b in spans]
    dm.reset_cache()
    third = [_run(hip, dm, ids[a:b], rg[a:b]) for a, b in spans]
    assert all(np.array_equal(x, y) for x, y in zip(again, third))


def test_model_tied_embeddings_without_biases_or_adapters(hip):
    """A model with no biases and no adapters, the LM head tied to the 4-bit embedding."""
    cfg, w, lora, scales, rank = tiny_model(seed=3, bias=False, n_adapters=1)
    w["lm_head"] = w["embed"]
    rng = np.random.default_rng(8)
    ids = rng.integers(0, cfg["vocab"], 5)
    rg = np.zeros(5, oracle.RING_DTYPE)
    dm = _device_model(hip, cfg, w, lora, scales, rank, max_seq=16)
    dm.set_adapters([])
    om = oracle.ModelOracle(cfg, w, [[{}] for _ in range(cfg["num_layers"])], np.zeros(1, np.float32), rank)
    g = _run(hip, dm, ids, rg)
    assert_parity("model tied embeddings, no biases or adapters", g, om.forward(ids, rg), rel_tol=TOL)


def test_model_cache_errors(hip):
    import torch

    cfg, w, lora, scales, rank = tiny_model(seed=4, n_adapters=1)
    dm = _device_model(hip, cfg, w, lora, scales, rank, max_seq=8)
    ids = torch.zeros(5, dtype=torch.int32, device="cuda")
    rg = torch.zeros(5 * 40, dtype=torch.uint8, device="cuda")
    logits = torch.zeros(cfg["vocab"], dtype=torch.float32, device="cuda")
    dm.forward(ids, rg, logits)
    with pytest.raises(hip.AosError, match="position_offset"):
        dm.forward(ids, rg, logits, position_offset=0)
    with pytest.raises(hip.AosError, match="full"):
        dm.forward(ids, rg, logits)
    torch.cuda.synchronize()


@pytest.mark.parametrize("hd", [32, 128])
def test_model_long_context_attention_splits(hip, hd):
    """Contexts past one 64-position block: the attention runs in several splits whose last wave
    merges them, for a 190-token prefill (the separate RoPE launch), single-token steps (RoPE and
    the cache append inside the attention launch) and a 5-token step; every call against the
    oracle, and the cache written by the single-token steps serves the steps after it."""
    cfg, w, lora, scales, rank = tiny_model(seed=3, hd=hd, bias=True)
    rng = np.random.default_rng(hd)
    spans = [(0, 190), (190, 191), (191, 192), (192, 193), (193, 198), (198, 199)]
    n = spans[-1][1]
    ids = rng.integers(0, cfg["vocab"], n)
    rg = rings(rng, n, len(scales))
    dm = _device_model(hip, cfg, w, lora, scales, rank, max_seq=256)
    om = oracle.ModelOracle(cfg, w, lora, scales, rank)
    for a, b in spans:
        print(f"hd {hd} span {a}:{b}", flush=True)
        g = _run(hip, dm, ids[a:b], rg[a:b])
        r = om.forward(ids[a:b], rg[a:b])
        assert_parity(f"model hd {hd} span {a}:{b}", g, r, rel_tol=TOL)
    dm.reset_cache()
    again = [_run(hip, dm, ids[a:b], rg[a:b]) for a, b in spans]
    dm.reset_cache()
    third = [_run(hip, dm, ids[a:b], rg[a:b]) for a, b in spans]
    assert all(np.array_equal(x, y) for x, y in zip(again, third))
    assert all(layer.wait_timeouts() == 0 for layer in dm.layers)


def test_model_7b_head_layout(hip):
    """Two layers of the Qwen2.5-7B layout (28 query / 4 key-value heads of 128, hidden 3584,
    intermediate 18944, vocabulary 152064, q/k/v biases), 4 rank-16 adapters on every module: a
    512-token prefill, single-token decode steps at positions 512 and 513, a 5-token step and a
    40-token continuation (context 559), each call's logits against the oracle (its float32 BLAS
    path) within 2e-2 element-wise and norm-wise."""
    cfg, w, lora, scales, rank = tiny_model(seed=21, L=2, H=3584, I=18944, nh=28, nkv=4, hd=128, vocab=152064,
                                            n_adapters=4, rank=16)
    rng = np.random.default_rng(5)
    spans = [(0, 512), (512, 513), (513, 514), (514, 519), (519, 559)]
    n = spans[-1][1]
    ids = rng.integers(0, cfg["vocab"], n)
    rg = rings(rng, n, len(scales))
    dm = _device_model(hip, cfg, w, lora, scales, rank, max_seq=576)
    om = oracle.ModelOracle(cfg, w, lora, scales, rank, fast=True)
    for a, b in spans:
        print(f"7B layout span {a}:{b}", flush=True)
        g = _run(hip, dm, ids[a:b], rg[a:b])
        r = om.forward(ids[a:b], rg[a:b])
        assert_parity(f"model 7B layout span {a}:{b}", g, r, rel_tol=TOL)
        assert dm.cache_len() == b
    assert all(layer.wait_timeouts() == 0 for layer in dm.layers)
