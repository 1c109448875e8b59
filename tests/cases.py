"""Shared builders for the parity tests: synthetic layers on the GPU and their oracle twins."""
from __future__ import annotations

import functools

import numpy as np

import workloads as W

# Float outputs must agree with the CPU oracle to 2e-2 relative (bf16): an element passes when
# |gpu - ref| <= 2e-2 * (|ref| + rms(ref)); the rms term keeps outputs near zero from demanding a
# relative precision no bf16 result has.
REL_TOL = 2e-2


def tol_ratio(y, ref) -> float:
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    rms = float(np.sqrt(np.mean(ref * ref)))
    return float(np.max(np.abs(y - ref) / (np.abs(ref) + rms)))


def norm_rel_err(y, ref) -> float:
    """||y - ref|| / ||ref|| over all elements (float64)."""
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.linalg.norm(y - ref) / max(np.linalg.norm(ref), 1e-300))


def report(name: str, y, ref) -> float:
    """Prints the achieved tolerance ratio (max over elements of |y - ref| / (|ref| + rms(ref)),
    which must stay <= REL_TOL) and the norm-wise relative error; returns the ratio."""
    ratio = tol_ratio(y, ref)
    print(f"[parity] {name}: worst tolerance ratio {ratio:.4g} (limit {REL_TOL}), "
          f"norm-wise relative error {norm_rel_err(y, ref):.3g}", flush=True)
    return ratio


# ... and the norm-wise relative error ||y - ref|| / ||ref|| must stay within 2e-2 as well
NORM_TOL = 2e-2


def assert_parity(name: str, y, ref, rel_tol: float = REL_TOL, norm_tol: float = NORM_TOL) -> float:
    """Prints both figures for this case and asserts them (finite outputs, the worst tolerance
    ratio <= rel_tol, the norm-wise relative error <= norm_tol); returns the ratio."""
    y = np.asarray(y, np.float64)
    ratio = tol_ratio(y, ref)
    ne = norm_rel_err(y, ref)
    print(f"[parity] {name}: worst tolerance ratio {ratio:.4g} (limit {rel_tol}), "
          f"norm-wise relative error {ne:.3g} (limit {norm_tol})", flush=True)
    assert np.isfinite(y).all(), f"{name}: non-finite outputs"
    assert ratio <= rel_tol, f"{name}: worst tolerance ratio {ratio:.4g}"
    assert ne <= norm_tol, f"{name}: norm-wise relative error {ne:.3g}"
    return ratio


def tile_sample(perm, T: int, tile: int = 128):
    """Tokens at the first, middle and last sorted position of every tile of the grouped order."""
    pos = []
    for t0 in range(0, T, tile):
        last = min(t0 + tile, T) - 1
        pos += [t0, (t0 + last) // 2, last]
    return np.unique(np.asarray(perm)[np.asarray(pos)])


def adapter_sets(rings, n_adapters: int):
    """Each token's active adapter set (prepare_lora_for_ring's rule: slot < top_k, q > 0, index
    < n), as a frozenset."""
    out = []
    for r in rings:
        k = int(r["top_k"])
        out.append(frozenset(int(r["adapter_indices"][s]) for s in range(min(k, 8))
                             if r["gates_q15"][s] > 0 and r["adapter_indices"][s] < n_adapters))
    return out


def check_grouping(perm, rings, n_adapters: int):
    """The grouped order is a permutation in which the tokens of each adapter set are contiguous
    and ascending (the sort's tie-break)."""
    T = len(rings)
    assert sorted(int(t) for t in perm) == list(range(T)), "not a permutation"
    sets = adapter_sets(rings, n_adapters)
    seq = [sets[int(t)] for t in perm]
    runs = 1 + sum(1 for a, b in zip(seq, seq[1:]) if a != b)
    assert runs == len(set(sets)), f"{len(set(sets))} adapter sets in {runs} runs"
    for a, b in zip(perm, perm[1:]):
        if sets[int(a)] == sets[int(b)]:
            assert int(a) < int(b), "tokens of one set out of order"


@functools.lru_cache(maxsize=4)
def base(cid: int):
    cfg = W.CONFIGS[cid]
    return {m: W.base_weights(cfg, m) for m in cfg.modules}


@functools.lru_cache(maxsize=4)
def lora(cid: int):
    cfg = W.CONFIGS[cid]
    return [{m: W.lora_weights(cfg, a, m) for m in cfg.modules} for a in range(cfg.n_adapters)]


def rings_for(cid: int, T: int):
    """Oracle rings for T tokens of config cid (and the priors that produced them)."""
    import oracle

    cfg = W.CONFIGS[cid]
    if cfg.routing == "features":
        f, w = W.router_inputs(cfg, T)
        pri = oracle.priors(f, w)
    else:
        pri = W.priors(cfg, T)
    sid = np.arange(cfg.n_adapters, dtype=np.uint64)
    rings = oracle.route_batch(pri, cfg.k, cfg.tau, cfg.eps, 1.0, sid)
    return rings, pri


def gpu_layer(aoship, cid: int):
    cfg = W.CONFIGS[cid]
    layer = aoship.Layer(0)
    for m, (p, s, b) in base(cid).items():
        layer.set_base(m, p, s, b)
    ads = []
    for a, mods in enumerate(lora(cid)):
        ad = aoship.LoraAdapter(a, 1, W.lora_scale(cfg))
        for m, (A, B) in mods.items():
            ad.set_module(0, m, A, B)
        ads.append(ad)
    layer.set_adapters(ads)
    return layer, ads


def oracle_mlp(cid: int, x, rings, mode=0):
    import oracle

    cfg = W.CONFIGS[cid]
    bw = base(cid)
    scales = np.full(cfg.n_adapters, W.lora_scale(cfg), np.float32)
    return oracle.mlp_forward(x, bw["gate_proj"], bw["up_proj"], bw["down_proj"], lora(cid), scales, cfg.rank,
                              rings, mode)


def oracle_proj(cid: int, module: str, x, rings, mode=0):
    import oracle

    cfg = W.CONFIGS[cid]
    scales = np.full(cfg.n_adapters, W.lora_scale(cfg), np.float32)
    return oracle.proj_forward(x, base(cid)[module], module, list(cfg.modules), lora(cid), scales, cfg.rank, rings,
                               mode)
