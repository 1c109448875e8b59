"""GPU layer parity: the int4 + LoRA layer kernels against the CPU oracle.

Tolerance (from the workload definition): every output element within 2e-2 relative of the
oracle, |gpu - ref| <= 2e-2 * (|ref| + rms(ref)). Run-to-run results must be bit-identical.
"""
import numpy as np
import pytest

import workloads as W
from cases import REL_TOL, assert_parity, check_grouping, gpu_layer, oracle_mlp, oracle_proj, report, rings_for, tile_sample, tol_ratio

pytestmark = pytest.mark.gpu


def _dev(a, dtype=None):
    import torch

    t = torch.from_numpy(np.ascontiguousarray(a))
    return t.cuda()


def _run_mlp(hip, layer, xb, rings):
    import torch

    T, H = xb.shape
    x = _dev(xb.view(np.int16))
    r = _dev(rings.view(np.uint8))
    y = torch.empty((T, H), dtype=torch.int16, device="cuda")
    layer.mlp_forward(x, r, y)
    torch.cuda.synchronize()
    return y.cpu().numpy().view(np.uint16)


@pytest.mark.parametrize("cid,T", [(1, 1), (2, 1), (2, 2), (2, 8), (2, 31), (2, 32)])
def test_mlp_decode_parity(hip, cid, T):
    xb, xf = W.activations(W.CONFIGS[cid], T)
    rings, _ = rings_for(cid, T)
    layer, ads = gpu_layer(hip, cid)
    y1 = _run_mlp(hip, layer, xb, rings)
    y2 = _run_mlp(hip, layer, xb, rings)
    assert layer.wait_timeouts() == 0
    assert np.array_equal(y1, y2), "run-to-run outputs differ"
    ref = oracle_mlp(cid, xf, rings)
    ratio = assert_parity(f"test_mlp_decode_parity cid={cid} T={T}", W.bf16_bits_to_f32(y1).reshape(ref.shape), ref)
    assert ratio <= REL_TOL, f"max tolerance ratio {ratio:.4g}"


@pytest.mark.parametrize("T", [1, 8])
def test_mlp_decode_unfused_launches(hip, T):
    """The decode MLP with each shrink in a launch of its own instead of in the first workgroups
    of the GEMV launch that reads it: the same tolerance, bit-identical run to run, and the fused
    path afterwards still matches its own earlier output."""
    cid = 2
    xb, xf = W.activations(W.CONFIGS[cid], T)
    rings, _ = rings_for(cid, T)
    layer, ads = gpu_layer(hip, cid)
    fused = _run_mlp(hip, layer, xb, rings)
    layer.set_separate_shrinks(True)
    y1 = _run_mlp(hip, layer, xb, rings)
    y2 = _run_mlp(hip, layer, xb, rings)
    layer.set_separate_shrinks(False)
    assert np.array_equal(y1, y2), "run-to-run outputs differ"
    ref = oracle_mlp(cid, xf, rings)
    assert_parity(f"test_mlp_decode_unfused_launches T={T}", W.bf16_bits_to_f32(y1).reshape(ref.shape), ref)
    assert np.array_equal(_run_mlp(hip, layer, xb, rings), fused)


@pytest.mark.parametrize("one_launch,lines", [(True, True), (True, False), (False, False)])
@pytest.mark.parametrize("T", [1, 2, 8])
def test_mlp_decode_handoff_variants(hip, T, one_launch, lines):
    """The decode MLP with the other in-launch hand-offs: the 1-2 token MLP as one launch (gate/up
    row blocks hand h to the down GEMV workgroups of the same grid), and the counted hand-off (the
    producers count in, the last raises one flag per consumer) instead of per-producer lines. Each
    is bit-identical run to run, within the tolerance, and leaves no timed-out wait; the default
    afterwards reproduces its own earlier output."""
    cid = 2
    xb, xf = W.activations(W.CONFIGS[cid], T)
    rings, _ = rings_for(cid, T)
    layer, ads = gpu_layer(hip, cid)
    default = _run_mlp(hip, layer, xb, rings)
    layer.set_decode_handoff(one_launch, lines)
    y1 = _run_mlp(hip, layer, xb, rings)
    y2 = _run_mlp(hip, layer, xb, rings)
    layer.set_decode_handoff(False, True)
    assert layer.wait_timeouts() == 0
    assert np.array_equal(y1, y2), "run-to-run outputs differ"
    ref = oracle_mlp(cid, xf, rings)
    assert_parity(f"test_mlp_decode_handoff_variants T={T} one_launch={one_launch} lines={lines}", W.bf16_bits_to_f32(y1).reshape(ref.shape), ref)
    assert np.array_equal(_run_mlp(hip, layer, xb, rings), default)


@pytest.mark.parametrize("T", [1, 2, 8, 32])
def test_decode_plan_pointer_lists(hip, T):
    """The decode plan lists the union's row pointers in the LoRA tables (default), so a fused
    launch's first expand step loads in two round trips after its wait; without the lists each
    reader looks the pointers up through the plan's adapter list. Only the order of the loads
    changes: the MLP and the q/k/v and o projections are identical either way, within tolerance of
    the oracle, and leave no timed-out wait."""
    import torch

    cid = 2
    xb, xf = W.activations(W.CONFIGS[cid], T)
    rings, _ = rings_for(cid, T)
    layer, ads = gpu_layer(hip, cid)
    on = _run_mlp(hip, layer, xb, rings)
    layer.set_plan_pointers(False)
    off = _run_mlp(hip, layer, xb, rings)
    layer.set_plan_pointers(True)
    assert layer.wait_timeouts() == 0
    assert np.array_equal(on, off), "MLP outputs differ with and without the plan's pointer lists"
    ref = oracle_mlp(cid, xf, rings)
    assert_parity(f"test_decode_plan_pointer_lists T={T}", W.bf16_bits_to_f32(on).reshape(ref.shape), ref)

    cid = 4
    cfg = W.CONFIGS[cid]
    xb, xf = W.activations(cfg, T)
    rings, _ = rings_for(cid, T)
    layer, ads = gpu_layer(hip, cid)
    x = _dev(xb.view(np.int16))
    r = _dev(rings.view(np.uint8))
    outs = []
    for lists in (True, False):
        layer.set_plan_pointers(lists)
        q = torch.empty((T, cfg.q_out), dtype=torch.int16, device="cuda")
        k = torch.empty((T, cfg.kv_out), dtype=torch.int16, device="cuda")
        v = torch.empty((T, cfg.kv_out), dtype=torch.int16, device="cuda")
        o = torch.empty((T, cfg.hidden), dtype=torch.int16, device="cuda")
        layer.qkv_forward(x, r, q, k, v)
        layer.proj_forward("o_proj", x, r, o)
        torch.cuda.synchronize()
        outs.append([t.cpu().numpy().view(np.uint16) for t in (q, k, v, o)])
    layer.set_plan_pointers(True)
    assert layer.wait_timeouts() == 0
    for name, a, b in zip(cfg.modules, outs[0], outs[1]):
        assert np.array_equal(a, b), f"{name}: outputs differ with and without the plan's pointer lists"
        ref = oracle_proj(cid, name, xf, rings)
        assert_parity(f"test_decode_plan_pointer_lists T={T} {name}", W.bf16_bits_to_f32(a).reshape(ref.shape), ref)


def test_mlp_no_adapters_matches_base(hip):
    """Zero gates / empty rings: the layer is the plain int4 SwiGLU MLP."""
    cid, T = 1, 4
    xb, xf = W.activations(W.CONFIGS[cid], T)
    rings = np.zeros(T, dtype=hip.RING_DTYPE)
    layer, ads = gpu_layer(hip, cid)
    y = _run_mlp(hip, layer, xb, rings)
    ref = oracle_mlp(cid, xf, rings)
    assert_parity(f"test_mlp_no_adapters_matches_base", W.bf16_bits_to_f32(y).reshape(ref.shape), ref)


@pytest.mark.parametrize("T", [1, 8, 40])
def test_mlp_without_bound_adapters(hip, T):
    """A layer with no adapter bound at all (decode and prefill paths): the plain int4 SwiGLU MLP,
    whatever the rings say."""
    cid = 1
    xb, xf = W.activations(W.CONFIGS[cid], T)
    rings, _ = rings_for(cid, T)
    layer, ads = gpu_layer(hip, cid)
    layer.set_adapters([])
    y = _run_mlp(hip, layer, xb, rings)
    ref = oracle_mlp(cid, xf, np.zeros(T, dtype=hip.RING_DTYPE))
    assert_parity(f"test_mlp_without_bound_adapters T={T}", W.bf16_bits_to_f32(y).reshape(ref.shape), ref)


def test_mlp_prefill_shape_parity(hip):
    """2048-token prefill of the 7B-shaped layer (matrix-core GEMM path): the tokens are grouped by
    adapter set (each set contiguous, ascending within it); the first, middle and last token of
    every 128-token tile of the grouped order, and the first and last tokens, are checked against
    the oracle; bit-identical run to run."""
    cid, T = 3, 2048
    xb, xf = W.activations(W.CONFIGS[cid], T)
    rings, _ = rings_for(cid, T)
    layer, ads = gpu_layer(hip, cid)
    y = _run_mlp(hip, layer, xb, rings)
    perm = layer.last_perm()
    y2 = _run_mlp(hip, layer, xb, rings)
    assert np.array_equal(y, y2), "run-to-run outputs differ"
    check_grouping(perm, rings, W.CONFIGS[cid].n_adapters)
    sample = np.union1d(tile_sample(perm, T), [0, 1, T - 2, T - 1])
    assert len(np.unique(np.argsort(perm)[sample] // 128)) == T // 128  # a token of every tile
    ref = oracle_mlp(cid, xf[sample], rings[sample])
    got = W.bf16_bits_to_f32(y.reshape(T, -1)[sample])
    assert_parity(f"C3 prefill T={T}, {len(sample)} tokens over {T // 128} tiles", got, ref)


def test_mlp_stress_32b_prefill(hip):
    """Qwen2.5-32B-shaped stress layer: 4096 tokens, 64 rank-64 adapters on gate/up/down, K = 8
    with adversarial routing (ties, signed zeros, Q15 rounding boundaries, a dominant adapter).
    Device-routed rings equal the oracle's; outputs within tolerance on a sample of tokens across
    tiles; bit-identical run to run."""
    import torch

    cid, T = 5, 4096
    cfg = W.CONFIGS[cid]
    rings, pri = rings_for(cid, T)
    router = hip.Router(cfg.n_adapters, cfg.k, cfg.tau, cfg.eps, 1.0, np.arange(cfg.n_adapters, dtype=np.uint64))
    rdev = torch.zeros(T * 40, dtype=torch.uint8, device="cuda")
    router.route(_dev(pri), rdev)
    torch.cuda.synchronize()
    assert rdev.cpu().numpy().tobytes() == rings.view(np.uint8).tobytes()
    xb, xf = W.activations(cfg, T)
    layer, ads = gpu_layer(hip, cid)
    x = _dev(xb.view(np.int16))
    y1 = torch.empty((T, cfg.hidden), dtype=torch.int16, device="cuda")
    y2 = torch.empty_like(y1)
    layer.mlp_forward(x, rdev, y1)
    perm = layer.last_perm()
    assert layer.last_expand() == 1, "the wide unions' gate/up expand did not run as its own launch"
    layer.mlp_forward(x, rdev, y2)
    torch.cuda.synchronize()
    assert torch.equal(y1, y2), "run-to-run outputs differ"
    check_grouping(perm, rings, cfg.n_adapters)
    sample = np.union1d(tile_sample(perm, T), [0, 1, T - 2, T - 1])
    ref = oracle_mlp(cid, xf[sample], rings[sample])
    got = W.bf16_bits_to_f32(y1.cpu().numpy().view(np.uint16)[sample])
    ratio = assert_parity(f"C5 prefill T={T}, {len(sample)} tokens over {T // 128} tiles", got, ref)
    assert ratio <= REL_TOL, f"max tolerance ratio {ratio:.4g}"


@pytest.mark.parametrize("T", [1024, 1100])
def test_mlp_prefill_expand_launch(hip, T):
    """The gate/up LoRA expand of wide tile unions as a launch of its own, whose sums the SwiGLU
    GEMM adds before the activation (32B-shaped stress layer, 64 rank-64 adapters, K = 8,
    adversarial routing; 1024 tokens in 8 tiles, and 1100 in 9 with a ragged last tile and the
    GEMMs as stream-K): for every tile (the default width, 512 columns), for none (0), and for
    the tiles of 50 adapters or more (3200 columns: the tiles of tokens with random adapter sets
    hold 63-64, the others 31-42, so that both forms meet in one GEMM launch).
    Each form is bit-identical run to run and within tolerance of the oracle on every tile; the
    forms agree with each other up to float32 summation order."""
    cid = 5
    cfg = W.CONFIGS[cid]
    xb, xf = W.activations(cfg, T)
    rings, _ = rings_for(cid, T)
    layer, ads = gpu_layer(hip, cid)
    layer.set_prefill_shrink(False)
    out = {}
    for cols in (-1, 0, 50 * cfg.rank):
        layer.set_prefill_expand(cols)
        y = _run_mlp(hip, layer, xb, rings)
        assert layer.last_expand() == (0 if cols == 0 else 1), f"cols={cols}: expand launch state"
        assert np.array_equal(y, _run_mlp(hip, layer, xb, rings)), f"cols={cols}: run-to-run outputs differ"
        out[cols] = W.bf16_bits_to_f32(y).reshape(T, -1)
    layer.set_prefill_expand(-1)
    perm = layer.last_perm()
    sample = np.union1d(tile_sample(perm, T), [0, 1, T - 2, T - 1])
    ref = oracle_mlp(cid, xf[sample], rings[sample])
    for cols, y in out.items():
        ratio = assert_parity(f"C5 prefill T={T} expand width {cols}", y[sample], ref)
        assert ratio <= REL_TOL, f"cols={cols}: max tolerance ratio {ratio:.4g}"
    assert tol_ratio(out[-1], out[0]) <= REL_TOL / 2
    assert tol_ratio(out[50 * cfg.rank], out[0]) <= REL_TOL / 2


@pytest.mark.parametrize("cid,T,mixed", [(5, 1024, 50), (5, 1100, 50), (3, 2048, 6), (1, 300, 4)])
def test_mlp_prefill_adapter_major(hip, cid, T, mixed):
    """The prefill LoRA shrinks adapter-major (each adapter's users gathered into tiles of their
    own, K split into slices whose sums add in slice order) for no tile (0), every tile (1) and the
    tiles whose union holds at least `mixed` adapters, so that both forms meet in one call: on the
    32B-shaped stress layer (64 rank-64 adapters, K = 8, adversarial routing; a ragged last tile at
    1100 tokens), the 7B-shaped layer (rank 16, clustered) and the 0.5B-shaped one (rank 8, padded
    to 16). Each form is bit-identical run to run and within tolerance of the oracle on every
    tile; the forms agree with each other up to float32 summation order."""
    cfg = W.CONFIGS[cid]
    xb, xf = W.activations(cfg, T)
    rings, _ = rings_for(cid, T)
    layer, ads = gpu_layer(hip, cid)
    layer.set_prefill_shrink(False)
    out = {}
    for tu in (0, 1, mixed):
        layer.set_prefill_adapter_major(tu)
        y = _run_mlp(hip, layer, xb, rings)
        assert layer.last_adapter_major() & 3 == (3 if tu else 0), f"tu={tu}: adapter-major state"
        assert np.array_equal(y, _run_mlp(hip, layer, xb, rings)), f"tu={tu}: run-to-run outputs differ"
        out[tu] = W.bf16_bits_to_f32(y).reshape(T, -1)
    layer.set_prefill_adapter_major(-1)
    perm = layer.last_perm()
    sample = np.union1d(tile_sample(perm, T), [0, 1, T - 2, T - 1])
    ref = oracle_mlp(cid, xf[sample], rings[sample])
    for tu, y in out.items():
        ratio = assert_parity(f"config {cid} prefill T={T} adapter-major from {tu}", y[sample], ref)
        assert ratio <= REL_TOL, f"tu={tu}: max tolerance ratio {ratio:.4g}"
    assert tol_ratio(out[1], out[0]) <= REL_TOL / 2
    assert tol_ratio(out[mixed], out[0]) <= REL_TOL / 2


@pytest.mark.parametrize("cid,T,xe_cols,am_tu,forms",
                         [(5, 1024, -1, -1, (0, 8, 50)), (5, 1100, -1, -1, (0, 8, 50)), (3, 2048, 64, 1, (0, 4, 6)),
                          (1, 300, 32, 1, (0, 2, 3))])
def test_mlp_prefill_expand_adapter_major(hip, cid, T, xe_cols, am_tu, forms):
    """The gate/up LoRA expand adapter-major (each adapter's users gathered into MFMA tiles against
    its B rows, the sums of a range of 4 tiles added in LDS in adapter order) for no tile, every
    expand-launch tile, and the tiles whose union holds at least forms[2] adapters, the others
    expanded over their unions in the same call (a tile expands adapter-major only if it is an
    expand-launch tile: union columns of the wider module >= the launch's width): on the 32B-shaped stress layer (64 rank-64
    adapters, K = 8, adversarial routing; 1024 tokens, and 1100 with a ragged last tile), the
    7B-shaped layer (rank 16) and the 0.5B-shaped one (rank 8 padded to 16), the last two with the
    expand launch from 64 and 32 union columns. Each form is bit-identical run to run and within
    tolerance of the oracle on every tile; the forms agree up to float32 summation order."""
    cfg = W.CONFIGS[cid]
    xb, xf = W.activations(cfg, T)
    rings, _ = rings_for(cid, T)
    layer, ads = gpu_layer(hip, cid)
    layer.set_prefill_shrink(False)
    layer.set_prefill_expand(xe_cols)
    layer.set_prefill_adapter_major(am_tu)
    out = {}
    for tu in forms:
        layer.set_prefill_expand_adapter_major(tu)
        y = _run_mlp(hip, layer, xb, rings)
        assert layer.last_expand() == 1, f"tu={tu}: expand launch state"
        assert layer.last_adapter_major() == (7 if tu else 3), f"tu={tu}: adapter-major state"
        assert np.array_equal(y, _run_mlp(hip, layer, xb, rings)), f"tu={tu}: run-to-run outputs differ"
        out[tu] = W.bf16_bits_to_f32(y).reshape(T, -1)
    layer.set_prefill_expand_adapter_major(-1)
    layer.set_prefill_adapter_major(-1)
    layer.set_prefill_expand(-1)
    perm = layer.last_perm()
    sample = np.union1d(tile_sample(perm, T), [0, 1, T - 2, T - 1])
    ref = oracle_mlp(cid, xf[sample], rings[sample])
    for tu, y in out.items():
        ratio = assert_parity(f"config {cid} prefill T={T} expand adapter-major from {tu}", y[sample], ref)
        assert ratio <= REL_TOL, f"tu={tu}: max tolerance ratio {ratio:.4g}"
    assert tol_ratio(out[forms[1]], out[0]) <= REL_TOL / 2
    assert tol_ratio(out[forms[2]], out[0]) <= REL_TOL / 2


@pytest.mark.parametrize("cid,T", [(1, 300), (3, 2048)])
def test_mlp_prefill_shrink_modes(hip, cid, T):
    """The prefill LoRA shrinks as the first workgroups of the GEMM launches (default) and as
    launches of their own with K split into slices: both within tolerance of the oracle, each
    bit-identical run to run, and equal to each other up to float32 summation order."""
    xb, xf = W.activations(W.CONFIGS[cid], T)
    rings, _ = rings_for(cid, T)
    layer, ads = gpu_layer(hip, cid)
    out = {}
    for fused in (True, False):
        layer.set_prefill_shrink(fused)
        y = _run_mlp(hip, layer, xb, rings)
        assert np.array_equal(y, _run_mlp(hip, layer, xb, rings)), f"fused={fused}: run-to-run outputs differ"
        out[fused] = W.bf16_bits_to_f32(y).reshape(T, -1)
    layer.set_prefill_shrink(True)
    perm = layer.last_perm()
    sample = np.arange(T) if T <= 300 else np.union1d(tile_sample(perm, T), [0, 1, T - 2, T - 1])
    ref = oracle_mlp(cid, xf[sample], rings[sample])
    for fused in (True, False):
        ratio = assert_parity(f"C{cid} prefill T={T} shrink fused={fused}", out[fused][sample], ref)
        assert ratio <= REL_TOL, f"fused={fused}: max tolerance ratio {ratio:.4g}"
    # float32 order changes flip some bf16 roundings of SA and h: a small fraction of the
    # tolerance (a wrong column or adapter would give ratios near 1)
    assert tol_ratio(out[True], out[False]) <= REL_TOL / 2


@pytest.mark.parametrize("case", ["unfused_shrink", "ragged", "no_adapters"])
def test_mlp_prefill_stream_k(hip, case):
    """The prefill GEMMs as stream-K: the device's resident workgroups share the (token tile, row
    block) tasks' K groups evenly; a task cut between workgroups is finished by its owner, which
    adds the other pieces' partial sums in order. 7B-shaped layer with the shrinks in launches of
    their own at 1500 and 1100 tokens, and without adapters at 1500 (12 and 9 token tiles: not a
    multiple of 8, so both GEMMs then run as stream-K by default; the last round of the plain grid
    would be partly idle): both GEMMs ran as stream-K, the outputs are bit-identical run to run,
    within tolerance of the oracle on every tile, no wait timed out, and equal to the one-task-per-
    workgroup GEMMs up to float32 summation order."""
    cid = 3
    T = 1100 if case == "ragged" else 1500
    xb, xf = W.activations(W.CONFIGS[cid], T)
    rings, _ = rings_for(cid, T)
    layer, ads = gpu_layer(hip, cid)
    if case == "no_adapters":
        layer.set_adapters([])
        rings_ref = np.zeros(T, dtype=hip.RING_DTYPE)
    else:
        layer.set_prefill_shrink(False)
        rings_ref = rings
    y = _run_mlp(hip, layer, xb, rings)
    assert layer.last_stream_k() == 3, "the prefill GEMMs did not run as stream-K"
    assert np.array_equal(y, _run_mlp(hip, layer, xb, rings)), "run-to-run outputs differ"
    assert layer.wait_timeouts() == 0
    perm = layer.last_perm() if case != "no_adapters" else np.arange(T)
    layer.set_prefill_sk(False)
    y_plain = _run_mlp(hip, layer, xb, rings)
    assert layer.last_stream_k() == 0
    layer.set_prefill_sk(True)
    sample = np.union1d(tile_sample(perm, T), [0, 1, T - 2, T - 1])
    ref = oracle_mlp(cid, xf[sample], rings_ref[sample])
    got = W.bf16_bits_to_f32(y.reshape(T, -1)[sample])
    assert_parity(f"C3 prefill stream-K {case} T={T}, {len(sample)} tokens", got, ref)
    a, b = W.bf16_bits_to_f32(y).reshape(T, -1), W.bf16_bits_to_f32(y_plain).reshape(T, -1)
    assert tol_ratio(a, b) <= REL_TOL / 2


@pytest.mark.parametrize("T", [33, 100, 128, 129, 300])
def test_mlp_prefill_ragged_full_parity(hip, T):
    """Prefill path at token counts around the 128-token tile (0.5B-shaped layer, every token
    checked)."""
    cid = 1
    xb, xf = W.activations(W.CONFIGS[cid], T)
    rings, _ = rings_for(cid, T)
    layer, ads = gpu_layer(hip, cid)
    y = _run_mlp(hip, layer, xb, rings)
    ref = oracle_mlp(cid, xf, rings)
    ratio = assert_parity(f"test_mlp_prefill_ragged_full_parity T={T}", W.bf16_bits_to_f32(y).reshape(ref.shape), ref)
    assert ratio <= REL_TOL, f"max tolerance ratio {ratio:.4g}"


def test_mlp_prefill_mixed_rings(hip):
    """Prefill with empty rings, zero gates and out-of-table indices mixed in: those slots add
    nothing (backend.rs:409-425)."""
    cid, T = 1, 160
    cfg = W.CONFIGS[cid]
    xb, xf = W.activations(cfg, T)
    rings, _ = rings_for(cid, T)
    rings = rings.copy()
    rings[5:40] = np.zeros(35, dtype=rings.dtype)
    rings["gates_q15"][50:60, 0] = 0
    rings["adapter_indices"][70:80, 1] = 999
    layer, ads = gpu_layer(hip, cid)
    y = _run_mlp(hip, layer, xb, rings)
    ref = oracle_mlp(cid, xf, rings)
    assert_parity(f"test_mlp_prefill_mixed_rings", W.bf16_bits_to_f32(y).reshape(ref.shape), ref)


@pytest.mark.parametrize("T", [5, 160])
def test_mlp_rings_naming_an_adapter_twice(hip, T):
    """A ring may name one adapter in two slots: both gates apply (the plan sums the two
    coefficients in ring order), on the decode and the prefill path."""
    cid = 1
    cfg = W.CONFIGS[cid]
    xb, xf = W.activations(cfg, T)
    rings, _ = rings_for(cid, T)
    rings = rings.copy()
    rng = np.random.default_rng(T)
    for t in range(0, T, 2):
        rings["top_k"][t] = 3
        a = int(rng.integers(0, cfg.n_adapters))
        rings["adapter_indices"][t, :3] = [a, (a + 1) % cfg.n_adapters, a]
        rings["gates_q15"][t, :3] = rng.integers(1000, 20000, 3)
    layer, ads = gpu_layer(hip, cid)
    y = _run_mlp(hip, layer, xb, rings)
    ref = oracle_mlp(cid, xf, rings)
    assert_parity(f"test_mlp_rings_naming_an_adapter_twice T={T}", W.bf16_bits_to_f32(y).reshape(ref.shape), ref)


def test_projections_prefill_parity(hip):
    """q/k/v and o projections of the 3B-shaped attention layer at 96 tokens (GEMM path)."""
    import torch

    cid, T = 4, 96
    cfg = W.CONFIGS[cid]
    xb, xf = W.activations(cfg, T)
    rings, _ = rings_for(cid, T)
    layer, ads = gpu_layer(hip, cid)
    x = _dev(xb.view(np.int16))
    r = _dev(rings.view(np.uint8))
    q = torch.empty((T, cfg.q_out), dtype=torch.int16, device="cuda")
    k = torch.empty((T, cfg.kv_out), dtype=torch.int16, device="cuda")
    v = torch.empty((T, cfg.kv_out), dtype=torch.int16, device="cuda")
    layer.qkv_forward(x, r, q, k, v)
    o = torch.empty((T, cfg.hidden), dtype=torch.int16, device="cuda")
    layer.proj_forward("o_proj", x, r, o)
    torch.cuda.synchronize()
    for name, dev in (("q_proj", q), ("k_proj", k), ("v_proj", v), ("o_proj", o)):
        got = W.bf16_bits_to_f32(dev.cpu().numpy().view(np.uint16))
        ref = oracle_proj(cid, name, xf, rings)
        ratio = assert_parity(f"test_projections_prefill_parity {name}", got.reshape(ref.shape), ref)
        assert ratio <= REL_TOL, f"{name}: {ratio:.4g}"


def test_lora_projection_known_answer(hip):
    """crates/adapteros-lora-mlx-ffi/src/lora_cpp_tests.rs:57-119 through the C ABI: W = I,
    x = [2, 3], A = [[1, 1]], B = [[1], [2]], scale 1, gate q = 16384 -> [2 + 5g, 3 + 10g],
    g = 16384 / 32767 (the 2x2 case embedded in a 32 x 64 int4 projection), on the decode and
    the prefill path."""
    import torch

    out, n = 32, 64
    q = np.zeros((out, n), np.uint32)
    for o in range(out):
        q[o, o] = 1
    packed = np.zeros((out, n // 8), np.uint32)
    for j in range(8):
        packed |= q[:, j::8] << np.uint32(4 * j)
    scales = np.full((out, 1), 0x3C00, np.uint16)  # float16 1.0
    biases = np.zeros((out, 1), np.uint16)
    layer = hip.Layer(0)
    layer.set_base("q_proj", packed, scales, biases)
    A = np.zeros((1, n), np.float32)
    A[0, :2] = 1
    B = np.zeros((out, 1), np.float32)
    B[:2, 0] = [1, 2]
    ad = hip.LoraAdapter(1, 1, 1.0)
    ad.set_module(0, "q_proj", A, B)
    layer.set_adapters([ad])
    g = np.float32(16384) / np.float32(32767)
    for T in (1, 40):
        xb = np.zeros((T, n), np.uint16)
        xb[:, 0] = 0x4000  # bf16 2.0
        xb[:, 1] = 0x4040  # bf16 3.0
        rings = np.zeros(T, hip.RING_DTYPE)
        rings["top_k"] = 1
        rings["gates_q15"][:, 0] = 16384
        y = torch.empty((T, out), dtype=torch.int16, device="cuda")
        layer.proj_forward("q_proj", _dev(xb.view(np.int16)), _dev(rings.view(np.uint8)), y)
        torch.cuda.synchronize()
        yf = W.bf16_bits_to_f32(y.cpu().numpy().view(np.uint16)).reshape(T, out)
        # bf16 output: 2 + 5 g = 4.50008 rounds to 4.5, 3 + 10 g = 8.00015 to 8.0
        assert np.allclose(yf[:, 0], 2 + 5 * g, atol=2e-2) and np.allclose(yf[:, 1], 3 + 10 * g, atol=4e-2)
        assert np.all(yf[:, 2:] == 0)


@pytest.mark.parametrize("unfused", [False, True], ids=["fused", "unfused"])
@pytest.mark.parametrize("T", [1, 32])
def test_attention_projections_parity(hip, T, unfused):
    """q/k/v in one launch (with the x shrink in its first workgroups, or in a launch of its own)
    and o: each within tolerance of the oracle and bit-identical run to run."""
    import torch

    cid = 4
    cfg = W.CONFIGS[cid]
    xb, xf = W.activations(cfg, T)
    rings, _ = rings_for(cid, T)
    layer, ads = gpu_layer(hip, cid)
    layer.set_separate_shrinks(unfused)
    x = _dev(xb.view(np.int16))
    r = _dev(rings.view(np.uint8))
    q = torch.empty((T, cfg.q_out), dtype=torch.int16, device="cuda")
    k = torch.empty((T, cfg.kv_out), dtype=torch.int16, device="cuda")
    v = torch.empty((T, cfg.kv_out), dtype=torch.int16, device="cuda")
    layer.qkv_forward(x, r, q, k, v)
    o = torch.empty((T, cfg.hidden), dtype=torch.int16, device="cuda")
    layer.proj_forward("o_proj", x, r, o)  # o's input: any [T, 3072] activation; reuse x
    torch.cuda.synchronize()
    first = [t.cpu().numpy().copy() for t in (q, k, v, o)]
    layer.qkv_forward(x, r, q, k, v)
    layer.proj_forward("o_proj", x, r, o)
    torch.cuda.synchronize()
    for a, t in zip(first, (q, k, v, o)):
        assert np.array_equal(a, t.cpu().numpy()), "run-to-run outputs differ"
    for name, dev in (("q_proj", q), ("k_proj", k), ("v_proj", v), ("o_proj", o)):
        got = W.bf16_bits_to_f32(dev.cpu().numpy().view(np.uint16))
        ref = oracle_proj(cid, name, xf, rings)
        ratio = assert_parity(f"test_attention_projections_parity T={T} unfused={unfused} {name}", got.reshape(ref.shape), ref)
        assert ratio <= REL_TOL, f"{name}: {ratio:.4g}"


@pytest.mark.parametrize("T", [1, 40, 200])
def test_mlp_rank_not_multiple_of_16_and_missing_modules(hip, T):
    """Rank-40 adapters (rows padded to 48, so a 64-column expand step spans two slots) where
    some adapters have no up_proj or no down_proj (those slots add nothing for that module), on
    the decode and prefill paths against the oracle."""
    import dataclasses

    import oracle

    cfg = dataclasses.replace(W.CONFIGS[1], rank=40, n_adapters=6)
    missing = {1: "up_proj", 4: "up_proj", 2: "down_proj"}
    lora = []
    for a in range(cfg.n_adapters):
        lora.append({m: W.lora_weights(cfg, a, m) for m in cfg.modules if missing.get(a) != m})
    base = {m: W.base_weights(cfg, m) for m in cfg.modules}
    layer = hip.Layer(0)
    for m, (p, s, b) in base.items():
        layer.set_base(m, p, s, b)
    ads = []
    for a, mods in enumerate(lora):
        ad = hip.LoraAdapter(a, 1, W.lora_scale(cfg))
        for m, (A, B) in mods.items():
            ad.set_module(0, m, A, B)
        ads.append(ad)
    layer.set_adapters(ads)
    f, w = W.router_inputs(cfg, T)
    rings = oracle.route_batch(oracle.priors(f, w), cfg.k, cfg.tau, cfg.eps, 1.0,
                               np.arange(cfg.n_adapters, dtype=np.uint64))
    xb, xf = W.activations(cfg, T)
    y = _run_mlp(hip, layer, xb, rings)
    scales = np.full(cfg.n_adapters, W.lora_scale(cfg), np.float32)
    ref = oracle.mlp_forward(xf, base["gate_proj"], base["up_proj"], base["down_proj"], lora, scales, cfg.rank,
                             rings)
    ratio = assert_parity(f"test_mlp_rank_not_multiple_of_16_and_missing_modules T={T}", W.bf16_bits_to_f32(y).reshape(ref.shape), ref)
    assert ratio <= REL_TOL, f"max tolerance ratio {ratio:.4g}"


@pytest.mark.parametrize("case", ["rank40_missing_modules", "160_adapters"])
def test_mlp_prefill_adapter_major_edges(hip, case):
    """The adapter-major prefill paths at their edges, against the oracle and bit-identical run to
    run: rank-40 adapters (rows padded to 48: three MFMA steps per chunk) some of which have no
    up_proj or no down_proj (their A rows read as zeros in the shrink, their B through an empty
    range in the expand), every tile adapter-major in the shrinks and the gate/up expand; and 160
    adapters (K = 2 of random sets at 300 tokens), more than the adapter-major expand takes, so the
    shrinks run adapter-major and the expand over the tile unions."""
    import dataclasses

    import oracle

    if case == "rank40_missing_modules":
        cfg = dataclasses.replace(W.CONFIGS[1], rank=40, n_adapters=6)
        missing = {1: "up_proj", 4: "up_proj", 2: "down_proj"}
        T = 200
    else:
        cfg = dataclasses.replace(W.CONFIGS[1], n_adapters=160)
        missing = {}
        T = 300
    lora = [{m: W.lora_weights(cfg, a, m) for m in cfg.modules if missing.get(a) != m} for a in range(cfg.n_adapters)]
    base = {m: W.base_weights(cfg, m) for m in cfg.modules}
    layer = hip.Layer(0)
    for m, (p, s, b) in base.items():
        layer.set_base(m, p, s, b)
    ads = []
    for a, mods in enumerate(lora):
        ad = hip.LoraAdapter(a, 1, W.lora_scale(cfg))
        for m, (A, B) in mods.items():
            ad.set_module(0, m, A, B)
        ads.append(ad)
    layer.set_adapters(ads)
    layer.set_prefill_shrink(False)
    if case == "rank40_missing_modules":
        layer.set_prefill_expand(48)
        layer.set_prefill_adapter_major(1)
        layer.set_prefill_expand_adapter_major(1)
        want = 7
    else:
        want = 3
    f, w = W.router_inputs(cfg, T)
    rings = oracle.route_batch(oracle.priors(f, w), cfg.k, cfg.tau, cfg.eps, 1.0,
                               np.arange(cfg.n_adapters, dtype=np.uint64))
    xb, xf = W.activations(cfg, T)
    y = _run_mlp(hip, layer, xb, rings)
    assert layer.last_expand() == 1, "expand launch state"
    assert layer.last_adapter_major() == want, "adapter-major state"
    assert np.array_equal(y, _run_mlp(hip, layer, xb, rings)), "run-to-run outputs differ"
    scales = np.full(cfg.n_adapters, W.lora_scale(cfg), np.float32)
    ref = oracle.mlp_forward(xf, base["gate_proj"], base["up_proj"], base["down_proj"], lora, scales, cfg.rank,
                             rings)
    ratio = assert_parity(f"test_mlp_prefill_adapter_major_edges {case} T={T}", W.bf16_bits_to_f32(y).reshape(ref.shape), ref)
    assert ratio <= REL_TOL, f"max tolerance ratio {ratio:.4g}"
