"""Decode launch geometry (CPU): every wave of every GEMV launch gets at least one K group.

The decode GEMVs split K over the waves of a workgroup and over ks workgroups per row block, and
the LDS budget for the staged activations can force more splits than the waves per workgroup
allow. The geometry then falls back to 4-wave workgroups; a wave with no group would otherwise
prime its weight ring from before the matrix. This replays the library's own geometry (the same
function the forwards call) for every workload shape at every decode token count.
"""
import pytest

import aoship

# (hidden, intermediate) of the MLP shapes: the 0.5B plumbing layer, the 7B layer, the 32B
# stress layer; then projection row counts sharing one input (q+k+v, o) at their input widths.
MLP_SHAPES = [(896, 4864), (3584, 18944), (5120, 27648)]
PROJ_SHAPES = [(3072 + 1024 + 1024, 3072), (3072, 3072), (3584 + 512 + 512, 3584), (3584, 3584),
               (152064, 3584)]
# x-shrink rank rows (adapters x padded rank x modules) and h-shrink rows
SHRINK_ROWS = [(8 * 16 * 2, 896), (16 * 16 * 2, 3584), (32 * 16 * 3, 3072), (64 * 64 * 2, 5120),
               (16 * 48 * 2, 3584)]
H_SHRINK_ROWS = [(8 * 16, 4864), (16 * 16, 18944), (64 * 64, 27648), (16 * 48, 18944)]


@pytest.mark.parametrize("T", range(1, 33))
def test_every_gemv_wave_gets_a_group(T):
    for H, I in MLP_SHAPES:
        for kind, out, inp in ((0, I, H), (1, H, I)):
            w, ks, wr, g = aoship.decode_geometry(kind, out, inp, T)
            assert w in (4, 8) and 1 <= ks <= inp // 64 and wr in (1, 2, 4, 8) and w % wr == 0
            assert wr == 1 or T > 2, "1-2 tokens keep one row block per workgroup (the h shrink needs it)"
            assert g >= 1, f"kind {kind} {out}x{inp} T={T}: waves {w}, splits {ks}, rows {wr}"
            budget = 64 * 1024 if (kind == 1 and w == 8 and T > 2) else 32 * 1024
            assert 128 + T * -(-(inp // 64) // ks) * 136 <= budget, "staged x exceeds the LDS budget"
    for out, inp in PROJ_SHAPES:
        w, ks, wr, g = aoship.decode_geometry(2, out, inp, T)
        assert g >= 1, f"projection {out}x{inp} T={T}: waves {w}, splits {ks}, rows {wr}"
        budget = 64 * 1024 if (w == 8 and T > 2) else 32 * 1024
        assert 128 + T * -(-(inp // 64) // ks) * 136 <= budget, "staged x exceeds the LDS budget"


@pytest.mark.parametrize("T", range(1, 33))
def test_shrink_geometry_within_limits(T):
    """Shrinks: the K splits stay within the groups and the LDS budget (64 KB for the x shrink above
    16 tokens, else 32 KB). A shrink wave may get no
    group when its launch runs more waves per workgroup than its splits leave groups; it then
    reads the zero row and adds nothing."""
    for kind, shapes in ((3, SHRINK_ROWS), (4, H_SHRINK_ROWS)):
        for rows, inp in shapes:
            w, ks, _, g = aoship.decode_geometry(kind, rows, inp, T)
            G = inp // 64
            assert 1 <= ks <= G
            # the x shrink above 16 tokens runs in launches held to two waves per SIMD by their
            # registers: 64 KB of staged x costs them no residency
            budget = 64 * 1024 if (kind == 3 and T > 16) else 32 * 1024
            assert 128 + T * -(-G // ks) * 128 <= budget


@pytest.mark.parametrize("T", [1, 2])
@pytest.mark.parametrize("wr", [1, 2, 4])
@pytest.mark.parametrize("ks", [0, 1, 2, 4])
def test_pinned_gate_up_keeps_one_row_block_at_one_or_two_tokens(T, wr, ks):
    """A pinned row-split shape is not applied to the 1-2 token gate/up launch, whose wave 0 forms
    the h shrink's partials for the workgroup's one row block; other launches take the pin."""
    for H, I in MLP_SHAPES:
        w, k, r, g = aoship.decode_geometry(0, I, H, T, wr, ks)
        assert r == 1 and g >= 1
        if ks and (H // 64) // ks >= w:  # a pin that leaves a wave without a K group is not applied
            assert k == ks
    w, k, r, g = aoship.decode_geometry(0, 18944, 3584, 3, 4, 0)
    assert r == 4


def test_geometry_rejects_bad_shapes():
    with pytest.raises(aoship.AosError):
        aoship.decode_geometry(0, 3584, 100, 1)
    with pytest.raises(aoship.AosError):
        aoship.decode_geometry(0, 3584, 3584, 33)
