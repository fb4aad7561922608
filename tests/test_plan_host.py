"""Planner targets (host mirror of csrc/abi.hip target_items_for and
plan_target_for) on a 256-CU device: the indexed rule every staged plan uses,
and the contiguous 16-head rule of the fused entry points."""
import pytest

from amd_optimization_challenge_amd import ops

NCU = 256


@pytest.mark.parametrize("batch,heads,mode,want", [
    (32, 16, 0, 512),      # below the slots: one item per slot (2 per CU)
    (600, 16, 1, 768),     # past the slots: 1.5 per slot
    (4096, 16, 0, 2048),   # capped at four rounds of slots
    (64, 128, 0, 256),     # H = 128: one slot per CU
    (256, 128, 2, 384),
    (64, 16, 2, 256),      # both caches at 16 heads: one slot per CU
])
def test_indexed_target(batch, heads, mode, want):
    assert ops.target_items(batch, heads, mode, NCU) == want
    assert ops.plan_target(batch, heads, mode, NCU) == (want, 128, 0)


@pytest.mark.parametrize("batch,heads,mode,want", [
    (32, 16, 0, (256, 128, 32)),    # below the CU count: one item per CU
    (4, 16, 1, (256, 128, 32)),
    (256, 16, 1, (512, 1024, 32)),  # from the CU count up: 1024-token chunk floor
    (300, 16, 0, (512, 1024, 32)),
    (600, 16, 0, (768, 1024, 32)),
    (64, 16, 2, (256, 128, 32)),    # one slot per CU already
    (64, 128, 0, (256, 128, 0)),   # H = 128 keeps the indexed rule
])
def test_contiguous_target(batch, heads, mode, want):
    assert ops.plan_target(batch, heads, mode, NCU, contiguous=True) == want


def test_auto_route_choice():
    """kv_mode 'auto': the MXFP4 cache at 16 heads when present, else fp8."""
    from amd_optimization_challenge_amd.submission import auto_kv_mode

    both = {"bf16": 0, "fp8": 0, "mxfp4": 0}
    assert auto_kv_mode(16, both) == "mxfp4"
    assert auto_kv_mode(128, both) == "fp8"
    assert auto_kv_mode(16, {"fp8": 0}) == "fp8"
    with pytest.raises(ValueError):
        auto_kv_mode(128, {"mxfp4": 0})
