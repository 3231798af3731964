"""The fused rollout's choice of first pass (CPU: the query reads only the
game's extents and unit table, never device memory).

Two games per wave pay where at least three waves per SIMD fit; the slot
window (32 slots a player) brings basesWorkers16x16 and the 24x24 and 32x32
boards there.  Widths that are not a multiple of 4 have no first pass, and
GardenOfWar64x64's block (its 64x64 occupancy grid) keeps one game per wave.
"""
from __future__ import annotations

import pytest

from tests.helpers import game_for


def _first_pass(case: str) -> int:
    import torch

    from nanorts_amd import native
    from nanorts_amd.env import DeviceGame

    game, _ = game_for(case)
    return native.load().nanorts_amd_rollout_first_pass(DeviceGame(game, torch.device("cpu")).ref)


@pytest.mark.parametrize("case, want", [
    ("16x16-random-partial", 2), ("16x16-noprofile-random", 2), ("8x8-original-both", 2), ("melee-both", 2),
    ("24x24-barricades-alternating", 2), ("32x32-random-partial", 2), ("gow-alternating", 1),
    ("10x10-random-partial", 0), ("9x8-alternating", 0),
])
def test_first_pass_by_board(case, want, monkeypatch):
    monkeypatch.delenv("NANORTS_AMD_FIRST_PASS", raising=False)
    assert _first_pass(case) == want


def test_environment_variable_forces_either_pass(monkeypatch):
    monkeypatch.setenv("NANORTS_AMD_FIRST_PASS", "lean")
    assert _first_pass("16x16-random-partial") == 1
    monkeypatch.setenv("NANORTS_AMD_FIRST_PASS", "pair")
    assert _first_pass("gow-alternating") == 2
    # a board with no first pass has none whatever is asked
    assert _first_pass("10x10-random-partial") == 0
