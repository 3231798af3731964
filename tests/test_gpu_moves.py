"""Completion's turns when every member of a cycle MOVEs, on the GPU against
the oracle, with core.step's records off (the kernels take such a cycle's
turns at once where its movers write distinct cells, in order otherwise).

The moves are admitted normally and the movers then set down by hand
(Board.place), so that at completion one mover's destination is another
mover's cell, or two movers share a destination: states that admission
never makes (a move's destination is free when issued and claimed since),
but that core.step takes like any other.  The reference applies the turns in
pending order (N/core/completion.py:106-117, N/core/kinds/move.py:25-27);
the expected cells below are traced by hand from that rule.
basesWorkers8x8 (ORIGINAL): slot 3 is player 0's worker, slot 50 player
1's; a worker's MOVE takes 10 cycles.
"""
from __future__ import annotations

import numpy as np
import pytest

from tests import test_oracle_rules as rules
from tests.helpers import assert_states_equal

pytestmark = pytest.mark.gpu

FIELDS = ("kind", "direction", "none_duration", "target_cell", "produced_type", "request_order")
MOVE, UP, RIGHT, DOWN, ABSENT = rules.MOVE, rules.UP, rules.RIGHT, rules.DOWN, rules.ABSENT


def _commands(bd: rules.Board, orders: dict | None) -> dict:
    shape = (1, 2, bd.C)
    cmds = {f: np.full(shape, ABSENT, np.int32) for f in FIELDS}
    cmds["none_duration"] = np.zeros(shape, np.int32)
    for slot, fields in (orders or {}).items():
        player, p = bd.pos(slot)
        for name, value in fields.items():
            cmds[name][0, player, p] = value
    return cmds


def _step(bd: rules.Board, orders: dict | None = None) -> None:
    """One core.step of the oracle and of the GPU (records off) from the same
    state; the GPU's leaves must equal the oracle's."""
    import torch

    from nanorts_amd import core
    from nanorts_amd.env import State
    from nanorts_amd.model import LEAF_NAMES

    cmds = _commands(bd, orders)
    dev = State({name: torch.as_tensor(np.ascontiguousarray(bd.st[name]), device="cuda:0") for name in LEAF_NAMES})
    bd.o.core_step(bd.st, cmds, bd.root)
    core.step(bd.root.copy(), dev, {f: torch.as_tensor(cmds[f], device="cuda:0") for f in FIELDS}, bd.game,
              records=False)
    leaves = {name: t.cpu().numpy() for name, t in dev.leaves.items()}
    assert_states_equal({k: v for k, v in bd.st.items() if k in leaves}, leaves, f"time {int(bd.st['time'][0])}")


def _run_to_completion(bd: rules.Board) -> None:
    for _ in range(8):  # times 1..9: nothing completes
        _step(bd)
    assert int(bd.st["time"][0]) == 9
    _step(bd)  # time 9 -> 10: both MOVEs complete


@pytest.mark.parametrize("first", [3, 50])
def test_a_mover_enters_the_cell_another_mover_leaves(first):
    """`first` moves from cell 26 RIGHT into 27; the other worker, admitted
    moving RIGHT from 19 into 20, is set down on 27, so its MOVE now leads
    from 27 to 28.  Player 0's worker holds pending order 0 (admission takes
    player 0 first).  When the mover into 27 goes first, the later mover
    empties 27 behind it: the first mover's cell reads 27 with no entity
    there.  When the mover out of 27 goes first, both land."""
    import torch

    print(f"all-MOVE chain, first mover slot {first}", flush=True)
    torch.cuda.set_device(0)
    other = 50 if first == 3 else 3
    bd = rules.Board("basesWorkers8x8")
    bd.place(first, 26)
    bd.place(other, 19)
    _step(bd, {first: {"kind": MOVE, "direction": RIGHT}, other: {"kind": MOVE, "direction": RIGHT}})
    assert bd.pending(first)[0] == MOVE and bd.pending(other)[0] == MOVE
    assert bd.pending(first)[2] == bd.pending(other)[2] == 10
    bd.place(other, 27)
    _run_to_completion(bd)
    assert int(bd.st["cell"][0, first]) == 27 and int(bd.st["cell"][0, other]) == 28
    assert bd.at(26) == ABSENT and bd.at(28) == other
    assert bd.at(27) == (ABSENT if first == 3 else first)


def test_two_movers_enter_one_cell():
    """Player 0's worker moves from 26 RIGHT into 27 (order 0); player 1's,
    admitted moving DOWN from 11 into 19, is set down on 19, so its MOVE now
    leads into 27 as well (order 1).  Both land on 27, and the grid holds the
    later one."""
    import torch

    print("all-MOVE shared destination", flush=True)
    torch.cuda.set_device(0)
    bd = rules.Board("basesWorkers8x8")
    bd.place(3, 26)
    bd.place(50, 11)
    _step(bd, {3: {"kind": MOVE, "direction": RIGHT}, 50: {"kind": MOVE, "direction": DOWN}})
    assert bd.pending(3)[2] == bd.pending(50)[2] == 10
    bd.place(50, 19)
    _run_to_completion(bd)
    assert int(bd.st["cell"][0, 3]) == 27 and int(bd.st["cell"][0, 50]) == 27
    assert bd.at(27) == 50 and bd.at(26) == ABSENT and bd.at(19) == ABSENT


def test_independent_movers_all_land():
    """Control: player 0's worker moves from 26 RIGHT into 27 and player 1's
    from 19 UP into 11, cells apart: both land (the turns at once)."""
    import torch

    print("all-MOVE independent", flush=True)
    torch.cuda.set_device(0)
    bd = rules.Board("basesWorkers8x8")
    bd.place(3, 26)
    bd.place(50, 19)
    _step(bd, {3: {"kind": MOVE, "direction": RIGHT}, 50: {"kind": MOVE, "direction": UP}})
    _run_to_completion(bd)
    assert int(bd.st["cell"][0, 3]) == 27 and int(bd.st["cell"][0, 50]) == 11
    assert bd.at(27) == 3 and bd.at(11) == 50 and bd.at(26) == ABSENT and bd.at(19) == ABSENT
