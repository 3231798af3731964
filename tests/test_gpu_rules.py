"""The hand-traced rule scenarios of tests/test_oracle_rules.py on the GPU.

Every cycle of every scenario is also run through the HIP core.step
(nanorts_amd.core.step -> the library's step entry) on a device copy of the
state taken just before the cycle; after the cycle every State leaf and the
step results must equal the oracle's, which those scenarios pin to values
worked out by hand (a dead attacker still hits, a dead returner still
credits, a dead producer still spawns, the admitted counts, the settled
durations of two conflicts and of a three-unit race under every strategy,
budgets, birth order, appended ranking, cross-cycle settling, dead movers and
harvesters, pile depletion, attacker damage, truncation).  The scenarios that
read legality rows also compare the GPU's rows with the oracle's.
"""
from __future__ import annotations

import numpy as np
import pytest

from tests import test_oracle_rules as rules
from tests.helpers import assert_states_equal

pytestmark = pytest.mark.gpu

FIELDS = ("kind", "direction", "none_duration", "target_cell", "produced_type", "request_order")


class DeviceBoard(rules.Board):
    """A Board whose every core.step also runs on the GPU."""

    def before_step(self) -> None:
        import torch

        from nanorts_amd.env import State
        from nanorts_amd.model import LEAF_NAMES

        self.dev = State({name: torch.as_tensor(np.ascontiguousarray(self.st[name]), device="cuda:0")
                          for name in LEAF_NAMES})

    def after_step(self, commands: dict, out: dict) -> None:
        import torch

        from nanorts_amd import core

        got = core.step(self.root.copy(), self.dev, {f: torch.as_tensor(commands[f], device="cuda:0") for f in FIELDS},
                        self.game, records=True)
        leaves = {name: t.cpu().numpy() for name, t in self.dev.leaves.items()}
        want = {k: v for k, v in self.st.items() if k in leaves}
        assert_states_equal(want, leaves, f"time {int(self.st['time'][0])}")
        for name in ("terminated", "truncated", "reward", "admitted_harvest", "admitted_return", "admitted_produce",
                     "admitted_attack", "is_member", "records_i32", "records_i16", "records_i8"):
            np.testing.assert_array_equal(got[name].cpu().numpy().astype(out[name].dtype), out[name], err_msg=name)
        self.cycles = getattr(self, "cycles", 0) + 1

    def check_rows(self, rows: np.ndarray) -> None:
        import torch

        from nanorts_amd import core
        from nanorts_amd.env import State
        from nanorts_amd.model import LEAF_NAMES

        dev = State({name: torch.as_tensor(np.ascontiguousarray(self.st[name]), device="cuda:0")
                     for name in LEAF_NAMES})
        got = core.legal_commands(dev, self.game).cpu().numpy()[0]
        np.testing.assert_array_equal(got.astype(np.uint8), rows.astype(np.uint8), err_msg="legality rows")
        self.cycles = getattr(self, "cycles", 0) + 1

    def check_avail(self, rows: np.ndarray) -> None:
        import torch

        from nanorts_amd import core, native
        from nanorts_amd.env import State, _ptr, _stream
        from nanorts_amd.model import LEAF_NAMES

        dev = State({name: torch.as_tensor(np.ascontiguousarray(self.st[name]), device="cuda:0")
                     for name in LEAF_NAMES})
        out = torch.empty((1, 2, self.C, rows.shape[-1]), dtype=torch.uint8, device="cuda:0")
        native.check(native.load().nanorts_amd_avail_actions(_stream(), core.device_game(self.game).ref,
                                                             core._native_state(dev), 1, _ptr(out), None),
                     "nanorts_amd_avail_actions")
        np.testing.assert_array_equal(out.cpu().numpy()[0], rows.astype(np.uint8), err_msg="available rows")


SCENARIOS = [
    ("dead attacker", rules.test_dead_attacker_still_hits, ()),
    ("dead returner", rules.test_dead_returner_still_credits, ()),
    ("live returner", rules.test_live_returner_credits_and_empties_its_hands, ()),
    ("dead producer", rules.test_dead_producer_still_spawns, ()),
    ("admitted counts", rules.test_admitted_counts_follow_the_post_legality_kind, ()),
    ("settle both", rules.test_two_conflicts_settle_durations, ("both", rules.BOTH, 0)),
    ("settle alternating 0", rules.test_two_conflicts_settle_durations, ("alternating0", rules.ALTERNATING, 0)),
    ("settle alternating 1", rules.test_two_conflicts_settle_durations, ("alternating1", rules.ALTERNATING, 1)),
    ("settle random", rules.test_two_conflicts_settle_durations_random, ()),
    ("settle plays out", rules.test_two_conflicts_play_out, ()),
    ("race both", rules.test_three_unit_race, ("both", rules.BOTH, 0)),
    ("race alternating 0", rules.test_three_unit_race, ("alternating0", rules.ALTERNATING, 0)),
    ("race alternating 1", rules.test_three_unit_race, ("alternating1", rules.ALTERNATING, 1)),
    ("race random", rules.test_three_unit_race_random, ()),
    ("race arrival", rules.test_three_unit_race_the_mover_arrives_on_time, ()),
    ("cross-player budget", rules.test_over_budget_counts_only_the_same_players_pending_cost, ()),
    ("free request beside overdrawn pending", rules.test_free_request_beside_an_overdrawn_pending, ()),
    ("no overflow unaffordable", rules.test_spawn_overflow_only_when_affordable, (2, 0, 0)),
    ("overflow affordable", rules.test_spawn_overflow_only_when_affordable, (3, 1, 1)),
    ("birth order alternating 0", rules.test_admission_ranks_by_birth_before_position, (0, 10, (4, 19))),
    ("birth order alternating 1", rules.test_admission_ranks_by_birth_before_position, (1, 4, (10, 26))),
    ("birth order random", rules.test_admission_ranks_by_birth_before_position_random, ()),
    ("appended order both", rules.test_appended_orders_rank_in_admission_order, ("both", rules.BOTH)),
    ("appended order alternating", rules.test_appended_orders_rank_in_admission_order,
     ("alternating0", rules.ALTERNATING)),
    ("cross-cycle settle both", rules.test_pending_after_a_cross_cycle_conflict_settles_to_minus_one,
     (rules.BOTH, 0)),
    ("cross-cycle settle alternating", rules.test_pending_after_a_cross_cycle_conflict_settles_to_minus_one,
     (rules.ALTERNATING, 1)),
    ("dead mover", rules.test_dead_mover_stays_put, (False,)),
    ("dead mover refilled slot", rules.test_dead_mover_stays_put, (True,)),
    ("dead harvester", rules.test_dead_harvester_still_drains_the_pile, (20, 19)),
    ("dead harvester depletes", rules.test_dead_harvester_still_drains_the_pile, (1, 0)),
    ("exact depletion", rules.test_harvest_removes_a_pile_left_at_exactly_zero, (1,)),
    ("pile stands", rules.test_harvest_removes_a_pile_left_at_exactly_zero, (2,)),
    ("attacker damage", rules.test_attack_damage_is_the_attackers, ()),
    ("truncation", rules.test_truncation_at_max_cycles, ()),
    ("won at max_cycles", rules.test_a_game_won_at_max_cycles_is_terminated_not_truncated, ()),
    ("built legality rows", rules.test_legality_rows_of_a_built_position, ()),
    ("return into enemy base", rules.test_return_into_an_enemy_base_is_not_admitted, ()),
    ("ranged at range", rules.test_ranged_attack_at_exactly_its_range, ()),
]


@pytest.mark.parametrize("label,scenario,args", SCENARIOS, ids=[s[0] for s in SCENARIOS])
def test_rule_scenario_on_gpu(label, scenario, args, monkeypatch):
    import torch

    print(f"rule scenario {label}", flush=True)
    torch.cuda.set_device(0)
    boards = []

    def make(*a, **k):
        board = DeviceBoard(*a, **k)
        boards.append(board)
        return board

    monkeypatch.setattr(rules, "BOARD", make)
    scenario(*args)
    assert boards and all(getattr(b, "cycles", 0) > 0 for b in boards)
