"""Pins of the scripted-bot part of the CPU oracle (CPU only, no GPU).

The A* search is checked against a second formulation written from the
reference's program form (src/nanorts/bots/pathfinding.py:170-245: a global
argmin over f * (cells + 1) + (cells - sequence) keys, where the oracle keeps
stacks of buckets) and against breadth-first distances.  The bot's decisions
are checked by a cycle traced by hand on the shipped 8x8 map, the ring walk of
building sites by an independent perimeter walk, the Commands contract of the
reference (src/nanorts/model/commands.py:37-70), and whole games against a
passive opponent (WorkerRush wins, LightRush builds barracks and trains light
units).
"""
from __future__ import annotations

from collections import deque

import numpy as np
import pytest

from nanorts_amd.content import map_name_to_scenario
from nanorts_amd.model import STATE_LEAVES, UnitTypeTableVersion
from oracle import oracle as orc
from oracle.oracle import Oracle, batch_initial, empty_carry
from tests import bots_program as program
from tests.bots_program import astar_by_keys

NONE, MOVE, HARVEST, RETURN, PRODUCE, ATTACK = range(6)
UP, RIGHT, DOWN, LEFT = range(4)
RESOURCE, BASE, BARRACKS, WORKER, LIGHT = 0, 1, 2, 3, 4
WORKER_RUSH, BARRACKS_RUSH = 0, 1
STEPS = ((0, -1), (1, 0), (0, 1), (-1, 0))


# ---------------------------------------------------------------------------
# A*
# ---------------------------------------------------------------------------
def bfs(free: np.ndarray, start: int):
    H, W = free.shape
    dist = np.full(H * W, -1, np.int64)
    dist[start] = 0
    queue = deque([start])
    while queue:
        c = queue.popleft()
        for dx, dy in STEPS:
            x, y = c % W + dx, c // W + dy
            n = y * W + x
            if 0 <= x < W and 0 <= y < H and free.reshape(-1)[n] and dist[n] < 0:
                dist[n] = dist[c] + 1
                queue.append(n)
    return dist


def test_astar_matches_key_formulation_and_bfs():
    rng = np.random.default_rng(5)
    for trial in range(400):
        H, W = int(rng.integers(1, 9)), int(rng.integers(1, 9))
        free = rng.random((H, W)) < rng.uniform(0.5, 0.95)
        start, target = int(rng.integers(0, H * W)), int(rng.integers(0, H * W))
        if trial % 3:
            free.reshape(-1)[start] = False  # a unit stands on its start cell
        range_ = int(rng.integers(0, 4))
        got = orc.astar(free, start, target, range_)
        assert got == astar_by_keys(free, start, target, range_), (trial, H, W, start, target, range_)
        # completeness and, for a point goal, optimality
        open_ = free.copy()
        open_.reshape(-1)[start] = True
        dist = bfs(open_, start)
        cells = np.arange(H * W)
        within = (cells % W - target % W) ** 2 + (cells // W - target // W) ** 2 <= range_ * range_
        reachable = within & (dist >= 0)
        assert got[0] == int(reachable.any())
        if range_ == 0 and got[0]:
            assert got[2] == dist[target]
        if got[0] and got[2] > 0 and W > 1:
            first = start + {UP: -W, RIGHT: 1, DOWN: W, LEFT: -1}[got[1]]
            assert open_.reshape(-1)[first] and dist[first] == 1


def test_astar_last_inserted_first_among_equal_f():
    """Open 3x3 board from the centre to the bottom-right corner: right and
    down tie on f; down, pushed later, is expanded first."""
    free = np.ones((3, 3), bool)
    assert orc.astar(free, 4, 8, 0)[:3] == (1, DOWN, 2)
    free[2, 1] = False  # below the centre blocked: right leads
    assert orc.astar(free, 4, 8, 0)[:3] == (1, RIGHT, 2)


# ---------------------------------------------------------------------------
# Bots on basesWorkers8x8: slots 0/1 piles at cells 0 / 63; player 0 base
# (slot 2, birth 2) at 10 and worker (slot 3, birth 4) at 9; player 1 base
# (slot 49, birth 3) at 53 and worker (slot 50, birth 5) at 54; balances 5/5.
# ---------------------------------------------------------------------------
def _eight(utt=UnitTypeTableVersion.ORIGINAL_FINETUNED, max_cycles=5000):
    game = map_name_to_scenario("basesWorkers8x8", utt=utt, max_cycles=max_cycles)
    return game, Oracle(game), batch_initial(game, 1, np.asarray([[1, 2]], np.uint32))


def test_worker_rush_first_cycle_by_hand():
    game, o, st = _eight()
    C = game.bucket.per_player_capacity
    carry = empty_carry(1, C)
    cmds = o.abstraction_act(st, carry, WORKER_RUSH, LIGHT, 1)
    # player 0's rows stay empty
    assert (cmds["kind"][0, 0] == -1).all() and (cmds["request_order"][0, 0] == -1).all()
    k, d, t, r = (cmds[f][0, 1] for f in ("kind", "direction", "produced_type", "request_order"))
    # the base trains a worker toward the nearer pile: below it (cell 61) is
    # 2 from pile 63, above and left are 4
    assert (k[0], d[0], t[0], r[0]) == (PRODUCE, DOWN, WORKER, 0)
    # the worker heads for pile 63: right (55) and down (62) tie on f; down
    # was pushed last and is reached first
    assert (k[1], d[1], r[1]) == (MOVE, DOWN, 1)
    assert (k[2:] == -1).all()
    # carry: TRAIN (executed, so trained) and HARVEST of pile 1 to base 49
    assert carry["kind"][0, :2].tolist() == [3, 2] and carry["trained"][0, :2].tolist() == [1, 0]
    assert carry["target"][0, 1] == 1 and carry["target_birth"][0, 1] == 1
    assert carry["base"][0, 1] == 49 and carry["base_birth"][0, 1] == 3
    assert carry["order"][0, :2].tolist() == [0, 1] and carry["next_order"][0] == 2
    assert carry["unit_type"][0, 0] == WORKER and (carry["kind"][0, 2:] == -1).all()


def test_worker_rush_second_cycle_drops_the_trained_entry():
    """The TRAIN entry was executed, so the next act sees it completed unless
    the base is chosen again; the base is busy producing, so it is not."""
    game, o, st = _eight()
    C = game.bucket.per_player_capacity
    carry = empty_carry(1, C)
    cmds = o.abstraction_act(st, carry, WORKER_RUSH, LIGHT, 1)
    merged = {f: v.copy() for f, v in cmds.items()}
    merged["kind"][0, 0, :] = -1
    o.core_step(st, merged, np.asarray([[1, 2]], np.uint32))
    assert st["pending_kind"][0, 49] == PRODUCE and st["pending_kind"][0, 50] == MOVE
    cmds = o.abstraction_act(st, carry, WORKER_RUSH, LIGHT, 1)
    assert (cmds["kind"][0, 1] == -1).all()  # both units busy: nothing issued
    assert carry["kind"][0, 0] == -1 and carry["kind"][0, 1] == 2 and carry["next_order"][0] == 1


def _ring_walk(H, W, desired):
    """Cells around `desired` ring by ring: top side left to right, right side
    downward, bottom side left to right, left side downward."""
    x0, y0 = desired % W, desired // W
    for ring in range(1, max(H, W)):
        side = [(x0 + dx, y0 - ring) for dx in range(-ring, ring + 1)]
        side += [(x0 + ring, y0 + dy) for dy in range(-ring + 1, ring + 1)]
        side += [(x0 + dx, y0 + ring) for dx in range(-ring, ring)]
        side += [(x0 - ring, y0 + dy) for dy in range(-ring + 1, ring)]
        for x, y in side:
            if 0 <= x < W and 0 <= y < H:
                yield y * W + x


def _clear(st, slot):
    st["entity_at"].reshape(1, -1)[0, int(st["cell"][0, slot])] = -1
    for leaf in STATE_LEAVES:
        if leaf.kind == "slot":
            st[leaf.name][0, slot] = leaf.fill


def _place(st, slot, cell):
    st["entity_at"].reshape(1, -1)[0, int(st["cell"][0, slot])] = -1
    st["entity_at"].reshape(1, -1)[0, cell] = slot
    st["cell"][0, slot] = cell


@pytest.mark.parametrize("worker_cell", [54, 27, 0 + 8, 36])
def test_build_site_follows_the_ring_walk(worker_cell):
    """Without a base and with 10 resources, WorkerRush's worker builds one at
    the first open cell of the ring walk around it."""
    game, o, st = _eight()
    H, W = game.bucket.height, game.bucket.width
    C = game.bucket.per_player_capacity
    _clear(st, 49)
    _place(st, 50, worker_cell)
    st["player_resources"][0, 1] = 10
    carry = empty_carry(1, C)
    o.abstraction_act(st, carry, WORKER_RUSH, LIGHT, 1)
    occupied = st["entity_at"].reshape(-1) != -1
    want = next(c for c in _ring_walk(H, W, worker_cell) if not occupied[c] and not game.terrain.reshape(-1)[c])
    assert carry["kind"][0, 1] == 4 and carry["unit_type"][0, 1] == BASE and carry["cell"][0, 1] == want


def _check_commands(cmds, st, game, bot):
    """Commands.check_values (src/nanorts/model/commands.py:37-70) plus the
    translate contract: only available units of the bot get a command, the
    issued request orders are 0..k-1, fillers wait 10."""
    C, N = game.bucket.per_player_capacity, game.bucket.neutral_capacity
    for l in range(cmds["kind"].shape[0]):
        assert (cmds["kind"][l, 1 - bot] == -1).all()
        kind, order = cmds["kind"][l, bot], cmds["request_order"][l, bot]
        slots = N + bot * C + np.arange(C)
        available = (st["birth"][l, slots] != -1) & (st["pending_kind"][l, slots] == -1)
        issued = kind != -1
        assert (issued == available).all()
        assert (order[~issued] == -1).all()
        assert sorted(order[issued].tolist()) == list(range(int(issued.sum())))
        filler = kind == NONE
        assert (cmds["none_duration"][l, bot][filler] == 10).all()


def _seat_games(strategy, trained, envs, steps, utt=UnitTypeTableVersion.ORIGINAL_FINETUNED, passive=False,
                seed=3):
    game = map_name_to_scenario("basesWorkers8x8", utt=utt, max_cycles=5000)
    o = Oracle(game)
    C = game.bucket.per_player_capacity
    st = batch_initial(game, envs, np.stack([np.arange(envs), np.arange(envs) + 7], 1).astype(np.uint32))
    carry = empty_carry(envs, C)
    log = []
    for t in range(steps):
        if passive:
            actions = np.zeros((envs, C, 7), np.int32)
        else:
            rows = o.avail_rows(st)
            actions = o.sample_actions(rows, (seed, seed + 9), t)[:, 0]
        probe = {k: v.copy() for k, v in carry.items()}
        cmds = o.abstraction_act({k: v.copy() for k, v in st.items()}, probe, strategy, trained, 1)
        _check_commands(cmds, st, game, 1)
        out = o.seat_step(st, carry, strategy, trained, 0, actions, False, observe=False)
        assert (o.violations(st) == 0).all(), t
        log.append((out, st["unit_type"].copy(), st["owner"].copy(), st["birth"].copy()))
    return game, st, carry, log


def test_worker_rush_beats_a_passive_opponent():
    game, st, carry, log = _seat_games(WORKER_RUSH, LIGHT, 2, 700, passive=True)
    ends = [(t, int(out["winner"][l])) for t, (out, *_) in enumerate(log) for l in range(2) if out["done"][l]]
    assert ends, "no game ended"
    assert all(w == 1 for _, w in ends)


def test_light_rush_builds_barracks_and_trains_light_units():
    game, st, carry, log = _seat_games(BARRACKS_RUSH, LIGHT, 2, 900, passive=True)
    seen_barracks = seen_light = False
    for out, utype, owner, birth in log:
        live = birth != -1
        seen_barracks |= bool(((utype == BARRACKS) & (owner == 1) & live).any())
        seen_light |= bool(((utype == LIGHT) & (owner == 1) & live).any())
    assert seen_barracks and seen_light


@pytest.mark.parametrize("strategy", [WORKER_RUSH, BARRACKS_RUSH])
def test_seat_rollout_keeps_invariants_against_random_play(strategy):
    game, st, carry, log = _seat_games(strategy, LIGHT, 3, 250)
    # the carry is empty after a reset and never names a dead unit's entry as standing
    for l in range(3):
        live = carry["kind"][l] != -1
        assert (carry["order"][l][live] >= 0).all()
        assert sorted(carry["order"][l][live].tolist()) == list(range(int(live.sum())))
        assert carry["next_order"][l] == int(live.sum())


def _settled_properties(before, after, l, where):
    """What put and _settled (N/bots/abstraction.py:172-227, 1099-1119) fix
    for one env's carry after an act: the standing entries' orders are
    0 .. n - 1 with next_order n (a dense rank of their orders); an entry that
    is not standing holds ABSENT in every field and trained 0; an entry whose
    unit held one before the act keeps its order through any put, so such
    entries keep their relative order, and every new entry (stamped from
    next_order on) ranks after all of them.  Returns how many new entries
    ranked behind a held entry in a lower-numbered slot."""
    live = after["kind"][l] != -1
    n = int(live.sum())
    assert sorted(after["order"][l][live].tolist()) == list(range(n)), where
    assert int(after["next_order"][l]) == n, where
    for f in program.CARRY_FIELDS:
        assert (after[f][l][~live] == -1).all(), (where, f)
    assert (after["trained"][l][~live] == 0).all(), where
    held = live & (before["kind"][l] != -1) & (before["unit_birth"][l] == after["unit_birth"][l])
    fresh = live & ~held
    h = np.flatnonzero(held)
    ob, oa = before["order"][l], after["order"][l]
    for i in h:
        for j in h:
            if ob[i] < ob[j]:
                assert oa[i] < oa[j], (where, int(i), int(j))
    if held.any() and fresh.any():
        assert oa[held].max() < oa[fresh].min(), where
        return int(sum(1 for j in np.flatnonzero(fresh) if (h > j).any()))
    return 0


@pytest.mark.parametrize("strategy", [WORKER_RUSH, BARRACKS_RUSH])
def test_every_act_leaves_a_settled_carry(strategy):
    """The settled carry's properties after every act of six games against
    random play, for the bot's seat and a shadow carry of player 0 (acted on,
    never executed)."""
    game = map_name_to_scenario("basesWorkers8x8", max_cycles=5000)
    o = Oracle(game)
    C = game.bucket.per_player_capacity
    L = 6
    st = batch_initial(game, L, np.stack([np.arange(L) + 5, np.arange(L) + 9], 1).astype(np.uint32))
    carry, shadow = empty_carry(L, C), empty_carry(L, C)
    carried = inverted = 0
    for t in range(600):
        for player, held in ((1, carry), (0, shadow)):
            probe = {k: v.copy() for k, v in held.items()}
            o.abstraction_act({k: v.copy() for k, v in st.items()}, probe, strategy, LIGHT, player)
            for l in range(L):
                inverted += _settled_properties(held, probe, l, f"t={t} player {player} env {l}")
                carried += int(((held["kind"][l] != -1) & (probe["kind"][l] != -1)).sum())
            if player == 0:
                shadow = probe
        actions = o.sample_actions(o.avail_rows(st), (31, 37), t)[:, 0]
        o.seat_step(st, carry, strategy, LIGHT, 0, actions, False, observe=False)
    assert carried > 100  # entries did stand across acts
    assert inverted > 0  # and new entries in lower slots ranked behind held ones


# ---------------------------------------------------------------------------
# The act against its array form (tests/bots_program.py): every cycle of
# games played by the oracle's seat against random play, on boards with walls,
# several bases, barracks and melee-only armies, for both seats' carries.
# ---------------------------------------------------------------------------
HEAVY, RANGED = 5, 6
PROGRAM_GAMES = [
    ("basesWorkers8x8", WORKER_RUSH, LIGHT, 220),
    ("basesWorkers8x8", BARRACKS_RUSH, LIGHT, 320),
    ("NoWhereToRun9x8", WORKER_RUSH, LIGHT, 200),
    ("basesWorkers8x8Obstacle", BARRACKS_RUSH, RANGED, 320),
    ("FourBasesWorkers8x8", WORKER_RUSH, LIGHT, 200),
    ("TwoBasesBarracks16x16", BARRACKS_RUSH, HEAVY, 160),
    ("melee8x8Mixed4", WORKER_RUSH, LIGHT, 120),
    ("basesWorkersBarracks8x8", BARRACKS_RUSH, RANGED, 260),
]


def _compare_act(game, o, st, carry, strategy, trained, player, where):
    """One act of the oracle against the array form, for every env."""
    probe = {k: v.copy() for k, v in carry.items()}
    cmds = o.abstraction_act({k: v.copy() for k, v in st.items()}, probe, strategy, trained, player)
    for l in range(st["time"].shape[0]):
        want, settled = program.act(game, st, carry, l, strategy, trained, player)
        for f, v in want.items():
            np.testing.assert_array_equal(cmds[f][l, player], v, err_msg=f"{where} env {l} command {f}")
            assert (cmds[f][l, 1 - player] == -1).all() or f == "none_duration", (where, l, f)
        for f in program.CARRY_FIELDS:
            np.testing.assert_array_equal(probe[f][l], getattr(settled, f), err_msg=f"{where} env {l} carry {f}")
        np.testing.assert_array_equal(probe["trained"][l] != 0, settled.trained, err_msg=f"{where} env {l} trained")
        assert probe["next_order"][l] == settled.next_order, (where, l)
    return probe


@pytest.mark.parametrize("name,strategy,trained,steps", PROGRAM_GAMES)
def test_act_matches_the_array_form_over_whole_games(name, strategy, trained, steps):
    game = map_name_to_scenario(name, max_cycles=5000)
    o = Oracle(game)
    C = game.bucket.per_player_capacity
    L = 2
    st = batch_initial(game, L, np.stack([np.arange(L) + 11, np.arange(L) + 3], 1).astype(np.uint32))
    carry = empty_carry(L, C)
    shadow = empty_carry(L, C)  # player 0's carry, acted on but never executed
    for t in range(steps):
        actions = o.sample_actions(o.avail_rows(st), (17, 29), t)[:, 0]
        _compare_act(game, o, st, carry, strategy, trained, 1, f"{name} t={t} seat")
        shadow = _compare_act(game, o, st, shadow, strategy, trained, 0, f"{name} t={t} shadow")
        o.seat_step(st, carry, strategy, trained, 0, actions, False, observe=False)


# ---------------------------------------------------------------------------
# The walk of the FFI target nanorts_astar_chain (N/bots/cuda/abstraction.cu:
# 98-215), restated by the oracle: hand-traced on small open boards.
# Row columns: start, goal, radius, draws, options, then the fallback's kind,
# claim, cost (5-7) and the blocked desire's (8-10).
# ---------------------------------------------------------------------------
FALLBACK, BLOCKED = (5, 6, 7), (8, 9, 10)


def _chain_row(start, goal, radius=0, draws=0, options=0, fallback=(-1, -1, 0), blocked=(-1, -1, 0)):
    return [start, goal, radius, draws, options, *fallback, *blocked]


def _chain(rows, queue=None, count=None, moves=True, reserved=0, balance=10, draws=(0,), drawing=False,
           free=None, claimed=None, W=4, H=4):
    from oracle.oracle import astar_chain

    rows = np.asarray(rows, np.int32)
    queue = np.arange(len(rows), dtype=np.int32) if queue is None else np.asarray(queue, np.int32)
    free = np.ones((H, W), bool) if free is None else free
    claimed = np.zeros((H, W), bool) if claimed is None else claimed
    return astar_chain(free, claimed, rows, queue, len(rows) if count is None else count, moves, reserved, balance,
                       np.asarray(draws, np.int32), drawing, FALLBACK, BLOCKED)


def test_chain_moves_and_claims_in_queue_order():
    """4x4 open board.  Row 0 walks from cell 5 toward 7: first step RIGHT
    into 6, kept at rank 0; its claim closes 6 to later searches.  Row 1
    walks from 10 toward 2: with 6 closed every neighbour lies farther from
    the goal, and the last one inserted, LEFT (9), is popped first: kept at
    rank 1.  Row 2 stands at its goal (no step) and takes its fallback, a
    claim on 6 at cost 0: taken, not kept.  Totals: 2 kept, no draws."""
    out = _chain([_chain_row(5, 7), _chain_row(10, 2), _chain_row(13, 13, fallback=(0, 6, 0))])
    assert out[:3].tolist() == [[0, 2, 1, 0], [1, 2, 3, 0], [-1, 0, -1, 0]]
    assert out[3].tolist() == [2, 0, 0, 0]


def test_chain_blocked_when_moves_are_not_allowed():
    """may_move false: a row that can step takes its blocked desire
    (selector 1, no direction), one that cannot its fallback; a desire of
    kind -1 is never kept."""
    out = _chain([_chain_row(5, 7, blocked=(4, 9, 0)), _chain_row(6, 6, fallback=(-1, 3, 0))], moves=False)
    assert out[:2].tolist() == [[0, 1, -1, 0], [-1, 0, -1, 0]]
    assert out[2].tolist() == [1, 0, 0, 0]


def test_chain_budget_counts_reserve_and_kept_costs():
    """balance 5, reserve 1: a fallback of cost 3 is kept (1 + 3 <= 5), the
    next of cost 2 is not (1 + 3 + 2 > 5), the third of cost 1 is (5 <= 5)."""
    rows = [_chain_row(0, 0, fallback=(4, 4, 3)), _chain_row(1, 1, fallback=(4, 8, 2)),
            _chain_row(2, 2, fallback=(4, 12, 1))]
    out = _chain(rows, reserved=1, balance=5)
    assert [r[0] for r in out[:3].tolist()] == [0, -1, 1]
    assert out[3, 0] == 2


def test_chain_queue_order_count_and_skipped_slots():
    """The queue visits slot 2, then an out-of-range slot (skipped), then slot
    0; count 3 leaves slot 1 unvisited (rank -1, selector 0, no direction).
    Slot 2 goes first: from 10 toward 2, UP into 6.  Slot 0, from 5 toward
    7, then goes round the closed 6: the LEFT branch is popped first but
    only leads away, and the first path found starts DOWN (9): rank 1."""
    rows = [_chain_row(5, 7), _chain_row(0, 3), _chain_row(10, 2)]
    out = _chain(rows, queue=[2, 7, 0], count=3)
    assert out[:3].tolist() == [[1, 2, 2, 0], [-1, 0, -1, 0], [0, 2, 0, 0]]


@pytest.mark.parametrize("closing_row", [False, True])
def test_chain_taken_cells_refuse_and_closed_cells_divert(closing_row):
    """Cell 6 is claimed (taken) but free (open to the search).  Alone, the
    row from 5 toward 7 steps RIGHT into 6 and is refused (rank -1).  After a
    row whose fallback claims 6 (refused too, but closing 6), the search goes
    round below it: DOWN (9), kept."""
    claimed = np.zeros((4, 4), bool)
    claimed.reshape(-1)[6] = True
    rows = ([_chain_row(0, 0, fallback=(4, 6, 0))] if closing_row else []) + [_chain_row(5, 7)]
    out = _chain(rows, claimed=claimed)
    if closing_row:
        assert out[:2].tolist() == [[-1, 0, -1, 0], [0, 2, 2, 0]]
    else:
        assert out[:1].tolist() == [[-1, 2, 1, 0]]


def test_chain_drawing_pass_turns_to_an_allowed_direction():
    """A drawing pass: a row with draws that cannot move (moves false) takes
    the first direction from its draw, turning +1 mod 4, that its options
    allow.  Draw 0 with options {LEFT, DOWN} (bits 3, 2) gives DOWN; the
    second row's draw 3 with options {UP} gives UP; draws used 2."""
    rows = [_chain_row(5, 7, draws=1, options=0b1100), _chain_row(10, 10, draws=1, options=0b0001)]
    out = _chain(rows, moves=False, draws=[0, 3], drawing=True)
    assert out[:2].tolist() == [[0, 2, 2, 1], [1, 2, 0, 1]]
    assert out[2].tolist() == [2, 2, 0, 0]
