"""Pins of the GridNet decode in the CPU oracle (CPU only, no GPU).

The GridNet surface (src/nanorts/adapters/gridnet/actions.py) reads one
action row per cell and keeps, per player in cell order, the rows whose
claimed position is still free and whose cost does not overdraw
(source_filter.py).  It is checked here by a cycle traced by hand on the
shipped 8x8 map, and on many mid-game states against the JaxMARL decode (the
kept rows decode to the same commands) and against the filter's own
invariants (no two kept claims share a position, kept rows are ranked in cell
order, dropped and silent units wait as NONE fillers ranked by birth).
"""
from __future__ import annotations

import numpy as np
import pytest

from nanorts_amd.content import map_name_to_scenario
from oracle.oracle import Oracle, batch_initial
from tests.helpers import advanced_states, game_for

NONE, MOVE, HARVEST, RETURN, PRODUCE, ATTACK = range(6)
UP, RIGHT, DOWN, LEFT = range(4)
WORKER = 3
STEP = {UP: (0, -1), RIGHT: (1, 0), DOWN: (0, 1), LEFT: (-1, 0)}


def _place(st, slot, cell):
    st["entity_at"].reshape(1, -1)[0, int(st["cell"][0, slot])] = -1
    st["entity_at"].reshape(1, -1)[0, cell] = slot
    st["cell"][0, slot] = cell


def test_two_claims_on_one_cell_by_hand():
    """Player 0's worker (slot 3) moved to cell 1 and its base (slot 2, cell
    10): the worker MOVEs right and the base PRODUCEs up, both into cell 2.
    The worker's cell comes first, so it keeps the cell; the base waits as a
    filler.  Player 1 sends NONE everywhere: both its units keep NONE with
    duration -1, ranked by cell."""
    game = map_name_to_scenario("basesWorkers8x8")
    o = Oracle(game)
    st = batch_initial(game, 1, np.asarray([[1, 2]], np.uint32))
    _place(st, 3, 1)
    H, W = game.bucket.height, game.bucket.width
    actions = np.zeros((1, 2, H * W, 7), np.int32)
    actions[0, 0, 1] = [MOVE, RIGHT, 0, 0, 0, 0, 0]
    actions[0, 0, 10] = [PRODUCE, 0, 0, 0, UP, WORKER, 0]
    c = o.gridnet_decode(st, actions)
    C = game.bucket.per_player_capacity
    pick = lambda p, i: tuple(int(c[f][0, p, i]) for f in
                              ("kind", "direction", "none_duration", "target_cell", "produced_type", "request_order"))
    assert pick(0, 1) == (MOVE, RIGHT, 0, -1, -1, 0)      # the worker (slot 3 = position 1)
    assert pick(0, 0) == (NONE, -1, 1, -1, -1, 1)         # the base: dropped, filler after the survivor
    assert pick(1, 0) == (NONE, -1, -1, -1, -1, 0)        # player 1's base at cell 53
    assert pick(1, 1) == (NONE, -1, -1, -1, -1, 1)        # its worker at cell 54
    assert (c["kind"][0, :, 2:] == -1).all() and (c["request_order"][0, :, 2:] == -1).all()
    # without the worker's claim the base keeps its production; both rows
    # are kept, ranked by cell (the worker's cell 1 first)
    actions[0, 0, 1] = [NONE, 0, 0, 0, 0, 0, 0]
    c = o.gridnet_decode(st, actions)
    assert pick(0, 0) == (PRODUCE, UP, 0, -1, WORKER, 1) and pick(0, 1) == (NONE, -1, -1, -1, -1, 0)
    # an ABSENT kind (-1) claims nothing and survives the filter, so it takes
    # rank 0 in cell order; it submitted no command, so the worker still waits
    # as an idle filler ranked after both survivors (actions.py:139-164)
    actions[0, 0, 1] = [-1, 0, 0, 0, 0, 0, 0]
    c = o.gridnet_decode(st, actions)
    assert pick(0, 0) == (PRODUCE, UP, 0, -1, WORKER, 1) and pick(0, 1) == (NONE, -1, 1, -1, -1, 2)
    del C


BARRACKS = 2
FIELDS = ("kind", "direction", "none_duration", "target_cell", "produced_type", "request_order")


def seeding_cases():
    """Hand-built basesWorkers8x8 states in which player 0's issued usage
    decides player 1's claim on cell 27 (source_filter.py:124-139: player 0's
    rows that survive its filter, claim a position and are legal seed player
    1's filter with their positions and production costs).  Player 1's worker
    (slot 50, position 1) stands on cell 28 and MOVEs LEFT into 27; its base
    (slot 49, position 0) on cell 53 sends NONE.  Player 0's base is slot 2
    (position 0), its worker slot 3 (position 1).  Each case gives the state,
    the per-cell actions and the commands traced by hand from the rule:
    (player, position) -> (kind, direction, none_duration, target_cell,
    produced_type, request_order); a row dropped by the filter waits as a NONE
    filler of duration 1 ranked after the survivors, a NONE row keeps
    duration -1."""
    game = map_name_to_scenario("basesWorkers8x8")
    H, W = game.bucket.height, game.bucket.width

    def start(moves):
        st = batch_initial(game, 1, np.asarray([[1, 2]], np.uint32))
        for slot, cell in moves:
            _place(st, slot, cell)
        acts = np.zeros((1, 2, H * W, 7), np.int32)
        acts[0, 1, 28] = [MOVE, LEFT, 0, 0, 0, 0, 0]
        return st, acts

    cases = []
    # player 0's worker MOVEs from 26 into 27: kept and legal, so 27 is
    # used for player 1, whose worker's claim is dropped
    st, acts = start([(3, 26), (50, 28)])
    acts[0, 0, 26] = [MOVE, RIGHT, 0, 0, 0, 0, 0]
    cases.append(("seeded move", game, st, acts, {
        (0, 0): (NONE, -1, -1, -1, -1, 0), (0, 1): (MOVE, RIGHT, 0, -1, -1, 1),
        (1, 0): (NONE, -1, -1, -1, -1, 0), (1, 1): (NONE, -1, 1, -1, -1, 1)}))
    # the same without player 0's claim: player 1's worker keeps its MOVE,
    # ranked first by its cell
    st, acts = start([(3, 26), (50, 28)])
    cases.append(("no claim", game, st, acts, {
        (0, 0): (NONE, -1, -1, -1, -1, 0), (0, 1): (NONE, -1, -1, -1, -1, 1),
        (1, 0): (NONE, -1, -1, -1, -1, 1), (1, 1): (MOVE, LEFT, 0, -1, -1, 0)}))
    # player 0's base, set down on 26, MOVEs into 27: its own filter keeps
    # the row, but a base cannot move, so the claim is not legal and does not
    # seed player 1's filter
    st, acts = start([(2, 26), (50, 28)])
    acts[0, 0, 26] = [MOVE, RIGHT, 0, 0, 0, 0, 0]
    cases.append(("illegal claim", game, st, acts, {
        (0, 0): (MOVE, RIGHT, 0, -1, -1, 1), (0, 1): (NONE, -1, -1, -1, -1, 0),
        (1, 0): (NONE, -1, -1, -1, -1, 1), (1, 1): (MOVE, LEFT, 0, -1, -1, 0)}))
    # player 0's base (cell 10) PRODUCEs a Worker UP into 2 (cost 1), then its
    # worker on 26 a Barracks RIGHT into 27 (cost 5): 1 + 5 overdraws the
    # balance of 5 after a spend, so player 0's own filter drops the worker's
    # row, and 27 is not seeded; the base's kept, legal claim seeds cell 2 and
    # a spend of 1, which leaves player 1's move affordable
    st, acts = start([(3, 26), (50, 28)])
    acts[0, 0, 10] = [PRODUCE, 0, 0, 0, UP, WORKER, 0]
    acts[0, 0, 26] = [PRODUCE, 0, 0, 0, RIGHT, BARRACKS, 0]
    cases.append(("dropped claim", game, st, acts, {
        (0, 0): (PRODUCE, UP, 0, -1, WORKER, 0), (0, 1): (NONE, -1, 1, -1, -1, 1),
        (1, 0): (NONE, -1, -1, -1, -1, 1), (1, 1): (MOVE, LEFT, 0, -1, -1, 0)}))
    return cases


def picks(commands, want):
    return {key: tuple(int(commands[f][0, key[0], key[1]]) for f in FIELDS) for key in want}


@pytest.mark.parametrize("index", range(4))
def test_player_zeros_issued_usage_seeds_player_one_by_hand(index):
    name, game, st, acts, want = seeding_cases()[index]
    got = picks(Oracle(game).gridnet_decode(st, acts), want)
    assert got == want, name


def _gridnet_rows(game, st, per_agent):
    """Per-cell actions [L][2][cells][7]: each unit's JaxMARL row at its cell."""
    L = st["time"].shape[0]
    N, C, cells = game.bucket.neutral_capacity, game.bucket.per_player_capacity, game.bucket.cell_count
    out = np.zeros((L, 2, cells, 7), np.int32)
    for l in range(L):
        for p in range(2):
            for i in range(C):
                s = N + p * C + i
                if st["birth"][l, s] != -1:
                    out[l, p, st["cell"][l, s]] = per_agent[l, p, i]
    return out


@pytest.mark.parametrize("case", ["16x16-finetuned-both", "8x8-original-both", "barracks-random"])
def test_kept_rows_decode_like_jaxmarl_and_keep_the_filter_invariants(case, oracle_threads):
    game, partial = game_for(case)
    oracle, st = advanced_states(game, 64, 300, partial, oracle_threads, seed=19)
    rows = oracle.avail_rows(st)
    sampled = oracle.sample_actions(rows, (7, 8), 3)
    grid = oracle.gridnet_decode(st, _gridnet_rows(game, st, sampled))
    jax_like = oracle.decode_actions(st, sampled)
    b = game.bucket
    N, C, W = b.neutral_capacity, b.per_player_capacity, b.width
    kept_total = dropped_total = 0
    for l in range(64):
        for p in range(2):
            slots = N + p * C + np.arange(C)
            available = (st["birth"][l, slots] != -1) & (st["pending_kind"][l, slots] == -1)
            order = grid["request_order"][l, p]
            kind = grid["kind"][l, p]
            assert ((kind == -1) == ~available).all()
            assert (order[~available] == -1).all()
            # kept rows: the JaxMARL command (NONE waits -1), ranked 0.. in cell order
            fillers = available & (kind == NONE) & (grid["none_duration"][l, p] == 1)
            kept = available & ~fillers
            cells = st["cell"][l, slots]
            kept_idx = np.nonzero(kept)[0]
            assert sorted(order[kept].tolist()) == list(range(kept.sum()))
            assert (np.argsort(cells[kept_idx]) == np.argsort(order[kept_idx])).all()
            for i in kept_idx:
                for f in ("kind", "direction", "target_cell", "produced_type"):
                    assert grid[f][l, p, i] == jax_like[f][l, p, i], (l, p, i, f)
                want_none = -1 if kind[i] == NONE else 0
                assert grid["none_duration"][l, p, i] == want_none
            # fillers: NONE for 1 cycle, ranked after the kept rows by birth
            fill_idx = np.nonzero(fillers)[0]
            births = st["birth"][l, slots][fill_idx]
            assert (np.argsort(births, kind="stable") == np.argsort(order[fill_idx], kind="stable")).all()
            assert sorted(order[fill_idx].tolist()) == list(range(kept.sum(), kept.sum() + len(fill_idx)))
            # no two kept claims of a player share a position
            claims = [cells[i] + STEP[grid["direction"][l, p, i]][0] + W * STEP[grid["direction"][l, p, i]][1]
                      for i in kept_idx if kind[i] in (MOVE, PRODUCE)]
            assert len(claims) == len(set(claims))
            # a dropped row was a claim or a cost (the filter only drops those)
            for i in fill_idx:
                assert jax_like["kind"][l, p, i] in (MOVE, PRODUCE)
                dropped_total += 1
            kept_total += len(kept_idx)
    assert kept_total > 100 and dropped_total > 0


def test_gridnet_sampler_draws_legal_values_with_the_row_sampler_counters(oracle_threads):
    """The harness sampler over per-cell rows: a drawn factor is a set bit of
    its mask (0 for an empty factor), a cell with no row draws zeros, and the
    draw at flattened position q equals the row sampler's draw at its
    position q (same step key, counters (env, 2q) and (env, 2q + 1))."""
    game, partial = game_for("16x16-finetuned-both")
    oracle, st = advanced_states(game, 24, 200, partial, oracle_threads, seed=43)
    b = game.bucket
    L, N, C, cells = 24, b.neutral_capacity, b.per_player_capacity, b.cell_count
    legal = oracle.legality_rows(st)
    rows = np.zeros((L, 2, cells, 78), bool)
    for l in range(L):
        for p in range(2):
            for i in range(C):
                s = N + p * C + i
                if st["birth"][l, s] != -1 and st["pending_kind"][l, s] == -1:
                    rows[l, p, st["cell"][l, s]] = legal[l, p, i]
    got = oracle.gridnet_sample_actions(rows, (3, 4), 7, env0=5)
    lo = np.cumsum((0, 6, 4, 4, 4, 4, 7))
    widths = (6, 4, 4, 4, 4, 7, 49)
    drawn = 0
    for l in range(L):
        for p in range(2):
            for c in range(cells):
                r = rows[l, p, c]
                if not r.any():
                    assert (got[l, p, c] == 0).all()
                    continue
                drawn += 1
                for f in range(7):
                    m = r[lo[f]:lo[f] + widths[f]]
                    assert (m[got[l, p, c, f]] if m.any() else got[l, p, c, f] == 0)
    assert drawn > 20
    flat = rows.reshape(L, 2 * cells, 78)[:, :2 * C].reshape(L, 2, C, 78)
    want = oracle.sample_actions(flat, (3, 4), 7, env0=5)
    np.testing.assert_array_equal(got.reshape(L, 2 * cells, 7)[:, :2 * C], want.reshape(L, 2 * C, 7))
