"""Pins of the CPU oracle (CPU only, no GPU).

Each test checks the oracle against something it does not share code with:
published threefry known answers, the reference's own RNG header built into
oracle/_ref, closed forms from the unit tables (hand-traced cycles on the
shipped 8x8 map), brute force over every single command of a unit (masks
against admission), and closed forms of visibility, symbolic observations,
rewards and the sampler.  A planted mistake in the oracle (a dropped term, a
wrong index or sign) fails at least one of them.
"""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest

from nanorts_amd import keys as hostkeys
from nanorts_amd.content import map_name_to_scenario
from nanorts_amd.model import STATE_LEAVES, ConflictStrategy, UnitTypeTableVersion
from oracle import oracle as orc
from oracle.oracle import Oracle, batch_initial, copy_state
from tests.helpers import CASES, advanced_states, game_for

GOLDEN = Path(__file__).resolve().parent / "golden"

NONE, MOVE, HARVEST, RETURN, PRODUCE, ATTACK = range(6)
UP, RIGHT, DOWN, LEFT = range(4)
WORKER, BASE, RESOURCE = 3, 1, 0

# ---------------------------------------------------------------------------
# RNG
# ---------------------------------------------------------------------------
# Random123 threefry2x32_20 known answers (key, counter) -> output.
THREEFRY_KAT = [
    ((0x00000000, 0x00000000), (0x00000000, 0x00000000), (0x6B200159, 0x99BA4EFE)),
    ((0xFFFFFFFF, 0xFFFFFFFF), (0xFFFFFFFF, 0xFFFFFFFF), (0x1CB996FC, 0xBB002BE7)),
    ((0x13198A2E, 0x03707344), (0x243F6A88, 0x85A308D3), (0xC4923A9C, 0x483DF7A0)),
]


@pytest.mark.parametrize("key,ctr,want", THREEFRY_KAT)
def test_threefry_known_answers(key, ctr, want):
    assert orc.threefry2x32(None, key, ctr) == want
    y0, y1 = hostkeys.threefry2x32(np.asarray(key, np.uint32), np.uint32(ctr[0]), np.uint32(ctr[1]))
    assert (int(y0), int(y1)) == want


def test_threefry_matches_classic_jax_split():
    """jax.random.split(PRNGKey(0)) in JAX's original (non-partitionable)
    scheme is [[4146024105, 967050713], [2718843009, 1272950319]]: it hashes
    the counters (0, 2) and (1, 3) with key (0, 0) and interleaves the halves.
    An independent published vector for the same threefry core."""
    a = orc.threefry2x32(None, (0, 0), (0, 2))
    b = orc.threefry2x32(None, (0, 0), (1, 3))
    assert (a[0], b[0]) == (4146024105, 967050713)
    assert (a[1], b[1]) == (2718843009, 1272950319)


def test_host_keys_match_oracle():
    rng = np.random.default_rng(0)
    for _ in range(64):
        k = rng.integers(0, 2**32, 2, dtype=np.uint64).astype(np.uint32)
        d = int(rng.integers(0, 2**32))
        want = orc.threefry2x32(None, k, (0, d))
        assert tuple(int(v) for v in hostkeys.fold_in(k, d)) == want
    np.testing.assert_array_equal(hostkeys.split(hostkeys.key(7), 5)[3], hostkeys.fold_in(hostkeys.key(7), 3))


def _golden_draws():
    return json.loads((GOLDEN / "conflict_draws.json").read_text())


def test_oracle_draws_match_reference_golden_vectors():
    """Vectors written by tests/golden/make_conflict_draws.py from the
    reference's own conflict_draw.cuh (oracle/_ref)."""
    lib = orc.load_library()
    import ctypes

    data = _golden_draws()
    for row in data["fold_in"]:
        k = (ctypes.c_uint32 * 2)(*row["key"])
        out = (ctypes.c_uint32 * 2)()
        lib.nro_fold_in(k, ctypes.c_uint32(row["data"] & 0xFFFFFFFF), out)
        assert [int(out[0]), int(out[1])] == row["out"]
    for row in data["randint01"]:
        k = (ctypes.c_uint32 * 2)(*row["key"])
        assert lib.nro_randint01(k) == row["out"]
    for row in data["conflict_draw"]:
        k = (ctypes.c_uint32 * 2)(*row["root"])
        got = lib.nro_conflict_draw(k, ctypes.c_int32(row["time"]), ctypes.c_int32(row["birth"]),
                                    ctypes.c_int32(row["ordinal"]))
        assert got == row["out"], row


def test_oracle_draws_match_reference_live():
    ref = orc.load_reference_draws()
    if ref is None:
        pytest.skip("oracle/_ref (the reference's RNG header) is not built here")
    import ctypes

    ref.ref_conflict_draw.restype = ctypes.c_int32
    ref.ref_randint01.restype = ctypes.c_int32
    lib = orc.load_library()
    rng = np.random.default_rng(3)
    ones = 0
    for _ in range(2000):
        root = rng.integers(0, 2**32, 2, dtype=np.uint64).astype(np.uint32)
        t, b, o = (int(v) for v in rng.integers(-5, 6000, 3))
        k = (ctypes.c_uint32 * 2)(*[int(v) for v in root])
        want = ref.ref_conflict_draw(k, ctypes.c_int32(t), ctypes.c_int32(b), ctypes.c_int32(o))
        got = lib.nro_conflict_draw(k, ctypes.c_int32(t), ctypes.c_int32(b), ctypes.c_int32(o))
        assert got == want
        ones += want
    assert 850 < ones < 1150  # a fair coin


def test_drawn_seat_is_randint_of_the_seat_stream():
    """The "drawn" seat (src/nanorts/bots/seat.py:32, 352-360) composes two
    draws the golden vectors pin, fold_in and randint(…, 0, 2), with the seat
    stream 2**32 - 2: it must equal that composition and differ from the
    neighbouring streams (2**32 - 1, 0) and from the root's own draw, which a
    dropped or wrong fold_in would give."""
    import ctypes

    lib = orc.load_library()
    rng = np.random.default_rng(11)
    ones, differs = 0, {0xFFFFFFFF: 0, 0: 0, None: 0}
    for _ in range(2000):
        root = (ctypes.c_uint32 * 2)(*[int(v) for v in rng.integers(0, 2**32, 2, dtype=np.uint64)])
        got = lib.nro_episode_seat(root)

        def draw(stream):
            if stream is None:
                return lib.nro_randint01(root)
            k = (ctypes.c_uint32 * 2)()
            lib.nro_fold_in(root, ctypes.c_uint32(stream), k)
            return lib.nro_randint01(k)

        assert got == draw(2**32 - 2)
        for stream in differs:
            differs[stream] += int(got != draw(stream))
        ones += got
    assert 850 < ones < 1150  # both seats, about evenly
    assert all(count > 800 for count in differs.values()), differs


# ---------------------------------------------------------------------------
# Content
# ---------------------------------------------------------------------------
def test_capacities_and_initial_units():
    def units(game):
        s = game.initial_state
        live = s["birth"] != -1
        return sorted(zip(s["unit_type"][live].tolist(), s["owner"][live].tolist()))

    g8 = map_name_to_scenario("basesWorkers8x8", utt=UnitTypeTableVersion.ORIGINAL)
    assert (g8.bucket.per_player_capacity, g8.bucket.neutral_capacity, g8.bucket.entity_capacity) == (47, 2, 96)
    assert units(g8) == [(0, -1), (0, -1), (1, 0), (1, 1), (3, 0), (3, 1)]
    assert g8.initial_state["carried_resources"][:2].tolist() == [20, 20]
    g16 = map_name_to_scenario("basesWorkers16x16")
    assert (g16.bucket.per_player_capacity, g16.bucket.neutral_capacity, g16.bucket.entity_capacity) == (70, 4, 144)
    assert units(g16).count((0, -1)) == 4 and units(g16).count((3, 0)) == 1 and units(g16).count((1, 1)) == 1
    gow = map_name_to_scenario("GardenOfWar64x64", capacity_profile=False)
    assert (gow.bucket.per_player_capacity, gow.bucket.neutral_capacity, gow.bucket.entity_capacity) == (388, 22, 798)
    assert units(gow).count((3, 0)) == 2 and units(gow).count((3, 1)) == 2 and units(gow).count((0, -1)) == 22
    g16n = map_name_to_scenario("basesWorkers16x16", capacity_profile=False)
    assert g16n.bucket.per_player_capacity == 107


# ---------------------------------------------------------------------------
# Hand-traced cycles on basesWorkers8x8 (2 neutral slots, 47 per player):
#   slot 0/1 resource piles of 20 at cells 0 and 63; player 0 base (slot 2)
#   at cell 10 and worker (slot 3) at cell 9; player 1 base (slot 49) at
#   cell 53 and worker (slot 50) at cell 54; balances 5 / 5.
# ---------------------------------------------------------------------------
def _eight(strategy=ConflictStrategy.CANCEL_BOTH):
    game = map_name_to_scenario("basesWorkers8x8", conflict_strategy=strategy)
    return game, Oracle(game), batch_initial(game, 1, np.asarray([[1, 2]], np.uint32))


def _actions(game, orders: dict) -> np.ndarray:
    """int32[1,2,C,7] rows: every unit NONE except the listed (player, pos)."""
    a = np.zeros((1, 2, game.bucket.per_player_capacity, 7), np.int32)
    for (player, pos), row in orders.items():
        a[0, player, pos] = row
    return a


def _cycle(o: Oracle, game, st, orders=None, key=(1, 2)):
    commands = o.decode_actions(st, _actions(game, orders or {}))
    return o.core_step(st, commands, np.asarray([key], np.uint32))


def _place(st, slot: int, cell: int) -> None:
    old = int(st["cell"][0, slot])
    st["entity_at"].reshape(1, -1)[0, old] = -1
    st["entity_at"].reshape(1, -1)[0, cell] = slot
    st["cell"][0, slot] = cell


def _clear(st, slot: int) -> None:
    st["entity_at"].reshape(1, -1)[0, int(st["cell"][0, slot])] = -1
    for leaf in STATE_LEAVES:
        if leaf.kind == "slot":
            st[leaf.name][0, slot] = leaf.fill


def test_worker_move_completes_after_ten_cycles():
    game, o, st = _eight()
    _cycle(o, game, st, {(0, 1): [MOVE, UP, 0, 0, 0, 0, 0]})
    assert st["pending_kind"][0, 3] == MOVE and st["pending_completes_at"][0, 3] == 10
    for _ in range(8):
        _cycle(o, game, st)
    assert st["cell"][0, 3] == 9 and st["time"][0] == 9
    _cycle(o, game, st)
    assert st["time"][0] == 10 and st["cell"][0, 3] == 1
    assert st["entity_at"][0, 0, 1] == 3 and st["entity_at"][0, 1, 1] == -1
    assert st["pending_kind"][0, 3] == -1
    assert o.violations(st).tolist() == [0]


def test_harvest_then_return_credits_one():
    game, o, st = _eight()
    _place(st, 3, 1)  # worker above its base's row, right of pile 0
    _cycle(o, game, st, {(0, 1): [HARVEST, 0, LEFT, 0, 0, 0, 0]})
    for _ in range(18):
        _cycle(o, game, st)
    assert st["carried_resources"][0, 3] == 0 and st["carried_resources"][0, 0] == 20
    _cycle(o, game, st)  # cycle 20: harvest_time of a worker
    assert st["carried_resources"][0, 3] == 1 and st["carried_resources"][0, 0] == 19
    # back down next to the base (cell 10 is right of cell 9), then return
    _cycle(o, game, st, {(0, 1): [MOVE, DOWN, 0, 0, 0, 0, 0]})
    for _ in range(9):
        _cycle(o, game, st)
    assert st["cell"][0, 3] == 9
    _cycle(o, game, st, {(0, 1): [RETURN, 0, 0, RIGHT, 0, 0, 0]})
    for _ in range(8):
        _cycle(o, game, st)
    assert st["player_resources"][0].tolist() == [5, 5]
    _cycle(o, game, st)  # RETURN takes move_time (10)
    assert st["player_resources"][0].tolist() == [6, 5] and st["carried_resources"][0, 3] == 0
    assert o.violations(st).tolist() == [0]


def test_base_trains_worker_for_one_in_fifty_cycles():
    game, o, st = _eight()
    _cycle(o, game, st, {(0, 0): [PRODUCE, 0, 0, 0, UP, WORKER, 0]})
    for _ in range(48):
        _cycle(o, game, st)
    assert st["player_resources"][0, 0] == 5 and (st["birth"][0] != -1).sum() == 6
    _cycle(o, game, st)
    assert st["player_resources"][0, 0] == 4  # the cost is paid on completion
    slot = 2 + 2  # lowest free slot of player 0's block
    assert st["birth"][0, slot] == 6 and st["unit_type"][0, slot] == WORKER and st["owner"][0, slot] == 0
    assert st["cell"][0, slot] == 2 and st["hit_points"][0, slot] == 1 and st["next_birth"][0] == 7
    assert o.violations(st).tolist() == [0]


def test_attack_kills_and_ends_the_game():
    game, o, st = _eight()
    _clear(st, 49)  # player 1 keeps only its worker
    _place(st, 50, 17)  # below player 0's worker
    off = (1 + 3) * 7 + (0 + 3)  # dy = +1, dx = 0
    out = _cycle(o, game, st, {(0, 1): [ATTACK, 0, 0, 0, 0, 0, off]})
    assert out["admitted_attack"][0, 0].tolist() == [0, 0, 1]  # by target owner -1 / 0 / 1
    for _ in range(3):
        out = _cycle(o, game, st)
        assert not out["terminated"][0]
    out = _cycle(o, game, st)  # attack_time 5
    assert st["birth"][0, 50] == -1 and st["entity_at"][0, 2, 1] == -1
    assert out["terminated"][0] and st["winner"][0] == 0
    assert out["reward"][0].tolist() == [1.0, -1.0]


def _same_cycle_race(strategy, root=(1, 2), alternating=0):
    game, o, st = _eight(strategy)
    _place(st, 50, 2)
    st["alternating_conflict_count"][0] = alternating
    _cycle(o, game, st, {(0, 1): [MOVE, UP, 0, 0, 0, 0, 0], (1, 1): [MOVE, LEFT, 0, 0, 0, 0, 0]}, key=root)
    for _ in range(12):
        _cycle(o, game, st, key=root)
    assert o.violations(st).tolist() == [0]
    return st


def test_same_cycle_conflict_cancel_both():
    st = _same_cycle_race(ConflictStrategy.CANCEL_BOTH)
    assert st["cell"][0, 3] == 9 and st["cell"][0, 50] == 2


@pytest.mark.parametrize("alternating,mover", [(0, 3), (1, 50), (6, 3)])
def test_same_cycle_conflict_alternating(alternating, mover):
    """Player 1's request is admitted second; with an even running count the
    request is cancelled (the pending MOVE survives), with an odd one the
    pending MOVE is cancelled."""
    st = _same_cycle_race(ConflictStrategy.CANCEL_ALTERNATING, alternating=alternating)
    assert st["cell"][0, mover] == 1
    other = 50 if mover == 3 else 3
    assert st["cell"][0, other] == (2 if other == 50 else 9)
    assert st["alternating_conflict_count"][0] == alternating + 1


def test_same_cycle_conflict_random_follows_reference_draw():
    """CANCEL_RANDOM: the later request (player 1's worker, birth 5) is
    cancelled iff the draw at (root, time 0, birth 5, ordinal 0) is 0.  The
    draws come from the reference's own conflict_draw.cuh (golden vectors)."""
    draws = {tuple(r["root"]): r["out"] for r in _golden_draws()["race"]}
    seen = set()
    for root, draw in draws.items():
        st = _same_cycle_race(ConflictStrategy.CANCEL_RANDOM, root=root)
        mover = 3 if draw == 0 else 50
        assert st["cell"][0, mover] == 1, (root, draw)
        seen.add(draw)
    assert seen == {0, 1}


def test_cross_cycle_conflict_cancels_the_request():
    game, o, st = _eight(ConflictStrategy.CANCEL_RANDOM)
    _place(st, 50, 2)
    _cycle(o, game, st, {(0, 1): [MOVE, UP, 0, 0, 0, 0, 0], (1, 1): [NONE, 0, 0, 0, 0, 0, 0]})
    _cycle(o, game, st, {(1, 1): [MOVE, LEFT, 0, 0, 0, 0, 0]})
    # cancelled with duration -1: due at once, the worker is free again
    assert st["pending_kind"][0, 50] == -1 and st["pending_kind"][0, 3] == MOVE
    for _ in range(8):
        _cycle(o, game, st)
    assert st["cell"][0, 3] == 1 and st["cell"][0, 50] == 2


# ---------------------------------------------------------------------------
# Masks against admission, by brute force over every single command
# ---------------------------------------------------------------------------
def _decode_row(width_t: int, kind: int, param: int) -> list[int]:
    row = [kind, 0, 0, 0, 0, 0, 0]
    if kind in (MOVE, HARVEST, RETURN):
        row[kind] = param
    elif kind == PRODUCE:
        row[4], row[5] = param % 4, param // 4
    elif kind == ATTACK:
        row[6] = param
    return row


def _masks_against_admission(game, o, st) -> int:
    """For every available unit of every env of `st` and every single
    command: a mask-legal command is admitted as itself (unless a pending
    MOVE/PRODUCE of another unit conflicts with it), a mask-illegal one
    becomes NONE for the requested duration.  Every active unit's row has its
    NONE bit (core/kinds/none.py:19-20: `grid.active`).  Returns the number
    of commands tried."""
    b = game.bucket
    T, C, N = b.unit_type_capacity, b.per_player_capacity, b.neutral_capacity
    rows = o.legality_rows(st)
    checked = 0
    for l in range(st["time"].shape[0]):
        one = {k: np.ascontiguousarray(v[l:l + 1]) for k, v in st.items()}
        pending_claims = ((one["pending_kind"][0] == MOVE) | (one["pending_kind"][0] == PRODUCE)).any()
        for player in (0, 1):
            for pos in range(C):
                slot = N + player * C + pos
                active = one["birth"][0, slot] != -1
                assert rows[l, player, pos, NONE] == active, (l, slot)
                if not active:
                    assert not rows[l, player, pos].any(), (l, slot)
                if not active or one["pending_kind"][0, slot] != -1:
                    continue
                utype = int(one["unit_type"][0, slot])
                for kind, params in ((MOVE, 4), (HARVEST, 4), (RETURN, 4), (PRODUCE, 4 * T), (ATTACK, b.attack_offset_capacity)):
                    for param in range(params):
                        row = _decode_row(T, kind, param)
                        if kind == PRODUCE:
                            legal = rows[l, player, pos, 18 + row[4]] and rows[l, player, pos, 22 + row[5]] \
                                and rows[l, player, pos, PRODUCE]
                        else:
                            base = {MOVE: 6, HARVEST: 10, RETURN: 14, ATTACK: 22 + T}[kind]
                            legal = rows[l, player, pos, kind] and rows[l, player, pos, base + param]
                        trial = copy_state(one)
                        _cycle(o, game, trial, {(player, pos): row})
                        got = int(trial["pending_kind"][0, slot])
                        completes = int(trial["pending_completes_at"][0, slot]) - int(one["time"][0])
                        cols = game.columns
                        duration = {MOVE: cols["move_time"][utype], HARVEST: cols["harvest_time"][utype],
                                    RETURN: cols["move_time"][utype], ATTACK: cols["attack_time"][utype],
                                    PRODUCE: cols["produce_time"][min(max(row[5], 0), T - 1)]}[kind]
                        if legal:
                            if got == kind:
                                assert completes == duration
                            else:
                                assert kind in (MOVE, PRODUCE) and pending_claims, (l, slot, kind, param, got)
                        else:
                            # NONE for the requested duration (completed at once
                            # only when the duration is < 1)
                            if duration >= 1:
                                assert got == NONE and completes == duration, (l, slot, kind, param, got, completes)
                        checked += 1
    return checked


@pytest.mark.parametrize("case", ["16x16-finetuned-both", "melee-both", "barracks-random"])
def test_mask_bits_agree_with_admission(case):
    """Mid-game states of three games (90 random cycles)."""
    game, partial = game_for(case)
    o, st = advanced_states(game, 10, 90, partial, 4, seed=19)
    assert _masks_against_admission(game, o, st) > 400


@pytest.mark.parametrize("melee_pair", [False, True])
def test_mask_bits_agree_with_admission_on_built_positions(melee_pair):
    """Positions the random ones rarely reach: a carrying worker between its
    own base and the enemy's, a melee unit next to an enemy building (and,
    with `melee_pair`, next to an enemy Light), a Ranged unit with targets at
    and beyond range 3, and available buildings."""
    from tests.test_oracle_rules import _built_position

    bd = _built_position()
    if melee_pair:
        bd.place(51, 22)  # right of player 0's Light at cell 21
    rows = bd.o.legality_rows(bd.st)
    assert rows[0, 0, 3, ATTACK] == melee_pair  # player 0's Light (slot 5, position 3)
    assert _masks_against_admission(bd.game, bd.o, bd.st) > 600


# ---------------------------------------------------------------------------
# Closed forms: visibility, symbolic observation, rewards, invariants
# ---------------------------------------------------------------------------
def _closed_visibility(game, st, observer):
    b = game.bucket
    H, W, C, N = b.height, b.width, b.per_player_capacity, b.neutral_capacity
    sight = game.columns["sight_radius"]
    L = st["time"].shape[0]
    yy, xx = np.mgrid[0:H, 0:W]
    out = np.zeros((L, H, W), bool)
    for l in range(L):
        for s in range(N + observer * C, N + (observer + 1) * C):
            if st["birth"][l, s] == -1:
                continue
            cy, cx = divmod(int(st["cell"][l, s]), W)
            r = int(sight[st["unit_type"][l, s]])
            out[l] |= (yy - cy) ** 2 + (xx - cx) ** 2 <= r * r
    return out


def _closed_symbolic(game, st, partial):
    b = game.bucket
    H, W = b.height, b.width
    L = st["time"].shape[0]
    maps = np.zeros((L, 2, H, W, 6), np.uint8)
    scal = np.zeros((L, 2, 4), np.int32)
    for observer in (0, 1):
        vis = _closed_visibility(game, st, observer)
        for l in range(L):
            for c in range(H * W):
                y, x = divmod(c, W)
                maps[l, observer, y, x, 5] = game.terrain.reshape(-1)[c]
                s = int(st["entity_at"][l, y, x])
                if s == -1:
                    continue
                owner = int(st["owner"][l, s])
                if partial and owner != observer and not vis[l, y, x]:
                    continue
                maps[l, observer, y, x, 0] = st["hit_points"][l, s]
                maps[l, observer, y, x, 1] = st["carried_resources"][l, s]
                maps[l, observer, y, x, 2] = 0 if owner < 0 else (1 if owner == observer else 2)
                maps[l, observer, y, x, 3] = st["unit_type"][l, s] + 1
                maps[l, observer, y, x, 4] = max(int(st["pending_kind"][l, s]), 0)
            res = st["player_resources"][l]
            scal[l, observer] = [res[observer], res[1 - observer], st["time"][l],
                                 st["alternating_conflict_count"][l]]
    return maps, scal


@pytest.mark.parametrize("case", ["16x16-random-partial", "melee-both", "obstacle-alternating"])
def test_visibility_and_symbolic_closed_form(case):
    game, _ = game_for(case)
    o, st = advanced_states(game, 8, 160, True, 4, seed=5)
    for observer in (0, 1):
        np.testing.assert_array_equal(o.visible_cells(st, observer), _closed_visibility(game, st, observer))
    for partial in (False, True):
        maps, scal = o.symbolic(st, partial)
        want_maps, want_scal = _closed_symbolic(game, st, partial)
        np.testing.assert_array_equal(maps, want_maps)
        np.testing.assert_array_equal(scal, want_scal)


@pytest.mark.parametrize("case", list(CASES))
def test_rollout_invariants_and_rewards(case):
    game, partial = game_for(case)
    L = 4 if case.startswith("gow") else 24
    steps = 60 if case.startswith("gow") else 400
    o, st = advanced_states(game, L, 0, partial, 4, seed=2)
    res = o.rollout(st, (4, 4), 0, steps, partial, threads=4)
    assert (o.violations(st) == 0).all()
    rewards, dones = res["rewards"], res["dones"].astype(bool)
    # reward[p] = ended ? (p == winner ? 1 : -1) : 0, so every done cycle
    # pays (1, -1), (-1, 1) or, with no winner, (-1, -1)
    assert (rewards[~dones] == 0).all()
    ended = {tuple(r) for r in rewards[dones].tolist()}
    assert ended <= {(1.0, -1.0), (-1.0, 1.0), (-1.0, -1.0)}
    assert (st["time"] >= 0).all() and (st["next_birth"] >= 0).all()


# ---------------------------------------------------------------------------
# Synthetic sampler
# ---------------------------------------------------------------------------
def _row_fields(T, O):
    return [(0, 6), (6, 4), (10, 4), (14, 4), (18, 4), (22, T), (22 + T, O)]


def test_sampler_picks_legal_bits_and_is_uniform():
    game, partial = game_for("16x16-finetuned-both")
    o, st = advanced_states(game, 32, 120, partial, 4, seed=9)
    rows = o.avail_rows(st)
    b = game.bucket
    fields = _row_fields(b.unit_type_capacity, b.attack_offset_capacity)
    counts = {}
    for step in range(200):
        acts = o.sample_actions(rows, (8, 9), step)
        for l, p, c in zip(*np.nonzero(rows.any(-1))):
            row = rows[l, p, c]
            if row.sum() == 1 and row[0]:
                assert (acts[l, p, c] == 0).all()
                continue
            for f, (lo, width) in enumerate(fields):
                bits = np.nonzero(row[lo:lo + width])[0]
                v = acts[l, p, c, f]
                if len(bits) == 0:
                    assert v == 0
                else:
                    assert v in bits
                    if f == 0 and step < 200:
                        counts.setdefault((l, p, c), {}).setdefault(int(v), 0)
                        counts[(l, p, c)][int(v)] += 1
    # kind factor: each legal kind drawn roughly 200 / popcount times
    for key, hist in counts.items():
        row = rows[key][0:6]
        n = int(row.sum())
        for k in np.nonzero(row)[0]:
            assert abs(hist.get(int(k), 0) - 200 / n) < 6 * np.sqrt(200 / n) + 3, (key, hist)
    # distinct envs, steps and keys draw differently
    a = o.sample_actions(rows, (8, 9), 0)
    assert not np.array_equal(a, o.sample_actions(rows, (8, 9), 1))
    assert not np.array_equal(a, o.sample_actions(rows, (8, 10), 0))
    assert not np.array_equal(a[:16], o.sample_actions(rows[:16], (8, 9), 0, env0=16))


def test_decode_actions_closed_form():
    """decode_actions (adapters/jaxmarl/actions.py:61-84, factors.py:117-151)
    worked out by hand on basesWorkers8x8 (C 47): the direction comes from the
    kind's own column, the produced type only for PRODUCE, the target cell
    only for an on-board ATTACK (7x7 window, radius 3), a NONE lasts 1 cycle,
    and a position without an available unit issues nothing."""
    game, o, st = _eight()
    st["pending_kind"][0, 50] = MOVE  # player 1's worker is busy
    rows = _actions(game, {
        (0, 0): [PRODUCE, 3, 2, 1, UP, WORKER, 11],       # base: direction UP, Worker
        (0, 1): [ATTACK, 1, 2, 3, 1, 2, (0 + 3) * 7 + (2 + 3)],  # worker (1,1): (+2, 0) -> cell 11
        (1, 0): [NONE, 3, 3, 3, 3, 3, 40],                # base: NONE for 1
        (1, 1): [MOVE, LEFT, 0, 0, 0, 0, 0],              # busy: not issued
        (0, 2): [MOVE, UP, 0, 0, 0, 0, 0],                # empty position: not issued
    })
    c = o.decode_actions(st, rows)
    got = {f: c[f][0] for f in ("kind", "direction", "none_duration", "target_cell", "produced_type", "request_order")}
    want = {
        (0, 0): (PRODUCE, UP, 0, -1, WORKER, -1),
        (0, 1): (ATTACK, -1, 0, 11, -1, -1),
        (1, 0): (NONE, -1, 1, -1, -1, -1),
        (1, 1): (-1, -1, 0, -1, -1, -1),
        (0, 2): (-1, -1, 0, -1, -1, -1),
    }
    names = ("kind", "direction", "none_duration", "target_cell", "produced_type", "request_order")
    for (p, pos), fields in want.items():
        assert tuple(int(got[n][p, pos]) for n in names) == fields, (p, pos)
    # HARVEST / RETURN read their own columns; an ATTACK off the board has no
    # target: the worker at (1,1) aiming (-3, 0) -> x = -2
    st["pending_kind"][0, 50] = -1
    rows = _actions(game, {(0, 1): [HARVEST, 1, 2, 3, 0, 0, 0], (1, 1): [RETURN, 1, 2, 3, 0, 0, 0]})
    c = o.decode_actions(st, rows)
    assert (int(c["direction"][0, 0, 1]), int(c["direction"][0, 1, 1])) == (2, 3)
    rows = _actions(game, {(0, 1): [ATTACK, 0, 0, 0, 0, 0, (0 + 3) * 7 + (-3 + 3)]})
    c = o.decode_actions(st, rows)
    assert int(c["kind"][0, 0, 1]) == ATTACK and int(c["target_cell"][0, 0, 1]) == -1


def test_sampler_follows_its_definition():
    """The harness sampler's definition, restated in numpy over the host
    threefry (itself pinned by the known answers above): per step the key is
    fold_in(sample_key, step); position p = player * C + row of env e draws
    (w0, w1) = threefry(k, (e, 2p)) and (w2, w3) = threefry(k, (e, 2p + 1));
    factor f takes the 16-bit half f of w0..w3 (low half first) and picks the
    ((h * popcount) >> 16)-th set bit of its mask, 0 when none is set; a row
    with only the NONE bit comes out all zeros."""
    from nanorts_amd import keys as hostkeys

    game, partial = game_for("16x16-finetuned-both")
    o, st = advanced_states(game, 6, 60, partial, 4, seed=5)
    rows = o.avail_rows(st)
    b = game.bucket
    C = b.per_player_capacity
    fields = _row_fields(b.unit_type_capacity, b.attack_offset_capacity)
    sample_key = np.asarray([8, 9], np.uint32)
    for step, env0 in ((0, 0), (7, 0), (3, 100)):
        got = o.sample_actions(rows, sample_key, step, env0=env0)
        k = hostkeys.fold_in(sample_key, step)
        for l in range(rows.shape[0]):
            for player in (0, 1):
                for c in range(C):
                    row = rows[l, player, c]
                    if row[0] and row.sum() == 1:
                        assert (got[l, player, c] == 0).all()
                        continue
                    p = player * C + c
                    w0, w1 = hostkeys.threefry2x32(k, np.uint32(env0 + l), np.uint32(2 * p))
                    w2, w3 = hostkeys.threefry2x32(k, np.uint32(env0 + l), np.uint32(2 * p + 1))
                    words = [int(w0), int(w1), int(w2), int(w3)]
                    for f, (lo, width) in enumerate(fields):
                        h = (words[f // 2] >> (16 * (f % 2))) & 0xFFFF
                        bits = np.nonzero(row[lo:lo + width])[0]
                        want = int(bits[(h * len(bits)) >> 16]) if len(bits) else 0
                        assert int(got[l, player, c, f]) == want, (step, l, player, c, f)
