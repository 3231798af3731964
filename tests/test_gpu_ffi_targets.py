"""The operand-form entries of the bots, the A* targets, the GridNet decode and
the multi-group step, on the GPU, each called through ctypes with the
reference's operand and result order and compared bit for bit with the
oracle:

- nanorts_amd_step_groups_ffi: the FFI target nanorts_step_groups
  (src/nanorts/core/cuda/step.cu:704-808): five groups in one call (two
  launches), with per-lane and broadcast keys and Commands, aliased and
  separate results, against the oracle's core.step per group;
- nanorts_amd_abstraction_act_ffi: nanorts_abstraction_act
  (src/nanorts/bots/cuda/abstraction_act.cu:1231-1324, operands of
  src/nanorts/bots/whole_act.py:125-162): both rush strategies and seats,
  the player and the State leaves per lane or shared, the carry aliased or
  not, against the oracle's family.act;
- nanorts_amd_astar_search_ffi / nanorts_amd_astar_chain_ffi:
  nanorts_astar_search and nanorts_astar_chain
  (src/nanorts/bots/cuda/pathfinding.cu:20-104, abstraction.cu:98-301)
  against the oracle's A* and chain walk on random boards, rows and draws;
- nanorts_amd_gridnet_decode_ffi: nanorts_gridnet_decode
  (src/nanorts/adapters/gridnet/cuda/decode.cu:426-540, operands of
  src/nanorts/adapters/gridnet/actions.py:199-232) with player 0's legality
  operands, against the oracle's GridNet decode.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from nanorts_amd.model import LEAF_NAMES
from oracle.oracle import ABSTRACT_FIELDS, Oracle, astar, astar_chain, batch_initial, copy_state, empty_carry
from tests.helpers import advanced_states, assert_states_equal, game_for, roots
from tests.test_gpu_ffi import COMMAND_FIELDS, reference_tables

pytestmark = pytest.mark.gpu

D = "cuda:0"
ACT_LEAVES = ("birth", "unit_type", "owner", "cell", "carried_resources", "pending_kind", "pending_direction",
              "pending_produced_type", "entity_at", "player_resources")
BOT_TABLE = ("can_harvest", "is_resource", "is_stockpile", "can_attack", "attack_range", "cost")
WORKER_RUSH, BARRACKS_RUSH, LIGHT = 0, 1, 4


class Keep:
    """Device copies of host arrays, kept alive for the call."""

    def __init__(self):
        self.tensors = []

    def __call__(self, array):
        import torch

        t = torch.as_tensor(np.ascontiguousarray(array), device=D)
        self.tensors.append(t)
        return t


def _lib():
    from nanorts_amd import native

    return native.load()


def _stream() -> int:
    import torch

    return torch.cuda.current_stream().cuda_stream


def _ok(code):
    assert code == 0, _lib().nanorts_amd_last_error().decode()


# ---------------------------------------------------------------------------
# nanorts_step_groups
# ---------------------------------------------------------------------------
def test_step_groups_ffi_matches_oracle(oracle_threads):
    import torch

    from nanorts_amd.model import STRATEGY_CODES

    print("step_groups_ffi", flush=True)
    game, partial = game_for("16x16-random-partial")
    b = game.bucket
    E, T = b.entity_capacity, b.unit_type_capacity
    table, timings = reference_tables(game)
    sizes, alias, broadcast = (64, 32, 16, 8, 4), (True, False, True, False, True), (False, True, False, False, True)
    keep = Keep()
    operands, results, lanes, key_lanes, command_lanes, expect = [], [], [], [], [], []
    rng = np.random.default_rng(17)
    for k, L in enumerate(sizes):
        oracle, st = advanced_states(game, L, 60 + 10 * k, partial, oracle_threads, seed=40 + k)
        cmds = oracle.decode_actions(st, oracle.sample_actions(oracle.avail_rows(st), (3, k), 5))
        keys = rng.integers(0, 2**32, size=(L, 2), dtype=np.uint64).astype(np.uint32)
        if broadcast[k]:
            cmds = {f: np.ascontiguousarray(v[:1]) for f, v in cmds.items()}
            keys = keys[:1]
            want_cmds = {f: np.ascontiguousarray(np.broadcast_to(v, (L, *v.shape[1:]))) for f, v in cmds.items()}
            want_keys = np.ascontiguousarray(np.broadcast_to(keys, (L, 2)))
        else:
            want_cmds, want_keys = cmds, keys
        leaves = [keep(st[name]) for name in LEAF_NAMES]
        operands += [keep(keys)] + [keep(cmds[f]) for f in COMMAND_FIELDS] + \
            [keep(game.terrain.astype(np.bool_)[None]), keep(table), keep(timings)] + leaves
        written = leaves if alias[k] else [keep(np.full_like(st[name], 77)) for name in LEAF_NAMES]
        events = [keep(np.full(shape, -7, dtype)) for shape, dtype in (
            ((L, 2), np.int32), ((L, 2), np.int32), ((L, 2, T), np.int32), ((L, 2, 3), np.int32),
            ((L, E), np.bool_), ((L, E, 6), np.int32), ((L, E, 4), np.int16), ((L, E, 6), np.int8))]
        results += written + events
        lanes.append(L)
        key_lanes.append(keys.shape[0])
        command_lanes.append(cmds["kind"].shape[0])
        want_state = copy_state(st)
        want = oracle.core_step(want_state, want_cmds, want_keys)
        expect.append((written, events, want_state, want))
    ops = (ctypes.c_void_p * len(operands))(*[t.data_ptr() for t in operands])
    rets = (ctypes.c_void_p * len(results))(*[t.data_ptr() for t in results])
    I64 = ctypes.c_int64 * len(sizes)
    _ok(_lib().nanorts_amd_step_groups_ffi(_stream(), len(sizes), ops, rets, I64(*lanes), I64(*key_lanes),
                                           I64(*command_lanes), b.height, b.width, b.neutral_capacity,
                                           b.per_player_capacity, T, STRATEGY_CODES[b.conflict_strategy]))
    torch.cuda.synchronize()
    for k, (written, events, want_state, want) in enumerate(expect):
        got = {name: t.cpu().numpy() for name, t in zip(LEAF_NAMES, written)}
        assert_states_equal({n: v for n, v in want_state.items() if n in got}, got, f"group {k}")
        for name, value in zip(("admitted_harvest", "admitted_return", "admitted_produce", "admitted_attack"),
                               events):
            np.testing.assert_array_equal(value.cpu().numpy(), want[name], err_msg=f"group {k} {name}")
        for value, name in zip(events[4:], ("is_member", "records_i32", "records_i16", "records_i8")):
            np.testing.assert_array_equal(value.cpu().numpy().astype(want[name].dtype), want[name],
                                          err_msg=f"group {k} {name}")


# ---------------------------------------------------------------------------
# nanorts_abstraction_act
# ---------------------------------------------------------------------------
def _act_ffi(game, st, carry, strategy, player, *, shared_state: bool, shared_player: bool, alias: bool):
    import torch

    b = game.bucket
    L = st["time"].shape[0]
    keep = Keep()
    rows = {k: np.ascontiguousarray(v[:1]) if shared_state else v for k, v in st.items()}
    state_ops = [keep(rows[name]) for name in ACT_LEAVES]
    cols = game.columns
    table = np.stack([cols[c].astype(np.int32) for c in BOT_TABLE], -1)[None]
    players = np.full((1 if shared_player else L,), player, np.int32)
    carry_ops = [keep(carry[f].astype(np.bool_) if f == "trained" else carry[f]) for f in ABSTRACT_FIELDS]
    carry_out = carry_ops if alias else [keep(np.zeros_like(carry[f], np.bool_ if f == "trained" else None))
                                         for f in ABSTRACT_FIELDS]
    commands = keep(np.full((L, 6, 2, b.per_player_capacity), -9, np.int32))
    operands = state_ops + [keep(game.terrain.astype(np.bool_)[None]), keep(table), keep(players)] + carry_ops
    results = carry_out + [commands]
    extents = [1 if shared_state else L] * 10 + [1, 1, players.shape[0]]
    ops = (ctypes.c_void_p * 24)(*[t.data_ptr() for t in operands])
    rets = (ctypes.c_void_p * 12)(*[t.data_ptr() for t in results])
    _ok(_lib().nanorts_amd_abstraction_act_ffi(_stream(), ops, (ctypes.c_int64 * 13)(*extents), rets, L, b.height,
                                               b.width, b.entity_capacity, b.per_player_capacity,
                                               b.unit_type_capacity, strategy, LIGHT))
    torch.cuda.synchronize()
    got_carry = {f: t.cpu().numpy() for f, t in zip(ABSTRACT_FIELDS, carry_out)}
    got_carry["trained"] = got_carry["trained"].astype(np.uint8)
    return commands.cpu().numpy(), got_carry


@pytest.mark.parametrize("case", ["16x16-finetuned-both", "barracks-random"])
@pytest.mark.parametrize("shared_state,shared_player,alias", [(False, True, True), (False, False, False),
                                                              (True, True, False)])
def test_abstraction_act_ffi_matches_oracle(case, shared_state, shared_player, alias, oracle_threads):
    print(f"abstraction_act_ffi {case} shared_state={shared_state} shared_player={shared_player} alias={alias}",
          flush=True)
    game, _ = game_for(case)
    o = Oracle(game)
    C = game.bucket.per_player_capacity
    L = 32
    st = batch_initial(game, L, roots(L, 8))
    carry = empty_carry(L, C)
    checked = 0
    for t in range(121):
        if t in (0, 1, 40, 120):
            for strategy in (WORKER_RUSH, BARRACKS_RUSH):
                for player in (0, 1):
                    now = {k: np.ascontiguousarray(np.broadcast_to(v[:1], v.shape)) for k, v in st.items()} \
                        if shared_state else copy_state(st)
                    start = {k: np.ascontiguousarray(np.broadcast_to(v[:1], v.shape)) for k, v in carry.items()} \
                        if shared_state else copy_state(carry)
                    want_carry = copy_state(start)
                    want = o.abstraction_act(copy_state(now), want_carry, strategy, LIGHT, player)
                    got, got_carry = _act_ffi(game, now, copy_state(start), strategy, player,
                                              shared_state=shared_state, shared_player=shared_player, alias=alias)
                    where = f"{case} t={t} strategy={strategy} player={player}"
                    for i, f in enumerate(COMMAND_FIELDS):
                        np.testing.assert_array_equal(got[:, i], want[f], err_msg=f"{where}: {f}")
                    for f in ABSTRACT_FIELDS:
                        np.testing.assert_array_equal(got_carry[f].astype(np.int64), want_carry[f].astype(np.int64),
                                                      err_msg=f"{where}: carry {f}")
                    checked += 1
        rows = o.sample_actions(o.avail_rows(st), (41, 43), t)[:, 0]
        o.seat_step(st, carry, WORKER_RUSH, LIGHT, 0, np.ascontiguousarray(rows), False, observe=False)
    assert checked == 16


# ---------------------------------------------------------------------------
# nanorts_astar_search / nanorts_astar_chain
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("H,W", [(16, 16), (8, 8), (7, 1), (1, 9), (64, 64)])
def test_astar_search_ffi_matches_oracle(H, W):
    import torch

    print(f"astar_search_ffi {H}x{W}", flush=True)
    rng = np.random.default_rng(H * 100 + W)
    L = 96
    cells = H * W
    free = rng.random((L, H, W)) < 0.72
    start = rng.integers(-2, cells + 2, L).astype(np.int32)  # a few off the board
    target = rng.integers(0, cells, L).astype(np.int32)
    rng_ = rng.integers(0, 3, L).astype(np.int32)
    keep = Keep()
    out = keep(np.full((L, 4), -9, np.int32))
    _ok(_lib().nanorts_amd_astar_search_ffi(_stream(), keep(free).data_ptr(), L, keep(start).data_ptr(), L,
                                            keep(target).data_ptr(), L, keep(rng_).data_ptr(), L, W, H,
                                            out.data_ptr(), L))
    # one shared board and range for every lane
    out1 = keep(np.full((L, 4), -9, np.int32))
    _ok(_lib().nanorts_amd_astar_search_ffi(_stream(), keep(free[:1]).data_ptr(), 1, keep(start).data_ptr(), L,
                                            keep(target).data_ptr(), L, keep(rng_[:1]).data_ptr(), 1, W, H,
                                            out1.data_ptr(), L))
    torch.cuda.synchronize()
    got, got1 = out.cpu().numpy(), out1.cpu().numpy()
    found = 0
    for l in range(L):
        want = astar(free[l], int(start[l]), int(target[l]), int(rng_[l]))
        assert tuple(got[l]) == want, (l, int(start[l]), int(target[l]), int(rng_[l]))
        assert tuple(got1[l]) == astar(free[0], int(start[l]), int(target[l]), int(rng_[0])), l
        found += want[0]
    assert 0 < found < L


@pytest.mark.parametrize("drawing", [False, True])
@pytest.mark.parametrize("shared", [False, True])
def test_astar_chain_ffi_matches_oracle(drawing, shared):
    import torch

    print(f"astar_chain_ffi drawing={drawing} shared={shared}", flush=True)
    rng = np.random.default_rng(3 + 2 * drawing + shared)
    L, H, W, capacity, columns = 48, 12, 12, 24, 11
    cells = H * W
    fallback, blocked = (5, 6, 7), (8, 9, 10)
    free = rng.random((L, H, W)) < 0.8
    claimed = rng.random((L, H, W)) < 0.08
    rows = np.zeros((L, capacity, columns), np.int32)
    rows[..., 0] = rng.integers(0, cells, (L, capacity))
    rows[..., 1] = rng.integers(0, cells, (L, capacity))
    rows[..., 2] = rng.integers(0, 2, (L, capacity))
    rows[..., 3] = rng.integers(0, 2, (L, capacity))
    rows[..., 4] = rng.integers(0, 16, (L, capacity))
    for base in (5, 8):
        rows[..., base] = rng.choice([-1, 1, 4], (L, capacity))
        rows[..., base + 1] = rng.integers(-3, cells + 3, (L, capacity))
        rows[..., base + 2] = rng.choice([0, 0, 1, 2, 5], (L, capacity))
    queue = np.stack([rng.permutation(capacity) for _ in range(L)]).astype(np.int32)
    queue[:, -2] = capacity + 3  # an out-of-range entry
    count = rng.integers(-1, capacity + 3, L).astype(np.int32)
    moves = rng.random(L) < 0.7
    reserved = rng.integers(0, 4, L).astype(np.int32)
    balance = rng.integers(0, 12, L).astype(np.int32)
    draws = rng.integers(0, 4, (L, 7)).astype(np.int32)
    ops_host = [free, claimed, rows, queue, count, moves, reserved, balance, draws]
    if shared:  # every operand one shared row
        ops_host = [np.ascontiguousarray(x[:1]) for x in ops_host]
    keep = Keep()
    operands = [keep(x) for x in ops_host]
    out = keep(np.full((L, capacity + 1, 4), -9, np.int32))
    extents = [x.shape[0] for x in ops_host]
    _ok(_lib().nanorts_amd_astar_chain_ffi(_stream(), (ctypes.c_void_p * 9)(*[t.data_ptr() for t in operands]),
                                           (ctypes.c_int64 * 9)(*extents), out.data_ptr(), L, W, H, capacity, columns,
                                           7, int(drawing), (ctypes.c_int64 * 3)(*fallback),
                                           (ctypes.c_int64 * 3)(*blocked)))
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    kept = 0
    for l in range(L):
        r = 0 if shared else l
        want = astar_chain(free[r], claimed[r], rows[r], queue[r], int(count[r]), bool(moves[r]), int(reserved[r]),
                           int(balance[r]), draws[r], drawing, fallback, blocked)
        np.testing.assert_array_equal(got[l], want, err_msg=f"lane {l}")
        kept += int(want[capacity, 0])
    assert kept > 0


# ---------------------------------------------------------------------------
# nanorts_gridnet_decode
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("case", ["16x16-finetuned-both", "barracks-random"])
@pytest.mark.parametrize("shared", [False, True])
def test_gridnet_decode_ffi_matches_oracle(case, shared, oracle_threads):
    import torch

    from tests.test_gpu_gridnet import _per_cell_actions

    print(f"gridnet_decode_ffi {case} shared={shared}", flush=True)
    game, partial = game_for(case)
    b = game.bucket
    L, C, T = 64, b.per_player_capacity, b.unit_type_capacity
    oracle, st = advanced_states(game, L, 120, partial, oracle_threads, seed=29)
    acts = _per_cell_actions(game, oracle, st, 7)
    if shared:
        st = {k: np.ascontiguousarray(np.broadcast_to(v[:1], v.shape)) for k, v in st.items()}
        acts = np.ascontiguousarray(np.broadcast_to(acts[:1], acts.shape))
    rows = oracle.legality_rows(st)[:, 0]  # player 0's rows [L][C][78]
    legal = [rows[..., 6:10], rows[..., 18:22], rows[..., 22:22 + T]]
    want = oracle.gridnet_decode(st, acts)
    keep = Keep()
    host = [acts.reshape(L, 2, b.height, b.width, 7)] + [st[n] for n in (
        "birth", "pending_kind", "cell", "pending_direction", "pending_produced_type", "player_resources")] + \
        [x.astype(np.bool_) for x in legal]
    if shared:
        host = [np.ascontiguousarray(x[:1]) for x in host]
    operands = [keep(x) for x in host] + [keep(game.columns["cost"].astype(np.int32))]
    extents = [x.shape[0] for x in host] + [1]
    out = [keep(np.full((L, 2, C), -9, np.int32)) for _ in COMMAND_FIELDS]
    side = int(round(b.attack_offset_capacity ** 0.5))
    _ok(_lib().nanorts_amd_gridnet_decode_ffi(_stream(), (ctypes.c_void_p * 11)(*[t.data_ptr() for t in operands]),
                                              (ctypes.c_int64 * 11)(*extents),
                                              (ctypes.c_void_p * 6)(*[t.data_ptr() for t in out]), L, b.height,
                                              b.width, b.neutral_capacity, C, T, T, side))
    torch.cuda.synchronize()
    for f, t in zip(COMMAND_FIELDS, out):
        np.testing.assert_array_equal(t.cpu().numpy(), want[f], err_msg=f"{case}: {f}")
