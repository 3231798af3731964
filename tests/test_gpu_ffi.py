"""The operand-form entries (the bodies of the reference's FFI handlers), on
the GPU.

nanorts_amd_step_ffi takes the 33 operands and 31 results of the reference's
nanorts_step target (src/nanorts/core/cuda/step.cu:56-108, built by
src/nanorts/core/cycle.py:123-134, 198-211) as device pointers: the key, the
six Commands fields, terrain, the unit `table` and `timings` operands in the
reference's column layout (src/nanorts/core/unit_tables.py:9-48), and the 23
state leaves.  Each case is compared bit for bit with the oracle's core.step
(the state, the admitted counts and the per-slot completion records):
results aliased to the state operands and results in separate buffers, keys
and Commands per lane and broadcast from one row (extent 1).
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from nanorts_amd.model import LEAF_NAMES
from tests.helpers import advanced_states, assert_states_equal, game_for

pytestmark = pytest.mark.gpu

COMMAND_FIELDS = ("kind", "direction", "none_duration", "target_cell", "produced_type", "request_order")
TABLE_COLUMNS = ("can_move", "can_harvest", "is_resource", "is_stockpile", "can_attack", "attack_range", "cost")
TIMING_COLUMNS = ("move_time", "harvest_time", "attack_time", "produce_time", "hit_points", "attack_damage",
                  "harvest_amount")


def reference_tables(game) -> tuple[np.ndarray, np.ndarray]:
    """unit_table / unit_timings of the reference for this game's unit table."""
    cols = game.columns
    table = np.concatenate([np.stack([cols[c].astype(np.int32) for c in TABLE_COLUMNS], -1),
                            cols["produces"].astype(np.int32)], -1)
    timings = np.stack([cols[c].astype(np.int32) for c in TIMING_COLUMNS], -1)
    return table[None], timings[None]


def _call(game, st: dict, commands: dict, keys: np.ndarray, *, alias: bool):
    import torch

    from nanorts_amd import native
    from nanorts_amd.model import STRATEGY_CODES

    d = "cuda:0"
    b = game.bucket
    L = st["time"].shape[0]
    table, timings = reference_tables(game)
    keep = []

    def dev(array):
        t = torch.as_tensor(np.ascontiguousarray(array), device=d)
        keep.append(t)
        return t

    leaves = [dev(st[name]) for name in LEAF_NAMES]
    operands = [dev(keys)] + [dev(commands[f]) for f in COMMAND_FIELDS] + \
        [dev(game.terrain.astype(np.bool_)[None]), dev(table), dev(timings)] + leaves
    E, T = b.entity_capacity, b.unit_type_capacity
    events = [torch.full((L, 2), -7, dtype=torch.int32, device=d), torch.full((L, 2), -7, dtype=torch.int32, device=d),
              torch.full((L, 2, T), -7, dtype=torch.int32, device=d),
              torch.full((L, 2, 3), -7, dtype=torch.int32, device=d),
              torch.ones((L, E), dtype=torch.bool, device=d), torch.full((L, E, 6), -7, dtype=torch.int32, device=d),
              torch.full((L, E, 4), -7, dtype=torch.int16, device=d),
              torch.full((L, E, 6), -7, dtype=torch.int8, device=d)]
    written = leaves if alias else [torch.full_like(t, 99) for t in leaves]
    results = written + events
    keep.extend(results)
    ops = (ctypes.c_void_p * 33)(*[t.data_ptr() for t in operands])
    rets = (ctypes.c_void_p * 31)(*[t.data_ptr() for t in results])
    lib = native.load()
    code = lib.nanorts_amd_step_ffi(torch.cuda.current_stream().cuda_stream, ops, rets, L, keys.shape[0],
                                    commands["kind"].shape[0], b.height, b.width, b.neutral_capacity,
                                    b.per_player_capacity, T, STRATEGY_CODES[b.conflict_strategy])
    assert code == 0, lib.nanorts_amd_last_error().decode()
    torch.cuda.synchronize()
    state = {name: t.cpu().numpy() for name, t in zip(LEAF_NAMES, written)}
    inputs = {name: t.cpu().numpy() for name, t in zip(LEAF_NAMES, leaves)}
    return state, inputs, [t.cpu().numpy() for t in events]


@pytest.mark.parametrize("case", ["8x8-original-both", "16x16-random-partial", "barracks-random",
                                  "obstacle-alternating", "24x24-barricades-alternating", "32x32-random-partial"])
@pytest.mark.parametrize("alias,broadcast", [(True, False), (False, False), (True, True), (False, True)])
def test_step_ffi_matches_oracle(case, alias, broadcast, oracle_threads):
    from oracle.oracle import copy_state

    print(f"step_ffi {case} alias={alias} broadcast={broadcast}", flush=True)
    game, partial = game_for(case)
    L = 64
    oracle, st = advanced_states(game, L, 90, partial, oracle_threads, seed=31)
    rng = np.random.default_rng(9)
    if broadcast:
        # one Commands row and one key for every lane: lane 0's sampled rows
        one = oracle.decode_actions({k: np.ascontiguousarray(v[:1]) for k, v in st.items()},
                                    oracle.sample_actions(oracle.avail_rows({k: v[:1] for k, v in st.items()}), (3, 1), 5))
        commands = one
        keys = rng.integers(0, 2**32, size=(1, 2), dtype=np.uint64).astype(np.uint32)
        want_cmds = {f: np.ascontiguousarray(np.broadcast_to(v, (L, *v.shape[1:]))) for f, v in one.items()}
        want_keys = np.ascontiguousarray(np.broadcast_to(keys, (L, 2)))
    else:
        commands = oracle.decode_actions(st, oracle.sample_actions(oracle.avail_rows(st), (3, 1), 5))
        keys = rng.integers(0, 2**32, size=(L, 2), dtype=np.uint64).astype(np.uint32)
        want_cmds, want_keys = commands, keys
    before = copy_state(st)
    got, inputs, events = _call(game, st, commands, keys, alias=alias)
    want = oracle.core_step(st, want_cmds, want_keys)
    assert_states_equal({k: v for k, v in st.items() if k in got}, got, f"{case} step_ffi")
    if not alias:  # the operands are left as they were
        assert_states_equal({k: v for k, v in before.items() if k in inputs}, inputs, f"{case} operands")
    for name, value in zip(("admitted_harvest", "admitted_return", "admitted_produce", "admitted_attack"), events):
        np.testing.assert_array_equal(value, want[name], err_msg=name)
    # the per-slot completion records (results 27-30)
    for value, name in zip(events[4:], ("is_member", "records_i32", "records_i16", "records_i8")):
        np.testing.assert_array_equal(value.astype(want[name].dtype), want[name], err_msg=name)
    assert want["is_member"].any()


def _dev(array):
    import torch

    return torch.as_tensor(np.ascontiguousarray(array), device="cuda:0")


def _words_of(rows: np.ndarray) -> np.ndarray:
    """bool rows [..., width <= 96] as three little-endian uint32 words."""
    bits = np.zeros((*rows.shape[:-1], 96), np.uint64)
    bits[..., :rows.shape[-1]] = rows
    weights = (np.uint64(1) << np.arange(32, dtype=np.uint64))
    return np.stack([(bits[..., 32 * j:32 * j + 32] * weights).sum(-1) for j in range(3)], -1).astype(np.uint32)


@pytest.mark.parametrize("case", ["8x8-original-both", "16x16-random-partial", "barracks-random", "9x8-alternating",
                                  "gow-alternating", "24x24-barricades-alternating", "32x32-random-partial"])
def test_legality_ffi_matches_oracle(case, oracle_threads):
    import torch

    from nanorts_amd import native

    print(f"legality_ffi {case}", flush=True)
    game, partial = game_for(case)
    b = game.bucket
    L = 16 if case.startswith("gow") else 64
    oracle, st = advanced_states(game, L, 40 if case.startswith("gow") else 120, partial, oracle_threads, seed=13)
    table, _ = reference_tables(game)
    names = ("birth", "unit_type", "owner", "carried_resources", "cell", "entity_at", "player_resources")
    operands = [_dev(st[n]) for n in names] + [_dev(game.terrain.astype(np.bool_)[None]), _dev(table)]
    ops = (ctypes.c_void_p * 9)(*[t.data_ptr() for t in operands])
    want = oracle.legality_rows(st)
    width = want.shape[-1]
    lib = native.load()
    T, O = b.unit_type_capacity, b.attack_offset_capacity
    rows = torch.ones((L, 2, b.per_player_capacity, width), dtype=torch.bool, device="cuda:0")
    words = torch.full((L, 2, b.per_player_capacity, 3), 0x5A5A5A5A, dtype=torch.int32, device="cuda:0")
    stream = torch.cuda.current_stream().cuda_stream
    for out, form in ((rows, 0), (words, 1)):
        code = lib.nanorts_amd_legality_ffi(stream, ops, out.data_ptr(), form, L, b.height, b.width,
                                            b.entity_capacity, b.per_player_capacity, T, O)
        assert code == 0, lib.nanorts_amd_last_error().decode()
    torch.cuda.synchronize()
    np.testing.assert_array_equal(rows.cpu().numpy(), want)
    np.testing.assert_array_equal(words.cpu().numpy().view(np.uint32), _words_of(want))


def _visible_closed_form(birth, unit_type, cell, radius, first, count, height, width):
    """visible[l, y, x]: some slot of the block with a birth, an in-range
    cell and type, has (x - cx)^2 + (y - cy)^2 <= radius[type]^2."""
    L = birth.shape[0]
    yy, xx = np.mgrid[0:height, 0:width]
    out = np.zeros((L, height, width), bool)
    for l in range(L):
        for slot in range(first, first + count):
            c, t = int(cell[l, slot]), int(unit_type[l, slot])
            if birth[l, slot] == -1 or not (0 <= c < height * width) or not (0 <= t < radius.shape[0]):
                continue
            r = int(radius[t])
            out[l] |= (xx - c % width) ** 2 + (yy - c // width) ** 2 <= r * r
    return out


def _visible_call(lib, birth, unit_type, cell, radius, lanes, first, count, height, width):
    import torch

    t_birth, t_type, t_cell, t_radius = _dev(birth), _dev(unit_type), _dev(cell), _dev(radius)
    out = torch.ones((lanes, height, width), dtype=torch.bool, device="cuda:0")
    code = lib.nanorts_amd_visible_cells_ffi(torch.cuda.current_stream().cuda_stream, t_birth.data_ptr(),
                                             birth.shape[0], t_type.data_ptr(), unit_type.shape[0], t_cell.data_ptr(),
                                             cell.dtype.itemsize, cell.shape[0], birth.shape[1], t_radius.data_ptr(),
                                             radius.shape[0], out.data_ptr(), lanes, first, count, width, height)
    assert code == 0, lib.nanorts_amd_last_error().decode()
    torch.cuda.synchronize()
    return out.cpu().numpy()


@pytest.mark.parametrize("case", ["8x8-original-both", "16x16-random-partial", "9x8-alternating", "gow-alternating",
                                  "24x24-barricades-alternating", "32x32-random-partial"])
def test_visible_cells_ffi(case, oracle_threads):
    from nanorts_amd import native

    print(f"visible_cells_ffi {case}", flush=True)
    game, partial = game_for(case)
    b = game.bucket
    L = 16 if case.startswith("gow") else 48
    oracle, st = advanced_states(game, L, 40 if case.startswith("gow") else 120, partial, oracle_threads, seed=17)
    lib = native.load()
    radius = game.columns["sight_radius"].astype(np.int32)
    H, W, N, C, E = b.height, b.width, b.neutral_capacity, b.per_player_capacity, b.entity_capacity
    for p in (0, 1):  # each player's block, as the reference's visibility calls it
        got = _visible_call(lib, st["birth"], st["unit_type"], st["cell"], radius, L, N + p * C, C, H, W)
        np.testing.assert_array_equal(got, oracle.visible_cells(st, p))
    # the whole slot range, int32 cells, a larger radius table
    wide = np.concatenate([radius, [6, 0, -1]]).astype(np.int32)
    cell32 = st["cell"].astype(np.int32)
    got = _visible_call(lib, st["birth"], st["unit_type"], cell32, wide, L, 0, E, H, W)
    np.testing.assert_array_equal(got, _visible_closed_form(st["birth"], st["unit_type"], cell32, wide, 0, E, H, W))
    # a shared birth row (extent 1) and an odd block
    shared = np.ascontiguousarray(st["birth"][:1])
    got = _visible_call(lib, shared, st["unit_type"], st["cell"], radius, L, 3, E - 5, H, W)
    want = _visible_closed_form(np.broadcast_to(shared, st["birth"].shape), st["unit_type"], st["cell"], radius, 3,
                                E - 5, H, W)
    np.testing.assert_array_equal(got, want)
    if H * W <= 127:  # int8 cells
        cell8 = st["cell"].astype(np.int8)
        got = _visible_call(lib, st["birth"], st["unit_type"], cell8, radius, L, N, 2 * C, H, W)
        np.testing.assert_array_equal(got, _visible_closed_form(st["birth"], st["unit_type"], cell8, radius, N, 2 * C,
                                                                H, W))


ROW_LEAVES = ("birth", "unit_type", "owner", "cell", "hit_points", "carried_resources", "pending_kind",
              "pending_direction", "pending_none_duration", "pending_target_cell", "pending_produced_type",
              "pending_issued_at", "pending_completes_at", "pending_order", "entity_at")


@pytest.mark.parametrize("case", ["8x8-original-both", "16x16-random-partial", "gow-alternating"])
@pytest.mark.parametrize("form", ["aliased", "separate", "packed", "per-lane"])
def test_reset_rows_ffi(case, form, oracle_threads):
    import torch

    from nanorts_amd import native
    from oracle.oracle import copy_state

    print(f"reset_rows_ffi {case} {form}", flush=True)
    game, partial = game_for(case)
    L = 16 if case.startswith("gow") else 64
    oracle, st = advanced_states(game, L, 40 if case.startswith("gow") else 120, partial, oracle_threads, seed=19)
    done = (np.arange(L) % 3 == 1).astype(np.bool_)
    init = game.initial_state
    ending = [_dev(st[n]) for n in ROW_LEAVES]
    row_bytes = [int(st[n][0].nbytes) for n in ROW_LEAVES]
    keep = []
    if form == "packed":  # one shared uint8 row, each leaf at the next 16-byte offset
        chunks, offsets, at = [], [], 0
        for n in ROW_LEAVES:
            raw = np.ascontiguousarray(init[n]).view(np.uint8).ravel()
            pad = (-raw.size) % 16
            offsets.append(at)
            chunks.append(np.concatenate([raw, np.zeros(pad, np.uint8)]))
            at += raw.size + pad
        packed = _dev(np.concatenate(chunks))
        keep.append(packed)
        reset_ptrs = [packed.data_ptr() + o for o in offsets]
        reset_lanes = [1] * len(ROW_LEAVES)
    elif form == "per-lane":  # a reset row per lane: another mid-game batch
        _, other = advanced_states(game, L, 30, partial, oracle_threads, seed=23)
        resets = [_dev(other[n]) for n in ROW_LEAVES]
        keep.extend(resets)
        reset_ptrs = [t.data_ptr() for t in resets]
        reset_lanes = [L] * len(ROW_LEAVES)
    else:
        resets = [_dev(np.ascontiguousarray(init[n])[None]) for n in ROW_LEAVES]
        keep.extend(resets)
        reset_ptrs = [t.data_ptr() for t in resets]
        reset_lanes = [1] * len(ROW_LEAVES)
    results = ending if form != "separate" else [torch.full_like(t, 77) for t in ending]
    t_done = _dev(done)
    k = len(ROW_LEAVES)
    lib = native.load()
    code = lib.nanorts_amd_reset_rows_ffi(torch.cuda.current_stream().cuda_stream, t_done.data_ptr(), L, k,
                                          (ctypes.c_void_p * k)(*reset_ptrs), (ctypes.c_int64 * k)(*reset_lanes),
                                          (ctypes.c_void_p * k)(*[t.data_ptr() for t in ending]),
                                          (ctypes.c_void_p * k)(*[t.data_ptr() for t in results]),
                                          (ctypes.c_int64 * k)(*row_bytes))
    assert code == 0, lib.nanorts_amd_last_error().decode()
    torch.cuda.synchronize()
    if form == "per-lane":
        for n, t in zip(ROW_LEAVES, results):
            want = np.where(done.reshape((L,) + (1,) * (st[n].ndim - 1)), other[n], st[n])
            np.testing.assert_array_equal(t.cpu().numpy(), want, err_msg=n)
        return
    expected = copy_state(st)
    oracle.reset_where_done(expected, done.astype(np.uint8))
    for n, t in zip(ROW_LEAVES, results):
        np.testing.assert_array_equal(t.cpu().numpy(), expected[n], err_msg=n)
