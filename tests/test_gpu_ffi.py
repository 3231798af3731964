"""The step entry in the reference's FFI operand and result order, on the GPU.

nanorts_amd_step_ffi takes the 33 operands and 31 results of the reference's
nanorts_step target (src/nanorts/core/cuda/step.cu:56-108, built by
src/nanorts/core/cycle.py:123-134, 198-211) as device pointers: the key, the
six Commands fields, terrain, the unit `table` and `timings` operands in the
reference's column layout (src/nanorts/core/unit_tables.py:9-48), and the 23
state leaves.  Each case is compared bit for bit with the oracle's core.step:
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
                                    b.per_player_capacity, T, b.attack_offset_capacity,
                                    STRATEGY_CODES[b.conflict_strategy])
    assert code == 0, lib.nanorts_amd_last_error().decode()
    torch.cuda.synchronize()
    state = {name: t.cpu().numpy() for name, t in zip(LEAF_NAMES, written)}
    inputs = {name: t.cpu().numpy() for name, t in zip(LEAF_NAMES, leaves)}
    return state, inputs, [t.cpu().numpy() for t in events]


@pytest.mark.parametrize("case", ["8x8-original-both", "16x16-random-partial", "barracks-random",
                                  "obstacle-alternating"])
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
    for value in events[4:]:  # the per-slot records: no member
        assert not value.any()
