"""Host logic of the multi-group step (CPU only, no kernel runs): which games
step together, and the library's refusals before any launch."""
from __future__ import annotations

import ctypes

import numpy as np
import torch

from nanorts_amd import groups, native
from nanorts_amd.content import map_name_to_scenario
from nanorts_amd.env import DeviceGame
from nanorts_amd.model import UnitTypeTableVersion


def _games():
    a = map_name_to_scenario("basesWorkers8x8", conflict_strategy="CANCEL_RANDOM")
    b = map_name_to_scenario("basesWorkers8x8Obstacle", conflict_strategy="CANCEL_RANDOM", max_cycles=150)
    c = map_name_to_scenario("basesWorkers8x8", conflict_strategy="CANCEL_RANDOM", utt=UnitTypeTableVersion.ORIGINAL)
    d = map_name_to_scenario("basesWorkers8x8", conflict_strategy="CANCEL_BOTH")
    return a, b, c, d


def test_games_step_together_on_one_bucket():
    a, b, c, d = _games()
    assert groups.steps_together([a, b])            # other terrain and horizon, same bucket
    assert not groups.steps_together([a])           # one game is an ordinary step
    assert not groups.steps_together([a, c])        # another unit table
    assert not groups.steps_together([a, d])        # another strategy
    assert not groups.steps_together([a] * 17)      # more groups than one call takes


def _call(lib, devs, template, L=2):
    G = len(devs)
    st = template.batch(L)
    state = native.State(*[st.leaves[n].data_ptr() for n in native.STATE_FIELDS[:-2]], None, None)
    C = template.game.bucket.per_player_capacity
    buf = torch.zeros((L, 2, C), dtype=torch.int32)
    key = torch.zeros((1, 2), dtype=torch.int32)
    games = (ctypes.POINTER(native.Game) * max(G, 1))(*[ctypes.pointer(d.struct) for d in devs])
    states = (native.State * max(G, 1))(*([state] * G))
    lanes = (ctypes.c_int64 * max(G, 1))(*([L] * G))
    keys = (ctypes.c_void_p * max(G, 1))(*([key.data_ptr()] * G))
    key_lanes = (ctypes.c_int64 * max(G, 1))(*([1] * G))
    cmds = (native.Commands * max(G, 1))(*([native.Commands(*([buf.data_ptr()] * 6))] * G))
    outs = (native.StepResults * max(G, 1))(*([native.StepResults()] * G))
    return lib.nanorts_amd_step_groups(None, G, games, states, lanes, keys, key_lanes, cmds, outs)


def test_the_library_refuses_groups_that_disagree():
    lib = native.load()
    a, b, c, d = _games()
    cpu = torch.device("cpu")
    da, dc, dd = DeviceGame(a, cpu), DeviceGame(c, cpu), DeviceGame(d, cpu)
    for devs, words in (([da, dc], "unit table"), ([da, dd], "bucket"), ([], "groups"), ([da] * 17, "groups")):
        assert _call(lib, devs, da) != 0
        assert words in lib.nanorts_amd_last_error().decode()
    np.testing.assert_equal(groups.MAX_GROUPS, 16)
