"""GPU parity of the facade's split and transition steps.

step_env is the transition without the auto-reset: compared cycle by cycle
with the oracle's decode -> core.step keyed by the episode root, the ending
state observed.  step_request -> step_groups -> step_response is compared
with the fused env.step on the same actions, cycle by cycle across episode
ends, including the reward components and the ending state's telemetry.
A small slot capacity makes production overflow the player's slot block,
so the telemetry counts are not all zero.
"""
from __future__ import annotations

import ctypes
import dataclasses
import sys

import numpy as np
import pytest

from oracle.oracle import Oracle, batch_initial, copy_state, load_library
from tests.helpers import assert_states_equal, roots, to_device, to_host

pytestmark = pytest.mark.gpu

FIELDS = ("kind", "direction", "none_duration", "target_cell", "produced_type", "request_order")


def _say(*parts):
    print(*parts, flush=True)
    sys.stdout.flush()


def _crowded_game():
    """basesWorkers8x8 with 3 slots per player (the population is 2), so
    produced units soon find the block full."""
    from nanorts_amd.content import load_game, shipped_map

    path = shipped_map("basesWorkers8x8")
    derived = load_game(path, conflict_strategy="CANCEL_RANDOM", max_cycles=200).bucket
    return load_game(path, conflict_strategy="CANCEL_RANDOM", max_cycles=200,
                     bucket=dataclasses.replace(derived, per_player_capacity=3))


def _episode_roots(st) -> np.ndarray:
    lib = load_library()
    out = np.zeros((st["time"].shape[0], 2), np.uint32)
    for l, (root, ep) in enumerate(zip(st["environment_root"].reshape(-1, 2), st["episode_index"])):
        o = (ctypes.c_uint32 * 2)()
        lib.nro_fold_in((ctypes.c_uint32 * 2)(int(root[0]), int(root[1])), ctypes.c_uint32(int(ep)), o)
        out[l] = (o[0], o[1])
    return out


def _acts(env, actions):
    import torch

    return {a: torch.as_tensor(np.ascontiguousarray(actions[:, i]), device="cuda:0") for i, a in enumerate(env.agents)}


@pytest.mark.parametrize("partial", [False, True])
def test_step_env_is_the_transition(partial, oracle_threads):
    import torch

    import nanorts_amd

    _say(f"step_env partial={partial}")
    torch.cuda.set_device(0)
    game = _crowded_game()
    L = 64
    oracle = Oracle(game)
    st = batch_initial(game, L, roots(L, 11))
    oracle.rollout(st, (1, 2), 0, 150, partial, threads=oracle_threads, record=False)
    env = nanorts_amd.make("NanoRTS", scenario=game, partial_observability=partial, device="cuda:0")
    state = to_device(env, st)
    overflow = 0
    for t in range(60):
        actions = oracle.sample_actions(oracle.avail_rows(st), (3, 4), t)
        obs, state, rewards, dones, infos = env.step_env(None, state, _acts(env, actions), donate=True)
        cmds = oracle.decode_actions(st, actions)
        want = oracle.core_step(st, cmds, _episode_roots(st))
        done = (want["terminated"] | want["truncated"]).astype(bool)
        for p, agent in enumerate(env.agents):
            np.testing.assert_array_equal(rewards[agent].cpu().numpy(), want["reward"][:, p], err_msg=f"cycle {t}")
            np.testing.assert_array_equal(dones[agent].cpu().numpy(), done)
        np.testing.assert_array_equal(infos["winner"].cpu().numpy(), st["winner"])
        np.testing.assert_array_equal(infos["telemetry"]["spawn_overflow"].cpu().numpy(), st["spawn_overflow"])
        maps, scalars = oracle.symbolic(st, partial)
        for p, agent in enumerate(env.agents):
            np.testing.assert_array_equal(obs[agent].feature_maps.cpu().numpy(), maps[:, p], err_msg=f"cycle {t}")
            np.testing.assert_array_equal(obs[agent].scalars.cpu().numpy(), scalars[:, p])
        assert infos["final_observation"][env.agents[0]] is obs[env.agents[0]]
        assert_states_equal(st, to_host(state), f"cycle {t}")
        overflow = max(overflow, int(st["spawn_overflow"].max()))
    assert overflow > 0


@pytest.mark.parametrize("case", ["crowded", "16x16-finetuned-both"])
def test_request_groups_response_equals_the_fused_step(case, oracle_threads):
    import torch

    import nanorts_amd
    from nanorts_amd import groups
    from tests.helpers import advanced_states, game_for

    _say(f"step_request/step_response {case}")
    torch.cuda.set_device(0)
    if case == "crowded":
        game, partial = _crowded_game(), False
        oracle = Oracle(game)
        st = batch_initial(game, 48, roots(48, 13))
        oracle.rollout(st, (1, 2), 0, 150, partial, threads=oracle_threads, record=False)
    else:
        game, partial = game_for(case)
        oracle, st = advanced_states(game, 48, 200, partial, oracle_threads, seed=13)
    env = nanorts_amd.make("NanoRTS", scenario=game, partial_observability=partial, reward_components=True,
                           device="cuda:0")
    fused = to_device(env, st)
    split = to_device(env, copy_state(st))
    ended = 0
    for t in range(60):
        actions = oracle.sample_actions(oracle.avail_rows(st), (5, 6), t)
        a = env.step(None, fused, _acts(env, actions), donate=True)
        (keys, core, cmds), carry = env.step_request(split, _acts(env, actions))
        if t == 0:
            want = oracle.decode_actions(st, actions)
            for f in FIELDS:
                np.testing.assert_array_equal(cmds[f].cpu().numpy(), want[f], err_msg=f)
            np.testing.assert_array_equal(keys.cpu().numpy().view(np.uint32), _episode_roots(st))
        stepped = groups.step_groups([(keys, core, cmds, env)])[0]
        b = env.step_response(split, carry, stepped)
        oracle.env_step(st, actions, partial, observe=False)
        for agent in env.agents:
            assert torch.equal(a[0][agent].feature_maps, b[0][agent].feature_maps), f"cycle {t} obs"
            assert torch.equal(a[0][agent].scalars, b[0][agent].scalars)
            assert torch.equal(a[2][agent], b[2][agent]), f"cycle {t} rewards"
            assert torch.equal(a[3][agent], b[3][agent])
            assert torch.equal(a[4]["final_observation"][agent].feature_maps,
                               b[4]["final_observation"][agent].feature_maps)
            assert torch.equal(a[4]["reward_components"][agent], b[4]["reward_components"][agent]), f"cycle {t}"
        for name in ("terminated", "truncated", "winner", "spawn_overflowed", "final_valid"):
            assert torch.equal(a[4][name], b[4][name]), f"cycle {t} {name}"
        assert torch.equal(a[4]["telemetry"]["spawn_overflow"], b[4]["telemetry"]["spawn_overflow"])
        assert_states_equal(to_host(fused), to_host(split), f"cycle {t}")
        assert_states_equal(st, to_host(fused), f"cycle {t} oracle")
        ended += int(a[3]["__all__"].sum())
    assert env.agent_classes == {"player": list(env.agents)}
    if case == "crowded":
        assert ended > 0


@pytest.mark.parametrize("bot_name", ["workerRushAI", "lightRushAI"])
def test_seat_request_response_equals_the_fused_seat_step(bot_name, oracle_threads):
    import torch

    from nanorts_amd import bots, groups
    from nanorts_amd.content import map_name_to_scenario

    _say(f"seat step_request/step_response {bot_name}")
    torch.cuda.set_device(0)
    # a horizon inside the 120 cycles, so every game ends (and resets) once
    game = map_name_to_scenario("basesWorkers8x8", max_cycles=100)
    bot = getattr(bots, bot_name)
    seat = bots.SeatEnv(bot, scenario=game, reward_components=True, device="cuda:0")
    keys = roots(32, 17)
    _, fused = seat.reset(keys)
    _, split = seat.reset(keys)
    oracle = Oracle(game)
    C = game.bucket.per_player_capacity
    ended = 0
    for t in range(120):
        # the learner samples from its current masks
        rows = np.zeros((32, 2, C, 78), bool)
        rows[:, 0] = seat.get_avail_actions(fused)[bots.LEARNER].cpu().numpy()
        learner = oracle.sample_actions(rows, (7, 8), t)[:, 0].copy()
        acts = {bots.LEARNER: torch.as_tensor(learner, device="cuda:0")}
        a = seat.step(None, fused, acts, donate=True)
        (k, core, cmds), carry = seat.step_request(split, acts)
        stepped = groups.step_groups([(k, core, cmds, seat)])[0]
        b = seat.step_response(split, carry, stepped)
        learner_agent = bots.LEARNER
        assert torch.equal(a[0][learner_agent].feature_maps, b[0][learner_agent].feature_maps), f"cycle {t}"
        assert torch.equal(a[2][learner_agent], b[2][learner_agent]), f"cycle {t} reward"
        assert torch.equal(a[3][learner_agent], b[3][learner_agent])
        assert torch.equal(a[4]["reward_components"][learner_agent], b[4]["reward_components"][learner_agent])
        assert torch.equal(a[4]["final_observation"][learner_agent].feature_maps,
                           b[4]["final_observation"][learner_agent].feature_maps)
        for name in ("terminated", "truncated", "winner", "spawn_overflowed"):
            assert torch.equal(a[4][name], b[4][name]), f"cycle {t} {name}"
        assert_states_equal(to_host(fused.environment_state), to_host(split.environment_state), f"cycle {t}")
        for name in fused.carry:
            assert torch.equal(fused.carry[name], split.carry[name]), f"cycle {t} carry {name}"
        ended += int(a[3]["__all__"].sum())
    assert ended > 0
    assert seat.agent_classes == {bots.LEARNER: [bots.LEARNER]}
    assert seat.action_space(bots.LEARNER) == seat.env.action_space("player_0")


def test_seat_on_the_pixel_surface(oracle_threads):
    import torch

    from nanorts_amd import bots, rendering
    from nanorts_amd.content import map_name_to_scenario
    from oracle.oracle import empty_carry

    _say("seat pixels")
    torch.cuda.set_device(0)
    game = map_name_to_scenario("basesWorkers8x8", max_cycles=400)
    seat = bots.SeatEnv(bots.lightRushAI, scenario=game, surface="pixels", seat="player_1", device="cuda:0")
    keys = roots(8, 19)
    obs, state = seat.reset(keys)
    oracle = Oracle(game)
    ref = batch_initial(game, 8, keys)
    carry = empty_carry(8, game.bucket.per_player_capacity)
    tiles = rendering.tile_table(game.bucket.unit_type_capacity)
    for t in range(10):
        learner = oracle.sample_actions(oracle.avail_rows(ref), (9, 10), t)[:, 1].copy()
        obs, state, rewards, dones, infos = seat.step(None, state, {bots.LEARNER: torch.as_tensor(learner,
                                                                                                 device="cuda:0")},
                                                      donate=True)
        want = oracle.seat_step(ref, carry, bots.lightRushAI.strategy, bots.lightRushAI.trained, 1, learner, False,
                                observe=False)
        image, scalars = oracle.pixels(ref, False, tiles)
        np.testing.assert_array_equal(obs[bots.LEARNER].image.cpu().numpy(), image[:, 1], err_msg=f"cycle {t}")
        np.testing.assert_array_equal(obs[bots.LEARNER].scalars.cpu().numpy(), scalars[:, 1])
        np.testing.assert_array_equal(rewards[bots.LEARNER].cpu().numpy(), want["reward"][:, 1])
