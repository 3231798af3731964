"""The five benchmark configurations at their full sizes.

Each configuration runs on the GPU at its published game count and length.
The smallest (basesWorkers8x8, 1024 games, 1000 steps) is compared with the
oracle game for game.  For the larger ones every game's final state is
checked against the state invariants (src/nanorts/model/state.py:87-165),
and a seeded sample of games is replayed alone by the oracle and compared
bit for bit: rewards and dones of every step, the final state and the last
observation.  A game replays alone because every key derives from its global
index (its root is split(root, L)[i], and the harness sampler numbers it
env0 + i).
"""
from __future__ import annotations

import sys

import numpy as np
import pytest

from oracle.oracle import Oracle, batch_initial, empty_carry
from tests.helpers import assert_states_equal, to_host

pytestmark = pytest.mark.gpu

KEY = (101, 202)


def _say(*parts):
    print(*parts, flush=True)
    sys.stdout.flush()


def _env(game, partial, **kw):
    import torch

    import nanorts_amd

    torch.cuda.set_device(0)
    return nanorts_amd.make("NanoRTS", scenario=game, partial_observability=partial, final_observation=False,
                            device="cuda:0", **kw)


def _one(state: dict[str, np.ndarray], i: int) -> dict[str, np.ndarray]:
    return {k: np.ascontiguousarray(v[i:i + 1]) for k, v in state.items()}


def _no_violations(game, state):
    bad = np.nonzero(Oracle(game).violations(state))[0]
    assert bad.size == 0, f"state invariants broken in games {bad[:10].tolist()}"


def _rollout_case(game, partial, L, steps, sample, oracle_threads):
    """GPU fused rollout of L games; the oracle replays `sample` games alone."""
    import torch

    from nanorts_amd import env as envmod

    env = _env(game, partial)
    roots = envmod.env_roots(0, L)
    _, state = env.reset(roots)
    out = env.rollout(state, steps, KEY, observation_depth=2)
    torch.cuda.synchronize()
    got = to_host(state)
    _no_violations(game, got)
    idx = torch.as_tensor(sample, device="cuda:0")
    rewards = out["rewards"].index_select(1, idx).cpu().numpy()
    dones = out["dones"].index_select(1, idx).cpu().numpy()
    slot = (steps - 1) % 2
    maps = out["feature_maps"][slot].index_select(0, idx).cpu().numpy()
    oracle = Oracle(game)
    for k, i in enumerate(sample):
        ref = batch_initial(game, 1, roots[i:i + 1])
        want = oracle.rollout(ref, KEY, 0, steps, partial, threads=1, env0=int(i))
        np.testing.assert_array_equal(rewards[:, k], want["rewards"][:, 0], err_msg=f"game {i} rewards")
        np.testing.assert_array_equal(dones[:, k].astype(np.uint8), want["dones"][:, 0], err_msg=f"game {i} dones")
        np.testing.assert_array_equal(maps[k], want["feature_maps"][0], err_msg=f"game {i} last observation")
        assert_states_equal(ref, _one(got, i), f"game {i}")
    return out


def _sample(L, n, seed):
    rng = np.random.default_rng(seed)
    return np.unique(np.concatenate([[0, L - 1], rng.choice(L, n, replace=False)]))


def test_config0_8x8_every_game_matches(oracle_threads):
    """basesWorkers8x8, VERSION_ORIGINAL, CANCEL_BOTH, 47 slots per player,
    1024 games, 1000 steps: every game against the oracle."""
    import torch

    from nanorts_amd import env as envmod
    from nanorts_amd.content import map_name_to_scenario
    from nanorts_amd.model import UnitTypeTableVersion

    _say("config 0: basesWorkers8x8 x 1024 x 1000")
    game = map_name_to_scenario("basesWorkers8x8", utt=UnitTypeTableVersion.ORIGINAL, conflict_strategy="CANCEL_BOTH")
    assert game.bucket.per_player_capacity == 47
    L, steps = 1024, 1000
    env = _env(game, False)
    roots = envmod.env_roots(0, L)
    _, state = env.reset(roots)
    out = env.rollout(state, steps, KEY, observation_depth=1)
    torch.cuda.synchronize()
    ref = batch_initial(game, L, roots)
    want = Oracle(game).rollout(ref, KEY, 0, steps, False, threads=oracle_threads)
    np.testing.assert_array_equal(out["rewards"].cpu().numpy(), want["rewards"])
    np.testing.assert_array_equal(out["dones"].cpu().numpy().astype(np.uint8), want["dones"])
    np.testing.assert_array_equal(out["feature_maps"][0].cpu().numpy(), want["feature_maps"])
    assert_states_equal(ref, to_host(state), "config 0")
    assert want["dones"].sum() > 0


def test_config1_16x16_cancel_both_16384_games(oracle_threads):
    """basesWorkers16x16, VERSION_ORIGINAL_FINETUNED, CANCEL_BOTH, 70 slots,
    16384 games, 2000 steps, max_cycles 5000."""
    from nanorts_amd.content import map_name_to_scenario

    _say("config 1: basesWorkers16x16 CANCEL_BOTH x 16384 x 2000")
    game = map_name_to_scenario("basesWorkers16x16", conflict_strategy="CANCEL_BOTH", max_cycles=5000)
    assert game.bucket.per_player_capacity == 70
    _rollout_case(game, False, 16384, 2000, _sample(16384, 14, 1), oracle_threads)


def test_config2_16x16_random_partial_65536_games(oracle_threads):
    """basesWorkers16x16, CANCEL_RANDOM, partial observability, 65536 games,
    1000 steps."""
    from nanorts_amd.content import map_name_to_scenario

    _say("config 2: basesWorkers16x16 CANCEL_RANDOM partial x 65536 x 1000")
    game = map_name_to_scenario("basesWorkers16x16", conflict_strategy="CANCEL_RANDOM")
    _rollout_case(game, True, 65536, 1000, _sample(65536, 22, 2), oracle_threads)


@pytest.mark.parametrize("bot_name", ["workerRushAI", "lightRushAI"])
def test_config3_seat_32768_games_full_episodes(bot_name):
    """basesWorkers16x16, player_1 the scripted bot on the device, player_0
    the seeded sampler, 32768 games, 3000 cycles (max_cycles 3000)."""
    import torch

    from nanorts_amd import bots
    from nanorts_amd import env as envmod
    from nanorts_amd.content import map_name_to_scenario

    _say(f"config 3: seat {bot_name} x 32768 x 3000")
    torch.cuda.set_device(0)
    game = map_name_to_scenario("basesWorkers16x16", max_cycles=3000)
    bot = getattr(bots, bot_name)
    seat = bots.SeatEnv(bot, scenario=game, final_observation=False, device="cuda:0")
    L, steps = 32768, 3000
    roots = envmod.env_roots(0, L)
    _, state = seat.reset(roots)
    out = seat.rollout(state, steps, KEY)
    torch.cuda.synchronize()
    got = to_host(state.environment_state)
    _no_violations(game, got)
    dones = out["dones"]
    assert int(dones.sum()) >= L  # every game ends at least once by the horizon
    sample = _sample(L, 5, 3)
    idx = torch.as_tensor(sample, device="cuda:0")
    rewards = out["rewards"].index_select(1, idx).cpu().numpy()
    carry = {k: v.index_select(0, idx).cpu().numpy() for k, v in state.carry.items()}
    oracle = Oracle(game)
    C = game.bucket.per_player_capacity
    for k, i in enumerate(sample):
        ref = batch_initial(game, 1, roots[i:i + 1])
        c = empty_carry(1, C)
        for t in range(steps):
            acts = oracle.sample_actions(oracle.avail_rows(ref), KEY, t, env0=int(i))[:, 0].copy()
            want = oracle.seat_step(ref, c, bot.strategy, bot.trained, 0, acts, False, observe=False)
            assert np.array_equal(want["reward"][0], rewards[t, k]), f"game {i} cycle {t}"
        assert_states_equal(ref, _one(got, i), f"game {i}")
        for name, w in c.items():
            np.testing.assert_array_equal(np.asarray(carry[name][k]).astype(np.int64).reshape(w[0].shape),
                                          w[0].astype(np.int64), err_msg=f"game {i} carry {name}")


def test_config4_garden_of_war(oracle_threads):
    """GardenOfWar64x64, capacity_profile=False, CANCEL_ALTERNATING: 4096
    games of symbolic observations over 500 steps, and 256 games of pixel
    observations (uint8[1024, 1024, 3]) over the same 500 steps, three games
    followed by the oracle every cycle and their images compared with the
    oracle's renderer every 50th cycle and at the last."""
    import torch

    import nanorts_amd
    from nanorts_amd import env as envmod
    from nanorts_amd import rendering
    from nanorts_amd.content import map_name_to_scenario

    _say("config 4: GardenOfWar64x64 x 4096 x 500, pixels x 256")
    game = map_name_to_scenario("GardenOfWar64x64", conflict_strategy="CANCEL_ALTERNATING", capacity_profile=False)
    _rollout_case(game, False, 4096, 500, _sample(4096, 3, 4), oracle_threads)
    # the pixel surface at its full batch: per-call steps from the same start
    env = nanorts_amd.make("NanoRTS", scenario=game, surface="pixels", final_observation=False, device="cuda:0")
    L = 256
    roots = envmod.env_roots(5, L)
    obs, state = env.reset(roots)
    assert obs[env.agents[0]].image.shape == (L, 1024, 1024, 3)
    sample = (0, 97, 255)
    refs = [batch_initial(game, 1, roots[i:i + 1]) for i in sample]
    oracle = Oracle(game)
    tiles = rendering.tile_table(game.bucket.unit_type_capacity)
    steps = 500
    compared = 0
    for t in range(steps):
        words = env.get_avail_actions(state, form="words")
        acts = env.sample_actions(words, KEY, t)
        obs, state, _, _, _ = env.step(None, state, acts, donate=True)
        rows = {a: acts[a][list(sample)].cpu().numpy() for a in env.agents}
        for k, i in enumerate(sample):
            oracle.env_step(refs[k], np.stack([rows[a][k:k + 1] for a in env.agents], 1), False, observe=False)
        if t % 50 == 49 or t == steps - 1:
            torch.cuda.synchronize()
            _say(f"pixels x {L}: cycle {t}")
            for k, i in enumerate(sample):
                image, _ = oracle.pixels(refs[k], False, tiles)
                for p, agent in enumerate(env.agents):
                    np.testing.assert_array_equal(obs[agent].image[i].cpu().numpy(), image[0, p],
                                                  err_msg=f"game {i} cycle {t} {agent}")
                compared += 1
    assert compared == 3 * 10
