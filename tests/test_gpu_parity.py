"""GPU parity: every HIP entry point against the C oracle on the same inputs.

Integer/byte/index outputs must match bit for bit; rewards are exact +-1/0
floats, compared exactly.  States come from oracle rollouts of the shipped
maps under each conflict strategy, so they are reachable mid-game states.
"""
from __future__ import annotations

import numpy as np
import pytest

from tests.helpers import CASES, advanced_states, assert_states_equal, game_for, to_device, to_host
from oracle.oracle import copy_state

pytestmark = pytest.mark.gpu

FAST_CASES = ["8x8-original-both", "16x16-finetuned-both", "16x16-random-partial", "16x16-alternating",
              "melee-both", "barracks-random", "obstacle-alternating"]


def _env(game, partial, **kw):
    import nanorts_amd

    return nanorts_amd.make("NanoRTS", scenario=game, partial_observability=partial, **kw)


@pytest.mark.parametrize("case", FAST_CASES + ["gow-alternating"])
def test_masks_visibility_observation(case, oracle_threads):
    game, partial = game_for(case)
    L = 16 if case.startswith("gow") else 96
    oracle, st = advanced_states(game, L, 40 if case.startswith("gow") else 150, partial, oracle_threads)
    env = _env(game, partial)
    dev = to_device(env, st)
    words = env.get_avail_actions(dev, form="words")
    got_words = np.stack([words[a].cpu().numpy() for a in env.agents], 1).view(np.uint32)
    np.testing.assert_array_equal(got_words, oracle.avail_words(st))
    rows = env.get_avail_actions(dev)
    got_rows = np.stack([rows[a].cpu().numpy() for a in env.agents], 1)
    np.testing.assert_array_equal(got_rows, oracle.avail_rows(st))
    legal = env.legality(dev, form="rows").cpu().numpy()
    np.testing.assert_array_equal(legal, oracle.legality_rows(st))
    for observer in (0, 1):
        np.testing.assert_array_equal(env.visible_cells(dev, observer).cpu().numpy(), oracle.visible_cells(st, observer))
    for p in (False, True):
        env_p = _env(game, p)
        obs = env_p.get_obs(dev)
        want_maps, want_scalars = oracle.symbolic(st, p)
        for i, agent in enumerate(env.agents):
            np.testing.assert_array_equal(obs[agent].feature_maps.cpu().numpy(), want_maps[:, i])
            np.testing.assert_array_equal(obs[agent].scalars.cpu().numpy(), want_scalars[:, i])


@pytest.mark.parametrize("case", FAST_CASES)
def test_core_step(case, oracle_threads):
    """nanorts_step against core.step on decoded sampled actions, one cycle
    from many mid-game states, with random episode-root keys."""
    game, partial = game_for(case)
    L = 128
    oracle, st = advanced_states(game, L, 120, partial, oracle_threads, seed=11)
    rows = oracle.avail_rows(st)
    actions = oracle.sample_actions(rows, (3, 4), 999)
    commands = oracle.decode_actions(st, actions)
    rng = np.random.default_rng(5)
    keys = rng.integers(0, 2**32, size=(L, 2), dtype=np.uint64).astype(np.uint32)
    env = _env(game, partial)
    dev = to_device(env, st)
    import torch

    out = env.core_step(dev, {k: torch.as_tensor(v) for k, v in commands.items()}, keys)
    want = oracle.core_step(st, commands, keys)
    assert_states_equal(st, to_host(dev), f"{case} core.step")
    for name in ("terminated", "truncated", "reward", "admitted_harvest", "admitted_return", "admitted_produce",
                 "admitted_attack"):
        np.testing.assert_array_equal(out[name].cpu().numpy().astype(want[name].dtype), want[name], err_msg=name)


@pytest.mark.parametrize("case", FAST_CASES)
def test_env_step_per_call(case, oracle_threads):
    """The per-call path (avail words -> sampler -> env.step) cycle by cycle
    against the oracle: actions, rewards, dones, infos, observations and the
    whole state after every cycle."""
    import torch

    game, partial = game_for(case)
    L, steps = 64, 60
    oracle, st = advanced_states(game, L, 80, partial, oracle_threads, seed=3)
    env = _env(game, partial, reward_components=True)
    dev = to_device(env, st)
    key = (17, 23)
    for t in range(steps):
        words = env.get_avail_actions(dev, form="words")
        stacked = torch.stack([words[a] for a in env.agents], 1)
        acts = env.sample_actions(stacked, key, t)
        want_rows = oracle.avail_rows(st)
        want_actions = oracle.sample_actions(want_rows, key, t)
        got_actions = np.stack([acts[a].cpu().numpy() for a in env.agents], 1)
        np.testing.assert_array_equal(got_actions, want_actions, err_msg=f"actions at cycle {t}")
        obs, dev, rewards, dones, infos = env.step(None, dev, acts, donate=True)
        want = oracle.env_step(st, want_actions, partial)
        assert_states_equal(st, to_host(dev), f"{case} cycle {t}")
        got_reward = np.stack([rewards[a].cpu().numpy() for a in env.agents], 1)
        np.testing.assert_array_equal(got_reward, want["reward"])
        np.testing.assert_array_equal(dones["__all__"].cpu().numpy(), want["done"].astype(bool))
        np.testing.assert_array_equal(infos["terminated"].cpu().numpy(), want["terminated"].astype(bool))
        np.testing.assert_array_equal(infos["truncated"].cpu().numpy(), want["truncated"].astype(bool))
        np.testing.assert_array_equal(infos["winner"].cpu().numpy(), want["winner"])
        np.testing.assert_array_equal(infos["spawn_overflowed"].cpu().numpy(), want["spawn_overflowed"].astype(bool))
        for i, agent in enumerate(env.agents):
            np.testing.assert_array_equal(obs[agent].feature_maps.cpu().numpy(), want["feature_maps"][:, i])
            np.testing.assert_array_equal(obs[agent].scalars.cpu().numpy(), want["scalars"][:, i])


@pytest.mark.parametrize("case", FAST_CASES + ["16x16-noprofile-random"])
@pytest.mark.parametrize("recorded", [True, False])
def test_fused_rollout_matches_oracle(case, recorded, oracle_threads):
    """The fused rollout kernel over a long horizon against the oracle's
    rollout: per-cycle rewards and dones, the recorded actions, last
    observation and the final state.  Unrecorded, the kernel draws only the
    factors its decode reads; the game must not change."""
    game, partial = game_for(case)
    L = 64
    steps = 1000
    oracle, st = advanced_states(game, L, 0, partial, oracle_threads, seed=21)
    env = _env(game, partial)
    dev = to_device(env, st)
    got = env.rollout(dev, steps, (5, 9), record=True, record_actions=recorded)
    want = oracle.rollout(st, (5, 9), 0, steps, partial, threads=oracle_threads, record_actions=recorded)
    if recorded:
        np.testing.assert_array_equal(got["actions"].cpu().numpy(), want["actions"])
    np.testing.assert_array_equal(got["rewards"].cpu().numpy(), want["rewards"])
    np.testing.assert_array_equal(got["dones"].cpu().numpy(), want["dones"].astype(bool))
    np.testing.assert_array_equal(got["feature_maps"][0].cpu().numpy(), want["feature_maps"])
    np.testing.assert_array_equal(got["scalars"][0].cpu().numpy(), want["scalars"])
    assert_states_equal(st, to_host(dev), f"{case} rollout")


@pytest.mark.parametrize("case", ["16x16-random-partial", "melee-both", "gow-alternating"])
def test_pixels(case, oracle_threads):
    """nanorts_pixels (from the state) and nanorts_pixels_from_maps (from the
    symbolic maps) against the oracle's renderer, both observability modes."""
    import torch

    from nanorts_amd import rendering

    game, _ = game_for(case)
    gow = case.startswith("gow")
    L = 4 if gow else 32
    oracle, st = advanced_states(game, L, 40 if gow else 120, True, oracle_threads, seed=4)
    tiles = rendering.tile_table(game.bucket.unit_type_capacity)
    for partial in (False, True):
        env = _env(game, partial, surface="pixels")
        dev = to_device(env, st)
        want_image, want_scalars = oracle.pixels(st, partial, tiles)
        obs = env.get_obs(dev)
        for i, agent in enumerate(env.agents):
            np.testing.assert_array_equal(obs[agent].image.cpu().numpy(), want_image[:, i])
            np.testing.assert_array_equal(obs[agent].scalars.cpu().numpy(), want_scalars[:, i])
        sym = _env(game, partial).get_obs(dev)
        maps = torch.stack([sym[a].feature_maps for a in env.agents], 1)
        np.testing.assert_array_equal(env.pixels_from_maps(maps).cpu().numpy(), want_image)


def test_pixel_surface_env_step(oracle_threads):
    """env.step on the pixel surface: published images against the oracle's
    renderer of the post-step (auto-reset) state, cycle by cycle."""
    import torch

    from nanorts_amd import rendering

    game, partial = game_for("barracks-random")
    L = 16
    oracle, st = advanced_states(game, L, 100, partial, oracle_threads, seed=8)
    tiles = rendering.tile_table(game.bucket.unit_type_capacity)
    env = _env(game, partial, surface="pixels")
    dev = to_device(env, st)
    for t in range(12):
        words = env.get_avail_actions(dev, form="words")
        acts = env.sample_actions(torch.stack([words[a] for a in env.agents], 1), (2, 3), t)
        obs, dev, rewards, dones, infos = env.step(None, dev, acts, donate=True)
        oracle.env_step(st, np.stack([acts[a].cpu().numpy() for a in env.agents], 1), partial, observe=False)
        want_image, want_scalars = oracle.pixels(st, partial, tiles)
        for i, agent in enumerate(env.agents):
            np.testing.assert_array_equal(obs[agent].image.cpu().numpy(), want_image[:, i], err_msg=f"cycle {t}")
            np.testing.assert_array_equal(obs[agent].scalars.cpu().numpy(), want_scalars[:, i])
        final = infos["final_observation"]
        assert final[env.agents[0]].image.shape == obs[env.agents[0]].image.shape


def test_pixel_surface_with_a_custom_asset_set(oracle_threads):
    """The pixel surface drawing a prepared Asset set other than the shipped
    sheet (recoloured floor and player-0 sprites): images against the
    oracle's renderer with the same table."""
    from nanorts_amd import rendering

    game, partial = game_for("16x16-random-partial")
    oracle, st = advanced_states(game, 16, 80, partial, oracle_threads, seed=12)
    sheet = {name: rendering.read_png(rendering.ART_DIRECTORY / f"{name}.png").copy()
             for name in rendering.sprite_names()}
    sheet["floor"][..., 1] ^= 0x30
    for name in sheet:
        if name.startswith("player0-"):
            sheet[name][..., 2] ^= 0x55
    assets = rendering.prepare_assets(game.bucket, tiles=sheet)
    env = _env(game, partial, surface="pixels", assets=assets)
    obs = env.get_obs(to_device(env, st))
    want_image, _ = oracle.pixels(st, partial, assets.tiles)
    default_image, _ = oracle.pixels(st, partial, rendering.tile_table(game.bucket.unit_type_capacity))
    assert not np.array_equal(want_image, default_image)
    for i, agent in enumerate(env.agents):
        np.testing.assert_array_equal(obs[agent].image.cpu().numpy(), want_image[:, i])


def test_reset_where_done(oracle_threads):
    import torch

    game, partial = game_for("16x16-finetuned-both")
    oracle, st = advanced_states(game, 32, 50, partial, oracle_threads)
    env = _env(game, partial)
    dev = to_device(env, st)
    done = (np.arange(32) % 3 == 0).astype(np.uint8)
    env.reset_where_done(dev, torch.as_tensor(done.astype(bool)))
    want = copy_state(st)
    oracle.reset_where_done(want, done)
    assert_states_equal(want, to_host(dev), "reset_where_done")


def test_self_check_and_build_id():
    from nanorts_amd import native

    lib = native.load()
    import ctypes

    dev = (ctypes.c_int32 * 1)(0)
    assert lib.nanorts_self_check(dev, 1).decode() == ""
    assert len(lib.nanorts_build_id().decode()) > 0


_ = CASES
