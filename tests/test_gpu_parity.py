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
              "melee-both", "barracks-random", "obstacle-alternating", "10x10-random-partial", "9x8-alternating",
              "ranged-random", "24x24-barricades-alternating", "32x32-random-partial"]


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
    """nanorts_amd_step against core.step on decoded sampled actions, one cycle
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
    against the oracle: actions, rewards, dones, infos, observations, the
    ending state's observation (final_observation), the reward components and
    the whole state after every cycle."""
    import torch

    print(f"env.step per call {case}", flush=True)
    game, partial = game_for(case)
    L, steps = 64, 60
    oracle, st = advanced_states(game, L, 80, partial, oracle_threads, seed=3)
    env = _env(game, partial, reward_components=True)
    dev = to_device(env, st)
    key = (17, 23)
    ended = 0
    for t in range(steps):
        words = env.get_avail_actions(dev, form="words")
        stacked = torch.stack([words[a] for a in env.agents], 1)
        acts = env.sample_actions(stacked, key, t)
        want_rows = oracle.avail_rows(st)
        want_actions = oracle.sample_actions(want_rows, key, t)
        got_actions = np.stack([acts[a].cpu().numpy() for a in env.agents], 1)
        np.testing.assert_array_equal(got_actions, want_actions, err_msg=f"actions at cycle {t}")
        obs, dev, rewards, dones, infos = env.step(None, dev, acts, donate=True)
        want = oracle.env_step(st, want_actions, partial, final=True)
        assert_states_equal(st, to_host(dev), f"{case} cycle {t}")
        ended += int(want["done"].sum())
        final = infos["final_observation"]
        for i, agent in enumerate(env.agents):
            np.testing.assert_array_equal(final[agent].feature_maps.cpu().numpy(), want["final_feature_maps"][:, i],
                                          err_msg=f"final observation at cycle {t}")
            np.testing.assert_array_equal(final[agent].scalars.cpu().numpy(), want["final_scalars"][:, i])
            np.testing.assert_array_equal(infos["reward_components"][agent].cpu().numpy(),
                                          want["reward_components"][:, i], err_msg=f"components at cycle {t}")
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
    if game.max_cycles <= 80 + steps:  # a horizon inside the run: episode ends were compared
        assert ended > 0


def _poison_allocator(nbytes: int) -> None:
    """Fill `nbytes` of device memory with a sentinel and free it, so that the
    next allocations (torch's caching allocator reuses the block) start with
    values no kernel writes: an output row a kernel leaves unwritten then
    differs from the oracle's instead of reading as a lucky zero."""
    import torch

    junk = torch.full((nbytes // 4,), 0x4D4D4D4D, dtype=torch.int32, device="cuda")
    torch.cuda.synchronize()
    del junk


def _first_pass(monkeypatch, mode: str) -> None:
    """Select the rollout's first pass: "auto" (the library's choice by
    board), "lean" (one game per wave) or "pair" (two games per wave)."""
    if mode == "auto":
        monkeypatch.delenv("NANORTS_AMD_FIRST_PASS", raising=False)
    else:
        monkeypatch.setenv("NANORTS_AMD_FIRST_PASS", mode)


@pytest.mark.parametrize("case", FAST_CASES + ["16x16-noprofile-random"])
@pytest.mark.parametrize("recorded", [True, False])
@pytest.mark.parametrize("first_pass", ["auto", "lean", "pair"])
def test_fused_rollout_matches_oracle(case, recorded, first_pass, monkeypatch, oracle_threads):
    """The fused rollout kernel over a long horizon against the oracle's
    rollout: per-cycle rewards and dones, the recorded actions, last
    observation and the final state, with each first pass.  Unrecorded, the
    kernel draws only the factors its decode reads; the game must not
    change."""
    _first_pass(monkeypatch, first_pass)
    game, partial = game_for(case)
    L = 64
    steps = 1000
    oracle, st = advanced_states(game, L, 0, partial, oracle_threads, seed=21)
    env = _env(game, partial)
    dev = to_device(env, st)
    _poison_allocator(steps * L * 2 * game.bucket.per_player_capacity * 7 * 4 + (64 << 20))
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
    """nanorts_amd_pixels (from the state) and nanorts_amd_pixels_from_maps (from the
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
    assert lib.nanorts_amd_self_check(dev, 1).decode() == ""
    from nanorts_amd import build

    assert lib.nanorts_amd_build_id().decode() == build.source_digest()


_ = CASES


def _crowded(game, L: int, units0: int = 72, units1: int = 12, seed: int = 5) -> dict:
    """GardenOfWar64x64 starting states with `units0` extra Workers for player
    0 and `units1` for player 1 on open cells, each born in its block's lowest
    free slot: more available units than the 64 lanes of a wave."""
    from oracle.oracle import batch_initial
    from tests.helpers import roots

    st = batch_initial(game, L, roots(L, seed))
    b = game.bucket
    rng = np.random.default_rng(seed)
    worker = 3
    hp = int(game.columns["hit_points"][worker])
    walls = game.terrain.reshape(-1)
    for l in range(L):
        em = st["entity_at"][l].reshape(-1)
        cells = rng.permutation(np.flatnonzero((em == -1) & ~walls))[:units0 + units1]
        for k, cell in enumerate(cells):
            player = 0 if k < units0 else 1
            start = b.neutral_capacity + player * b.per_player_capacity
            slot = start + int(np.flatnonzero(st["birth"][l, start:start + b.per_player_capacity] == -1)[0])
            birth = int(st["next_birth"][l])
            st["next_birth"][l] = birth + 1
            st["birth"][l, slot], st["unit_type"][l, slot], st["owner"][l, slot] = birth, worker, player
            st["cell"][l, slot], st["hit_points"][l, slot] = cell, hp
            em[cell] = slot
    return st


def test_crowded_rollout_takes_the_general_admission(oracle_threads):
    """With more than 64 available units a cycle's requests do not fit one
    wave, and the fused rollout admits them request by request.  The
    rollout's own count shows that path ran in every game, and the result
    matches the oracle."""
    from oracle.oracle import Oracle

    print("crowded rollout", flush=True)
    game, partial = game_for("gow-alternating")
    L, steps = 8, 24
    st = _crowded(game, L)
    oracle = Oracle(game)
    assert (oracle.violations(st) == 0).all()
    assert ((st["birth"][:, game.bucket.neutral_capacity:] != -1).sum(1) > 64).all()
    env = _env(game, partial)
    dev = to_device(env, st)
    got = env.rollout(dev, steps, (2, 7), record=True, count_general=True)
    want = oracle.rollout(st, (2, 7), 0, steps, partial, threads=oracle_threads)
    general = got["general_admissions"].cpu().numpy()
    assert (general >= 1).all(), general
    np.testing.assert_array_equal(got["rewards"].cpu().numpy(), want["rewards"])
    np.testing.assert_array_equal(got["dones"].cpu().numpy(), want["dones"].astype(bool))
    np.testing.assert_array_equal(got["feature_maps"][0].cpu().numpy(), want["feature_maps"])
    assert_states_equal(st, to_host(dev), "crowded rollout")
    # an ordinary start never leaves the one-wave admission
    plain = _env(game, partial)
    fresh = to_device(plain, _crowded(game, L, units0=0, units1=0))
    quiet = plain.rollout(fresh, 4, (2, 7), record=False, count_general=True)
    assert (quiet["general_admissions"].cpu().numpy() == 0).all()


def _packed(game, extra: list[int], seed: int = 3, alternate: bool = True) -> dict:
    """Starting states of `game` with extra[l] Workers added to lane l on open
    cells, alternating between the players (or all for player 0), each born
    in its block's lowest free slot."""
    from oracle.oracle import batch_initial
    from tests.helpers import roots

    L = len(extra)
    st = batch_initial(game, L, roots(L, seed))
    b = game.bucket
    rng = np.random.default_rng(seed)
    worker = 3
    hp = int(game.columns["hit_points"][worker])
    walls = game.terrain.reshape(-1)
    for l in range(L):
        em = st["entity_at"][l].reshape(-1)
        cells = rng.permutation(np.flatnonzero((em == -1) & ~walls))[:extra[l]]
        for k, cell in enumerate(cells):
            player = k & 1 if alternate else 0
            start = b.neutral_capacity + player * b.per_player_capacity
            slot = start + int(np.flatnonzero(st["birth"][l, start:start + b.per_player_capacity] == -1)[0])
            birth = int(st["next_birth"][l])
            st["next_birth"][l] = birth + 1
            st["birth"][l, slot], st["unit_type"][l, slot], st["owner"][l, slot] = birth, worker, player
            st["cell"][l, slot], st["hit_points"][l, slot] = cell, hp
            em[cell] = slot
    return st


@pytest.mark.parametrize("first_pass", ["lean", "pair"])
def test_two_pass_rollout_hands_games_to_the_second_pass(first_pass, monkeypatch, oracle_threads):
    """The rollout's first pass stages a 32-slot window of each player's 70
    slots and runs a game until a unit could spawn past its window (its
    units plus the PRODUCE actions due next cycle exceed 32), or a cycle
    needs more than the first pass's lanes (two games per wave: more than 32
    available units or 64 live slots); the second pass, on the full block,
    runs the rest of that game's cycles.  Games that start with 22..38 live
    slots, the added Workers all player 0's and 200 resources each, cross a
    bound part-way through the launch (spawns), or never, and with two games
    per wave also at cycle 0 (available units).  All of them match the
    oracle and the one-pass launch."""
    from oracle.oracle import Oracle

    _first_pass(monkeypatch, first_pass)
    print("two-pass rollout", first_pass, flush=True)
    game, partial = game_for("16x16-random-partial")
    b = game.bucket
    base = int((_packed(game, [0])["birth"][0] != -1).sum())
    extra = [22 - base + k for k in range(17)]
    st = _packed(game, extra, alternate=False)
    st["player_resources"][:] = 200
    live = (st["birth"] != -1).sum(1)
    assert live.min() == 22 and live.max() == 38
    units0 = (st["birth"][:, b.neutral_capacity:b.neutral_capacity + b.per_player_capacity] != -1).sum(1)
    oracle = Oracle(game)
    assert (oracle.violations(st) == 0).all()
    L, steps = len(extra), 128  # one launch
    env = _env(game, partial)
    dev = to_device(env, st)
    one = to_device(env, st)
    got = env.rollout(dev, steps, (1, 2), record=True, count_general=True)
    first = got["first_pass_cycles"].cpu().numpy()
    print("first-pass cycles per game:", first.tolist(), flush=True)
    assert (first[units0 > 32] == 0).all()
    assert ((first > 0) & (first < steps)).any()
    assert (first == steps).any()
    if first_pass == "pair":
        assert (first == 0).any()
    want = oracle.rollout(st, (1, 2), 0, steps, partial, threads=oracle_threads)
    np.testing.assert_array_equal(got["rewards"].cpu().numpy(), want["rewards"])
    np.testing.assert_array_equal(got["dones"].cpu().numpy(), want["dones"].astype(bool))
    np.testing.assert_array_equal(got["feature_maps"][0].cpu().numpy(), want["feature_maps"])
    np.testing.assert_array_equal(got["scalars"][0].cpu().numpy(), want["scalars"])
    assert_states_equal(st, to_host(dev), "two-pass rollout")
    single = env.rollout(one, steps, (1, 2), record=True, count_general=True, two_pass=False)
    np.testing.assert_array_equal(single["rewards"].cpu().numpy(), want["rewards"])
    np.testing.assert_array_equal(single["general_admissions"].cpu().numpy(),
                                  got["general_admissions"].cpu().numpy())
    assert (single["first_pass_cycles"] is None)
    assert_states_equal(st, to_host(one), "one-pass rollout")


@pytest.mark.parametrize("first_pass", ["auto", "pair"])
def test_pair_first_pass_hands_games_to_the_second_pass(first_pass, monkeypatch, oracle_threads):
    """With two games per wave (the choice on 8x8 boards) the first pass runs
    a game while it has at most 32 available units, 64 live slots and room
    in its slot window; the second pass runs the rest.  Games that start with
    24..40 live slots on basesWorkers8x8, the added Workers all player 0's
    and 200 resources each, cross a bound at cycle 0 or not at all (on this
    crowded board no spawn takes a game past its window within the launch;
    the 16x16 test above crosses part-way).  All of them match the oracle;
    an odd number of games leaves the last wave's second half without a
    game."""
    from oracle.oracle import Oracle

    _first_pass(monkeypatch, first_pass)
    print("pair two-pass rollout", flush=True)
    game, partial = game_for("8x8-original-both")
    base = int((_packed(game, [0])["birth"][0] != -1).sum())
    extra = [24 - base + k for k in range(17)]
    st = _packed(game, extra, alternate=False)
    st["player_resources"][:] = 200
    live = (st["birth"] != -1).sum(1)
    assert live.min() == 24 and live.max() == 40
    oracle = Oracle(game)
    assert (oracle.violations(st) == 0).all()
    L, steps = len(extra), 128  # one launch
    env = _env(game, partial)
    dev = to_device(env, st)
    got = env.rollout(dev, steps, (1, 2), record=True, count_general=True)
    first = got["first_pass_cycles"].cpu().numpy()
    print("first-pass cycles per game:", first.tolist(), flush=True)
    assert (first == 0).any()
    assert (first == steps).any()
    want = oracle.rollout(st, (1, 2), 0, steps, partial, threads=oracle_threads)
    np.testing.assert_array_equal(got["rewards"].cpu().numpy(), want["rewards"])
    np.testing.assert_array_equal(got["dones"].cpu().numpy(), want["dones"].astype(bool))
    np.testing.assert_array_equal(got["feature_maps"][0].cpu().numpy(), want["feature_maps"])
    np.testing.assert_array_equal(got["scalars"][0].cpu().numpy(), want["scalars"])
    assert_states_equal(st, to_host(dev), "pair two-pass rollout")


@pytest.mark.parametrize("first_pass", ["auto", "pair"])
def test_pair_first_pass_holds_two_live_slots_and_two_entries_a_lane(first_pass, monkeypatch, oracle_threads):
    """Two games per wave with 33..64 live slots and 33..64 pending MOVE /
    PRODUCE entries per game: each lane of a half-wave team holds two of
    each (completion's members, admission's claims).  Crowded 16x16 games
    (44..51 live slots, Workers of both players), advanced 12 cycles by the
    oracle so that most units hold a pending action, stay in the first pass
    for the whole launch, reach more than 32 entries, and match the
    oracle."""
    from oracle.oracle import Oracle

    _first_pass(monkeypatch, first_pass)
    print("pair pass, crowded", first_pass, flush=True)
    game, partial = game_for("16x16-random-partial")
    b = game.bucket
    base = int((_packed(game, [0])["birth"][0] != -1).sum())
    st = _packed(game, [44 - base + k for k in range(8)])
    st["player_resources"][:] = 20
    oracle = Oracle(game)
    oracle.rollout(st, (1, 2), 0, 12, partial, threads=oracle_threads, record=False)
    assert (oracle.violations(st) == 0).all()
    live = (st["birth"] != -1).sum(1)
    assert live.min() > 32
    L, steps = st["birth"].shape[0], 64
    env = _env(game, partial)
    dev = to_device(env, st)
    got = env.rollout(dev, steps, (1, 2), step0=12, record=True, count_general=True)
    want = oracle.rollout(st, (1, 2), 12, steps, partial, threads=oracle_threads)
    first = got["first_pass_cycles"].cpu().numpy()
    assert (first == steps).all(), first
    pk, birth = st["pending_kind"], st["birth"]
    np.testing.assert_array_equal(got["rewards"].cpu().numpy(), want["rewards"])
    np.testing.assert_array_equal(got["dones"].cpu().numpy(), want["dones"].astype(bool))
    np.testing.assert_array_equal(got["feature_maps"][0].cpu().numpy(), want["feature_maps"])
    np.testing.assert_array_equal(got["scalars"][0].cpu().numpy(), want["scalars"])
    assert_states_equal(st, to_host(dev), "crowded pair rollout")
    # the oracle's run reached more than 32 entries (final state shown)
    print("entries at the end:", (((pk == 1) | (pk == 4)) & (birth != -1)).sum(1).tolist(), flush=True)


def test_crowded_env_step_per_call(oracle_threads):
    """env.step on the same crowded states, cycle by cycle, against the oracle."""
    import torch

    from oracle.oracle import Oracle

    print("crowded env.step", flush=True)
    game, partial = game_for("gow-alternating")
    L = 8
    st = _crowded(game, L, seed=6)
    oracle = Oracle(game)
    env = _env(game, partial)
    dev = to_device(env, st)
    for t in range(6):
        words = env.get_avail_actions(dev, form="words")
        acts = env.sample_actions(torch.stack([words[a] for a in env.agents], 1), (4, 4), t)
        obs, dev, rewards, dones, infos = env.step(None, dev, acts, donate=True)
        want = oracle.env_step(st, np.stack([acts[a].cpu().numpy() for a in env.agents], 1), partial)
        assert_states_equal(st, to_host(dev), f"crowded cycle {t}")
        for i, agent in enumerate(env.agents):
            np.testing.assert_array_equal(obs[agent].feature_maps.cpu().numpy(), want["feature_maps"][:, i])
