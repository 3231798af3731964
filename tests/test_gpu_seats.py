"""GPU parity of per-lane seats (src/nanorts/bots/seat.py:335-375) against
the oracle: the "drawn" rule, whose learner is drawn from each episode's root
at reset and again when a game ends, and a fixed per-lane seat array through
reset_seat / step_seat.

basesWorkers8x8 with a 60-cycle horizon, so that every game ends (and draws
its next seat) more than once.  Each cycle the learner's rows are the
harness sampler's rows at the lane's seat; the oracle's seat step takes the
same per-lane seats and re-draws them where a game ended.  Compared bit for
bit: the seats, the learner's reward (at the seat before the step), dones,
the learner's observation (at the seat after it), the state and the carry.
"""
from __future__ import annotations

import sys

import numpy as np
import pytest

from oracle.oracle import Oracle, batch_initial, empty_carry
from tests.helpers import assert_states_equal, roots, to_host

pytestmark = pytest.mark.gpu

HORIZON = 60


def _say(*parts):
    print(*parts, flush=True)
    sys.stdout.flush()


def _game():
    from nanorts_amd.content import map_name_to_scenario

    return map_name_to_scenario("basesWorkers8x8", max_cycles=HORIZON)


def _carry_equal(want, got, where):
    from nanorts_amd.bots import carry_numpy

    host = carry_numpy(got)
    for name, w in want.items():
        np.testing.assert_array_equal(np.asarray(host[name]).astype(np.int64).reshape(w.shape), w.astype(np.int64),
                                      err_msg=f"{where}: carry {name}")


def _at(per_player: np.ndarray, seats: np.ndarray) -> np.ndarray:
    return per_player[np.arange(per_player.shape[0]), seats]


@pytest.mark.parametrize("bot_name", ["workerRushAI", "lightRushAI"])
def test_drawn_seat_steps_match_oracle(bot_name):
    import torch

    from nanorts_amd import bots

    _say(f"drawn seat steps {bot_name}")
    torch.cuda.set_device(0)
    game = _game()
    bot = getattr(bots, bot_name)
    seat = bots.SeatEnv(bot, scenario=game, seat="drawn", device="cuda:0")
    L = 48
    keys = roots(L, 23)
    obs, sst = seat.reset(keys)
    oracle = Oracle(game)
    ref = batch_initial(game, L, keys)
    carry = empty_carry(L, game.bucket.per_player_capacity)
    seats = oracle.episode_seats(ref)
    assert 0 < int(seats.sum()) < L, "both seats are drawn among 48 games"
    np.testing.assert_array_equal(sst.seat.cpu().numpy(), seats)
    maps, scalars = oracle.symbolic(ref, False)
    np.testing.assert_array_equal(obs[bots.LEARNER].feature_maps.cpu().numpy(), _at(maps, seats))
    np.testing.assert_array_equal(obs[bots.LEARNER].scalars.cpu().numpy(), _at(scalars, seats))
    redrawn = 0
    for t in range(2 * HORIZON + 30):
        acts = np.ascontiguousarray(_at(oracle.sample_actions(oracle.avail_rows(ref), (7, 9), t), seats))
        before = seats.copy()
        want = oracle.seat_step(ref, carry, bot.strategy, bot.trained, seats, acts, False, draw=True)
        obs, sst, rew, done, info = seat.step(None, sst, {bots.LEARNER: torch.as_tensor(acts, device="cuda:0")},
                                              donate=True)
        np.testing.assert_array_equal(sst.seat.cpu().numpy(), seats, err_msg=f"cycle {t} seats")
        np.testing.assert_array_equal(rew[bots.LEARNER].cpu().numpy(), _at(want["reward"], before),
                                      err_msg=f"cycle {t} reward")
        np.testing.assert_array_equal(done[bots.LEARNER].cpu().numpy(), want["done"].astype(bool))
        np.testing.assert_array_equal(obs[bots.LEARNER].feature_maps.cpu().numpy(), _at(want["feature_maps"], seats),
                                      err_msg=f"cycle {t} observation")
        np.testing.assert_array_equal(obs[bots.LEARNER].scalars.cpu().numpy(), _at(want["scalars"], seats))
        np.testing.assert_array_equal(info["winner"].cpu().numpy(), want["winner"])
        kept = ~want["done"].astype(bool)
        final = info["final_observation"][bots.LEARNER].feature_maps.cpu().numpy()
        np.testing.assert_array_equal(final[kept], obs[bots.LEARNER].feature_maps.cpu().numpy()[kept])
        redrawn += int((before != seats).sum())
    assert_states_equal(ref, to_host(sst.environment_state), "final state")
    _carry_equal(carry, sst.carry, "final")
    assert redrawn > 0, "some game changed seat at an episode end"


def test_drawn_seat_rollout_matches_oracle():
    """The fused rollout under the drawn rule: rewards of both players, dones,
    the learner's recorded rows, the seat of every cycle, the final seats,
    state and carry, against the oracle's per-cycle seat steps."""
    import torch

    from nanorts_amd import bots

    _say("drawn seat rollout")
    torch.cuda.set_device(0)
    game = _game()
    bot = bots.lightRushAI
    seat = bots.SeatEnv(bot, scenario=game, seat="drawn", final_observation=False, device="cuda:0")
    L = 40
    keys = roots(L, 29)
    _, sst = seat.reset(keys)
    oracle = Oracle(game)
    ref = batch_initial(game, L, keys)
    carry = empty_carry(L, game.bucket.per_player_capacity)
    seats = oracle.episode_seats(ref)
    steps = 3 * HORIZON + 10
    key = (31, 37)
    got = seat.rollout(sst, steps, key, record_actions=True)
    rewards, dones, actions, record = (got[k].cpu().numpy() for k in ("rewards", "dones", "actions", "seats"))
    for t in range(steps):
        np.testing.assert_array_equal(record[t], seats, err_msg=f"cycle {t} seats")
        acts = np.ascontiguousarray(_at(oracle.sample_actions(oracle.avail_rows(ref), key, t), seats))
        np.testing.assert_array_equal(actions[t], acts, err_msg=f"cycle {t} learner rows")
        want = oracle.seat_step(ref, carry, bot.strategy, bot.trained, seats, acts, False,
                                observe=t == steps - 1, draw=True)
        np.testing.assert_array_equal(rewards[t], want["reward"], err_msg=f"cycle {t}")
        np.testing.assert_array_equal(dones[t], want["done"].astype(bool), err_msg=f"cycle {t}")
    np.testing.assert_array_equal(sst.seat.cpu().numpy(), seats)
    assert_states_equal(ref, to_host(sst.environment_state), "final state")
    _carry_equal(carry, sst.carry, "final")
    np.testing.assert_array_equal(got["feature_maps"][0].cpu().numpy(), want["feature_maps"])
    assert len(np.unique(record, axis=0)) > 1, "the seats changed during the rollout"


def test_drawn_seat_request_response_equals_the_fused_step():
    import torch

    from nanorts_amd import bots, groups

    _say("drawn seat step_request/step_response")
    torch.cuda.set_device(0)
    game = _game()
    seat = bots.SeatEnv(bots.workerRushAI, scenario=game, seat="drawn", reward_components=True, device="cuda:0")
    L = 32
    keys = roots(L, 31)
    _, fused = seat.reset(keys)
    _, split = seat.reset(keys)
    oracle = Oracle(game)
    C = game.bucket.per_player_capacity
    ended = 0
    for t in range(HORIZON + 40):
        words = seat.get_avail_actions(fused)[bots.LEARNER].cpu().numpy()
        rows = np.zeros((L, 2, C, words.shape[-1]), bool)
        rows[:, 0] = words
        acts = {bots.LEARNER: torch.as_tensor(oracle.sample_actions(rows, (3, 5), t)[:, 0].copy(), device="cuda:0")}
        a = seat.step(None, fused, acts, donate=True)
        (k, core, cmds), carry = seat.step_request(split, acts)
        stepped = groups.step_groups([(k, core, cmds, seat)])[0]
        b = seat.step_response(split, carry, stepped)
        agent = bots.LEARNER
        assert torch.equal(fused.seat, split.seat), f"cycle {t} seats"
        assert torch.equal(a[0][agent].feature_maps, b[0][agent].feature_maps), f"cycle {t}"
        assert torch.equal(a[2][agent], b[2][agent]), f"cycle {t} reward"
        assert torch.equal(a[3][agent], b[3][agent])
        assert torch.equal(a[4]["reward_components"][agent], b[4]["reward_components"][agent])
        assert torch.equal(a[4]["final_observation"][agent].feature_maps,
                           b[4]["final_observation"][agent].feature_maps), f"cycle {t} final observation"
        assert_states_equal(to_host(fused.environment_state), to_host(split.environment_state), f"cycle {t}")
        for name in fused.carry:
            assert torch.equal(fused.carry[name], split.carry[name]), f"cycle {t} carry {name}"
        ended += int(a[3]["__all__"].sum())
    assert ended > 0
    assert 0 < int(fused.seat.sum()) < L


def test_seat_functions_with_a_per_lane_seat():
    """reset_seat / step_seat with an int32[L] seat: the seats stay as given
    across episode ends; a Player index and the rules give their seats."""
    import torch

    from nanorts_amd import bots
    from nanorts_amd.model import ModelError

    _say("seat functions per-lane")
    torch.cuda.set_device(0)
    game = _game()
    bot = bots.workerRushAI
    L = 24
    keys = roots(L, 37)
    given = np.array([(l * 7) % 3 == 1 for l in range(L)], np.int32)
    state, obs = bots.reset_seat(keys, game, bot=bot, seat=torch.as_tensor(given, device="cuda:0"), device="cuda:0")
    np.testing.assert_array_equal(state.seat.cpu().numpy(), given)
    oracle = Oracle(game)
    ref = batch_initial(game, L, keys)
    carry = empty_carry(L, game.bucket.per_player_capacity)
    seats = given.copy()
    maps, _ = oracle.symbolic(ref, False)
    np.testing.assert_array_equal(obs.feature_maps.cpu().numpy(), _at(maps, seats))
    ended = 0
    for t in range(HORIZON + 20):
        acts = np.ascontiguousarray(_at(oracle.sample_actions(oracle.avail_rows(ref), (11, 13), t), seats))
        want = oracle.seat_step(ref, carry, bot.strategy, bot.trained, seats, acts, False)
        out = bots.step_seat(state, torch.as_tensor(acts, device="cuda:0"), game, bot=bot, seat=given,
                             donate=True, device="cuda:0")
        state = out.seat_state
        np.testing.assert_array_equal(out.reward.cpu().numpy(), _at(want["reward"], given), err_msg=f"cycle {t}")
        np.testing.assert_array_equal(out.done.cpu().numpy(), want["done"].astype(bool))
        np.testing.assert_array_equal(out.observation.feature_maps.cpu().numpy(), _at(want["feature_maps"], given))
        ended += int(want["done"].sum())
    np.testing.assert_array_equal(state.seat.cpu().numpy(), given)
    np.testing.assert_array_equal(seats, given)
    assert_states_equal(ref, to_host(state.environment_state), "final state")
    _carry_equal(carry, state.carry, "final")
    assert ended > 0
    # the other seat functions read the learner's side of each lane
    masks = bots.legal_seat_actions(state, game, seat=given, device="cuda:0").cpu().numpy()
    np.testing.assert_array_equal(masks, _at(oracle.avail_rows(ref), given))
    maps, scalars = oracle.symbolic(ref, False)
    seen = bots.observe_seat(state, game, seat=given, device="cuda:0")
    np.testing.assert_array_equal(seen.feature_maps.cpu().numpy(), _at(maps, given))
    np.testing.assert_array_equal(seen.scalars.cpu().numpy(), _at(scalars, given))
    n = game.bucket.neutral_capacity
    cells = ref["cell"][:, n:].astype(np.int32).reshape(L, 2, -1)
    np.testing.assert_array_equal(bots.seat_slot_cells(state, game, seat=given, device="cuda:0").cpu().numpy(),
                                  _at(cells, given))
    before = {k: v.clone() for k, v in state.carry.items()}
    new_carry, cmds = bots.seat_commands(state, game, bot=bot, seat=given, device="cuda:0")
    for name in before:
        assert torch.equal(state.carry[name], before[name]), "seat_commands leaves the seat state's carry"
    want = oracle.abstraction_act(ref, carry, bot.strategy, bot.trained, (1 - given).astype(np.int32))
    for name, value in want.items():
        np.testing.assert_array_equal(cmds[name].cpu().numpy(), value, err_msg=f"bot Commands {name}")
    _carry_equal(carry, new_carry, "after seat_commands")
    one, _ = bots.reset_seat(keys, game, bot=bot, seat=1, device="cuda:0")
    assert torch.equal(one.seat, torch.ones(L, dtype=torch.int32, device="cuda:0"))
    drawn, _ = bots.reset_seat(keys, game, bot=bot, seat="drawn", device="cuda:0")
    np.testing.assert_array_equal(drawn.seat.cpu().numpy(), Oracle(game).episode_seats(batch_initial(game, L, keys)))
    with pytest.raises(ModelError):
        bots.reset_seat(keys, game, bot=bot, seat=2, device="cuda:0")
    with pytest.raises(ModelError):
        bots.reset_seat(keys, game, bot=bot, seat=torch.full((L,), 3, dtype=torch.int32, device="cuda:0"),
                        device="cuda:0")
    with pytest.raises(ModelError):
        bots.SeatEnv(bot, scenario=game, seat="random", device="cuda:0")


def test_drawn_seat_on_the_pixel_surface():
    """The per-lane pick on images: each lane's learner image (at its drawn
    seat) against the oracle's renderer, across an episode end."""
    import torch

    from nanorts_amd import bots, rendering

    _say("drawn seat pixels")
    torch.cuda.set_device(0)
    game = _game()
    bot = bots.lightRushAI
    seat = bots.SeatEnv(bot, scenario=game, surface="pixels", seat="drawn", device="cuda:0")
    L = 12
    keys = roots(L, 41)
    obs, sst = seat.reset(keys)
    oracle = Oracle(game)
    ref = batch_initial(game, L, keys)
    carry = empty_carry(L, game.bucket.per_player_capacity)
    seats = oracle.episode_seats(ref)
    tiles = rendering.tile_table(game.bucket.unit_type_capacity)
    image, _ = oracle.pixels(ref, False, tiles)
    np.testing.assert_array_equal(obs[bots.LEARNER].image.cpu().numpy(), _at(image, seats))
    for t in range(HORIZON + 4):
        acts = np.ascontiguousarray(_at(oracle.sample_actions(oracle.avail_rows(ref), (43, 47), t), seats))
        oracle.seat_step(ref, carry, bot.strategy, bot.trained, seats, acts, False, observe=False, draw=True)
        obs, sst, _, _, _ = seat.step(None, sst, {bots.LEARNER: torch.as_tensor(acts, device="cuda:0")}, donate=True)
        if t % 8 == 0 or t >= HORIZON - 2:
            image, scalars = oracle.pixels(ref, False, tiles)
            np.testing.assert_array_equal(obs[bots.LEARNER].image.cpu().numpy(), _at(image, seats),
                                          err_msg=f"cycle {t}")
            np.testing.assert_array_equal(obs[bots.LEARNER].scalars.cpu().numpy(), _at(scalars, seats))
    np.testing.assert_array_equal(sst.seat.cpu().numpy(), seats)
