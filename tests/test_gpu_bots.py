"""GPU parity of the scripted bots and the learner-vs-bot seat against the C
oracle: the bot's Commands and carry after one act from many mid-game states,
and whole seat rollouts (learner = player 0 on seeded uniform-legal actions,
bot = player 1) cycle by cycle, bit for bit.
"""
from __future__ import annotations

import numpy as np
import pytest

from nanorts_amd.content import map_name_to_scenario
from nanorts_amd.model import ConflictStrategy, UnitTypeTableVersion
from oracle.oracle import Oracle, batch_initial, copy_state, empty_carry
from tests.helpers import assert_states_equal, roots, to_device, to_host

pytestmark = pytest.mark.gpu

WORKER_RUSH, BARRACKS_RUSH, LIGHT = 0, 1, 4

# (map, utt, strategy, max_cycles, partial, bot)
SEAT_CASES = {
    "16x16-workerrush": ("basesWorkers16x16", UnitTypeTableVersion.ORIGINAL_FINETUNED, ConflictStrategy.CANCEL_BOTH,
                         3000, False, WORKER_RUSH),
    "16x16-lightrush": ("basesWorkers16x16", UnitTypeTableVersion.ORIGINAL_FINETUNED, ConflictStrategy.CANCEL_BOTH,
                        3000, False, BARRACKS_RUSH),
    "8x8-lightrush-random-partial": ("basesWorkers8x8", UnitTypeTableVersion.ORIGINAL, ConflictStrategy.CANCEL_RANDOM,
                                     600, True, BARRACKS_RUSH),
    "barracks8x8-workerrush-alternating": ("basesWorkersBarracks8x8", UnitTypeTableVersion.ORIGINAL,
                                           ConflictStrategy.CANCEL_ALTERNATING, 500, False, WORKER_RUSH),
}


def _game(case):
    name, utt, strategy, max_cycles, partial, bot = SEAT_CASES[case]
    return map_name_to_scenario(name, utt=utt, conflict_strategy=strategy, max_cycles=max_cycles), partial, bot


def _carry_to_device(carry, device):
    import torch

    out = {k: torch.as_tensor(np.ascontiguousarray(v), device=device) for k, v in carry.items()}
    out["trained"] = out["trained"].to(torch.bool)
    return out


def _carry_to_host(carry):
    out = {k: v.cpu().numpy() for k, v in carry.items()}
    out["trained"] = out["trained"].astype(np.uint8)
    return out


def _assert_carry_equal(want, got, where):
    for name, w in want.items():
        np.testing.assert_array_equal(np.asarray(got[name]).astype(np.int64), w.astype(np.int64),
                                      err_msg=f"{where}: carry {name}")


def _learner_actions(o: Oracle, st, t: int):
    rows = o.avail_rows(st)
    return np.ascontiguousarray(o.sample_actions(rows, (41, 43), t)[:, 0])


def _seat_env(game, partial, bot):
    from nanorts_amd import bots

    return bots.SeatEnv(bots.workerRushAI if bot == WORKER_RUSH else bots.lightRushAI, scenario=game,
                        partial_observability=partial)


@pytest.mark.parametrize("case", list(SEAT_CASES))
def test_abstraction_act_from_mid_game_states(case):
    """One act of each bot for both seats from states and carries the oracle
    reached after seat rollouts of several lengths."""
    import torch

    from nanorts_amd import bots

    game, partial, bot = _game(case)
    o = Oracle(game)
    C = game.bucket.per_player_capacity
    L = 48
    st = batch_initial(game, L, roots(L, 5))
    carry = empty_carry(L, C)
    env = _seat_env(game, partial, bot).env
    checked = 0
    for t in range(260):
        if t % 40 == 0 or t < 3:
            for strategy in (WORKER_RUSH, BARRACKS_RUSH):
                for player in (0, 1):
                    want_carry = copy_state(carry)
                    want = o.abstraction_act(copy_state(st), want_carry, strategy, LIGHT, player)
                    dev = to_device(env, st)
                    got_carry = _carry_to_device(carry, env.device)
                    got = bots.abstraction_act(env, dev, got_carry, bots.Bot("probe", strategy, LIGHT), player)
                    where = f"{case} t={t} strategy={strategy} player={player}"
                    for name, w in want.items():
                        np.testing.assert_array_equal(got[name].cpu().numpy(), w, err_msg=f"{where}: {name}")
                    _assert_carry_equal(want_carry, _carry_to_host(got_carry), where)
                    assert_states_equal(st, to_host(dev), f"{where}: state untouched")
                    checked += 1
        o.seat_step(st, carry, bot, LIGHT, 0, _learner_actions(o, st, t), partial, observe=False)
    assert checked == 4 * 9
    torch.cuda.synchronize()


@pytest.mark.parametrize("case", list(SEAT_CASES))
def test_seat_rollout_matches_oracle(case):
    """SeatEnv.step against the oracle's step_seat for whole episodes: learner
    rewards, dones, winners and observations every cycle; the state and the
    bot's carry every 20 cycles and at the end."""
    import torch

    game, partial, bot = _game(case)
    o = Oracle(game)
    C = game.bucket.per_player_capacity
    L = 24
    steps = game.max_cycles + 20
    st = batch_initial(game, L, roots(L, 9))
    carry = empty_carry(L, C)
    seat = _seat_env(game, partial, bot)
    obs, sst = seat.reset(torch.as_tensor(st["environment_root"].view(np.int32)))
    fresh = to_host(sst.environment_state)
    for name, w in st.items():
        np.testing.assert_array_equal(fresh[name].reshape(L, -1), w.reshape(L, -1), err_msg=f"reset {name}")
    # continue from the oracle's leaf shapes (scalar leaves [L, 1])
    from nanorts_amd.bots import SeatState

    sst = SeatState(to_device(seat.env, st), sst.carry, sst.seat)
    ended = 0
    for t in range(steps):
        actions = _learner_actions(o, st, t)
        want = o.seat_step(st, carry, bot, LIGHT, 0, actions, partial)
        obs, sst, rewards, dones, infos = seat.step(None, sst, {"learner": torch.as_tensor(actions, device=seat.device)},
                                                    donate=True)
        where = f"{case} cycle {t}"
        np.testing.assert_array_equal(rewards["learner"].cpu().numpy(), want["reward"][:, 0], err_msg=where)
        np.testing.assert_array_equal(dones["__all__"].cpu().numpy(), want["done"].astype(bool), err_msg=where)
        np.testing.assert_array_equal(infos["winner"].cpu().numpy(), want["winner"], err_msg=where)
        np.testing.assert_array_equal(obs["learner"].feature_maps.cpu().numpy(), want["feature_maps"][:, 0],
                                      err_msg=where)
        np.testing.assert_array_equal(obs["learner"].scalars.cpu().numpy(), want["scalars"][:, 0], err_msg=where)
        ended += int(want["done"].sum())
        if t % 20 == 0 or t == steps - 1:
            assert_states_equal(st, to_host(sst.environment_state), where)
            _assert_carry_equal(carry, _carry_to_host(sst.carry), where)
    assert ended >= L  # every env finished at least one episode


def _first_pass(monkeypatch, mode: str) -> None:
    """The seat rollout's first pass: "auto" (two games per wave on the slot
    window where that holds more games per CU) or "lean" (one pass, one game
    per wave on the full block)."""
    if mode == "auto":
        monkeypatch.delenv("NANORTS_AMD_FIRST_PASS", raising=False)
    else:
        monkeypatch.setenv("NANORTS_AMD_FIRST_PASS", mode)


def _poison_allocator(nbytes: int) -> None:
    """A sentinel in the next allocations' memory (see test_gpu_parity)."""
    import torch

    junk = torch.full((nbytes // 4,), 0x4D4D4D4D, dtype=torch.int32, device="cuda")
    torch.cuda.synchronize()
    del junk


@pytest.mark.parametrize("case", list(SEAT_CASES))
@pytest.mark.parametrize("first_pass", ["auto", "lean"])
def test_fused_seat_rollout_matches_oracle(case, first_pass, monkeypatch):
    """The fused seat rollout (learner sampled in the kernel) over whole
    episodes against the oracle's seat steps on the same sampler: per-cycle
    rewards and dones, the learner's recorded actions, the last observation,
    the final state and carry, with each first pass."""
    import torch

    from nanorts_amd.bots import SeatState

    _first_pass(monkeypatch, first_pass)
    game, partial, bot = _game(case)
    o = Oracle(game)
    C = game.bucket.per_player_capacity
    L = 32
    steps = game.max_cycles + 40
    st = batch_initial(game, L, roots(L, 13))
    carry = empty_carry(L, C)
    seat = _seat_env(game, partial, bot)
    sst = SeatState(to_device(seat.env, st), _carry_to_device(carry, seat.device),
                    torch.zeros(L, dtype=torch.int32, device=seat.device))
    key = (41, 43)
    _poison_allocator(steps * L * C * 7 * 4 + (64 << 20))
    got = seat.rollout(sst, steps, key, record_actions=True)
    rewards, dones, actions = (got[k].cpu().numpy() for k in ("rewards", "dones", "actions"))
    for t in range(steps):
        want_actions = _learner_actions(o, st, t)
        np.testing.assert_array_equal(actions[t], want_actions, err_msg=f"{case} actions at cycle {t}")
        want = o.seat_step(st, carry, bot, LIGHT, 0, want_actions, partial, observe=t == steps - 1)
        np.testing.assert_array_equal(rewards[t], want["reward"], err_msg=f"{case} cycle {t}")
        np.testing.assert_array_equal(dones[t], want["done"].astype(bool), err_msg=f"{case} cycle {t}")
    assert_states_equal(st, to_host(sst.environment_state), f"{case} final state")
    _assert_carry_equal(carry, _carry_to_host(sst.carry), f"{case} final carry")
    np.testing.assert_array_equal(got["feature_maps"][0].cpu().numpy(), want["feature_maps"])
    np.testing.assert_array_equal(got["scalars"][0].cpu().numpy(), want["scalars"])


@pytest.mark.parametrize("bot", [WORKER_RUSH, BARRACKS_RUSH])
def test_seat_two_pass_hands_games_to_the_second_pass(bot):
    """The seat rollout's first pass (two games per wave on a 32-slot window
    of each player's 70 slots) runs a game until a unit could spawn past its
    window, or a cycle leaves the one-team path; the second pass runs the rest
    with the carry the first stored.  Learner games (player 0) that start with
    22..38 live slots, the added Workers all the learner's and 200 resources
    each, cross at cycle 0, part-way through the launch, or never, and match
    the oracle's seat steps cycle by cycle, with the final state and carry."""
    import torch

    from nanorts_amd.bots import SeatState
    from tests.test_gpu_parity import _packed

    game = map_name_to_scenario("basesWorkers16x16", conflict_strategy="CANCEL_RANDOM", max_cycles=3000)
    partial = True
    base = int((_packed(game, [0])["birth"][0] != -1).sum())
    st = _packed(game, [22 - base + k for k in range(17)], alternate=False)
    st["player_resources"][:] = 200
    o = Oracle(game)
    assert (o.violations(st) == 0).all()
    L, C, steps = st["birth"].shape[0], game.bucket.per_player_capacity, 128
    carry = empty_carry(L, C)
    seat = _seat_env(game, partial, bot)
    sst = SeatState(to_device(seat.env, st), _carry_to_device(carry, seat.device),
                    torch.zeros(L, dtype=torch.int32, device=seat.device))
    key = (41, 43)
    got = seat.rollout(sst, steps, key, record_actions=True)
    first = got["first_pass_cycles"].cpu().numpy()
    print("first-pass cycles per game:", first.tolist(), flush=True)
    assert (first == 0).any()
    assert ((first > 0) & (first < steps)).any()
    assert (first == steps).any()
    rewards, dones, actions = (got[k].cpu().numpy() for k in ("rewards", "dones", "actions"))
    for t in range(steps):
        want_actions = _learner_actions(o, st, t)
        np.testing.assert_array_equal(actions[t], want_actions, err_msg=f"actions at cycle {t}")
        want = o.seat_step(st, carry, bot, LIGHT, 0, want_actions, partial, observe=t == steps - 1)
        np.testing.assert_array_equal(rewards[t], want["reward"], err_msg=f"cycle {t}")
        np.testing.assert_array_equal(dones[t], want["done"].astype(bool), err_msg=f"cycle {t}")
    assert_states_equal(st, to_host(sst.environment_state), "final state")
    _assert_carry_equal(carry, _carry_to_host(sst.carry), "final carry")
    np.testing.assert_array_equal(got["feature_maps"][0].cpu().numpy(), want["feature_maps"])
