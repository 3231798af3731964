"""GPU parity of the multi-group step and the group mix.

step_groups runs core.step for six groups (two maps of one bucket, three
horizons, per-lane and broadcast keys) in one call, which the library splits
into two launches; every group's state and outputs are compared bit for bit
with the oracle's core.step of that group alone.  GroupMix publishes a
facade group and two learner-vs-bot groups (one under the drawn seat rule)
agent-major; its rows are compared with each environment stepped on its own.
"""
from __future__ import annotations

import sys

import numpy as np
import pytest

from oracle.oracle import Oracle, batch_initial
from tests.helpers import assert_states_equal, roots, to_device, to_host

pytestmark = pytest.mark.gpu

FIELDS = ("kind", "direction", "none_duration", "target_cell", "produced_type", "request_order")


def _say(*parts):
    print(*parts, flush=True)
    sys.stdout.flush()


def _games():
    from nanorts_amd.content import map_name_to_scenario

    plain = map_name_to_scenario("basesWorkers8x8", conflict_strategy="CANCEL_RANDOM")
    walls = map_name_to_scenario("basesWorkers8x8Obstacle", conflict_strategy="CANCEL_RANDOM", max_cycles=150)
    short = map_name_to_scenario("basesWorkers8x8", conflict_strategy="CANCEL_RANDOM", max_cycles=130)
    return plain, walls, short


def test_step_groups_matches_each_group_alone(oracle_threads):
    import torch

    import nanorts_amd
    from nanorts_amd import groups

    _say("step_groups: six groups, two launches")
    torch.cuda.set_device(0)
    plain, walls, short = _games()
    plan = [(plain, 24, True), (walls, 40, False), (short, 5, True), (walls, 1, True), (plain, 64, False),
            (short, 17, True)]
    assert groups.steps_together([g for g, _, _ in plan])
    rng = np.random.default_rng(3)
    requests, expected = [], []
    for i, (game, L, per_lane) in enumerate(plan):
        oracle = Oracle(game)
        st = batch_initial(game, L, roots(L, 50 + i))
        # one cycle short of the horizon where there is a short one, so the
        # step truncates the games still running
        advance = game.max_cycles - 1 if game.max_cycles < 1000 else 140
        oracle.rollout(st, (i, i + 1), 0, advance, False, threads=oracle_threads, record=False)
        cmds = oracle.decode_actions(st, oracle.sample_actions(oracle.avail_rows(st), (9, i), 3))
        keys = rng.integers(0, 2**32, size=(L if per_lane else 1, 2), dtype=np.uint64).astype(np.uint32)
        env = nanorts_amd.make("NanoRTS", scenario=game, device="cuda:0")
        dev_state = to_device(env, st)
        requests.append((keys, dev_state, {f: torch.as_tensor(cmds[f], device="cuda:0") for f in FIELDS}, env))
        want = oracle.core_step(st, cmds, np.ascontiguousarray(np.broadcast_to(keys, (L, 2))))
        expected.append((st, want))
    outs = groups.step_groups(requests)
    for i, ((st, want), (_, dev_state, _, _), out) in enumerate(zip(expected, requests, outs)):
        assert_states_equal(st, to_host(dev_state), f"group {i}")
        for name in ("terminated", "truncated"):
            np.testing.assert_array_equal(out[name].cpu().numpy(), want[name].astype(bool), err_msg=f"{i} {name}")
        for name in ("reward", "admitted_harvest", "admitted_return", "admitted_produce", "admitted_attack"):
            np.testing.assert_array_equal(out[name].cpu().numpy(), want[name], err_msg=f"{i} {name}")
    assert any(w["truncated"].any() for _, w in expected)


def test_group_mix_publishes_each_group_agent_major():
    import torch

    import nanorts_amd
    from nanorts_amd import bots
    from nanorts_amd.groups import Group, GroupMix
    from nanorts_amd.model import ModelError

    _say("GroupMix: facade + WorkerRush seat + LightRush seat")
    torch.cuda.set_device(0)
    plain, _, _ = _games()
    both = nanorts_amd.make("NanoRTS", scenario=plain, device="cuda:0")
    worker = bots.SeatEnv(bots.workerRushAI, scenario=plain, device="cuda:0")
    light = bots.SeatEnv(bots.lightRushAI, scenario=plain, seat="drawn", device="cuda:0")
    lanes = (8, 6, 5)
    envs = (both, worker, light)
    mix = GroupMix([Group(env, n) for env, n in zip(envs, lanes)])
    assert mix.lanes == 19 and mix.rows == 27
    # one bucket, every environment with a split step: one core.step launch
    # per cycle, checked below against each environment's own fused step
    assert mix.shared_launches() == [[0, 1, 2]]
    assert [(s.start, s.stop) for s in mix.slices()] == [(0, 16), (16, 22), (22, 27)]
    with pytest.raises(ModelError):
        GroupMix([])
    with pytest.raises(ModelError):
        GroupMix([Group(both, 0)])
    with pytest.raises(ModelError):
        GroupMix([Group(both, 2), Group(nanorts_amd.make("NanoRTS", scenario=plain, final_observation=False,
                                                         device="cuda:0"), 2)])
    keys = roots(19, 7)
    obs, states = mix.reset(keys)
    starts = np.cumsum((0,) + lanes)
    alone = []
    for env, a, b in zip(envs, starts[:-1], starts[1:]):
        o, s = env.reset(keys[a:b])
        alone.append(s)
        agents = list(env.agents)
        got = obs.feature_maps[mix.slices()[envs.index(env)]]
        want = torch.cat([o[agent].feature_maps for agent in agents])
        assert torch.equal(got, want)
    oracle = Oracle(plain)
    for t in range(12):
        rows = mix.get_avail_actions(states).cpu().numpy()
        padded = np.concatenate([rows, np.zeros((1,) + rows.shape[1:], bool)])
        sampled = oracle.sample_actions(padded.reshape(14, 2, *rows.shape[1:]), (4, 5), t).reshape(28, -1, 7)[:27]
        actions = torch.as_tensor(np.ascontiguousarray(sampled), device="cuda:0")
        mobs, states, mrew, mdone, minfo = mix.step(None, states, actions)
        for i, env in enumerate(envs):
            bound = mix.slices()[i]
            agents = list(env.agents)
            per_agent = dict(zip(agents, torch.split(actions[bound], lanes[i])))
            o, alone[i], r, d, info = env.step(None, alone[i], per_agent)
            assert torch.equal(mobs.feature_maps[bound], torch.cat([o[a].feature_maps for a in agents]))
            assert torch.equal(mobs.scalars[bound], torch.cat([o[a].scalars for a in agents]))
            assert torch.equal(mrew[bound], torch.cat([r[a] for a in agents]))
            assert torch.equal(mdone[bound], torch.cat([d[a] for a in agents]))
            assert torch.equal(minfo["winner"][bound], torch.cat([info["winner"]] * len(agents)))
            assert torch.equal(minfo["final_observation"].feature_maps[bound],
                               torch.cat([info["final_observation"][a].feature_maps for a in agents]))
        cells = mix.get_slot_cells(states)
        assert cells.shape[0] == 27
