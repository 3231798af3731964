"""GPU parity of the GridNet surface against the C oracle and closed forms.

decode_actions is compared bit for bit with the oracle's GridNet decode on
mid-game states under per-cell actions that collide (legal rows at unit
cells, random in-range rows elsewhere, and wild out-of-range values).  The
observation is compared with its closed form: the one-hot (or index) of the
oracle's full-observation feature maps clipped to the plane widths, the
source mask of available own units, and the oracle's legality row at every
source cell.  Whole GridNet steps (and step_against a given player 1) are
compared cycle by cycle with the oracle's decode -> core.step keyed by the
episode root, the reward components and reward dones restated from the
step's events and ending state, the ending state's planes, auto-reset and
the next observation.
"""
from __future__ import annotations

import ctypes
import sys

import numpy as np
import pytest

from nanorts_amd.model import (TYPE_BARRACKS, TYPE_BASE, TYPE_HEAVY, TYPE_LIGHT, TYPE_RANGED, TYPE_WORKER)
from oracle.oracle import copy_state, load_library
from tests.helpers import advanced_states, assert_states_equal, game_for, roots, to_device, to_host

pytestmark = pytest.mark.gpu

SIZES = (6, 4, 4, 4, 4, 7, 49)
WIDTHS = np.asarray((5, 5, 3, 8, 6, 2))
OFFSETS = np.asarray((0, 5, 10, 13, 21, 27))
FIELDS = ("kind", "direction", "none_duration", "target_cell", "produced_type", "request_order")


def _say(*parts):
    print(*parts, flush=True)
    sys.stdout.flush()


def _per_cell_actions(game, oracle, st, seed: int, wild: bool = False) -> np.ndarray:
    """[L][2][cells][7]: random in-range rows everywhere (wild: any values),
    and at 70% of the unit cells the unit's uniform-legal JaxMARL row."""
    b = game.bucket
    L, N, C, cells = st["time"].shape[0], b.neutral_capacity, b.per_player_capacity, b.cell_count
    rng = np.random.default_rng(seed)
    if wild:
        acts = rng.integers(-70, 70, size=(L, 2, cells, 7), dtype=np.int32)
    else:
        acts = np.stack([rng.integers(0, s, size=(L, 2, cells), dtype=np.int32) for s in SIZES], -1)
    legal = oracle.sample_actions(oracle.avail_rows(st), (seed, seed + 3), 0)
    keep = rng.random((L, 2, C)) < 0.7
    for l in range(L):
        for p in range(2):
            for i in range(C):
                s = N + p * C + i
                if st["birth"][l, s] != -1 and keep[l, p, i]:
                    acts[l, p, st["cell"][l, s]] = legal[l, p, i]
    return acts


def _episode_roots(st) -> np.ndarray:
    lib = load_library()
    roots = st["environment_root"].reshape(-1, 2)
    out = np.zeros_like(roots, dtype=np.uint32)
    for l in range(roots.shape[0]):
        k = (ctypes.c_uint32 * 2)(int(roots[l, 0]), int(roots[l, 1]))
        o = (ctypes.c_uint32 * 2)()
        lib.nro_fold_in(k, ctypes.c_uint32(int(st["episode_index"][l])), o)
        out[l] = (o[0], o[1])
    return out


def _want_planes(oracle, st, form: str) -> np.ndarray:
    maps = oracle.symbolic(st, False)[0].astype(np.int64)  # [L][2][H][W][6]
    clipped = np.minimum(maps, WIDTHS - 1)
    if form == "indices":
        return clipped.astype(np.int8)
    hot = np.zeros(maps.shape[:-1] + (29,), np.int64)
    for f in range(6):
        np.put_along_axis(hot, (OFFSETS[f] + clipped[..., f])[..., None], 1, axis=-1)
    return hot


def _want_masks(game, oracle, st) -> tuple[np.ndarray, np.ndarray]:
    b = game.bucket
    L, N, C, H, W = st["time"].shape[0], b.neutral_capacity, b.per_player_capacity, b.height, b.width
    slot = st["entity_at"].reshape(L, H * W).astype(np.int64)
    occupied = slot >= 0
    s = np.clip(slot, 0, b.entity_capacity - 1)
    owner = np.where(occupied, np.take_along_axis(st["owner"].astype(np.int64), s, 1), -1)
    pending = np.take_along_axis(st["pending_kind"].astype(np.int64), s, 1)
    available = occupied & (owner >= 0) & (pending == -1)
    source = np.stack([available & (owner == p) for p in range(2)], 1)  # [L][2][cells]
    rows = oracle.legality_rows(st).reshape(L, 2 * C, 78)
    index = np.clip(slot - N, 0, 2 * C - 1)
    at = np.take_along_axis(rows, index[..., None], 1)  # [L][cells][78]
    mask = source[..., None] & at[:, None]
    return source.reshape(L, 2, H, W), mask.reshape(L, 2, H, W, 78)


def _pack(mask: np.ndarray) -> np.ndarray:
    bits = mask.astype(np.uint64)
    words = np.zeros(mask.shape[:-1] + (3,), np.uint64)
    for lo, hi, w in ((0, 29, 0), (29, 61, 1), (61, 78, 2)):
        words[..., w] = (bits[..., lo:hi] << np.arange(hi - lo, dtype=np.uint64)).sum(-1)
    return words.astype(np.uint32)


def _want_rewards(game, oracle_step_out, nxt, done) -> tuple[np.ndarray, np.ndarray]:
    """encode_rewards (src/nanorts/adapters/rewards.py:30-71) from the step's
    events and ending state."""
    L = done.shape[0]
    h, r = oracle_step_out["admitted_harvest"], oracle_step_out["admitted_return"]
    prod, att = oracle_step_out["admitted_produce"], oracle_step_out["admitted_attack"]
    comps = np.zeros((L, 2, 6), np.float32)
    for p in range(2):
        o = 1 - p
        over = nxt["game_over"].astype(bool)
        comps[:, p, 0] = np.where(over, np.where(nxt["winner"] == p, 1.0, -1.0), 0.0)
        comps[:, p, 1] = h[:, p] + r[:, p]
        comps[:, p, 2] = prod[:, p, TYPE_WORKER]
        comps[:, p, 3] = prod[:, p, TYPE_BASE] + prod[:, p, TYPE_BARRACKS]
        comps[:, p, 4] = att[:, p, o + 1] - att[:, p, p + 1]
        comps[:, p, 5] = prod[:, p, TYPE_LIGHT] + prod[:, p, TYPE_HEAVY] + prod[:, p, TYPE_RANGED]
    is_resource = np.asarray(game.columns["is_resource"]).astype(bool)
    types = np.clip(nxt["unit_type"].astype(np.int64), 0, game.bucket.unit_type_capacity - 1)
    stacked = ((nxt["birth"] != -1) & is_resource[types] & (nxt["carried_resources"] > 0)).any(1)
    dones = np.zeros((L, 2, 6), bool)
    dones[:, :, 0] = done[:, None]
    dones[:, :, 1] = ~stacked[:, None]
    return comps, dones


ODD_MAP = """<rts.PhysicalGameState width="9" height="7">
  <terrain>000000000000000000000100000000100000000000000000000000000000000</terrain>
  <players>
    <rts.Player ID="0" resources="8"></rts.Player>
    <rts.Player ID="1" resources="8"></rts.Player>
  </players>
  <units>
    <rts.units.Unit type="Resource" ID="1" player="-1" x="0" y="0" resources="20" hitpoints="1"></rts.units.Unit>
    <rts.units.Unit type="Resource" ID="2" player="-1" x="8" y="6" resources="20" hitpoints="1"></rts.units.Unit>
    <rts.units.Unit type="Base" ID="3" player="0" x="2" y="1" resources="0" hitpoints="10"></rts.units.Unit>
    <rts.units.Unit type="Base" ID="4" player="1" x="6" y="5" resources="0" hitpoints="10"></rts.units.Unit>
    <rts.units.Unit type="Worker" ID="5" player="0" x="1" y="1" resources="0" hitpoints="1"></rts.units.Unit>
    <rts.units.Unit type="Worker" ID="6" player="1" x="7" y="5" resources="0" hitpoints="1"></rts.units.Unit>
  </units>
</rts.PhysicalGameState>
"""


def _game(case):
    """The named case, or "odd-9x7": a 63-cell map, so rows of the second
    player and the last chunk start at odd cells (the writers' element path)."""
    if case != "odd-9x7":
        return game_for(case)
    import tempfile
    from pathlib import Path

    from nanorts_amd.content import load_game
    from nanorts_amd.model import ConflictStrategy

    path = Path(tempfile.mkdtemp(prefix="nr_map_")) / "odd9x7.xml"
    path.write_text(ODD_MAP)
    return load_game(path, conflict_strategy=ConflictStrategy.CANCEL_RANDOM, max_cycles=200), False


def _surface(game, **kw):
    import torch

    from nanorts_amd import gridnet

    torch.cuda.set_device(0)
    return gridnet.GridNet(game, gridnet.prepare(game, **kw), device="cuda:0")


@pytest.mark.parametrize("case", ["16x16-finetuned-both", "8x8-original-both", "barracks-random", "gow-alternating"])
@pytest.mark.parametrize("wild", [False, True])
def test_decode_matches_oracle(case, wild, oracle_threads):
    import torch

    _say(f"gridnet decode {case} wild={wild}")
    game, partial = game_for(case)
    L = 16 if case == "gow-alternating" else 96
    oracle, st = advanced_states(game, L, 150, partial, oracle_threads, seed=23)
    acts = _per_cell_actions(game, oracle, st, 5, wild)
    want = oracle.gridnet_decode(st, acts)
    g = _surface(game)
    b = game.bucket
    got = g.decode_actions(torch.as_tensor(acts.reshape(L, 2, b.height, b.width, 7), device="cuda:0"),
                           to_device(g, st))
    for f in FIELDS:
        np.testing.assert_array_equal(got[f].cpu().numpy(), want[f], err_msg=f"{case}: {f}")


@pytest.mark.parametrize("index", range(4))
def test_decode_seeds_player_one_with_player_zeros_issued_usage(index, oracle_threads):
    """The hand-built states of tests/test_gridnet_oracle.py (player 0's kept,
    legal claim on a cell drops player 1's claim on it; an illegal or dropped
    one does not) through the GPU's decode, against the commands traced by
    hand and the oracle's."""
    import torch

    from oracle.oracle import Oracle
    from tests.test_gridnet_oracle import picks, seeding_cases

    name, game, st, acts, want = seeding_cases()[index]
    _say(f"gridnet decode, issued usage: {name}")
    g = _surface(game)
    b = game.bucket
    got = g.decode_actions(torch.as_tensor(acts.reshape(1, 2, b.height, b.width, 7), device="cuda:0"),
                           to_device(g, st))
    got = {f: got[f].cpu().numpy() for f in FIELDS}
    assert picks(got, want) == want, name
    ref = Oracle(game).gridnet_decode(st, acts)
    for f in FIELDS:
        np.testing.assert_array_equal(got[f], ref[f], err_msg=f"{name}: {f}")


@pytest.mark.parametrize("case", ["16x16-finetuned-both", "barracks-random", "melee-both", "odd-9x7"])
@pytest.mark.parametrize("form", [("one_hot", "int32", "rows", "int32"), ("one_hot", "uint8", "rows", "bool"),
                                  ("one_hot", "bool", "packed", "int32"), ("indices", "int32", "rows", "uint8")])
def test_observe_matches_closed_form(case, form, oracle_threads):
    import torch

    from nanorts_amd import gridnet

    _say(f"gridnet observe {case} {form}")
    planes_form, planes_dtype, mask_form, mask_dtype = form
    game, partial = _game(case)
    oracle, st = advanced_states(game, 64, 120, partial, oracle_threads, seed=29)
    g = _surface(game, planes_form=planes_form, planes_dtype=getattr(torch, planes_dtype), mask_form=mask_form,
                 mask_dtype=getattr(torch, mask_dtype))
    obs = g.observe(to_device(g, st))
    want_planes = _want_planes(oracle, st, planes_form)
    got_planes = obs.planes.cpu().numpy()
    assert got_planes.dtype == (np.int8 if planes_form == "indices" else np.dtype(planes_dtype))
    np.testing.assert_array_equal(got_planes.astype(np.int64).reshape(want_planes.shape), want_planes)
    source, mask = _want_masks(game, oracle, st)
    np.testing.assert_array_equal(obs.source_mask.cpu().numpy(), source)
    if mask_form == "packed":
        np.testing.assert_array_equal(obs.action_mask.cpu().numpy().view(np.uint32), _pack(mask))
    else:
        np.testing.assert_array_equal(obs.action_mask.cpu().numpy().astype(bool), mask)
    np.testing.assert_array_equal(gridnet.unpack_mask(obs.action_mask, layout=g.layout).cpu().numpy(), mask)
    np.testing.assert_array_equal(g.planes(to_device(g, st)).cpu().numpy(), got_planes)


def _check_step(game, oracle, g, st, out, acts_cells, against=None):
    """One oracle GridNet step on `st` (in place) checked against the kernel's `out`."""
    b = game.bucket
    L = st["time"].shape[0]
    if against is None:
        cmds = oracle.gridnet_decode(st, acts_cells)
    else:
        both = np.zeros((L, 2, b.cell_count, 7), np.int32)
        both[:, 0] = acts_cells
        cmds = oracle.gridnet_decode(st, both)
        for f in FIELDS:
            cmds[f][:, 1] = against[f][:, 1]
    step = oracle.core_step(st, cmds, _episode_roots(st))
    done = (step["terminated"] | step["truncated"]).astype(bool)
    comps, rdones = _want_rewards(game, step, st, done)
    np.testing.assert_array_equal(out.reward_components.cpu().numpy(), comps)
    np.testing.assert_array_equal(out.reward_dones.cpu().numpy(), rdones)
    np.testing.assert_array_equal(out.terminated.cpu().numpy(), step["terminated"].astype(bool))
    np.testing.assert_array_equal(out.truncated.cpu().numpy(), step["truncated"].astype(bool))
    np.testing.assert_array_equal(out.done.cpu().numpy(), done)
    np.testing.assert_array_equal(out.winner.cpu().numpy(), st["winner"])
    np.testing.assert_array_equal(out.spawn_overflowed.cpu().numpy(), (st["spawn_overflow"] > 0).any(1))
    want_final = _want_planes(oracle, st, g.layout.planes_form)
    np.testing.assert_array_equal(out.final_observation.cpu().numpy().astype(np.int64).reshape(want_final.shape),
                                  want_final)
    oracle.reset_where_done(st, done.astype(np.uint8))
    assert_states_equal(st, to_host(out.environment_state))
    want_planes = _want_planes(oracle, st, g.layout.planes_form)
    np.testing.assert_array_equal(out.observation.planes.cpu().numpy().astype(np.int64).reshape(want_planes.shape),
                                  want_planes)
    source, mask = _want_masks(game, oracle, st)
    np.testing.assert_array_equal(out.observation.source_mask.cpu().numpy(), source)
    np.testing.assert_array_equal(out.observation.action_mask.cpu().numpy().astype(bool), mask)
    return done


@pytest.mark.parametrize("case", ["16x16-alternating", "barracks-random", "8x8-original-both", "odd-9x7"])
def test_steps_match_oracle(case, oracle_threads):
    import torch

    _say(f"gridnet step {case}")
    game, partial = _game(case)
    b = game.bucket
    L = 48
    # near the time limit for the short cases, so episodes end and reset
    advance = {"16x16-alternating": 280, "barracks-random": 130, "8x8-original-both": 200, "odd-9x7": 180}[case]
    oracle, st = advanced_states(game, L, advance, partial, oracle_threads, seed=31)
    g = _surface(game)
    state = to_device(g, st)
    ended = 0
    for t in range(30):
        acts = _per_cell_actions(game, oracle, st, 100 + t)
        out = g.step(state, torch.as_tensor(acts.reshape(L, 2, b.height, b.width, 7), device="cuda:0"), donate=True)
        ended += int(_check_step(game, oracle, g, st, out, acts).sum())
        state = out.environment_state
    if case not in ("8x8-original-both", "odd-9x7"):
        assert ended > 0


@pytest.mark.parametrize("case", ["16x16-finetuned-both", "barracks-random"])
def test_step_against_matches_oracle(case, oracle_threads):
    import torch

    _say(f"gridnet step_against {case}")
    game, partial = game_for(case)
    b = game.bucket
    L = 48
    oracle, st = advanced_states(game, L, 120, partial, oracle_threads, seed=37)
    g = _surface(game)
    state = to_device(g, st)
    for t in range(20):
        acts = _per_cell_actions(game, oracle, st, 200 + t)[:, 0]
        given = oracle.decode_actions(st, oracle.sample_actions(oracle.avail_rows(st), (7, 9), t))
        gt = {f: torch.as_tensor(given[f], device="cuda:0") for f in FIELDS}
        out = g.step_against(state, torch.as_tensor(acts.reshape(L, b.height, b.width, 7), device="cuda:0"), gt,
                             donate=True)
        _check_step(game, oracle, g, st, out, acts, against=given)
        state = out.environment_state


@pytest.mark.parametrize("case", ["16x16-finetuned-both", "barracks-random"])
def test_sampler_matches_oracle(case, oracle_threads):
    _say(f"gridnet sampler {case}")
    game, partial = game_for(case)
    oracle, st = advanced_states(game, 64, 150, partial, oracle_threads, seed=47)
    g = _surface(game, mask_form="packed")
    obs = g.observe(to_device(g, st))
    got = g.sample_actions(obs.action_mask, (21, 22), 9, env0=3).cpu().numpy()
    _, mask = _want_masks(game, oracle, st)
    want = oracle.gridnet_sample_actions(mask, (21, 22), 9, env0=3)
    np.testing.assert_array_equal(got.reshape(want.shape), want)


def test_reset_observes_the_initial_state(oracle_threads):
    from nanorts_amd import gridnet  # noqa: F401

    _say("gridnet reset")
    game, _ = game_for("16x16-finetuned-both")
    oracle, st = advanced_states(game, 8, 0, False, oracle_threads, seed=41)
    g = _surface(game)
    state, obs = g.reset(st["environment_root"])
    got = to_host(state)
    for name, want in st.items():
        assert got[name].shape == want.shape, name
    assert_states_equal(copy_state(st), got)
    np.testing.assert_array_equal(obs.planes.cpu().numpy(), _want_planes(oracle, st, "one_hot"))


@pytest.mark.parametrize("bot_name", ["workerRushAI", "lightRushAI"])
def test_gridnet_seat_matches_oracle(bot_name, oracle_threads):
    """step_gridnet_seat: the bot's act (player 1) on its carry, step_against
    with the learner's per-cell rows, the carry emptied where the game ended."""
    import torch

    from nanorts_amd import bots, gridnet
    from oracle.oracle import empty_carry

    _say(f"gridnet seat {bot_name}")
    torch.cuda.set_device(0)
    from nanorts_amd.content import map_name_to_scenario

    # a horizon inside the 80 cycles, so every game ends (and resets) once
    game = map_name_to_scenario("basesWorkers8x8", max_cycles=60)
    bot = getattr(bots, bot_name)
    L = 24
    oracle, st = advanced_states(game, L, 0, False, oracle_threads, seed=53)
    seat = gridnet.GridNetSeat(bot, game, device="cuda:0")
    state, obs = seat.reset(st["environment_root"])
    carry = empty_carry(L, game.bucket.per_player_capacity)
    b = game.bucket
    ended = 0
    for t in range(80):
        learner = _per_cell_actions(game, oracle, st, 300 + t)[:, 0]
        out = seat.step(state, torch.as_tensor(learner.reshape(L, b.height, b.width, 7), device="cuda:0"),
                        donate=True)
        state = out.seat_state
        bot_cmds = oracle.abstraction_act(st, carry, bot.strategy, bot.trained, 1)
        both = np.zeros((L, 2, b.cell_count, 7), np.int32)
        both[:, 0] = learner
        cmds = oracle.gridnet_decode(st, both)
        for f in FIELDS:
            cmds[f][:, 1] = bot_cmds[f][:, 1]
        step = oracle.core_step(st, cmds, _episode_roots(st))
        done = (step["terminated"] | step["truncated"]).astype(bool)
        comps, rdones = _want_rewards(game, step, st, done)
        np.testing.assert_array_equal(out.reward_components.cpu().numpy(), comps[:, 0], err_msg=f"cycle {t}")
        np.testing.assert_array_equal(out.reward_dones.cpu().numpy(), rdones[:, 0])
        np.testing.assert_array_equal(out.done.cpu().numpy(), done)
        want_final = _want_planes(oracle, st, "one_hot")[:, 0]
        np.testing.assert_array_equal(out.final_observation.cpu().numpy().astype(np.int64), want_final)
        oracle.reset_where_done(st, done.astype(np.uint8))
        for name in carry:
            if name != "next_order":
                carry[name][done] = -1 if name != "trained" else 0
        carry["next_order"][done] = 0
        assert_states_equal(st, to_host(state.environment_state), f"cycle {t}")
        for name, want in carry.items():
            np.testing.assert_array_equal(state.carry[name].cpu().numpy().astype(np.int64), want.astype(np.int64),
                                          err_msg=f"cycle {t} carry {name}")
        ended += int(done.sum())
    assert ended > 0


def test_gridnet_mix_rows(oracle_threads):
    """GridNetMix: self-play rows (game-major, two per game) then the seat
    groups' rows, each equal to its environment stepped on its own."""
    import torch

    from nanorts_amd import bots, gridnet

    _say("gridnet mix")
    torch.cuda.set_device(0)
    game, _ = game_for("8x8-original-both")
    b = game.bucket
    mix = gridnet.GridNetMix(4, [gridnet.GridNetGroup(bots.workerRushAI, 3), gridnet.GridNetGroup(bots.lightRushAI, 2)],
                             game, device="cuda:0")
    assert mix.lanes == 9 and mix.rows == 13
    assert [(s.start, s.stop) for s in mix.slices()] == [(0, 8), (8, 11), (11, 13)]
    keys = roots(9, 61)
    mstate, mobs = mix.reset(keys)
    alone_self, _ = gridnet.GridNet(game, mix.grid.layout, device="cuda:0").reset(keys[:4])
    solo = gridnet.GridNet(game, mix.grid.layout, device="cuda:0")
    seat_w = gridnet.GridNetSeat(bots.workerRushAI, game, mix.grid.layout, device="cuda:0")
    seat_l = gridnet.GridNetSeat(bots.lightRushAI, game, mix.grid.layout, device="cuda:0")
    sw, _ = seat_w.reset(keys[4:7])
    sl, _ = seat_l.reset(keys[7:9])
    rng = np.random.default_rng(9)
    for t in range(60):
        acts = np.stack([rng.integers(0, s, size=(13, b.height, b.width), dtype=np.int32)
                         for s in (6, 4, 4, 4, 4, 7, 49)], -1)
        a = torch.as_tensor(acts, device="cuda:0")
        m = mix.step(mstate, a)
        mstate = m.mix_state
        o = solo.step(alone_self, a[:8].reshape(4, 2, b.height, b.width, 7))
        alone_self = o.environment_state
        ow = seat_w.step(sw, a[8:11])
        sw = ow.seat_state
        ol = seat_l.step(sl, a[11:13])
        sl = ol.seat_state
        assert torch.equal(m.observation.planes[:8], o.observation.planes.reshape(8, *o.observation.planes.shape[2:]))
        assert torch.equal(m.observation.planes[8:11], ow.observation.planes)
        assert torch.equal(m.observation.action_mask[11:13], ol.observation.action_mask)
        assert torch.equal(m.reward_components[:8], o.reward_components.reshape(8, 6))
        assert torch.equal(m.done[:8], torch.repeat_interleave(o.done, 2))
        assert torch.equal(m.done[8:11], ow.done) and torch.equal(m.done[11:13], ol.done)
        assert torch.equal(m.winner[11:13], ol.winner)
        assert torch.equal(m.final_observation[8:11], ow.final_observation)
    for name in sw.carry:
        assert torch.equal(mstate.seats[0].carry[name], sw.carry[name])
