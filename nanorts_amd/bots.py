"""Scripted opponents on the GPU: WorkerRush and LightRush, and the
learner-vs-bot seat.

Mirrors src/nanorts/bots/{bot,family,worker_rush,light_rush}.py (the `Bot`
records and family.act) and src/nanorts/bots/seat.py (SeatEnv and the seat
functions): the bot's decisions run in the nanorts_amd_abstraction_act kernel,
and a whole seat step (bot act, learner decode, core.step, auto-reset, carry
reset, the next seat) is one nanorts_amd_seat_step launch.  Every call is
batched over L envs on the current HIP stream.

Seats follow src/nanorts/bots/seat.py:335-375: "player_0" and "player_1"
are static; "drawn" draws each episode's learner from its episode root,
randint(fold_in(root, 2**32 - 2), (), 0, 2), at reset and again when a game
ends; an int32[L] array (through reset_seat / step_seat) fixes a seat per
lane.  Per-lane seats pick each lane's learner outputs with a select.
"""
from __future__ import annotations

import ctypes
import dataclasses
import weakref
from typing import Any, Final

import numpy as np
import torch

from nanorts_amd import native
from nanorts_amd.content import GameConfig, with_unit_type_table
from nanorts_amd.env import (
    ALL_AGENTS,
    NanoRTS,
    EnvironmentState,
    _ptr,
    _stream,
)
from nanorts_amd.model import ModelError, UnitTypeTableVersion

WORKER_RUSH: Final = 0
BARRACKS_RUSH: Final = 1
TYPE_LIGHT: Final = 4
LEARNER: Final = "learner"
SEAT_RULES: Final = ("player_0", "player_1", "drawn")
_PLAYERS: Final = ("player_0", "player_1")


@dataclasses.dataclass(frozen=True)
class Bot:
    """An abstraction-family bot (src/nanorts/bots/bot.py:13-22): the
    family strategy and the unit type its barracks train."""

    name: str
    strategy: int
    trained: int = TYPE_LIGHT


workerRushAI: Final = Bot("workerRushAI", WORKER_RUSH)  # src/nanorts/bots/worker_rush.py:18-20
lightRushAI: Final = Bot("lightRushAI", BARRACKS_RUSH, TYPE_LIGHT)  # src/nanorts/bots/light_rush.py:20-22
ROSTER: Final = {bot.name: bot for bot in (workerRushAI, lightRushAI)}


def empty_actions(num_envs: int, capacity: int, device) -> dict[str, torch.Tensor]:
    """abstraction.empty_actions for L envs (src/nanorts/bots/abstraction.py:118-133)."""
    carry = {f: torch.full((num_envs, capacity), -1, dtype=torch.int32, device=device)
             for f in native.ABSTRACT_FIELDS[:9]}
    carry["trained"] = torch.zeros((num_envs, capacity), dtype=torch.bool, device=device)
    carry["next_order"] = torch.zeros(num_envs, dtype=torch.int32, device=device)
    return carry


def _carry_struct(carry: dict[str, torch.Tensor]) -> native.AbstractActions:
    return native.AbstractActions(*[_ptr(carry[f]) for f in native.ABSTRACT_FIELDS])


def abstraction_act(env: NanoRTS, state: EnvironmentState, carry: dict[str, torch.Tensor], bot: Bot,
                    player) -> dict[str, torch.Tensor]:
    """family.act (src/nanorts/bots/family.py:34-41): Commands [L, 2, C] per
    field for `player` (an int or int32[L]); the carry is updated in place."""
    L = state.num_envs
    C = env.bucket.per_player_capacity
    players = torch.as_tensor(player, dtype=torch.int32, device=env.device).reshape(-1).contiguous()
    commands = torch.empty((L, 6, 2, C), dtype=torch.int32, device=env.device)
    native.check(env.lib.nanorts_amd_abstraction_act(_stream(), env.dev.ref, state.native(), L, bot.strategy,
                                                 bot.trained, _ptr(players), players.numel(), _carry_struct(carry),
                                                 _ptr(commands)), "nanorts_amd_abstraction_act")
    names = ("kind", "direction", "none_duration", "target_cell", "produced_type", "request_order")
    return {name: commands[:, f] for f, name in enumerate(names)}


@dataclasses.dataclass
class SeatState:
    """src/nanorts/bots/seat.py:37-44"""

    environment_state: EnvironmentState
    carry: dict[str, torch.Tensor]
    seat: torch.Tensor

    def clone(self) -> "SeatState":
        return SeatState(self.environment_state.clone(), {k: v.clone() for k, v in self.carry.items()},
                         self.seat.clone())


def _pick(per_agent: dict[str, Any], seat: torch.Tensor) -> Any:
    """_learners (src/nanorts/bots/seat.py:368-375) for per-lane seats: lane
    l's value of player seat[l], for a tensor or an observation record."""
    first, second = (per_agent[agent] for agent in _PLAYERS)

    def one(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
        return torch.where(seat.reshape((-1,) + (1,) * (a.dim() - 1)) == 0, a, b)

    if dataclasses.is_dataclass(first):
        return type(first)(**{f.name: one(getattr(first, f.name), getattr(second, f.name))
                              for f in dataclasses.fields(first)})
    return one(first, second)


def episode_seats(env: NanoRTS, state: EnvironmentState) -> torch.Tensor:
    """The "drawn" rule's learner of each lane's current episode, int32[L]
    (_episode_seat, src/nanorts/bots/seat.py:352-360)."""
    out = torch.empty(state.num_envs, dtype=torch.int32, device=env.device)
    native.check(env.lib.nanorts_amd_episode_seats(_stream(), _ptr(state.environment_root), _ptr(state.episode_index),
                                               state.num_envs, _ptr(out)), "nanorts_amd_episode_seats")
    return out


class SeatEnv:
    """One learner against a scripted bot (src/nanorts/bots/seat.py:181-332)
    with a seat rule: "player_0", "player_1" or "drawn"."""

    def __init__(self, bot: Bot, *, scenario: GameConfig, utt: UnitTypeTableVersion | None = None,
                 seat: str = "player_0", surface: str = "symbolic", partial_observability: bool = False,
                 final_observation: bool = True, feature_dtype: Any = None, reward_components: bool = False,
                 device: str | torch.device | None = None):
        if not isinstance(seat, str) or seat not in SEAT_RULES:
            raise ModelError(f"seat={seat!r} is not a seat rule ({list(SEAT_RULES)}); per-lane seat arrays are taken by "
                             "reset_seat / step_seat")
        if bot.strategy not in (WORKER_RUSH, BARRACKS_RUSH):
            raise ModelError(f"bot {bot.name!r} is not available here; the seat plays WorkerRush or LightRush")
        game = scenario if utt is None else with_unit_type_table(scenario, utt)
        self.env = NanoRTS(game, surface=surface, partial_observability=partial_observability,
                           final_observation=final_observation, feature_dtype=feature_dtype,
                           reward_components=reward_components, device=device)
        self.bot = bot
        self.seat = seat
        # the static player, or None where the seat is per lane
        self.learner = _PLAYERS.index(seat) if seat in _PLAYERS else None
        self.draw = seat == "drawn"
        self.agents = [LEARNER]
        self.game = game
        self.device = self.env.device

    def _learners(self, per_agent: dict[str, Any], seat: torch.Tensor) -> Any:
        return per_agent[_PLAYERS[self.learner]] if self.learner is not None else _pick(per_agent, seat)

    def _start_seats(self, state: EnvironmentState, seat) -> torch.Tensor:
        L = state.num_envs
        if self.learner is not None:
            return torch.full((L,), self.learner, dtype=torch.int32, device=self.device)
        if self.draw:
            return episode_seats(self.env, state)
        lanes = torch.as_tensor(seat, device=self.device).to(torch.int32).reshape(-1)
        lanes = lanes.expand(L).contiguous() if lanes.numel() == 1 else lanes.contiguous()
        if lanes.numel() != L or bool(((lanes < 0) | (lanes > 1)).any()):
            raise ModelError(f"a per-lane seat is int32[{L}] of players 0 and 1")
        return lanes.clone()

    def reset(self, key, seat=None) -> tuple[dict[str, Any], SeatState]:
        """seat.reset_seat (src/nanorts/bots/seat.py:73-81); `seat` is the
        per-lane int32[L] seat of an env built by reset_seat."""
        obs, state = self.env.reset(key)
        L = state.num_envs
        carry = empty_actions(L, self.env.bucket.per_player_capacity, self.device)
        seats = self._start_seats(state, seat)
        return {LEARNER: self._learners(obs, seats)}, SeatState(state, carry, seats)

    def step(self, key, state: SeatState, actions: dict[str, torch.Tensor], reset_state=None, *,
             donate: bool = False):
        """seat.step_seat in one launch; the state (and carry) are updated in
        place with donate=True, else copied first."""
        del key
        if reset_state is not None:
            raise ModelError("step resets finished games to the content's start by itself; reset_state is not taken")
        env = self.env
        nxt = state if donate else state.clone()
        es = nxt.environment_state
        L = es.num_envs
        b = env.bucket
        d = self.device
        acts = torch.as_tensor(actions[LEARNER], device=d)
        if acts.dtype != torch.int32 or tuple(acts.shape) != (L, b.per_player_capacity, 7):
            raise ModelError(f"learner actions must be int32[{L}, {b.per_player_capacity}, 7]")
        acts = acts.contiguous()
        out = {
            "reward": torch.empty((L, 2), dtype=torch.float32, device=d),
            "done": torch.empty(L, dtype=torch.bool, device=d),
            "terminated": torch.empty(L, dtype=torch.bool, device=d),
            "truncated": torch.empty(L, dtype=torch.bool, device=d),
            "winner": torch.empty(L, dtype=torch.int32, device=d),
            "spawn_overflowed": torch.empty(L, dtype=torch.bool, device=d),
            "spawn_overflow": torch.empty((L, 2), dtype=torch.int32, device=d),
        }
        maps = torch.empty((L, 2, b.height, b.width, 6), dtype=torch.uint8, device=d)
        scalars = torch.empty((L, 2, 4), dtype=torch.int32, device=d)
        fmaps = torch.empty_like(maps) if env.final_observation else None
        fscal = torch.empty_like(scalars) if env.final_observation else None
        comps = torch.empty((L, 2, 6), dtype=torch.float32, device=d) if env.layout.reward_components else None
        results = native.EnvResults(
            _ptr(out["reward"]), _ptr(out["done"]), _ptr(out["terminated"]), _ptr(out["truncated"]),
            _ptr(out["winner"]), _ptr(out["spawn_overflowed"]), _ptr(maps), _ptr(scalars), _ptr(fmaps), _ptr(fscal),
            _ptr(comps), _ptr(out["spawn_overflow"]))
        if self.learner is not None:
            current = nxt.seat
            native.check(env.lib.nanorts_amd_seat_step(_stream(), env.dev.ref, es.native(), L, self.bot.strategy,
                                                   self.bot.trained, self.learner, _carry_struct(nxt.carry),
                                                   _ptr(acts), env.partial, results), "nanorts_amd_seat_step")
        else:
            if nxt.seat.dtype != torch.int32 or tuple(nxt.seat.shape) != (L,) or not nxt.seat.is_contiguous():
                raise ModelError(f"the seat state's seat must be a contiguous int32[{L}]")
            current = nxt.seat.clone()
            native.check(env.lib.nanorts_amd_seat_step_lanes(_stream(), env.dev.ref, es.native(), L, self.bot.strategy,
                                                         self.bot.trained, _ptr(nxt.seat), int(self.draw),
                                                         _carry_struct(nxt.carry), _ptr(acts), env.partial, results),
                         "nanorts_amd_seat_step_lanes")
        publish = env._symbolic if env.layout.surface == "symbolic" else env._pixels
        obs = self._learners(publish(maps, scalars), nxt.seat)
        infos: dict[str, Any] = {
            "terminated": out["terminated"], "truncated": out["truncated"], "winner": out["winner"],
            "telemetry": {"spawn_overflow": out["spawn_overflow"]},
            "spawn_overflowed": out["spawn_overflowed"], "final_valid": out["done"],
        }
        if env.final_observation:
            infos["final_observation"] = {LEARNER: self._learners(publish(fmaps, fscal), current)}
        if comps is not None:
            infos["reward_components"] = {LEARNER: self._learners({a: comps[:, p] for p, a in enumerate(_PLAYERS)},
                                                                  current)}
        reward = self._learners({a: out["reward"][:, p] for p, a in enumerate(_PLAYERS)}, current)
        return ({LEARNER: obs}, nxt, {LEARNER: reward}, {LEARNER: out["done"], ALL_AGENTS: out["done"]}, infos)

    def rollout(self, state: SeatState, steps: int, sample_key, *, step0: int = 0, env0: int = 0,
                record: bool = True, record_actions: bool = False, observation_depth: int = 1,
                two_pass: bool = True) -> dict[str, Any]:
        """Fused rollout of `steps` cycles in place: the learner's rows from the
        synthetic harness's uniform-over-legal sampler, the bot's act and the
        seat step, with the state resident in LDS.  Bit-equal to
        get_avail_actions(form="words") -> sample_actions -> step per cycle.
        Rewards are both players' [steps, L, 2]; with per-lane seats "seats"
        holds the learner of every cycle [steps, L].  With two_pass (the
        default) a launch may run each game first with two games per wave on
        a window of the slots and hand the rest of a game's cycles to the
        one-game-per-wave pass; out["first_pass_cycles"] int32[L] holds the
        first pass's cycles of each game in the last launch."""
        env = self.env
        es = state.environment_state
        L = es.num_envs
        b = env.bucket
        d = self.device
        rewards = torch.empty((steps, L, 2), dtype=torch.float32, device=d) if record else None
        dones = torch.empty((steps, L), dtype=torch.bool, device=d) if record else None
        actions = torch.empty((steps, L, b.per_player_capacity, 7), dtype=torch.int32, device=d) \
            if record_actions else None
        depth = max(1, int(observation_depth))
        maps = torch.empty((depth, L, 2, b.height, b.width, 6), dtype=torch.uint8, device=d)
        scalars = torch.empty((depth, L, 2, 4), dtype=torch.int32, device=d)
        key = (ctypes.c_uint32 * 2)(*[int(v) for v in np.asarray(sample_key, np.uint32).reshape(2)])
        results = native.RolloutResults(_ptr(rewards), _ptr(dones), _ptr(actions), _ptr(maps), _ptr(scalars), depth)
        progress = torch.empty(L, dtype=torch.int32, device=d) if two_pass else None
        results.progress = _ptr(progress)
        seats = None
        if self.learner is not None:
            native.check(env.lib.nanorts_amd_seat_rollout(_stream(), env.dev.ref, es.native(), L, self.bot.strategy,
                                                      self.bot.trained, self.learner, _carry_struct(state.carry), key,
                                                      int(step0), int(steps), env.partial, int(env0), results),
                         "nanorts_amd_seat_rollout")
        else:
            seats = torch.empty((steps, L), dtype=torch.int32, device=d) if record else None
            native.check(env.lib.nanorts_amd_seat_rollout_lanes(_stream(), env.dev.ref, es.native(), L, self.bot.strategy,
                                                            self.bot.trained, _ptr(state.seat), int(self.draw),
                                                            _ptr(seats), _carry_struct(state.carry), key, int(step0),
                                                            int(steps), env.partial, int(env0), results),
                         "nanorts_amd_seat_rollout_lanes")
        return {"rewards": rewards, "dones": dones, "actions": actions, "feature_maps": maps, "scalars": scalars,
                "seats": seats, "first_pass_cycles": progress}

    def _bot_players(self, state: SeatState):
        return 1 - self.learner if self.learner is not None else (1 - state.seat).contiguous()

    def step_request(self, state: SeatState, actions: dict[str, torch.Tensor]):
        """seat.step_request (src/nanorts/bots/seat.py:100-111, 249-258): the
        bot's act on a copy of the carry, the learner's decoded rows and the
        bot's Commands merged ((episode-root keys, core State, Commands),
        the bot's new carry), ready for groups.step_groups."""
        env = self.env
        es = state.environment_state
        L = es.num_envs
        C = env.bucket.per_player_capacity
        acts = torch.as_tensor(actions[LEARNER], device=self.device)
        if acts.dtype != torch.int32 or tuple(acts.shape) != (L, C, 7):
            raise ModelError(f"learner actions must be int32[{L}, {C}, 7]")
        carry = {k: v.clone() for k, v in state.carry.items()}
        bot_player = self._bot_players(state)
        bot_cmds = abstraction_act(env, es, carry, self.bot, bot_player)
        # the learner's rows at its seat, zeros at the bot's (replaced below)
        rows = torch.zeros((L, 2, C, 7), dtype=torch.int32, device=self.device)
        seat = state.seat.long() if self.learner is None else torch.full((L,), self.learner, device=self.device)
        rows[torch.arange(L, device=self.device), seat] = acts
        (keys, core, cmds), _ = env.step_request(es, {agent: rows[:, p] for p, agent in enumerate(env.agents)})
        bots_side = (torch.arange(2, device=self.device)[None, :] != seat[:, None]).reshape(L, 2, 1)
        for name in cmds:
            cmds[name] = torch.where(bots_side, bot_cmds[name], cmds[name])
        return (keys, core, cmds), carry

    def step_response(self, state: SeatState, carry: dict[str, torch.Tensor], stepped: dict[str, torch.Tensor]):
        """seat.step_response (src/nanorts/bots/seat.py:114-149, 260-272) on a
        state that core.step has advanced in place: the facade's response for
        the learner, the bot's new carry emptied where the game ended, and the
        next seat (drawn from the next episode's root where the game ended,
        under the "drawn" rule).  The state is updated in place."""
        obs, es, rewards, dones, infos = self.env.step_response(state.environment_state, None, stepped)
        done = dones[ALL_AGENTS]
        fresh = empty_actions(es.num_envs, self.env.bucket.per_player_capacity, self.device)
        for name, value in carry.items():
            mask = done.reshape((-1,) + (1,) * (value.dim() - 1))
            state.carry[name] = torch.where(mask, fresh[name], value)
        current = state.seat
        if self.draw:
            state.seat = torch.where(done, episode_seats(self.env, es), current).contiguous()
        out_infos = dict(infos)
        if "final_observation" in infos:
            out_infos["final_observation"] = {LEARNER: self._learners(infos["final_observation"], current)}
        if "reward_components" in infos:
            out_infos["reward_components"] = {LEARNER: self._learners(infos["reward_components"], current)}
        return ({LEARNER: self._learners(obs, state.seat)}, state, {LEARNER: self._learners(rewards, current)},
                {LEARNER: done, ALL_AGENTS: done}, out_infos)

    def observation_space(self, agent: str) -> dict[str, Any]:
        """src/nanorts/bots/seat.py:208-213: player_0's space, the same for
        either seat."""
        if agent != LEARNER:
            raise ModelError(f"SeatEnv has the one agent {LEARNER!r}, not {agent!r}")
        return self.env.observation_space(_PLAYERS[0])

    def action_space(self, agent: str) -> dict[str, Any]:
        if agent != LEARNER:
            raise ModelError(f"SeatEnv has the one agent {LEARNER!r}, not {agent!r}")
        return self.env.action_space(_PLAYERS[0])

    @property
    def agent_classes(self) -> dict[str, list[str]]:
        """src/nanorts/bots/seat.py:330-332"""
        return {LEARNER: [LEARNER]}

    def get_avail_actions(self, state: SeatState, *, form: str = "rows") -> dict[str, torch.Tensor]:
        return {LEARNER: self._learners(self.env.get_avail_actions(state.environment_state, form=form), state.seat)}

    def get_obs(self, state: SeatState) -> dict[str, Any]:
        return {LEARNER: self._learners(self.env.get_obs(state.environment_state), state.seat)}

    def get_slot_cells(self, state: SeatState) -> dict[str, torch.Tensor]:
        return {LEARNER: self._learners(self.env.get_slot_cells(state.environment_state), state.seat)}

    def commands(self, state: SeatState) -> dict[str, torch.Tensor]:
        """The bot's Commands for the current state (seat.seat_commands,
        src/nanorts/bots/seat.py:152-157); the carry is updated in place."""
        return abstraction_act(self.env, state.environment_state, state.carry, self.bot, self._bot_players(state))


@dataclasses.dataclass
class SeatStep:
    """src/nanorts/bots/seat.py:46-70"""

    seat_state: SeatState
    observation: Any
    reward: torch.Tensor
    reward_components: torch.Tensor | None
    terminated: torch.Tensor
    truncated: torch.Tensor
    done: torch.Tensor
    winner: torch.Tensor
    telemetry: dict[str, torch.Tensor]
    spawn_overflowed: torch.Tensor
    final_observation: Any
    final_valid: torch.Tensor


# The SeatEnvs behind the seat functions, per game and (bot, rule, options).
_SEAT_ENVS: "weakref.WeakKeyDictionary[GameConfig, dict[tuple, SeatEnv]]" = weakref.WeakKeyDictionary()


def _seat_env(bot: Bot, game: GameConfig, seat, options: dict[str, Any]) -> SeatEnv:
    """The SeatEnv that runs the seat functions for (bot, game, rule, options);
    an array seat runs as the per-lane rule (the seats stay as given)."""
    if isinstance(seat, str):
        rule = seat
    elif isinstance(seat, int) and not isinstance(seat, bool):
        if seat not in (0, 1):
            raise ModelError(f"seat={seat} names no player; use 0 or 1")
        rule = _PLAYERS[seat]
    else:
        rule = "lanes"
    per_game = _SEAT_ENVS.setdefault(game, {})
    key = (bot, rule, tuple(sorted((k, str(v)) for k, v in options.items())))
    env = per_game.get(key)
    if env is None:
        env = SeatEnv(bot, scenario=game, seat="drawn" if rule == "lanes" else rule, **options)
        if rule == "lanes":
            env.seat, env.draw = "lanes", False
        per_game[key] = env
    return env


def reset_seat(environment_root, game: GameConfig, *, bot: Bot, seat="player_0",
               **options) -> tuple[SeatState, Any]:
    """seat.reset_seat (src/nanorts/bots/seat.py:73-81) over L envs: `seat`
    is a rule ("player_0", "player_1", "drawn"), a Player index or an int32[L]
    per-lane seat; `options` are SeatEnv's (surface, partial_observability,
    final_observation, feature_dtype, reward_components, device)."""
    env = _seat_env(bot, game, seat, options)
    obs, state = env.reset(environment_root, seat=None if isinstance(seat, (str, int)) else seat)
    return state, obs[LEARNER]


def step_seat(seat_state: SeatState, actions: torch.Tensor, game: GameConfig, *, bot: Bot, seat="player_0",
              donate: bool = False, **options) -> SeatStep:
    """seat.step_seat (src/nanorts/bots/seat.py:84-97) with the learner's
    actions int32[L, C, 7]; the same `seat` and options as reset_seat."""
    env = _seat_env(bot, game, seat, options)
    obs, state, reward, done, infos = env.step(None, seat_state, {LEARNER: actions}, donate=donate)
    final = infos.get("final_observation")
    comps = infos.get("reward_components")
    return SeatStep(state, obs[LEARNER], reward[LEARNER], None if comps is None else comps[LEARNER],
                    infos["terminated"], infos["truncated"], done[LEARNER], infos["winner"], infos["telemetry"],
                    infos["spawn_overflowed"], None if final is None else final[LEARNER], infos["final_valid"])


def carry_numpy(carry: dict[str, torch.Tensor]) -> dict[str, np.ndarray]:
    out = {k: v.cpu().numpy() for k, v in carry.items()}
    out["trained"] = out["trained"].astype(np.uint8)
    return out


def seat_commands(seat_state: SeatState, game: GameConfig, *, bot: Bot, seat="player_0",
                  **options) -> tuple[dict[str, torch.Tensor], dict[str, torch.Tensor]]:
    """seat.seat_commands (src/nanorts/bots/seat.py:152-157): (the bot's new
    carry, its Commands [L, 2, C] per field); the seat state is left as it is."""
    env = _seat_env(bot, game, seat, options)
    carry = {k: v.clone() for k, v in seat_state.carry.items()}
    return carry, abstraction_act(env.env, seat_state.environment_state, carry, bot, env._bot_players(seat_state))


def observe_seat(seat_state: SeatState, game: GameConfig, *, seat="player_0", **options) -> Any:
    """seat.observe_seat (src/nanorts/bots/seat.py:160-164): the learner's
    observation of each lane."""
    return _seat_env(workerRushAI, game, seat, options).get_obs(seat_state)[LEARNER]


def legal_seat_actions(seat_state: SeatState, game: GameConfig, *, seat="player_0", **options) -> torch.Tensor:
    """seat.legal_seat_actions (src/nanorts/bots/seat.py:167-171): the
    learner's masks bool[L, C, 78]."""
    return _seat_env(workerRushAI, game, seat, options).get_avail_actions(seat_state)[LEARNER]


def seat_slot_cells(seat_state: SeatState, game: GameConfig, *, seat="player_0", **options) -> torch.Tensor:
    """seat.seat_slot_cells (src/nanorts/bots/seat.py:174-178): the learner's
    slot cells int32[L, C]."""
    return _seat_env(workerRushAI, game, seat, options).get_slot_cells(seat_state)[LEARNER]
