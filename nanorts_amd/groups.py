"""Several groups of games in one batch.

`step_groups` is core.step_groups (src/nanorts/core/__init__.py:63-89,
src/nanorts/core/cycle.py:137-175): core.step for up to 16 groups of lanes,
each with its own State, Commands and keys, in one kernel launch per four
groups when the groups' games share one bucket and unit table (they may
differ in terrain and horizon), else one launch per group.

`GroupMix` is src/nanorts/bots/mix.py:17-275: a batch of groups, each an
environment (the JaxMARL facade or a learner-vs-bot seat) with its own lanes,
published agent-major: every output row is one agent of one lane, groups
concatenated in order.  Groups whose environments split their step
(step_request / step_response) and whose games step together (one bucket)
share one core.step launch per cycle: each builds its request (decode, and
the bot's act for a seat), `step_groups` steps them all, and each answers
its own (rewards, observation, auto-reset).  Any other group steps in its
own fused launch.  The rows of all groups must have equal shapes, so the
groups' environments publish equal observation and action spaces and equal
infos.
"""
from __future__ import annotations

import ctypes
import dataclasses
from collections.abc import Sequence
from typing import Any

import numpy as np
import torch

from nanorts_amd import native
from nanorts_amd.env import DeviceGame, EnvironmentState, State, _ptr, _stream
from nanorts_amd.model import ModelError

MAX_GROUPS = 16
_COMMAND_FIELDS = ("kind", "direction", "none_duration", "target_cell", "produced_type", "request_order")


def _device_game(holder: Any) -> DeviceGame:
    """The DeviceGame of a facade (NanoRTS, SeatEnv, GridNet) or a DeviceGame."""
    if isinstance(holder, DeviceGame):
        return holder
    for path in (("dev",), ("env", "dev")):
        obj = holder
        for name in path:
            obj = getattr(obj, name, None)
        if isinstance(obj, DeviceGame):
            return obj
    raise ModelError(f"step_groups takes a facade or a DeviceGame per request, not {type(holder).__name__}")


def _tables_equal(a, b) -> bool:
    return a.bucket == b.bucket and tuple(a.unit_types) == tuple(b.unit_types)


def steps_together(games: Sequence[Any]) -> bool:
    """src/nanorts/core/__init__.py:63-68: more than one game, all on one
    bucket (and so one unit table and strategy)."""
    games = [g.game if isinstance(g, DeviceGame) else g for g in games]
    return 1 < len(games) <= MAX_GROUPS and all(_tables_equal(games[0], g) for g in games[1:])


def step_groups(requests: Sequence[tuple[Any, Any, dict[str, torch.Tensor], Any]], *,
                records: bool = False) -> list[dict[str, torch.Tensor]]:
    """core.step over every request (key, state, commands, game holder), in
    place: `key` is uint32 key data [L, 2] or [2] (host data, or an int32
    device tensor holding it bit for bit); `state` an
    EnvironmentState or the core State; `commands` int32[L, 2, C] per
    field; the holder a facade or DeviceGame.  Returns each group's
    terminated, truncated, reward and admitted event counts, and with
    `records` the per-slot completion records (is_member, records_i32,
    records_i16, records_i8; core.step_events decodes them)."""
    if not requests:
        return []
    devs = [_device_game(holder) for *_, holder in requests]
    prepared = []
    for (key, state, commands, _), dev in zip(requests, devs, strict=True):
        core = state.core_state if isinstance(state, EnvironmentState) else state
        if not isinstance(core, State):
            raise ModelError("step_groups takes an EnvironmentState or a core State per request")
        L = int(core.leaves["time"].shape[0])
        d = dev.device
        if isinstance(key, torch.Tensor) and key.device == d and key.dtype == torch.int32:
            keyt = key.reshape(-1, 2).contiguous()  # key data already on the device, bit for bit
        else:
            keyt = torch.as_tensor(np.ascontiguousarray(np.asarray(key.cpu() if isinstance(key, torch.Tensor) else key,
                                                                   np.uint32).reshape(-1, 2)).view(np.int32), device=d)
        if keyt.shape[0] not in (1, L):
            raise ModelError(f"a step_groups key holds {keyt.shape[0]} keys for {L} lanes")
        cmd = {f: commands[f].to(device=d, dtype=torch.int32).contiguous() for f in _COMMAND_FIELDS}
        b = dev.game.bucket
        out = {"terminated": torch.empty(L, dtype=torch.bool, device=d),
               "truncated": torch.empty(L, dtype=torch.bool, device=d),
               "reward": torch.empty((L, 2), dtype=torch.float32, device=d),
               "admitted_harvest": torch.empty((L, 2), dtype=torch.int32, device=d),
               "admitted_return": torch.empty((L, 2), dtype=torch.int32, device=d),
               "admitted_produce": torch.empty((L, 2, b.unit_type_capacity), dtype=torch.int32, device=d),
               "admitted_attack": torch.empty((L, 2, 3), dtype=torch.int32, device=d)}
        if records:
            E = b.entity_capacity
            out.update(is_member=torch.empty((L, E), dtype=torch.bool, device=d),
                       records_i32=torch.empty((L, E, 6), dtype=torch.int32, device=d),
                       records_i16=torch.empty((L, E, 4), dtype=torch.int16, device=d),
                       records_i8=torch.empty((L, E, 6), dtype=torch.int8, device=d))
        leaves = core.leaves
        st = native.State(*[_ptr(leaves[name]) for name in native.STATE_FIELDS[:-2]], None, None)
        prepared.append((L, keyt, cmd, out, st))
    lib = native.load()
    results = [p[3] for p in prepared]
    if len(devs) > 1 and all(_tables_equal(devs[0].game, d.game) for d in devs[1:]):
        for c0 in range(0, len(prepared), MAX_GROUPS):
            part, pdevs = prepared[c0:c0 + MAX_GROUPS], devs[c0:c0 + MAX_GROUPS]
            G = len(part)
            games = (ctypes.POINTER(native.Game) * G)(*[ctypes.pointer(d.struct) for d in pdevs])
            states = (native.State * G)(*[p[4] for p in part])
            lanes = (ctypes.c_int64 * G)(*[p[0] for p in part])
            keys = (ctypes.c_void_p * G)(*[_ptr(p[1]) for p in part])
            key_lanes = (ctypes.c_int64 * G)(*[p[1].shape[0] for p in part])
            cmds = (native.Commands * G)(*[native.Commands(*[_ptr(p[2][f]) for f in _COMMAND_FIELDS]) for p in part])
            outs = (native.StepResults * G)(*[native.StepResults(*[_ptr(p[3].get(f)) for f, _ in
                                                                   native.StepResults._fields_]) for p in part])
            native.check(lib.nanorts_amd_step_groups(_stream(), G, games, states, lanes, keys, key_lanes, cmds, outs),
                         "nanorts_amd_step_groups")
        return results
    for dev, (L, keyt, cmd, out, st) in zip(devs, prepared, strict=True):
        c = native.Commands(*[_ptr(cmd[f]) for f in _COMMAND_FIELDS])
        r = native.StepResults(*[_ptr(out.get(f)) for f, _ in native.StepResults._fields_])
        native.check(lib.nanorts_amd_step(_stream(), dev.ref, st, L, _ptr(keyt), keyt.shape[0], c, r), "nanorts_amd_step")
    return results


# ---------------------------------------------------------------------------
# GroupMix
# ---------------------------------------------------------------------------
@dataclasses.dataclass(frozen=True)
class Group:
    """src/nanorts/bots/mix.py:17-19"""

    environment: Any
    lanes: int


def _concat(parts: list[Any]) -> Any:
    """Concatenate matching trees of tensors (dicts, dataclasses) along dim 0."""
    first = parts[0]
    if isinstance(first, torch.Tensor):
        return torch.cat(parts)
    if isinstance(first, dict):
        return {k: _concat([p[k] for p in parts]) for k in first}
    if dataclasses.is_dataclass(first):
        return type(first)(**{f.name: _concat([getattr(p, f.name) for p in parts])
                              for f in dataclasses.fields(first)})
    raise ModelError(f"GroupMix cannot concatenate {type(first).__name__}")


def _agents(env: Any) -> list[str]:
    return list(env.agents)


def _agent_major(per_agent: dict[str, Any], env: Any) -> Any:
    return _concat([per_agent[a] for a in _agents(env)])


def _info_rows(infos: dict[str, Any], env: Any) -> dict[str, Any]:
    agents = _agents(env)
    return {name: (_agent_major(value, env) if isinstance(value, dict) and list(value) == agents
                   else _concat([value] * len(agents)))
            for name, value in infos.items()}


def _facade(env: Any) -> Any:
    return getattr(env, "env", env)


def _row_signature(env: Any) -> tuple:
    """What every row of a group looks like: the observation and action
    spaces and the infos a step publishes."""
    f = _facade(env)
    y = f.layout
    return (y.surface, y.partial_observability, y.feature_maps_shape, y.actions_shape, y.mask_width,
            y.final_observation, y.reward_components)


class GroupMix:
    """src/nanorts/bots/mix.py:22-275, batched over each group's lanes."""

    def __init__(self, groups: Sequence[Group]) -> None:
        self.groups = tuple(groups)
        if not self.groups:
            raise ModelError("a GroupMix needs at least one group")
        for index, group in enumerate(self.groups):
            if not isinstance(group.lanes, int) or isinstance(group.lanes, bool) or group.lanes < 1:
                raise ModelError(f"group {index} asks for lanes={group.lanes!r}; give a positive int")
        signatures = [_row_signature(group.environment) for group in self.groups]
        for index, signature in enumerate(signatures[1:], start=1):
            if signature != signatures[0]:
                raise ModelError(f"group {index} publishes rows unlike group 0's; every group needs the same observation and "
                                 "action spaces and the same final_observation and reward_components settings")

    @property
    def lanes(self) -> int:
        return sum(group.lanes for group in self.groups)

    @property
    def rows(self) -> int:
        return sum(self._row_counts())

    def slices(self) -> tuple[slice, ...]:
        return tuple(self._bounds(self._row_counts()))

    def reset(self, roots) -> tuple[Any, tuple[Any, ...]]:
        """uint32 key data [lanes, 2] -> (agent-major observations, per-group states)."""
        roots = np.asarray(roots.cpu() if isinstance(roots, torch.Tensor) else roots, np.uint32).reshape(-1, 2)
        if roots.shape[0] != self.lanes:
            raise ModelError(f"GroupMix.reset takes {self.lanes} roots, got {roots.shape[0]}")
        observations, states = [], []
        for group, bound in zip(self.groups, self._bounds(self._lane_counts()), strict=True):
            obs, state = group.environment.reset(roots[bound])
            observations.append(_agent_major(obs, group.environment))
            states.append(state)
        return _concat(observations), tuple(states)

    def step(self, key, states: tuple[Any, ...], actions: torch.Tensor, *, donate: bool = False):
        """Actions int32[rows, C, 7], agent-major per group -> (observations,
        next states, rewards, dones, infos), each agent-major
        (src/nanorts/bots/mix.py:105-166)."""
        if actions.shape[0] != self.rows:
            raise ModelError(f"GroupMix.step takes {self.rows} action rows, got {actions.shape[0]}")
        per_agent = []
        for group, bound in zip(self.groups, self._bounds(self._row_counts()), strict=True):
            rows = actions[bound]
            per_agent.append(dict(zip(_agents(group.environment), torch.split(rows, group.lanes), strict=True)))
        stepped: dict[int, tuple] = {}
        for members in self.shared_launches():
            envs = [self.groups[i].environment for i in members]
            # the split step updates its state in place
            mine = [states[i] if donate else states[i].clone() for i in members]
            requests = [env.step_request(state, per_agent[i]) for env, state, i in zip(envs, mine, members, strict=True)]
            results = step_groups([(*request, env) for env, (request, _) in zip(envs, requests, strict=True)])
            for env, state, i, (_, carry), result in zip(envs, mine, members, requests, results, strict=True):
                stepped[i] = env.step_response(state, carry, result)
        observations, following, rewards, dones, infos = [], [], [], [], []
        for i, (group, state) in enumerate(zip(self.groups, states, strict=True)):
            env = group.environment
            obs, nxt, reward, done, info = (stepped[i] if i in stepped
                                            else env.step(key, state, per_agent[i], donate=donate))
            observations.append(_agent_major(obs, env))
            following.append(nxt)
            rewards.append(_agent_major(reward, env))
            dones.append(_agent_major({a: done[a] for a in _agents(env)}, env))
            infos.append(_info_rows(info, env))
        return _concat(observations), tuple(following), _concat(rewards), _concat(dones), _concat(infos)

    def shared_launches(self) -> list[list[int]]:
        """The groups that share a core.step launch, by bucket
        (src/nanorts/bots/mix.py:124-141): environments with a split step
        whose games step together."""
        by_bucket: dict[Any, list[int]] = {}
        for index, group in enumerate(self.groups):
            env = group.environment
            if callable(getattr(env, "step_request", None)) and callable(getattr(env, "step_response", None)):
                by_bucket.setdefault(_device_game(env).game.bucket, []).append(index)
        return [members for members in by_bucket.values()
                if steps_together([_device_game(self.groups[i].environment).game for i in members])]

    def get_avail_actions(self, states: tuple[Any, ...]) -> torch.Tensor:
        return _concat([_agent_major(group.environment.get_avail_actions(state), group.environment)
                        for group, state in zip(self.groups, states, strict=True)])

    def get_slot_cells(self, states: tuple[Any, ...]) -> torch.Tensor:
        return _concat([_agent_major(group.environment.get_slot_cells(state), group.environment)
                        for group, state in zip(self.groups, states, strict=True)])

    def _lane_counts(self) -> list[int]:
        return [group.lanes for group in self.groups]

    def _row_counts(self) -> list[int]:
        return [group.lanes * len(_agents(group.environment)) for group in self.groups]

    @staticmethod
    def _bounds(sizes: list[int]) -> list[slice]:
        out, start = [], 0
        for size in sizes:
            out.append(slice(start, start + size))
            start += size
        return out
