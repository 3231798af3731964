"""The GridNet surface (MicroRTS-Py's per-cell interface) over the gfx950 kernels.

Mirrors src/nanorts/adapters/gridnet/{layout,actions,observation,env}.py of
the reference: `prepare` fixes the output forms, `reset` / `step` /
`step_against` run the environment with auto-reset, `observe` and `planes`
encode a state, `decode_actions` turns per-cell actions into Commands and
`check_actions` / `unpack_mask` are the host-side helpers.  The reference
applies these to one env and is vmapped; here every call is batched over a
leading env dimension L, and each call is one kernel launch on the current
HIP stream (step and step_against fuse decode, core.step, rewards, the
ending state's planes, auto-reset and the next observation).
"""
from __future__ import annotations

import ctypes
import dataclasses
from typing import Any, Final

import numpy as np
import torch

from nanorts_amd import native
from nanorts_amd.content import GameConfig
from nanorts_amd.env import DeviceGame, EnvironmentState, _ptr, _stream
from nanorts_amd.model import PLAYER_COUNT, ModelError

ACTION_FACTORS: Final = ("action_type", "move_direction", "harvest_direction", "return_direction",
                         "produce_direction", "produce_type", "attack_offset")
ACTION_FACTOR_SIZES: Final = (6, 4, 4, 4, 4, 7, 49)
PLANE_WIDTHS: Final = (5, 5, 3, 8, 6, 2)
MASK_WIDTH: Final = 78
MASK_WORDS: Final = 3
OUTPUT_DTYPES: Final = (torch.int32, torch.uint8, torch.bool)
PLANE_FORMS: Final = ("one_hot", "indices")
MASK_FORMS: Final = ("rows", "packed")
PLANE_INDEX_DTYPE: Final = torch.int8
MASK_WORD_DTYPE: Final = torch.int32  # uint32 words, stored bit-for-bit
REWARD_COMPONENTS: Final = ("win_loss", "resource_gather", "produce_worker", "produce_building", "attack",
                            "produce_combat_unit")
_COMMAND_FIELDS: Final = ("kind", "direction", "none_duration", "target_cell", "produced_type", "request_order")


def _offsets(widths: tuple[int, ...]) -> tuple[int, ...]:
    return tuple(int(v) for v in np.cumsum((0,) + tuple(widths[:-1])))


@dataclasses.dataclass(frozen=True)
class GridNetLayout:
    """src/nanorts/adapters/gridnet/layout.py:57-108"""

    bucket: Any
    plane_widths: tuple[int, ...]
    plane_offsets: tuple[int, ...]
    plane_count: int
    action_factor_sizes: tuple[int, ...]
    mask_width: int
    mask_offsets: tuple[int, ...]
    planes_form: str
    planes_dtype: torch.dtype
    mask_form: str
    mask_dtype: torch.dtype
    partial_observability: bool

    @property
    def actions_shape(self) -> tuple[int, int, int, int]:
        return (PLAYER_COUNT, self.bucket.height, self.bucket.width, len(ACTION_FACTORS))

    @property
    def planes_shape(self) -> tuple[int, int, int, int]:
        width = self.plane_count if self.planes_form == "one_hot" else len(self.plane_widths)
        return (PLAYER_COUNT, self.bucket.height, self.bucket.width, width)

    @property
    def source_shape(self) -> tuple[int, int, int]:
        return (PLAYER_COUNT, self.bucket.height, self.bucket.width)

    @property
    def mask_shape(self) -> tuple[int, int, int, int]:
        width = self.mask_width if self.mask_form == "rows" else MASK_WORDS
        return (PLAYER_COUNT, self.bucket.height, self.bucket.width, width)


def _dtype(keyword: str, dtype: Any) -> torch.dtype:
    table = {np.dtype(np.int32): torch.int32, np.dtype(np.uint8): torch.uint8, np.dtype(np.bool_): torch.bool}
    if isinstance(dtype, torch.dtype):
        found = dtype
    else:
        try:
            found = table.get(np.dtype(dtype))
        except TypeError:
            found = None
    if found not in OUTPUT_DTYPES:
        raise ModelError(f"{keyword}={dtype!r} is not a GridNet output type; planes and masks hold 0/1 values as int32 "
                         "(MicroRTS-Py's choice, the default), uint8 or bool")
    return found


def prepare(game: GameConfig, *, partial_observability: bool = False, planes_form: str = "one_hot",
            planes_dtype: Any = torch.int32, mask_form: str = "rows", mask_dtype: Any = torch.int32) -> GridNetLayout:
    """src/nanorts/adapters/gridnet/layout.py:111-141 with its refusals (:144-231)."""
    if partial_observability is not False:
        raise ModelError(f"partial_observability={partial_observability!r}: the GridNet surface here is the fully "
                         "observed one; MicroRTS-Py's 31-plane hidden-information form is not offered")
    bucket = game.bucket
    if bucket.unit_type_capacity != PLANE_WIDTHS[3] - 1:
        raise ModelError(f"a bucket of {bucket.unit_type_capacity} unit types does not fit GridNet, whose unit-type "
                         f"planes are {PLANE_WIDTHS[3]} wide and whose produce-type factor has {ACTION_FACTOR_SIZES[5]} "
                         "values")
    if bucket.attack_offset_capacity != ACTION_FACTOR_SIZES[6]:
        raise ModelError(f"an attack window of {bucket.attack_offset_capacity} cells does not fit GridNet's attack "
                         f"factor of {ACTION_FACTOR_SIZES[6]} values")
    if planes_form not in PLANE_FORMS:
        raise ModelError(f"planes_form={planes_form!r} is unknown; choose one of {list(PLANE_FORMS)}")
    if mask_form not in MASK_FORMS:
        raise ModelError(f"mask_form={mask_form!r} is unknown; choose one of {list(MASK_FORMS)}")
    planes = _dtype("planes_dtype", planes_dtype)
    mask = _dtype("mask_dtype", mask_dtype)
    if planes_form == "indices":
        if planes != torch.int32:
            raise ModelError(f"planes_dtype={planes_dtype!r} conflicts with planes_form='indices', which always holds "
                             "int8 indices")
        planes = PLANE_INDEX_DTYPE
    if mask_form == "packed":
        if mask != torch.int32:
            raise ModelError(f"mask_dtype={mask_dtype!r} conflicts with mask_form='packed', which always holds uint32 "
                             "words")
        mask = MASK_WORD_DTYPE
    if bool(game.initial_state["game_over"]):
        raise ModelError("this content's starting position is already won or drawn, so there is no game to step")
    return GridNetLayout(bucket=bucket, plane_widths=PLANE_WIDTHS, plane_offsets=_offsets(PLANE_WIDTHS),
                         plane_count=sum(PLANE_WIDTHS), action_factor_sizes=ACTION_FACTOR_SIZES,
                         mask_width=MASK_WIDTH, mask_offsets=_offsets(ACTION_FACTOR_SIZES), planes_form=planes_form,
                         planes_dtype=planes, mask_form=mask_form, mask_dtype=mask, partial_observability=False)


@dataclasses.dataclass(frozen=True)
class GridNetObservation:
    """src/nanorts/adapters/gridnet/observation.py:15-24, batched: planes
    [L, 2, H, W, 29 or 6], source_mask bool[L, 2, H, W], action_mask
    [L, 2, H, W, 78 or 3]."""

    planes: torch.Tensor
    source_mask: torch.Tensor
    action_mask: torch.Tensor


@dataclasses.dataclass(frozen=True)
class GridNetStep:
    """src/nanorts/adapters/gridnet/env.py:31-57, batched over L."""

    environment_state: EnvironmentState
    observation: GridNetObservation
    reward_components: torch.Tensor  # float32[L, 2, 6]
    reward_dones: torch.Tensor       # bool[L, 2, 6]
    terminated: torch.Tensor
    truncated: torch.Tensor
    done: torch.Tensor
    winner: torch.Tensor
    telemetry: dict[str, torch.Tensor]
    spawn_overflowed: torch.Tensor
    final_observation: torch.Tensor  # planes of the ending state
    final_valid: torch.Tensor


class GridNet:
    """The GridNet surface of one game on one device (the reference's
    module-level functions with `game` and `layout` bound)."""

    def __init__(self, game: GameConfig, layout: GridNetLayout | None = None, *,
                 device: str | torch.device | None = None):
        self.lib = native.load()
        self.layout = layout if layout is not None else prepare(game)
        if self.layout.bucket != game.bucket:
            raise ModelError("the GridNet layout was prepared for another bucket")
        self.game = game
        self.bucket = game.bucket
        self.device = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
        self.dev = DeviceGame(game, self.device)

    # --------------------------------------------------------------- buffers
    def _obs_buffers(self, L: int) -> tuple[GridNetObservation, native.GridNetObs]:
        y, d = self.layout, self.device
        planes = torch.empty((L, *y.planes_shape), dtype=y.planes_dtype, device=d)
        source = torch.empty((L, *y.source_shape), dtype=torch.bool, device=d)
        mask = torch.empty((L, *y.mask_shape), dtype=y.mask_dtype, device=d)
        return GridNetObservation(planes, source, mask), self._obs_struct(planes, source, mask)

    def _obs_struct(self, planes, source, mask) -> native.GridNetObs:
        y = self.layout
        return native.GridNetObs(
            0 if y.planes_form == "one_hot" else 1, 4 if y.planes_dtype == torch.int32 else 1, _ptr(planes),
            _ptr(source), 0 if y.mask_form == "rows" else 1, 4 if y.mask_dtype == torch.int32 else 1, _ptr(mask))

    # ------------------------------------------------------------------ API
    def reset(self, environment_root) -> tuple[EnvironmentState, GridNetObservation]:
        """env.reset (src/nanorts/adapters/gridnet/env.py:60-62): `environment_root`
        is uint32 key data [L, 2]."""
        roots = np.ascontiguousarray(np.asarray(environment_root.cpu() if isinstance(environment_root, torch.Tensor)
                                                else environment_root).astype(np.uint32).reshape(-1, 2))
        L = roots.shape[0]
        state = EnvironmentState(core_state=self.dev.batch(L),
                                 environment_root=torch.as_tensor(roots.view(np.int32), device=self.device),
                                 episode_index=torch.zeros(L, dtype=torch.int32, device=self.device))
        return state, self.observe(state)

    def observe(self, state: EnvironmentState) -> GridNetObservation:
        """observation.observe (src/nanorts/adapters/gridnet/observation.py:27-33)."""
        obs, struct = self._obs_buffers(state.num_envs)
        native.check(self.lib.nanorts_amd_gridnet_observe(_stream(), self.dev.ref, state.native(), state.num_envs, struct),
                     "nanorts_amd_gridnet_observe")
        return obs

    def planes(self, state: EnvironmentState) -> torch.Tensor:
        """observation.planes (src/nanorts/adapters/gridnet/observation.py:36-51)."""
        y = self.layout
        planes = torch.empty((state.num_envs, *y.planes_shape), dtype=y.planes_dtype, device=self.device)
        struct = self._obs_struct(planes, None, None)
        native.check(self.lib.nanorts_amd_gridnet_observe(_stream(), self.dev.ref, state.native(), state.num_envs, struct),
                     "nanorts_amd_gridnet_observe")
        return planes

    def decode_actions(self, actions: torch.Tensor, state: EnvironmentState) -> dict[str, torch.Tensor]:
        """actions.decode_actions (src/nanorts/adapters/gridnet/actions.py:31-52):
        int32[L, 2, H, W, 7] -> Commands, int32[L, 2, C] per field."""
        L = state.num_envs
        acts = self._actions(actions, L, PLAYER_COUNT)
        out = {f: torch.empty((L, PLAYER_COUNT, self.game.bucket.per_player_capacity), dtype=torch.int32,
                              device=self.device) for f in _COMMAND_FIELDS}
        bufs = native.Commands(*[_ptr(out[f]) for f in _COMMAND_FIELDS])
        native.check(self.lib.nanorts_amd_gridnet_decode(_stream(), self.dev.ref, state.native(), L, _ptr(acts), bufs),
                     "nanorts_amd_gridnet_decode")
        return out

    def sample_actions(self, action_mask: torch.Tensor, sample_key, step: int, env0: int = 0) -> torch.Tensor:
        """The synthetic harness's integer uniform-over-legal sampler on the
        packed action mask [L, 2, H, W, 3]: per-cell actions int32[L, 2, H, W, 7]
        (cells without a source draw zeros)."""
        if self.layout.mask_form != "packed":
            raise ModelError("GridNet.sample_actions reads the packed action mask: prepare(..., mask_form='packed')")
        mask = action_mask.contiguous()
        L = mask.shape[0]
        b = self.game.bucket
        if tuple(mask.shape) != (L, *self.layout.mask_shape):
            raise ModelError(f"the action mask has shape {tuple(mask.shape)}, expected {(L, *self.layout.mask_shape)}")
        key = (ctypes.c_uint32 * 2)(*[int(v) for v in np.asarray(sample_key, np.uint32).reshape(2)])
        actions = torch.empty((L, PLAYER_COUNT, b.height, b.width, len(ACTION_FACTORS)), dtype=torch.int32,
                              device=self.device)
        native.check(self.lib.nanorts_amd_gridnet_sample_actions(_stream(), self.dev.ref, L, _ptr(mask), key, int(step),
                                                             int(env0), _ptr(actions)),
                     "nanorts_amd_gridnet_sample_actions")
        return actions

    def step(self, state: EnvironmentState, actions: torch.Tensor, *, donate: bool = False) -> GridNetStep:
        """env.step (src/nanorts/adapters/gridnet/env.py:65-70); with
        donate=True the input state's buffers are updated in place."""
        nxt = state if donate else state.clone()
        acts = self._actions(actions, nxt.num_envs, PLAYER_COUNT)
        return self._step(nxt, acts, None)

    def step_against(self, state: EnvironmentState, actions: torch.Tensor, commands: dict[str, torch.Tensor], *,
                     donate: bool = False) -> GridNetStep:
        """env.step_against (src/nanorts/adapters/gridnet/env.py:73-83): player 0
        plays the per-cell actions int32[L, H, W, 7], player 1 the given
        Commands ([L, 2, C] per field; player 0's rows are not read)."""
        nxt = state if donate else state.clone()
        acts = self._actions(actions, nxt.num_envs, 1)
        given = {f: commands[f].to(device=self.device, dtype=torch.int32).contiguous() for f in _COMMAND_FIELDS}
        return self._step(nxt, acts, given)

    # -------------------------------------------------------------- helpers
    def _actions(self, actions: torch.Tensor, L: int, players: int) -> torch.Tensor:
        b = self.game.bucket
        want = (L, *((PLAYER_COUNT,) if players == PLAYER_COUNT else ()), b.height, b.width, len(ACTION_FACTORS))
        acts = torch.as_tensor(actions, device=self.device)
        if tuple(acts.shape) != want:
            raise ModelError(f"gridnet actions have shape {tuple(acts.shape)}, expected {want}")
        if acts.dtype != torch.int32:
            raise ModelError(f"gridnet actions have dtype {acts.dtype}, expected int32")
        return acts.contiguous()

    def _step(self, nxt: EnvironmentState, acts: torch.Tensor, given: dict[str, torch.Tensor] | None) -> GridNetStep:
        L, d, y = nxt.num_envs, self.device, self.layout
        comps = torch.empty((L, PLAYER_COUNT, len(REWARD_COMPONENTS)), dtype=torch.float32, device=d)
        rdones = torch.empty((L, PLAYER_COUNT, len(REWARD_COMPONENTS)), dtype=torch.bool, device=d)
        flags = {k: torch.empty(L, dtype=torch.bool, device=d)
                 for k in ("terminated", "truncated", "done", "spawn_overflowed")}
        winner = torch.empty(L, dtype=torch.int32, device=d)
        telemetry = torch.empty((L, PLAYER_COUNT), dtype=torch.int32, device=d)
        final = torch.empty((L, *y.planes_shape), dtype=y.planes_dtype, device=d)
        obs, struct = self._obs_buffers(L)
        results = native.GridNetResults(_ptr(comps), _ptr(rdones), _ptr(flags["terminated"]), _ptr(flags["truncated"]),
                                        _ptr(flags["done"]), _ptr(winner), _ptr(flags["spawn_overflowed"]),
                                        _ptr(final), struct, _ptr(telemetry))
        if given is None:
            code = self.lib.nanorts_amd_gridnet_step(_stream(), self.dev.ref, nxt.native(), L, _ptr(acts), results)
            native.check(code, "nanorts_amd_gridnet_step")
        else:
            c = native.Commands(*[_ptr(given[f]) for f in _COMMAND_FIELDS])
            code = self.lib.nanorts_amd_gridnet_step_against(_stream(), self.dev.ref, nxt.native(), L, _ptr(acts), c,
                                                         results)
            native.check(code, "nanorts_amd_gridnet_step_against")
        return GridNetStep(environment_state=nxt, observation=obs, reward_components=comps, reward_dones=rdones,
                           terminated=flags["terminated"], truncated=flags["truncated"], done=flags["done"],
                           winner=winner, telemetry={"spawn_overflow": telemetry},
                           spawn_overflowed=flags["spawn_overflowed"], final_observation=final,
                           final_valid=flags["done"])


def check_actions(actions: Any, *, layout: GridNetLayout) -> None:
    """actions.check_actions (src/nanorts/adapters/gridnet/actions.py:55-71)
    for one env's int32[2, H, W, 7] (or a batch with leading dimensions)."""
    array = np.asarray(actions.cpu() if isinstance(actions, torch.Tensor) else actions)
    if array.shape[-4:] != layout.actions_shape:
        raise ModelError(f"gridnet actions have shape {array.shape}, expected {layout.actions_shape} - the leading "
                         f"{PLAYER_COUNT} is player identity, not an environment batch")
    if array.dtype != np.int32:
        raise ModelError(f"gridnet actions have dtype {array.dtype}, expected int32")
    for index, (name, size) in enumerate(zip(ACTION_FACTORS, layout.action_factor_sizes, strict=True)):
        factor = array[..., index]
        if factor.size and (factor.min() < 0 or factor.max() >= size):
            raise ModelError(f"gridnet action factor {index} ({name}) carries values in [{int(factor.min())}, "
                             f"{int(factor.max())}], expected [0, {size - 1}]; every factor obeys its range including "
                             "an unused one and one at a non-source cell")


def unpack_mask(action_mask: torch.Tensor, *, layout: GridNetLayout) -> torch.Tensor:
    """observation.unpack_mask (src/nanorts/adapters/gridnet/observation.py:75-78):
    bool rows [..., 78] from either form."""
    if layout.mask_form != "packed":
        return action_mask != 0
    head = sum(layout.action_factor_sizes[:-1])
    shifts = torch.arange(32, device=action_mask.device, dtype=torch.int32)
    bits = ((action_mask.to(torch.int32)[..., None] >> shifts) & 1) != 0
    bits = bits.reshape(*action_mask.shape[:-1], MASK_WORDS * 32)
    return torch.cat([bits[..., :head], bits[..., 32:32 + layout.action_factor_sizes[-1]]], dim=-1)


# ---------------------------------------------------------------------------
# The learner-vs-bot seat and the mix on the GridNet surface
# (src/nanorts/bots/gridnet_seat.py): the learner is player 0, the bot
# player 1; a step is the bot's act on a copy of its carry, then step_against
# (one launch each), and the carry is emptied where the game ended.
# ---------------------------------------------------------------------------
@dataclasses.dataclass
class GridNetSeatState:
    """src/nanorts/bots/gridnet_seat.py:20-26"""

    environment_state: EnvironmentState
    carry: dict[str, torch.Tensor]


@dataclasses.dataclass(frozen=True)
class GridNetSeatStep:
    """src/nanorts/bots/gridnet_seat.py:28-53: the learner's rows."""

    seat_state: GridNetSeatState
    observation: GridNetObservation
    reward_components: torch.Tensor  # float32[L, 6]
    reward_dones: torch.Tensor       # bool[L, 6]
    terminated: torch.Tensor
    truncated: torch.Tensor
    done: torch.Tensor
    winner: torch.Tensor
    telemetry: dict[str, torch.Tensor]
    spawn_overflowed: torch.Tensor
    final_observation: torch.Tensor
    final_valid: torch.Tensor


LEARNER_PLAYER: Final = 0
BOT_PLAYER: Final = 1


def _learner(obs: GridNetObservation) -> GridNetObservation:
    return GridNetObservation(obs.planes[:, LEARNER_PLAYER], obs.source_mask[:, LEARNER_PLAYER],
                              obs.action_mask[:, LEARNER_PLAYER])


class GridNetSeat:
    """reset_gridnet_seat / step_gridnet_seat / gridnet_seat_commands
    (src/nanorts/bots/gridnet_seat.py:56-95) with `bot` and `game` bound."""

    def __init__(self, bot, game: GameConfig, layout: GridNetLayout | None = None, *,
                 device: str | torch.device | None = None):
        from nanorts_amd import bots

        if bot.strategy not in (bots.WORKER_RUSH, bots.BARRACKS_RUSH):
            raise ModelError(f"bot {bot.name!r} is not available here; the seat plays WorkerRush or LightRush")
        self.bot = bot
        self.grid = GridNet(game, layout, device=device)
        self.game = game
        self.layout = self.grid.layout
        self.device = self.grid.device

    def reset(self, environment_root) -> tuple[GridNetSeatState, GridNetObservation]:
        from nanorts_amd import bots

        state, obs = self.grid.reset(environment_root)
        carry = bots.empty_actions(state.num_envs, self.game.bucket.per_player_capacity, self.device)
        return GridNetSeatState(state, carry), _learner(obs)

    def commands(self, seat_state: GridNetSeatState) -> tuple[dict[str, torch.Tensor], dict[str, torch.Tensor]]:
        """gridnet_seat_commands: (the bot's new carry, its Commands [L, 2, C]
        per field); the seat state's carry is left as it is."""
        from nanorts_amd import bots

        carry = {k: v.clone() for k, v in seat_state.carry.items()}
        cmds = bots.abstraction_act(self.grid, seat_state.environment_state, carry, self.bot, BOT_PLAYER)
        return carry, cmds

    def step(self, seat_state: GridNetSeatState, actions: torch.Tensor, *, donate: bool = False) -> GridNetSeatStep:
        """step_gridnet_seat: the learner's per-cell actions int32[L, H, W, 7]."""
        from nanorts_amd import bots

        carry, cmds = self.commands(seat_state)
        out = self.grid.step_against(seat_state.environment_state, actions, cmds, donate=donate)
        fresh = bots.empty_actions(out.environment_state.num_envs, self.game.bucket.per_player_capacity, self.device)
        carry = {k: torch.where(out.done.reshape((-1,) + (1,) * (v.dim() - 1)), fresh[k], v) for k, v in carry.items()}
        p = LEARNER_PLAYER
        return GridNetSeatStep(seat_state=GridNetSeatState(out.environment_state, carry),
                               observation=_learner(out.observation),
                               reward_components=out.reward_components[:, p], reward_dones=out.reward_dones[:, p],
                               terminated=out.terminated, truncated=out.truncated, done=out.done, winner=out.winner,
                               telemetry=out.telemetry, spawn_overflowed=out.spawn_overflowed,
                               final_observation=out.final_observation[:, p], final_valid=out.final_valid)


@dataclasses.dataclass(frozen=True)
class GridNetGroup:
    """src/nanorts/bots/gridnet_seat.py:98-101"""

    bot: Any
    lanes: int


@dataclasses.dataclass
class GridNetMixState:
    """src/nanorts/bots/gridnet_seat.py:104-109"""

    self_play: EnvironmentState | None
    seats: tuple[GridNetSeatState, ...]


_MIX_FIELDS: Final = ("observation", "reward_components", "reward_dones", "terminated", "truncated", "done", "winner",
                      "telemetry", "spawn_overflowed", "final_observation", "final_valid")


@dataclasses.dataclass(frozen=True)
class GridNetMixStep:
    """src/nanorts/bots/gridnet_seat.py:112-127: one row per self-play player
    (game-major) and one per seat lane, in that order."""

    mix_state: GridNetMixState
    observation: GridNetObservation
    reward_components: torch.Tensor
    reward_dones: torch.Tensor
    terminated: torch.Tensor
    truncated: torch.Tensor
    done: torch.Tensor
    winner: torch.Tensor
    telemetry: dict[str, torch.Tensor]
    spawn_overflowed: torch.Tensor
    final_observation: torch.Tensor
    final_valid: torch.Tensor


def _rows_of_games(tree):
    """[L, 2, ...] -> [2L, ...], game-major."""
    if isinstance(tree, torch.Tensor):
        return tree.reshape(tree.shape[0] * PLAYER_COUNT, *tree.shape[2:])
    if isinstance(tree, dict):
        return {k: _rows_of_games(v) for k, v in tree.items()}
    return type(tree)(*[_rows_of_games(getattr(tree, f.name)) for f in dataclasses.fields(tree)])


def _rows_of_lanes(tree):
    """[L, ...] -> [2L, ...], each lane's value for both of its players."""
    if isinstance(tree, torch.Tensor):
        return torch.repeat_interleave(tree, PLAYER_COUNT, dim=0)
    return {k: _rows_of_lanes(v) for k, v in tree.items()}


def _joined(parts):
    first = parts[0]
    if isinstance(first, torch.Tensor):
        return torch.cat(parts)
    if isinstance(first, dict):
        return {k: _joined([p[k] for p in parts]) for k in first}
    return type(first)(*[_joined([getattr(p, f.name) for p in parts]) for f in dataclasses.fields(first)])


class GridNetMix:
    """src/nanorts/bots/gridnet_seat.py:130-214: `self_play` self-play games
    and learner-vs-bot groups on one GridNet game and layout."""

    def __init__(self, self_play: int, groups, game: GameConfig, layout: GridNetLayout | None = None, *,
                 device: str | torch.device | None = None):
        self.groups = tuple(groups)
        if not isinstance(self_play, int) or isinstance(self_play, bool) or self_play < 0:
            raise ModelError(f"self_play={self_play!r} should be the number of self-play games (an int)")
        for index, group in enumerate(self.groups):
            if not isinstance(group.lanes, int) or isinstance(group.lanes, bool) or group.lanes < 1:
                raise ModelError(f"group {index} asks for lanes={group.lanes!r}; give a positive int")
            if not hasattr(group.bot, "strategy"):
                raise ModelError(f"group {index} holds no scripted Bot")
        self.self_play = self_play
        if self.lanes == 0:
            raise ModelError("the mix has no games in it")
        self.grid = GridNet(game, layout, device=device)
        self.seats = tuple(GridNetSeat(group.bot, game, self.grid.layout, device=device) for group in self.groups)

    @property
    def lanes(self) -> int:
        return self.self_play + sum(group.lanes for group in self.groups)

    @property
    def rows(self) -> int:
        return PLAYER_COUNT * self.self_play + sum(group.lanes for group in self.groups)

    def slices(self) -> tuple[slice, ...]:
        sizes = ([PLAYER_COUNT * self.self_play] if self.self_play else []) + [g.lanes for g in self.groups]
        out, start = [], 0
        for size in sizes:
            out.append(slice(start, start + size))
            start += size
        return tuple(out)

    def reset(self, roots) -> tuple[GridNetMixState, GridNetObservation]:
        roots = np.asarray(roots.cpu() if isinstance(roots, torch.Tensor) else roots, np.uint32).reshape(-1, 2)
        if roots.shape[0] != self.lanes:
            raise ModelError(f"GridNetMix.reset takes {self.lanes} roots, got {roots.shape[0]}")
        rows, start, self_play, seats = [], 0, None, []
        if self.self_play:
            self_play, obs = self.grid.reset(roots[:self.self_play])
            rows.append(_rows_of_games(obs))
            start = self.self_play
        for group, seat in zip(self.groups, self.seats, strict=True):
            state, obs = seat.reset(roots[start:start + group.lanes])
            seats.append(state)
            rows.append(obs)
            start += group.lanes
        return GridNetMixState(self_play, tuple(seats)), _joined(rows)

    def step(self, mix_state: GridNetMixState, actions: torch.Tensor, *, donate: bool = False) -> GridNetMixStep:
        """Per-cell actions int32[rows, H, W, 7], one row per slice row."""
        if actions.shape[0] != self.rows:
            raise ModelError(f"GridNetMix.step takes {self.rows} action rows, got {actions.shape[0]}")
        bounds = list(self.slices())
        rows, self_play, seats = [], None, []
        if self.self_play:
            grids = actions[bounds.pop(0)].reshape(self.self_play, PLAYER_COUNT, *actions.shape[1:])
            out = self.grid.step(mix_state.self_play, grids, donate=donate)
            self_play = out.environment_state
            rows.append({"observation": _rows_of_games(out.observation),
                         "reward_components": _rows_of_games(out.reward_components),
                         "reward_dones": _rows_of_games(out.reward_dones),
                         "terminated": _rows_of_lanes(out.terminated), "truncated": _rows_of_lanes(out.truncated),
                         "done": _rows_of_lanes(out.done), "winner": _rows_of_lanes(out.winner),
                         "telemetry": _rows_of_lanes(out.telemetry),
                         "spawn_overflowed": _rows_of_lanes(out.spawn_overflowed),
                         "final_observation": _rows_of_games(out.final_observation),
                         "final_valid": _rows_of_lanes(out.final_valid)})
        for seat, state, bound in zip(self.seats, mix_state.seats, bounds, strict=True):
            out = seat.step(state, actions[bound], donate=donate)
            seats.append(out.seat_state)
            rows.append({name: getattr(out, name) for name in _MIX_FIELDS})
        joined = _joined(rows)
        return GridNetMixStep(mix_state=GridNetMixState(self_play, tuple(seats)), **joined)
