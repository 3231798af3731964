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
        raise ModelError(f"gridnet.prepare refuses {keyword}={dtype!r}: the Planes and the action mask publish one of "
                         "['int32', 'uint8', 'bool'], each holding the surface's 0/1 values, with int32 the pinned "
                         "MicroRTS-Py default")
    return found


def prepare(game: GameConfig, *, partial_observability: bool = False, planes_form: str = "one_hot",
            planes_dtype: Any = torch.int32, mask_form: str = "rows", mask_dtype: Any = torch.int32) -> GridNetLayout:
    """src/nanorts/adapters/gridnet/layout.py:111-141 with its refusals (:144-231)."""
    if partial_observability is not False:
        raise ModelError(f"gridnet.prepare refuses partial_observability={partial_observability!r}: MicroRTS-Py's "
                         "31-plane partial-observation form is outside the supported release matrix")
    bucket = game.bucket
    if bucket.unit_type_capacity != PLANE_WIDTHS[3] - 1:
        raise ModelError(f"gridnet.prepare refuses BucketSpec.unit_type_capacity {bucket.unit_type_capacity}: the "
                         f"pinned surface's type Plane group is {PLANE_WIDTHS[3]} wide and its produce-type factor "
                         f"{ACTION_FACTOR_SIZES[5]} wide")
    if bucket.attack_offset_capacity != ACTION_FACTOR_SIZES[6]:
        raise ModelError(f"gridnet.prepare refuses BucketSpec.attack_offset_capacity {bucket.attack_offset_capacity}: "
                         f"the pinned attack window is {ACTION_FACTOR_SIZES[6]}")
    if planes_form not in PLANE_FORMS:
        raise ModelError(f"gridnet.prepare refuses planes_form={planes_form!r}: the Planes publish one of "
                         f"{list(PLANE_FORMS)}")
    if mask_form not in MASK_FORMS:
        raise ModelError(f"gridnet.prepare refuses mask_form={mask_form!r}: the action mask publishes one of "
                         f"{list(MASK_FORMS)}")
    planes = _dtype("planes_dtype", planes_dtype)
    mask = _dtype("mask_dtype", mask_dtype)
    if planes_form == "indices":
        if planes != torch.int32:
            raise ModelError(f"gridnet.prepare refuses planes_dtype={planes_dtype!r} beside planes_form='indices': the "
                             "indices form publishes int8 Plane indices")
        planes = PLANE_INDEX_DTYPE
    if mask_form == "packed":
        if mask != torch.int32:
            raise ModelError(f"gridnet.prepare refuses mask_dtype={mask_dtype!r} beside mask_form='packed': the packed "
                             "form publishes uint32 words")
        mask = MASK_WORD_DTYPE
    if bool(game.initial_state["game_over"]):
        raise ModelError("gridnet.prepare refuses a configuration whose initial State is already decided: a public "
                         "environment steps only a playable State")
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
        native.check(self.lib.nanorts_gridnet_observe(_stream(), self.dev.ref, state.native(), state.num_envs, struct),
                     "nanorts_gridnet_observe")
        return obs

    def planes(self, state: EnvironmentState) -> torch.Tensor:
        """observation.planes (src/nanorts/adapters/gridnet/observation.py:36-51)."""
        y = self.layout
        planes = torch.empty((state.num_envs, *y.planes_shape), dtype=y.planes_dtype, device=self.device)
        struct = self._obs_struct(planes, None, None)
        native.check(self.lib.nanorts_gridnet_observe(_stream(), self.dev.ref, state.native(), state.num_envs, struct),
                     "nanorts_gridnet_observe")
        return planes

    def decode_actions(self, actions: torch.Tensor, state: EnvironmentState) -> dict[str, torch.Tensor]:
        """actions.decode_actions (src/nanorts/adapters/gridnet/actions.py:31-52):
        int32[L, 2, H, W, 7] -> Commands, int32[L, 2, C] per field."""
        L = state.num_envs
        acts = self._actions(actions, L, PLAYER_COUNT)
        out = {f: torch.empty((L, PLAYER_COUNT, self.game.bucket.per_player_capacity), dtype=torch.int32,
                              device=self.device) for f in _COMMAND_FIELDS}
        bufs = native.Commands(*[_ptr(out[f]) for f in _COMMAND_FIELDS])
        native.check(self.lib.nanorts_gridnet_decode(_stream(), self.dev.ref, state.native(), L, _ptr(acts), bufs),
                     "nanorts_gridnet_decode")
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
        native.check(self.lib.nanorts_gridnet_sample_actions(_stream(), self.dev.ref, L, _ptr(mask), key, int(step),
                                                             int(env0), _ptr(actions)),
                     "nanorts_gridnet_sample_actions")
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
            code = self.lib.nanorts_gridnet_step(_stream(), self.dev.ref, nxt.native(), L, _ptr(acts), results)
            native.check(code, "nanorts_gridnet_step")
        else:
            c = native.Commands(*[_ptr(given[f]) for f in _COMMAND_FIELDS])
            code = self.lib.nanorts_gridnet_step_against(_stream(), self.dev.ref, nxt.native(), L, _ptr(acts), c,
                                                         results)
            native.check(code, "nanorts_gridnet_step_against")
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
