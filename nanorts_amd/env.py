"""The JaxMARL-shaped NanoRTS facade over the gfx950 kernels.

Mirrors src/nanorts/adapters/jaxmarl/facade.py:43-268 and env.py:64-184 of the
reference: `make`, `reset`, `step`, `get_avail_actions`, `get_slot_cells`,
`get_obs`, int32[C, 7] action rows, uint8[H, W, 6] feature maps and int32[4]
scalars per agent, rewards, dones and infos.  The reference applies these to
one env and is vmapped; here every call is batched over a leading env
dimension L (what jax.vmap(env.step) returns), and each call is one kernel
launch on the current HIP stream.  Tensors are torch tensors on the GPU.
"""
from __future__ import annotations

import ctypes
import dataclasses
from typing import Any, Final

import numpy as np
import torch

from nanorts_amd import keys as _keys
from nanorts_amd import native
from nanorts_amd.content import GameConfig, with_unit_type_table
from nanorts_amd.model import (
    ACTION_KIND_COUNT,
    DIRECTION_COUNT,
    KIND_NONE,
    PLAYER_COUNT,
    STATE_LEAVES,
    STRATEGY_CODES,
    ModelError,
    UnitTypeTableVersion,
    leaf_shape,
)

AGENTS: Final = tuple(f"player_{p}" for p in range(PLAYER_COUNT))
ALL_AGENTS: Final = "__all__"
ENVIRONMENT_IDS: Final = ("NanoRTS",)
SURFACES: Final = ("symbolic", "pixels")
ACTION_FACTORS: Final = ("kind", "move_direction", "harvest_direction", "return_direction", "produce_direction",
                         "produce_type", "attack_offset")
REWARD_COMPONENTS: Final = ("win_loss", "resource_gather", "produce_worker", "produce_building", "attack",
                            "produce_combat_unit")
NONE_DURATION: Final = 1

_TORCH_DTYPES = {np.dtype(np.int32): torch.int32, np.dtype(np.int16): torch.int16, np.dtype(np.int8): torch.int8,
                 np.dtype(np.bool_): torch.bool, np.dtype(np.uint8): torch.uint8}


def _ptr(t: torch.Tensor | None) -> int | None:
    if t is None:
        return None
    if not t.is_contiguous():
        raise ModelError("kernel operands must be contiguous")
    return t.data_ptr()


# The feature-map dtypes the reference publishes
# (src/nanorts/observations/symbolic.py:48-52), narrowest last.
FEATURE_MAP_DTYPES: Final = (torch.int32, torch.int16, torch.uint8)
_BYTE_CEILING: Final = 255


def feature_bounds(game: GameConfig) -> dict[str, int]:
    """The largest value each feature-map group can take for this content
    (src/nanorts/observations/symbolic.py:186-199): hit points and carried
    resources from the unit table and the initial units, the rest from the
    vocabulary and the bucket."""
    cols, start = game.columns, game.initial_state
    return {
        "hit_points": max(int(cols["hit_points"].max()), int(start["hit_points"].max())),
        "carried_resources": max(int(cols["harvest_amount"].max()), int(start["carried_resources"].max())),
        "owner": PLAYER_COUNT,
        "unit_type": game.bucket.unit_type_capacity,
        "pending_action_kind": ACTION_KIND_COUNT - 1,
        "terrain": 1,
    }


def _as_feature_dtype(value: Any) -> torch.dtype | None:
    if isinstance(value, torch.dtype):
        return value if value in FEATURE_MAP_DTYPES else None
    try:
        name = np.dtype(value).name
    except TypeError:
        return None
    return {"int32": torch.int32, "int16": torch.int16, "uint8": torch.uint8}.get(name)


def feature_dtype(game: GameConfig, requested: Any = None) -> torch.dtype:
    """The published feature-map dtype: `requested`, or the narrowest of
    FEATURE_MAP_DTYPES whose range holds every bound of the content
    (src/nanorts/adapters/jaxmarl/layout.py:146-158).  The kernels encode one
    byte per feature, so content with a bound above 255 is refused here;
    wider published dtypes are exact widenings of those bytes."""
    bounds = feature_bounds(game)
    largest = max(bounds.values())
    if requested is None:
        chosen = next(t for t in reversed(FEATURE_MAP_DTYPES) if torch.iinfo(t).max >= largest)
    else:
        chosen = _as_feature_dtype(requested)
        if chosen is None:
            raise ModelError(f"feature_dtype {requested!r} is not one of the published feature-map dtypes "
                             f"{[str(t).removeprefix('torch.') for t in FEATURE_MAP_DTYPES]}")
        too_big = {name: bound for name, bound in bounds.items() if bound > torch.iinfo(chosen).max}
        if too_big:
            raise ModelError(f"feature_dtype {requested!r} cannot hold this content's feature values: {too_big}")
    if largest > _BYTE_CEILING:
        wide = {name: bound for name, bound in bounds.items() if bound > _BYTE_CEILING}
        raise ModelError(f"this content has feature values above {_BYTE_CEILING} ({wide}); the observation "
                         "kernels encode one byte per feature, so such content is refused rather than wrapped")
    return chosen


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


@dataclasses.dataclass
class State:
    """The State leaves of L envs (src/nanorts/model/state.py:33-84), each a
    torch tensor with a leading env dimension."""

    leaves: dict[str, torch.Tensor]

    def __getattr__(self, name: str) -> torch.Tensor:
        leaves = self.__dict__.get("leaves")
        if leaves is not None and name in leaves:
            return leaves[name]
        raise AttributeError(name)

    @property
    def active(self) -> torch.Tensor:
        return self.leaves["birth"] != -1

    def clone(self) -> "State":
        return State({k: v.clone() for k, v in self.leaves.items()})

    def numpy(self) -> dict[str, np.ndarray]:
        return {k: v.cpu().numpy() for k, v in self.leaves.items()}


@dataclasses.dataclass
class EnvironmentState:
    """src/nanorts/adapters/lifecycle.py:24-31.  `environment_root` holds the
    uint32 key data [L, 2] and `episode_index` the uint32 counter [L], both
    stored bit-for-bit in int32 tensors."""

    core_state: State
    environment_root: torch.Tensor
    episode_index: torch.Tensor

    @property
    def num_envs(self) -> int:
        return int(self.environment_root.shape[0])

    def clone(self) -> "EnvironmentState":
        return EnvironmentState(self.core_state.clone(), self.environment_root.clone(), self.episode_index.clone())

    def native(self) -> native.State:
        leaves = self.core_state.leaves
        return native.State(*[_ptr(leaves[name]) for name in native.STATE_FIELDS[:-2]],
                            _ptr(self.environment_root), _ptr(self.episode_index))


@dataclasses.dataclass(frozen=True)
class SymbolicObservation:
    feature_maps: torch.Tensor  # uint8[L, H, W, 6]
    scalars: torch.Tensor       # int32[L, 4]


@dataclasses.dataclass(frozen=True)
class PixelObservation:
    image: torch.Tensor         # uint8[L, 16H, 16W, 3]
    scalars: torch.Tensor       # int32[L, 4]


@dataclasses.dataclass(frozen=True)
class JaxMARLLayout:
    """src/nanorts/adapters/jaxmarl/layout.py:34-67"""

    surface: str
    partial_observability: bool
    action_factors: tuple[str, ...]
    action_widths: tuple[int, ...]
    mask_offsets: tuple[int, ...]
    mask_width: int
    actions_shape: tuple[int, int]
    feature_maps_shape: tuple[int, int, int]
    final_observation: bool
    reward_components: bool

    @property
    def agents(self) -> tuple[str, ...]:
        return AGENTS


def _components(stepped: dict[str, torch.Tensor], over: torch.Tensor, winner: torch.Tensor) -> torch.Tensor:
    """encode_components (src/nanorts/adapters/rewards.py:47-71) from a
    core.step result's event counts and the ending state's game_over and
    winner: float32[L, 2, 6]."""
    prod, att = stepped["admitted_produce"], stepped["admitted_attack"]
    L = prod.shape[0]
    out = torch.zeros((L, 2, 6), dtype=torch.float32, device=prod.device)
    for p in range(2):
        o = 1 - p
        out[:, p, 1] = (stepped["admitted_harvest"][:, p] + stepped["admitted_return"][:, p]).float()
        out[:, p, 2] = prod[:, p, 3].float()
        out[:, p, 3] = (prod[:, p, 1] + prod[:, p, 2]).float()
        out[:, p, 4] = (att[:, p, o + 1] - att[:, p, p + 1]).float()
        out[:, p, 5] = (prod[:, p, 4] + prod[:, p, 5] + prod[:, p, 6]).float()
        out[:, p, 0] = torch.where(over, torch.where(winner == p, 1.0, -1.0), 0.0)
    return out


class DeviceGame:
    """The static game on the device: the native game struct, terrain and the
    decided initial State of one env."""

    def __init__(self, game: GameConfig, device: torch.device):
        bucket = game.bucket
        self.game = game
        self.device = device
        self.terrain = torch.as_tensor(game.terrain.reshape(-1).astype(np.uint8), device=device)
        # np.array keeps 0-d leaves 0-d (ascontiguousarray would make them
        # 1-d), so a batch of L envs has scalar leaves of shape [L]
        self.initial = {leaf.name: torch.as_tensor(np.array(game.initial_state[leaf.name], order="C")[None],
                                                   device=device) for leaf in STATE_LEAVES}
        cols = game.columns
        g = native.Game()
        g.height, g.width, g.cells = bucket.height, bucket.width, bucket.cell_count
        g.neutral, g.capacity, g.entities = bucket.neutral_capacity, bucket.per_player_capacity, bucket.entity_capacity
        g.types, g.offsets = bucket.unit_type_capacity, bucket.attack_offset_capacity
        g.strategy = STRATEGY_CODES[bucket.conflict_strategy]
        g.max_cycles = game.max_cycles
        T = bucket.unit_type_capacity
        for name in ("cost", "hit_points", "produce_time", "move_time", "attack_time", "harvest_time",
                     "attack_range", "attack_damage", "harvest_amount", "sight_radius", "is_resource",
                     "is_stockpile", "can_harvest", "can_move", "can_attack"):
            arr = getattr(g, name)
            for t in range(T):
                arr[t] = int(cols[name][t])
        for p in range(T):
            for q in range(T):
                g.produces[p * native.MAX_TYPES + q] = int(cols["produces"][p, q])
        g.terrain = _ptr(self.terrain)
        g.initial = native.State(*[_ptr(self.initial[name]) for name in native.STATE_FIELDS[:-2]], None, None)
        self.struct = g
        self.ref = ctypes.byref(g)

    def batch(self, num_envs: int) -> State:
        return State({name: t.expand(num_envs, *t.shape[1:]).contiguous() for name, t in self.initial.items()})


def make(env_id: str, *, scenario: GameConfig, utt: UnitTypeTableVersion | None = None, surface: str = "symbolic",
         partial_observability: bool = False, final_observation: bool = True, feature_dtype: Any = None,
         reward_components: bool = False, device: str | torch.device | None = None, assets: Any = None) -> "NanoRTS":
    """src/nanorts/adapters/jaxmarl/facade.py:43-56"""
    if env_id not in ENVIRONMENT_IDS:
        raise ModelError(f"there is no environment called {env_id!r}; this package registers {list(ENVIRONMENT_IDS)}")
    game = scenario if utt is None else with_unit_type_table(scenario, utt)
    return NanoRTS(game, surface=surface, partial_observability=partial_observability,
                   final_observation=final_observation, feature_dtype=feature_dtype,
                   reward_components=reward_components, device=device, assets=assets)


def feature_dtype_for_surface(game: GameConfig, surface: str, requested: Any) -> torch.dtype:
    """feature_dtype on the symbolic surface; the pixel surface publishes
    uint8 images whatever the content (its glyphs draw bytes too), so the
    bounds are checked there as well."""
    chosen = feature_dtype(game, None if surface == "pixels" else requested)
    return torch.uint8 if surface == "pixels" else chosen


class NanoRTS:
    """Two-player NanoRTS over L envs at once (src/nanorts/adapters/jaxmarl/facade.py:59-225)."""

    def __init__(self, scenario: GameConfig, *, surface: str = "symbolic", partial_observability: bool = False,
                 final_observation: bool = True, feature_dtype: Any = None, reward_components: bool = False,
                 device: str | torch.device | None = None, assets: Any = None):
        if surface not in SURFACES:
            raise ModelError(f"surface={surface!r} is unknown; choose one of {list(SURFACES)}")
        if surface == "pixels" and feature_dtype is not None and _as_feature_dtype(feature_dtype) != torch.int32:
            raise ModelError(f"feature_dtype={feature_dtype!r} has no meaning on the pixel surface, which publishes "
                             "an image and no feature maps")
        for name, flag in (("partial_observability", partial_observability), ("final_observation", final_observation),
                           ("reward_components", reward_components)):
            if not isinstance(flag, bool):
                raise ModelError(f"{name} must be True or False, not {flag!r}")
        if bool(scenario.initial_state["game_over"]):
            raise ModelError("this content's starting position is already won or drawn, so there is no game to step")
        published = feature_dtype_for_surface(scenario, surface, feature_dtype)
        self.lib = native.load()
        self.device = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
        self.game = scenario
        self.bucket = scenario.bucket
        self.dev = DeviceGame(scenario, self.device)
        self.agents = list(AGENTS)
        self.num_agents = PLAYER_COUNT
        b = self.bucket
        widths = (ACTION_KIND_COUNT, DIRECTION_COUNT, DIRECTION_COUNT, DIRECTION_COUNT, DIRECTION_COUNT,
                  b.unit_type_capacity, b.attack_offset_capacity)
        offsets = tuple(int(v) for v in np.cumsum((0,) + widths[:-1]))
        self.layout = JaxMARLLayout(surface=surface, partial_observability=partial_observability,
                                    action_factors=ACTION_FACTORS, action_widths=widths, mask_offsets=offsets,
                                    mask_width=int(sum(widths)), actions_shape=(b.per_player_capacity, 7),
                                    feature_maps_shape=(b.height, b.width, 6), final_observation=final_observation,
                                    reward_components=reward_components)
        self.final_observation = final_observation
        self.partial = int(partial_observability)
        self.feature_dtype = published
        self._tiles: torch.Tensor | None = None
        # the drawing table (src/nanorts/adapters/jaxmarl/layout.py:168-205):
        # none under the symbolic surface; under the pixel surface the shipped
        # sprite sheet unless an Asset set of 16-pixel cells is given
        if surface == "symbolic" and assets is not None:
            raise ModelError(f"assets ({type(assets).__name__}) only apply to surface='pixels'; the symbolic surface draws "
                             "no images")
        if surface == "pixels":
            from nanorts_amd import rendering

            if assets is None:
                table = rendering.tile_table(b.unit_type_capacity)
            else:
                if assets.cell_pixels != rendering.SPRITE_PIXELS:
                    raise ModelError(f"the pixel surface draws {rendering.SPRITE_PIXELS}-pixel cells; these assets were "
                                     f"prepared for {assets.cell_pixels}")
                if assets.unit_type_capacity != b.unit_type_capacity:
                    raise ModelError(f"these assets draw {assets.unit_type_capacity} unit types; the game has "
                                     f"{b.unit_type_capacity}")
                table = np.ascontiguousarray(assets.tiles, np.uint8)
            self._tiles = torch.as_tensor(table, device=self.device)

    # ------------------------------------------------------------------ API
    def reset(self, key) -> tuple[dict[str, Any], EnvironmentState]:
        """jax.vmap(env.reset)(keys): `key` is uint32 key data [L, 2]; every
        env starts from the decided initial state and keeps its key as the
        root of all its episodes (src/nanorts/adapters/jaxmarl/env.py:64-69)."""
        roots = np.ascontiguousarray(np.asarray(key.cpu() if isinstance(key, torch.Tensor) else key)
                                     .astype(np.uint32).reshape(-1, 2))
        L = roots.shape[0]
        state = EnvironmentState(
            core_state=self.dev.batch(L),
            environment_root=torch.as_tensor(roots.view(np.int32), device=self.device),
            episode_index=torch.zeros(L, dtype=torch.int32, device=self.device),
        )
        return self.get_obs(state), state

    def step(self, key, state: EnvironmentState, actions: dict[str, torch.Tensor], reset_state=None, *,
             donate: bool = False):
        """env.step (src/nanorts/adapters/jaxmarl/facade.py:107-119); `key` is
        accepted and ignored, as in the reference.  With donate=True the input
        state's buffers are updated in place (XLA donation)."""
        del key
        if reset_state is not None:
            raise ModelError("step resets finished games to the content's start by itself; reset_state is not taken")
        return self._fused_step(state, actions, donate, reset=True)

    def step_env(self, key, state: EnvironmentState, actions: dict[str, torch.Tensor], *, donate: bool = False):
        """env.step_env (src/nanorts/adapters/jaxmarl/facade.py:130-165): the
        transition without the auto-reset; the observation, the final
        observation and the state are the ending state's."""
        del key
        return self._fused_step(state, actions, donate, reset=False)

    def step_request(self, state: EnvironmentState, actions: dict[str, torch.Tensor]):
        """env.step_request (src/nanorts/adapters/jaxmarl/facade.py:121-122):
        ((episode-root keys int32[L, 2] holding uint32 key data, the core
        State, Commands int32[L, 2, C] per field), None), ready for
        groups.step_groups or core_step."""
        L = state.num_envs
        b = self.bucket
        d = self.device
        acts = self._stack_actions(actions, L)
        commands = {f: torch.empty((L, 2, b.per_player_capacity), dtype=torch.int32, device=d)
                    for f, _ in native.Commands._fields_}
        keys = torch.empty((L, 2), dtype=torch.int32, device=d)
        bufs = native.Commands(*[_ptr(commands[f]) for f, _ in native.Commands._fields_])
        native.check(self.lib.nanorts_amd_decode_actions(_stream(), self.dev.ref, state.native(), L, _ptr(acts), bufs,
                                                     _ptr(keys)), "nanorts_amd_decode_actions")
        return (keys, state.core_state, commands), None

    def step_response(self, state: EnvironmentState, carry, stepped: dict[str, torch.Tensor]):
        """env.step_response (src/nanorts/adapters/jaxmarl/facade.py:124-128,
        respond in src/nanorts/adapters/jaxmarl/env.py:99-127) on a state that
        core.step has already advanced in place (`stepped` is its
        terminated / truncated / reward / admitted event counts): rewards,
        the ending state's observation, auto-reset and the next observation.
        The state is updated in place."""
        del carry
        core = state.core_state
        done = (stepped["terminated"] | stepped["truncated"]).to(torch.bool)
        winner = core.winner.reshape(-1).to(torch.int32).clone()
        telemetry = core.spawn_overflow.clone()
        final = self.get_obs(state) if self.final_observation else None
        over = core.game_over.reshape(-1).to(torch.bool)
        comps = _components(stepped, over, winner) if self.layout.reward_components else None
        self.reset_where_done(state, done)
        obs = self.get_obs(state)
        reward = stepped["reward"]
        infos: dict[str, Any] = {
            "terminated": stepped["terminated"].to(torch.bool), "truncated": stepped["truncated"].to(torch.bool),
            "winner": winner, "telemetry": {"spawn_overflow": telemetry},
            "spawn_overflowed": (telemetry > 0).any(dim=1), "final_valid": done,
        }
        if final is not None:
            infos["final_observation"] = final
        if comps is not None:
            infos["reward_components"] = {agent: comps[:, p] for p, agent in enumerate(self.agents)}
        return (obs, state, {agent: reward[:, p] for p, agent in enumerate(self.agents)},
                {agent: done for agent in self.agents} | {ALL_AGENTS: done}, infos)

    @property
    def agent_classes(self) -> dict[str, list[str]]:
        """src/nanorts/adapters/jaxmarl/facade.py:186-188"""
        return {"player": list(self.agents)}

    def _fused_step(self, state: EnvironmentState, actions: dict[str, torch.Tensor], donate: bool, reset: bool):
        nxt = state if donate else state.clone()
        L = nxt.num_envs
        b = self.bucket
        acts = self._stack_actions(actions, L)
        d = self.device
        out = {
            "reward": torch.empty((L, 2), dtype=torch.float32, device=d),
            "done": torch.empty(L, dtype=torch.bool, device=d),
            "terminated": torch.empty(L, dtype=torch.bool, device=d),
            "truncated": torch.empty(L, dtype=torch.bool, device=d),
            "winner": torch.empty(L, dtype=torch.int32, device=d),
            "spawn_overflowed": torch.empty(L, dtype=torch.bool, device=d),
            "spawn_overflow": torch.empty((L, 2), dtype=torch.int32, device=d),
        }
        symbolic = self.layout.surface == "symbolic"
        # the pixel surface renders from the symbolic maps the step writes
        maps = torch.empty((L, 2, b.height, b.width, 6), dtype=torch.uint8, device=d)
        scalars = torch.empty((L, 2, 4), dtype=torch.int32, device=d)
        fmaps = fscal = None
        if self.final_observation and reset:
            fmaps = torch.empty_like(maps)
            fscal = torch.empty_like(scalars)
        comps = torch.empty((L, 2, 6), dtype=torch.float32, device=d) if self.layout.reward_components else None
        results = native.EnvResults(
            _ptr(out["reward"]), _ptr(out["done"]), _ptr(out["terminated"]), _ptr(out["truncated"]),
            _ptr(out["winner"]), _ptr(out["spawn_overflowed"]), _ptr(maps), _ptr(scalars), _ptr(fmaps), _ptr(fscal),
            _ptr(comps), _ptr(out["spawn_overflow"]))
        if reset:
            native.check(self.lib.nanorts_amd_env_step(_stream(), self.dev.ref, nxt.native(), L, _ptr(acts), self.partial,
                                                   results), "nanorts_amd_env_step")
        else:
            native.check(self.lib.nanorts_amd_env_transition(_stream(), self.dev.ref, nxt.native(), L, _ptr(acts),
                                                         self.partial, results), "nanorts_amd_env_transition")
        obs = self._symbolic(maps, scalars) if symbolic else self._pixels(maps, scalars)
        rewards = {agent: out["reward"][:, p] for p, agent in enumerate(self.agents)}
        dones = {agent: out["done"] for agent in self.agents} | {ALL_AGENTS: out["done"]}
        infos: dict[str, Any] = {
            "terminated": out["terminated"], "truncated": out["truncated"], "winner": out["winner"],
            "telemetry": {"spawn_overflow": out["spawn_overflow"]},
            "spawn_overflowed": out["spawn_overflowed"], "final_valid": out["done"],
        }
        if self.final_observation:
            if reset:
                infos["final_observation"] = self._symbolic(fmaps, fscal) if symbolic else self._pixels(fmaps, fscal)
            else:
                infos["final_observation"] = obs
        if comps is not None:
            infos["reward_components"] = {agent: comps[:, p] for p, agent in enumerate(self.agents)}
        return obs, nxt, rewards, dones, infos

    def get_avail_actions(self, state: EnvironmentState, *, form: str = "rows") -> dict[str, torch.Tensor]:
        """bool[L, C, 78] per agent (src/nanorts/adapters/jaxmarl/actions.py:28-41);
        form="words" returns the same rows as uint32[L, C, 3] bitsets."""
        L = state.num_envs
        b = self.bucket
        if form == "rows":
            rows = torch.empty((L, 2, b.per_player_capacity, self.layout.mask_width), dtype=torch.bool,
                               device=self.device)
            native.check(self.lib.nanorts_amd_avail_actions(_stream(), self.dev.ref, state.native(), L, _ptr(rows), None),
                         "nanorts_amd_avail_actions")
        elif form == "words":
            rows = torch.empty((L, 2, b.per_player_capacity, 3), dtype=torch.int32, device=self.device)
            native.check(self.lib.nanorts_amd_avail_actions(_stream(), self.dev.ref, state.native(), L, None, _ptr(rows)),
                         "nanorts_amd_avail_actions")
        else:
            raise ModelError(f"form={form!r} is unknown; get_avail_actions returns 'rows' or 'words'")
        return {agent: rows[:, p] for p, agent in enumerate(self.agents)}

    def get_slot_cells(self, state: EnvironmentState) -> dict[str, torch.Tensor]:
        """int32[L, C] per agent (src/nanorts/adapters/jaxmarl/actions.py:44-52)."""
        b = self.bucket
        cells = state.core_state.cell[:, b.neutral_capacity:].to(torch.int32).reshape(-1, 2, b.per_player_capacity)
        return {agent: cells[:, p] for p, agent in enumerate(self.agents)}

    def get_obs(self, state: EnvironmentState) -> dict[str, Any]:
        L = state.num_envs
        b = self.bucket
        scalars = torch.empty((L, 2, 4), dtype=torch.int32, device=self.device)
        if self.layout.surface == "pixels":
            image = torch.empty((L, 2, 16 * b.height, 16 * b.width, 3), dtype=torch.uint8, device=self.device)
            native.check(self.lib.nanorts_amd_pixels(_stream(), self.dev.ref, state.native(), L, self.partial,
                                                 _ptr(self._tiles), _ptr(image), _ptr(scalars)), "nanorts_amd_pixels")
            return {agent: PixelObservation(image[:, p], scalars[:, p]) for p, agent in enumerate(self.agents)}
        maps = torch.empty((L, 2, b.height, b.width, 6), dtype=torch.uint8, device=self.device)
        native.check(self.lib.nanorts_amd_observe(_stream(), self.dev.ref, state.native(), L, self.partial, _ptr(maps),
                                              _ptr(scalars)), "nanorts_amd_observe")
        return self._symbolic(maps, scalars)

    # ------------------------------------------------------- beyond the API
    def core_step(self, state: EnvironmentState, commands: dict[str, torch.Tensor], key) -> dict[str, torch.Tensor]:
        """core.step with explicit Commands [L, 2, C] per field (in place) and
        episode-root keys [L, 2] or [2] (src/nanorts/core/__init__.py:46-60)."""
        L = state.num_envs
        b = self.bucket
        d = self.device
        keyt = torch.as_tensor(np.ascontiguousarray(np.asarray(key, np.uint32).reshape(-1, 2)).view(np.int32),
                               device=d)
        cmd = {f: commands[f].to(device=d, dtype=torch.int32).contiguous() for f in
               ("kind", "direction", "none_duration", "target_cell", "produced_type", "request_order")}
        out = {"terminated": torch.empty(L, dtype=torch.bool, device=d),
               "truncated": torch.empty(L, dtype=torch.bool, device=d),
               "reward": torch.empty((L, 2), dtype=torch.float32, device=d),
               "admitted_harvest": torch.empty((L, 2), dtype=torch.int32, device=d),
               "admitted_return": torch.empty((L, 2), dtype=torch.int32, device=d),
               "admitted_produce": torch.empty((L, 2, b.unit_type_capacity), dtype=torch.int32, device=d),
               "admitted_attack": torch.empty((L, 2, 3), dtype=torch.int32, device=d)}
        c = native.Commands(*[_ptr(cmd[f]) for f, _ in native.Commands._fields_])
        r = native.StepResults(*[_ptr(out.get(f)) for f, _ in native.StepResults._fields_])
        native.check(self.lib.nanorts_amd_step(_stream(), self.dev.ref, state.native(), L, _ptr(keyt), keyt.shape[0], c,
                                           r), "nanorts_amd_step")
        return out

    def legality(self, state: EnvironmentState, *, form: str = "words") -> torch.Tensor:
        """Factored legality before availability (core.legal_commands), as the
        reference's nanorts_amd_legality[_words] targets publish it."""
        L = state.num_envs
        b = self.bucket
        if form == "words":
            out = torch.empty((L, 2, b.per_player_capacity, 3), dtype=torch.int32, device=self.device)
            native.check(self.lib.nanorts_amd_legality_words(_stream(), self.dev.ref, state.native(), L, _ptr(out)),
                         "nanorts_amd_legality_words")
        else:
            out = torch.empty((L, 2, b.per_player_capacity, self.layout.mask_width), dtype=torch.bool,
                              device=self.device)
            native.check(self.lib.nanorts_amd_legality(_stream(), self.dev.ref, state.native(), L, _ptr(out)),
                         "nanorts_amd_legality")
        return out

    def visible_cells(self, state: EnvironmentState, observer: int) -> torch.Tensor:
        L = state.num_envs
        b = self.bucket
        out = torch.empty((L, b.height, b.width), dtype=torch.bool, device=self.device)
        native.check(self.lib.nanorts_amd_visible_cells(_stream(), self.dev.ref, state.native(), L, int(observer),
                                                    _ptr(out)), "nanorts_amd_visible_cells")
        return out

    def reset_where_done(self, state: EnvironmentState, done: torch.Tensor) -> None:
        done = done.to(device=self.device, dtype=torch.bool).contiguous()
        native.check(self.lib.nanorts_amd_reset_where_done(_stream(), self.dev.ref, state.native(), state.num_envs,
                                                       _ptr(done)), "nanorts_amd_reset_where_done")

    def sample_actions(self, words, sample_key, step: int, env0: int = 0) -> dict[str, torch.Tensor]:
        """The synthetic harness's integer uniform-over-legal sampler on
        get_avail_actions(form="words") output: the per-agent dict, or the
        words stacked as [L, 2, C, 3]."""
        if isinstance(words, dict):
            per_agent = [words[a] for a in self.agents]
            stacked = self._agent_stack(per_agent)
            words = stacked if stacked is not None else torch.stack(per_agent, dim=1)
        words = words.contiguous()
        L = words.shape[0]
        b = self.bucket
        key = (ctypes.c_uint32 * 2)(*[int(v) for v in np.asarray(sample_key, np.uint32).reshape(2)])
        actions = torch.empty((L, 2, b.per_player_capacity, 7), dtype=torch.int32, device=self.device)
        native.check(self.lib.nanorts_amd_sample_actions(_stream(), self.dev.ref, L, _ptr(words), key, int(step), int(env0),
                                                     _ptr(actions)), "nanorts_amd_sample_actions")
        return {agent: actions[:, p] for p, agent in enumerate(self.agents)}

    def rollout_first_pass(self) -> str | None:
        """The first pass rollout() runs on this game (with two_pass): "pair"
        (two games per wave), "lean" (one game per wave) or None (one pass
        on the full block).  The environment variable NANORTS_AMD_FIRST_PASS
        ("lean" or "pair") overrides the library's choice by board."""
        code = self.lib.nanorts_amd_rollout_first_pass(self.dev.ref)
        if code < 0:
            native.check(code, "nanorts_amd_rollout_first_pass")
        return {2: "pair", 1: "lean"}.get(code)

    def rollout(self, state: EnvironmentState, steps: int, sample_key, *, step0: int = 0, env0: int = 0,
                record: bool = True, record_actions: bool = False, observation_depth: int = 1,
                count_general: bool = False, two_pass: bool = True) -> dict[str, Any]:
        """Fused rollout: `steps` cycles of masks -> sample -> env.step with the
        state resident in LDS, in place.  Bit-equal to the per-call API.  With
        count_general, out["general_admissions"] int32[L] counts each env's
        cycles that took the request-at-a-time admission.  With two_pass (the
        default), each launch first runs the games on a smaller LDS block
        and hands the cycles that need the full block to a second pass;
        out["first_pass_cycles"] int32[L] holds the cycles of the last launch
        each game ran in the first pass (steps of it when the launch needed
        no second pass).  two_pass=False runs one pass on the full block."""
        L = state.num_envs
        b = self.bucket
        d = self.device
        out: dict[str, Any] = {}
        rewards = torch.empty((steps, L, 2), dtype=torch.float32, device=d) if record else None
        dones = torch.empty((steps, L), dtype=torch.bool, device=d) if record else None
        actions = torch.empty((steps, L, 2, b.per_player_capacity, 7), dtype=torch.int32, device=d) \
            if record_actions else None
        depth = max(1, int(observation_depth))
        maps = torch.empty((depth, L, 2, b.height, b.width, 6), dtype=torch.uint8, device=d)
        scalars = torch.empty((depth, L, 2, 4), dtype=torch.int32, device=d)
        key = (ctypes.c_uint32 * 2)(*[int(v) for v in np.asarray(sample_key, np.uint32).reshape(2)])
        general = torch.empty(L, dtype=torch.int32, device=d) if count_general else None
        progress = torch.empty(L, dtype=torch.int32, device=d) if two_pass else None
        results = native.RolloutResults(_ptr(rewards), _ptr(dones), _ptr(actions), _ptr(maps), _ptr(scalars), depth,
                                        _ptr(general), _ptr(progress))
        native.check(self.lib.nanorts_amd_rollout(_stream(), self.dev.ref, state.native(), L, key, int(step0), int(steps),
                                              self.partial, int(env0), results), "nanorts_amd_rollout")
        out.update(rewards=rewards, dones=dones, actions=actions, feature_maps=maps, scalars=scalars,
                   general_admissions=general, first_pass_cycles=progress)
        return out

    # -------------------------------------------------------------- helpers
    def _symbolic(self, maps: torch.Tensor, scalars: torch.Tensor) -> dict[str, SymbolicObservation]:
        if self.feature_dtype != torch.uint8:
            maps = maps.to(self.feature_dtype)
        return {agent: SymbolicObservation(maps[:, p], scalars[:, p]) for p, agent in enumerate(self.agents)}

    def pixels_from_maps(self, maps: torch.Tensor) -> torch.Tensor:
        """uint8[..., 16H, 16W, 3] images of symbolic maps uint8[..., H, W, 6]
        (src/nanorts/observations/pixels.py:91-110)."""
        b = self.bucket
        if self._tiles is None:
            from nanorts_amd import rendering

            self._tiles = torch.as_tensor(rendering.tile_table(b.unit_type_capacity), device=self.device)
        maps = maps.contiguous()
        if maps.dtype != torch.uint8 or tuple(maps.shape[-3:]) != (b.height, b.width, 6):
            raise ModelError(f"feature maps are {maps.dtype} {tuple(maps.shape)}, expected uint8 [..., "
                             f"{b.height}, {b.width}, 6]")
        lead = tuple(maps.shape[:-3])
        images = int(np.prod(lead)) if lead else 1
        image = torch.empty((*lead, 16 * b.height, 16 * b.width, 3), dtype=torch.uint8, device=self.device)
        native.check(self.lib.nanorts_amd_pixels_from_maps(_stream(), self.dev.ref, images, _ptr(maps), _ptr(self._tiles),
                                                       _ptr(image)), "nanorts_amd_pixels_from_maps")
        return image

    def _pixels(self, maps: torch.Tensor, scalars: torch.Tensor) -> dict[str, PixelObservation]:
        image = self.pixels_from_maps(maps)
        return {agent: PixelObservation(image[:, p], scalars[:, p]) for p, agent in enumerate(self.agents)}

    def _agent_stack(self, per_agent: list[torch.Tensor]) -> torch.Tensor | None:
        """The [L, 2, ...] tensor the per-agent values are views of (agent p
        = base[:, p], as sample_actions and get_avail_actions return them),
        or None when they are separate tensors."""
        a0, a1 = per_agent
        if not (isinstance(a0, torch.Tensor) and isinstance(a1, torch.Tensor)) or a0.device != self.device:
            return None
        if a0.dtype != a1.dtype or a0.shape != a1.shape or a0.dim() < 1 or a1.device != a0.device:
            return None
        inner = a0[0].numel() if a0.shape[0] > 0 else 0
        row = tuple(a0.shape[1:])
        dense = [1]
        for extent in reversed(row[1:]):
            dense.insert(0, dense[0] * extent)
        if a0.shape[0] == 0 or tuple(a0.stride()[1:]) != tuple(dense[:len(row)]) or a0.stride() != a1.stride():
            return None
        if a0.stride(0) != 2 * inner or a1.data_ptr() != a0.data_ptr() + inner * a0.element_size():
            return None
        return torch.as_strided(a0, (a0.shape[0], 2, *row), (2 * inner, inner, *a0.stride()[1:]))

    def _stack_actions(self, actions: dict[str, torch.Tensor], L: int) -> torch.Tensor:
        if set(actions) != set(self.agents):
            raise ModelError(f"actions are keyed by {sorted(actions)}, expected {self.agents}")
        per_agent = [torch.as_tensor(actions[a], device=self.device) for a in self.agents]
        stacked = self._agent_stack(per_agent)
        if stacked is None:
            stacked = torch.stack(per_agent, dim=1)
        if stacked.dtype != torch.int32:
            raise ModelError(f"actions have dtype {stacked.dtype}, expected int32")
        if tuple(stacked.shape) != (L, 2, *self.layout.actions_shape):
            raise ModelError(f"actions have shape {tuple(stacked.shape)}, expected {(L, 2, *self.layout.actions_shape)}")
        return stacked.contiguous()

    def observation_space(self, agent: str) -> dict[str, Any]:
        b = self.bucket
        if self.layout.surface == "pixels":
            return {"image": ((16 * b.height, 16 * b.width, 3), torch.uint8), "scalars": ((4,), torch.int32)}
        return {"feature_maps": (self.layout.feature_maps_shape, self.feature_dtype), "scalars": ((4,), torch.int32)}

    def action_space(self, agent: str) -> dict[str, Any]:
        return {"shape": self.layout.actions_shape, "high": tuple(w - 1 for w in self.layout.action_widths)}


def env_roots(seed: int, num_envs: int) -> np.ndarray:
    """Per-env reset keys split(key(seed), num_envs), as the README rollout
    derives them (jax.random.split(reset_key, NUM_ENVS))."""
    return _keys.split(_keys.key(seed), num_envs)


def check_actions(actions: dict[str, Any], *, layout: JaxMARLLayout) -> None:
    """Host-side range check (src/nanorts/adapters/jaxmarl/actions.py:87-111)."""
    if set(actions) != set(layout.agents):
        raise ModelError(f"actions are keyed by {sorted(actions)}, expected {list(layout.agents)}")
    for agent in layout.agents:
        array = np.asarray(actions[agent].cpu() if isinstance(actions[agent], torch.Tensor) else actions[agent])
        if array.shape[-2:] != layout.actions_shape:
            raise ModelError(f"actions for {agent} have shape {array.shape}, expected [..., {layout.actions_shape}]")
        if array.dtype != np.int32:
            raise ModelError(f"actions for {agent} have dtype {array.dtype}, expected int32")
        for index, (name, size) in enumerate(zip(layout.action_factors, layout.action_widths)):
            factor = array[..., index]
            if factor.size and (factor.min() < 0 or factor.max() >= size):
                raise ModelError(f"action factor {index} ({name}) of {agent} carries values in "
                                 f"[{int(factor.min())}, {int(factor.max())}], expected [0, {size - 1}]")


_ = KIND_NONE, leaf_shape, _TORCH_DTYPES
