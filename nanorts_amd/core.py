"""Core-level functions over the kernels, batched over a leading env dimension.

Mirrors src/nanorts/core/__init__.py (reset, step, step_groups,
steps_together, legal_commands) and src/nanorts/observations (symbolic,
pixels, pixels_from_symbolic, visibility) of the reference, which are
single-env JAX functions that callers vmap; here each call takes L envs'
State leaves (torch tensors on the GPU) and is one kernel launch.  The game's
device copy (unit table, terrain, initial state) is built once per game and
device and cached.
"""
from __future__ import annotations

import weakref
from typing import Any

import torch

from nanorts_amd import native
from nanorts_amd.content import GameConfig
from nanorts_amd.env import DeviceGame, EnvironmentState, PixelObservation, State, SymbolicObservation, _ptr, _stream
from nanorts_amd.groups import step_groups, steps_together
from nanorts_amd.model import ModelError

__all__ = ["legal_commands", "pixels", "pixels_from_symbolic", "reset", "step", "step_events", "step_groups",
           "steps_together", "symbolic", "visibility"]

_DEVICE_GAMES: "weakref.WeakKeyDictionary[GameConfig, dict[str, DeviceGame]]" = weakref.WeakKeyDictionary()
_COMMAND_FIELDS = ("kind", "direction", "none_duration", "target_cell", "produced_type", "request_order")


def device_game(game: GameConfig, device: torch.device | str | None = None) -> DeviceGame:
    """The cached device copy of `game` (unit table, terrain, initial state)."""
    device = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
    per_game = _DEVICE_GAMES.setdefault(game, {})
    key = str(device)
    if key not in per_game:
        per_game[key] = DeviceGame(game, device)
    return per_game[key]


def _core(state: Any) -> State:
    core = state.core_state if isinstance(state, EnvironmentState) else state
    if not isinstance(core, State):
        raise ModelError("expected a State (or an EnvironmentState) of L envs")
    return core


def _native_state(core: State) -> native.State:
    return native.State(*[_ptr(core.leaves[name]) for name in native.STATE_FIELDS[:-2]], None, None)


def _lanes(core: State) -> int:
    return int(core.leaves["time"].shape[0])


def _device_of(core: State) -> torch.device:
    return core.leaves["time"].device


def reset(key, game: GameConfig, num_envs: int, *, device: torch.device | str | None = None) -> State:
    """core.reset (src/nanorts/core/__init__.py:30-32) for `num_envs` envs: the
    decided initial state; the key is not read, as in the reference."""
    del key
    return device_game(game, device).batch(num_envs)


def step(key, state: Any, commands: dict[str, torch.Tensor], game: GameConfig, *,
         records: bool = False) -> dict[str, torch.Tensor]:
    """core.step (src/nanorts/core/__init__.py:46-60) in place: `key` is
    uint32 key data [L, 2] or [2] (or an int32 device tensor holding it),
    Commands int32[L, 2, C] per field.  Returns terminated, truncated, reward
    and the admitted event counts; with `records`, also the per-slot
    completion records, which step_events decodes into StepEvents' fields."""
    core = _core(state)
    return step_groups([(key, core, commands, device_game(game, _device_of(core)))], records=records)[0]


# The per-slot StepEvents fields (src/nanorts/model/step.py:39-112) and where
# each comes from in the records (src/nanorts/core/cycle.py:48-81, 281-300):
# (field, record flag, column group and index or None for `valid`, fill).
_FLAG = {"hit": 1, "death": 2, "harvest": 4, "return": 16, "spawn": 32}
_ACTOR = (("actor_birth", ("i32", 0)), ("actor_owner", ("i8", 1)), ("actor_unit_type", ("i8", 2)))
_FACTS = {
    "hit": (("target_slot", ("i16", 0), -1), ("target_birth", ("i32", 1), -1), ("damage", ("i32", 2), 0)),
    "death": (("slot", ("i16", 3), -1), ("birth", ("i32", 5), -1), ("owner", ("i8", 4), -1),
              ("unit_type", ("i8", 5), -1)),
    "harvest": (("target_slot", ("i16", 0), -1), ("target_birth", ("i32", 1), -1), ("amount", ("i32", 2), 0)),
    "return": (("target_slot", ("i16", 0), -1), ("target_birth", ("i32", 1), -1), ("amount", ("i32", 2), 0),
               ("balance", ("i32", 3), -1)),
    "spawn": (("produced_type", ("i8", 3), -1), ("slot", ("i16", 1), -1), ("birth", ("i32", 4), -1),
              ("cell", ("i16", 2), -1), ("balance", ("i32", 3), -1)),
}


def step_events(out: dict[str, torch.Tensor]) -> dict[str, torch.Tensor]:
    """The per-slot StepEvents fields of a core.step(..., records=True)
    result, decoded as the reference decodes its step target's records
    (src/nanorts/core/cycle.py:281-311): a record is valid where the slot
    took a turn and its flag is set; its fields read the record's columns
    there and their fills elsewhere.  bool / int32 [L, E] each."""
    if "is_member" not in out:
        raise ModelError("step_events needs a core.step result taken with records=True")
    cols = {"i32": out["records_i32"].to(torch.int32), "i16": out["records_i16"].to(torch.int32),
            "i8": out["records_i8"].to(torch.int32)}
    flags = cols["i8"][..., 0]
    member = out["is_member"].to(torch.bool)
    events: dict[str, torch.Tensor] = {}
    for name, flag in _FLAG.items():
        valid = member & ((flags & flag) != 0)
        events[f"{name}_valid"] = valid
        for fact, (group, k) in _ACTOR:
            events[f"{name}_{fact}"] = torch.where(valid, cols[group][..., k], -1)
        for fact, (group, k), fill in _FACTS[name]:
            events[f"{name}_{fact}"] = torch.where(valid, cols[group][..., k], fill)
        if name == "harvest":
            events["harvest_depleted"] = valid & ((flags & 8) != 0)
    return events


def legal_commands(state: Any, game: GameConfig, *, stored: str = "rows") -> torch.Tensor:
    """core.legal_commands (src/nanorts/core/__init__.py:35-43): the factored
    legality of every owned position before availability, bool[L, 2, C, 78]
    (stored="rows") or uint32 words in int32[L, 2, C, 3] (stored="words")."""
    core = _core(state)
    dev = device_game(game, _device_of(core))
    L = _lanes(core)
    b = game.bucket
    lib = native.load()
    if stored == "words":
        out = torch.empty((L, 2, b.per_player_capacity, 3), dtype=torch.int32, device=dev.device)
        native.check(lib.nanorts_amd_legality_words(_stream(), dev.ref, _native_state(core), L, _ptr(out)),
                     "nanorts_amd_legality_words")
    elif stored == "rows":
        width = 6 + 4 * 4 + b.unit_type_capacity + b.attack_offset_capacity
        out = torch.empty((L, 2, b.per_player_capacity, width), dtype=torch.bool, device=dev.device)
        native.check(lib.nanorts_amd_legality(_stream(), dev.ref, _native_state(core), L, _ptr(out)), "nanorts_amd_legality")
    else:
        raise ModelError(f"stored={stored!r} is unknown; the legality grid comes as 'rows' or 'words'")
    return out


def visibility(game: GameConfig, state: Any, *, observer: int) -> torch.Tensor:
    """observations.visibility (src/nanorts/observations/visibility.py:36-47):
    the cells `observer` sees, bool[L, H, W]."""
    if observer not in (0, 1):
        raise ModelError(f"observer={observer!r} names no player; use 0 or 1")
    core = _core(state)
    dev = device_game(game, _device_of(core))
    L = _lanes(core)
    b = game.bucket
    out = torch.empty((L, b.height, b.width), dtype=torch.bool, device=dev.device)
    native.check(native.load().nanorts_amd_visible_cells(_stream(), dev.ref, _native_state(core), L, int(observer),
                                                     _ptr(out)), "nanorts_amd_visible_cells")
    return out


def _both_symbolic(game: GameConfig, core: State, partial: bool) -> tuple[torch.Tensor, torch.Tensor]:
    dev = device_game(game, _device_of(core))
    L = _lanes(core)
    b = game.bucket
    maps = torch.empty((L, 2, b.height, b.width, 6), dtype=torch.uint8, device=dev.device)
    scalars = torch.empty((L, 2, 4), dtype=torch.int32, device=dev.device)
    native.check(native.load().nanorts_amd_observe(_stream(), dev.ref, _native_state(core), L, int(bool(partial)),
                                               _ptr(maps), _ptr(scalars)), "nanorts_amd_observe")
    return maps, scalars


def symbolic(game: GameConfig, state: Any, *, observer: int, partial_observability: bool) -> SymbolicObservation:
    """observations.symbolic (src/nanorts/observations/symbolic.py:99-127):
    uint8[L, H, W, 6] feature maps and int32[L, 4] scalars of `observer`."""
    if observer not in (0, 1):
        raise ModelError(f"observer={observer!r} names no player; use 0 or 1")
    maps, scalars = _both_symbolic(game, _core(state), partial_observability)
    return SymbolicObservation(maps[:, observer], scalars[:, observer])


def pixels(game: GameConfig, state: Any, assets, *, observer: int, partial_observability: bool) -> PixelObservation:
    """observations.pixels (src/nanorts/observations/pixels.py:78-88):
    uint8[L, 16H, 16W, 3] images and int32[L, 4] scalars of `observer`,
    drawn with a prepared Asset set of 16-pixel cells."""
    if observer not in (0, 1):
        raise ModelError(f"observer={observer!r} names no player; use 0 or 1")
    if assets.cell_pixels != 16:
        raise ModelError("the pixel kernel draws 16-pixel cells")
    core = _core(state)
    dev = device_game(game, _device_of(core))
    L = _lanes(core)
    b = game.bucket
    tiles = torch.as_tensor(assets.tiles, device=dev.device).contiguous()
    image = torch.empty((L, 2, 16 * b.height, 16 * b.width, 3), dtype=torch.uint8, device=dev.device)
    scalars = torch.empty((L, 2, 4), dtype=torch.int32, device=dev.device)
    native.check(native.load().nanorts_amd_pixels(_stream(), dev.ref, _native_state(core), L,
                                              int(bool(partial_observability)), _ptr(tiles), _ptr(image),
                                              _ptr(scalars)), "nanorts_amd_pixels")
    return PixelObservation(image[:, observer], scalars[:, observer])


def pixels_from_symbolic(feature_maps: torch.Tensor, assets, game: GameConfig) -> torch.Tensor:
    """observations.pixels_from_symbolic (src/nanorts/observations/pixels.py:91-110):
    uint8[..., 16H, 16W, 3] images of feature maps uint8[..., H, W, 6]."""
    b = game.bucket
    maps = feature_maps.contiguous()
    if tuple(maps.shape[-3:]) != (b.height, b.width, 6) or maps.dtype != torch.uint8:
        raise ModelError(f"feature maps must be uint8[..., {b.height}, {b.width}, 6]")
    dev = device_game(game, maps.device)
    images = maps.numel() // (b.height * b.width * 6)
    tiles = torch.as_tensor(assets.tiles, device=maps.device).contiguous()
    out = torch.empty((*maps.shape[:-3], 16 * b.height, 16 * b.width, 3), dtype=torch.uint8, device=maps.device)
    native.check(native.load().nanorts_amd_pixels_from_maps(_stream(), dev.ref, images, _ptr(maps), _ptr(tiles),
                                                        _ptr(out)), "nanorts_amd_pixels_from_maps")
    return out
