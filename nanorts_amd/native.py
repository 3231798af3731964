"""ctypes binding of the C ABI in include/nanorts_amd.h.

This is the Python side of the drop-in boundary: the same entry points an XLA
FFI handler would wrap.  Loading fails loudly when the library is missing;
there is no fallback implementation.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

from nanorts_amd import build as _build

MAX_TYPES = 8

_VP = ctypes.c_void_p
_I32x8 = ctypes.c_int32 * MAX_TYPES

STATE_FIELDS = (
    "birth", "unit_type", "owner", "cell", "hit_points", "carried_resources", "pending_kind",
    "pending_direction", "pending_none_duration", "pending_target_cell", "pending_produced_type",
    "pending_issued_at", "pending_completes_at", "pending_order", "entity_at", "time", "player_resources",
    "next_birth", "next_pending_order", "alternating_conflict_count", "game_over", "winner", "spawn_overflow",
    "environment_root", "episode_index",
)


class State(ctypes.Structure):
    _fields_ = [(name, _VP) for name in STATE_FIELDS]


class Game(ctypes.Structure):
    _fields_ = [
        ("height", ctypes.c_int32), ("width", ctypes.c_int32), ("cells", ctypes.c_int32),
        ("neutral", ctypes.c_int32), ("capacity", ctypes.c_int32), ("entities", ctypes.c_int32),
        ("types", ctypes.c_int32), ("offsets", ctypes.c_int32), ("strategy", ctypes.c_int32),
        ("max_cycles", ctypes.c_int32),
        ("cost", _I32x8), ("hit_points", _I32x8), ("produce_time", _I32x8), ("move_time", _I32x8),
        ("attack_time", _I32x8), ("harvest_time", _I32x8), ("attack_range", _I32x8), ("attack_damage", _I32x8),
        ("harvest_amount", _I32x8), ("sight_radius", _I32x8), ("is_resource", _I32x8), ("is_stockpile", _I32x8),
        ("can_harvest", _I32x8), ("can_move", _I32x8), ("can_attack", _I32x8),
        ("produces", ctypes.c_int32 * (MAX_TYPES * MAX_TYPES)),
        ("terrain", _VP),
        ("initial", State),
    ]


class Commands(ctypes.Structure):
    _fields_ = [(name, _VP) for name in
                ("kind", "direction", "none_duration", "target_cell", "produced_type", "request_order")]


class StepResults(ctypes.Structure):
    _fields_ = [(name, _VP) for name in
                ("terminated", "truncated", "reward", "admitted_harvest", "admitted_return", "admitted_produce",
                 "admitted_attack", "is_member", "records_i32", "records_i16", "records_i8")]


class EnvResults(ctypes.Structure):
    _fields_ = [(name, _VP) for name in
                ("reward", "done", "terminated", "truncated", "winner", "spawn_overflowed", "feature_maps", "scalars",
                 "final_feature_maps", "final_scalars", "reward_components", "spawn_overflow")]


class RolloutResults(ctypes.Structure):
    _fields_ = [("rewards", _VP), ("dones", _VP), ("actions", _VP), ("feature_maps", _VP), ("scalars", _VP),
                ("depth", ctypes.c_int32), ("general_admissions", _VP), ("progress", _VP)]


ABSTRACT_FIELDS = ("kind", "unit_birth", "order", "target", "target_birth", "base", "base_birth", "cell",
                   "unit_type", "trained", "next_order")


class AbstractActions(ctypes.Structure):
    _fields_ = [(name, _VP) for name in ABSTRACT_FIELDS]


class GridNetObs(ctypes.Structure):
    _fields_ = [("planes_form", ctypes.c_int32), ("planes_bytes", ctypes.c_int32), ("planes", _VP),
                ("source_mask", _VP), ("mask_form", ctypes.c_int32), ("mask_bytes", ctypes.c_int32),
                ("action_mask", _VP)]


class GridNetResults(ctypes.Structure):
    _fields_ = [(name, _VP) for name in
                ("reward_components", "reward_dones", "terminated", "truncated", "done", "winner",
                 "spawn_overflowed", "final_planes")] + [("observation", GridNetObs), ("spawn_overflow", _VP)]


# Every extern "C" symbol include/nanorts_amd.h declares.
EXPORTS = (
    "nanorts_amd_build_id", "nanorts_amd_entries", "nanorts_amd_last_error", "nanorts_amd_shared_opt_in",
    "nanorts_amd_self_check", "nanorts_amd_self_check_no_alloc", "nanorts_amd_step", "nanorts_amd_step_ffi",
    "nanorts_amd_legality_ffi", "nanorts_amd_visible_cells_ffi", "nanorts_amd_reset_rows_ffi",
    "nanorts_amd_step_groups", "nanorts_amd_env_transition", "nanorts_amd_decode_actions",
    "nanorts_amd_legality", "nanorts_amd_legality_words", "nanorts_amd_avail_actions", "nanorts_amd_visible_cells",
    "nanorts_amd_observe", "nanorts_amd_pixels", "nanorts_amd_pixels_from_maps", "nanorts_amd_reset_where_done", "nanorts_amd_env_step", "nanorts_amd_sample_actions",
    "nanorts_amd_rollout", "nanorts_amd_abstraction_act", "nanorts_amd_seat_step", "nanorts_amd_seat_rollout",
    "nanorts_amd_seat_step_lanes", "nanorts_amd_seat_rollout_lanes", "nanorts_amd_episode_seats",
    "nanorts_amd_gridnet_decode", "nanorts_amd_gridnet_observe", "nanorts_amd_gridnet_step", "nanorts_amd_gridnet_step_against",
    "nanorts_amd_gridnet_sample_actions", "nanorts_amd_step_groups_ffi", "nanorts_amd_abstraction_act_ffi",
    "nanorts_amd_astar_search_ffi", "nanorts_amd_astar_chain_ffi", "nanorts_amd_gridnet_decode_ffi",
    "nanorts_amd_rollout_first_pass",
)

_I64 = ctypes.c_int64
_I32 = ctypes.c_int32
_GP = ctypes.POINTER(Game)

_SIGNATURES = {
    "nanorts_amd_build_id": (ctypes.c_char_p, []),
    "nanorts_amd_entries": (ctypes.c_char_p, []),
    "nanorts_amd_last_error": (ctypes.c_char_p, []),
    "nanorts_amd_shared_opt_in": (ctypes.c_int64, [_VP, _I64]),
    "nanorts_amd_self_check": (ctypes.c_char_p, [_VP, _I64]),
    "nanorts_amd_self_check_no_alloc": (ctypes.c_char_p, [_VP, _I64, _I32, _VP]),
    "nanorts_amd_step": (ctypes.c_int, [_VP, _GP, State, _I64, _VP, _I64, Commands, StepResults]),
    "nanorts_amd_step_ffi": (ctypes.c_int, [_VP, _VP, _VP, _I64, _I64, _I64, _I32, _I32, _I32, _I32, _I32, _I64]),
    "nanorts_amd_legality_ffi": (ctypes.c_int, [_VP, _VP, _VP, _I32, _I64, _I32, _I32, _I32, _I32, _I32, _I32]),
    "nanorts_amd_visible_cells_ffi": (ctypes.c_int, [_VP, _VP, _I64, _VP, _I64, _VP, _I32, _I64, _I64, _VP, _I64, _VP,
                                                     _I64, _I64, _I64, _I32, _I32]),
    "nanorts_amd_reset_rows_ffi": (ctypes.c_int, [_VP, _VP, _I64, _I32, _VP, _VP, _VP, _VP, _VP]),
    "nanorts_amd_step_groups": (ctypes.c_int, [_VP, _I32, _VP, _VP, _VP, _VP, _VP, _VP, _VP]),
    "nanorts_amd_legality": (ctypes.c_int, [_VP, _GP, State, _I64, _VP]),
    "nanorts_amd_legality_words": (ctypes.c_int, [_VP, _GP, State, _I64, _VP]),
    "nanorts_amd_avail_actions": (ctypes.c_int, [_VP, _GP, State, _I64, _VP, _VP]),
    "nanorts_amd_visible_cells": (ctypes.c_int, [_VP, _GP, State, _I64, _I32, _VP]),
    "nanorts_amd_observe": (ctypes.c_int, [_VP, _GP, State, _I64, _I32, _VP, _VP]),
    "nanorts_amd_pixels": (ctypes.c_int, [_VP, _GP, State, _I64, _I32, _VP, _VP, _VP]),
    "nanorts_amd_pixels_from_maps": (ctypes.c_int, [_VP, _GP, _I64, _VP, _VP, _VP]),
    "nanorts_amd_reset_where_done": (ctypes.c_int, [_VP, _GP, State, _I64, _VP]),
    "nanorts_amd_env_step": (ctypes.c_int, [_VP, _GP, State, _I64, _VP, _I32, EnvResults]),
    "nanorts_amd_env_transition": (ctypes.c_int, [_VP, _GP, State, _I64, _VP, _I32, EnvResults]),
    "nanorts_amd_decode_actions": (ctypes.c_int, [_VP, _GP, State, _I64, _VP, Commands, _VP]),
    "nanorts_amd_sample_actions": (ctypes.c_int, [_VP, _GP, _I64, _VP, _VP, _I32, _I64, _VP]),
    "nanorts_amd_rollout": (ctypes.c_int, [_VP, _GP, State, _I64, _VP, _I32, _I32, _I32, _I64, RolloutResults]),
    "nanorts_amd_rollout_first_pass": (ctypes.c_int, [_GP]),
    "nanorts_amd_abstraction_act": (ctypes.c_int, [_VP, _GP, State, _I64, _I32, _I32, _VP, _I64, AbstractActions, _VP]),
    "nanorts_amd_seat_step": (ctypes.c_int, [_VP, _GP, State, _I64, _I32, _I32, _I32, AbstractActions, _VP, _I32,
                                         EnvResults]),
    "nanorts_amd_seat_rollout": (ctypes.c_int, [_VP, _GP, State, _I64, _I32, _I32, _I32, AbstractActions, _VP, _I32, _I32,
                                            _I32, _I64, RolloutResults]),
    "nanorts_amd_seat_step_lanes": (ctypes.c_int, [_VP, _GP, State, _I64, _I32, _I32, _VP, _I32, AbstractActions, _VP,
                                               _I32, EnvResults]),
    "nanorts_amd_seat_rollout_lanes": (ctypes.c_int, [_VP, _GP, State, _I64, _I32, _I32, _VP, _I32, _VP, AbstractActions,
                                                  _VP, _I32, _I32, _I32, _I64, RolloutResults]),
    "nanorts_amd_episode_seats": (ctypes.c_int, [_VP, _VP, _VP, _I64, _VP]),
    # the command buffers have the layout of Commands (six int32 pointers)
    "nanorts_amd_gridnet_decode": (ctypes.c_int, [_VP, _GP, State, _I64, _VP, Commands]),
    "nanorts_amd_gridnet_observe": (ctypes.c_int, [_VP, _GP, State, _I64, GridNetObs]),
    "nanorts_amd_gridnet_step": (ctypes.c_int, [_VP, _GP, State, _I64, _VP, GridNetResults]),
    "nanorts_amd_gridnet_step_against": (ctypes.c_int, [_VP, _GP, State, _I64, _VP, Commands, GridNetResults]),
    "nanorts_amd_gridnet_sample_actions": (ctypes.c_int, [_VP, _GP, _I64, _VP, _VP, _I32, _I64, _VP]),
    "nanorts_amd_step_groups_ffi": (ctypes.c_int, [_VP, _I32, _VP, _VP, _VP, _VP, _VP, _I32, _I32, _I32, _I32, _I32,
                                                   _I64]),
    "nanorts_amd_abstraction_act_ffi": (ctypes.c_int, [_VP, _VP, _VP, _VP, _I64, _I32, _I32, _I32, _I32, _I32, _I64,
                                                       _I64]),
    "nanorts_amd_astar_search_ffi": (ctypes.c_int, [_VP, _VP, _I64, _VP, _I64, _VP, _I64, _VP, _I64, _I32, _I32, _VP,
                                                    _I64]),
    "nanorts_amd_astar_chain_ffi": (ctypes.c_int, [_VP, _VP, _VP, _VP, _I64, _I32, _I32, _I64, _I64, _I64, _I32, _VP,
                                                   _VP]),
    "nanorts_amd_gridnet_decode_ffi": (ctypes.c_int, [_VP, _VP, _VP, _VP, _I64, _I32, _I32, _I32, _I32, _I32, _I32,
                                                      _I32]),
}

_LIBRARY: ctypes.CDLL | None = None


class NativeError(RuntimeError):
    """An entry point of the kernel library returned an error code."""


def load(path: Path | None = None) -> ctypes.CDLL:
    """Load the in-tree kernel library, building it only when none is built."""
    global _LIBRARY
    if _LIBRARY is not None and path is None:
        return _LIBRARY
    target = Path(path) if path is not None else _build.library_path()
    if not target.exists():
        if path is not None:
            raise RuntimeError(f"no kernel library at {target}")
        _build.build()
    lib = ctypes.CDLL(str(target))
    for name, (restype, argtypes) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    if path is None:
        # The in-tree library must be the build of the sources beside it
        # (the reference's loader refuses a digest mismatch the same way,
        # src/nanorts/kernels/library.py:53-54).
        built, sources = lib.nanorts_amd_build_id().decode(), _build.source_digest()
        if built != sources:
            raise RuntimeError(f"{target} was built from sources with digest {built}, but the sources here have "
                               f"digest {sources}: rebuild it (python -m nanorts_amd.build)")
        _LIBRARY = lib
    return lib


def check(code: int, what: str) -> None:
    if code != 0:
        message = load().nanorts_amd_last_error().decode()
        raise NativeError(f"{what} failed with code {code}: {message}")
