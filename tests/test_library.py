"""The C-ABI library builds for gfx950, loads, and exports every entry point
include/nanorts_amd.h declares (no compute calls: this runs without a GPU)."""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

from nanorts_amd import build, native

ROOT = Path(__file__).resolve().parent.parent


def declared_entry_points() -> list[str]:
    text = (ROOT / "include" / "nanorts_amd.h").read_text()
    return sorted(set(re.findall(r"^(?:const char\*|int|int64_t)\s+(nanorts_\w+)\s*\(", text, flags=re.M)))


def test_header_declarations_match_binding():
    assert declared_entry_points() == sorted(native.EXPORTS)


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(str(build.library_path()))
    for name in declared_entry_points():
        assert hasattr(lib, name), name


def test_build_id_and_targets():
    lib = native.load()
    assert lib.nanorts_build_id().decode() == build.source_digest()
    targets = lib.nanorts_targets().decode().split(",")
    for target in ("nanorts_step", "nanorts_legality", "nanorts_legality_words", "nanorts_visible_cells",
                   "nanorts_reset_where_done"):
        assert target in targets


def test_invalid_game_is_refused_without_touching_a_device():
    lib = native.load()
    game = native.Game()
    game.height, game.width, game.cells = 4, 4, 17  # inconsistent
    code = lib.nanorts_legality_words(None, ctypes.byref(game), native.State(), 1, None)
    assert code == 1
    assert "cells" in lib.nanorts_last_error().decode()


def test_targets_name_every_compute_entry_point():
    lib = native.load()
    targets = set(lib.nanorts_targets().decode().split(","))
    meta = {"nanorts_build_id", "nanorts_targets", "nanorts_last_error", "nanorts_shared_opt_in", "nanorts_self_check"}
    assert targets == set(declared_entry_points()) - meta


def test_seat_entry_points_refuse_bad_arguments_without_touching_a_device():
    """The per-lane seat entries validate before any launch: NULL seats, a
    learner outside 0/1, NULL or negative-size episode seat operands."""
    lib = native.load()
    buf = (ctypes.c_uint8 * 64)()
    addr = ctypes.cast(buf, ctypes.c_void_p)
    state = native.State(*[addr] * len(native.STATE_FIELDS))
    carry = native.AbstractActions(*[addr] * len(native.ABSTRACT_FIELDS))
    results = native.EnvResults()
    game = native.Game()
    code = lib.nanorts_seat_step_lanes(None, ctypes.byref(game), state, 1, 0, 4, None, 1, carry, addr, 0, results)
    assert code == 1 and "seats is NULL" in lib.nanorts_last_error().decode()
    code = lib.nanorts_seat_step(None, ctypes.byref(game), state, 1, 0, 4, 2, carry, addr, 0, results)
    assert code == 1 and "learner must be 0 or 1" in lib.nanorts_last_error().decode()
    key = (ctypes.c_uint32 * 2)(1, 2)
    code = lib.nanorts_seat_rollout_lanes(None, ctypes.byref(game), state, 1, 0, 4, None, 1, None, carry, key, 0, 1,
                                          0, 0, native.RolloutResults())
    assert code == 1 and "seats is NULL" in lib.nanorts_last_error().decode()
    code = lib.nanorts_episode_seats(None, None, addr, 1, addr)
    assert code == 1 and "NULL" in lib.nanorts_last_error().decode()
    code = lib.nanorts_episode_seats(None, addr, addr, -1, addr)
    assert code == 1 and "lanes" in lib.nanorts_last_error().decode()
    assert lib.nanorts_episode_seats(None, addr, addr, 0, addr) == 0
