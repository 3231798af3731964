"""The C-ABI library builds for gfx950, loads, and exports every entry point
include/nanorts_amd.h declares (no compute calls: this runs without a GPU)."""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

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
    assert lib.nanorts_amd_build_id().decode() == build.source_digest()
    targets = lib.nanorts_amd_entries().decode().split(",")
    for target in ("nanorts_amd_step", "nanorts_amd_legality", "nanorts_amd_legality_words", "nanorts_amd_visible_cells",
                   "nanorts_amd_reset_where_done"):
        assert target in targets


def test_invalid_game_is_refused_without_touching_a_device():
    lib = native.load()
    game = native.Game()
    game.height, game.width, game.cells = 4, 4, 17  # inconsistent
    code = lib.nanorts_amd_legality_words(None, ctypes.byref(game), native.State(), 1, None)
    assert code == 1
    assert "cells" in lib.nanorts_amd_last_error().decode()


def test_targets_name_every_compute_entry_point():
    lib = native.load()
    targets = set(lib.nanorts_amd_entries().decode().split(","))
    meta = {"nanorts_amd_build_id", "nanorts_amd_entries", "nanorts_amd_last_error", "nanorts_amd_shared_opt_in",
            "nanorts_amd_self_check", "nanorts_amd_self_check_no_alloc", "nanorts_amd_rollout_first_pass"}
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
    code = lib.nanorts_amd_seat_step_lanes(None, ctypes.byref(game), state, 1, 0, 4, None, 1, carry, addr, 0, results)
    assert code == 1 and "seats is NULL" in lib.nanorts_amd_last_error().decode()
    code = lib.nanorts_amd_seat_step(None, ctypes.byref(game), state, 1, 0, 4, 2, carry, addr, 0, results)
    assert code == 1 and "learner must be 0 or 1" in lib.nanorts_amd_last_error().decode()
    key = (ctypes.c_uint32 * 2)(1, 2)
    code = lib.nanorts_amd_seat_rollout_lanes(None, ctypes.byref(game), state, 1, 0, 4, None, 1, None, carry, key, 0, 1,
                                          0, 0, native.RolloutResults())
    assert code == 1 and "seats is NULL" in lib.nanorts_amd_last_error().decode()
    code = lib.nanorts_amd_episode_seats(None, None, addr, 1, addr)
    assert code == 1 and "NULL" in lib.nanorts_amd_last_error().decode()
    code = lib.nanorts_amd_episode_seats(None, addr, addr, -1, addr)
    assert code == 1 and "lanes" in lib.nanorts_amd_last_error().decode()
    assert lib.nanorts_amd_episode_seats(None, addr, addr, 0, addr) == 0


# The reference's own C-ABI names: its registry functions
# (src/nanorts/kernels/cuda/registry.cu:201-230) and its XLA FFI targets.  An
# FFI shim defines these; the kernel library must not, or the two collide.
REFERENCE_SYMBOLS = ("nanorts_build_id", "nanorts_targets", "nanorts_shared_opt_in", "nanorts_self_check",
                     "nanorts_step", "nanorts_step_groups", "nanorts_legality", "nanorts_legality_words",
                     "nanorts_visible_cells", "nanorts_reset_where_done", "nanorts_reset_packed_where_done",
                     "nanorts_abstraction_act", "nanorts_gridnet_decode")


def test_library_exports_no_reference_symbol():
    lib = ctypes.CDLL(str(build.library_path()))
    for name in REFERENCE_SYMBOLS:
        assert not hasattr(lib, name), name


def test_load_refuses_a_library_built_from_other_sources(monkeypatch):
    monkeypatch.setattr(native, "_LIBRARY", None)
    monkeypatch.setattr(native._build, "source_digest", lambda: "0" * 16)
    with pytest.raises(RuntimeError, match="rebuild"):
        native.load()


def test_step_ffi_refuses_bad_arguments_without_touching_a_device():
    """nanorts_amd_step_ffi validates its operand and result lists, extents
    and strategy before any copy or launch."""
    lib = native.load()
    buf = (ctypes.c_uint8 * 64)()
    addr = ctypes.cast(buf, ctypes.c_void_p).value
    operands = (ctypes.c_void_p * 33)(*[addr] * 33)
    results = (ctypes.c_void_p * 31)(*[addr] * 31)
    ok = dict(lanes=4, key_lanes=1, command_lanes=4, height=8, width=8, neutral=2, capacity=47, types=7, strategy=0)

    def call(ops=operands, rets=results, **kw):
        a = {**ok, **kw}
        return lib.nanorts_amd_step_ffi(None, ops, rets, a["lanes"], a["key_lanes"], a["command_lanes"], a["height"],
                                        a["width"], a["neutral"], a["capacity"], a["types"], a["strategy"])

    assert call(strategy=3) == 1 and "strategy" in lib.nanorts_amd_last_error().decode()
    assert call(key_lanes=2) == 1 and "key" in lib.nanorts_amd_last_error().decode()
    assert call(command_lanes=3) == 1 and "Commands" in lib.nanorts_amd_last_error().decode()
    holes = (ctypes.c_void_p * 33)(*[addr] * 33)
    holes[8] = None  # the table operand
    assert call(ops=holes) == 1 and "operand 8" in lib.nanorts_amd_last_error().decode()
    assert call(types=9) == 1 and "types" in lib.nanorts_amd_last_error().decode()
    assert call(ops=None) == 1


def test_no_alloc_self_check_refuses_sizes_beyond_its_scratch():
    lib = native.load()
    device = (ctypes.c_int32 * 1)(0)
    for waves in (0, 1025, -1):
        message = lib.nanorts_amd_self_check_no_alloc(device, 1, waves, None).decode()
        assert "1 to 1024" in message, message


def test_operand_entries_refuse_bad_arguments_without_touching_a_device():
    """The legality, visibility and reset entries in the reference's operand
    forms validate their buffers and extents before any launch."""
    lib = native.load()
    buf = (ctypes.c_uint8 * 64)()
    addr = ctypes.cast(buf, ctypes.c_void_p).value
    err = lambda: lib.nanorts_amd_last_error().decode()  # noqa: E731

    nine = (ctypes.c_void_p * 9)(*[addr] * 9)
    assert lib.nanorts_amd_legality_ffi(None, nine, None, 1, 4, 8, 8, 96, 47, 7, 49) == 1 and "NULL" in err()
    holes = (ctypes.c_void_p * 9)(*[addr] * 9)
    holes[8] = None
    assert lib.nanorts_amd_legality_ffi(None, holes, addr, 1, 4, 8, 8, 96, 47, 7, 49) == 1 and "operand 8" in err()
    assert lib.nanorts_amd_legality_ffi(None, nine, addr, 1, 4, 8, 8, 96, 47, 7, 48) == 1 and "odd square" in err()
    assert lib.nanorts_amd_legality_ffi(None, nine, addr, 0, 4, 8, 8, 90, 47, 7, 49) == 1 and "entities" in err()

    def visible(**kw):
        a = dict(birth=addr, birth_lanes=4, unit_type=addr, unit_type_lanes=1, cell=addr, cell_bytes=2, cell_lanes=4,
                 slots=16, radius=addr, types=7, out=addr, lanes=4, first=2, count=7, width=8, height=8)
        a.update(kw)
        return lib.nanorts_amd_visible_cells_ffi(None, *a.values())

    assert visible(cell_bytes=3) == 1 and "1, 2 or 4" in err()
    assert visible(width=300, height=200) == 1 and "48K" in err()
    assert visible(birth_lanes=2) == 1 and "shared row" in err()
    assert visible(first=10, count=7) == 1 and "block" in err()
    assert visible(out=None) == 1 and "NULL" in err()
    assert visible(lanes=0) == 0

    ptrs = (ctypes.c_void_p * 2)(addr, addr)
    one = (ctypes.c_int64 * 2)(1, 4)
    rows = (ctypes.c_int64 * 2)(16, 16)
    assert lib.nanorts_amd_reset_rows_ffi(None, addr, 4, 33, ptrs, one, ptrs, ptrs, rows) == 1 and "0 to 32" in err()
    bad = (ctypes.c_int64 * 2)(1, 3)
    assert lib.nanorts_amd_reset_rows_ffi(None, addr, 4, 2, ptrs, bad, ptrs, ptrs, rows) == 1 and "shared row" in err()
    assert lib.nanorts_amd_reset_rows_ffi(None, None, 4, 2, ptrs, one, ptrs, ptrs, rows) == 1 and "NULL" in err()
    assert lib.nanorts_amd_reset_rows_ffi(None, addr, 0, 2, ptrs, one, ptrs, ptrs, rows) == 0
