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
