"""Tile table of the pixel observation surface.

The pixel kernel draws each cell as a 16x16 RGB tile picked by
terrain * (1 + 3T) + occupant, occupant = 0 (empty) or 1 + (owner + 1) * T +
type with owner -1 neutral, 0 the observer, 1 the opponent, then overlays
the glyph band (rows 12-14, columns 1-14: pending kind one-hot, carried
resources in binary, hit points in unary).  This module builds the table on
the host from the sprite sheet under nanorts_amd/art (16x16 RGBA PNGs):
ground = the terrain sprite's RGB; a 1-pixel ring in the owner's aura colour;
sprite pixels with alpha >= 128 drawn over it
(src/nanorts/rendering/assets.py:52-155, src/nanorts/rendering/raster.py:17-67).

The PNG reader is a small stdlib (zlib) decoder for the non-interlaced
8-bit RGBA files the sprite sheet holds.
"""
from __future__ import annotations

import functools
import struct
import zlib
from pathlib import Path

import numpy as np

ART_DIRECTORY = Path(__file__).resolve().parent / "art"
SPRITE_PIXELS = 16
TERRAIN_NAMES = ("floor", "wall")
OWNER_NAMES = ("neutral", "player0", "player1")
TYPE_STEMS = ("resource", "base", "barracks", "worker", "light", "heavy", "ranged")
AURA_COLOURS = ((0xAD, 0xBB, 0xC7), (0x0C, 0x7B, 0xDC), (0xBF, 0x36, 0x82))
BAND_ROWS = (12, 13, 14)
BAND_COLUMN = 1
BAND_WIDTH = SPRITE_PIXELS - 2 * BAND_COLUMN


class RenderError(Exception):
    pass


def _paeth(a: int, b: int, c: int) -> int:
    p = a + b - c
    pa, pb, pc = abs(p - a), abs(p - b), abs(p - c)
    if pa <= pb and pa <= pc:
        return a
    return b if pb <= pc else c


def read_png(path: Path) -> np.ndarray:
    """uint8[H, W, 4] from an 8-bit RGBA (colour type 6), non-interlaced PNG."""
    data = Path(path).read_bytes()
    if data[:8] != b"\x89PNG\r\n\x1a\n":
        raise RenderError(f"{path} is not a PNG file")
    pos, idat, header = 8, b"", None
    while pos < len(data):
        (length,) = struct.unpack(">I", data[pos:pos + 4])
        kind = data[pos + 4:pos + 8]
        body = data[pos + 8:pos + 8 + length]
        pos += 12 + length
        if kind == b"IHDR":
            header = struct.unpack(">IIBBBBB", body)
        elif kind == b"IDAT":
            idat += body
        elif kind == b"IEND":
            break
    if header is None:
        raise RenderError(f"{path} has no IHDR chunk")
    width, height, depth, colour, _, _, interlace = header
    if depth != 8 or colour != 6 or interlace != 0:
        raise RenderError(f"{path}: only 8-bit non-interlaced RGBA is read (depth {depth}, colour {colour})")
    raw = zlib.decompress(idat)
    bpp, stride = 4, width * 4
    out = bytearray(height * stride)
    prev = bytearray(stride)
    for y in range(height):
        f = raw[y * (stride + 1)]
        line = bytearray(raw[y * (stride + 1) + 1:(y + 1) * (stride + 1)])
        for x in range(stride):
            a = line[x - bpp] if x >= bpp else 0
            b = prev[x]
            c = prev[x - bpp] if x >= bpp else 0
            if f == 1:
                line[x] = (line[x] + a) & 0xFF
            elif f == 2:
                line[x] = (line[x] + b) & 0xFF
            elif f == 3:
                line[x] = (line[x] + ((a + b) >> 1)) & 0xFF
            elif f == 4:
                line[x] = (line[x] + _paeth(a, b, c)) & 0xFF
            elif f != 0:
                raise RenderError(f"{path}: unknown PNG filter {f}")
        out[y * stride:(y + 1) * stride] = line
        prev = line
    return np.frombuffer(bytes(out), np.uint8).reshape(height, width, 4)


def sprite_names() -> tuple[str, ...]:
    return TERRAIN_NAMES + tuple(f"{o}-{t}" for o in OWNER_NAMES for t in TYPE_STEMS)


def occupant_states(types: int) -> int:
    return 1 + 3 * types


@functools.lru_cache(maxsize=4)
def tile_table(types: int = len(TYPE_STEMS)) -> np.ndarray:
    """uint8[2 * (1 + 3T), 16, 16, 3]: index terrain * (1 + 3T) + occupant."""
    if types != len(TYPE_STEMS):
        raise RenderError(f"the sprite sheet draws {len(TYPE_STEMS)} unit types, the game has {types}")
    sprites = {name: read_png(ART_DIRECTORY / f"{name}.png") for name in sprite_names()}
    for name, image in sprites.items():
        if image.shape != (SPRITE_PIXELS, SPRITE_PIXELS, 4):
            raise RenderError(f"sprite {name} is {image.shape}, expected (16, 16, 4)")
    for name in TERRAIN_NAMES:
        if not (sprites[name][..., 3] >= 128).all():
            raise RenderError(f"terrain sprite {name} is not opaque")
    ring = np.zeros((SPRITE_PIXELS, SPRITE_PIXELS), bool)
    ring[0, :] = ring[-1, :] = ring[:, 0] = ring[:, -1] = True
    states = occupant_states(types)
    table = np.zeros((2 * states, SPRITE_PIXELS, SPRITE_PIXELS, 3), np.uint8)
    for terrain, tname in enumerate(TERRAIN_NAMES):
        ground = sprites[tname][..., :3]
        table[terrain * states] = ground
        for owner_bucket, oname in enumerate(OWNER_NAMES):
            for t, stem in enumerate(TYPE_STEMS):
                art = sprites[f"{oname}-{stem}"]
                tile = ground.copy()
                tile[ring] = AURA_COLOURS[owner_bucket]
                drawn = art[..., 3] >= 128
                tile[drawn] = art[..., :3][drawn]
                table[terrain * states + 1 + owner_bucket * types + t] = tile
    return table
