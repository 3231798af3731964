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

import dataclasses
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


@dataclasses.dataclass(frozen=True, eq=False)
class RenderAssets:
    """A prepared tile table (src/nanorts/rendering/raster.py RenderAssets):
    uint8[2 * (1 + 3T), cell_pixels, cell_pixels, 3]."""

    tiles: np.ndarray
    cell_pixels: int
    unit_type_capacity: int


def _class_name(index: int, types: int) -> str:
    terrain, occupant = divmod(index, occupant_states(types))
    if occupant == 0:
        return f"{TERRAIN_NAMES[terrain]} + empty"
    owner, unit_type = divmod(occupant - 1, types)
    return f"{TERRAIN_NAMES[terrain]} + {OWNER_NAMES[owner]} {TYPE_STEMS[unit_type]}"


def prepare_assets(bucket, cell_pixels: int = SPRITE_PIXELS, tiles=None) -> RenderAssets:
    """src/nanorts/rendering/assets.py:52-195: the tile table from the
    shipped sprite sheet (or `tiles`, a name -> 16x16 RGBA uint8 mapping
    naming every sprite of sprite_names()), each sprite upscaled to
    `cell_pixels` (a multiple of 16) with a ring of cell_pixels / 16 pixels.
    Refuses a table whose tiles would be indistinguishable: two equal
    composites, or two occupied tiles equal outside the glyph band."""
    if cell_pixels <= 0 or cell_pixels % SPRITE_PIXELS:
        raise RenderError(f"cell_pixels is {cell_pixels}, expected a positive integer multiple of the "
                          f"{SPRITE_PIXELS}-pixel sprite side")
    types = len(TYPE_STEMS)
    if bucket.unit_type_capacity != types:
        raise RenderError(f"BucketSpec.unit_type_capacity is {bucket.unit_type_capacity}, and an Asset set draws the "
                          f"{types} types the supported unit type table holds")
    names = sprite_names()
    supplied = ({name: read_png(ART_DIRECTORY / f"{name}.png") for name in names} if tiles is None
                else dict(tiles))
    if set(supplied) != set(names):
        raise RenderError(f"the Asset set does not name the Tile classes a Bucket of {types} unit types has: it is "
                          f"missing {sorted(set(names) - set(supplied))} and holds an unused "
                          f"{sorted(set(supplied) - set(names))}")
    sprites = {}
    for name in names:
        image = np.asarray(supplied[name])
        if image.shape != (SPRITE_PIXELS, SPRITE_PIXELS, 4) or image.dtype != np.uint8:
            raise RenderError(f"the sprite {name!r} is {image.shape} {image.dtype}, expected a "
                              f"({SPRITE_PIXELS}, {SPRITE_PIXELS}, 4) uint8 RGBA image")
        sprites[name] = image
    for name in TERRAIN_NAMES:
        if not (sprites[name][..., 3] >= 128).all():
            raise RenderError(f"the terrain tile {name!r} is not fully opaque, and terrain is the ground every "
                              "occupant is drawn over")
    scale = cell_pixels // SPRITE_PIXELS

    def up(image: np.ndarray) -> np.ndarray:
        return np.repeat(np.repeat(image, scale, axis=0), scale, axis=1)

    ring = np.zeros((cell_pixels, cell_pixels), bool)
    ring[:scale, :] = ring[-scale:, :] = ring[:, :scale] = ring[:, -scale:] = True
    states = occupant_states(types)
    table = np.zeros((2 * states, cell_pixels, cell_pixels, 3), np.uint8)
    for terrain, tname in enumerate(TERRAIN_NAMES):
        ground = up(sprites[tname])[..., :3]
        table[terrain * states] = ground
        for owner_bucket, oname in enumerate(OWNER_NAMES):
            for t, stem in enumerate(TYPE_STEMS):
                art = up(sprites[f"{oname}-{stem}"])
                tile = ground.copy()
                tile[ring] = AURA_COLOURS[owner_bucket]
                drawn = art[..., 3] >= 128
                tile[drawn] = art[..., :3][drawn]
                table[terrain * states + 1 + owner_bucket * types + t] = tile
    band_rows = slice(BAND_ROWS[0] * scale, (BAND_ROWS[-1] + 1) * scale)
    band_cols = slice(BAND_COLUMN * scale, (BAND_COLUMN + BAND_WIDTH) * scale)
    composites: dict[bytes, str] = {}
    outside: dict[bytes, str] = {}
    for index, tile in enumerate(table):
        name = _class_name(index, types)
        for seen, picture, verb in ((composites, tile.tobytes(), "composite"), (outside, None, "draw as")):
            if picture is None:
                if index % states == 0:
                    continue
                blanked = tile.copy()
                blanked[band_rows, band_cols] = 0
                picture = blanked.tobytes()
            if picture in seen:
                raise RenderError(f"the Tile classes {seen[picture]!r} and {name!r} {verb} the same picture, which "
                                  "would make them indistinguishable in a Rendering")
            seen[picture] = name
    return RenderAssets(tiles=table, cell_pixels=cell_pixels, unit_type_capacity=types)


@functools.lru_cache(maxsize=4)
def tile_table(types: int = len(TYPE_STEMS)) -> np.ndarray:
    """uint8[2 * (1 + 3T), 16, 16, 3] of the shipped sprite sheet: index
    terrain * (1 + 3T) + occupant."""
    if types != len(TYPE_STEMS):
        raise RenderError(f"the sprite sheet draws {len(TYPE_STEMS)} unit types, the game has {types}")

    class _Types:
        unit_type_capacity = types

    return prepare_assets(_Types()).tiles
