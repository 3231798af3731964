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


def _tile_label(index: int, types: int) -> str:
    """A readable name of tile `index` of the table, e.g. "wall under player1 heavy"."""
    terrain, occupant = divmod(index, occupant_states(types))
    if occupant == 0:
        return f"empty {TERRAIN_NAMES[terrain]}"
    owner, unit_type = divmod(occupant - 1, types)
    return f"{TERRAIN_NAMES[terrain]} under {OWNER_NAMES[owner]} {TYPE_STEMS[unit_type]}"


def _first_repeat(pictures: np.ndarray) -> tuple[int, int] | None:
    """(earlier, later) indices of the first row of `pictures` [n, bytes]
    that repeats an earlier row, by the later index, or None."""
    _, first, owner = np.unique(pictures, axis=0, return_index=True, return_inverse=True)
    owner = owner.reshape(-1)
    repeats = np.flatnonzero(first[owner] != np.arange(len(pictures)))
    if repeats.size == 0:
        return None
    later = int(repeats[0])
    return int(first[owner[later]]), later


def _sprite_sheet(tiles) -> dict[str, np.ndarray]:
    """The sprites of an Asset set, checked: every name of sprite_names() and
    no other, each a 16x16 RGBA uint8 image, the terrain sprites opaque."""
    names = sprite_names()
    sheet = ({name: read_png(ART_DIRECTORY / f"{name}.png") for name in names} if tiles is None
             else {name: np.asarray(image) for name, image in dict(tiles).items()})
    lacking, extra = sorted(set(names) - set(sheet)), sorted(set(sheet) - set(names))
    if lacking or extra:
        raise RenderError(f"an Asset set names exactly the sprites {list(names)}; this one lacks {lacking} and "
                          f"adds {extra}")
    for name in names:
        image = sheet[name]
        if image.dtype != np.uint8 or image.shape != (SPRITE_PIXELS, SPRITE_PIXELS, 4):
            raise RenderError(f"sprite {name!r} must be uint8 RGBA of {SPRITE_PIXELS}x{SPRITE_PIXELS} pixels, not "
                              f"{image.dtype} {image.shape}")
    for name in TERRAIN_NAMES:
        if (sheet[name][..., 3] < 128).any():
            raise RenderError(f"sprite {name!r} has see-through pixels; a terrain sprite is the ground of its "
                              "cell and must cover all of it")
    return sheet


def prepare_assets(bucket, cell_pixels: int = SPRITE_PIXELS, tiles=None) -> RenderAssets:
    """The tile table of an Asset set (src/nanorts/rendering/assets.py:52-67):
    the shipped sprite sheet, or `tiles`, a mapping from every name of
    sprite_names() to a 16x16 RGBA uint8 image.  Each cell tile is
    `cell_pixels` square (a multiple of 16; sprites are upscaled by pixel
    repetition).  Tile rules (assets.py:133-155): an empty cell is its terrain
    sprite's RGB; an occupied cell is that ground with a ring cell_pixels / 16
    pixels wide in the occupant owner's aura colour, under the occupant's
    sprite wherever its alpha is at least 128.  The table is refused when two
    tiles are equal, or two occupied tiles are equal once the glyph band is
    blanked (assets.py:158-188): the picture would not tell them apart."""
    if cell_pixels < SPRITE_PIXELS or cell_pixels % SPRITE_PIXELS:
        raise RenderError(f"cell_pixels must be a positive multiple of the {SPRITE_PIXELS}-pixel sprite side, "
                          f"not {cell_pixels}")
    types = len(TYPE_STEMS)
    if bucket.unit_type_capacity != types:
        raise RenderError(f"the sprite sheet draws {types} unit types; this bucket has "
                          f"{bucket.unit_type_capacity}")
    sheet = _sprite_sheet(tiles)
    k = cell_pixels // SPRITE_PIXELS

    def enlarge(stack: np.ndarray) -> np.ndarray:  # [..., 16, 16, C] -> [..., P, P, C]
        return stack.repeat(k, axis=-3).repeat(k, axis=-2)

    ground = enlarge(np.stack([sheet[name][..., :3] for name in TERRAIN_NAMES]))            # [2, P, P, 3]
    art = enlarge(np.stack([[sheet[f"{o}-{t}"] for t in TYPE_STEMS] for o in OWNER_NAMES]))  # [3, T, P, P, 4]
    edge = np.zeros((cell_pixels, cell_pixels), bool)
    edge[:k], edge[-k:], edge[:, :k], edge[:, -k:] = True, True, True, True
    aura = np.asarray(AURA_COLOURS, np.uint8)[:, None, None, None, :]                        # [3, 1, 1, 1, 3]
    ringed = np.where(edge[None, None, None, :, :, None], aura[None], ground[:, None, None])  # [2, 3, 1, P, P, 3]
    painted = np.where((art[..., 3:] >= 128)[None], art[None, ..., :3], ringed)             # [2, 3, T, P, P, 3]
    table = np.concatenate([ground[:, None], painted.reshape(2, 3 * types, cell_pixels, cell_pixels, 3)], axis=1)
    table = np.ascontiguousarray(table.reshape(2 * occupant_states(types), cell_pixels, cell_pixels, 3))

    clash = _first_repeat(table.reshape(len(table), -1))
    if clash is not None:
        a, b = clash
        raise RenderError(f"the tiles for {_tile_label(a, types)} and {_tile_label(b, types)} are identical, so an "
                          "image could not tell those cells apart")
    occupied = np.flatnonzero(np.arange(len(table)) % occupant_states(types) != 0)
    blanked = table[occupied].copy()
    blanked[:, BAND_ROWS[0] * k:(BAND_ROWS[-1] + 1) * k, BAND_COLUMN * k:(BAND_COLUMN + BAND_WIDTH) * k] = 0
    clash = _first_repeat(blanked.reshape(len(blanked), -1))
    if clash is not None:
        a, b = (int(occupied[i]) for i in clash)
        raise RenderError(f"the tiles for {_tile_label(a, types)} and {_tile_label(b, types)} differ only inside "
                          "the glyph band, which the hit point / carry / action glyphs overwrite")
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
