"""Pixel surface on the CPU: the sprite decoder against PIL, the tile table's
composite rules, and the oracle's pixel renderer against a closed form (the
symbolic maps of the state drawn through the tile table and glyph band,
src/nanorts/observations/pixels.py:91-110, src/nanorts/rendering/raster.py:53-91)."""
from __future__ import annotations

import numpy as np
import pytest

from nanorts_amd import rendering
from tests.helpers import advanced_states, game_for
from tests.test_oracle import _closed_symbolic


def test_png_reader_matches_pil():
    Image = pytest.importorskip("PIL.Image")
    for name in rendering.sprite_names():
        path = rendering.ART_DIRECTORY / f"{name}.png"
        want = np.asarray(Image.open(path).convert("RGBA"))
        np.testing.assert_array_equal(rendering.read_png(path), want, err_msg=name)


def test_tile_table_composite():
    T = 7
    table = rendering.tile_table(T)
    states = 1 + 3 * T
    assert table.shape == (2 * states, 16, 16, 3)
    assert len({t.tobytes() for t in table}) == 2 * states
    for terrain, name in enumerate(rendering.TERRAIN_NAMES):
        ground = rendering.read_png(rendering.ART_DIRECTORY / f"{name}.png")[..., :3]
        np.testing.assert_array_equal(table[terrain * states], ground)
        for owner in range(3):
            for t, stem in enumerate(rendering.TYPE_STEMS):
                art = rendering.read_png(rendering.ART_DIRECTORY / f"{rendering.OWNER_NAMES[owner]}-{stem}.png")
                tile = table[terrain * states + 1 + owner * T + t]
                drawn = art[..., 3] >= 128
                np.testing.assert_array_equal(tile[drawn], art[..., :3][drawn])
                # the aura ring shows wherever the sprite is transparent
                ring = np.zeros((16, 16), bool)
                ring[0, :] = ring[-1, :] = ring[:, 0] = ring[:, -1] = True
                assert (tile[ring & ~drawn] == rendering.AURA_COLOURS[owner]).all()
                inside = ~ring & ~drawn
                np.testing.assert_array_equal(tile[inside], ground[inside])


def render_maps(maps: np.ndarray, tiles: np.ndarray, T: int) -> np.ndarray:
    """Closed form of pixels_from_symbolic for uint8 maps [..., H, W, 6]."""
    m = maps.astype(np.int32)
    hp, carried, owner, utype, kind, terrain = (m[..., i] for i in range(6))
    present = utype != 0
    states = 1 + 3 * T
    occupant = np.where(present, 1 + owner * T + (utype - 1), 0)  # owner here is symbolic (0/1/2)
    cells = tiles[np.clip(terrain * states + occupant, 0, 2 * states - 1)].copy()  # [..., H, W, 16, 16, 3]
    x = np.arange(16)
    pos = np.clip(x - 1, 0, 13)
    lit12 = kind[..., None] == pos + 1
    lit13 = ((carried[..., None] >> pos) & 1) != 0
    lit14 = hp[..., None] > pos
    band_cols = (x >= 1) & (x < 15)
    for row, lit in ((12, lit12), (13, lit13), (14, lit14)):
        on = present[..., None] & band_cols
        colour = np.where(lit, 255, 0).astype(np.uint8)
        sel = cells[..., row, :, :]
        sel[on] = colour[on][:, None]
        cells[..., row, :, :] = sel
    lead = maps.shape[:-3]
    H, W = maps.shape[-3], maps.shape[-2]
    out = np.moveaxis(cells, -4, -3)  # [..., H, 16, W, 16, 3]
    return out.reshape(*lead, H * 16, W * 16, 3)


@pytest.mark.parametrize("case", ["16x16-random-partial", "melee-both"])
@pytest.mark.parametrize("partial", [False, True])
def test_oracle_pixels_closed_form(case, partial):
    game, _ = game_for(case)
    T = game.bucket.unit_type_capacity
    o, st = advanced_states(game, 4, 140, partial, 4, seed=13)
    tiles = rendering.tile_table(T)
    image, scalars = o.pixels(st, partial, tiles)
    maps, want_scalars = _closed_symbolic(game, st, partial)
    np.testing.assert_array_equal(image, render_maps(maps, tiles, T))
    np.testing.assert_array_equal(scalars, want_scalars)


def _bucket(types=7):
    class B:
        unit_type_capacity = types
    return B()


def _sheet():
    return {name: rendering.read_png(rendering.ART_DIRECTORY / f"{name}.png") for name in rendering.sprite_names()}


def test_prepare_assets_upscales_and_checks_the_sheet():
    """prepare_assets (src/nanorts/rendering/assets.py:52-195): 16-pixel
    cells give the shipped table; 32-pixel cells are its exact 2x upscale
    (ground, art and the ring all scale by pixel repetition); every refusal
    of the asset contract fires."""
    base = rendering.prepare_assets(_bucket())
    np.testing.assert_array_equal(base.tiles, rendering.tile_table(7))
    double = rendering.prepare_assets(_bucket(), cell_pixels=32)
    np.testing.assert_array_equal(double.tiles, np.repeat(np.repeat(base.tiles, 2, axis=1), 2, axis=2))
    assert double.cell_pixels == 32 and double.unit_type_capacity == 7
    for bad in (0, 24, -16):
        with pytest.raises(rendering.RenderError):
            rendering.prepare_assets(_bucket(), cell_pixels=bad)
    with pytest.raises(rendering.RenderError):
        rendering.prepare_assets(_bucket(6))
    sheet = _sheet()
    missing = dict(sheet)
    del missing["player0-worker"]
    with pytest.raises(rendering.RenderError, match="lacks"):
        rendering.prepare_assets(_bucket(), tiles=missing)
    see_through = dict(sheet)
    see_through["wall"] = sheet["wall"].copy()
    see_through["wall"][0, 0, 3] = 0
    with pytest.raises(rendering.RenderError, match="see-through"):
        rendering.prepare_assets(_bucket(), tiles=see_through)
    small = dict(sheet)
    small["floor"] = sheet["floor"][:8]
    with pytest.raises(rendering.RenderError, match="must be uint8"):
        rendering.prepare_assets(_bucket(), tiles=small)
    twins = dict(sheet)
    twins["player0-light"] = sheet["player0-heavy"]
    with pytest.raises(rendering.RenderError, match="identical"):
        rendering.prepare_assets(_bucket(), tiles=twins)
    band = dict(sheet)
    band["player0-light"] = sheet["player0-heavy"].copy()
    band["player0-light"][13, 5, :3] ^= 0x01  # inside the glyph band
    band["player0-light"][13, 5, 3] = 255
    with pytest.raises(rendering.RenderError, match="glyph band"):
        rendering.prepare_assets(_bucket(), tiles=band)
    # a recoloured sheet is accepted and changes only what it draws
    tinted = {name: image.copy() for name, image in sheet.items()}
    tinted["floor"][..., 0] ^= 0x40
    custom = rendering.prepare_assets(_bucket(), tiles=tinted)
    assert not np.array_equal(custom.tiles[0], base.tiles[0])
    np.testing.assert_array_equal(custom.tiles[1 + 3 * 7], base.tiles[1 + 3 * 7])  # the wall + empty tile
