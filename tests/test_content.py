"""The content loader (CPU only): map XML -> GameConfig.

Covers the reference loader's contract (src/nanorts/content/loading.py,
acceptance.py, normalize.py, scenarios.py): every acceptance clause refuses
with its clause number, a built game equals the loaded one, a supplied
BucketSpec is checked against the derived one, the slot capacities follow
the resource bound (pinned by hand on three shipped maps), units go into
their blocks in document order, and another unit type table must keep the
types and the attack window.
"""
from __future__ import annotations

import dataclasses

import numpy as np
import pytest

from nanorts_amd import content
from nanorts_amd.content import (ContentError, UnitRecord, build_game, load_game, map_name_to_scenario,
                                 read_map_xml, scenario_names, shipped_map, with_unit_type_table)
from nanorts_amd.model import ConflictStrategy, UnitTypeTableVersion

BASE = """<rts.PhysicalGameState width="{w}" height="{h}">
  <terrain>{terrain}</terrain>
  <players>
{players}
  </players>
  <units>
{units}
  </units>
</rts.PhysicalGameState>
"""
PLAYERS = ('    <rts.Player ID="0" resources="5"></rts.Player>\n'
           '    <rts.Player ID="1" resources="5"></rts.Player>')
UNITS = ('    <rts.units.Unit type="Resource" ID="1" player="-1" x="0" y="0" resources="20" hitpoints="1"/>\n'
         '    <rts.units.Unit type="Base" ID="2" player="0" x="1" y="1" resources="0" hitpoints="10"/>\n'
         '    <rts.units.Unit type="Worker" ID="3" player="0" x="2" y="1" resources="0" hitpoints="1"/>\n'
         '    <rts.units.Unit type="Base" ID="4" player="1" x="3" y="3" resources="0" hitpoints="10"/>\n'
         '    <rts.units.Unit type="Worker" ID="5" player="1" x="2" y="3" resources="0" hitpoints="1"/>')


def _doc(w=4, h=4, terrain=None, players=PLAYERS, units=UNITS):
    return BASE.format(w=w, h=h, terrain="0" * (w * h) if terrain is None else terrain, players=players, units=units)


def _write(tmp_path, text):
    path = tmp_path / "m.xml"
    path.write_text(text)
    return path


def _refused(tmp_path, text, clause):
    with pytest.raises(ContentError) as info:
        load_game(_write(tmp_path, text))
    assert info.value.clause == clause, str(info.value)
    assert str(info.value).startswith(f"clause {clause}:")


def test_a_good_document_loads(tmp_path):
    game = load_game(_write(tmp_path, _doc()))
    st = game.initial_state
    b = game.bucket
    assert (b.height, b.width, b.neutral_capacity) == (4, 4, 1)
    # units in document order: births 0..4, each in its block's next slot
    assert st["birth"][0] == 0 and st["unit_type"][0] == 0 and st["owner"][0] == -1
    p0, p1 = b.player_slot_start(0), b.player_slot_start(1)
    assert list(st["birth"][p0:p0 + 2]) == [1, 2] and list(st["birth"][p1:p1 + 2]) == [3, 4]
    assert list(st["cell"][p0:p0 + 2]) == [1 + 4, 2 + 4] and st["entity_at"][1, 2] == p0 + 1
    assert st["hit_points"][p0] == 10 and st["carried_resources"][0] == 20
    assert list(st["player_resources"]) == [5, 5] and int(st["next_birth"]) == 5
    assert not bool(st["game_over"]) and int(st["winner"]) == -1


@pytest.mark.parametrize("text, clause", [
    ("<rts.PhysicalGameState width='4'", 1),                                      # not XML
    (_doc().replace('width="4"', 'width="four"'), 1),                              # not an integer
    (_doc().replace('width="4"', 'width="0"'), 1),                                 # not positive
    (_doc().replace('width="4"', 'width="4294967296"'), 1),                        # outside int32
    (_doc(terrain="0" * 15), 2),                                                   # too short
    (_doc(terrain="0" * 15 + "x"), 2),                                             # not a digit
    (_doc(terrain="0" * 15 + "2"), 3),                                             # not binary
    (_doc(players='    <rts.Player ID="0" resources="5"></rts.Player>'), 4),       # one record
    (_doc(players=PLAYERS.replace('ID="1"', 'ID="2"')), 4),                        # not positional
    (_doc(players=PLAYERS.replace('resources="5"', 'resources="9999999999"', 1)), 4),
    (_doc(units=UNITS.replace('type="Worker" ID="3"', 'type="Dragon" ID="3"')), 5),  # unknown type
    (_doc(units=UNITS.replace('ID="3"', 'ID="2"')), 5),                            # duplicate ID
    (_doc(units=UNITS.replace('x="2" y="1"', 'x="4" y="1"')), 5),                  # off the board
    (_doc(units=UNITS.replace('x="2" y="1"', 'x="1" y="1"')), 5),                  # occupied
    (_doc(units=UNITS.replace('player="0" x="2"', 'player="3" x="2"')), 5),        # undeclared owner
    (_doc(units=UNITS.replace('ID="3" player="0"', 'ID="3"')), 5),                 # missing attribute
    (_doc(units=UNITS.replace('hitpoints="10"', 'hitpoints="32768"', 1)), 6),      # hit points
    (_doc(units=UNITS.replace('hitpoints="1"/>', 'hitpoints="-1"/>', 1)), 6),
])
def test_each_clause_refuses_with_its_number(tmp_path, text, clause):
    _refused(tmp_path, text, clause)


def test_build_game_equals_the_loaded_map():
    loaded = load_game(shipped_map("basesWorkers8x8"))
    doc = read_map_xml(shipped_map("basesWorkers8x8").read_text())
    built = build_game(width=doc.width, height=doc.height, terrain=doc.terrain,
                       players=[resources for _, resources in doc.players], units=doc.units)
    assert built.bucket == loaded.bucket
    for name, want in loaded.initial_state.items():
        np.testing.assert_array_equal(built.initial_state[name], want, err_msg=name)
    np.testing.assert_array_equal(built.terrain, loaded.terrain)
    with pytest.raises(ContentError) as info:
        build_game(width=2, height=2, terrain="0000", players=[0, 0],
                   units=[UnitRecord("Worker", 1, 0, 0, 0, 1, 0), UnitRecord("Worker", 2, 1, 0, 0, 1, 0)])
    assert info.value.clause == 5


def test_capacities_follow_the_resource_bound():
    """Hand-computed resource bounds (normalize.py:45-93): a player can own at
    most its population plus (its resources + every pile's resources) // the
    cheapest producible cost (a Worker, 1), capped at the cell count.
    basesWorkers8x8: 2 + (5 + 20 + 20) // 1 = 47 of 64 cells.
    basesWorkers4x4: 2 + 45 = 47, capped at the 16 cells.
    melee8x8Mixed4: no piles and no resources: its population, 4."""
    expect = {"basesWorkers8x8": (47, 2), "basesWorkers4x4": (16, 2), "melee8x8Mixed4": (4, 0)}
    for name, (capacity, neutral) in expect.items():
        b = load_game(shipped_map(name)).bucket
        assert (b.per_player_capacity, b.neutral_capacity) == (capacity, neutral), name
        assert b.unit_type_capacity == 7 and b.attack_offset_capacity == 49
    # the shipped capacity profile caps 16x16 at 70 slots per player
    assert map_name_to_scenario("basesWorkers16x16").bucket.per_player_capacity == 70
    assert map_name_to_scenario("basesWorkers16x16", capacity_profile=False).bucket.per_player_capacity > 70
    assert set(scenario_names()) >= {"basesWorkers8x8", "basesWorkers16x16", "GardenOfWar64x64"}


def test_a_supplied_bucket_is_checked(tmp_path):
    path = _write(tmp_path, _doc())
    derived = load_game(path).bucket
    wider = dataclasses.replace(derived, per_player_capacity=derived.cell_count)
    assert load_game(path, bucket=wider).bucket == wider
    narrow = dataclasses.replace(derived, per_player_capacity=2, neutral_capacity=3)
    game = load_game(path, bucket=narrow)
    assert game.bucket == narrow and game.initial_state["birth"].shape == (3 + 2 * 2,)
    for bad in (dataclasses.replace(derived, per_player_capacity=1),        # below the population
                dataclasses.replace(derived, neutral_capacity=0),
                dataclasses.replace(derived, per_player_capacity=17),       # above the cells
                dataclasses.replace(derived, width=5),
                dataclasses.replace(derived, conflict_strategy=ConflictStrategy.CANCEL_RANDOM)):
        with pytest.raises(ContentError):
            load_game(path, bucket=bad)


def test_another_unit_type_table_keeps_the_content():
    game = map_name_to_scenario("basesWorkers8x8", utt=UnitTypeTableVersion.ORIGINAL_FINETUNED)
    other = with_unit_type_table(game, UnitTypeTableVersion.ORIGINAL)
    assert other.bucket.utt_identity == UnitTypeTableVersion.ORIGINAL
    assert other.initial_state is game.initial_state
    assert with_unit_type_table(game, UnitTypeTableVersion.ORIGINAL_FINETUNED) is game
    with pytest.raises(ContentError):
        with_unit_type_table(game, "no-such-table")


def test_every_shipped_map_loads():
    """All 138 maps the reference ships (src/nanorts/maps) load under both
    unit tables, with int16 indices, a decided initial state and every unit
    on its own cell."""
    names = scenario_names()
    assert len(names) == 138 and len(set(names)) == 138
    for name in names:
        for utt in UnitTypeTableVersion:
            game = map_name_to_scenario(name, utt=utt)
            st, b = game.initial_state, game.bucket
            live = st["birth"] != -1
            assert (st["entity_at"] != -1).sum() == live.sum(), name
            cells = st["cell"][live].astype(np.int64)
            assert len(set(cells.tolist())) == live.sum(), name
            assert (st["entity_at"].reshape(-1)[cells] == np.flatnonzero(live)).all(), name
            assert b.entity_capacity == b.neutral_capacity + 2 * b.per_player_capacity


def test_unknown_names_are_refused():
    with pytest.raises(content.ModelError):
        shipped_map("noSuchMap")
    with pytest.raises(ContentError):
        load_game(shipped_map("basesWorkers8x8"), conflict_strategy="NOT_A_STRATEGY")


@pytest.mark.parametrize("w,h,capacity", [(200, 200, None), (130, 130, 16400)])
def test_buckets_past_int16_indices_are_refused(tmp_path, w, h, capacity):
    """The reference lays out int32 cell (or slot) indices once a bucket's
    cell count (or entity capacity) passes 32767 (src/nanorts/model/leaf.py:
    85-98); this build lays out int16 indices only and refuses such a bucket
    when the game is built: a 200x200 board (40 000 cells), and a 130x130
    board (16 900 cells) with a supplied per-player capacity of 16 400
    (entity capacity past 32 767).  The int16 extremes themselves load."""
    from nanorts_amd.model import ModelError

    doc = _doc(w=w, h=h)
    bucket = None
    if capacity is not None:
        derived = load_game(_write(tmp_path, doc)).bucket
        bucket = dataclasses.replace(derived, per_player_capacity=capacity)
    with pytest.raises(ModelError, match="int16"):
        load_game(_write(tmp_path, doc), bucket=bucket)
    # the largest board that keeps int16 cells: 181 x 181 = 32 761 cells
    assert load_game(_write(tmp_path, _doc(w=181, h=181))).bucket.cell_count == 32761
