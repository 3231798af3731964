"""Game content: a MicroRTS map document -> GameConfig (board, unit table,
bucket shapes and the decided initial State of one env).

Follows the reference's content package (src/nanorts/content/): the map XML
(loading.py:34-113), six numbered acceptance clauses (acceptance.py), the
bucket derived from the content (normalize.py:45-116), units placed in
document order into their owner's slot block (normalize.py:119-170) and the
shipped maps with their capacity profiles (scenarios.py).

How it is organised here:
- `read_map_xml` turns the XML into a `MapDocument` of plain values through
  an `_XmlReader` that knows which clause each element belongs to;
- `findings` walks a document and yields (clause, what is wrong) pairs in
  clause order; `check_document` refuses on the first one;
- `population_ceiling` is the most units one player can ever own, from the
  map's wealth and the cheapest trainable unit; `derive_bucket` sizes the
  slot blocks from it;
- `_SlotCursor` hands out each block's next slot while the units are placed.
"""
from __future__ import annotations

import dataclasses
import os
import re
from collections.abc import Iterator, Sequence
from pathlib import Path
from typing import Final
from xml.etree import ElementTree

import numpy as np

from nanorts_amd.model import (
    ABSENT,
    OWNER_NEUTRAL,
    PLAYER_COUNT,
    STATE_LEAVES,
    TABLES,
    BucketSpec,
    ConflictStrategy,
    ModelError,
    UnitType,
    UnitTypeTableVersion,
    leaf_shape,
    require_int16_indices,
    unit_columns,
)

MAP_DIRECTORY: Final = Path(__file__).resolve().parent / "maps"

# Slot profiles of the shipped maps (src/nanorts/content/scenarios.py:20-22):
# a per-player capacity below the derived one, applied by map_name_to_scenario.
CAPACITY_PROFILES: Final = {"basesWorkers8x8": 52, "basesWorkers16x16": 70}

_SHIPPED: Final = {path.stem: path for path in sorted(MAP_DIRECTORY.rglob("*.xml"))}
SCENARIO_NAMES: Final = tuple(sorted(_SHIPPED))

_SIGNED_32: Final = range(-(2**31), 2**31)
_HIT_POINT_RANGE: Final = range(0, 2**15)
_WHOLE_NUMBER: Final = re.compile(r"[+-]?\d+")


class ContentError(ModelError):
    """Content the loader refuses.  `clause` is the acceptance clause it
    breaks (src/nanorts/content/document.py:6-10): 1 the document and its
    extents, 2 the terrain payload, 3 binary terrain, 4 the player records,
    5 the unit records, 6 hit points; None for a refusal outside the
    clauses (a bucket, a table, a full slot block)."""

    def __init__(self, message: str, *, clause: int | None = None) -> None:
        super().__init__(message)
        self.clause = clause


def _refusal(clause: int, finding: str) -> ContentError:
    return ContentError(f"clause {clause}: {finding}", clause=clause)


@dataclasses.dataclass(frozen=True)
class UnitRecord:
    """One <rts.units.Unit> of a map (field order of the reference's
    UnitRecord, src/nanorts/content/document.py:13-21)."""

    type: str
    id: int
    player: int
    x: int
    y: int
    hitpoints: int
    resources: int


@dataclasses.dataclass(frozen=True)
class MapDocument:
    """A map as plain values: extents, terrain digits, the player records as
    (ID, starting resources) and the unit records in document order."""

    width: int
    height: int
    terrain: str
    players: tuple[tuple[int, int], ...]
    units: tuple[UnitRecord, ...]


@dataclasses.dataclass(frozen=True, eq=False)
class GameConfig:
    """The static game: board, unit type table, horizon and initial state
    (src/nanorts/model/config.py:44-69).  `initial_state` maps each State leaf
    name to a numpy array of one env's shape."""

    terrain: np.ndarray  # bool[H, W]
    max_cycles: int
    initial_state: dict[str, np.ndarray]
    unit_types: tuple[UnitType, ...]
    bucket: BucketSpec
    name: str = ""

    @property
    def columns(self) -> dict[str, np.ndarray]:
        return unit_columns(self.unit_types)


# ---------------------------------------------------------------------------
# Acceptance (src/nanorts/content/acceptance.py): findings in clause order
# ---------------------------------------------------------------------------
def _extent_findings(width: int, height: int) -> Iterator[tuple[int, str]]:
    for label, value in (("width", width), ("height", height)):
        if value not in _SIGNED_32:
            yield 1, f"the {label} {value} does not fit a signed 32-bit integer"
        elif value < 1:
            yield 1, f"the {label} must be at least 1, not {value}"


def _terrain_findings(terrain: str, width: int, height: int) -> Iterator[tuple[int, str]]:
    cells = width * height
    if len(terrain) != cells:
        yield 2, f"a {width}x{height} board needs {cells} terrain digits, the map gives {len(terrain)}"
        return
    for index, char in enumerate(terrain):
        if not ("0" <= char <= "9"):
            yield 2, f"terrain character {index} is {char!r}, which is not a digit"
            return
    for index, char in enumerate(terrain):
        if char not in "01":
            yield 3, f"terrain digit {index} is {char}; a cell is open (0) or wall (1)"
            return


def _player_findings(players: Sequence[tuple[int, int]]) -> Iterator[tuple[int, str]]:
    if len(players) != PLAYER_COUNT:
        yield 4, f"the map lists {len(players)} players; a game has {PLAYER_COUNT}"
        return
    for position, (declared, resources) in enumerate(players):
        if declared != position:
            yield 4, f"the player listed at position {position} carries ID {declared}; IDs must count up from 0"
        elif resources not in _SIGNED_32:
            yield 4, f"player {position} starts with {resources} resources, beyond a signed 32-bit integer"


def _unit_findings(document: MapDocument, table: Sequence[UnitType]) -> Iterator[tuple[int, str]]:
    known = {unit.name for unit in table}
    owners = {declared for declared, _ in document.players}
    ids: set[int] = set()
    holder: dict[tuple[int, int], int] = {}
    for index, unit in enumerate(document.units):
        numbers = (("ID", unit.id), ("player", unit.player), ("x", unit.x), ("y", unit.y),
                   ("hitpoints", unit.hitpoints), ("resources", unit.resources))
        wide = next((label for label, value in numbers if value not in _SIGNED_32), None)
        if wide is not None:
            yield 5, f"record {index} has a {wide} beyond a signed 32-bit integer"
        elif unit.type not in known:
            yield 5, f"unit {unit.id} is a {unit.type!r}, a type this unit table lacks"
        elif unit.id in ids:
            yield 5, f"two records share unit ID {unit.id}"
        elif not (0 <= unit.x < document.width and 0 <= unit.y < document.height):
            yield 5, f"unit {unit.id} at ({unit.x}, {unit.y}) lies off the {document.width}x{document.height} board"
        elif (unit.x, unit.y) in holder:
            yield 5, f"unit {unit.id} and unit {holder[unit.x, unit.y]} both stand on ({unit.x}, {unit.y})"
        elif unit.player != OWNER_NEUTRAL and unit.player not in owners:
            yield 5, f"unit {unit.id} belongs to player {unit.player}, whom the map does not list"
        if wide is not None:
            continue
        ids.add(unit.id)
        holder.setdefault((unit.x, unit.y), unit.id)


def _hit_point_findings(document: MapDocument) -> Iterator[tuple[int, str]]:
    for unit in document.units:
        if unit.hitpoints not in _HIT_POINT_RANGE:
            yield 6, (f"unit {unit.id} has {unit.hitpoints} hit points; the int16 leaf holds "
                      f"{_HIT_POINT_RANGE.start} to {_HIT_POINT_RANGE.stop - 1}")


def findings(document: MapDocument, table: Sequence[UnitType]) -> Iterator[tuple[int, str]]:
    """Every broken acceptance clause of `document`, lowest clause first (and
    clause 5 in record order)."""
    yield from _extent_findings(document.width, document.height)
    yield from _terrain_findings(document.terrain, document.width, document.height)
    yield from _player_findings(document.players)
    yield from _unit_findings(document, table)
    yield from _hit_point_findings(document)


def check_document(document: MapDocument, table: Sequence[UnitType]) -> None:
    """Refuse `document` on the first broken clause (acceptance.py:158-164)."""
    for clause, finding in findings(document, table):
        raise _refusal(clause, finding)


# ---------------------------------------------------------------------------
# Map XML (src/nanorts/content/loading.py:34-113)
# ---------------------------------------------------------------------------
class _XmlReader:
    """Reads the values of one element, refusing under `clause`."""

    def __init__(self, element: ElementTree.Element, clause: int) -> None:
        self.element, self.clause = element, clause

    def text(self, name: str) -> str:
        value = self.element.get(name)
        if value is None:
            raise _refusal(self.clause, f"a <{self.element.tag}> element lacks the {name!r} attribute")
        return value

    def number(self, name: str) -> int:
        value = self.text(name)
        if not _WHOLE_NUMBER.fullmatch(value):
            raise _refusal(self.clause, f"<{self.element.tag}> gives {name}={value!r}, which is not a whole number")
        return int(value)

    def child(self, tag: str) -> ElementTree.Element:
        found = self.element.find(tag)
        if found is None:
            raise _refusal(self.clause, f"the map has no <{tag}> section")
        return found


def read_map_xml(text: str) -> MapDocument:
    """The document of a MicroRTS map XML.  The extents, terrain and player
    records are checked as they are read (clauses 1-4); the unit records by
    check_document."""
    try:
        root = ElementTree.fromstring(text)
    except ElementTree.ParseError as error:
        raise _refusal(1, f"the XML does not parse ({error})") from error
    board = _XmlReader(root, 1)
    width, height = board.number("width"), board.number("height")
    for clause, finding in _extent_findings(width, height):
        raise _refusal(clause, finding)
    terrain = _XmlReader(root, 2).child("terrain").text or ""
    for clause, finding in _terrain_findings(terrain, width, height):
        raise _refusal(clause, finding)
    players = tuple((reader.number("ID"), reader.number("resources"))
                    for reader in (_XmlReader(p, 4) for p in _XmlReader(root, 4).child("players")))
    for clause, finding in _player_findings(players):
        raise _refusal(clause, finding)
    units = []
    for element in _XmlReader(root, 5).child("units"):
        r = _XmlReader(element, 5)
        units.append(UnitRecord(type=r.text("type"), id=r.number("ID"), player=r.number("player"), x=r.number("x"),
                                y=r.number("y"), hitpoints=r.number("hitpoints"), resources=r.number("resources")))
    return MapDocument(width=width, height=height, terrain=terrain, players=players, units=tuple(units))


# ---------------------------------------------------------------------------
# Buckets (src/nanorts/content/normalize.py:45-116)
# ---------------------------------------------------------------------------
def _headcount(document: MapDocument, owner: int) -> int:
    return sum(unit.player == owner for unit in document.units)


def population_ceiling(document: MapDocument, table: Sequence[UnitType]) -> int | None:
    """The most units one player can ever own, or None when the table gives
    no such bound (normalize.py:45-73).  The map's wealth is every unit's
    resources, a resource pile counting its stock (at least 1) rounded up to
    whole harvests of the largest harvest amount; a player can own its
    starting units plus whatever its balance and all that wealth can buy at
    the cheapest trainable cost."""
    trainable = [unit for unit in table if unit.produced_by]
    gatherers = [unit for unit in table if unit.can_harvest]
    if not trainable or not gatherers:
        return None
    if any(unit.cost <= 0 or unit.is_resource for unit in trainable):
        return None
    if any(unit.is_resource or unit.harvest_amount < 0 for unit in gatherers):
        return None
    is_pile = {unit.name: unit.is_resource for unit in table}
    grab = max(unit.harvest_amount for unit in gatherers)
    wealth = 0
    for unit in document.units:
        wealth += max(unit.resources, 1) + grab - 1 if is_pile[unit.type] else max(unit.resources, 0)
    price = min(unit.cost for unit in trainable)
    return max(_headcount(document, player) + max(0, balance + wealth) // price
               for player, balance in document.players)


def derive_bucket(document: MapDocument, table: Sequence[UnitType], utt: UnitTypeTableVersion,
                  conflict_strategy: ConflictStrategy) -> BucketSpec:
    """The bucket the content implies (normalize.py:77-93): a neutral block
    of the map's neutral units, player blocks of the population ceiling
    clamped to [1, cells] (the cells when there is no ceiling), every type of
    the table, and the square attack window of the longest range."""
    cells = document.width * document.height
    ceiling = population_ceiling(document, table)
    side = 2 * max(unit.attack_range for unit in table) + 1
    return BucketSpec(height=document.height, width=document.width,
                      neutral_capacity=_headcount(document, OWNER_NEUTRAL),
                      per_player_capacity=cells if ceiling is None else min(cells, max(1, ceiling)),
                      unit_type_capacity=len(table), attack_offset_capacity=side * side, utt_identity=utt,
                      conflict_strategy=conflict_strategy)


_CHOSEN_BY_CALLER: Final = ("neutral_capacity", "per_player_capacity")


def check_supplied_bucket(derived: BucketSpec, supplied: BucketSpec, document: MapDocument) -> None:
    """A caller's bucket may resize the two slot blocks, each to any size from
    the units the map puts in it up to the cell count, and must match the
    derived bucket everywhere else (normalize.py:96-116)."""
    problems = []
    for field in dataclasses.fields(BucketSpec):
        if field.name in _CHOSEN_BY_CALLER:
            continue
        mine, theirs = getattr(derived, field.name), getattr(supplied, field.name)
        if mine != theirs:
            problems.append(f"{field.name} {theirs!r} should be {mine!r}")
    least = {"neutral_capacity": _headcount(document, OWNER_NEUTRAL),
             "per_player_capacity": max(_headcount(document, p) for p in range(PLAYER_COUNT))}
    for name, low in least.items():
        size = getattr(supplied, name)
        if size < low or size > derived.cell_count:
            problems.append(f"{name} {size!r} should lie in [{low}, {derived.cell_count}] (the map's units in that "
                            "block up to the cell count)")
    if problems:
        raise ContentError("the supplied bucket does not fit this content: " + ", ".join(problems))


# ---------------------------------------------------------------------------
# Initial state (src/nanorts/content/normalize.py:119-170)
# ---------------------------------------------------------------------------
class _SlotCursor:
    """The next free slot of each block: neutral, player 0, player 1."""

    def __init__(self, bucket: BucketSpec) -> None:
        self.bounds = {OWNER_NEUTRAL: (0, bucket.neutral_capacity)}
        for player in range(PLAYER_COUNT):
            self.bounds[player] = (bucket.player_slot_start(player), bucket.per_player_capacity)
        self.used = dict.fromkeys(self.bounds, 0)

    def take(self, unit: UnitRecord) -> int:
        start, size = self.bounds[unit.player]
        if self.used[unit.player] == size:
            owner = "the neutral" if unit.player == OWNER_NEUTRAL else f"player {unit.player}'s"
            raise ContentError(f"unit {unit.id} finds {owner} block of {size} slots already full")
        self.used[unit.player] += 1
        return start + self.used[unit.player] - 1


def initial_state(document: MapDocument, table: Sequence[UnitType], bucket: BucketSpec) -> dict[str, np.ndarray]:
    """The State of one env at the start of an episode: each unit, born in
    document order, in its block's next slot; the players' balances; the
    outcome decided (outcome.decide, src/nanorts/core/outcome.py:11-25)."""
    state = {leaf.name: np.full(leaf_shape(leaf, bucket), leaf.fill, leaf.dtype) for leaf in STATE_LEAVES}
    code = {unit.name: index for index, unit in enumerate(table)}
    cursor = _SlotCursor(bucket)
    for birth, unit in enumerate(document.units):
        if unit.type not in code:
            raise ContentError(f"unit {unit.id} is a {unit.type!r}, a type this unit table lacks")
        slot = cursor.take(unit)
        for name, value in (("birth", birth), ("unit_type", code[unit.type]), ("owner", unit.player),
                            ("cell", unit.y * bucket.width + unit.x), ("hit_points", unit.hitpoints),
                            ("carried_resources", unit.resources)):
            state[name][slot] = value
        state["entity_at"][unit.y, unit.x] = slot
    state["player_resources"][:] = [balance for _, balance in document.players]
    state["next_birth"][()] = len(document.units)
    owned = state["birth"][bucket.neutral_capacity:].reshape(PLAYER_COUNT, bucket.per_player_capacity) != ABSENT
    standing = np.flatnonzero(owned.any(axis=1))
    state["game_over"][()] = standing.size <= 1
    state["winner"][()] = int(standing[0]) if standing.size == 1 else ABSENT
    return state


# ---------------------------------------------------------------------------
# Games
# ---------------------------------------------------------------------------
def _release(utt, conflict_strategy) -> tuple[UnitTypeTableVersion, ConflictStrategy, tuple[UnitType, ...]]:
    """The unit table and strategy of the supported releases
    (src/nanorts/content/loading.py:160-173)."""
    try:
        utt = UnitTypeTableVersion(utt)
    except ValueError:
        raise ContentError(f"no unit type table is called {utt!r}; the supported ones are "
                           f"{', '.join(v.value for v in UnitTypeTableVersion)}") from None
    try:
        conflict_strategy = ConflictStrategy(conflict_strategy)
    except ValueError:
        raise ContentError(f"no conflict strategy is called {conflict_strategy!r}; the supported ones are "
                           f"{', '.join(v.value for v in ConflictStrategy)}") from None
    return utt, conflict_strategy, TABLES[utt]


def _game(document: MapDocument, utt, conflict_strategy, max_cycles: int, bucket: BucketSpec | None,
          name: str) -> GameConfig:
    utt, conflict_strategy, table = _release(utt, conflict_strategy)
    check_document(document, table)
    if max_cycles < 1:
        raise ContentError(f"the horizon max_cycles must be at least 1, not {max_cycles}")
    shape = derive_bucket(document, table, utt, conflict_strategy)
    if bucket is not None:
        check_supplied_bucket(shape, bucket, document)
        shape = bucket
    require_int16_indices(shape)
    walls = np.frombuffer(document.terrain.encode("ascii"), np.uint8) == ord("1")
    return GameConfig(terrain=walls.reshape(shape.height, shape.width), max_cycles=int(max_cycles),
                      initial_state=initial_state(document, table, shape), unit_types=table, bucket=shape, name=name)


def load_game(path: str | os.PathLike[str], *, utt: UnitTypeTableVersion = UnitTypeTableVersion.ORIGINAL_FINETUNED,
              conflict_strategy: ConflictStrategy = ConflictStrategy.CANCEL_BOTH, max_cycles: int = 5000,
              bucket: BucketSpec | None = None) -> GameConfig:
    """A game from a map file (src/nanorts/content/loading.py:116-121)."""
    source = Path(path)
    return _game(read_map_xml(source.read_text(encoding="utf-8")), utt, conflict_strategy, max_cycles, bucket,
                 source.stem)


def build_game(*, width: int, height: int, terrain: str, players: Sequence[int], units: Sequence[UnitRecord],
               utt: UnitTypeTableVersion = UnitTypeTableVersion.ORIGINAL_FINETUNED,
               conflict_strategy: ConflictStrategy = ConflictStrategy.CANCEL_BOTH, max_cycles: int = 5000,
               bucket: BucketSpec | None = None, name: str = "") -> GameConfig:
    """A game from values instead of a file (src/nanorts/content/loading.py:124-133);
    `players` lists each player's starting resources."""
    document = MapDocument(width=width, height=height, terrain=terrain,
                           players=tuple((index, balance) for index, balance in enumerate(players)), units=tuple(units))
    return _game(document, utt, conflict_strategy, max_cycles, bucket, name)


def with_unit_type_table(game: GameConfig, utt: UnitTypeTableVersion) -> GameConfig:
    """The same content under another unit table, which must list the same
    type names and give the same attack window
    (src/nanorts/content/loading.py:136-157)."""
    utt, _, table = _release(utt, game.bucket.conflict_strategy)
    if utt == game.bucket.utt_identity:
        return game
    mine, theirs = [unit.name for unit in game.unit_types], [unit.name for unit in table]
    if mine != theirs:
        raise ContentError(f"table {utt} lists the types {theirs}; this game is built on {mine}")
    side = 2 * max(unit.attack_range for unit in table) + 1
    if side * side != game.bucket.attack_offset_capacity:
        raise ContentError(f"table {utt} needs an attack window of {side * side} cells; this game's bucket has "
                           f"{game.bucket.attack_offset_capacity}")
    return dataclasses.replace(game, unit_types=table, bucket=dataclasses.replace(game.bucket, utt_identity=utt))


# ---------------------------------------------------------------------------
# Shipped maps (src/nanorts/content/scenarios.py)
# ---------------------------------------------------------------------------
def scenario_names() -> tuple[str, ...]:
    """The names of the shipped maps (their file stems, one per map)."""
    return SCENARIO_NAMES


def shipped_map(name: str) -> Path:
    """The file of a shipped map."""
    try:
        return _SHIPPED[name]
    except KeyError:
        raise ModelError(f"{name!r} is not a shipped map; scenario_names() lists the {len(SCENARIO_NAMES)} there "
                         "are, and content.load_game(path) loads any other map file") from None


def map_name_to_scenario(name: str, *, utt: UnitTypeTableVersion = UnitTypeTableVersion.ORIGINAL_FINETUNED,
                         conflict_strategy: ConflictStrategy = ConflictStrategy.CANCEL_BOTH, max_cycles: int = 5000,
                         capacity_profile: bool = True) -> GameConfig:
    """A shipped map as a game, its player blocks cut to the map's capacity
    profile when it has one that is smaller than the derived capacity
    (src/nanorts/content/scenarios.py:25-42)."""
    game = load_game(shipped_map(name), utt=utt, conflict_strategy=conflict_strategy, max_cycles=max_cycles)
    profile = CAPACITY_PROFILES.get(name) if capacity_profile else None
    if profile is None or profile >= game.bucket.per_player_capacity:
        return game
    return load_game(shipped_map(name), utt=utt, conflict_strategy=conflict_strategy, max_cycles=max_cycles,
                     bucket=dataclasses.replace(game.bucket, per_player_capacity=profile))
