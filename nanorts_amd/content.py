"""Map XML -> game configuration and initial state.

Restates src/nanorts/content/{loading,normalize,scenarios}.py of the reference:
the MicroRTS map document is parsed, the slot capacities are derived from the
resource bound (normalize.py:87-154), units are placed in document order into
the neutral / player-0 / player-1 slot blocks (normalize.py:180-231), and the
shipped capacity profiles cap 16x16 at 70 slots per player (scenarios.py:20-42).
"""
from __future__ import annotations

import dataclasses
import os
import re
from pathlib import Path
from typing import Final
from xml.etree import ElementTree

import numpy as np

from nanorts_amd.model import (
    ABSENT,
    KIND_ABSENT,
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

CAPACITY_PROFILES: Final = {"basesWorkers8x8": 52, "basesWorkers16x16": 70}

_INTEGER = re.compile(r"[+-]?[0-9]+")


class ContentError(ModelError):
    """A map document the loader refuses (src/nanorts/content/document.py:6-10).
    `clause` names the acceptance clause the document breaks: 1 the document
    and its extents, 2 the terrain payload, 3 binary terrain, 4 the player
    records, 5 the unit records, 6 hit points."""

    def __init__(self, message: str, *, clause: int | None = None) -> None:
        super().__init__(message)
        self.clause = clause


@dataclasses.dataclass(frozen=True)
class UnitRecord:
    type: str
    id: int
    player: int
    x: int
    y: int
    hitpoints: int
    resources: int


@dataclasses.dataclass(frozen=True)
class ContentDocument:
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


_INT32 = range(-(2**31), 2**31)
_HIT_POINTS = range(2**15)


def _refuse(clause: int, message: str) -> ContentError:
    return ContentError(f"clause {clause}: {message}", clause=clause)


def _attribute(element: ElementTree.Element, name: str, clause: int) -> str:
    text = element.get(name)
    if text is None:
        raise _refuse(clause, f"<{element.tag}> carries no {name!r} attribute")
    return text


def _integer(element: ElementTree.Element, name: str, clause: int) -> int:
    text = _attribute(element, name, clause)
    if _INTEGER.fullmatch(text) is None:
        raise _refuse(clause, f"<{element.tag}> attribute {name}={text!r} is not an integer")
    return int(text)


def _child(root: ElementTree.Element, name: str, clause: int) -> ElementTree.Element:
    child = root.find(name)
    if child is None:
        raise _refuse(clause, f"the document has no <{name}> element")
    return child


def _int32(value: int, subject: str, clause: int) -> None:
    if value not in _INT32:
        raise _refuse(clause, f"{subject} is {value}, outside the 32-bit signed range")


def check_dimensions(width: int, height: int) -> None:
    """Clause 1 (src/nanorts/content/acceptance.py:18-25)."""
    for name, value in (("width", width), ("height", height)):
        _int32(value, name, 1)
        if value <= 0:
            raise _refuse(1, f"{name} is {value}, expected a positive integer")


def check_terrain_payload(terrain: str, width: int, height: int) -> None:
    """Clause 2 (acceptance.py:28-42): one digit per cell."""
    if len(terrain) != width * height:
        raise _refuse(2, f"the <terrain> payload is {len(terrain)} characters against a {width}x{height} field of "
                         f"{width * height} cells")
    bad = next((i for i, ch in enumerate(terrain) if ch not in "0123456789"), None)
    if bad is not None:
        raise _refuse(2, f"the <terrain> payload holds {terrain[bad]!r} at index {bad}, and the payload is digits only")


def check_terrain_digits(terrain: str) -> None:
    """Clause 3 (acceptance.py:45-52): terrain is binary."""
    bad = next((i for i, ch in enumerate(terrain) if ch not in "01"), None)
    if bad is not None:
        raise _refuse(3, f"the <terrain> payload holds the digit {terrain[bad]} at index {bad}, and terrain is binary")


def check_players(players: tuple[tuple[int, int], ...]) -> None:
    """Clause 4 (acceptance.py:55-69): two positional player records."""
    if len(players) != PLAYER_COUNT:
        raise _refuse(4, f"the document declares {len(players)} player records, expected exactly {PLAYER_COUNT}")
    for expected, (declared, resources) in enumerate(players):
        if declared != expected:
            raise _refuse(4, f"player record {expected} declares ID {declared}, and the records are positional")
        _int32(resources, f"player record {expected}'s resources", 4)


def check_document(document: ContentDocument, table: tuple[UnitType, ...]) -> None:
    """Every acceptance clause (acceptance.py:72-168) on a parsed or built
    document: extents, terrain, players, then per unit in document order its
    32-bit fields, a known type, a unique ID, a cell on the board that no
    earlier unit holds and a declared owner (clause 5), then hit points in
    [0, 2^15 - 1] (clause 6)."""
    check_dimensions(document.width, document.height)
    check_terrain_payload(document.terrain, document.width, document.height)
    check_terrain_digits(document.terrain)
    check_players(document.players)
    names = {unit.name for unit in table}
    declared = {player for player, _ in document.players}
    ids: set[int] = set()
    held: dict[tuple[int, int], int] = {}
    for position, unit in enumerate(document.units):
        for field in ("id", "player", "x", "y", "hitpoints", "resources"):
            _int32(getattr(unit, field), f"unit {position}'s {'ID' if field == 'id' else field}", 5)
        if unit.type not in names:
            raise _refuse(5, f"unit ID {unit.id} names the type {unit.type!r}, which the supported unit type table "
                             "does not hold")
        if unit.id in ids:
            raise _refuse(5, f"unit ID {unit.id} is declared more than once")
        ids.add(unit.id)
        if not (0 <= unit.x < document.width and 0 <= unit.y < document.height):
            raise _refuse(5, f"unit ID {unit.id} sits at ({unit.x}, {unit.y}), outside the "
                             f"{document.width}x{document.height} field")
        if (unit.x, unit.y) in held:
            raise _refuse(5, f"unit ID {unit.id} sits at ({unit.x}, {unit.y}), which unit ID "
                             f"{held[unit.x, unit.y]} already occupies")
        held[unit.x, unit.y] = unit.id
        if unit.player != OWNER_NEUTRAL and unit.player not in declared:
            raise _refuse(5, f"unit ID {unit.id} names player {unit.player}, which no player record declares")
    for unit in document.units:
        if unit.hitpoints not in _HIT_POINTS:
            raise _refuse(6, f"unit ID {unit.id} declares {unit.hitpoints} hit points, outside "
                             f"[0, {_HIT_POINTS.stop - 1}]")


def parse_document(text: str) -> ContentDocument:
    """The MicroRTS map XML (src/nanorts/content/loading.py:34-113); the
    structural clauses are checked while reading, the rest by check_document."""
    try:
        root = ElementTree.fromstring(text)
    except ElementTree.ParseError as error:
        raise _refuse(1, f"the document is not well formed XML: {error}") from error
    width, height = _integer(root, "width", 1), _integer(root, "height", 1)
    check_dimensions(width, height)
    terrain = _child(root, "terrain", 2).text or ""
    check_terrain_payload(terrain, width, height)
    check_terrain_digits(terrain)
    players = tuple((_integer(p, "ID", 4), _integer(p, "resources", 4)) for p in _child(root, "players", 4))
    check_players(players)
    units = tuple(
        UnitRecord(type=_attribute(u, "type", 5), id=_integer(u, "ID", 5), player=_integer(u, "player", 5),
                   x=_integer(u, "x", 5), y=_integer(u, "y", 5), hitpoints=_integer(u, "hitpoints", 5),
                   resources=_integer(u, "resources", 5))
        for u in _child(root, "units", 5))
    return ContentDocument(width=width, height=height, terrain=terrain, players=players, units=units)


def _population(document: ContentDocument, owner: int) -> int:
    return sum(1 for unit in document.units if unit.player == owner)


def _resource_bound(document: ContentDocument, table: tuple[UnitType, ...]) -> int | None:
    """src/nanorts/content/normalize.py:45-73: the most units a player can ever
    own, from the resources on the map and the cheapest producible cost."""
    produced = [unit for unit in table if unit.produced_by]
    harvesters = [unit for unit in table if unit.can_harvest]
    applies = (bool(produced) and bool(harvesters)
               and all(unit.cost > 0 and not unit.is_resource for unit in produced)
               and all(not unit.is_resource and unit.harvest_amount >= 0 for unit in harvesters))
    if not applies:
        return None
    types = {unit.name: unit for unit in table}
    largest_harvest = max(unit.harvest_amount for unit in harvesters)
    on_map = sum(max(unit.resources, 1) + largest_harvest - 1 if types[unit.type].is_resource
                 else max(unit.resources, 0) for unit in document.units)
    cheapest = min(unit.cost for unit in produced)
    return max(_population(document, player) + max(0, balance + on_map) // cheapest
               for player, balance in document.players)


def derive_bucket(document: ContentDocument, table: tuple[UnitType, ...], utt: UnitTypeTableVersion,
                  conflict_strategy: ConflictStrategy) -> BucketSpec:
    """src/nanorts/content/normalize.py:77-93"""
    cells = document.width * document.height
    bound = _resource_bound(document, table)
    window = 2 * max(unit.attack_range for unit in table) + 1
    return BucketSpec(
        height=document.height, width=document.width,
        neutral_capacity=_population(document, OWNER_NEUTRAL),
        per_player_capacity=cells if bound is None else max(1, min(cells, bound)),
        unit_type_capacity=len(table), attack_offset_capacity=window * window,
        utt_identity=utt, conflict_strategy=conflict_strategy)


def initial_state(document: ContentDocument, table: tuple[UnitType, ...], bucket: BucketSpec) -> dict[str, np.ndarray]:
    """src/nanorts/content/normalize.py:119-154 + :157-170 (slot claims)."""
    state = {leaf.name: np.full(leaf_shape(leaf, bucket), leaf.fill, leaf.dtype) for leaf in STATE_LEAVES}
    names = {unit.name: index for index, unit in enumerate(table)}
    next_free = [0] * (PLAYER_COUNT + 1)
    for birth, unit in enumerate(document.units):
        if unit.type not in names:
            raise ContentError(f"unit ID {unit.id} names the unknown type {unit.type!r}")
        if unit.player == OWNER_NEUTRAL:
            start, capacity, block = 0, bucket.neutral_capacity, "neutral"
        else:
            start, capacity, block = bucket.player_slot_start(unit.player), bucket.per_player_capacity, f"player {unit.player}"
        offset = next_free[unit.player + 1]
        if offset >= capacity:
            raise ContentError(f"the {block} block holds {capacity} slots, which unit ID {unit.id} exceeds")
        next_free[unit.player + 1] = offset + 1
        slot = start + offset
        state["birth"][slot] = birth
        state["unit_type"][slot] = names[unit.type]
        state["owner"][slot] = unit.player
        state["cell"][slot] = unit.x + unit.y * bucket.width
        state["hit_points"][slot] = unit.hitpoints
        state["carried_resources"][slot] = unit.resources
        state["entity_at"][unit.y, unit.x] = slot
    state["player_resources"][:] = [resources for _, resources in document.players]
    state["next_birth"][()] = len(document.units)
    _decide(state, bucket)
    return state


def _decide(state: dict[str, np.ndarray], bucket: BucketSpec) -> None:
    """outcome.decide (src/nanorts/core/outcome.py:11-25) on one env."""
    owned = state["birth"][bucket.neutral_capacity:].reshape(PLAYER_COUNT, bucket.per_player_capacity)
    surviving = (owned != ABSENT).any(axis=1)
    count = int(surviving.sum())
    state["game_over"][()] = count <= 1
    state["winner"][()] = int(np.argmax(surviving)) if count == 1 else ABSENT


_CALLER_CHOSEN = ("neutral_capacity", "per_player_capacity")


def check_supplied_bucket(derived: BucketSpec, supplied: BucketSpec, document: ContentDocument) -> None:
    """src/nanorts/content/normalize.py:96-116: a supplied BucketSpec agrees
    with the derived one except for the two slot capacities, each of which
    lies between the population the content puts in its block and the cell
    count."""
    wrong = [f"{field.name} is {getattr(supplied, field.name)!r}, expected {getattr(derived, field.name)!r}"
             for field in dataclasses.fields(derived)
             if field.name not in _CALLER_CHOSEN and getattr(supplied, field.name) != getattr(derived, field.name)]
    floors = {"neutral_capacity": _population(document, OWNER_NEUTRAL),
              "per_player_capacity": max(_population(document, p) for p in range(PLAYER_COUNT))}
    for name, floor in floors.items():
        chosen = getattr(supplied, name)
        if not floor <= chosen <= derived.cell_count:
            wrong.append(f"{name} is {chosen!r}, expected the inclusive interval [{floor}, {derived.cell_count}] "
                         "between the population the content puts in that block and its cell count")
    if wrong:
        raise ContentError("the supplied BucketSpec disagrees with the content: " + "; ".join(wrong))


def _table(utt, conflict_strategy) -> tuple[UnitTypeTableVersion, ConflictStrategy, tuple[UnitType, ...]]:
    try:
        utt = UnitTypeTableVersion(utt)
    except ValueError:
        raise ContentError(f"unit type table {utt!r} is outside the supported release matrix, which is "
                           f"{[member.value for member in UnitTypeTableVersion]}") from None
    try:
        conflict_strategy = ConflictStrategy(conflict_strategy)
    except ValueError:
        raise ContentError(f"conflict strategy {conflict_strategy!r} is outside the supported release matrix, which "
                           f"is {[member.value for member in ConflictStrategy]}") from None
    return utt, conflict_strategy, TABLES[utt]


def _assemble(document: ContentDocument, utt, conflict_strategy, max_cycles: int, bucket: BucketSpec | None,
              name: str) -> GameConfig:
    """src/nanorts/content/loading.py:176-188: accept, derive (or check the
    supplied) bucket, place the units."""
    utt, conflict_strategy, table = _table(utt, conflict_strategy)
    check_document(document, table)
    if max_cycles <= 0:
        raise ContentError(f"max_cycles is {max_cycles}, expected a positive horizon")
    derived = derive_bucket(document, table, utt, conflict_strategy)
    if bucket is not None:
        check_supplied_bucket(derived, bucket, document)
        derived = bucket
    require_int16_indices(derived)
    terrain = np.asarray([c == "1" for c in document.terrain], np.bool_).reshape(derived.height, derived.width)
    return GameConfig(terrain=terrain, max_cycles=int(max_cycles), initial_state=initial_state(document, table, derived),
                      unit_types=table, bucket=derived, name=name)


def load_game(path: str | os.PathLike[str], *, utt: UnitTypeTableVersion = UnitTypeTableVersion.ORIGINAL_FINETUNED,
              conflict_strategy: ConflictStrategy = ConflictStrategy.CANCEL_BOTH, max_cycles: int = 5000,
              bucket: BucketSpec | None = None) -> GameConfig:
    """src/nanorts/content/loading.py:116-121"""
    text = Path(path).read_text(encoding="utf-8")
    return _assemble(parse_document(text), utt, conflict_strategy, max_cycles, bucket, Path(path).stem)


def build_game(*, width: int, height: int, terrain: str, players, units,
               utt: UnitTypeTableVersion = UnitTypeTableVersion.ORIGINAL_FINETUNED,
               conflict_strategy: ConflictStrategy = ConflictStrategy.CANCEL_BOTH, max_cycles: int = 5000,
               bucket: BucketSpec | None = None, name: str = "") -> GameConfig:
    """src/nanorts/content/loading.py:124-133: the same game from fields
    instead of a document; `players` lists each player's starting
    resources."""
    document = ContentDocument(width=width, height=height, terrain=terrain, players=tuple(enumerate(players)),
                               units=tuple(units))
    return _assemble(document, utt, conflict_strategy, max_cycles, bucket, name)


def scenario_names() -> tuple[str, ...]:
    return tuple(sorted(path.stem for path in MAP_DIRECTORY.glob("*.xml")))


def shipped_map(name: str) -> Path:
    path = MAP_DIRECTORY / f"{name}.xml"
    if not path.is_file():
        raise ModelError(f"scenario {name!r} is none of the shipped maps {list(scenario_names())}")
    return path


def map_name_to_scenario(name: str, *, utt: UnitTypeTableVersion = UnitTypeTableVersion.ORIGINAL_FINETUNED,
                         conflict_strategy: ConflictStrategy = ConflictStrategy.CANCEL_BOTH, max_cycles: int = 5000,
                         capacity_profile: bool = True) -> GameConfig:
    """src/nanorts/content/scenarios.py:25-42"""
    path = shipped_map(name)
    game = load_game(path, utt=utt, conflict_strategy=conflict_strategy, max_cycles=max_cycles)
    profile = CAPACITY_PROFILES.get(name)
    if profile is None or not capacity_profile or profile >= game.bucket.per_player_capacity:
        return game
    return load_game(path, utt=utt, conflict_strategy=conflict_strategy, max_cycles=max_cycles,
                     bucket=dataclasses.replace(game.bucket, per_player_capacity=profile))


def with_unit_type_table(game: GameConfig, utt: UnitTypeTableVersion) -> GameConfig:
    """src/nanorts/content/loading.py:136-157: the same content under another
    table, which must name the same types and derive the same attack window."""
    utt, _, table = _table(utt, game.bucket.conflict_strategy)
    if utt == game.bucket.utt_identity:
        return game
    names = tuple(unit.name for unit in table)
    if names != tuple(unit.name for unit in game.unit_types):
        raise ContentError(f"unit type table {utt} declares the types {list(names)}, which are not the scenario's "
                           f"{[unit.name for unit in game.unit_types]}")
    window = (2 * max(unit.attack_range for unit in table) + 1) ** 2
    if window != game.bucket.attack_offset_capacity:
        raise ContentError(f"unit type table {utt} derives an attack window of {window} offsets, not the scenario's "
                           f"{game.bucket.attack_offset_capacity}")
    bucket = dataclasses.replace(game.bucket, utt_identity=utt)
    return dataclasses.replace(game, unit_types=table, bucket=bucket)


def initial_pending_empty(state: dict[str, np.ndarray]) -> bool:
    return bool(np.all(state["pending_kind"] == KIND_ABSENT))
