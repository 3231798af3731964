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
    """A map document the loader refuses."""


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


def _attribute(element: ElementTree.Element, name: str) -> str:
    text = element.get(name)
    if text is None:
        raise ContentError(f"<{element.tag}> carries no {name!r} attribute")
    return text


def _integer(element: ElementTree.Element, name: str) -> int:
    text = _attribute(element, name)
    if _INTEGER.fullmatch(text) is None:
        raise ContentError(f"<{element.tag}> attribute {name}={text!r} is not an integer")
    return int(text)


def _child(root: ElementTree.Element, name: str) -> ElementTree.Element:
    child = root.find(name)
    if child is None:
        raise ContentError(f"the document has no <{name}> element")
    return child


def parse_document(text: str) -> ContentDocument:
    """src/nanorts/content/loading.py:34-92"""
    try:
        root = ElementTree.fromstring(text)
    except ElementTree.ParseError as error:
        raise ContentError(f"the document is not well formed XML: {error}") from error
    width, height = _integer(root, "width"), _integer(root, "height")
    if width <= 0 or height <= 0:
        raise ContentError(f"the field is {width}x{height}, expected positive extents")
    terrain = (_child(root, "terrain").text or "").strip()
    if len(terrain) != width * height or set(terrain) - {"0", "1"}:
        raise ContentError("the <terrain> payload must be width*height binary digits")
    players = tuple((_integer(p, "ID"), _integer(p, "resources")) for p in _child(root, "players"))
    if [declared for declared, _ in players] != list(range(PLAYER_COUNT)):
        raise ContentError(f"the document declares players {players}, expected IDs 0 and 1 in order")
    units = tuple(
        UnitRecord(type=_attribute(u, "type"), id=_integer(u, "ID"), player=_integer(u, "player"),
                   x=_integer(u, "x"), y=_integer(u, "y"), hitpoints=_integer(u, "hitpoints"),
                   resources=_integer(u, "resources"))
        for u in _child(root, "units"))
    seen: set[tuple[int, int]] = set()
    for unit in units:
        if not (0 <= unit.x < width and 0 <= unit.y < height):
            raise ContentError(f"unit ID {unit.id} sits outside the {width}x{height} field")
        if (unit.x, unit.y) in seen:
            raise ContentError(f"unit ID {unit.id} sits on an occupied cell")
        seen.add((unit.x, unit.y))
        if unit.player not in (OWNER_NEUTRAL, 0, 1):
            raise ContentError(f"unit ID {unit.id} names player {unit.player}")
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


def _assemble(document: ContentDocument, utt: UnitTypeTableVersion, conflict_strategy: ConflictStrategy,
              max_cycles: int, per_player_capacity: int | None, name: str) -> GameConfig:
    utt = UnitTypeTableVersion(utt)
    conflict_strategy = ConflictStrategy(conflict_strategy)
    table = TABLES[utt]
    if max_cycles <= 0:
        raise ContentError(f"max_cycles is {max_cycles}, expected a positive horizon")
    bucket = derive_bucket(document, table, utt, conflict_strategy)
    if per_player_capacity is not None:
        floor = max(_population(document, p) for p in range(PLAYER_COUNT))
        if not floor <= per_player_capacity <= bucket.cell_count:
            raise ContentError(f"per_player_capacity {per_player_capacity} is outside [{floor}, {bucket.cell_count}]")
        bucket = dataclasses.replace(bucket, per_player_capacity=per_player_capacity)
    require_int16_indices(bucket)
    terrain = np.asarray([c == "1" for c in document.terrain], np.bool_).reshape(bucket.height, bucket.width)
    return GameConfig(terrain=terrain, max_cycles=int(max_cycles), initial_state=initial_state(document, table, bucket),
                      unit_types=table, bucket=bucket, name=name)


def load_game(path: str | os.PathLike[str], *, utt: UnitTypeTableVersion = UnitTypeTableVersion.ORIGINAL_FINETUNED,
              conflict_strategy: ConflictStrategy = ConflictStrategy.CANCEL_BOTH, max_cycles: int = 5000,
              per_player_capacity: int | None = None) -> GameConfig:
    """src/nanorts/content/loading.py:116-131"""
    text = Path(path).read_text(encoding="utf-8")
    return _assemble(parse_document(text), utt, conflict_strategy, max_cycles, per_player_capacity, Path(path).stem)


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
                     per_player_capacity=profile)


def with_unit_type_table(game: GameConfig, utt: UnitTypeTableVersion) -> GameConfig:
    """src/nanorts/content/loading.py:134-155: same content, other rules."""
    utt = UnitTypeTableVersion(utt)
    if utt == game.bucket.utt_identity:
        return game
    bucket = dataclasses.replace(game.bucket, utt_identity=utt)
    return dataclasses.replace(game, unit_types=TABLES[utt], bucket=bucket)


def initial_pending_empty(state: dict[str, np.ndarray]) -> bool:
    return bool(np.all(state["pending_kind"] == KIND_ABSENT))
