"""Vocabulary, unit type tables, bucket shapes and the state leaf layout.

Restates the data model of the reference (src/nanorts/model/): the constants of
vocabulary.py, the two unit type tables of unit_types.py:47-148, BucketSpec of
bucket.py:24-58 and the per-slot struct-of-arrays State of state.py:33-84.  The
leaf order, dtypes and canonical empties are the ones the reference's pytree
declares, so a state laid out here is byte-compatible with a jax.vmap'd State.
"""
from __future__ import annotations

import dataclasses
import enum
import math
from typing import Final

import numpy as np

ABSENT: Final = -1
OWNER_NEUTRAL: Final = ABSENT
PLAYER_COUNT: Final = 2
ATTACK_TARGET_OWNER_COUNT: Final = 3

KIND_ABSENT: Final = ABSENT
KIND_NONE: Final = 0
KIND_MOVE: Final = 1
KIND_HARVEST: Final = 2
KIND_RETURN: Final = 3
KIND_PRODUCE: Final = 4
KIND_ATTACK: Final = 5
ACTION_KIND_COUNT: Final = 6

DIRECTION_COUNT: Final = 4
DIRECTION_OFFSETS: Final = ((0, -1), (1, 0), (0, 1), (-1, 0))


class UnitTypeTableVersion(str, enum.Enum):
    """src/nanorts/model/vocabulary.py:45-47"""

    ORIGINAL = "VERSION_ORIGINAL"
    ORIGINAL_FINETUNED = "VERSION_ORIGINAL_FINETUNED"

    def __str__(self) -> str:
        return self.value


class ConflictStrategy(str, enum.Enum):
    """src/nanorts/model/vocabulary.py:50-53"""

    CANCEL_BOTH = "CANCEL_BOTH"
    CANCEL_RANDOM = "CANCEL_RANDOM"
    CANCEL_ALTERNATING = "CANCEL_ALTERNATING"

    def __str__(self) -> str:
        return self.value


STRATEGY_CODES: Final = {
    ConflictStrategy.CANCEL_BOTH: 0,
    ConflictStrategy.CANCEL_RANDOM: 1,
    ConflictStrategy.CANCEL_ALTERNATING: 2,
}


class ModelError(ValueError):
    """Raised for content, shapes or arguments the model refuses."""


@dataclasses.dataclass(frozen=True)
class UnitType:
    """src/nanorts/model/unit_types.py:16-32 (defaults are MicroRTS's)."""

    name: str
    cost: int = 1
    hit_points: int = 1
    produce_time: int = 10
    move_time: int = 10
    attack_time: int = 10
    harvest_time: int = 10
    attack_range: int = 1
    attack_damage: int = 1
    harvest_amount: int = 1
    sight_radius: int = 4
    is_resource: bool = False
    is_stockpile: bool = False
    can_harvest: bool = False
    can_move: bool = True
    can_attack: bool = True
    produced_by: tuple[str, ...] = ()


# MicroRTS's UnitTypeTable, VERSION_ORIGINAL and VERSION_ORIGINAL_FINETUNED
# (src/nanorts/model/unit_types.py:47-148).  The values are the game's rules.
_RESOURCE = UnitType("Resource", sight_radius=0, is_resource=True, can_move=False, can_attack=False)
_BASE = UnitType("Base", cost=10, hit_points=10, produce_time=250, sight_radius=5, is_stockpile=True,
                 can_move=False, can_attack=False, produced_by=("Worker",))
_BARRACKS = UnitType("Barracks", cost=5, hit_points=4, produce_time=200, sight_radius=3, can_move=False,
                     can_attack=False, produced_by=("Worker",))
_WORKER = UnitType("Worker", produce_time=50, attack_time=5, harvest_time=20, sight_radius=3, can_harvest=True,
                   produced_by=("Base",))
_LIGHT = UnitType("Light", cost=2, hit_points=4, produce_time=80, move_time=8, attack_time=5, attack_damage=2,
                  sight_radius=2, produced_by=("Barracks",))
_HEAVY = UnitType("Heavy", cost=2, hit_points=4, produce_time=120, move_time=12, attack_time=5, attack_damage=4,
                  sight_radius=2, produced_by=("Barracks",))
_RANGED = UnitType("Ranged", cost=2, produce_time=100, attack_time=5, attack_range=3, sight_radius=3,
                   produced_by=("Barracks",))

TABLES: Final = {
    UnitTypeTableVersion.ORIGINAL: (_RESOURCE, _BASE, _BARRACKS, _WORKER, _LIGHT, _HEAVY, _RANGED),
    UnitTypeTableVersion.ORIGINAL_FINETUNED: (
        _RESOURCE,
        dataclasses.replace(_BASE, produce_time=200),
        dataclasses.replace(_BARRACKS, produce_time=100),
        _WORKER,
        _LIGHT,
        dataclasses.replace(_HEAVY, cost=3, hit_points=8, move_time=10),
        _RANGED,
    ),
}

TYPE_NAMES: Final = tuple(unit.name for unit in TABLES[UnitTypeTableVersion.ORIGINAL])
TYPE_RESOURCE, TYPE_BASE, TYPE_BARRACKS, TYPE_WORKER, TYPE_LIGHT, TYPE_HEAVY, TYPE_RANGED = range(7)

_INT_COLUMNS: Final = ("cost", "hit_points", "produce_time", "move_time", "attack_time", "harvest_time",
                       "attack_range", "attack_damage", "harvest_amount", "sight_radius")
_BOOL_COLUMNS: Final = ("is_resource", "is_stockpile", "can_harvest", "can_move", "can_attack")


def unit_columns(table: tuple[UnitType, ...]) -> dict[str, np.ndarray]:
    """Per-type columns and the produces[producer, produced] matrix
    (src/nanorts/model/unit_types.py:151-174)."""
    columns = {name: np.asarray([getattr(u, name) for u in table], np.int32) for name in _INT_COLUMNS}
    columns.update({name: np.asarray([getattr(u, name) for u in table], np.bool_) for name in _BOOL_COLUMNS})
    columns["produces"] = np.asarray([[producer.name in produced.produced_by for produced in table]
                                      for producer in table], np.bool_)
    return columns


@dataclasses.dataclass(frozen=True)
class BucketSpec:
    """Static shapes of one content (src/nanorts/model/bucket.py:24-58)."""

    height: int
    width: int
    neutral_capacity: int
    per_player_capacity: int
    unit_type_capacity: int
    attack_offset_capacity: int
    utt_identity: UnitTypeTableVersion
    conflict_strategy: ConflictStrategy

    @property
    def cell_count(self) -> int:
        return self.height * self.width

    @property
    def entity_capacity(self) -> int:
        return self.neutral_capacity + PLAYER_COUNT * self.per_player_capacity

    @property
    def attack_window_side(self) -> int:
        return math.isqrt(self.attack_offset_capacity)

    @property
    def max_attack_range(self) -> int:
        return (self.attack_window_side - 1) // 2

    def player_slot_start(self, player: int) -> int:
        return self.neutral_capacity + player * self.per_player_capacity


# ---------------------------------------------------------------------------
# State leaves (src/nanorts/model/state.py:33-84) in declaration order.
# kind: "slot" [E], "field" [H, W], "scalar" [], "player" [2]
# ---------------------------------------------------------------------------
@dataclasses.dataclass(frozen=True)
class LeafSpec:
    name: str
    kind: str
    dtype: np.dtype
    fill: int


def _leaf(name: str, kind: str, dtype: type, fill: int) -> LeafSpec:
    return LeafSpec(name, kind, np.dtype(dtype), fill)


STATE_LEAVES: Final[tuple[LeafSpec, ...]] = (
    _leaf("birth", "slot", np.int32, ABSENT),
    _leaf("unit_type", "slot", np.int8, ABSENT),
    _leaf("owner", "slot", np.int8, ABSENT),
    _leaf("cell", "slot", np.int16, ABSENT),
    _leaf("hit_points", "slot", np.int16, 0),
    _leaf("carried_resources", "slot", np.int32, 0),
    _leaf("pending_kind", "slot", np.int8, KIND_ABSENT),
    _leaf("pending_direction", "slot", np.int8, ABSENT),
    _leaf("pending_none_duration", "slot", np.int32, 0),
    _leaf("pending_target_cell", "slot", np.int16, ABSENT),
    _leaf("pending_produced_type", "slot", np.int8, ABSENT),
    _leaf("pending_issued_at", "slot", np.int32, 0),
    _leaf("pending_completes_at", "slot", np.int32, 0),
    _leaf("pending_order", "slot", np.int32, ABSENT),
    _leaf("entity_at", "field", np.int16, ABSENT),
    _leaf("time", "scalar", np.int32, 0),
    _leaf("player_resources", "player", np.int32, 0),
    _leaf("next_birth", "scalar", np.int32, 0),
    _leaf("next_pending_order", "scalar", np.int32, 0),
    _leaf("alternating_conflict_count", "scalar", np.int32, 0),
    _leaf("game_over", "scalar", np.bool_, 0),
    _leaf("winner", "scalar", np.int32, ABSENT),
    _leaf("spawn_overflow", "player", np.int32, 0),  # telemetry.spawn_overflow
)

LEAF_NAMES: Final = tuple(leaf.name for leaf in STATE_LEAVES)
SLOT_LEAVES: Final = tuple(leaf.name for leaf in STATE_LEAVES if leaf.kind == "slot")
ROW_LEAVES: Final = SLOT_LEAVES + ("entity_at",)


def leaf_shape(leaf: LeafSpec, bucket: BucketSpec) -> tuple[int, ...]:
    if leaf.kind == "slot":
        return (bucket.entity_capacity,)
    if leaf.kind == "field":
        return (bucket.height, bucket.width)
    if leaf.kind == "player":
        return (PLAYER_COUNT,)
    return ()


def require_int16_indices(bucket: BucketSpec) -> None:
    """The reference picks int16 for cell and slot indices when their extents fit
    (src/nanorts/model/leaf.py:85-98); this build lays out the int16 case only."""
    if bucket.cell_count > np.iinfo(np.int16).max or bucket.entity_capacity > np.iinfo(np.int16).max:
        raise ModelError(
            f"a {bucket.height}x{bucket.width} board with {bucket.entity_capacity} slots needs int32 "
            "indices; this build lays out int16 cell and slot indices only")
