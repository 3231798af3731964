"""ctypes binding of the C oracle.  TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this
module, and only as the checker of the HIP path.  States are dicts of numpy
arrays with a leading env dimension, keyed by the reference's State leaf names
plus "environment_root" (uint32[L, 2]) and "episode_index" (uint32[L]).
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

from nanorts_amd.content import GameConfig
from nanorts_amd.model import LEAF_NAMES, STATE_LEAVES, STRATEGY_CODES, leaf_shape

HERE = Path(__file__).resolve().parent
LIBRARY_PATH = HERE / "libnanorts_oracle.so"
REF_PATH = HERE / "_ref" / "libref_draws.so"

MAX_TYPES = 8


def build() -> None:
    """Compile the oracle (and oracle/_ref when the reference checkout exists)."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)


def _load() -> ctypes.CDLL:
    if not LIBRARY_PATH.exists():
        build()
    lib = ctypes.CDLL(str(LIBRARY_PATH))
    lib.nro_rollout.restype = ctypes.c_int32
    lib.nro_state_violations.restype = ctypes.c_int32
    lib.nro_conflict_draw.restype = ctypes.c_int32
    lib.nro_randint01.restype = ctypes.c_int32
    lib.nro_episode_seat.restype = ctypes.c_int32
    lib.nro_astar.restype = ctypes.c_int32
    return lib


def astar(open_cells: np.ndarray, start: int, target: int, range_: int) -> tuple[int, int, int, int]:
    """pathfinding.search over bool[H, W] open cells: (found, step, distance, pops)."""
    lib = _load()
    H, W = open_cells.shape
    cells = np.ascontiguousarray(open_cells.reshape(-1).astype(np.uint8))
    out = (ctypes.c_int32 * 4)()
    lib.nro_astar(_ptr(cells), ctypes.c_int32(W), ctypes.c_int32(H), ctypes.c_int32(start), ctypes.c_int32(target),
                  ctypes.c_int32(range_), out)
    return int(out[0]), int(out[1]), int(out[2]), int(out[3])


def astar_chain(free_cells: np.ndarray, claimed: np.ndarray, rows: np.ndarray, queue: np.ndarray, count: int,
                may_move: bool, reserved: int, balance: int, draws: np.ndarray, drawing: bool,
                fallback: tuple[int, int, int], blocked: tuple[int, int, int]) -> np.ndarray:
    """The FFI target nanorts_astar_chain for one lane over bool[H, W] free and
    claimed cells: decisions int32[capacity + 1, 4]."""
    lib = _load()
    H, W = free_cells.shape
    capacity, columns = rows.shape
    free_u8 = np.ascontiguousarray(free_cells.reshape(-1).astype(np.uint8))
    claimed_u8 = np.ascontiguousarray(claimed.reshape(-1).astype(np.uint8))
    rows = np.ascontiguousarray(rows, np.int32)
    queue = np.ascontiguousarray(queue, np.int32)
    draws = np.ascontiguousarray(np.asarray(draws, np.int32).reshape(-1))
    out = np.zeros((capacity + 1, 4), np.int32)
    f3 = (ctypes.c_int64 * 3)(*fallback)
    b3 = (ctypes.c_int64 * 3)(*blocked)
    lib.nro_astar_chain(_ptr(free_u8), _ptr(claimed_u8), _ptr(rows), _ptr(queue), ctypes.c_int32(count),
                        ctypes.c_int32(int(bool(may_move))), ctypes.c_int32(reserved), ctypes.c_int32(balance),
                        _ptr(draws), ctypes.c_int64(draws.size), ctypes.c_int32(int(bool(drawing))), ctypes.c_int32(W),
                        ctypes.c_int32(H), ctypes.c_int64(capacity), ctypes.c_int64(columns), f3, b3, _ptr(out))
    return out


_I32x8 = ctypes.c_int32 * MAX_TYPES


class Game(ctypes.Structure):
    _fields_ = [
        ("height", ctypes.c_int32), ("width", ctypes.c_int32), ("cells", ctypes.c_int32),
        ("neutral", ctypes.c_int32), ("capacity", ctypes.c_int32), ("entities", ctypes.c_int32),
        ("types", ctypes.c_int32), ("offsets", ctypes.c_int32), ("strategy", ctypes.c_int32),
        ("max_cycles", ctypes.c_int32),
        ("cost", _I32x8), ("hit_points", _I32x8), ("produce_time", _I32x8), ("move_time", _I32x8),
        ("attack_time", _I32x8), ("harvest_time", _I32x8), ("attack_range", _I32x8), ("attack_damage", _I32x8),
        ("harvest_amount", _I32x8), ("sight_radius", _I32x8), ("is_resource", _I32x8), ("is_stockpile", _I32x8),
        ("can_harvest", _I32x8), ("can_move", _I32x8), ("can_attack", _I32x8),
        ("produces", ctypes.c_int32 * (MAX_TYPES * MAX_TYPES)),
        ("terrain", ctypes.c_void_p),
    ]


_STATE_FIELDS = list(LEAF_NAMES) + ["environment_root", "episode_index"]


class State(ctypes.Structure):
    _fields_ = [(name, ctypes.c_void_p) for name in _STATE_FIELDS]


class Commands(ctypes.Structure):
    _fields_ = [(name, ctypes.c_void_p) for name in
                ("kind", "direction", "none_duration", "target_cell", "produced_type", "request_order")]


class StepOut(ctypes.Structure):
    _fields_ = [(name, ctypes.c_void_p) for name in
                ("terminated", "truncated", "reward", "admitted_harvest", "admitted_return", "admitted_produce",
                 "admitted_attack", "is_member", "records_i32", "records_i16", "records_i8")]


class EnvOut(ctypes.Structure):
    _fields_ = [(name, ctypes.c_void_p) for name in
                ("reward", "done", "terminated", "truncated", "winner", "spawn_overflowed", "feature_maps",
                 "scalars", "final_feature_maps", "final_scalars", "reward_components")]


ABSTRACT_FIELDS = ("kind", "unit_birth", "order", "target", "target_birth", "base", "base_birth", "cell",
                   "unit_type", "trained", "next_order")


class Abstract(ctypes.Structure):
    _fields_ = [(name, ctypes.c_void_p) for name in ABSTRACT_FIELDS]


def empty_carry(L: int, C: int) -> dict[str, np.ndarray]:
    """abstraction.empty_actions for L envs (src/nanorts/bots/abstraction.py:118-133)."""
    carry = {f: np.full((L, C), -1, np.int32) for f in ABSTRACT_FIELDS[:9]}
    carry["trained"] = np.zeros((L, C), np.uint8)
    carry["next_order"] = np.zeros(L, np.int32)
    return carry


def _ptr(array: np.ndarray | None) -> ctypes.c_void_p | None:
    if array is None:
        return None
    assert array.flags["C_CONTIGUOUS"], "oracle buffers must be C-contiguous"
    return ctypes.c_void_p(array.ctypes.data)


class Oracle:
    """The oracle bound to one game configuration."""

    def __init__(self, game: GameConfig):
        self.lib = _load()
        self.game = game
        bucket = game.bucket
        cols = game.columns
        self._terrain = np.ascontiguousarray(game.terrain.reshape(-1).astype(np.uint8))
        g = Game()
        g.height, g.width, g.cells = bucket.height, bucket.width, bucket.cell_count
        g.neutral, g.capacity, g.entities = bucket.neutral_capacity, bucket.per_player_capacity, bucket.entity_capacity
        g.types, g.offsets = bucket.unit_type_capacity, bucket.attack_offset_capacity
        g.strategy = STRATEGY_CODES[bucket.conflict_strategy]
        g.max_cycles = game.max_cycles
        T = bucket.unit_type_capacity
        for name in ("cost", "hit_points", "produce_time", "move_time", "attack_time", "harvest_time",
                     "attack_range", "attack_damage", "harvest_amount", "sight_radius", "is_resource",
                     "is_stockpile", "can_harvest", "can_move", "can_attack"):
            arr = getattr(g, name)
            for t in range(T):
                arr[t] = int(cols[name][t])
        for p in range(T):
            for q in range(T):
                g.produces[p * MAX_TYPES + q] = int(cols["produces"][p, q])
        g.terrain = self._terrain.ctypes.data
        self.g = g
        self.initial = batch_initial(game, 1, np.zeros((1, 2), np.uint32))
        self._initial_struct = state_struct(self.initial)
        self.width = 22 + T + bucket.attack_offset_capacity

    # -- helpers ---------------------------------------------------------
    def _s(self, state: dict[str, np.ndarray]) -> State:
        return state_struct(state)

    def core_step(self, state, commands: dict[str, np.ndarray], keys: np.ndarray) -> dict[str, np.ndarray]:
        L = state["time"].shape[0]
        T = self.game.bucket.unit_type_capacity
        E = self.game.bucket.entity_capacity
        out = {"terminated": np.zeros(L, np.uint8), "truncated": np.zeros(L, np.uint8),
               "reward": np.zeros((L, 2), np.float32), "admitted_harvest": np.zeros((L, 2), np.int32),
               "admitted_return": np.zeros((L, 2), np.int32), "admitted_produce": np.zeros((L, 2, T), np.int32),
               "admitted_attack": np.zeros((L, 2, 3), np.int32), "is_member": np.zeros((L, E), np.uint8),
               "records_i32": np.zeros((L, E, 6), np.int32), "records_i16": np.zeros((L, E, 4), np.int16),
               "records_i8": np.zeros((L, E, 6), np.int8)}
        keep = [np.ascontiguousarray(commands[f], np.int32) for f, _ in Commands._fields_]
        c = Commands(*[_ptr(a) for a in keep])
        o = StepOut(*[_ptr(out[f]) for f, _ in StepOut._fields_])
        keys = np.ascontiguousarray(keys, np.uint32)
        s = self._s(state)
        self.lib.nro_core_step(ctypes.byref(self.g), ctypes.byref(s), ctypes.byref(c), _ptr(keys),
                               ctypes.c_int64(L), ctypes.byref(o))
        return out

    def legality_rows(self, state) -> np.ndarray:
        L = state["time"].shape[0]
        rows = np.zeros((L, 2, self.game.bucket.per_player_capacity, self.width), np.uint8)
        self.lib.nro_legality_rows(ctypes.byref(self.g), ctypes.byref(self._s(state)), ctypes.c_int64(L), _ptr(rows))
        return rows.astype(bool)

    def avail_rows(self, state) -> np.ndarray:
        L = state["time"].shape[0]
        rows = np.zeros((L, 2, self.game.bucket.per_player_capacity, self.width), np.uint8)
        self.lib.nro_avail_rows(ctypes.byref(self.g), ctypes.byref(self._s(state)), ctypes.c_int64(L), _ptr(rows))
        return rows.astype(bool)

    def avail_words(self, state) -> np.ndarray:
        L = state["time"].shape[0]
        words = np.zeros((L, 2, self.game.bucket.per_player_capacity, 3), np.uint32)
        self.lib.nro_avail_words(ctypes.byref(self.g), ctypes.byref(self._s(state)), ctypes.c_int64(L), _ptr(words))
        return words

    def visible_cells(self, state, observer: int) -> np.ndarray:
        L = state["time"].shape[0]
        b = self.game.bucket
        cells = np.zeros((L, b.height, b.width), np.uint8)
        self.lib.nro_visible_cells(ctypes.byref(self.g), ctypes.byref(self._s(state)), ctypes.c_int64(L),
                                   ctypes.c_int32(observer), _ptr(cells))
        return cells.astype(bool)

    def symbolic(self, state, partial: bool) -> tuple[np.ndarray, np.ndarray]:
        L = state["time"].shape[0]
        b = self.game.bucket
        maps = np.zeros((L, 2, b.height, b.width, 6), np.uint8)
        scalars = np.zeros((L, 2, 4), np.int32)
        self.lib.nro_symbolic(ctypes.byref(self.g), ctypes.byref(self._s(state)), ctypes.c_int64(L),
                              ctypes.c_int32(int(partial)), _ptr(maps), _ptr(scalars))
        return maps, scalars

    def pixels(self, state, partial: bool, tiles: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
        L = state["time"].shape[0]
        b = self.game.bucket
        image = np.zeros((L, 2, 16 * b.height, 16 * b.width, 3), np.uint8)
        scalars = np.zeros((L, 2, 4), np.int32)
        tiles = np.ascontiguousarray(tiles, np.uint8)
        self.lib.nro_pixels(ctypes.byref(self.g), ctypes.byref(self._s(state)), ctypes.c_int64(L),
                            ctypes.c_int32(int(partial)), _ptr(tiles), _ptr(image), _ptr(scalars))
        return image, scalars

    def decode_actions(self, state, actions: np.ndarray) -> dict[str, np.ndarray]:
        L = state["time"].shape[0]
        C = self.game.bucket.per_player_capacity
        out = {f: np.zeros((L, 2, C), np.int32) for f, _ in Commands._fields_}
        c = Commands(*[_ptr(out[f]) for f, _ in Commands._fields_])
        actions = np.ascontiguousarray(actions, np.int32)
        self.lib.nro_decode_actions(ctypes.byref(self.g), ctypes.byref(self._s(state)), _ptr(actions),
                                    ctypes.c_int64(L), ctypes.byref(c))
        return out

    def sample_actions(self, rows: np.ndarray, sample_key, step: int, env0: int = 0) -> np.ndarray:
        L = rows.shape[0]
        C = self.game.bucket.per_player_capacity
        rows = np.ascontiguousarray(rows, np.uint8)
        key = np.ascontiguousarray(np.asarray(sample_key, np.uint32).reshape(2))
        actions = np.zeros((L, 2, C, 7), np.int32)
        self.lib.nro_sample_actions(ctypes.byref(self.g), _ptr(rows), _ptr(key), ctypes.c_int32(step),
                                    ctypes.c_int64(env0), ctypes.c_int64(L), _ptr(actions))
        return actions

    def reset_where_done(self, state, done: np.ndarray) -> None:
        L = state["time"].shape[0]
        done = np.ascontiguousarray(done, np.uint8)
        self.lib.nro_reset_where_done(ctypes.byref(self.g), ctypes.byref(self._initial_struct),
                                      ctypes.byref(self._s(state)), _ptr(done), ctypes.c_int64(L))

    def env_step(self, state, actions: np.ndarray, partial: bool, observe: bool = True,
                 final: bool = False) -> dict[str, np.ndarray]:
        """env.step with auto-reset; with final=True also the ending state's
        observation (final_feature_maps / final_scalars) and the reward
        components [L, 2, 6]."""
        L = state["time"].shape[0]
        b = self.game.bucket
        out = {"reward": np.zeros((L, 2), np.float32), "done": np.zeros(L, np.uint8),
               "terminated": np.zeros(L, np.uint8), "truncated": np.zeros(L, np.uint8),
               "winner": np.zeros(L, np.int32), "spawn_overflowed": np.zeros(L, np.uint8),
               "feature_maps": np.zeros((L, 2, b.height, b.width, 6), np.uint8) if observe else None,
               "scalars": np.zeros((L, 2, 4), np.int32) if observe else None,
               "final_feature_maps": np.zeros((L, 2, b.height, b.width, 6), np.uint8) if final else None,
               "final_scalars": np.zeros((L, 2, 4), np.int32) if final else None,
               "reward_components": np.zeros((L, 2, 6), np.float32) if final else None}
        o = EnvOut(*[_ptr(out.get(f)) for f, _ in EnvOut._fields_])
        actions = np.ascontiguousarray(actions, np.int32)
        self.lib.nro_env_step(ctypes.byref(self.g), ctypes.byref(self._initial_struct), ctypes.byref(self._s(state)),
                              _ptr(actions), ctypes.c_int64(L), ctypes.c_int32(int(partial)), ctypes.byref(o))
        return out

    def rollout(self, state, sample_key, step0: int, steps: int, partial: bool, threads: int = 1,
                record_actions: bool = False, record: bool = True, env0: int = 0) -> dict[str, np.ndarray]:
        L = state["time"].shape[0]
        b = self.game.bucket
        key = np.ascontiguousarray(np.asarray(sample_key, np.uint32).reshape(2))
        out = {
            "rewards": np.zeros((steps, L, 2), np.float32) if record else None,
            "dones": np.zeros((steps, L), np.uint8) if record else None,
            "actions": np.zeros((steps, L, 2, b.per_player_capacity, 7), np.int32) if record_actions else None,
            "feature_maps": np.zeros((L, 2, b.height, b.width, 6), np.uint8) if record else None,
            "scalars": np.zeros((L, 2, 4), np.int32) if record else None,
        }
        used = self.lib.nro_rollout(
            ctypes.byref(self.g), ctypes.byref(self._initial_struct), ctypes.byref(self._s(state)), _ptr(key),
            ctypes.c_int32(step0), ctypes.c_int32(steps), ctypes.c_int64(L), ctypes.c_int32(int(partial)),
            ctypes.c_int32(threads), _ptr(out["rewards"]), _ptr(out["dones"]), _ptr(out["actions"]),
            _ptr(out["feature_maps"]), _ptr(out["scalars"]), ctypes.c_int64(env0))
        out["threads"] = used
        return out

    def abstraction_act(self, state, carry: dict[str, np.ndarray], strategy: int, trained_type: int,
                        player) -> dict[str, np.ndarray]:
        """family.act: the bot's commands [L][2][C] per field; `carry` is updated in place."""
        L = state["time"].shape[0]
        C = self.game.bucket.per_player_capacity
        out = {f: np.zeros((L, 2, C), np.int32) for f, _ in Commands._fields_}
        c = Commands(*[_ptr(out[f]) for f, _ in Commands._fields_])
        players = np.ascontiguousarray(np.broadcast_to(np.asarray(player, np.int32), (L,)))
        a = Abstract(*[_ptr(carry[f]) for f in ABSTRACT_FIELDS])
        self.lib.nro_abstraction_act(ctypes.byref(self.g), ctypes.byref(self._s(state)), ctypes.c_int64(L),
                                     ctypes.c_int32(strategy), ctypes.c_int32(trained_type), _ptr(players),
                                     ctypes.byref(a), ctypes.byref(c))
        return out

    def seat_step(self, state, carry: dict[str, np.ndarray], strategy: int, trained_type: int, learner,
                  actions: np.ndarray, partial: bool, observe: bool = True, draw: bool = False) -> dict[str, np.ndarray]:
        """step_seat with the learner's action rows [L][C][7]; state and carry
        updated in place.  `learner` is 0, 1 or an int32[L] array of per-lane
        seats, which (with draw=True, the "drawn" rule) is updated in place
        where a game ended."""
        L = state["time"].shape[0]
        b = self.game.bucket
        out = {"reward": np.zeros((L, 2), np.float32), "done": np.zeros(L, np.uint8),
               "terminated": np.zeros(L, np.uint8), "truncated": np.zeros(L, np.uint8),
               "winner": np.zeros(L, np.int32), "spawn_overflowed": np.zeros(L, np.uint8),
               "feature_maps": np.zeros((L, 2, b.height, b.width, 6), np.uint8) if observe else None,
               "scalars": np.zeros((L, 2, 4), np.int32) if observe else None}
        o = EnvOut(*[_ptr(out.get(f)) for f, _ in EnvOut._fields_])
        a = Abstract(*[_ptr(carry[f]) for f in ABSTRACT_FIELDS])
        actions = np.ascontiguousarray(actions, np.int32)
        seats = None
        if isinstance(learner, np.ndarray):
            seats = learner
            if seats.dtype != np.int32 or seats.shape != (L,) or not seats.flags.c_contiguous:
                raise ValueError(f"per-lane seats must be a contiguous int32[{L}] array")
        self.lib.nro_seat_step(ctypes.byref(self.g), ctypes.byref(self._initial_struct), ctypes.byref(self._s(state)),
                               ctypes.c_int64(L), ctypes.c_int32(strategy), ctypes.c_int32(trained_type),
                               ctypes.c_int32(0 if seats is not None else int(learner)), _ptr(seats),
                               ctypes.c_int32(int(draw)), ctypes.byref(a), _ptr(actions),
                               ctypes.c_int32(int(partial)), ctypes.byref(o))
        return out

    def episode_seats(self, state) -> np.ndarray:
        """The "drawn" seat of each lane's current episode root, int32[L]."""
        lib = self.lib
        out = np.zeros(state["time"].shape[0], np.int32)
        for l, (root, ep) in enumerate(zip(state["environment_root"].reshape(-1, 2), state["episode_index"])):
            k = (ctypes.c_uint32 * 2)()
            lib.nro_fold_in((ctypes.c_uint32 * 2)(int(root[0]), int(root[1])), ctypes.c_uint32(int(ep)), k)
            out[l] = lib.nro_episode_seat(k)
        return out

    def gridnet_decode(self, state, actions: np.ndarray) -> dict[str, np.ndarray]:
        """GridNet decode_actions: per-cell actions [L][2][H][W][7] -> Commands [L][2][C] per field."""
        L = state["time"].shape[0]
        C = self.game.bucket.per_player_capacity
        out = {f: np.zeros((L, 2, C), np.int32) for f, _ in Commands._fields_}
        c = Commands(*[_ptr(out[f]) for f, _ in Commands._fields_])
        actions = np.ascontiguousarray(actions, np.int32)
        self.lib.nro_gridnet_decode(ctypes.byref(self.g), ctypes.byref(self._s(state)), _ptr(actions),
                                    ctypes.c_int64(L), ctypes.byref(c))
        return out

    def gridnet_sample_actions(self, rows: np.ndarray, sample_key, step: int, env0: int = 0) -> np.ndarray:
        """The harness sampler over per-cell rows [L][2][cells][78] -> actions [L][2][cells][7]."""
        L = rows.shape[0]
        cells = self.game.bucket.cell_count
        rows = np.ascontiguousarray(rows.reshape(L, 2, cells, self.width), np.uint8)
        key = np.ascontiguousarray(np.asarray(sample_key, np.uint32).reshape(2))
        actions = np.zeros((L, 2, cells, 7), np.int32)
        self.lib.nro_gridnet_sample_actions(ctypes.byref(self.g), _ptr(rows), _ptr(key), ctypes.c_int32(step),
                                            ctypes.c_int64(env0), ctypes.c_int64(L), _ptr(actions))
        return actions

    def violations(self, state) -> np.ndarray:
        L = state["time"].shape[0]
        s = self._s(state)
        return np.asarray([self.lib.nro_state_violations(ctypes.byref(self.g), ctypes.byref(s), ctypes.c_int64(l))
                           for l in range(L)], np.int32)


def state_struct(state: dict[str, np.ndarray]) -> State:
    for name in _STATE_FIELDS:
        if name in state:
            assert state[name].flags["C_CONTIGUOUS"], name
    return State(*[_ptr(state.get(name)) for name in _STATE_FIELDS])


def batch_initial(game: GameConfig, L: int, roots: np.ndarray) -> dict[str, np.ndarray]:
    """L copies of the decided initial state with the given env roots."""
    state = {leaf.name: np.ascontiguousarray(np.broadcast_to(game.initial_state[leaf.name],
                                                             (L, *leaf_shape(leaf, game.bucket))).copy())
             for leaf in STATE_LEAVES}
    state["environment_root"] = np.ascontiguousarray(np.asarray(roots, np.uint32).reshape(L, 2))
    state["episode_index"] = np.zeros(L, np.uint32)
    return state


def copy_state(state: dict[str, np.ndarray]) -> dict[str, np.ndarray]:
    return {k: v.copy() for k, v in state.items()}


# -- RNG helpers -------------------------------------------------------------
def threefry2x32(lib_or_none, key, x) -> tuple[int, int]:
    lib = lib_or_none or _load()
    k = (ctypes.c_uint32 * 2)(*[int(v) & 0xFFFFFFFF for v in key])
    xs = (ctypes.c_uint32 * 2)(*[int(v) & 0xFFFFFFFF for v in x])
    lib.nro_threefry2x32(k, xs)
    return int(xs[0]), int(xs[1])


def load_library() -> ctypes.CDLL:
    return _load()


def load_reference_draws() -> ctypes.CDLL | None:
    """oracle/_ref: the reference's own RNG header built with hipcc, or None."""
    if not REF_PATH.exists() and os.path.isdir("/root/reference"):
        build()
    return ctypes.CDLL(str(REF_PATH)) if REF_PATH.exists() else None
