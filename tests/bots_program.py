"""A second formulation of the scripted bots, in the reference's array form.

The oracle's act (oracle/bots.c) walks units one at a time the way a block of
threads does.  This module restates the same decisions the way the reference's
program stage writes them: whole-player numpy arrays, one mask per rule, the
abstract-action carry rewritten by `put` and settled after translation.  It
follows src/nanorts/bots/rush.py (WorkerRush, the barracks rushes),
src/nanorts/bots/defense.py (the two defenses) and
src/nanorts/bots/abstraction.py:136-1119 (own_units, put, the building-site
ring walk, pending usage, standing entries, plans, the in-order walk of A*
searches and keep rules, the Commands rows and the settled carry).  The A*
search is `astar_by_keys`, the global-argmin key form of
src/nanorts/bots/pathfinding.py:170-245, itself checked against breadth-first
distances in tests/test_bots_oracle.py.

Only tests import it; one env at a time, plain numpy, no oracle code.
"""
from __future__ import annotations

import numpy as np

ABSENT = -1
LAST = 2**31 - 1
NONE, MOVE, HARVEST_K, RETURN, PRODUCE, ATTACK_K = range(6)  # command kinds
UP, RIGHT, DOWN, LEFT = range(4)
STEP_X = (0, 1, 0, -1)
STEP_Y = (-1, 0, 1, 0)
BASE, BARRACKS, WORKER = 1, 2, 3
# abstract kinds (src/nanorts/bots/abstraction.py:34-44); the rush family holds four
ATTACK, HARVEST, TRAIN, BUILD = 1, 2, 3, 4
WORKER_RUSH, BARRACKS_RUSH, WORKER_DEFENSE, BARRACKS_DEFENSE = range(4)
FILLER_DURATION = 10
CARRY_FIELDS = ("kind", "unit_birth", "order", "target", "target_birth", "base", "base_birth", "cell", "unit_type")
DESIRE_FIELDS = ("kind", "direction", "target_cell", "produced_type", "claimed", "cost", "none_duration")


# ---------------------------------------------------------------------------
# A* in key form
# ---------------------------------------------------------------------------
def astar_by_keys(free: np.ndarray, start: int, target: int, range_: int):
    """The search in the program's key form: every open cell holds
    f * (cells + 1) + (cells - sequence); the least key is popped.
    Returns (found, first step, path length, pops)."""
    H, W = free.shape
    cells = H * W
    closed = 2**31 - 1
    blocked, unseen = closed - 1, closed - 2
    key = np.where(free.reshape(-1), unseen, blocked).astype(np.int64)
    after = np.full(cells, -1, np.int64)
    tx, ty = target % W, target // W

    def manhattan(c):
        return abs(c % W - tx) + abs(c // W - ty)

    if 0 <= start < cells:
        key[start] = manhattan(start) * (cells + 1) + cells
        after[start] = start
    inserted, goal, pops, searching = 1, -1, 0, True
    while searching and pops < cells:
        cell = int(np.argmin(key))
        k = int(key[cell])
        exhausted = k >= unseen
        reached = not exhausted and (cell % W - tx) ** 2 + (cell // W - ty) ** 2 <= range_ * range_
        expands = not exhausted and not reached
        if expands:
            g = k // (cells + 1) - manhattan(cell)
            fresh = []
            for dx, dy in zip(STEP_X, STEP_Y):
                x, y = cell % W + dx, cell // W + dy
                if 0 <= x < W and 0 <= y < H and key[y * W + x] == unseen:
                    fresh.append(y * W + x)
            key[cell] = closed
            for n in fresh:
                key[n] = (g + 1 + manhattan(n)) * (cells + 1) + (cells - inserted)
                after[n] = n if cell == start else after[cell]
                inserted += 1
        if reached:
            goal = cell
        searching = expands
        pops += 0 if exhausted else 1
    if goal < 0:
        return 0, -1, -1, pops
    offset = int(after[goal]) - start
    # jnp.select: the first matching case wins (on a one-wide board -1 is LEFT)
    step = next((d for o, d in ((W, DOWN), (-1, LEFT), (-W, UP), (1, RIGHT)) if offset == o), -1)
    return 1, step, int(key[goal]) // (cells + 1) - manhattan(goal), pops


# ---------------------------------------------------------------------------
# Board facts of one env
# ---------------------------------------------------------------------------
class Board:
    """One env's state leaves and the game's columns, as int64 arrays."""

    def __init__(self, game, state: dict[str, np.ndarray], env: int, player: int):
        b = game.bucket
        self.H, self.W, self.cells = b.height, b.width, b.cell_count
        self.N, self.C, self.T = b.neutral_capacity, b.per_player_capacity, b.unit_type_capacity
        self.col = {k: np.asarray(v).astype(np.int64) for k, v in game.columns.items() if k != "produces"}
        self.terrain = np.asarray(game.terrain).reshape(-1).astype(bool)
        s = {k: np.asarray(v[env]).astype(np.int64) for k, v in state.items()}
        self.birth, self.cell, self.owner = s["birth"], s["cell"], s["owner"]
        self.unit_type = s["unit_type"]
        self.every_type = np.clip(self.unit_type, 0, self.T - 1)
        self.carried = s["carried_resources"]
        self.pending_kind, self.pending_direction = s["pending_kind"], s["pending_direction"]
        self.pending_produced = s["pending_produced_type"]
        self.entity_at = s["entity_at"].reshape(-1)
        self.resources = s["player_resources"].reshape(-1)
        self.active = self.birth != ABSENT
        self.player = player

    def neighbour(self, cell, direction):
        known = np.clip(direction, 0, 3)
        return cell + np.asarray(STEP_Y)[known] * self.W + np.asarray(STEP_X)[known]

    def squared_distance(self, a, b):
        dx = a % self.W - b % self.W
        dy = a // self.W - b // self.W
        return dx * dx + dy * dy

    def exists(self, slot, birth):
        known = np.clip(slot, 0, self.birth.shape[0] - 1)
        return (slot != ABSENT) & (self.birth[known] == birth)

    def cell_of(self, slot):
        known = np.clip(slot, 0, self.cell.shape[0] - 1)
        return np.where(slot != ABSENT, self.cell[known], ABSENT)

    def enemies(self):
        return self.active & (self.owner != ABSENT) & (self.owner != self.player)


def rank(among, key):
    """How many of `among` hold a smaller key (abstraction.py:_rank)."""
    return np.sum(among[None, :] & (key[None, :] < key[:, None]), axis=1)


class Units:
    """abstraction.own_units (src/nanorts/bots/abstraction.py:136-158)."""

    def __init__(self, bd: Board):
        first = bd.N + bd.player * bd.C
        own = slice(first, first + bd.C)
        self.birth = bd.birth[own]
        self.cell = bd.cell[own]
        self.unit_type = np.clip(bd.unit_type[own], 0, bd.T - 1)
        self.carried = bd.carried[own]
        self.present = self.birth != ABSENT
        self.available = self.present & (bd.pending_kind[own] == ABSENT)
        self.birth_rank = rank(self.present, self.birth)


class Carry:
    """AbstractActions of one env: nine int64 columns, trained, next_order."""

    def __init__(self, carry: dict[str, np.ndarray], env: int):
        for f in CARRY_FIELDS:
            setattr(self, f, np.asarray(carry[f][env]).astype(np.int64).copy())
        self.trained = np.asarray(carry["trained"][env]).astype(bool).copy()
        self.next_order = int(carry["next_order"][env])


# ---------------------------------------------------------------------------
# put and the rush rules (src/nanorts/bots/rush.py)
# ---------------------------------------------------------------------------
def is_entry(a: Carry, u: Units, kind):
    return (a.kind == kind) & (a.unit_birth == u.birth)


def put(a: Carry, u: Units, chosen, last, kind, **fields):
    """abstraction.put: chosen rows take the entry; rows not already holding
    an entry for this unit take the stamp next_order + (C if last else the
    unit's birth rank); next_order advances by C + 1 on every call."""
    C = chosen.shape[0]
    known = (a.kind != ABSENT) & (a.unit_birth == u.birth)
    fresh = chosen & ~known
    stamp = a.next_order + np.where(last, C, u.birth_rank)
    values = {"kind": kind, "unit_birth": u.birth, **{f: fields.get(f, ABSENT) for f in CARRY_FIELDS[3:]}}
    for f, v in values.items():
        setattr(a, f, np.where(chosen, np.broadcast_to(np.asarray(v, np.int64), (C,)), getattr(a, f)))
    a.order = np.where(fresh, stamp, a.order)
    a.trained = np.where(chosen, False, a.trained)
    a.next_order += C + 1


def first_in_unit_order(chosen, u: Units):
    first = int(np.argmin(np.where(chosen, u.birth, LAST)))
    return chosen & (np.arange(chosen.shape[0]) == first)


class Closest:
    def __init__(self, bd: Board, origin, candidates):
        """rush._closest: Manhattan nearest candidate per origin, ties to the
        smallest birth."""
        d = np.abs(origin[:, None] % bd.W - bd.cell[None, :] % bd.W) + np.abs(
            origin[:, None] // bd.W - bd.cell[None, :] // bd.W)
        d = np.where(candidates[None, :], d, LAST)
        nearest = d.min(axis=1)
        tied = candidates[None, :] & (d == nearest[:, None])
        slot = np.argmin(np.where(tied, bd.birth[None, :], LAST), axis=1)
        self.found = np.broadcast_to(candidates.any(), slot.shape)
        self.slot = np.where(self.found, slot, ABSENT)
        self.birth = np.where(self.found, bd.birth[slot], ABSENT)
        self.distance = nearest


def nearest_enemy(bd: Board, u: Units):
    return Closest(bd, u.cell, bd.enemies())


def attack_nearest(a, u, attackers, last, enemy: Closest):
    put(a, u, attackers & enemy.found, last, ATTACK, target=enemy.slot, target_birth=enemy.birth)


def available_melee(bd: Board, u: Units):
    return u.present & (bd.col["can_attack"][u.unit_type] != 0) & (bd.col["can_harvest"][u.unit_type] == 0) & u.available


def train_workers(bd, a, u, resources):
    trains = u.present & (u.unit_type == BASE) & u.available & (resources >= bd.col["cost"][WORKER])
    put(a, u, trains, False, TRAIN, unit_type=WORKER)


def visit_order(bd: Board, desired: int):
    """abstraction._visits seen from `desired`: rings outward, each ring's top
    side, right side, bottom side, left side; the centre is never visited."""
    x = np.arange(bd.cells) % bd.W - desired % bd.W
    y = np.arange(bd.cells) // bd.W - desired // bd.W
    ring = np.maximum(np.abs(x), np.abs(y))
    side = np.where(y == -ring, 0, np.where(x == ring, 1, np.where(y == ring, 2, 3)))
    along = np.where((side == 0) | (side == 2), x, y) + ring
    longest = max(bd.H, bd.W)
    return np.where(ring == 0, LAST, (ring * 4 + side) * (2 * longest + 1) + along)


def building_site(bd: Board, desired: int, reserved):
    visit = visit_order(bd, desired)
    open_cells = ~bd.terrain & (bd.entity_at == ABSENT) & ~reserved & (visit != LAST)
    return int(np.argmin(np.where(open_cells, visit, LAST))) if open_cells.any() else ABSENT


def build_if_not_already_building(bd, a, u, builder, unit_type, reserved):
    building = is_entry(a, u, BUILD) & (a.unit_type == unit_type)
    builds = builder & ~building
    desired = int(np.sum(np.where(builder, u.cell, 0)))
    site = building_site(bd, desired, reserved)
    put(a, u, builds, False, BUILD, cell=site, unit_type=unit_type)
    return reserved | (builds.any() & (np.arange(bd.cells) == site))


def build_base(bd, a, u, workers):
    bases = u.present & (u.unit_type == BASE)
    builds = (not bases.any()) and bd.resources[bd.player] >= bd.col["cost"][BASE]
    builder = first_in_unit_order(workers, u) & builds
    reserved = build_if_not_already_building(bd, a, u, builder, BASE, np.zeros(bd.cells, bool))
    return builder, reserved


def train_at_base_and_barracks(bd, a, u, resources, trained_type):
    workers_held = int(np.sum(u.present & (u.unit_type == WORKER)))
    trains_worker = (u.present & (u.unit_type == BASE) & u.available & (workers_held < 1)
                     & (resources >= bd.col["cost"][WORKER]))
    put(a, u, trains_worker, False, TRAIN, unit_type=WORKER)
    barracks_train = (u.present & (u.unit_type == BARRACKS) & u.available
                      & (resources >= bd.col["cost"][trained_type]))
    put(a, u, barracks_train, False, TRAIN, unit_type=trained_type)


def harvest_sites(bd: Board, u: Units):
    resource = Closest(bd, u.cell, bd.active & (bd.col["is_resource"][bd.every_type] != 0))
    stockpile = Closest(bd, u.cell, bd.active & (bd.col["is_stockpile"][bd.every_type] != 0)
                        & (bd.owner == bd.player))
    return resource, stockpile


def rush_harvest(bd, a, u, harvesters):
    resource, stockpile = harvest_sites(bd, u)
    carrying = u.carried > 0
    same_base = (a.base == stockpile.slot) & (a.base_birth == stockpile.birth)
    same_target = (a.target == resource.slot) & (a.target_birth == resource.birth)
    occupied = np.where(carrying, stockpile.found, stockpile.found & resource.found)
    unchanged = is_entry(a, u, HARVEST) & same_base & (carrying | same_target)
    put(a, u, harvesters & occupied & ~unchanged, False, HARVEST,
        target=np.where(carrying, ABSENT, resource.slot), target_birth=np.where(carrying, ABSENT, resource.birth),
        base=stockpile.slot, base_birth=stockpile.birth)
    return harvesters & ~occupied


def build_base_and_barracks(bd, a, u):
    resources = bd.resources[bd.player]
    workers = u.present & (bd.col["can_harvest"][u.unit_type] != 0)
    barracks = u.present & (u.unit_type == BARRACKS)
    base_builder, reserved = build_base(bd, a, u, workers)
    used = bd.col["cost"][BASE] if base_builder.any() else 0
    builds_barracks = (not barracks.any()) and resources >= bd.col["cost"][BARRACKS] + used
    barracks_builder = first_in_unit_order(workers & ~base_builder, u) & builds_barracks
    build_if_not_already_building(bd, a, u, barracks_builder, BARRACKS, reserved)
    return workers & ~base_builder & ~barracks_builder


def worker_rush(bd, a, u):
    resources = bd.resources[bd.player]
    enemy = nearest_enemy(bd, u)
    train_workers(bd, a, u, resources)
    attack_nearest(a, u, available_melee(bd, u), False, enemy)
    workers = u.present & (bd.col["can_harvest"][u.unit_type] != 0)
    builder, _ = build_base(bd, a, u, workers)
    harvester = first_in_unit_order(workers & ~builder, u)
    idle_harvester = rush_harvest(bd, a, u, harvester)
    free = (workers & ~builder & ~harvester) | idle_harvester
    attack_nearest(a, u, free, idle_harvester, enemy)


def barracks_rush(bd, a, u, trained_type):
    resources = bd.resources[bd.player]
    enemy = nearest_enemy(bd, u)
    train_at_base_and_barracks(bd, a, u, resources, trained_type)
    attack_nearest(a, u, available_melee(bd, u), False, enemy)
    free = build_base_and_barracks(bd, a, u)
    idle = rush_harvest(bd, a, u, free)
    attack_nearest(a, u, idle, False, enemy)


# ---------------------------------------------------------------------------
# defense (src/nanorts/bots/defense.py)
# ---------------------------------------------------------------------------
def defend(bd, a, u, defenders, enemy: Closest):
    reach = bd.H // 2
    bases = u.present & (u.unit_type == BASE)
    base = u.cell[int(np.argmax(np.where(bases, u.birth, ABSENT)))]
    base_distance = (np.abs(u.cell % bd.W - base % bd.W) + np.abs(u.cell // bd.W - base // bd.W)
                     if bases.any() else np.zeros_like(u.cell))
    engages = enemy.found & ((enemy.distance < reach) | (base_distance < reach))
    put(a, u, defenders, False, ATTACK, target=np.where(engages, enemy.slot, ABSENT),
        target_birth=np.where(engages, enemy.birth, ABSENT))


def defense_harvest(bd, a, u, harvesters):
    resource, stockpile = harvest_sites(bd, u)
    unchanged = (is_entry(a, u, HARVEST) & (a.target == resource.slot) & (a.target_birth == resource.birth)
                 & (a.base == stockpile.slot) & (a.base_birth == stockpile.birth))
    put(a, u, harvesters & resource.found & stockpile.found & ~unchanged, False, HARVEST,
        target=resource.slot, target_birth=resource.birth, base=stockpile.slot, base_birth=stockpile.birth)


def worker_defense(bd, a, u):
    resources = bd.resources[bd.player]
    enemy = nearest_enemy(bd, u)
    train_workers(bd, a, u, resources)
    defend(bd, a, u, available_melee(bd, u), enemy)
    workers = u.present & (bd.col["can_harvest"][u.unit_type] != 0)
    builder, _ = build_base(bd, a, u, workers)
    harvester = first_in_unit_order(workers & ~builder, u)
    defense_harvest(bd, a, u, harvester)
    defend(bd, a, u, workers & ~builder & ~harvester, enemy)


def barracks_defense(bd, a, u, trained_type):
    resources = bd.resources[bd.player]
    enemy = nearest_enemy(bd, u)
    train_at_base_and_barracks(bd, a, u, resources, trained_type)
    defend(bd, a, u, available_melee(bd, u), enemy)
    free = build_base_and_barracks(bd, a, u)
    defense_harvest(bd, a, u, free)


# ---------------------------------------------------------------------------
# translate (src/nanorts/bots/abstraction.py:262-288, kinds = the rush family's)
# ---------------------------------------------------------------------------
def no_desire(n):
    d = {f: np.full(n, ABSENT, np.int64) for f in DESIRE_FIELDS}
    d["cost"][:] = 0
    d["none_duration"][:] = 0
    return d


def choose(chosen, mine, theirs):
    return {f: np.where(chosen, mine[f], theirs[f]) for f in DESIRE_FIELDS}


def adjacent_direction(bd: Board, origin, goal):
    dx = goal % bd.W - origin % bd.W
    dy = goal // bd.W - origin // bd.W
    matches = (dx[:, None] == np.asarray(STEP_X)) & (dy[:, None] == np.asarray(STEP_Y))
    found = (goal != ABSENT) & matches.any(axis=1)
    return np.where(found, np.argmax(matches, axis=1), ABSENT)


class Usage:
    """abstraction._pending_usage: cells claimed by pending moves and
    productions, the cost each player's pending productions hold back."""

    def __init__(self, bd: Board):
        claims = bd.active & ((bd.pending_kind == MOVE) | (bd.pending_kind == PRODUCE))
        target = bd.neighbour(bd.cell, bd.pending_direction)
        self.claimed = np.zeros(bd.cells, bool)
        self.claimed[target[claims & (target >= 0) & (target < bd.cells)]] = True
        produced = np.clip(bd.pending_produced, 0, bd.T - 1)
        cost = np.where(bd.active & (bd.pending_kind == PRODUCE), bd.col["cost"][produced], 0)
        self.reserved = cost[bd.N:].reshape(2, bd.C).sum(axis=1)
        self.balance = bd.resources

    def within_balance(self):
        return (self.reserved == 0) | (self.reserved <= self.balance)


def production(bd, usage: Usage, direction, produced_type, cell):
    own = bd.player
    claimed = np.where(direction != ABSENT, bd.neighbour(cell, direction), ABSENT)
    cost = bd.col["cost"][np.clip(produced_type, 0, bd.T - 1)]
    reserved = usage.reserved[own]
    allowed = ((direction != ABSENT) & ~usage.claimed[np.clip(claimed, 0, bd.cells - 1)]
               & ((reserved == 0) | (cost + reserved <= usage.balance[own])) & usage.within_balance()[1 - own])
    n = direction.shape[0]
    made = no_desire(n)
    made.update(kind=np.full(n, PRODUCE), direction=direction, produced_type=produced_type, claimed=claimed, cost=cost)
    return choose(allowed, made, no_desire(n))


def training_direction(bd: Board, a: Carry, u: Units, free):
    x = u.cell[:, None] % bd.W + np.asarray(STEP_X)
    y = u.cell[:, None] // bd.W + np.asarray(STEP_Y)
    on_board = (x >= 0) & (x < bd.W) & (y >= 0) & (y < bd.H)
    open_cells = on_board & free[np.where(on_board, y * bd.W + x, 0)]
    resource = bd.active & (bd.col["is_resource"][bd.every_type] != 0)
    harvests = bd.col["can_harvest"][np.clip(a.unit_type, 0, bd.T - 1)] != 0
    near = np.where(harvests[:, None], resource[None, :], bd.enemies()[None, :])
    distance = (np.abs(x[..., None] - bd.cell % bd.W) + np.abs(y[..., None] - bd.cell // bd.W))
    closest = np.where(near[:, None, :], distance, LAST).min(axis=-1)
    score = np.where(near.any(axis=-1)[:, None], -closest, 0)
    best = np.argmax(np.where(open_cells, score, -LAST), axis=-1)
    return np.where(open_cells.any(axis=-1), best, ABSENT)


def standing_entries(bd: Board, a: Carry, u: Units):
    alive = (a.kind != ABSENT) & (a.unit_birth == u.birth)
    carrying = u.carried > 0
    built_on = (a.cell != ABSENT) & (bd.entity_at[np.clip(a.cell, 0, bd.cells - 1)] != ABSENT)
    target_gone = ~bd.exists(a.target, a.target_birth)
    completed = np.select(
        [a.kind == ATTACK, a.kind == HARVEST, a.kind == TRAIN, a.kind == BUILD],
        [target_gone, np.where(carrying, ~bd.exists(a.base, a.base_birth), target_gone), a.trained, built_on],
        False)
    return alive & ~completed


def translate(bd: Board, a: Carry, wait: int = FILLER_DURATION):
    """The Commands rows of the acting player and the settled carry."""
    u = Units(bd)
    C = bd.C
    usage = Usage(bd)
    standing = standing_entries(bd, a, u)
    executes = standing & u.available
    kind = a.kind
    # _reach
    target_cell = bd.cell_of(a.target)
    attack_range = bd.col["attack_range"][u.unit_type]
    in_range = bd.squared_distance(u.cell, target_cell) <= attack_range * attack_range
    # _plan (no MOVE, COAC or drawing kinds in this family)
    free = ~(bd.terrain | (bd.entity_at != ABSENT) | usage.claimed)
    attacks, harvests, builds = kind == ATTACK, kind == HARVEST, kind == BUILD
    harvest_goal = np.where(u.carried > 0, bd.cell_of(a.base), target_cell)
    goal = np.select([attacks, harvests, builds], [target_cell, harvest_goal, a.cell], ABSENT)
    radius = np.select([attacks, harvests | builds], [attack_range, 1], 0)
    searches = (goal != ABSENT) & ~(attacks & in_range)
    plan_goal = np.where(searches, goal, u.cell)
    plan_radius = np.where(searches, radius, 0)
    # _fallback
    strike = no_desire(C)
    struck = in_range & (target_cell != ABSENT)
    strike.update(kind=np.where(struck, ATTACK_K, ABSENT), target_cell=np.where(struck, target_cell, ABSENT))
    hdir = adjacent_direction(bd, u.cell, harvest_goal)
    gather = no_desire(C)
    gather.update(kind=np.where(u.carried > 0, RETURN, HARVEST_K), direction=hdir)
    gather = choose(hdir != ABSENT, gather, no_desire(C))
    train = production(bd, usage, training_direction(bd, a, u, free), a.unit_type, u.cell)
    adjacent = production(bd, usage, adjacent_direction(bd, u.cell, a.cell), a.unit_type, u.cell)
    fallback = no_desire(C)
    for k, d in ((ATTACK, strike), (HARVEST, gather), (TRAIN, train), (BUILD, adjacent)):
        fallback = choose(kind == k, d, fallback)
    # the walk in queue order
    queue = np.argsort(np.where(executes, a.order, LAST), kind="stable")
    queued = int(executes.sum())
    moves_allowed = bool(usage.within_balance().all())
    used = np.zeros(bd.cells, bool)
    kept_cells = np.zeros(bd.cells, bool)
    kept_cost = kept_count = 0
    decided = no_desire(C)
    ranks = np.full(C, ABSENT, np.int64)
    for position in range(queued):
        i = int(queue[position])
        open_now = (free & ~used).reshape(bd.H, bd.W)
        _, step, _, _ = astar_by_keys(open_now, int(u.cell[i]), int(plan_goal[i]), int(plan_radius[i]))
        if step != ABSENT:
            desire = dict.fromkeys(DESIRE_FIELDS, ABSENT) | {"cost": 0, "none_duration": 0}
            if moves_allowed:
                desire.update(kind=MOVE, direction=step, claimed=int(bd.neighbour(u.cell[i], step)))
            else:
                desire["kind"] = ABSENT  # blocked: no desire for this family
        else:
            desire = {f: int(fallback[f][i]) for f in DESIRE_FIELDS}
        claimed = desire["claimed"]
        conflicting = claimed != ABSENT and (usage.claimed[claimed] or kept_cells[claimed])
        overdrawn = desire["cost"] > 0 and usage.reserved[bd.player] + kept_cost + desire["cost"] > usage.balance[bd.player]
        kept = desire["kind"] != ABSENT and not conflicting and not overdrawn
        if claimed != ABSENT:
            used[claimed] = True
            kept_cells[claimed] |= kept
        if kept:
            for f in DESIRE_FIELDS:
                decided[f][i] = desire[f]
            ranks[i] = kept_count
            kept_cost += desire["cost"]
            kept_count += 1
    # _commands
    kept = decided["kind"] != ABSENT
    filler = u.available & ~kept
    filler_rank = rank(filler, u.birth)
    commands = {
        "kind": np.where(kept, decided["kind"], np.where(filler, NONE, ABSENT)),
        "direction": np.where(kept, decided["direction"], ABSENT),
        "none_duration": np.where(kept & (decided["kind"] == NONE), decided["none_duration"],
                                  np.where(filler, wait, 0)),
        "target_cell": np.where(kept, decided["target_cell"], ABSENT),
        "produced_type": np.where(kept, decided["produced_type"], ABSENT),
        "request_order": np.where(kept, ranks, np.where(filler, kept_count + filler_rank, ABSENT)),
    }
    # _settled
    settled = Carry.__new__(Carry)
    for f in CARRY_FIELDS:
        setattr(settled, f, np.where(standing, getattr(a, f), ABSENT))
    settled.order = np.where(standing, rank(standing, a.order), ABSENT)
    settled.trained = standing & (a.trained | (executes & (kind == TRAIN)))
    settled.next_order = int(standing.sum())
    return commands, settled


def act(game, state, carry, env: int, strategy: int, trained_type: int, player: int):
    """family.act for one env: (commands of the acting player, settled carry)."""
    bd = Board(game, state, env, player)
    a = Carry(carry, env)
    u = Units(bd)
    if strategy == WORKER_RUSH:
        worker_rush(bd, a, u)
    elif strategy == BARRACKS_RUSH:
        barracks_rush(bd, a, u, trained_type)
    elif strategy == WORKER_DEFENSE:
        worker_defense(bd, a, u)
    elif strategy == BARRACKS_DEFENSE:
        barracks_defense(bd, a, u, trained_type)
    else:
        raise ValueError(f"no strategy numbered {strategy}")
    return translate(bd, a)
