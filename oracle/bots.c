/*
 * Scripted bots of the abstraction family and the learner-vs-bot seat.
 * TEST INFRASTRUCTURE ONLY (part of the CPU oracle; nanorts_oracle.c
 * includes this file so it shares the env view and the step).
 *
 * Restated here, citations relative to the reference root, N/ = src/nanorts/:
 *   N/bots/rush.py            worker_rush, barracks_rush and their helpers;
 *   N/bots/abstraction.py     put / _written, _building_site, translate with
 *                             the rush kinds {ATTACK, HARVEST, TRAIN, BUILD}
 *                             and the filler duration 10;
 *   N/bots/pathfinding.py     the A* search, as a bucket queue of LIFO
 *                             stacks (equal to the program's argmin over
 *                             f * (cells + 1) + (cells - sequence) keys);
 *   N/bots/family.py:34-41    act (WORKER_RUSH = 0, BARRACKS_RUSH = 1);
 *   N/bots/seat.py:84-149     step_seat with a static learner seat.
 *
 * The carry (AbstractActions, N/bots/abstraction.py:70-81) is nine int32
 * rows, a bool row and next_order per env.
 */

#define LAST INT32_MAX
#define AB_NO_ACTION (-1)
#define AB_ATTACK 1
#define AB_HARVEST 2
#define AB_TRAIN 3
#define AB_BUILD 4
#define AB_TRAIN_DIRECTION 6
#define TYPE_BASE 1
#define TYPE_BARRACKS 2
#define TYPE_WORKER 3
#define FILLER_DURATION 10
#define BOT_WORKER_RUSH 0
#define BOT_BARRACKS_RUSH 1

typedef struct ab_t {
    int32_t *kind, *unit_birth, *order, *target, *target_birth, *base, *base_birth, *cell, *unit_type;
    uint8_t* trained;
    int32_t* next_order;
} ab_t;

static ab_t ab_of(const nro_game* g, const nro_abstract* a, int64_t l) {
    const int64_t C = g->capacity;
    ab_t v;
    v.kind = a->kind + l * C;
    v.unit_birth = a->unit_birth + l * C;
    v.order = a->order + l * C;
    v.target = a->target + l * C;
    v.target_birth = a->target_birth + l * C;
    v.base = a->base + l * C;
    v.base_birth = a->base_birth + l * C;
    v.cell = a->cell + l * C;
    v.unit_type = a->unit_type + l * C;
    v.trained = a->trained + l * C;
    v.next_order = a->next_order + l;
    return v;
}

/* abstraction.empty_actions (N/bots/abstraction.py:118-133). */
static void ab_empty(const nro_game* g, const ab_t* a) {
    for (int32_t i = 0; i < g->capacity; ++i) {
        a->kind[i] = a->unit_birth[i] = a->order[i] = a->target[i] = a->target_birth[i] = ABSENT;
        a->base[i] = a->base_birth[i] = a->cell[i] = a->unit_type[i] = ABSENT;
        a->trained[i] = 0;
    }
    *a->next_order = 0;
}

typedef struct desire_t {
    int32_t kind, direction, target_cell, produced_type, claimed, cost, none_duration;
} desire_t;

static const desire_t NO_DESIRE = {KIND_ABSENT, ABSENT, ABSENT, ABSENT, ABSENT, 0, 0};

/* Work arrays of one act call. */
typedef struct bot_t {
    int32_t player;
    /* own_units (N/bots/abstraction.py:136-160) */
    int32_t *birth, *cell, *type, *carried, *rank;
    uint8_t *present, *available;
    /* nearest enemy / resource / own stockpile per unit (rush._closest) */
    int32_t *es, *eb, *rs, *rb, *ss, *sb;
    uint8_t *ef, *rf, *sf;
    /* candidate masks over slots */
    uint8_t *enemy, *resource, *stockpile;
    /* put's chosen / last rows and fields */
    uint8_t *chosen, *last, *mask, *mask2;
    int32_t *f_target, *f_tbirth, *f_base, *f_bbirth, *f_cell, *f_type;
    uint8_t* reserved; /* build sites, [cells] */
    /* translate */
    uint8_t *claimed, *free_cell, *used, *kept_cells, *open_cell; /* [cells] */
    int32_t reserved_cost[2];
    uint8_t *standing, *executes;
    int32_t *start, *goal, *radius, *queue, *rank_out;
    desire_t *fallback, *decided;
    /* A* scratch */
    int16_t *top, *below, *parent;
    uint8_t* seen;
} bot_t;

static void bot_init(const nro_game* g, bot_t* b) {
    const size_t C = (size_t)g->capacity, E = (size_t)g->entities, cells = (size_t)g->cells;
    int32_t** i32[] = {&b->birth, &b->cell, &b->type, &b->carried, &b->rank, &b->es, &b->eb, &b->rs, &b->rb,
                       &b->ss, &b->sb, &b->f_target, &b->f_tbirth, &b->f_base, &b->f_bbirth, &b->f_cell,
                       &b->f_type, &b->start, &b->goal, &b->radius, &b->queue, &b->rank_out};
    for (size_t k = 0; k < sizeof(i32) / sizeof(i32[0]); ++k) *i32[k] = (int32_t*)calloc(C, 4);
    uint8_t** u8c[] = {&b->present, &b->available, &b->ef, &b->rf, &b->sf, &b->chosen, &b->last,
                       &b->mask, &b->mask2, &b->standing, &b->executes};
    for (size_t k = 0; k < sizeof(u8c) / sizeof(u8c[0]); ++k) *u8c[k] = (uint8_t*)calloc(C, 1);
    b->enemy = (uint8_t*)calloc(E, 1);
    b->resource = (uint8_t*)calloc(E, 1);
    b->stockpile = (uint8_t*)calloc(E, 1);
    uint8_t** u8x[] = {&b->reserved, &b->claimed, &b->free_cell, &b->used, &b->kept_cells, &b->open_cell,
                       &b->seen};
    for (size_t k = 0; k < sizeof(u8x) / sizeof(u8x[0]); ++k) *u8x[k] = (uint8_t*)calloc(cells, 1);
    b->fallback = (desire_t*)calloc(C, sizeof(desire_t));
    b->decided = (desire_t*)calloc(C, sizeof(desire_t));
    b->top = (int16_t*)calloc(cells, 2);
    b->below = (int16_t*)calloc(cells, 2);
    b->parent = (int16_t*)calloc(cells, 2);
}

static void bot_free(bot_t* b) {
    void* all[] = {b->birth, b->cell, b->type, b->carried, b->rank, b->es, b->eb, b->rs, b->rb, b->ss, b->sb,
                   b->f_target, b->f_tbirth, b->f_base, b->f_bbirth, b->f_cell, b->f_type, b->start, b->goal,
                   b->radius, b->queue, b->rank_out, b->present, b->available, b->ef, b->rf, b->sf, b->chosen,
                   b->last, b->mask, b->mask2, b->standing, b->executes, b->enemy, b->resource, b->stockpile,
                   b->reserved, b->claimed, b->free_cell, b->used, b->kept_cells, b->open_cell, b->seen,
                   b->fallback, b->decided, b->top, b->below, b->parent};
    for (size_t k = 0; k < sizeof(all) / sizeof(all[0]); ++k) free(all[k]);
}

static inline int32_t type_col(const nro_game* g, const int32_t* col, int32_t t) {
    return col[clampi(t, 0, g->types - 1)];
}

/* own_units (N/bots/abstraction.py:136-160) and the candidate masks of
 * abstraction.enemies (:163-165) and rush.harvest_sites (N/bots/rush.py:136-153). */
static void own_units(const nro_game* g, const env_t* e, bot_t* b, int32_t player) {
    const int32_t C = g->capacity, E = g->entities, first = g->neutral + player * C;
    b->player = player;
    for (int32_t i = 0; i < C; ++i) {
        const int32_t s = first + i;
        b->birth[i] = e->birth[s];
        b->cell[i] = e->cell[s];
        b->type[i] = clampi(e->unit_type[s], 0, g->types - 1);
        b->carried[i] = e->carried[s];
        b->present[i] = b->birth[i] != ABSENT;
        b->available[i] = b->present[i] && e->pending_kind[s] == KIND_ABSENT;
    }
    for (int32_t i = 0; i < C; ++i) {
        int32_t r = 0;
        for (int32_t j = 0; j < C; ++j) r += b->present[j] && b->birth[j] < b->birth[i];
        b->rank[i] = r;
    }
    for (int32_t s = 0; s < E; ++s) {
        const int act = active(e, s);
        const int32_t owner = e->owner[s];
        const int32_t t = clampi(e->unit_type[s], 0, g->types - 1);
        b->enemy[s] = act && owner != ABSENT && owner != player;
        b->resource[s] = act && g->is_resource[t];
        b->stockpile[s] = act && g->is_stockpile[t] && owner == player;
    }
}

/* rush._closest (N/bots/rush.py:30-45): Manhattan-nearest candidate, ties by
 * the lowest birth, first slot index on equal births. */
static void closest(const nro_game* g, const env_t* e, int32_t origin, const uint8_t* cand, int32_t* slot,
                    int32_t* birth, uint8_t* found) {
    const int32_t W = g->width, E = g->entities;
    const int32_t ox = floor_mod(origin, W), oy = floor_div(origin, W);
    int32_t nearest = LAST, any = 0;
    for (int32_t j = 0; j < E; ++j) {
        if (!cand[j]) continue;
        any = 1;
        const int32_t c = e->cell[j];
        const int32_t d = abs(ox - floor_mod(c, W)) + abs(oy - floor_div(c, W));
        if (d < nearest) nearest = d;
    }
    int32_t best = 0, best_birth = LAST;
    for (int32_t j = 0; j < E; ++j) {
        if (!cand[j]) continue;
        const int32_t c = e->cell[j];
        const int32_t d = abs(ox - floor_mod(c, W)) + abs(oy - floor_div(c, W));
        if (d == nearest && e->birth[j] < best_birth) {
            best_birth = e->birth[j];
            best = j;
        }
    }
    *found = (uint8_t)any;
    *slot = any ? best : ABSENT;
    *birth = any ? e->birth[best] : ABSENT;
}

static void nearest_all(const nro_game* g, const env_t* e, const bot_t* b, const uint8_t* cand, int32_t* slot,
                        int32_t* birth, uint8_t* found) {
    for (int32_t i = 0; i < g->capacity; ++i) closest(g, e, b->cell[i], cand, &slot[i], &birth[i], &found[i]);
}

/* rush.first_in_unit_order (N/bots/rush.py:56-58): the chosen unit of least
 * birth, or -1. */
static int32_t first_in_unit_order(const nro_game* g, const bot_t* b, const uint8_t* chosen) {
    int32_t best = -1, best_birth = LAST;
    for (int32_t i = 0; i < g->capacity; ++i)
        if (chosen[i] && b->birth[i] < best_birth) {
            best_birth = b->birth[i];
            best = i;
        }
    return best;
}

static void fields_absent(const nro_game* g, bot_t* b) {
    for (int32_t i = 0; i < g->capacity; ++i)
        b->f_target[i] = b->f_tbirth[i] = b->f_base[i] = b->f_bbirth[i] = b->f_cell[i] = b->f_type[i] = ABSENT;
}

/* abstraction.put / _written (N/bots/abstraction.py:172-227): chosen units get
 * the entry; a unit without a live entry is stamped next_order + (last ?
 * C : birth rank); next_order advances by C + 1 on every call. */
static void put(const nro_game* g, bot_t* b, const ab_t* a, const uint8_t* chosen, const uint8_t* last,
                int32_t kind) {
    const int32_t C = g->capacity, n0 = *a->next_order;
    for (int32_t i = 0; i < C; ++i) {
        if (!chosen[i]) continue;
        const int known = a->kind[i] != AB_NO_ACTION && a->unit_birth[i] == b->birth[i];
        if (!known) a->order[i] = wadd(n0, (last && last[i]) ? C : b->rank[i]);
        a->kind[i] = kind;
        a->unit_birth[i] = b->birth[i];
        a->target[i] = b->f_target[i];
        a->target_birth[i] = b->f_tbirth[i];
        a->base[i] = b->f_base[i];
        a->base_birth[i] = b->f_bbirth[i];
        a->cell[i] = b->f_cell[i];
        a->unit_type[i] = b->f_type[i];
        a->trained[i] = 0;
    }
    *a->next_order = wadd(n0, C + 1);
}

static inline int is_entry(const ab_t* a, const bot_t* b, int32_t i, int32_t kind) {
    return a->kind[i] == kind && a->unit_birth[i] == b->birth[i];
}

/* abstraction._building_site (N/bots/abstraction.py:247-283): the open cell
 * first in the ring walk around `desired` (ring by Chebyshev distance; in a
 * ring the top side left to right, the right side downward, the bottom side
 * left to right, the left side downward). */
static int32_t building_site(const nro_game* g, const env_t* e, int32_t desired, const uint8_t* reserved) {
    const int32_t W = g->width, H = g->height, longest = W > H ? W : H;
    const int32_t x0 = floor_mod(desired, W), y0 = floor_div(desired, W);
    int32_t best = LAST, site = ABSENT;
    for (int32_t c = 0; c < g->cells; ++c) {
        const int32_t dx = c % W - x0, dy = c / W - y0;
        const int32_t ring = abs(dx) > abs(dy) ? abs(dx) : abs(dy);
        if (ring == 0) continue;
        const int32_t side = dy == -ring ? 0 : dx == ring ? 1 : dy == ring ? 2 : 3;
        const int32_t along = ((side == 0 || side == 2) ? dx : dy) + ring;
        const int32_t visit = (ring * 4 + side) * (2 * longest + 1) + along;
        const int open = !g->terrain[c] && e->entity_at[c] == ABSENT && !reserved[c];
        if (open && visit < best) {
            best = visit;
            site = c;
        }
    }
    return site;
}

/* abstraction.build_if_not_already_building (N/bots/abstraction.py:286-297)
 * for a one-unit builder (or none). */
static void build_unless_building(const nro_game* g, const env_t* e, bot_t* b, const ab_t* a, int32_t builder,
                                  int32_t unit_type, uint8_t* reserved) {
    const int32_t C = g->capacity;
    int any = 0;
    for (int32_t i = 0; i < C; ++i) {
        const int building = is_entry(a, b, i, AB_BUILD) && a->unit_type[i] == unit_type;
        b->chosen[i] = i == builder && !building;
        any |= b->chosen[i];
    }
    const int32_t site = any ? building_site(g, e, b->cell[builder], reserved) : ABSENT;
    fields_absent(g, b);
    for (int32_t i = 0; i < C; ++i) {
        b->f_cell[i] = site;
        b->f_type[i] = unit_type;
    }
    put(g, b, a, b->chosen, NULL, AB_BUILD);
    if (any && site >= 0 && site < g->cells) reserved[site] = 1;
}

/* rush.build_base (N/bots/rush.py:88-104); returns the builder or -1 and
 * leaves the reserved site in b->reserved. */
static int32_t build_base(const nro_game* g, const env_t* e, bot_t* b, const ab_t* a, const uint8_t* workers) {
    const int32_t C = g->capacity;
    int any_base = 0;
    for (int32_t i = 0; i < C; ++i) any_base |= b->present[i] && b->type[i] == TYPE_BASE;
    const int builds = !any_base && e->resources[b->player] >= g->cost[TYPE_BASE];
    const int32_t builder = builds ? first_in_unit_order(g, b, workers) : -1;
    memset(b->reserved, 0, (size_t)g->cells);
    build_unless_building(g, e, b, a, builder, TYPE_BASE, b->reserved);
    return builder;
}

/* rush._harvest (N/bots/rush.py:156-181); `idle` receives harvesters &
 * ~occupied. */
static void harvest(const nro_game* g, const env_t* e, bot_t* b, const ab_t* a, const uint8_t* harvesters,
                    uint8_t* idle) {
    const int32_t C = g->capacity;
    fields_absent(g, b);
    for (int32_t i = 0; i < C; ++i) {
        int32_t rs = ABSENT, rb = ABSENT, ss = ABSENT, sb = ABSENT;
        uint8_t rf = 0, sf = 0;
        if (harvesters[i]) {
            closest(g, e, b->cell[i], b->resource, &rs, &rb, &rf);
            closest(g, e, b->cell[i], b->stockpile, &ss, &sb, &sf);
        }
        const int carrying = b->carried[i] > 0;
        const int harvesting = is_entry(a, b, i, AB_HARVEST);
        const int same_base = a->base[i] == ss && a->base_birth[i] == sb;
        const int same_target = a->target[i] == rs && a->target_birth[i] == rb;
        const int occupied = carrying ? sf : (sf && rf);
        const int unchanged = harvesting && same_base && (carrying || same_target);
        b->chosen[i] = harvesters[i] && occupied && !unchanged;
        idle[i] = harvesters[i] && !occupied;
        b->f_target[i] = carrying ? ABSENT : rs;
        b->f_tbirth[i] = carrying ? ABSENT : rb;
        b->f_base[i] = ss;
        b->f_bbirth[i] = sb;
    }
    put(g, b, a, b->chosen, NULL, AB_HARVEST);
}

/* rush._attack_nearest (N/bots/rush.py:61-70). */
static void attack_nearest(const nro_game* g, bot_t* b, const ab_t* a, const uint8_t* attackers,
                           const uint8_t* last) {
    fields_absent(g, b);
    for (int32_t i = 0; i < g->capacity; ++i) {
        b->chosen[i] = attackers[i] && b->ef[i];
        b->f_target[i] = b->es[i];
        b->f_tbirth[i] = b->eb[i];
    }
    put(g, b, a, b->chosen, last, AB_ATTACK);
}

/* rush._melee_units_attack + available_melee (N/bots/rush.py:73-85). */
static void melee_attack(const nro_game* g, bot_t* b, const ab_t* a) {
    for (int32_t i = 0; i < g->capacity; ++i) {
        const int32_t t = b->type[i];
        b->mask[i] = b->present[i] && g->can_attack[t] && !g->can_harvest[t] && b->available[i];
    }
    attack_nearest(g, b, a, b->mask, NULL);
}

static void train(const nro_game* g, bot_t* b, const ab_t* a, int32_t unit_type) {
    fields_absent(g, b);
    for (int32_t i = 0; i < g->capacity; ++i) b->f_type[i] = unit_type;
    put(g, b, a, b->chosen, NULL, AB_TRAIN);
}

/* rush.worker_rush (N/bots/rush.py:213-220) with _rushing_workers (:204-210). */
static void worker_rush(const nro_game* g, const env_t* e, bot_t* b, const ab_t* a) {
    const int32_t C = g->capacity, res = e->resources[b->player];
    nearest_all(g, e, b, b->enemy, b->es, b->eb, b->ef);
    for (int32_t i = 0; i < C; ++i)
        b->chosen[i] = b->present[i] && b->type[i] == TYPE_BASE && b->available[i] && res >= g->cost[TYPE_WORKER];
    train(g, b, a, TYPE_WORKER);
    melee_attack(g, b, a);
    uint8_t* workers = b->mask;
    for (int32_t i = 0; i < C; ++i) workers[i] = b->present[i] && g->can_harvest[b->type[i]];
    const int32_t builder = build_base(g, e, b, a, workers);
    for (int32_t i = 0; i < C; ++i) b->mask2[i] = workers[i] && i != builder;
    const int32_t harvester = first_in_unit_order(g, b, b->mask2);
    for (int32_t i = 0; i < C; ++i) b->mask2[i] = i == harvester;
    harvest(g, e, b, a, b->mask2, b->last); /* b->last = idle harvester */
    for (int32_t i = 0; i < C; ++i) b->mask2[i] = (workers[i] && i != builder && i != harvester) || b->last[i];
    attack_nearest(g, b, a, b->mask2, b->last);
}

/* rush.barracks_rush (N/bots/rush.py:229-236) with train_at_base_and_barracks
 * (:107-133), build_base_and_barracks (:184-201) and _workers_behavior
 * (:223-226). */
static void barracks_rush(const nro_game* g, const env_t* e, bot_t* b, const ab_t* a, int32_t trained_type) {
    const int32_t C = g->capacity, res = e->resources[b->player];
    nearest_all(g, e, b, b->enemy, b->es, b->eb, b->ef);
    int32_t workers_held = 0;
    for (int32_t i = 0; i < C; ++i) workers_held += b->present[i] && b->type[i] == TYPE_WORKER;
    for (int32_t i = 0; i < C; ++i)
        b->chosen[i] = b->present[i] && b->type[i] == TYPE_BASE && b->available[i] && workers_held < 1 &&
                       res >= g->cost[TYPE_WORKER];
    train(g, b, a, TYPE_WORKER);
    const int32_t trained_cost = type_col(g, g->cost, trained_type);
    for (int32_t i = 0; i < C; ++i)
        b->chosen[i] = b->present[i] && b->type[i] == TYPE_BARRACKS && b->available[i] && res >= trained_cost;
    train(g, b, a, trained_type);
    melee_attack(g, b, a);
    uint8_t* workers = b->mask;
    int any_barracks = 0;
    for (int32_t i = 0; i < C; ++i) {
        workers[i] = b->present[i] && g->can_harvest[b->type[i]];
        any_barracks |= b->present[i] && b->type[i] == TYPE_BARRACKS;
    }
    const int32_t base_builder = build_base(g, e, b, a, workers);
    const int32_t used = base_builder >= 0 ? g->cost[TYPE_BASE] : 0;
    const int builds_barracks = !any_barracks && res >= wadd(g->cost[TYPE_BARRACKS], used);
    for (int32_t i = 0; i < C; ++i) b->mask2[i] = workers[i] && i != base_builder;
    const int32_t barracks_builder = builds_barracks ? first_in_unit_order(g, b, b->mask2) : -1;
    build_unless_building(g, e, b, a, barracks_builder, TYPE_BARRACKS, b->reserved);
    for (int32_t i = 0; i < C; ++i) b->mask2[i] = workers[i] && i != base_builder && i != barracks_builder;
    harvest(g, e, b, a, b->mask2, b->last); /* b->last = idle */
    for (int32_t i = 0; i < C; ++i) b->mask2[i] = b->last[i];
    attack_nearest(g, b, a, b->mask2, NULL);
}

/* ------------------------------------------------------------------------ */
/* pathfinding.search (N/bots/pathfinding.py:72-91, 152-245).               */
/* Open cells are popped by least f = g + Manhattan(cell, target), the most  */
/* recently inserted first among equal f; neighbours are inserted up, right, */
/* down, left; a cell is inserted at most once; the search ends at the first */
/* popped cell within `range` (squared Euclidean) of the target.  f grows by */
/* 0 or 2 per step, so stacks indexed by (f - f_start) / 2 hold the open     */
/* list.  out = {found, first step direction or -1, distance, pops}.         */
/* ------------------------------------------------------------------------ */
static int32_t astar(bot_t* b, const uint8_t* open_cell, int32_t W, int32_t H, int32_t start, int32_t target,
                     int32_t range, int32_t out[4]) {
    const int32_t cells = W * H;
    out[0] = 0;
    out[1] = ABSENT;
    out[2] = ABSENT;
    out[3] = 0;
    if (start < 0 || start >= cells) return ABSENT;
    enum { UNSEEN = 0, BLOCKED = 1, SEEN = 2 };
    for (int32_t c = 0; c < cells; ++c) {
        b->top[c] = -1;
        b->seen[c] = open_cell[c] ? UNSEEN : BLOCKED;
    }
    const int32_t tx = floor_mod(target, W), ty = floor_div(target, W);
    const int32_t r2 = (int32_t)((uint32_t)range * (uint32_t)range);
#define NRO_PUSH(stack, c, from)           \
    do {                                   \
        b->seen[c] = SEEN;                 \
        b->parent[c] = (int16_t)(from);    \
        b->below[c] = b->top[stack];       \
        b->top[stack] = (int16_t)(c);      \
    } while (0)
    NRO_PUSH(0, start, start);
    int32_t lowest = 0, open = 1, pops = 0;
    while (open > 0) {
        ++pops;
        while (b->top[lowest] == -1) ++lowest;
        const int32_t pos = b->top[lowest];
        b->top[lowest] = b->below[pos];
        --open;
        const int32_t y = pos / W, x = pos - y * W;
        const int32_t dx = x - tx, dy = y - ty;
        if (dx * dx + dy * dy <= r2) {
            int32_t at = pos, above = b->parent[pos], last = pos, distance = 0;
            while (above != at) {
                last = at;
                at = above;
                above = b->parent[at];
                ++distance;
            }
            int32_t step = ABSENT;
            if (last == at + W) step = 2;
            else if (last == at - 1) step = 3;
            else if (last == at - W) step = 0;
            else if (last == at + 1) step = 1;
            out[0] = 1;
            out[1] = step;
            out[2] = distance;
            out[3] = pops;
            return step;
        }
        const int32_t h = abs(dx) + abs(dy);
        for (int32_t d = 0; d < 4; ++d) {
            const int32_t nx = x + DIRECTION_DX[d], ny = y + DIRECTION_DY[d];
            if (nx < 0 || nx >= W || ny < 0 || ny >= H) continue;
            const int32_t nb = ny * W + nx;
            if (b->seen[nb] != UNSEEN) continue;
            const int32_t hn = abs(nx - tx) + abs(ny - ty);
            NRO_PUSH(lowest + (1 + hn - h) / 2, nb, pos);
            ++open;
        }
    }
#undef NRO_PUSH
    out[3] = pops;
    return ABSENT;
}

/* ------------------------------------------------------------------------ */
/* abstraction.translate with the rush kinds (N/bots/abstraction.py:300-319, */
/* 360-396 _standing, 399-407 _adjacent_direction, 440-462 _production,     */
/* 465-489 _training_direction, 552-572 _reach, 575-650 _fallback, 653-715   */
/* _plan, 787-800 _kept, 804-952 _execute_in_order / _walked, 1063-1096     */
/* _commands, 1099-1119 _settled).                                          */
/* ------------------------------------------------------------------------ */
static inline int32_t sq_distance(const nro_game* g, int32_t a, int32_t c) {
    const int32_t W = g->width;
    const int32_t dx = floor_mod(a, W) - floor_mod(c, W), dy = floor_div(a, W) - floor_div(c, W);
    return wadd(wmul(dx, dx), wmul(dy, dy));
}

static inline int32_t neighbour_cell(const nro_game* g, int32_t cell, int32_t direction) {
    const int32_t d = clampi(direction, 0, 3);
    return wadd(cell, DIRECTION_DY[d] * g->width + DIRECTION_DX[d]);
}

static int32_t adjacent_direction(const nro_game* g, int32_t origin, int32_t goal) {
    if (goal == ABSENT) return ABSENT;
    const int32_t W = g->width;
    const int32_t dx = floor_mod(goal, W) - floor_mod(origin, W), dy = floor_div(goal, W) - floor_div(origin, W);
    for (int32_t d = 0; d < 4; ++d)
        if (dx == DIRECTION_DX[d] && dy == DIRECTION_DY[d]) return d;
    return ABSENT;
}

static int within_balance(const bot_t* b, const env_t* e, int32_t p) {
    return b->reserved_cost[p] == 0 || b->reserved_cost[p] <= e->resources[p];
}

static desire_t production(const nro_game* g, const env_t* e, const bot_t* b, int32_t direction,
                           int32_t produced_type, int32_t cell) {
    const int32_t own = b->player;
    const int32_t claimed = direction != ABSENT ? neighbour_cell(g, cell, direction) : ABSENT;
    const int32_t cost = type_col(g, g->cost, produced_type);
    const int32_t reserved = b->reserved_cost[own];
    const int allowed = direction != ABSENT && !b->claimed[clampi(claimed, 0, g->cells - 1)] &&
                        (reserved == 0 || wadd(cost, reserved) <= e->resources[own]) &&
                        within_balance(b, e, 1 - own);
    if (!allowed) return NO_DESIRE;
    desire_t d = {KIND_PRODUCE, direction, ABSENT, produced_type, claimed, cost, 0};
    return d;
}

static int32_t training_direction(const nro_game* g, const env_t* e, const bot_t* b, const ab_t* a, int32_t i) {
    const int32_t W = g->width, H = g->height, E = g->entities;
    const int32_t cx = floor_mod(b->cell[i], W), cy = floor_div(b->cell[i], W);
    const int harvests = type_col(g, g->can_harvest, a->unit_type[i]) != 0;
    const uint8_t* near = harvests ? b->resource : b->enemy;
    int any_near = 0;
    for (int32_t j = 0; j < E; ++j) any_near |= near[j];
    int32_t best = ABSENT, best_score = 0;
    for (int32_t d = 0; d < 4; ++d) {
        const int32_t x = cx + DIRECTION_DX[d], y = cy + DIRECTION_DY[d];
        const int on_board = x >= 0 && x < W && y >= 0 && y < H;
        if (!on_board || !b->free_cell[y * W + x]) continue;
        int32_t nearest = LAST;
        for (int32_t j = 0; j < E; ++j) {
            if (!near[j]) continue;
            const int32_t c = e->cell[j];
            const int32_t dist = abs(x - floor_mod(c, W)) + abs(y - floor_div(c, W));
            if (dist < nearest) nearest = dist;
        }
        const int32_t score = any_near ? -nearest : 0;
        if (best == ABSENT || score > best_score) {
            best = d;
            best_score = score;
        }
    }
    return best;
}

static inline int exists(const env_t* e, int32_t E, int32_t slot, int32_t birth) {
    return slot != ABSENT && e->birth[clampi(slot, 0, E - 1)] == birth;
}

static inline int32_t cell_of(const env_t* e, int32_t E, int32_t slot) {
    return slot != ABSENT ? e->cell[clampi(slot, 0, E - 1)] : ABSENT;
}

static void translate(const nro_game* g, const env_t* e, bot_t* b, const ab_t* a, cmd_t* cmds) {
    const int32_t C = g->capacity, E = g->entities, N = g->neutral, cells = g->cells, own = b->player;
    own_units(g, e, b, own);
    /* _pending_usage (:331-359) */
    memset(b->claimed, 0, (size_t)cells);
    b->reserved_cost[0] = b->reserved_cost[1] = 0;
    for (int32_t s = 0; s < E; ++s) {
        if (!active(e, s)) continue;
        const int32_t kind = e->pending_kind[s];
        if (kind == KIND_MOVE || kind == KIND_PRODUCE) {
            int32_t t = neighbour_cell(g, e->cell[s], e->pending_direction[s]);
            if (t < 0) t += cells;
            if (t >= 0 && t < cells) b->claimed[t] = 1;
        }
        if (kind == KIND_PRODUCE && s >= N)
            b->reserved_cost[(s - N) / C] =
                wadd(b->reserved_cost[(s - N) / C], type_col(g, g->cost, e->pending_produced_type[s]));
    }
    for (int32_t c = 0; c < cells; ++c) b->free_cell[c] = !g->terrain[c] && e->entity_at[c] == ABSENT && !b->claimed[c];
    /* _standing */
    for (int32_t i = 0; i < C; ++i) {
        const int32_t kind = a->kind[i];
        const int alive = kind != AB_NO_ACTION && a->unit_birth[i] == b->birth[i];
        const int carrying = b->carried[i] > 0;
        const int built_on = a->cell[i] != ABSENT && e->entity_at[clampi(a->cell[i], 0, cells - 1)] != ABSENT;
        const int target_gone = !exists(e, E, a->target[i], a->target_birth[i]);
        int completed = 0;
        if (kind == AB_ATTACK) completed = target_gone;
        else if (kind == AB_HARVEST) completed = carrying ? !exists(e, E, a->base[i], a->base_birth[i]) : target_gone;
        else if (kind == AB_TRAIN) completed = a->trained[i] != 0;
        else if (kind == AB_BUILD) completed = built_on;
        b->standing[i] = alive && !completed;
        b->executes[i] = b->standing[i] && b->available[i];
    }
    /* _plan for the executing units */
    for (int32_t i = 0; i < C; ++i) {
        if (!b->executes[i]) continue;
        const int32_t kind = a->kind[i], cell = b->cell[i];
        const int32_t target_cell = cell_of(e, E, a->target[i]);
        const int32_t range = g->attack_range[b->type[i]];
        const int in_range = sq_distance(g, cell, target_cell) <= wmul(range, range);
        const int32_t harvest_goal = b->carried[i] > 0 ? cell_of(e, E, a->base[i]) : target_cell;
        int32_t goal = ABSENT, radius = 0;
        desire_t fb = NO_DESIRE;
        if (kind == AB_ATTACK) {
            goal = target_cell;
            radius = range;
            if (in_range && target_cell != ABSENT) {
                desire_t d = {KIND_ATTACK, ABSENT, target_cell, ABSENT, ABSENT, 0, 0};
                fb = d;
            }
        } else if (kind == AB_HARVEST) {
            goal = harvest_goal;
            radius = 1;
            const int32_t dir = adjacent_direction(g, cell, harvest_goal);
            if (dir != ABSENT) {
                desire_t d = {b->carried[i] > 0 ? KIND_RETURN : KIND_HARVEST, dir, ABSENT, ABSENT, ABSENT, 0, 0};
                fb = d;
            }
        } else if (kind == AB_TRAIN) {
            fb = production(g, e, b, training_direction(g, e, b, a, i), a->unit_type[i], cell);
        } else if (kind == AB_BUILD) {
            goal = a->cell[i];
            radius = 1;
            fb = production(g, e, b, adjacent_direction(g, cell, a->cell[i]), a->unit_type[i], cell);
        }
        const int searches = goal != ABSENT && !(kind == AB_ATTACK && in_range);
        b->start[i] = cell;
        b->goal[i] = searches ? goal : cell;
        b->radius[i] = searches ? radius : 0;
        b->fallback[i] = fb;
    }
    /* _queue: executing units by order, ties by unit index (stable argsort) */
    int32_t queued = 0;
    for (int32_t i = 0; i < C; ++i)
        if (b->executes[i]) b->queue[queued++] = i;
    for (int32_t x = 1; x < queued; ++x) {
        const int32_t v = b->queue[x];
        int32_t y = x - 1;
        while (y >= 0 && a->order[b->queue[y]] > a->order[v]) {
            b->queue[y + 1] = b->queue[y];
            --y;
        }
        b->queue[y + 1] = v;
    }
    /* _walked */
    const int may_move = within_balance(b, e, 0) && within_balance(b, e, 1);
    memset(b->used, 0, (size_t)cells);
    memset(b->kept_cells, 0, (size_t)cells);
    int32_t spent = 0, granted = 0;
    for (int32_t i = 0; i < C; ++i) {
        b->decided[i] = NO_DESIRE;
        b->rank_out[i] = ABSENT;
    }
    for (int32_t q = 0; q < queued; ++q) {
        const int32_t i = b->queue[q];
        for (int32_t c = 0; c < cells; ++c) b->open_cell[c] = b->free_cell[c] && !b->used[c];
        int32_t path[4];
        const int32_t step = astar(b, b->open_cell, g->width, g->height, b->start[i], b->goal[i], b->radius[i], path);
        desire_t d = b->fallback[i];
        if (step != ABSENT) {
            desire_t mv = {KIND_MOVE, step, ABSENT, ABSENT, neighbour_cell(g, b->start[i], step), 0, 0};
            d = may_move ? mv : NO_DESIRE;
        }
        const int has_cell = d.claimed != ABSENT && d.claimed >= 0 && d.claimed < cells;
        const int conflicting = has_cell && (b->claimed[d.claimed] || b->kept_cells[d.claimed]);
        const int over_budget = d.cost > 0 && wadd(wadd(b->reserved_cost[own], spent), d.cost) > e->resources[own];
        const int kept = d.kind != KIND_ABSENT && !conflicting && !over_budget;
        if (has_cell) {
            b->used[d.claimed] = 1;
            if (kept) b->kept_cells[d.claimed] = 1;
        }
        if (kept) {
            spent = wadd(spent, d.cost);
            b->decided[i] = d;
            b->rank_out[i] = granted++;
        }
    }
    /* _commands */
    for (int32_t p = 0; p < 2 * C; ++p) {
        cmd_t x = {KIND_ABSENT, ABSENT, 0, ABSENT, ABSENT, ABSENT};
        cmds[p] = x;
    }
    for (int32_t i = 0; i < C; ++i) {
        const desire_t* d = &b->decided[i];
        const int kept = d->kind != KIND_ABSENT;
        const int filler = b->available[i] && !kept;
        int32_t filler_rank = 0;
        for (int32_t j = 0; j < C; ++j)
            filler_rank += b->available[j] && b->decided[j].kind == KIND_ABSENT && b->birth[j] < b->birth[i];
        cmd_t* c = &cmds[own * C + i];
        c->kind = kept ? d->kind : (filler ? KIND_NONE : KIND_ABSENT);
        c->direction = kept ? d->direction : ABSENT;
        c->none_duration = (kept && d->kind == KIND_NONE) ? d->none_duration : (filler ? FILLER_DURATION : 0);
        c->target_cell = kept ? d->target_cell : ABSENT;
        c->produced_type = kept ? d->produced_type : ABSENT;
        c->request_order = kept ? b->rank_out[i] : (filler ? wadd(granted, filler_rank) : ABSENT);
    }
    /* _settled */
    int32_t standing = 0;
    for (int32_t i = 0; i < C; ++i) {
        b->rank[i] = 0;
        for (int32_t j = 0; j < C; ++j) b->rank[i] += b->standing[j] && a->order[j] < a->order[i];
        standing += b->standing[i];
    }
    for (int32_t i = 0; i < C; ++i) {
        if (b->standing[i]) {
            a->trained[i] = a->trained[i] ||
                            (b->executes[i] && (a->kind[i] == AB_TRAIN || a->kind[i] == AB_TRAIN_DIRECTION));
            a->order[i] = b->rank[i];
        } else {
            a->kind[i] = a->unit_birth[i] = a->order[i] = a->target[i] = a->target_birth[i] = ABSENT;
            a->base[i] = a->base_birth[i] = a->cell[i] = a->unit_type[i] = ABSENT;
            a->trained[i] = 0;
        }
    }
    *a->next_order = standing;
}

/* family.act (N/bots/family.py:34-41, 71-80) for one env. */
static void bot_act_one(const nro_game* g, const env_t* e, bot_t* b, const ab_t* a, int32_t strategy,
                        int32_t trained_type, int32_t player, cmd_t* cmds) {
    own_units(g, e, b, player);
    if (strategy == BOT_WORKER_RUSH) worker_rush(g, e, b, a);
    else barracks_rush(g, e, b, a, trained_type);
    translate(g, e, b, a, cmds);
}

void nro_abstraction_act(const nro_game* g, const nro_state* s, int64_t L, int32_t strategy, int32_t trained_type,
                         const int32_t* player, nro_abstract* carry, nro_commands* out) {
    const int32_t owned = 2 * g->capacity;
    bot_t b;
    bot_init(g, &b);
    cmd_t* cmds = (cmd_t*)malloc(sizeof(cmd_t) * (size_t)owned);
    for (int64_t l = 0; l < L; ++l) {
        env_t e = env_of(g, s, l);
        ab_t a = ab_of(g, carry, l);
        bot_act_one(g, &e, &b, &a, strategy, trained_type, player[l], cmds);
        for (int32_t p = 0; p < owned; ++p) {
            const int64_t at = l * owned + p;
            out->kind[at] = cmds[p].kind;
            out->direction[at] = cmds[p].direction;
            out->none_duration[at] = cmds[p].none_duration;
            out->target_cell[at] = cmds[p].target_cell;
            out->produced_type[at] = cmds[p].produced_type;
            out->request_order[at] = cmds[p].request_order;
        }
    }
    free(cmds);
    bot_free(&b);
}

int32_t nro_astar(const uint8_t* open_cell, int32_t W, int32_t H, int32_t start, int32_t target, int32_t range,
                  int32_t out[4]) {
    bot_t b;
    memset(&b, 0, sizeof(b));
    const size_t cells = (size_t)W * (size_t)H;
    b.top = (int16_t*)calloc(cells, 2);
    b.below = (int16_t*)calloc(cells, 2);
    b.parent = (int16_t*)calloc(cells, 2);
    b.seen = (uint8_t*)calloc(cells, 1);
    const int32_t step = astar(&b, open_cell, W, H, start, target, range, out);
    free(b.top);
    free(b.below);
    free(b.parent);
    free(b.seen);
    return step;
}

/* The FFI target nanorts_astar_chain for one lane (N/bots/cuda/abstraction.cu:
 * 98-215, fed by _chain, N/bots/abstraction.py:1001-1033): the rows of the
 * queue's first `count` entries (clamped to [0, capacity]), in order, each
 * searched from its start (column 0) toward its goal (1) within its radius
 * (2) over the cells still open.  A unit that steps and may move desires the
 * step's cell at cost 0 (selector 2); one that steps but may not takes its
 * blocked desire (selector 1); one that cannot takes its fallback (0).  In a
 * drawing pass a row with draws (3) that did not move takes the direction
 * the next draw names among its options (4) instead (selector 2).  A desire
 * of kind != -1 is kept when its claim is not taken and its cost fits the
 * balance beside the reserve and the costs already kept (uint32 sums); a
 * claim on the board stops being open, and is taken when kept.  out
 * [capacity + 1][4]: per slot rank among the kept (or -1), selector,
 * direction (or -1), drew; then kept count, draws used, 0, 0. */
static int32_t chain_neighbour(int32_t cell, int32_t direction, int32_t W) {
    const int32_t offset = direction == 0 ? -W : (direction == 1 ? 1 : (direction == 2 ? W : -1));
    return (int32_t)((uint32_t)cell + (uint32_t)offset);
}

void nro_astar_chain(const uint8_t* free_cells, const uint8_t* claimed, const int32_t* rows, const int32_t* queue,
                     int32_t count, int32_t may_move, int32_t reserved, int32_t balance, const int32_t* draws,
                     int64_t draw_count, int32_t drawing, int32_t W, int32_t H, int64_t capacity, int64_t columns,
                     const int64_t fallback[3], const int64_t blocked[3], int32_t* out) {
    enum { OPEN = 1, TAKEN = 2 };
    const int32_t cells = W * H;
    uint8_t* flags = (uint8_t*)malloc((size_t)cells);
    uint8_t* open_cell = (uint8_t*)malloc((size_t)cells);
    bot_t b;
    memset(&b, 0, sizeof(b));
    b.top = (int16_t*)calloc((size_t)cells, 2);
    b.below = (int16_t*)calloc((size_t)cells, 2);
    b.parent = (int16_t*)calloc((size_t)cells, 2);
    b.seen = (uint8_t*)calloc((size_t)cells, 1);
    for (int32_t c = 0; c < cells; ++c) flags[c] = (uint8_t)((free_cells[c] ? OPEN : 0) | (claimed[c] ? TAKEN : 0));
    for (int64_t i = 0; i < capacity; ++i) {
        out[4 * i] = ABSENT;
        out[4 * i + 1] = 0;
        out[4 * i + 2] = ABSENT;
        out[4 * i + 3] = 0;
    }
    const int64_t searched = count < 0 ? 0 : (count > capacity ? capacity : (int64_t)count);
    uint32_t spent = 0;
    int32_t granted = 0, calls = 0;
    for (int64_t r = 0; r < searched; ++r) {
        const int32_t slot = queue[r];
        if (slot < 0 || slot >= capacity) continue;
        const int32_t* entry = rows + (int64_t)slot * columns;
        for (int32_t c = 0; c < cells; ++c) open_cell[c] = (flags[c] & OPEN) != 0;
        int32_t path[4];
        astar(&b, open_cell, W, H, entry[0], entry[1], entry[2], path);
        const int stepped = path[1] != ABSENT;
        int32_t selector = 0, direction = ABSENT;
        int eligible = entry[fallback[0]] != ABSENT;
        int32_t claim = entry[fallback[1]], cost = entry[fallback[2]];
        if (stepped && may_move) {
            selector = 2;
            direction = path[1];
            eligible = 1;
            claim = chain_neighbour(entry[0], direction, W);
            cost = 0;
        } else if (stepped) {
            selector = 1;
            eligible = entry[blocked[0]] != ABSENT;
            claim = entry[blocked[1]];
            cost = entry[blocked[2]];
        }
        const int drew = drawing && entry[3] != 0 && !(stepped && may_move);
        if (drew) {
            const int64_t at = calls < draw_count ? calls : draw_count - 1;
            direction = ABSENT;
            for (int32_t turn = 0; turn < 4; ++turn) {
                const int32_t d = (int32_t)(((uint32_t)draws[at] + (uint32_t)turn) & 3u);
                if ((entry[4] >> d) & 1) {
                    direction = d;
                    break;
                }
            }
            selector = 2;
            eligible = 1;
            claim = direction == ABSENT ? ABSENT : chain_neighbour(entry[0], direction, W);
            cost = 0;
            ++calls;
        }
        const int on_board = claim >= 0 && claim < cells;
        const int conflicting = on_board && (flags[claim] & TAKEN) != 0;
        const int over = cost > 0 && (int32_t)(uint32_t)((uint32_t)reserved + spent + (uint32_t)cost) > balance;
        const int kept = eligible && !conflicting && !over;
        if (on_board) flags[claim] = (uint8_t)((flags[claim] & ~OPEN) | (kept ? TAKEN : 0));
        out[4 * slot] = kept ? granted : ABSENT;
        out[4 * slot + 1] = selector;
        out[4 * slot + 2] = direction;
        out[4 * slot + 3] = drew;
        if (kept) {
            spent += (uint32_t)cost;
            ++granted;
        }
    }
    out[4 * capacity] = granted;
    out[4 * capacity + 1] = calls;
    out[4 * capacity + 2] = 0;
    out[4 * capacity + 3] = 0;
    free(flags);
    free(open_cell);
    free(b.top);
    free(b.below);
    free(b.parent);
    free(b.seen);
}

/* step_seat (N/bots/seat.py:84-149) with the learner at a static seat: the
 * bot's commands from the current state, the learner's actions decoded
 * (N/adapters/jaxmarl/env.py:78-96, every agent reading the same rows), the
 * merged commands stepped under the episode root, auto-reset, the carry back
 * to empty_actions where done. */
/* N/bots/seat.py:352-360: the "drawn" rule's learner for an episode root,
 * jax.random.randint(fold_in(root, 2**32 - 2), (), 0, 2). */
int32_t nro_episode_seat(const uint32_t episode_root[2]) {
    uint32_t k[2];
    nro_fold_in(episode_root, 0xFFFFFFFEu, k);
    return nro_randint01(k);
}

/* N/bots/seat.py:84-149: the learner of lane l is seats[l] when `seats` is
 * set (else `learner`); with `draw`, a lane whose game ended takes the seat
 * of its next episode's root (lines 121-125), otherwise it keeps its seat. */
void nro_seat_step(const nro_game* g, const nro_state* initial, nro_state* s, int64_t L, int32_t strategy,
                   int32_t trained_type, int32_t fixed, int32_t* seats, int32_t draw, nro_abstract* carry,
                   const int32_t* actions, int32_t partial, nro_env_out* out) {
    const int32_t C = g->capacity, owned = 2 * C;
    work_t w;
    work_init(g, &w);
    bot_t b;
    bot_init(g, &b);
    cmd_t* bot_cmds = (cmd_t*)malloc(sizeof(cmd_t) * (size_t)owned);
    int32_t* both = (int32_t*)malloc(sizeof(int32_t) * (size_t)owned * 7);
    for (int64_t l = 0; l < L; ++l) {
        env_t e = env_of(g, s, l);
        ab_t a = ab_of(g, carry, l);
        const int32_t learner = seats ? seats[l] : fixed;
        bot_act_one(g, &e, &b, &a, strategy, trained_type, 1 - learner, bot_cmds);
        const int32_t* rows = actions + (size_t)l * C * 7;
        memcpy(both, rows, sizeof(int32_t) * (size_t)C * 7);
        memcpy(both + (size_t)C * 7, rows, sizeof(int32_t) * (size_t)C * 7);
        decode_one(g, &e, both, w.cmds);
        for (int32_t i = 0; i < C; ++i) w.cmds[(1 - learner) * C + i] = bot_cmds[(1 - learner) * C + i];
        uint32_t root[2];
        nro_fold_in(e.root, *e.episode, root);
        events_t ev;
        float reward[2];
        int terminated, truncated;
        core_step_one(g, &e, w.cmds, root, &ev, &terminated, &truncated, reward, &w);
        const int done = terminated || truncated;
        const int32_t winner = *e.winner;
        const int overflowed = e.spawn_overflow[0] > 0 || e.spawn_overflow[1] > 0;
        if (done) {
            reset_one(g, initial, &e);
            *e.episode += 1u;
            ab_empty(g, &a);
            if (seats && draw) {
                uint32_t next[2];
                nro_fold_in(e.root, *e.episode, next);
                seats[l] = nro_episode_seat(next);
            }
        }
        if (out) {
            if (out->feature_maps) {
                const int64_t per = (int64_t)g->cells * 6;
                uint8_t* maps = out->feature_maps + (size_t)l * 2 * per;
                for (int32_t p = 0; p < 2; ++p) {
                    int32_t unused[4];
                    symbolic_one(g, &e, p, partial, maps + p * per, out->scalars ? out->scalars + l * 8 + p * 4 : unused,
                                 w.seen);
                }
            }
            if (out->reward) {
                out->reward[2 * l] = reward[0];
                out->reward[2 * l + 1] = reward[1];
            }
            if (out->done) out->done[l] = (uint8_t)done;
            if (out->terminated) out->terminated[l] = (uint8_t)terminated;
            if (out->truncated) out->truncated[l] = (uint8_t)truncated;
            if (out->winner) out->winner[l] = winner;
            if (out->spawn_overflowed) out->spawn_overflowed[l] = (uint8_t)overflowed;
        }
    }
    free(both);
    free(bot_cmds);
    bot_free(&b);
    work_free(&w);
}

void nro_empty_actions(const nro_game* g, nro_abstract* carry, int64_t L) {
    for (int64_t l = 0; l < L; ++l) {
        ab_t a = ab_of(g, carry, l);
        ab_empty(g, &a);
    }
}
