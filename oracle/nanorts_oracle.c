/*
 * CPU oracle for the NanoRTS batched game hot path.  TEST INFRASTRUCTURE ONLY:
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load it as
 * the checker; the product path never does.
 *
 * A plain-C restatement of the reference JAX program.  Citations are relative
 * to the reference repository root; N/ = src/nanorts/.
 *
 * JAX semantics restated here:
 *  - int32 arithmetic wraps (XLA integer ops are modular);
 *  - `%` and `//` on ints are floor mod / floor div (Python semantics);
 *  - a gather x[i] first wraps a negative index once (i + n) and then clamps
 *    it into [0, n-1] (JAX's default for retrieval);
 *  - residue.masked_set writes only where position == index
 *    (N/core/residue.py:24-26), so an out-of-range index is a no-op;
 *  - a store into a narrower leaf truncates (jnp.asarray(new, old.dtype)).
 *
 * How each part is pinned (tests/test_oracle.py, tests/test_rendering.py):
 * threefry by Random123 known answers and JAX's classic split vector; fold_in,
 * randint01 and the CANCEL_RANDOM draw by the reference's own
 * conflict_draw.cuh (oracle/_ref, and golden vectors from it); admission,
 * durations, completion and outcome by hand-traced cycles on the 8x8 map;
 * completions by actors that died before their turn, the admitted counts and
 * the settled durations of cancelled pendings when several conflicts meet in
 * one cycle (_settle_durations, N/core/reservations.py:169-228) by
 * hand-traced scenarios under every conflict strategy
 * (tests/test_oracle_rules.py); masks against admission by brute force over
 * every single command; visibility, symbolic and pixel observations by closed
 * forms; the state invariants over long rollouts of every case.
 */
#include "nanorts_oracle.h"

#include <limits.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#define ABSENT (-1)
#define KIND_ABSENT (-1)
#define KIND_NONE 0
#define KIND_MOVE 1
#define KIND_HARVEST 2
#define KIND_RETURN 3
#define KIND_PRODUCE 4
#define KIND_ATTACK 5
#define KINDS 6
#define DIRECTIONS 4
#define NO_CAP INT32_MAX
#define CROSS_CYCLE_STRIDE (1 << 15)
#define STRATEGY_BOTH 0
#define STRATEGY_RANDOM 1
#define STRATEGY_ALTERNATING 2

/* N/model/vocabulary.py:37-42 */
static const int32_t DIRECTION_DX[4] = {0, 1, 0, -1};
static const int32_t DIRECTION_DY[4] = {-1, 0, 1, 0};

static inline int32_t wadd(int32_t a, int32_t b) { return (int32_t)((uint32_t)a + (uint32_t)b); }
static inline int32_t wmul(int32_t a, int32_t b) { return (int32_t)((uint32_t)a * (uint32_t)b); }
static inline int32_t imin(int32_t a, int32_t b) { return a < b ? a : b; }
static inline int32_t imax(int32_t a, int32_t b) { return a > b ? a : b; }
static inline int32_t clampi(int32_t v, int32_t lo, int32_t hi) { return v < lo ? lo : (v > hi ? hi : v); }
static inline int32_t floor_div(int32_t a, int32_t b) {
    int32_t q = a / b;
    int32_t r = a % b;
    return (r != 0 && ((r < 0) != (b < 0))) ? q - 1 : q;
}
static inline int32_t floor_mod(int32_t a, int32_t b) {
    int32_t r = a % b;
    return (r != 0 && ((r < 0) != (b < 0))) ? r + b : r;
}
/* JAX retrieval index: wrap a negative index once, then clamp. */
static inline int32_t gidx(int32_t i, int32_t n) { return clampi(i < 0 ? i + n : i, 0, n - 1); }
static inline int32_t arith_shr(int32_t v, int s) { return v >> s; }

/* ------------------------------------------------------------------------ */
/* threefry2x32 (Random123 Threefry-2x32, 20 rounds) and JAX key plumbing.   */
/* JAX 0.11.1, jax_threefry_partitionable=True, as gated by                  */
/* N/core/reservations.py:309-315; restated in N/core/cuda/conflict_draw.cuh. */
/* ------------------------------------------------------------------------ */
static inline uint32_t rotl32(uint32_t x, uint32_t d) { return (x << d) | (x >> (32u - d)); }

void nro_threefry2x32(const uint32_t key[2], uint32_t x[2]) {
    static const uint32_t rot[8] = {13, 15, 26, 6, 17, 29, 16, 24};
    const uint32_t ks[3] = {key[0], key[1], key[0] ^ key[1] ^ 0x1BD11BDAu};
    uint32_t x0 = x[0] + ks[0];
    uint32_t x1 = x[1] + ks[1];
    for (int block = 0; block < 5; ++block) {
        for (int r = 0; r < 4; ++r) {
            x0 += x1;
            x1 = rotl32(x1, rot[(block & 1) * 4 + r]);
            x1 ^= x0;
        }
        x0 += ks[(block + 1) % 3];
        x1 += ks[(block + 2) % 3] + (uint32_t)(block + 1);
    }
    x[0] = x0;
    x[1] = x1;
}

/* jax.random.fold_in(key, d) = threefry(key, (0, uint32(d))). */
void nro_fold_in(const uint32_t key[2], uint32_t data, uint32_t out[2]) {
    uint32_t x[2] = {0u, data};
    nro_threefry2x32(key, x);
    out[0] = x[0];
    out[1] = x[1];
}

/* jax.random.split(key, n)[i] = threefry(key, (0, i)) in partitionable mode. */
void nro_split(const uint32_t key[2], uint32_t index, uint32_t out[2]) { nro_fold_in(key, index, out); }

/* jax.random.randint(key, (), 0, 2): k2 = split(key)[1]; bits = b0 ^ b1 of
 * threefry(k2, (0, 0)); the span-2 multiplier is 0, so the draw is bits % 2. */
int32_t nro_randint01(const uint32_t key[2]) {
    uint32_t k2[2];
    nro_split(key, 1u, k2);
    uint32_t b[2] = {0u, 0u};
    nro_threefry2x32(k2, b);
    return (int32_t)((b[0] ^ b[1]) % 2u);
}

/* N/core/reservations.py:297-306: draw = randint(fold_in(event_key, ordinal)),
 * event_key = fold_in(fold_in(fold_in(root, time), birth), 0). */
int32_t nro_conflict_draw(const uint32_t root[2], int32_t time, int32_t birth, int32_t ordinal) {
    uint32_t a[2], b[2], c[2], d[2];
    nro_fold_in(root, (uint32_t)time, a);
    nro_fold_in(a, (uint32_t)birth, b);
    nro_fold_in(b, 0u, c);
    nro_fold_in(c, (uint32_t)ordinal, d);
    return nro_randint01(d);
}

/* ------------------------------------------------------------------------ */
/* One env's view into the batched leaves.                                   */
/* ------------------------------------------------------------------------ */
typedef struct env_t {
    int32_t* birth;
    int8_t* unit_type;
    int8_t* owner;
    int16_t* cell;
    int16_t* hit_points;
    int32_t* carried;
    int8_t* pending_kind;
    int8_t* pending_direction;
    int32_t* pending_none_duration;
    int16_t* pending_target_cell;
    int8_t* pending_produced_type;
    int32_t* pending_issued_at;
    int32_t* pending_completes_at;
    int32_t* pending_order;
    int16_t* entity_at;
    int32_t* time;
    int32_t* resources;
    int32_t* next_birth;
    int32_t* next_pending_order;
    int32_t* alternating;
    uint8_t* game_over;
    int32_t* winner;
    int32_t* spawn_overflow;
    uint32_t* root;
    uint32_t* episode;
} env_t;

static env_t env_of(const nro_game* g, const nro_state* s, int64_t l) {
    const int64_t E = g->entities;
    const int64_t cells = g->cells;
    env_t e;
    e.birth = s->birth + l * E;
    e.unit_type = s->unit_type + l * E;
    e.owner = s->owner + l * E;
    e.cell = s->cell + l * E;
    e.hit_points = s->hit_points + l * E;
    e.carried = s->carried_resources + l * E;
    e.pending_kind = s->pending_kind + l * E;
    e.pending_direction = s->pending_direction + l * E;
    e.pending_none_duration = s->pending_none_duration + l * E;
    e.pending_target_cell = s->pending_target_cell + l * E;
    e.pending_produced_type = s->pending_produced_type + l * E;
    e.pending_issued_at = s->pending_issued_at + l * E;
    e.pending_completes_at = s->pending_completes_at + l * E;
    e.pending_order = s->pending_order + l * E;
    e.entity_at = s->entity_at + l * cells;
    e.time = s->time + l;
    e.resources = s->player_resources + l * 2;
    e.next_birth = s->next_birth + l;
    e.next_pending_order = s->next_pending_order + l;
    e.alternating = s->alternating_conflict_count + l;
    e.game_over = s->game_over + l;
    e.winner = s->winner + l;
    e.spawn_overflow = s->spawn_overflow + l * 2;
    e.root = s->environment_root ? s->environment_root + l * 2 : NULL;
    e.episode = s->episode_index ? s->episode_index + l : NULL;
    return e;
}

static inline int active(const env_t* e, int32_t slot) { return e->birth[slot] != ABSENT; }

/* N/core/units.py:21-31 + canonical empties of N/model/state.py:35-62. */
static void remove_slot(const env_t* e, int32_t slot) {
    e->birth[slot] = ABSENT;
    e->unit_type[slot] = (int8_t)ABSENT;
    e->owner[slot] = (int8_t)ABSENT;
    e->cell[slot] = (int16_t)ABSENT;
    e->hit_points[slot] = 0;
    e->carried[slot] = 0;
    e->pending_kind[slot] = (int8_t)KIND_ABSENT;
    e->pending_direction[slot] = (int8_t)ABSENT;
    e->pending_none_duration[slot] = 0;
    e->pending_target_cell[slot] = (int16_t)ABSENT;
    e->pending_produced_type[slot] = (int8_t)ABSENT;
    e->pending_issued_at[slot] = 0;
    e->pending_completes_at[slot] = 0;
    e->pending_order[slot] = ABSENT;
}

/* N/core/pending.py:70-76: clear the pending_* leaves to their empties. */
static void clear_pending(const env_t* e, int32_t slot) {
    e->pending_kind[slot] = (int8_t)KIND_ABSENT;
    e->pending_direction[slot] = (int8_t)ABSENT;
    e->pending_none_duration[slot] = 0;
    e->pending_target_cell[slot] = (int16_t)ABSENT;
    e->pending_produced_type[slot] = (int8_t)ABSENT;
    e->pending_issued_at[slot] = 0;
    e->pending_completes_at[slot] = 0;
    e->pending_order[slot] = ABSENT;
}

/* ------------------------------------------------------------------------ */
/* Board helpers: N/core/board.py                                            */
/* ------------------------------------------------------------------------ */
typedef struct neighbour_t {
    int free;
    int occupied;
    int32_t slot;
    int32_t unit_type;
    int32_t owner;
} neighbour_t;

/* N/core/board.py:23-56 */
static neighbour_t neighbour(const nro_game* g, const env_t* e, int32_t cell, int32_t direction) {
    const int32_t W = g->width, H = g->height, E = g->entities, T = g->types;
    const int32_t x = floor_mod(cell, W), y = floor_div(cell, W);
    const int32_t known = clampi(direction, 0, DIRECTIONS - 1);
    const int32_t nx = x + DIRECTION_DX[known], ny = y + DIRECTION_DY[known];
    const int is_direction = direction >= 0 && direction < DIRECTIONS;
    const int on_board = is_direction && nx >= 0 && nx < W && ny >= 0 && ny < H;
    const int32_t ncell = on_board ? ny * W + nx : 0;
    const int32_t occupant = e->entity_at[ncell];
    neighbour_t n;
    n.occupied = on_board && occupant != ABSENT;
    n.slot = n.occupied ? occupant : 0;
    n.free = on_board && occupant == ABSENT && !g->terrain[ncell];
    const int32_t slot = gidx(n.slot, E);
    n.unit_type = clampi(e->unit_type[slot], 0, T - 1);
    n.owner = e->owner[slot];
    return n;
}

/* N/core/board.py:59-64: no bounds check, may wrap rows. */
static inline int32_t reserved_position(const nro_game* g, int32_t cell, int32_t direction) {
    const int32_t known = clampi(direction, 0, DIRECTIONS - 1);
    return wadd(cell, DIRECTION_DX[known] + DIRECTION_DY[known] * g->width);
}

/* N/core/board.py:67-71 */
static inline int position_is_blocked(const nro_game* g, const env_t* e, int32_t position) {
    const int32_t p = gidx(position, g->cells);
    return g->terrain[p] || e->entity_at[p] != ABSENT;
}

/* ------------------------------------------------------------------------ */
/* Action kinds: N/core/kinds/<kind>.py                                         */
/* ------------------------------------------------------------------------ */

/* N/core/admission.py:310-319 with each kind's duration:
 * none.py:11-12, move.py:11-12, harvest.py:11-12, return_.py:11-12,
 * produce.py:17-18, attack.py:20-21. */
static int32_t action_duration(const nro_game* g, int32_t actor_type, int32_t kind, int32_t none_duration,
                               int32_t produced_type) {
    const int32_t T = g->types;
    const int32_t actor = clampi(actor_type, 0, T - 1);
    switch (kind) {
        case KIND_NONE: return none_duration;
        case KIND_MOVE: return g->move_time[actor];
        case KIND_HARVEST: return g->harvest_time[actor];
        case KIND_RETURN: return g->move_time[actor];
        case KIND_PRODUCE: return g->produce_time[clampi(produced_type, 0, T - 1)];
        case KIND_ATTACK: return g->attack_time[actor];
        default: return 0;
    }
}

/* N/core/kinds/produce.py:21-22 */
static inline int32_t produce_cost(const nro_game* g, int32_t produced_type) {
    return g->cost[clampi(produced_type, 0, g->types - 1)];
}

/* Request.of (N/core/kinds/action_kind.py:15-40) + each kind's is_valid:
 * none.py:15-16, move.py:15-16, harvest.py:15-21, return_.py:15-22,
 * produce.py:25-34, attack.py:33-54.  N/core/admission.py:322-329. */
static int can_execute(const nro_game* g, const env_t* e, int32_t slot, int32_t kind, int32_t direction,
                       int32_t target_cell, int32_t produced_type) {
    const int32_t T = g->types, W = g->width, cells = g->cells, E = g->entities;
    const int32_t actor = clampi(e->unit_type[slot], 0, T - 1);
    const int32_t owner = e->owner[slot];
    const int32_t carried = e->carried[slot];
    const int32_t cell = e->cell[slot];
    switch (kind) {
        case KIND_NONE: return 1;
        case KIND_MOVE: {
            neighbour_t n = neighbour(g, e, cell, direction);
            return g->can_move[actor] && n.free;
        }
        case KIND_HARVEST: {
            neighbour_t n = neighbour(g, e, cell, direction);
            return g->can_harvest[actor] && carried == 0 && n.occupied && g->is_resource[n.unit_type];
        }
        case KIND_RETURN: {
            neighbour_t n = neighbour(g, e, cell, direction);
            return g->can_harvest[actor] && carried > 0 && n.occupied && g->is_stockpile[n.unit_type] &&
                   n.owner == owner;
        }
        case KIND_PRODUCE: {
            neighbour_t n = neighbour(g, e, cell, direction);
            const int32_t balance = e->resources[clampi(owner, 0, 1)];
            const int32_t known = clampi(produced_type, 0, T - 1);
            return produced_type >= 0 && produced_type < T && g->produces[actor * NRO_MAX_TYPES + known] &&
                   balance >= produce_cost(g, produced_type) && n.free;
        }
        case KIND_ATTACK: {
            const int on_board = target_cell >= 0 && target_cell < cells;
            const int32_t target_slot = e->entity_at[on_board ? target_cell : 0];
            const int holds_unit = on_board && target_slot != ABSENT;
            const int32_t target_owner = holds_unit ? e->owner[gidx(target_slot, E)] : ABSENT;
            const int32_t range = g->attack_range[actor];
            const int32_t dx = floor_mod(target_cell, W) - floor_mod(cell, W);
            const int32_t dy = floor_div(target_cell, W) - floor_div(cell, W);
            return g->can_attack[actor] && target_owner >= 0 && target_owner != owner &&
                   wadd(wmul(dx, dx), wmul(dy, dy)) <= wmul(range, range);
        }
        default: return 0;
    }
}

static inline int claims_position(int32_t kind) { return kind == KIND_MOVE || kind == KIND_PRODUCE; }

/* _keeps: which payload a kind stores (payload= of each kind module). */
static inline int keeps_direction(int32_t kind) {
    return kind == KIND_MOVE || kind == KIND_HARVEST || kind == KIND_RETURN || kind == KIND_PRODUCE;
}

typedef struct reservation_t {
    int claims;
    int32_t position;
    int32_t cost;
    int32_t player;
} reservation_t;

/* N/core/admission.py:332-346 (_reservation). */
static reservation_t reservation(const nro_game* g, int32_t cell, int32_t owner, int32_t kind, int32_t direction,
                                 int32_t produced_type, int has_action) {
    reservation_t r;
    r.cost = (has_action && kind == KIND_PRODUCE) ? produce_cost(g, produced_type) : 0;
    r.claims = has_action && claims_position(kind);
    r.position = reserved_position(g, cell, direction);
    r.player = clampi(owner, 0, 1);
    return r;
}

/* N/core/reservations.py:122-135 */
static int reservations_conflict(const reservation_t* existing, const reservation_t* requested,
                                 const int32_t* balance) {
    const int shared = existing->claims && requested->claims && existing->position == requested->position;
    const int32_t same_player_cost = existing->player == requested->player ? existing->cost : 0;
    const int32_t claimed = wadd(same_player_cost, requested->cost);
    const int over = requested->cost != 0 && claimed > 0 && claimed > balance[requested->player];
    return shared || over;
}

/* ------------------------------------------------------------------------ */
/* Admission: N/core/admission.py                                           */
/* ------------------------------------------------------------------------ */
typedef struct events_t {
    int32_t harvest[2];
    int32_t ret[2];
    int32_t produce[2][NRO_MAX_TYPES];
    int32_t attack[2][3];
} events_t;

typedef struct sort_item_t {
    int32_t k0, k1, k2;
} sort_item_t;

static int cmp_items(const void* a, const void* b) {
    const sort_item_t* x = (const sort_item_t*)a;
    const sort_item_t* y = (const sort_item_t*)b;
    if (x->k0 != y->k0) return x->k0 < y->k0 ? -1 : 1;
    if (x->k1 != y->k1) return x->k1 < y->k1 ? -1 : 1;
    if (x->k2 != y->k2) return x->k2 < y->k2 ? -1 : 1;
    return 0;
}

static int32_t bit_length(int32_t v) {
    int32_t n = 0;
    while (v > 0) {
        ++n;
        v >>= 1;
    }
    return n;
}

typedef struct cmd_t {
    int32_t kind, direction, none_duration, target_cell, produced_type, request_order;
} cmd_t;

typedef struct retained_t {
    int32_t kind, direction, target_cell, produced_type, birth, owner, unit_type, cell, carried;
} retained_t;

/* One member's completion records (N/core/cycle.py:48-81: flags hit 1,
 * death 2, harvest 4, depleted 8, return 16, spawn 32; the columns each
 * record writes: the records of each N/core/kinds module, N/core/completion.py:68-99). */
typedef struct record_t {
    int32_t flags, actor_birth, actor_owner, actor_type;
    int32_t target_slot, target_birth, amount, balance;
    int32_t produced_type, spawn_slot, spawn_birth, spawn_cell;
    int32_t death_slot, death_birth, death_owner, death_type;
} record_t;

enum { REC_HIT = 1, REC_DEATH = 2, REC_HARVEST = 4, REC_DEPLETED = 8, REC_RETURN = 16, REC_SPAWN = 32 };

/* Per-thread buffers so one env step allocates nothing. */
typedef struct work_t {
    int32_t* scratch; /* 9 E */
    sort_item_t* items;
    int32_t* order;
    int32_t* issued_sorted;
    int32_t* ranking;
    int32_t* keys;
    uint8_t* completed;
    uint8_t* members;
    record_t* records;
    retained_t* retained;
    cmd_t* cmds;
    uint8_t* seen;
    uint8_t* rows;
    int32_t* actions;
    uint8_t* maps;
} work_t;

static void work_init(const nro_game* g, work_t* w) {
    const size_t E = (size_t)g->entities, owned = (size_t)(2 * g->capacity);
    const size_t width = (size_t)(22 + g->types + g->offsets);
    w->scratch = (int32_t*)malloc(sizeof(int32_t) * 9 * E);
    w->items = (sort_item_t*)malloc(sizeof(sort_item_t) * (owned > E ? owned : E));
    w->order = (int32_t*)malloc(sizeof(int32_t) * owned);
    w->issued_sorted = (int32_t*)malloc(sizeof(int32_t) * owned);
    w->ranking = (int32_t*)malloc(sizeof(int32_t) * E);
    w->keys = (int32_t*)malloc(sizeof(int32_t) * owned);
    w->completed = (uint8_t*)malloc(E);
    w->members = (uint8_t*)malloc(E);
    w->records = (record_t*)malloc(sizeof(record_t) * E);
    w->retained = (retained_t*)malloc(sizeof(retained_t) * E);
    w->cmds = (cmd_t*)malloc(sizeof(cmd_t) * owned);
    w->seen = (uint8_t*)malloc((size_t)g->cells);
    w->rows = (uint8_t*)malloc(owned * width);
    w->actions = (int32_t*)malloc(sizeof(int32_t) * owned * 7);
    w->maps = (uint8_t*)malloc((size_t)2 * (size_t)g->cells * 6);
}

static void work_free(work_t* w) {
    free(w->scratch);
    free(w->items);
    free(w->order);
    free(w->issued_sorted);
    free(w->ranking);
    free(w->keys);
    free(w->completed);
    free(w->members);
    free(w->records);
    free(w->retained);
    free(w->cmds);
    free(w->seen);
    free(w->rows);
    free(w->actions);
    free(w->maps);
}

/* N/core/reservations.py:69-111 (resolve) with its helpers :138-259.
 * Returns the request's kind and none duration after conflicts. */
static void resolve(const nro_game* g, const env_t* e, const uint32_t key[2], const int32_t* ranking,
                    int32_t slot, int32_t* kind, int32_t* none_duration, int32_t requested_duration,
                    const reservation_t* request, int32_t* scratch) {
    const int32_t E = g->entities;
    const int32_t time = *e->time;
    int32_t* same = scratch;          /* same_cycle_conflict in ranking order */
    int32_t* cross = scratch + E;     /* cross_cycle_conflict */
    int32_t* duration = scratch + 2 * E;
    int32_t* same_before = scratch + 3 * E;
    int32_t* cross_before = scratch + 4 * E;
    int32_t* draws = scratch + 5 * E;
    int32_t* cancels_request = scratch + 6 * E;
    int32_t* cancels_pending = scratch + 7 * E;
    int32_t* pending_duration = scratch + 8 * E;

    /* conflicts, cross_cycle, _in_pending_order (:71-77, :138-151) */
    for (int32_t i = 0; i < E; ++i) {
        const int32_t s = ranking[i];
        const int has_action = e->pending_kind[s] != KIND_ABSENT;
        const reservation_t existing = reservation(g, e->cell[s], e->owner[s], e->pending_kind[s],
                                                   e->pending_direction[s], e->pending_produced_type[s], has_action);
        const int conflicts = has_action && reservations_conflict(&existing, request, e->resources);
        const int cross_cycle = e->pending_issued_at[s] != time;
        const int32_t existing_duration = action_duration(g, e->unit_type[s], e->pending_kind[s],
                                                          e->pending_none_duration[s], e->pending_produced_type[s]);
        const int32_t packed = wadd(wadd(wmul(existing_duration, 4), (conflicts && !cross_cycle) ? 2 : 0),
                                    (conflicts && cross_cycle) ? 1 : 0);
        cross[i] = packed & 1;
        same[i] = arith_shr(packed, 1) & 1;
        duration[i] = arith_shr(packed, 2);
    }
    /* _running_conflict_counts (:154-166) */
    int32_t running = 0;
    for (int32_t i = 0; i < E; ++i) {
        running = wadd(running, wadd(same[i], wmul(cross[i], CROSS_CYCLE_STRIDE)));
        same_before[i] = floor_mod(running, CROSS_CYCLE_STRIDE) - same[i];
        cross_before[i] = (floor_div(running, CROSS_CYCLE_STRIDE) - cross[i]) > 0;
    }
    const int32_t same_total = floor_mod(running, CROSS_CYCLE_STRIDE);
    const int any_cross = running >= CROSS_CYCLE_STRIDE;

    /* _consumed_draws (:271-294): ordinals below the same-cycle total. */
    for (int32_t j = 0; j < E; ++j) draws[j] = 0;
    if (g->strategy == STRATEGY_RANDOM) {
        for (int32_t j = 0; j < same_total && j < E; ++j)
            draws[j] = nro_conflict_draw(key, time, e->birth[slot], j);
    }
    /* _cancelled_sides (:249-259) */
    for (int32_t i = 0; i < E; ++i) {
        if (g->strategy == STRATEGY_BOTH) {
            cancels_request[i] = 1;
            cancels_pending[i] = 1;
        } else if (g->strategy == STRATEGY_ALTERNATING) {
            cancels_request[i] = floor_mod(wadd(*e->alternating, same_before[i]), 2) == 0;
            cancels_pending[i] = !cancels_request[i];
        } else {
            cancels_request[i] = draws[gidx(same_before[i], E)] == 0;
            cancels_pending[i] = !cancels_request[i];
        }
    }
    /* _settle_durations (:169-192) */
    int32_t cap = NO_CAP;
    int32_t after_previous = requested_duration;
    int32_t after = requested_duration;
    for (int32_t i = 0; i < E; ++i) {
        const int32_t candidate = (same[i] && cancels_request[i]) ? duration[i] : NO_CAP;
        cap = imin(cap, candidate);
        after = imin(requested_duration, cap);
        const int32_t before = cross_before[i] ? -1 : (i == 0 ? requested_duration : after_previous);
        pending_duration[i] = imin(duration[i], before);
        after_previous = after;
    }
    const int request_cancelled = any_cross || cap != NO_CAP;
    const int32_t final_request_duration = any_cross ? -1 : after;

    /* _back_in_slot_order (:195-204) + _cancel_pending (:207-228) */
    for (int32_t i = 0; i < E; ++i) {
        if (!(same[i] && cancels_pending[i])) continue;
        const int32_t s = ranking[i];
        const int32_t d = arith_shr(wadd(wmul(pending_duration[i], 2), 1), 1);
        e->pending_kind[s] = (int8_t)KIND_NONE;
        e->pending_direction[s] = (int8_t)ABSENT;
        e->pending_none_duration[s] = d;
        e->pending_target_cell[s] = (int16_t)ABSENT;
        e->pending_produced_type[s] = (int8_t)ABSENT;
        e->pending_completes_at[s] = wadd(e->pending_issued_at[s], d);
    }
    if (g->strategy == STRATEGY_ALTERNATING) *e->alternating = wadd(*e->alternating, same_total);
    if (request_cancelled) {
        *kind = KIND_NONE;
        *none_duration = final_request_duration;
    }
}

/* N/core/admission.py:432-440 */
static int32_t owner_at(const nro_game* g, const env_t* e, int32_t cell) {
    const int32_t occupant = e->entity_at[clampi(cell, 0, g->cells - 1)];
    return occupant == ABSENT ? ABSENT : e->owner[clampi(occupant, 0, g->entities - 1)];
}

/* N/core/admission.py:242-289 (_admit_one) with :302-325, :374-429. */
static void admit_one(const nro_game* g, const env_t* e, const uint32_t key[2], const int32_t* ranking,
                      int32_t player, int32_t slot, const cmd_t* command, events_t* events, int32_t* scratch) {
    const int32_t T = g->types;
    const int issued = active(e, slot) && command->kind != KIND_ABSENT;
    const int32_t requested_duration = action_duration(g, e->unit_type[slot], command->kind, command->none_duration,
                                                       command->produced_type);
    /* _none_if_illegal */
    const int legal = can_execute(g, e, slot, command->kind, command->direction, command->target_cell,
                                  command->produced_type);
    int32_t kind = legal ? command->kind : KIND_NONE;
    int32_t none_duration = legal ? command->none_duration : requested_duration;
    /* _none_if_blocked */
    {
        const int32_t reserved = reserved_position(g, e->cell[slot], command->direction);
        const int blocked = claims_position(kind) && position_is_blocked(g, e, reserved);
        if (blocked) {
            kind = KIND_NONE;
            none_duration = requested_duration;
        }
    }
    /* _count_admitted (:406-429) */
    if (issued) {
        if (kind == KIND_HARVEST) events->harvest[player] += 1;
        if (kind == KIND_RETURN) events->ret[player] += 1;
        if (kind == KIND_PRODUCE) events->produce[player][clampi(command->produced_type, 0, T - 1)] += 1;
        if (kind == KIND_ATTACK) {
            const int32_t target_owner = owner_at(g, e, command->target_cell);
            if (target_owner + 1 >= 0 && target_owner + 1 < 3) events->attack[player][target_owner + 1] += 1;
        }
    }
    /* _resolve_conflicts with _requested_reservation */
    const reservation_t request = reservation(g, e->cell[slot], e->owner[slot], kind, command->direction,
                                              command->produced_type, issued);
    resolve(g, e, key, ranking, slot, &kind, &none_duration, requested_duration, &request, scratch);
    const int32_t duration = kind == KIND_NONE ? none_duration : requested_duration;
    /* _assign_pending_action (:374-403) */
    if (issued) {
        const int32_t held = e->pending_order[slot];
        const int appends = held == ABSENT;
        const int32_t order = held == ABSENT ? *e->next_pending_order : held;
        const int32_t time = *e->time;
        e->pending_kind[slot] = (int8_t)kind;
        e->pending_direction[slot] = (int8_t)(keeps_direction(kind) ? command->direction : ABSENT);
        e->pending_none_duration[slot] = kind == KIND_NONE ? none_duration : 0;
        e->pending_target_cell[slot] = (int16_t)(kind == KIND_ATTACK ? command->target_cell : ABSENT);
        e->pending_produced_type[slot] = (int8_t)(kind == KIND_PRODUCE ? command->produced_type : ABSENT);
        e->pending_issued_at[slot] = time;
        e->pending_completes_at[slot] = wadd(time, duration);
        e->pending_order[slot] = order;
        if (appends) *e->next_pending_order = wadd(*e->next_pending_order, 1);
    }
}

/* N/core/admission.py:181-239 (admit, _ordered_requests, _issued_player_rank_key)
 * and N/core/pending.py:28-44 (ranking). */
static void admit(const nro_game* g, const env_t* e, const cmd_t* cmds, const uint32_t key[2], events_t* events,
                  work_t* w) {
    const int32_t N = g->neutral, C = g->capacity;
    const int32_t owned = 2 * C;
    sort_item_t* items = w->items;
    int32_t* order = w->order;
    int32_t* issued_sorted = w->issued_sorted;
    int32_t* ranking = w->ranking;
    int32_t* keys = w->keys;
    const int32_t rank_bits = imax(1, bit_length(C - 1));
    int32_t issued_count = 0;
    for (int32_t p = 0; p < owned; ++p) {
        const int act = e->birth[N + p] != ABSENT;
        const int issued = act && cmds[p].kind != KIND_ABSENT;
        issued_count += issued;
        const int32_t ro = cmds[p].request_order;
        const int32_t rank = clampi(ro == ABSENT ? 0 : ro, 0, (1 << rank_bits) - 1);
        items[p].k0 = ((!issued) << (rank_bits + 1)) | ((p / C) << rank_bits) | rank;
        items[p].k1 = act ? e->birth[N + p] : INT32_MAX;
        items[p].k2 = p;
    }
    qsort(items, (size_t)owned, sizeof(sort_item_t), cmp_items);
    for (int32_t i = 0; i < owned; ++i) {
        const int32_t p = items[i].k2;
        order[i] = p;
        issued_sorted[i] = (e->birth[N + p] != ABSENT) && cmds[p].kind != KIND_ABSENT;
    }
    /* pending.ranking */
    for (int32_t p = 0; p < owned; ++p) {
        const int32_t held = e->pending_order[N + p];
        keys[p] = held == ABSENT ? INT32_MAX : held;
    }
    int32_t appended_before = 0;
    for (int32_t i = 0; i < owned; ++i) {
        const int32_t p = order[i];
        const int appends = issued_sorted[i] && e->pending_order[N + p] == ABSENT;
        if (appends) keys[p] = wadd(*e->next_pending_order, appended_before);
        appended_before += appends;
    }
    for (int32_t p = 0; p < owned; ++p) {
        items[p].k0 = keys[p];
        items[p].k1 = p;
        items[p].k2 = 0;
    }
    qsort(items, (size_t)owned, sizeof(sort_item_t), cmp_items);
    for (int32_t i = 0; i < N; ++i) ranking[i] = i;
    for (int32_t i = 0; i < owned; ++i) ranking[N + i] = N + items[i].k1;

    for (int32_t position = 0; position < issued_count; ++position) {
        const int32_t p = order[position];
        admit_one(g, e, key, ranking, p / C, N + p, &cmds[p], events, w->scratch);
    }
}

/* ------------------------------------------------------------------------ */
/* Completion: N/core/completion.py, N/core/pending.py:47-76                 */
/* ------------------------------------------------------------------------ */
/* N/core/completion.py:134-180 (_take_turn) with _member_at :158-174 and each
 * kind's _complete: move.py:19-27, harvest.py:24-45, return_.py:25-43,
 * produce.py:47-81, attack.py:78-98.  Effects are computed against the state
 * at the start of the turn and written in list order. */
static void record(record_t* rec, const retained_t* r, int32_t flag) {
    rec->flags |= flag;
    rec->actor_birth = r->birth;
    rec->actor_owner = r->owner;
    rec->actor_type = r->unit_type;
}

static void take_turn(const nro_game* g, const env_t* e, int32_t slot, const retained_t* r, record_t* rec) {
    const int32_t T = g->types, N = g->neutral, C = g->capacity, cells = g->cells, E = g->entities;
    const int32_t actor_type = clampi(r->unit_type, 0, T - 1);
    const int32_t player = clampi(r->owner, 0, 1);
    const int alive = active(e, slot) && e->birth[slot] == r->birth;
    const int32_t destination = reserved_position(g, r->cell, r->direction);
    const neighbour_t nb = neighbour(g, e, r->cell, r->direction);

    int removal = 0;
    int32_t removed_slot = 0;
    switch (r->kind) {
        case KIND_MOVE: {
            if (alive) {
                if (destination >= 0 && destination < cells) e->entity_at[destination] = (int16_t)slot;
                if (r->cell >= 0 && r->cell < cells) e->entity_at[r->cell] = (int16_t)ABSENT;
                e->cell[slot] = (int16_t)destination;
            }
            break;
        }
        case KIND_HARVEST: {
            const int harvesting = nb.occupied && g->is_resource[nb.unit_type];
            const int32_t amount = g->harvest_amount[actor_type];
            const int32_t left = wadd(e->carried[gidx(nb.slot, E)], -amount);
            if (harvesting) {
                record(rec, r, left <= 0 ? REC_HARVEST | REC_DEPLETED : REC_HARVEST);
                rec->target_slot = nb.slot;
                rec->target_birth = e->birth[nb.slot];
                rec->amount = amount;
                e->carried[nb.slot] = left;
                if (alive) e->carried[slot] = amount;
                if (left <= 0) {
                    removal = 1;
                    removed_slot = nb.slot;
                }
            }
            break;
        }
        case KIND_RETURN: {
            const int returning = nb.occupied && g->is_stockpile[nb.unit_type] && r->carried > 0;
            if (returning) {
                const int32_t balance = wadd(e->resources[player], r->carried);
                record(rec, r, REC_RETURN);
                rec->target_slot = nb.slot;
                rec->target_birth = e->birth[nb.slot];
                rec->amount = r->carried;
                rec->balance = balance;
                if (alive) e->carried[slot] = 0;
                e->resources[player] = balance;
            }
            break;
        }
        case KIND_PRODUCE: {
            const int32_t newborn_type = clampi(r->produced_type, 0, T - 1);
            const int32_t balance = wadd(e->resources[player], -produce_cost(g, r->produced_type));
            const int affordable = balance >= 0;
            /* units.lowest_free_slot (N/core/units.py:12-18) */
            const int32_t block = N + player * C;
            int32_t newborn = 0;
            int has_free = 0;
            for (int32_t s = block; s < block + C; ++s) {
                if (!active(e, s)) {
                    has_free = 1;
                    newborn = s;
                    break;
                }
            }
            const int spawns = affordable && has_free;
            const int overflows = affordable && !has_free;
            if (spawns) {
                const int32_t birth = *e->next_birth;
                record(rec, r, REC_SPAWN);
                rec->produced_type = newborn_type;
                rec->spawn_slot = newborn;
                rec->spawn_birth = birth;
                rec->spawn_cell = destination;
                rec->balance = balance;
                e->resources[player] = balance;
                if (destination >= 0 && destination < cells) e->entity_at[destination] = (int16_t)newborn;
                e->birth[newborn] = birth;
                e->unit_type[newborn] = (int8_t)newborn_type;
                e->owner[newborn] = (int8_t)player;
                e->cell[newborn] = (int16_t)destination;
                e->hit_points[newborn] = (int16_t)g->hit_points[newborn_type];
                *e->next_birth = wadd(birth, 1);
            }
            if (overflows) e->spawn_overflow[player] = wadd(e->spawn_overflow[player], 1);
            break;
        }
        case KIND_ATTACK: {
            const int32_t occupant = e->entity_at[clampi(r->target_cell, 0, cells - 1)];
            const int hit = occupant != ABSENT;
            if (hit) {
                const int32_t victim = occupant;
                const int32_t left = wadd(e->hit_points[gidx(victim, E)], -g->attack_damage[actor_type]);
                record(rec, r, REC_HIT);
                rec->target_slot = victim;
                rec->target_birth = e->birth[gidx(victim, E)];
                rec->amount = g->attack_damage[actor_type];
                e->hit_points[victim] = (int16_t)left;
                if (left <= 0) {
                    removal = 1;
                    removed_slot = victim;
                }
            }
            break;
        }
        default: break;
    }
    if (removal) {
        /* the turn-start cell of the removed slot (:143); removal leaves the
         * removed slot's row unchanged by the writes above, so reading it now
         * is reading the turn-start value. */
        const int32_t at = e->cell[gidx(removed_slot, E)];
        record(rec, r, REC_DEATH);
        rec->death_slot = removed_slot;
        rec->death_birth = e->birth[gidx(removed_slot, E)];
        rec->death_owner = e->owner[gidx(removed_slot, E)];
        rec->death_type = e->unit_type[gidx(removed_slot, E)];
        if (at >= 0 && at < cells) e->entity_at[at] = (int16_t)ABSENT;
        remove_slot(e, removed_slot);
    }
}

/* N/core/completion.py:106-117 with N/core/pending.py:47-67. */
static void complete(const nro_game* g, const env_t* e, work_t* w) {
    const int32_t N = g->neutral, C = g->capacity, E = g->entities;
    const int32_t owned = 2 * C;
    *e->time = wadd(*e->time, 1);
    const int32_t time = *e->time;
    uint8_t* completed = w->completed;
    retained_t* retained = w->retained;
    sort_item_t* items = w->items;
    for (int32_t s = 0; s < E; ++s) {
        completed[s] = e->pending_kind[s] != KIND_ABSENT && e->pending_completes_at[s] <= time;
        retained[s].kind = e->pending_kind[s];
        retained[s].direction = e->pending_direction[s];
        retained[s].target_cell = e->pending_target_cell[s];
        retained[s].produced_type = e->pending_produced_type[s];
        retained[s].birth = e->birth[s];
        retained[s].owner = e->owner[s];
        retained[s].unit_type = e->unit_type[s];
        retained[s].cell = e->cell[s];
        retained[s].carried = e->carried[s];
    }
    int32_t members = 0;
    for (int32_t p = 0; p < owned; ++p) {
        const int32_t s = N + p;
        const int acting = completed[s] && e->pending_kind[s] != KIND_NONE;
        members += acting;
        items[p].k0 = acting ? e->pending_order[s] : INT32_MAX;
        items[p].k1 = p;
        items[p].k2 = 0;
    }
    qsort(items, (size_t)owned, sizeof(sort_item_t), cmp_items);
    for (int32_t s = 0; s < E; ++s)
        if (completed[s]) clear_pending(e, s);
    for (int32_t s = 0; s < E; ++s) {
        w->members[s] = 0;
        memset(&w->records[s], 0, sizeof(record_t));
    }
    for (int32_t position = 0; position < members; ++position) {
        const int32_t s = N + items[position].k1;
        w->members[s] = 1;
        take_turn(g, e, s, &retained[s], &w->records[s]);
    }
}

/* N/core/outcome.py:11-25 */
static void decide(const nro_game* g, const env_t* e) {
    const int32_t N = g->neutral, C = g->capacity;
    int surviving[2] = {0, 0};
    for (int32_t p = 0; p < 2; ++p)
        for (int32_t i = 0; i < C; ++i)
            if (e->birth[N + p * C + i] != ABSENT) surviving[p] = 1;
    const int32_t count = surviving[0] + surviving[1];
    *e->game_over = count <= 1;
    *e->winner = count == 1 ? (surviving[0] ? 0 : 1) : ABSENT;
}

/* N/core/__init__.py:99-110 (_t1_step) + outcome.truncates/sparse_reward. */
static void core_step_one(const nro_game* g, const env_t* e, const cmd_t* cmds, const uint32_t key[2],
                          events_t* events, int* terminated, int* truncated, float reward[2], work_t* w) {
    memset(events, 0, sizeof(*events));
    admit(g, e, cmds, key, events, w);
    complete(g, e, w);
    decide(g, e);
    *terminated = *e->game_over != 0;
    *truncated = !*e->game_over && *e->time >= g->max_cycles;
    const int ended = *terminated || *truncated;
    for (int32_t p = 0; p < 2; ++p) reward[p] = ended ? (p == *e->winner ? 1.0f : -1.0f) : 0.0f;
}

void nro_core_step(const nro_game* g, nro_state* s, const nro_commands* c, const uint32_t* key, int64_t L,
                   nro_step_out* out) {
    work_t w;
    work_init(g, &w);
    const int32_t owned = 2 * g->capacity;
    cmd_t* cmds = w.cmds;
    for (int64_t l = 0; l < L; ++l) {
        env_t e = env_of(g, s, l);
        for (int32_t p = 0; p < owned; ++p) {
            const int64_t at = l * owned + p;
            cmds[p].kind = c->kind[at];
            cmds[p].direction = c->direction[at];
            cmds[p].none_duration = c->none_duration[at];
            cmds[p].target_cell = c->target_cell[at];
            cmds[p].produced_type = c->produced_type[at];
            cmds[p].request_order = c->request_order[at];
        }
        events_t ev;
        int terminated, truncated;
        float reward[2];
        core_step_one(g, &e, cmds, key + 2 * l, &ev, &terminated, &truncated, reward, &w);
        if (out) {
            const int32_t T = g->types;
            if (out->terminated) out->terminated[l] = (uint8_t)terminated;
            if (out->truncated) out->truncated[l] = (uint8_t)truncated;
            if (out->reward) {
                out->reward[2 * l] = reward[0];
                out->reward[2 * l + 1] = reward[1];
            }
            if (out->is_member && out->records_i32 && out->records_i16 && out->records_i8) {
                const int32_t E = g->entities;
                for (int32_t s2 = 0; s2 < E; ++s2) {
                    const record_t* rc = &w.records[s2];
                    const int64_t at = l * E + s2;
                    out->is_member[at] = w.members[s2];
                    int32_t* wide = out->records_i32 + at * 6;
                    int16_t* index = out->records_i16 + at * 4;
                    int8_t* narrow = out->records_i8 + at * 6;
                    wide[0] = rc->actor_birth;
                    wide[1] = rc->target_birth;
                    wide[2] = rc->amount;
                    wide[3] = rc->balance;
                    wide[4] = rc->spawn_birth;
                    wide[5] = rc->death_birth;
                    index[0] = (int16_t)rc->target_slot;
                    index[1] = (int16_t)rc->spawn_slot;
                    index[2] = (int16_t)rc->spawn_cell;
                    index[3] = (int16_t)rc->death_slot;
                    narrow[0] = (int8_t)rc->flags;
                    narrow[1] = (int8_t)rc->actor_owner;
                    narrow[2] = (int8_t)rc->actor_type;
                    narrow[3] = (int8_t)rc->produced_type;
                    narrow[4] = (int8_t)rc->death_owner;
                    narrow[5] = (int8_t)rc->death_type;
                }
            }
            for (int32_t p = 0; p < 2; ++p) {
                if (out->admitted_harvest) out->admitted_harvest[2 * l + p] = ev.harvest[p];
                if (out->admitted_return) out->admitted_return[2 * l + p] = ev.ret[p];
                if (out->admitted_produce)
                    for (int32_t t = 0; t < T; ++t) out->admitted_produce[(2 * l + p) * T + t] = ev.produce[p][t];
                if (out->admitted_attack)
                    for (int32_t o = 0; o < 3; ++o) out->admitted_attack[(2 * l + p) * 3 + o] = ev.attack[p][o];
            }
        }
    }
    work_free(&w);
}

/* ------------------------------------------------------------------------ */
/* Legality: N/core/legality.py:32-64 and each kind's _legality.            */
/* Row layout (N/adapters/factors.py:31-62): kind[6], move_dir[4],           */
/* harvest_dir[4], return_dir[4], produce_dir[4], produce_type[T], attack[O]. */
/* ------------------------------------------------------------------------ */
static inline int32_t row_width(const nro_game* g) { return 22 + g->types + g->offsets; }

static void legality_row(const nro_game* g, const env_t* e, int32_t slot, uint8_t* row) {
    const int32_t T = g->types, W = g->width, H = g->height, E = g->entities;
    const int32_t width = row_width(g);
    memset(row, 0, (size_t)width);
    if (!active(e, slot)) return;
    const int32_t actor = clampi(e->unit_type[slot], 0, T - 1);
    const int32_t owner = e->owner[slot];
    const int32_t carried = e->carried[slot];
    const int32_t cell = e->cell[slot];
    row[KIND_NONE] = 1; /* none.py:19-20 */
    for (int32_t d = 0; d < DIRECTIONS; ++d) {
        const neighbour_t n = neighbour(g, e, cell, d);
        /* move.py:15-16, 19-21 */
        if (g->can_move[actor] && n.free) row[6 + d] = 1;
        /* harvest.py:15-27 */
        if (g->can_harvest[actor] && carried == 0 && n.occupied && g->is_resource[n.unit_type]) row[10 + d] = 1;
        /* return_.py:15-31 */
        if (g->can_harvest[actor] && carried > 0 && n.occupied && g->is_stockpile[n.unit_type] && n.owner == owner)
            row[14 + d] = 1;
        /* produce.py:25-44 */
        const int32_t balance = e->resources[clampi(owner, 0, 1)];
        for (int32_t t = 0; t < T; ++t) {
            if (g->produces[actor * NRO_MAX_TYPES + t] && balance >= g->cost[t] && n.free) {
                row[18 + d] = 1;
                row[22 + t] = 1;
            }
        }
    }
    for (int32_t k = 1; k <= 4; ++k) {
        const int32_t base = 6 + (k - 1) * 4;
        for (int32_t d = 0; d < DIRECTIONS; ++d)
            if (row[base + d]) row[k] = 1;
    }
    /* attack.py:57-75 with window_targets (N/model/bucket.py:134-140) */
    int32_t window = 1;
    while (window * window < g->offsets) ++window;
    const int32_t radius = (window - 1) / 2;
    const int32_t range = g->attack_range[actor];
    const int32_t x0 = floor_mod(cell, W), y0 = floor_div(cell, W);
    for (int32_t o = 0; o < g->offsets; ++o) {
        const int32_t dx = o % window - radius, dy = o / window - radius;
        const int32_t x = x0 + dx, y = y0 + dy;
        const int on_board = x >= 0 && x < W && y >= 0 && y < H;
        int32_t target_owner = ABSENT;
        if (on_board) {
            const int32_t occupant = e->entity_at[y * W + x];
            if (occupant != ABSENT) target_owner = e->owner[gidx(occupant, E)];
        }
        if (g->can_attack[actor] && target_owner >= 0 && target_owner != owner && dx * dx + dy * dy <= range * range) {
            row[22 + T + o] = 1;
            row[KIND_ATTACK] = 1;
        }
    }
    /* produce kind bit = any produce_type (produce.py:41) */
    row[KIND_PRODUCE] = 0;
    for (int32_t t = 0; t < T; ++t)
        if (row[22 + t]) row[KIND_PRODUCE] = 1;
}

void nro_legality_rows(const nro_game* g, const nro_state* s, int64_t L, uint8_t* rows) {
    const int32_t N = g->neutral, C = g->capacity, width = row_width(g);
    for (int64_t l = 0; l < L; ++l) {
        env_t e = env_of(g, s, l);
        for (int32_t p = 0; p < 2 * C; ++p) legality_row(g, &e, N + p, rows + ((l * 2 * C) + p) * width);
    }
}

/* N/adapters/jaxmarl/actions.py:28-41: rows & available, | NONE if unavailable. */
static void avail_rows_one(const nro_game* g, const env_t* e, uint8_t* rows) {
    const int32_t N = g->neutral, C = g->capacity, width = row_width(g);
    for (int32_t p = 0; p < 2 * C; ++p) {
        uint8_t* row = rows + (size_t)p * width;
        const int32_t slot = N + p;
        const int available = active(e, slot) && e->pending_kind[slot] == KIND_ABSENT;
        if (available) {
            legality_row(g, e, slot, row);
        } else {
            memset(row, 0, (size_t)width);
            row[KIND_NONE] = 1;
        }
    }
}

void nro_avail_rows(const nro_game* g, const nro_state* s, int64_t L, uint8_t* rows) {
    const int32_t C = g->capacity, width = row_width(g);
    for (int64_t l = 0; l < L; ++l) {
        env_t e = env_of(g, s, l);
        avail_rows_one(g, &e, rows + (size_t)l * 2 * C * width);
    }
}

void nro_avail_words(const nro_game* g, const nro_state* s, int64_t L, uint32_t* words) {
    const int32_t C = g->capacity, width = row_width(g);
    uint8_t* rows = (uint8_t*)malloc((size_t)(2 * C * width));
    for (int64_t l = 0; l < L; ++l) {
        env_t e = env_of(g, s, l);
        avail_rows_one(g, &e, rows);
        for (int32_t p = 0; p < 2 * C; ++p) {
            uint32_t* w = words + ((l * 2 * C) + p) * 3;
            w[0] = w[1] = w[2] = 0;
            for (int32_t b = 0; b < width && b < 96; ++b)
                if (rows[p * width + b]) w[b / 32] |= 1u << (b % 32);
        }
    }
    free(rows);
}

/* ------------------------------------------------------------------------ */
/* Observations                                                              */
/* ------------------------------------------------------------------------ */

/* N/observations/visibility.py:56-71 (_cells_by_test) over the observer's block. */
static void visible_cells_one(const nro_game* g, const env_t* e, int32_t observer, uint8_t* out) {
    const int32_t W = g->width, H = g->height, T = g->types;
    const int32_t first = g->neutral + observer * g->capacity;
    memset(out, 0, (size_t)g->cells);
    for (int32_t s = first; s < first + g->capacity; ++s) {
        if (!active(e, s)) continue;
        const int32_t cell = e->cell[s];
        const int32_t r = g->sight_radius[gidx(e->unit_type[s], T)];
        const int32_t cx = floor_mod(cell, W), cy = floor_div(cell, W);
        for (int32_t y = 0; y < H; ++y)
            for (int32_t x = 0; x < W; ++x) {
                const int32_t dx = x - cx, dy = y - cy;
                if (dx * dx + dy * dy <= r * r) out[y * W + x] = 1;
            }
    }
}

void nro_visible_cells(const nro_game* g, const nro_state* s, int64_t L, int32_t observer, uint8_t* cells) {
    for (int64_t l = 0; l < L; ++l) {
        env_t e = env_of(g, s, l);
        visible_cells_one(g, &e, observer, cells + l * g->cells);
    }
}

/* N/observations/symbolic.py:130-180 (_byte_feature_maps, _occupant_words,
 * scalar_vector) for one observer. */
static void symbolic_one(const nro_game* g, const env_t* e, int32_t player, int32_t partial, uint8_t* maps,
                         int32_t* scalars, uint8_t* seen) {
    const int32_t cells = g->cells, E = g->entities;
    if (partial) visible_cells_one(g, e, player, seen);
    for (int32_t c = 0; c < cells; ++c) {
        const int32_t occupant = e->entity_at[c];
        uint32_t word = 0;
        if (occupant != ABSENT) {
            const int32_t s = clampi(occupant, 0, E - 1);
            const uint32_t hp = (uint32_t)(int32_t)e->hit_points[s] & 0xFFu;
            const uint32_t carried = (uint32_t)e->carried[s] & 0xFFu;
            const uint32_t type = (uint32_t)((int32_t)e->unit_type[s] + 1) & 0xFFu;
            const uint32_t kind = (uint32_t)imax(e->pending_kind[s], KIND_NONE) & 0xFu;
            const uint32_t owner = (uint32_t)((int32_t)e->owner[s] + 1) & 0x3u;
            word = hp | (carried << 8) | (type << 16) | (kind << 24) | (owner << 28);
        }
        uint32_t hp = word & 0xFFu, carried = (word >> 8) & 0xFFu, type = (word >> 16) & 0xFFu;
        uint32_t kind = (word >> 24) & 0xFu, owner = (word >> 28) & 0x3u;
        if (partial) {
            const int shown = owner == (uint32_t)(player + 1) || seen[c];
            if (!shown) hp = carried = type = kind = owner = 0;
        }
        const uint32_t relabelled = owner > 0 ? (uint32_t)(((int32_t)owner - 1 + player) % 2 + 1) : 0u;
        uint8_t* m = maps + (size_t)c * 6;
        m[0] = (uint8_t)hp;
        m[1] = (uint8_t)carried;
        m[2] = (uint8_t)relabelled;
        m[3] = (uint8_t)type;
        m[4] = (uint8_t)kind;
        m[5] = g->terrain[c] ? 1 : 0;
    }
    scalars[0] = e->resources[player];
    scalars[1] = e->resources[(player + 1) % 2];
    scalars[2] = *e->time;
    scalars[3] = *e->alternating;
}

void nro_symbolic(const nro_game* g, const nro_state* s, int64_t L, int32_t partial, uint8_t* feature_maps,
                  int32_t* scalars) {
    uint8_t* seen = (uint8_t*)malloc((size_t)g->cells);
    const int64_t per = (int64_t)g->cells * 6;
    for (int64_t l = 0; l < L; ++l) {
        env_t e = env_of(g, s, l);
        for (int32_t p = 0; p < 2; ++p)
            symbolic_one(g, &e, p, partial, feature_maps + (l * 2 + p) * per, scalars + (l * 2 + p) * 4, seen);
    }
    free(seen);
}

/* N/observations/pixels.py:71-88 (_relabel, pixels) with
 * N/observations/visibility.py:106-124 (project) and
 * N/rendering/raster.py:53-127 (draw, _banded, render) at 16 px per cell. */
static void pixels_one(const nro_game* g, const env_t* e, int32_t player, int32_t partial, const uint8_t* tiles,
                       uint8_t* image, int32_t* scalars, uint8_t* seen) {
    const int32_t W = g->width, H = g->height, E = g->entities, T = g->types;
    const int32_t P = 16;
    const int32_t occupant_states = 1 + 3 * T;
    if (partial) visible_cells_one(g, e, player, seen);
    for (int32_t c = 0; c < g->cells; ++c) {
        const int32_t occ = e->entity_at[c];
        int present = occ != ABSENT;
        const int32_t s = clampi(occ, 0, E - 1);
        if (present && partial) {
            /* project: kept = active & (owner == observer | seen[clip(cell)]) */
            const int32_t cell_of = clampi(e->cell[s], 0, g->cells - 1);
            const int kept = active(e, s) && (e->owner[s] == player || seen[cell_of]);
            present = kept;
        }
        int32_t owner = present ? e->owner[s] : ABSENT;
        if (owner >= 0) owner = (owner + player) % 2;
        const int32_t type = present ? e->unit_type[s] : ABSENT;
        const int32_t kind = present ? imax(e->pending_kind[s], KIND_NONE) : 0;
        const int32_t carried = present ? e->carried[s] : 0;
        const int32_t hp = present ? e->hit_points[s] : 0;
        const int32_t occupant = present ? 1 + (owner + 1) * T + type : 0;
        const int32_t tile = (g->terrain[c] ? 1 : 0) * occupant_states + occupant;
        const uint8_t* src = tiles + (size_t)gidx(tile, 2 * occupant_states) * P * P * 3;
        const int32_t cx = c % W, cy = c / W;
        for (int32_t py = 0; py < P; ++py)
            for (int32_t px = 0; px < P; ++px) {
                uint8_t* dst = image + (((size_t)(cy * P + py) * (size_t)(W * P)) + (size_t)(cx * P + px)) * 3;
                const int band = py >= 12 && py <= 14 && px >= 1 && px < 15;
                if (present && band) {
                    const int32_t position = clampi(px - 1, 0, 13);
                    int lit;
                    if (py == 12) lit = kind == position + 1;
                    else if (py == 13) lit = ((carried >> position) & 1) != 0;
                    else lit = hp > position;
                    dst[0] = dst[1] = dst[2] = lit ? 0xFF : 0x00;
                } else {
                    const uint8_t* t = src + ((size_t)py * P + (size_t)px) * 3;
                    dst[0] = t[0];
                    dst[1] = t[1];
                    dst[2] = t[2];
                }
            }
    }
    (void)H;
    scalars[0] = e->resources[player];
    scalars[1] = e->resources[(player + 1) % 2];
    scalars[2] = *e->time;
    scalars[3] = *e->alternating;
}

void nro_pixels(const nro_game* g, const nro_state* s, int64_t L, int32_t partial, const uint8_t* tiles,
                uint8_t* image, int32_t* scalars) {
    uint8_t* seen = (uint8_t*)malloc((size_t)g->cells);
    const size_t per = (size_t)g->cells * 256 * 3;
    for (int64_t l = 0; l < L; ++l) {
        env_t e = env_of(g, s, l);
        for (int32_t p = 0; p < 2; ++p)
            pixels_one(g, &e, p, partial, tiles, image + ((size_t)l * 2 + (size_t)p) * per,
                       scalars + (l * 2 + p) * 4, seen);
    }
    free(seen);
}

/* ------------------------------------------------------------------------ */
/* Actions: N/adapters/jaxmarl/actions.py:61-84, N/adapters/factors.py:117-151 */
/* ------------------------------------------------------------------------ */
static void decode_one(const nro_game* g, const env_t* e, const int32_t* actions, cmd_t* cmds) {
    const int32_t N = g->neutral, C = g->capacity, W = g->width, H = g->height;
    int32_t side = 1;
    while (side * side < g->offsets) ++side;
    const int32_t radius = (side - 1) / 2;
    for (int32_t p = 0; p < 2 * C; ++p) {
        const int32_t* row = actions + (size_t)p * 7;
        const int32_t slot = N + p;
        const int available = active(e, slot) && e->pending_kind[slot] == KIND_ABSENT;
        const int32_t kind = row[0];
        int32_t direction = ABSENT;
        if (kind == KIND_MOVE) direction = row[1];
        else if (kind == KIND_HARVEST) direction = row[2];
        else if (kind == KIND_RETURN) direction = row[3];
        else if (kind == KIND_PRODUCE) direction = row[4];
        const int32_t produced = kind == KIND_PRODUCE ? row[5] : ABSENT;
        const int32_t cell = e->cell[slot];
        const int32_t tx = wadd(floor_mod(cell, W), floor_mod(row[6], side) - radius);
        const int32_t ty = wadd(floor_div(cell, W), floor_div(row[6], side) - radius);
        const int on_board = tx >= 0 && tx < W && ty >= 0 && ty < H;
        cmds[p].kind = available ? kind : KIND_ABSENT;
        cmds[p].direction = available ? direction : ABSENT;
        cmds[p].none_duration = available ? (kind == KIND_NONE ? 1 : 0) : 0;
        cmds[p].target_cell = available ? ((kind == KIND_ATTACK && on_board) ? ty * W + tx : ABSENT) : ABSENT;
        cmds[p].produced_type = available ? produced : ABSENT;
        cmds[p].request_order = ABSENT;
    }
}

void nro_decode_actions(const nro_game* g, const nro_state* s, const int32_t* actions, int64_t L,
                        nro_commands* c) {
    const int32_t owned = 2 * g->capacity;
    cmd_t* cmds = (cmd_t*)malloc(sizeof(cmd_t) * (size_t)owned);
    for (int64_t l = 0; l < L; ++l) {
        env_t e = env_of(g, s, l);
        decode_one(g, &e, actions + (size_t)l * owned * 7, cmds);
        for (int32_t p = 0; p < owned; ++p) {
            const int64_t at = l * owned + p;
            c->kind[at] = cmds[p].kind;
            c->direction[at] = cmds[p].direction;
            c->none_duration[at] = cmds[p].none_duration;
            c->target_cell[at] = cmds[p].target_cell;
            c->produced_type[at] = cmds[p].produced_type;
            c->request_order[at] = cmds[p].request_order;
        }
    }
    free(cmds);
}

/* ------------------------------------------------------------------------ */
/* Synthetic harness sampler (this build's own definition, replacing the     */
/* README's float jax.random.categorical with an integer uniform draw):       */
/*   k_step = fold_in(sample_key, step), p = agent*C + row                    */
/*   (w0,w1) = threefry(k_step, (env, 2p)),                                   */
/*   (w2,w3) = threefry(k_step, (env, 2p + 1))                                */
/*   factor f draws h_f = 16-bit half f of w0..w3 (low half first);          */
/*   value = the ((h_f * popcount) >> 16)-th set bit of the factor's mask    */
/*   (multiply-shift range reduction), or 0 when the factor has no set bit   */
/*   (argmax over all -inf is 0).                                            */
/* Rows with only the NONE bit set come out as all zeros.                    */
/* ------------------------------------------------------------------------ */
static void factor_bounds(const nro_game* g, int32_t lo[7], int32_t width[7]) {
    const int32_t w[7] = {6, 4, 4, 4, 4, g->types, g->offsets};
    int32_t at = 0;
    for (int f = 0; f < 7; ++f) {
        lo[f] = at;
        width[f] = w[f];
        at += w[f];
    }
}

static void sample_positions(const nro_game* g, const uint8_t* rows, int32_t positions, const uint32_t sample_key[2],
                             int32_t step, int64_t env, int32_t* actions) {
    const int32_t width = row_width(g);
    int32_t lo[7], wid[7];
    factor_bounds(g, lo, wid);
    uint32_t kt[2];
    nro_fold_in(sample_key, (uint32_t)step, kt);
    for (int32_t p = 0; p < positions; ++p) {
        const uint8_t* row = rows + (size_t)p * width;
        int32_t* out = actions + (size_t)p * 7;
        int only_none = row[0];
        for (int32_t b = 1; b < width && only_none; ++b)
            if (row[b]) only_none = 0;
        if (only_none) {
            for (int f = 0; f < 7; ++f) out[f] = 0;
            continue;
        }
        uint32_t w01[2] = {(uint32_t)env, (uint32_t)(2 * p)}, w23[2] = {(uint32_t)env, (uint32_t)(2 * p + 1)};
        nro_threefry2x32(kt, w01);
        nro_threefry2x32(kt, w23);
        const uint32_t words[4] = {w01[0], w01[1], w23[0], w23[1]};
        for (int f = 0; f < 7; ++f) {
            const uint32_t h = (words[f / 2] >> (16 * (f % 2))) & 0xFFFFu;
            int32_t count = 0;
            for (int32_t b = 0; b < wid[f]; ++b) count += row[lo[f] + b] != 0;
            int32_t value = 0;
            if (count > 0) {
                int32_t k = (int32_t)((h * (uint32_t)count) >> 16);
                for (int32_t b = 0; b < wid[f]; ++b) {
                    if (row[lo[f] + b]) {
                        if (k == 0) {
                            value = b;
                            break;
                        }
                        --k;
                    }
                }
            }
            out[f] = value;
        }
    }
}

static void sample_env(const nro_game* g, const uint8_t* rows, const uint32_t sample_key[2], int32_t step,
                       int64_t env, int32_t* actions) {
    sample_positions(g, rows, 2 * g->capacity, sample_key, step, env, actions);
}

/* The same sampler over GridNet's per-cell rows [2][cells][78], at position
   player * cells + cell. */
void nro_gridnet_sample_actions(const nro_game* g, const uint8_t* rows, const uint32_t sample_key[2], int32_t step,
                                int64_t env0, int64_t L, int32_t* actions) {
    const int32_t n = 2 * g->cells, width = row_width(g);
    for (int64_t l = 0; l < L; ++l)
        sample_positions(g, rows + (size_t)l * n * width, n, sample_key, step, env0 + l, actions + (size_t)l * n * 7);
}

void nro_sample_actions(const nro_game* g, const uint8_t* rows, const uint32_t sample_key[2], int32_t step,
                        int64_t env0, int64_t L, int32_t* actions) {
    const int32_t C = g->capacity, width = row_width(g);
    for (int64_t l = 0; l < L; ++l)
        sample_env(g, rows + (size_t)l * 2 * C * width, sample_key, step, env0 + l, actions + (size_t)l * 2 * C * 7);
}

/* ------------------------------------------------------------------------ */
/* Lifecycle: N/adapters/lifecycle.py:53-79 (advance) and N/core/__init__.py */
/* :30-32 (reset ignores its key: every episode starts from the decided      */
/* initial state).                                                           */
/* ------------------------------------------------------------------------ */
static void copy_env(const nro_game* g, const env_t* dst, const env_t* src) {
    const size_t E = (size_t)g->entities, cells = (size_t)g->cells;
    memcpy(dst->birth, src->birth, E * 4);
    memcpy(dst->unit_type, src->unit_type, E);
    memcpy(dst->owner, src->owner, E);
    memcpy(dst->cell, src->cell, E * 2);
    memcpy(dst->hit_points, src->hit_points, E * 2);
    memcpy(dst->carried, src->carried, E * 4);
    memcpy(dst->pending_kind, src->pending_kind, E);
    memcpy(dst->pending_direction, src->pending_direction, E);
    memcpy(dst->pending_none_duration, src->pending_none_duration, E * 4);
    memcpy(dst->pending_target_cell, src->pending_target_cell, E * 2);
    memcpy(dst->pending_produced_type, src->pending_produced_type, E);
    memcpy(dst->pending_issued_at, src->pending_issued_at, E * 4);
    memcpy(dst->pending_completes_at, src->pending_completes_at, E * 4);
    memcpy(dst->pending_order, src->pending_order, E * 4);
    memcpy(dst->entity_at, src->entity_at, cells * 2);
    *dst->time = *src->time;
    dst->resources[0] = src->resources[0];
    dst->resources[1] = src->resources[1];
    *dst->next_birth = *src->next_birth;
    *dst->next_pending_order = *src->next_pending_order;
    *dst->alternating = *src->alternating;
    *dst->game_over = *src->game_over;
    *dst->winner = *src->winner;
    dst->spawn_overflow[0] = src->spawn_overflow[0];
    dst->spawn_overflow[1] = src->spawn_overflow[1];
}

static void reset_one(const nro_game* g, const nro_state* initial, const env_t* e) {
    env_t start = env_of(g, initial, 0);
    copy_env(g, e, &start);
    decide(g, e);
}

void nro_reset_where_done(const nro_game* g, const nro_state* initial, nro_state* s, const uint8_t* done,
                          int64_t L) {
    for (int64_t l = 0; l < L; ++l) {
        if (!done[l]) continue;
        env_t e = env_of(g, s, l);
        reset_one(g, initial, &e);
        if (e.episode) *e.episode += 1u;
    }
}

/* encode_components (N/adapters/rewards.py:47-71): per player win_loss,
 * resource_gather, produce_worker, produce_building, attack,
 * produce_combat_unit from the admitted counts and the ending state's
 * outcome.  Type codes are the vocabulary's (N/model/unit_types.py:9-15). */
static void reward_components(const env_t* e, const events_t* ev, float out[2][6]) {
    enum { BASE = 1, BARRACKS = 2, WORKER = 3, LIGHT = 4, HEAVY = 5, RANGED = 6 };
    for (int32_t p = 0; p < 2; ++p) {
        const int32_t opponent = (p + 1) % 2;
        out[p][0] = *e->game_over ? (*e->winner == p ? 1.0f : -1.0f) : 0.0f;
        out[p][1] = (float)(ev->harvest[p] + ev->ret[p]);
        out[p][2] = (float)ev->produce[p][WORKER];
        out[p][3] = (float)(ev->produce[p][BASE] + ev->produce[p][BARRACKS]);
        out[p][4] = (float)(ev->attack[p][opponent + 1] - ev->attack[p][p + 1]);
        out[p][5] = (float)(ev->produce[p][LIGHT] + ev->produce[p][HEAVY] + ev->produce[p][RANGED]);
    }
}

/* N/adapters/jaxmarl/env.py:72-184 for one env: request (decode, episode
 * root) -> core.step -> respond (advance + observe the post-reset state).
 * The ending state's observation (final_observation, :161-170) and the
 * reward components (:173-174) are taken before the reset. */
static void env_step_one(const nro_game* g, const nro_state* initial, const env_t* e, const int32_t* actions,
                         int32_t partial, float reward[2], int* done, int* terminated, int* truncated,
                         int32_t* winner, int* overflowed, uint8_t* maps, int32_t* scalars, uint8_t* final_maps,
                         int32_t* final_scalars, float components[2][6], work_t* w) {
    decode_one(g, e, actions, w->cmds);
    uint32_t root[2];
    nro_fold_in(e->root, *e->episode, root);
    events_t ev;
    core_step_one(g, e, w->cmds, root, &ev, terminated, truncated, reward, w);
    *done = *terminated || *truncated;
    *winner = *e->winner;
    *overflowed = e->spawn_overflow[0] > 0 || e->spawn_overflow[1] > 0;
    if (components) reward_components(e, &ev, components);
    if (final_maps) {
        const int64_t per = (int64_t)g->cells * 6;
        for (int32_t p = 0; p < 2; ++p)
            symbolic_one(g, e, p, partial, final_maps + p * per, final_scalars + p * 4, w->seen);
    }
    if (*done) {
        reset_one(g, initial, e);
        *e->episode += 1u;
    }
    if (maps) {
        const int64_t per = (int64_t)g->cells * 6;
        for (int32_t p = 0; p < 2; ++p) symbolic_one(g, e, p, partial, maps + p * per, scalars + p * 4, w->seen);
    }
}

void nro_env_step(const nro_game* g, const nro_state* initial, nro_state* s, const int32_t* actions, int64_t L,
                  int32_t partial, nro_env_out* out) {
    const int32_t owned = 2 * g->capacity;
    work_t w;
    work_init(g, &w);
    for (int64_t l = 0; l < L; ++l) {
        env_t e = env_of(g, s, l);
        float reward[2];
        int done, terminated, truncated, overflowed;
        int32_t winner;
        uint8_t* maps = out && out->feature_maps ? out->feature_maps + (size_t)l * 2 * g->cells * 6 : NULL;
        int32_t* scal = out && out->scalars ? out->scalars + l * 8 : NULL;
        uint8_t* fmaps = out && out->final_feature_maps && out->final_scalars
                             ? out->final_feature_maps + (size_t)l * 2 * g->cells * 6
                             : NULL;
        int32_t* fscal = fmaps ? out->final_scalars + l * 8 : NULL;
        float components[2][6];
        const int wants_components = out && out->reward_components;
        env_step_one(g, initial, &e, actions + (size_t)l * owned * 7, partial, reward, &done, &terminated,
                     &truncated, &winner, &overflowed, maps, scal, fmaps, fscal,
                     wants_components ? components : NULL, &w);
        if (wants_components)
            for (int32_t p = 0; p < 2; ++p)
                for (int32_t c = 0; c < 6; ++c) out->reward_components[(l * 2 + p) * 6 + c] = components[p][c];
        if (out) {
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
    work_free(&w);
}

/* ------------------------------------------------------------------------ */
/* Threaded rollout driver (the CPU baseline and the long-rollout checker).  */
/* ------------------------------------------------------------------------ */
typedef struct rollout_job {
    const nro_game* g;
    const nro_state* initial;
    nro_state* s;
    const uint32_t* sample_key;
    int32_t step0, steps, partial;
    int64_t L, begin, end, env0;
    float* rewards;
    uint8_t* dones;
    int32_t* actions;
    uint8_t* last_maps;
    int32_t* last_scalars;
} rollout_job;

static void* rollout_worker(void* arg) {
    rollout_job* job = (rollout_job*)arg;
    const nro_game* g = job->g;
    const int32_t C = g->capacity;
    const size_t maps_per = (size_t)2 * g->cells * 6;
    work_t w;
    work_init(g, &w);
    for (int64_t l = job->begin; l < job->end; ++l) {
        env_t e = env_of(g, job->s, l);
        for (int32_t t = 0; t < job->steps; ++t) {
            const int32_t step = job->step0 + t;
            float reward[2];
            int done, terminated, truncated, overflowed;
            int32_t winner;
            int32_t scalars[8];
            avail_rows_one(g, &e, w.rows);
            sample_env(g, w.rows, job->sample_key, step, job->env0 + l, w.actions);
            if (job->actions)
                memcpy(job->actions + ((size_t)t * job->L + l) * 2 * C * 7, w.actions, sizeof(int32_t) * 2 * C * 7);
            env_step_one(g, job->initial, &e, w.actions, job->partial, reward, &done, &terminated, &truncated,
                         &winner, &overflowed, w.maps, scalars, NULL, NULL, NULL, &w);
            if (job->rewards) {
                job->rewards[((size_t)t * job->L + l) * 2] = reward[0];
                job->rewards[((size_t)t * job->L + l) * 2 + 1] = reward[1];
            }
            if (job->dones) job->dones[(size_t)t * job->L + l] = (uint8_t)done;
            if (t == job->steps - 1 && job->last_maps) {
                memcpy(job->last_maps + (size_t)l * maps_per, w.maps, maps_per);
                if (job->last_scalars) memcpy(job->last_scalars + l * 8, scalars, sizeof(scalars));
            }
        }
    }
    work_free(&w);
    return NULL;
}

int32_t nro_rollout(const nro_game* g, const nro_state* initial, nro_state* s, const uint32_t sample_key[2],
                    int32_t step0, int32_t steps, int64_t L, int32_t partial, int32_t threads, float* rewards,
                    uint8_t* dones, int32_t* actions, uint8_t* last_feature_maps, int32_t* last_scalars,
                    int64_t env0) {
    if (threads < 1) threads = 1;
    if (threads > L) threads = (int32_t)(L > 0 ? L : 1);
    pthread_t* ids = (pthread_t*)malloc(sizeof(pthread_t) * (size_t)threads);
    rollout_job* jobs = (rollout_job*)malloc(sizeof(rollout_job) * (size_t)threads);
    for (int32_t t = 0; t < threads; ++t) {
        rollout_job* j = &jobs[t];
        j->g = g;
        j->initial = initial;
        j->s = s;
        j->sample_key = sample_key;
        j->step0 = step0;
        j->steps = steps;
        j->partial = partial;
        j->L = L;
        j->env0 = env0;
        j->begin = L * t / threads;
        j->end = L * (t + 1) / threads;
        j->rewards = rewards;
        j->dones = dones;
        j->actions = actions;
        j->last_maps = last_feature_maps;
        j->last_scalars = last_scalars;
    }
    for (int32_t t = 1; t < threads; ++t) pthread_create(&ids[t], NULL, rollout_worker, &jobs[t]);
    rollout_worker(&jobs[0]);
    for (int32_t t = 1; t < threads; ++t) pthread_join(ids[t], NULL);
    free(ids);
    free(jobs);
    return threads;
}

/* ------------------------------------------------------------------------ */
/* N/model/state.py:87-165 (state_invariant_violations).                     */
/* bit 0: active cell out of bounds; 1: entity_at misses an active slot;     */
/* 2: entity_at names a slot outside capacity; 3: entity_at names a slot not */
/* at that cell; 4: owner disagrees with block; 5: inactive slot not empty.  */
/* ------------------------------------------------------------------------ */
int32_t nro_state_violations(const nro_game* g, const nro_state* s, int64_t l) {
    env_t e = env_of(g, s, l);
    const int32_t E = g->entities, cells = g->cells, N = g->neutral, C = g->capacity;
    int32_t bits = 0;
    for (int32_t slot = 0; slot < E; ++slot) {
        const int act = active(&e, slot);
        const int32_t cell = e.cell[slot];
        const int in_bounds = cell >= 0 && cell < cells;
        if (act && !in_bounds) bits |= 1;
        if (act && (!in_bounds || e.entity_at[cell] != slot)) bits |= 2;
        const int32_t block_owner = slot < N ? -1 : (slot - N) / C;
        if (act && e.owner[slot] != block_owner) bits |= 16;
        if (!act) {
            if (e.unit_type[slot] != -1 || e.owner[slot] != -1 || e.cell[slot] != -1 || e.hit_points[slot] != 0 ||
                e.carried[slot] != 0 || e.pending_kind[slot] != -1 || e.pending_direction[slot] != -1 ||
                e.pending_none_duration[slot] != 0 || e.pending_target_cell[slot] != -1 ||
                e.pending_produced_type[slot] != -1 || e.pending_issued_at[slot] != 0 ||
                e.pending_completes_at[slot] != 0 || e.pending_order[slot] != -1)
                bits |= 32;
        }
    }
    for (int32_t c = 0; c < cells; ++c) {
        const int32_t occ = e.entity_at[c];
        if (occ == ABSENT) continue;
        if (occ < 0 || occ >= E) {
            bits |= 4;
            continue;
        }
        if (!active(&e, occ) || e.cell[occ] != c) bits |= 8;
    }
    return bits;
}

/* ------------------------------------------------------------------------ */
/* Scripted bots and the learner-vs-bot seat (bots.c shares the env view).   */
/* ------------------------------------------------------------------------ */
#include "bots.c"

/* ------------------------------------------------------------------------ */
/* GridNet action decode (gridnet.c shares the env view and legality rows).  */
/* ------------------------------------------------------------------------ */
#include "gridnet.c"
