/*
 * CPU oracle for the NanoRTS batched game hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This is a plain-C restatement of the reference
 * JAX program (src/nanorts/core, src/nanorts/adapters, src/nanorts/observations
 * of Doguhan58/NanoRTS).  It exists to check the HIP kernels and to time a CPU
 * baseline.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * may load it, and only as the checker.  The product path never calls it.
 *
 * Every function cites the reference file:line it restates.  Layouts mirror the
 * reference pytree leaves (src/nanorts/model/state.py:33-84) with a leading env
 * dimension L, exactly as jax.vmap lays them out.
 */
#ifndef NANORTS_ORACLE_H
#define NANORTS_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NRO_MAX_TYPES 8

/* Static game description (BucketSpec + GameConfig unit columns).
 * src/nanorts/model/bucket.py:24-58, src/nanorts/model/config.py:44-69. */
typedef struct nro_game {
    int32_t height, width, cells;
    int32_t neutral, capacity, entities; /* N, C, E = N + 2C */
    int32_t types;                       /* T */
    int32_t offsets;                     /* attack window cells, (2R+1)^2 */
    int32_t strategy;                    /* 0 CANCEL_BOTH, 1 CANCEL_RANDOM, 2 CANCEL_ALTERNATING */
    int32_t max_cycles;
    int32_t cost[NRO_MAX_TYPES];
    int32_t hit_points[NRO_MAX_TYPES];
    int32_t produce_time[NRO_MAX_TYPES];
    int32_t move_time[NRO_MAX_TYPES];
    int32_t attack_time[NRO_MAX_TYPES];
    int32_t harvest_time[NRO_MAX_TYPES];
    int32_t attack_range[NRO_MAX_TYPES];
    int32_t attack_damage[NRO_MAX_TYPES];
    int32_t harvest_amount[NRO_MAX_TYPES];
    int32_t sight_radius[NRO_MAX_TYPES];
    int32_t is_resource[NRO_MAX_TYPES];
    int32_t is_stockpile[NRO_MAX_TYPES];
    int32_t can_harvest[NRO_MAX_TYPES];
    int32_t can_move[NRO_MAX_TYPES];
    int32_t can_attack[NRO_MAX_TYPES];
    int32_t produces[NRO_MAX_TYPES * NRO_MAX_TYPES]; /* [producer * 8 + produced] */
    const uint8_t* terrain;                           /* bool[cells] */
} nro_game;

/* Batched state: every leaf has a leading env dim.  Per-slot leaves [L][E],
 * entity_at [L][cells], scalars [L], per-player [L][2].
 * src/nanorts/model/state.py:33-84, src/nanorts/adapters/lifecycle.py:24-31. */
typedef struct nro_state {
    int32_t* birth;
    int8_t* unit_type;
    int8_t* owner;
    int16_t* cell;
    int16_t* hit_points;
    int32_t* carried_resources;
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
    int32_t* player_resources;
    int32_t* next_birth;
    int32_t* next_pending_order;
    int32_t* alternating_conflict_count;
    uint8_t* game_over;
    int32_t* winner;
    int32_t* spawn_overflow;
    uint32_t* environment_root; /* [L][2] */
    uint32_t* episode_index;    /* [L] */
} nro_state;

/* Commands, [L][2][C] per field.  src/nanorts/model/commands.py:22-35. */
typedef struct nro_commands {
    int32_t* kind;
    int32_t* direction;
    int32_t* none_duration;
    int32_t* target_cell;
    int32_t* produced_type;
    int32_t* request_order;
} nro_commands;

/* Per-env step outputs (StepResult minus the per-slot records that nothing
 * consumes).  src/nanorts/model/step.py:22-127. */
typedef struct nro_step_out {
    uint8_t* terminated;        /* [L] */
    uint8_t* truncated;         /* [L] */
    float* reward;              /* [L][2] */
    int32_t* admitted_harvest;  /* [L][2] */
    int32_t* admitted_return;   /* [L][2] */
    int32_t* admitted_produce;  /* [L][2][T] */
    int32_t* admitted_attack;   /* [L][2][3] */
    /* The per-slot completion records of the FFI target's results 27-30
     * (src/nanorts/core/cycle.py:48-81, 254-300): is_member [L][E], int32
     * [L][E][6] (actor_birth, target_birth, amount, balance, spawn_birth,
     * death_birth), int16 [L][E][4] (target_slot, spawn_slot, spawn_cell,
     * death_slot), int8 [L][E][6] (flags, actor_owner, actor_unit_type,
     * produced_type, death_owner, death_unit_type).  Non-members' rows are
     * zero; a member's columns its records do not set are zero.  Any may
     * be NULL (then none is written). */
    uint8_t* is_member;
    int32_t* records_i32;
    int16_t* records_i16;
    int8_t* records_i8;
} nro_step_out;

/* threefry2x32 and the JAX key plumbing (partitionable mode). */
void nro_threefry2x32(const uint32_t key[2], uint32_t x[2]);
void nro_fold_in(const uint32_t key[2], uint32_t data, uint32_t out[2]);
void nro_split(const uint32_t key[2], uint32_t index, uint32_t out[2]);
int32_t nro_randint01(const uint32_t key[2]);
int32_t nro_conflict_draw(const uint32_t root[2], int32_t time, int32_t birth, int32_t ordinal);

/* core.step for envs [0, L): key is [L][2] (episode roots). */
void nro_core_step(const nro_game* g, nro_state* s, const nro_commands* c, const uint32_t* key,
                   int64_t L, nro_step_out* out);

/* Legality rows bool[L][2][C][W] (W = 22 + T + O) and words uint32[L][2][C][3]
 * exactly as get_avail_actions publishes them (NONE forced on unavailable rows). */
void nro_avail_rows(const nro_game* g, const nro_state* s, int64_t L, uint8_t* rows);
void nro_avail_words(const nro_game* g, const nro_state* s, int64_t L, uint32_t* words);
/* Factored legality before the availability merge (legality.derive). */
void nro_legality_rows(const nro_game* g, const nro_state* s, int64_t L, uint8_t* rows);

void nro_visible_cells(const nro_game* g, const nro_state* s, int64_t L, int32_t observer,
                       uint8_t* cells);
void nro_symbolic(const nro_game* g, const nro_state* s, int64_t L, int32_t partial,
                  uint8_t* feature_maps /* [L][2][H][W][6] */, int32_t* scalars /* [L][2][4] */);
void nro_pixels(const nro_game* g, const nro_state* s, int64_t L, int32_t partial,
                const uint8_t* tiles /* [2*(1+3T)][16][16][3] */,
                uint8_t* image /* [L][2][16H][16W][3] */, int32_t* scalars);

void nro_decode_actions(const nro_game* g, const nro_state* s, const int32_t* actions /* [L][2][C][7] */,
                        int64_t L, nro_commands* c);

/* The synthetic harness sampler: uniform over each factor's legal values. */
void nro_sample_actions(const nro_game* g, const uint8_t* rows /* [L][2][C][W] */,
                        const uint32_t sample_key[2], int32_t step, int64_t env0, int64_t L,
                        int32_t* actions);

/* Reset envs whose done flag is set to the initial state (lifecycle.advance). */
void nro_reset_where_done(const nro_game* g, const nro_state* initial, nro_state* s,
                          const uint8_t* done, int64_t L);

/* env.step through the drop-in API: decode -> core.step -> advance -> observe. */
typedef struct nro_env_out {
    float* reward;          /* [L][2] */
    uint8_t* done;          /* [L] */
    uint8_t* terminated;    /* [L] */
    uint8_t* truncated;     /* [L] */
    int32_t* winner;        /* [L] (pre-reset) */
    uint8_t* spawn_overflowed; /* [L] */
    uint8_t* feature_maps;  /* [L][2][H][W][6] or NULL */
    int32_t* scalars;       /* [L][2][4] or NULL */
    uint8_t* final_feature_maps; /* [L][2][H][W][6] of the ending (pre-reset) state, or NULL */
    int32_t* final_scalars;      /* [L][2][4] of the ending state, or NULL */
    float* reward_components;    /* [L][2][6] (src/nanorts/adapters/rewards.py:47-71), or NULL */
} nro_env_out;

void nro_env_step(const nro_game* g, const nro_state* initial, nro_state* s, const int32_t* actions,
                  int64_t L, int32_t partial, nro_env_out* out);

/* Multi-threaded synthetic rollout: masks -> sample -> env.step for `steps`
 * cycles over envs [0, L), which the sampler numbers env0 + l.  Per-step
 * rewards [steps][L][2] and dones
 * [steps][L] are recorded when non-NULL; actions [steps][L][2][C][7] too.
 * Feature maps and scalars of the last step go to `last_*` when non-NULL.
 * Returns the number of threads used. */
int32_t nro_rollout(const nro_game* g, const nro_state* initial, nro_state* s,
                    const uint32_t sample_key[2], int32_t step0, int32_t steps, int64_t L,
                    int32_t partial, int32_t threads, float* rewards, uint8_t* dones,
                    int32_t* actions, uint8_t* last_feature_maps, int32_t* last_scalars, int64_t env0);

/* Carry of an abstraction-family bot (AbstractActions,
 * src/nanorts/bots/abstraction.py:70-81): [L][C] rows and next_order [L]. */
typedef struct nro_abstract {
    int32_t* kind;
    int32_t* unit_birth;
    int32_t* order;
    int32_t* target;
    int32_t* target_birth;
    int32_t* base;
    int32_t* base_birth;
    int32_t* cell;
    int32_t* unit_type;
    uint8_t* trained;
    int32_t* next_order;
} nro_abstract;

/* family.act (src/nanorts/bots/family.py:34-41): strategy 0 WorkerRush,
 * 1 barracks rush training `trained_type` (LightRush: 4).  Commands for both
 * players [L][2][C] (the other player's rows empty); carry updated in place. */
void nro_abstraction_act(const nro_game* g, const nro_state* s, int64_t L, int32_t strategy,
                         int32_t trained_type, const int32_t* player, nro_abstract* carry,
                         nro_commands* out);
/* abstraction.empty_actions for envs [0, L). */
void nro_empty_actions(const nro_game* g, nro_abstract* carry, int64_t L);
/* pathfinding.search over open cells bool[H*W]: returns the first step
 * direction or -1; out = {found, step, distance, pops}. */
int32_t nro_astar(const uint8_t* open_cell, int32_t W, int32_t H, int32_t start, int32_t target,
                  int32_t range, int32_t out[4]);
/* The walk of the FFI target nanorts_astar_chain for one lane: free and
 * claimed bool[H*W], rows [capacity][columns], queue [capacity]; out
 * [capacity + 1][4] (see bots.c). */
void nro_astar_chain(const uint8_t* free_cells, const uint8_t* claimed, const int32_t* rows, const int32_t* queue,
                     int32_t count, int32_t moves_allowed, int32_t reserved, int32_t balance, const int32_t* draws,
                     int64_t draw_count, int32_t drawing, int32_t W, int32_t H, int64_t capacity, int64_t columns,
                     const int64_t fallback[3], const int64_t blocked[3], int32_t* out);
/* seat.step_seat: actions [L][C][7] are the learner's rows; the learner is
 * seats[l] when `seats` is set, else `fixed`; the bot plays 1 - learner.
 * With `draw`, a lane whose game ended takes nro_episode_seat of its next
 * episode root. */
void nro_seat_step(const nro_game* g, const nro_state* initial, nro_state* s, int64_t L, int32_t strategy,
                   int32_t trained_type, int32_t fixed, int32_t* seats, int32_t draw, nro_abstract* carry,
                   const int32_t* actions, int32_t partial, nro_env_out* out);
/* The "drawn" seat of an episode root: randint(fold_in(root, 2**32 - 2), 0, 2). */
int32_t nro_episode_seat(const uint32_t episode_root[2]);

/* GridNet decode_actions (src/nanorts/adapters/gridnet/actions.py:31-52):
 * per-cell actions [L][2][H*W][7] -> Commands [L][2][C] per field. */
void nro_gridnet_decode(const nro_game* g, const nro_state* s, const int32_t* actions, int64_t L,
                        nro_commands* out);

/* The harness sampler over GridNet's per-cell rows [L][2][H*W][78] at
 * position player * H*W + cell -> actions [L][2][H*W][7]. */
void nro_gridnet_sample_actions(const nro_game* g, const uint8_t* rows, const uint32_t sample_key[2], int32_t step,
                                int64_t env0, int64_t L, int32_t* actions);

/* Invariant check (src/nanorts/model/state.py:87-165); returns a bitmask of
 * violated invariants for env l, 0 when the state is well formed. */
int32_t nro_state_violations(const nro_game* g, const nro_state* s, int64_t l);

#ifdef __cplusplus
}
#endif

#endif
