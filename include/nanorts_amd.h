/*
 * nanorts_amd: MI355X (gfx950) kernels for the NanoRTS batched game hot path.
 *
 * The C ABI below is the drop-in boundary.  Every entry point takes plain
 * device pointers and sizes, runs asynchronously on the given HIP stream
 * (`stream` is a hipStream_t; NULL is the default stream), allocates no
 * device memory, and returns NANORTS_OK or an error code; the message of the
 * last failure on the calling thread is nanorts_amd_last_error().
 *
 * Layouts are the reference's pytree leaves with a leading lane (env) dim L,
 * exactly as jax.vmap hands them to its XLA FFI handlers
 * (src/nanorts/model/state.py:33-84, src/nanorts/kernels/batching.py:41-100):
 *   per-slot leaves [L][E], entity_at [L][H][W], scalars [L], per-player [L][2].
 * Index leaves (cell, pending_target_cell, entity_at) are int16, which the
 * reference selects whenever the extents fit (src/nanorts/model/leaf.py:85-98).
 */
#ifndef NANORTS_AMD_H
#define NANORTS_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NANORTS_OK 0
#define NANORTS_INVALID_ARGUMENT 1
#define NANORTS_INTERNAL 2

#define NANORTS_MAX_TYPES 8

#define NANORTS_CANCEL_BOTH 0
#define NANORTS_CANCEL_RANDOM 1
#define NANORTS_CANCEL_ALTERNATING 2

/* Device pointers to the State leaves of L envs, in the reference's leaf
 * order, plus the EnvironmentState extras (src/nanorts/adapters/lifecycle.py:24-31). */
typedef struct nanorts_state {
    int32_t* birth;                 /* [L][E] */
    int8_t* unit_type;              /* [L][E] */
    int8_t* owner;                  /* [L][E] */
    int16_t* cell;                  /* [L][E] */
    int16_t* hit_points;            /* [L][E] */
    int32_t* carried_resources;     /* [L][E] */
    int8_t* pending_kind;           /* [L][E] */
    int8_t* pending_direction;      /* [L][E] */
    int32_t* pending_none_duration; /* [L][E] */
    int16_t* pending_target_cell;   /* [L][E] */
    int8_t* pending_produced_type;  /* [L][E] */
    int32_t* pending_issued_at;     /* [L][E] */
    int32_t* pending_completes_at;  /* [L][E] */
    int32_t* pending_order;         /* [L][E] */
    int16_t* entity_at;             /* [L][H][W] */
    int32_t* time;                  /* [L] */
    int32_t* player_resources;      /* [L][2] */
    int32_t* next_birth;            /* [L] */
    int32_t* next_pending_order;    /* [L] */
    int32_t* alternating_conflict_count; /* [L] */
    uint8_t* game_over;             /* [L] bool */
    int32_t* winner;                /* [L] */
    int32_t* spawn_overflow;        /* [L][2] telemetry.spawn_overflow */
    uint32_t* environment_root;     /* [L][2] key data; NULL where unused */
    uint32_t* episode_index;        /* [L]; NULL where unused */
} nanorts_state;

/* The static game: BucketSpec extents, the unit type table columns
 * (src/nanorts/model/unit_types.py:16-148; packed by the reference as the
 * `table` and `timings` operands, src/nanorts/core/unit_tables.py:9-48), the
 * terrain (device bool[H][W]) and the decided initial State of one env
 * (device rows, L = 1) that an auto-reset copies in. */
typedef struct nanorts_game {
    int32_t height, width, cells;
    int32_t neutral, capacity, entities; /* N, C, E = N + 2C */
    int32_t types;                       /* T <= 8 */
    int32_t offsets;                     /* attack window cells (2R+1)^2 <= 49 */
    int32_t strategy;                    /* NANORTS_CANCEL_* */
    int32_t max_cycles;
    int32_t cost[NANORTS_MAX_TYPES];
    int32_t hit_points[NANORTS_MAX_TYPES];
    int32_t produce_time[NANORTS_MAX_TYPES];
    int32_t move_time[NANORTS_MAX_TYPES];
    int32_t attack_time[NANORTS_MAX_TYPES];
    int32_t harvest_time[NANORTS_MAX_TYPES];
    int32_t attack_range[NANORTS_MAX_TYPES];
    int32_t attack_damage[NANORTS_MAX_TYPES];
    int32_t harvest_amount[NANORTS_MAX_TYPES];
    int32_t sight_radius[NANORTS_MAX_TYPES];
    int32_t is_resource[NANORTS_MAX_TYPES];
    int32_t is_stockpile[NANORTS_MAX_TYPES];
    int32_t can_harvest[NANORTS_MAX_TYPES];
    int32_t can_move[NANORTS_MAX_TYPES];
    int32_t can_attack[NANORTS_MAX_TYPES];
    int32_t produces[NANORTS_MAX_TYPES * NANORTS_MAX_TYPES]; /* [producer * 8 + produced] */
    const uint8_t* terrain;  /* device bool[H][W] */
    nanorts_state initial;   /* device rows of one decided initial env */
} nanorts_game;

/* Commands [L][2][C] per field (src/nanorts/model/commands.py:22-35). */
typedef struct nanorts_commands {
    const int32_t* kind;
    const int32_t* direction;
    const int32_t* none_duration;
    const int32_t* target_cell;
    const int32_t* produced_type;
    const int32_t* request_order;
} nanorts_commands;

/* core.step results besides the state.  Any pointer may be NULL; the four
 * record pointers are used only when all four are set. */
typedef struct nanorts_step_results {
    uint8_t* terminated;        /* [L] bool */
    uint8_t* truncated;         /* [L] bool */
    float* reward;              /* [L][2] */
    int32_t* admitted_harvest;  /* [L][2] */
    int32_t* admitted_return;   /* [L][2] */
    int32_t* admitted_produce;  /* [L][2][T] */
    int32_t* admitted_attack;   /* [L][2][3] by target owner + 1 */
    /* The per-slot completion records the step target returns as results
     * 27-30 and StepEvents decodes (src/nanorts/core/cycle.py:48-81,
     * 254-300): is_member [L][E] bool; int32 [L][E][6] actor_birth,
     * target_birth, amount, balance, spawn_birth, death_birth; int16
     * [L][E][4] target_slot, spawn_slot, spawn_cell, death_slot; int8
     * [L][E][6] flags (hit 1, death 2, harvest 4, depleted 8, return 16,
     * spawn 32), actor_owner, actor_unit_type, produced_type, death_owner,
     * death_unit_type.  A member's row holds its records (zero where none
     * writes); every other row is zero. */
    uint8_t* is_member;
    int32_t* records_i32;
    int16_t* records_i16;
    int8_t* records_i8;
} nanorts_step_results;

/* env.step outputs through the JaxMARL surface.  Any pointer may be NULL. */
typedef struct nanorts_env_results {
    float* reward;            /* [L][2] */
    uint8_t* done;            /* [L] bool */
    uint8_t* terminated;      /* [L] bool */
    uint8_t* truncated;       /* [L] bool */
    int32_t* winner;          /* [L] winner of the ending state */
    uint8_t* spawn_overflowed;/* [L] bool */
    uint8_t* feature_maps;    /* [L][2][H][W][6] of the post-reset state */
    int32_t* scalars;         /* [L][2][4] */
    uint8_t* final_feature_maps; /* [L][2][H][W][6] of the ending state */
    int32_t* final_scalars;      /* [L][2][4] */
    float* reward_components;    /* [L][2][6] MicroRTS-Py shaped components */
    int32_t* spawn_overflow;     /* [L][2] telemetry of the ending state */
} nanorts_env_results;

/* Outputs of a fused rollout.  Any pointer may be NULL. */
typedef struct nanorts_rollout_results {
    float* rewards;         /* [steps][L][2] */
    uint8_t* dones;         /* [steps][L] bool */
    int32_t* actions;       /* [steps][L][2][C][7] sampled actions */
    uint8_t* feature_maps;  /* [depth][L][2][H][W][6]; step t writes slot t % depth */
    int32_t* scalars;       /* [depth][L][2][4] */
    int32_t depth;          /* ring depth of feature_maps / scalars, >= 1 */
    int32_t* general_admissions; /* [L] cycles of the launch admitted request by request (an irregular
                                  * state or more than 64 requests); written by nanorts_amd_rollout only */
    int32_t* progress;           /* [L] caller-owned work words of nanorts_amd_rollout's two-pass launch, or
                                  * NULL for one pass on the full LDS block.  With them, a first pass runs
                                  * each game on a smaller LDS block (more games per CU) until a cycle needs
                                  * the request-by-request admission or more than 64 live slots complete;
                                  * the second pass runs the rest of that game's cycles on the full block.
                                  * On return: the cycles of the last launch each game ran in the first
                                  * pass.  Ignored by the seat rollouts. */
} nanorts_rollout_results;

/* Carry of an abstraction-family bot (AbstractActions,
 * src/nanorts/bots/abstraction.py:70-81), [L][C] rows updated in place. */
typedef struct nanorts_abstract_actions {
    int32_t* kind;
    int32_t* unit_birth;
    int32_t* order;
    int32_t* target;
    int32_t* target_birth;
    int32_t* base;
    int32_t* base_birth;
    int32_t* cell;
    int32_t* unit_type;
    uint8_t* trained;    /* [L][C] bool */
    int32_t* next_order; /* [L] */
} nanorts_abstract_actions;

/* Abstraction-family strategies (src/nanorts/bots/family.py:14-17). */
#define NANORTS_WORKER_RUSH 0
#define NANORTS_BARRACKS_RUSH 1

/* Writable Commands [L][2][C] per field. */
typedef struct nanorts_command_buffers {
    int32_t* kind;
    int32_t* direction;
    int32_t* none_duration;
    int32_t* target_cell;
    int32_t* produced_type;
    int32_t* request_order;
} nanorts_command_buffers;

/* GridNet observation buffers (src/nanorts/adapters/gridnet/observation.py:17-72,
 * layout.py:46-70).  Any pointer may be NULL. */
typedef struct nanorts_gridnet_obs {
    int32_t planes_form;  /* 0 one-hot [L][2][H][W][29], 1 indices int8 [L][2][H][W][6] */
    int32_t planes_bytes; /* one-hot element bytes: 1 (uint8 / bool) or 4 (int32) */
    void* planes;
    uint8_t* source_mask; /* [L][2][H][W] bool */
    int32_t mask_form;    /* 0 rows [L][2][H][W][78], 1 packed uint32 [L][2][H][W][3] */
    int32_t mask_bytes;   /* rows element bytes: 1 or 4 */
    void* action_mask;
} nanorts_gridnet_obs;

/* GridNet step outputs (src/nanorts/adapters/gridnet/env.py:30-58).  Any
 * pointer may be NULL. */
typedef struct nanorts_gridnet_results {
    float* reward_components; /* [L][2][6] */
    uint8_t* reward_dones;    /* [L][2][6] bool */
    uint8_t* terminated;      /* [L] */
    uint8_t* truncated;       /* [L] */
    uint8_t* done;            /* [L] */
    int32_t* winner;          /* [L] */
    uint8_t* spawn_overflowed;/* [L] */
    void* final_planes;       /* planes of the ending state, in observation's planes form */
    nanorts_gridnet_obs observation; /* of the post-reset state */
    int32_t* spawn_overflow;  /* [L][2] telemetry of the ending state */
} nanorts_gridnet_results;

const char* nanorts_amd_build_id(void);
const char* nanorts_amd_entries(void);
const char* nanorts_amd_last_error(void);

/* Least LDS bytes one workgroup may allocate over the listed devices (0 on
 * error).  Replaces nanorts_shared_opt_in
 * (src/nanorts/kernels/cuda/registry.cu:224-226), which the reference's
 * loader binds (src/nanorts/kernels/library.py:42-46). */
int64_t nanorts_amd_shared_opt_in(const int32_t* devices, int64_t n);

/* Runs a wave64 ballot / prefix-count / shuffle probe on each listed device;
 * returns "" when every device passes, else a static description.
 * Replaces src/nanorts/kernels/cuda/registry.cu:174-183 (nanorts_self_check). */
const char* nanorts_amd_self_check(const int32_t* devices, int64_t n);

/* The self check without a device allocation, for callers that cannot
 * allocate (serving loops, harnesses that forbid hipMalloc).  No counterpart
 * in the reference.  It launches on the default stream and copies the probe
 * words back synchronously: it synchronises the host, so it cannot run under
 * graph capture.  Runs `waves` probe waves (1..1024; more is refused with a
 * message) on each listed device and returns "" when every wave passes;
 * probe_words (host int32[waves], or NULL) receives the last device's probe
 * words, 1 per passing wave.  The words live in a 4 KiB array of the
 * library's own that every device holds until the process ends; calls that
 * overlap on one device race on it. */
const char* nanorts_amd_self_check_no_alloc(const int32_t* devices, int64_t n, int32_t waves, int32_t* probe_words);

/* core.step: Java admission order, durative timers, conflict resolution,
 * completion in pending order, outcome.  State leaves are updated in place.
 * `key` is [key_lanes][2] episode-root key data (key_lanes 1 broadcasts).
 * Replaces the FFI target nanorts_step (src/nanorts/core/cuda/step.cu:653-698,
 * called from src/nanorts/core/cycle.py:123-134). */
int nanorts_amd_step(void* stream, const nanorts_game* game, nanorts_state state, int64_t lanes, const uint32_t* key,
                 int64_t key_lanes, nanorts_commands commands, nanorts_step_results results);

/* core.step in the operand and result order of the reference's FFI target
 * nanorts_step (src/nanorts/core/cuda/step.cu:56-108, operands built by
 * src/nanorts/core/cycle.py:123-134, 198-211): the body an XLA FFI handler of
 * that name calls with its buffers' device pointers.
 *   operands[33]: 0 key u32[key_lanes][2]; 1-6 Commands kind, direction,
 *     none_duration, target_cell, produced_type, request_order
 *     s32[command_lanes][2][C]; 7 terrain pred[1][H][W]; 8 table
 *     s32[1][T][7+T]; 9 timings s32[1][T][7]; 10-32 the 23 state leaves in
 *     nanorts_state order (the last is telemetry.spawn_overflow s32[L][2]).
 *   results[31]: 0-22 the state leaves after the step (aliasing operands
 *     10-32 in place; an unaliased result is first filled from its operand);
 *     23 admitted_harvest s32[L][2]; 24 admitted_return s32[L][2];
 *     25 admitted_produce s32[L][2][T]; 26 admitted_attack s32[L][2][3];
 *     27 is_member pred[L][E]; 28 int32 records s32[L][E][6]; 29 index
 *     records s16[L][E][4]; 30 int8 records s8[L][E][6] (the completion
 *     records of nanorts_step_results).
 * Every size argument is an extent of those buffers, so a handler that sees
 * only the buffers and the `strategy` attribute can pass them: lanes = the
 * leading extent of result 0; key_lanes and command_lanes = the leading
 * extents of operands 0 and 1, each 1 (an unbatched operand of extent 1,
 * every lane reads row 0; src/nanorts/kernels/batching.py:63-79) or `lanes`;
 * height and width from terrain; capacity = the last extent of operand 1;
 * neutral = the entity extent of operand 10 minus 2 x capacity; types = the
 * T extent of table.  The attack window of the legality rows plays no part in
 * a step.  Index leaves are int16.  Errors as every entry: NANORTS_INVALID_ARGUMENT for a
 * NULL pointer, an extent or a strategy out of range, NANORTS_INTERNAL for a
 * failed launch or copy. */
int nanorts_amd_step_ffi(void* stream, const void* const* operands, void* const* results, int64_t lanes,
                         int64_t key_lanes, int64_t command_lanes, int32_t height, int32_t width, int32_t neutral,
                         int32_t capacity, int32_t types, int64_t strategy);

/* core.step over up to 16 groups of lanes, in one launch per 4 groups.  The
 * groups' games share one bucket (extents, capacities, unit types, attack
 * window, strategy) and one unit table, and may differ in terrain and
 * max_cycles; each group has its own State, keys ([lanes or 1][2]),
 * Commands and results, with nanorts_amd_step's meaning.  `games` holds one
 * pointer per group.  Replaces the FFI target nanorts_step_groups
 * (src/nanorts/core/cuda/step.cu:704-808, called from
 * src/nanorts/core/cycle.py:137-175 through core.step_groups,
 * src/nanorts/core/__init__.py:71-89). */
int nanorts_amd_step_groups(void* stream, int32_t groups, const nanorts_game* const* games, const nanorts_state* states,
                        const int64_t* lanes, const uint32_t* const* keys, const int64_t* key_lanes,
                        const nanorts_commands* commands, const nanorts_step_results* results);

/* core.step over `groups` groups (1..16) in the operand and result order of
 * the reference's FFI target nanorts_step_groups
 * (src/nanorts/core/cuda/step.cu:704-808, operands built by
 * src/nanorts/core/cycle.py:137-175, 198-211): group k's 33 operands are
 * operands[33k .. 33k + 32] and its 31 results results[31k .. 31k + 30], each
 * in nanorts_amd_step_ffi's order and meaning; lanes[k], key_lanes[k] and
 * command_lanes[k] are group k's extents as there.  The groups share one
 * bucket (height, width, neutral, capacity, types, the `strategy`
 * attribute); each brings its own key, Commands, terrain, table, timings and
 * state.  One launch per four groups, as nanorts_amd_step_groups. */
int nanorts_amd_step_groups_ffi(void* stream, int32_t groups, const void* const* operands, void* const* results,
                                const int64_t* lanes, const int64_t* key_lanes, const int64_t* command_lanes,
                                int32_t height, int32_t width, int32_t neutral, int32_t capacity, int32_t types,
                                int64_t strategy);

/* Factored legality rows bool[L][2][C][22+T+O] (active units, availability not
 * applied).  Replaces nanorts_legality (src/nanorts/core/cuda/legality.cu:535-545). */
int nanorts_amd_legality(void* stream, const nanorts_game* game, nanorts_state state, int64_t lanes, uint8_t* rows);

/* The same rows as contiguous 96-bit words uint32[L][2][C][3].  Replaces
 * nanorts_legality_words (src/nanorts/core/cuda/legality.cu:547-561). */
int nanorts_amd_legality_words(void* stream, const nanorts_game* game, nanorts_state state, int64_t lanes,
                           uint32_t* words);

/* Legality rows or words in the operand order of the reference's FFI targets
 * nanorts_legality and nanorts_legality_words
 * (src/nanorts/core/cuda/legality.cu:535-561, operands built by
 * src/nanorts/core/legality.py:84-125): the body a handler of either name
 * calls with its buffers' device pointers.
 *   operands[9]: birth s32[L][E], unit_type s8[L][E], owner s8[L][E],
 *     carried_resources s32[L][E], cell s16[L][E], entity_at s16[L][H][W],
 *     player_resources s32[L][2], terrain pred[1][H][W], table s32[1][T][7+T].
 *   result: rows bool[L][2][C][22+T+offsets] (words = 0) or uint32[L][2][C][3]
 *     (words = 1).
 * The sizes are extents: lanes = the result's leading extent; height and
 * width of entity_at; entities = birth's second extent; capacity = the
 * result's third extent; types = the table's second extent; offsets = the
 * rows' last extent - 22 - T, or the words target's `offsets` attribute.
 * Leaves hold one row per lane; terrain and table one shared row. */
int nanorts_amd_legality_ffi(void* stream, const void* const* operands, void* result, int32_t words, int64_t lanes,
                             int32_t height, int32_t width, int32_t entities, int32_t capacity, int32_t types,
                             int32_t offsets);

/* get_avail_actions masks: rows & available, only NONE on unavailable rows
 * (src/nanorts/adapters/jaxmarl/actions.py:28-41), as bool rows and/or words. */
int nanorts_amd_avail_actions(void* stream, const nanorts_game* game, nanorts_state state, int64_t lanes,
                          uint8_t* rows, uint32_t* words);

/* Sight-radius visibility bool[L][H][W] of `observer`'s block.  Replaces
 * nanorts_visible_cells (src/nanorts/observations/cuda/visibility.cu:86-138). */
int nanorts_amd_visible_cells(void* stream, const nanorts_game* game, nanorts_state state, int64_t lanes,
                          int32_t observer, uint8_t* cells);

/* Sight of one slot block in the operand order of the reference's FFI target
 * nanorts_visible_cells (src/nanorts/observations/cuda/visibility.cu:86-158,
 * called from src/nanorts/observations/visibility.py:85-103): every slot of
 * [first, first + count) whose birth is not -1 and whose cell and type are in
 * range marks the cells within radius[type] (dx^2 + dy^2 <= r^2) of its cell.
 * birth s32, unit_type s8 and cell (cell_bytes = 1, 2 or 4) hold `slots`
 * elements per row and one row per lane or one shared row (*_lanes = 1);
 * radius s32[types] is shared; out bool[lanes][height][width]; the board is
 * at most 48K cells.  The attributes first, count, width and height are the
 * target's own. */
int nanorts_amd_visible_cells_ffi(void* stream, const int32_t* birth, int64_t birth_lanes, const int8_t* unit_type,
                                  int64_t unit_type_lanes, const void* cell, int32_t cell_bytes, int64_t cell_lanes,
                                  int64_t slots, const int32_t* radius, int64_t types, uint8_t* out, int64_t lanes,
                                  int64_t first, int64_t count, int32_t width, int32_t height);

/* Symbolic uint8 observations of both agents
 * (src/nanorts/observations/symbolic.py:130-180). */
int nanorts_amd_observe(void* stream, const nanorts_game* game, nanorts_state state, int64_t lanes, int32_t partial,
                    uint8_t* feature_maps, int32_t* scalars);

/* Pixel observations uint8[L][2][16H][16W][3] from a tile table
 * uint8[2(1+3T)][16][16][3] (src/nanorts/observations/pixels.py:71-88,
 * src/nanorts/rendering/raster.py:53-127). */
int nanorts_amd_pixels(void* stream, const nanorts_game* game, nanorts_state state, int64_t lanes, int32_t partial,
                   const uint8_t* tiles, uint8_t* image, int32_t* scalars);

/* Pixel observations uint8[images][16H][16W][3] from symbolic feature maps
 * uint8[images][H][W][6] (images = L * 2 agents) and the same tile table;
 * equal to nanorts_amd_pixels of the state the maps were encoded from.  Replaces
 * pixels_from_symbolic (src/nanorts/observations/pixels.py:91-110); tiles and
 * image must be 16-byte aligned. */
int nanorts_amd_pixels_from_maps(void* stream, const nanorts_game* game, int64_t images, const uint8_t* feature_maps,
                             const uint8_t* tiles, uint8_t* image);

/* Auto-reset: envs whose done flag is set get the initial State and
 * episode_index + 1.  Replaces nanorts_reset_where_done
 * (src/nanorts/adapters/cuda/reset.cu:160-222). */
int nanorts_amd_reset_where_done(void* stream, const nanorts_game* game, nanorts_state state, int64_t lanes,
                             const uint8_t* done);

/* The masked row select of the reference's FFI targets
 * nanorts_reset_where_done and nanorts_reset_packed_where_done
 * (src/nanorts/adapters/cuda/reset.cu:160-246, called from
 * src/nanorts/adapters/lifecycle.py:108-134): for each of `leaves` (at most
 * 32) row leaves, results[k] row l = done[l] ? reset_rows[k] row (l, or 0
 * when reset_lanes[k] = 1) : ending[k] row l, rows of row_bytes[k] bytes.  A
 * result that aliases its ending rows is written on done lanes only.  The
 * packed target's handler passes its one shared uint8 row as reset_rows[k] =
 * packed + each leaf's 16-byte-aligned offset, with reset_lanes[k] = 1. */
int nanorts_amd_reset_rows_ffi(void* stream, const uint8_t* done, int64_t lanes, int32_t leaves,
                               const void* const* reset_rows, const int64_t* reset_lanes, const void* const* ending,
                               void* const* results, const int64_t* row_bytes);

/* env.step of the JaxMARL facade in one launch: decode int32[L][2][C][7]
 * actions, core.step keyed by the episode root, advance (auto-reset) and
 * observe (src/nanorts/adapters/jaxmarl/env.py:72-184). */
int nanorts_amd_env_step(void* stream, const nanorts_game* game, nanorts_state state, int64_t lanes,
                     const int32_t* actions, int32_t partial, nanorts_env_results results);

/* env.step_env of the JaxMARL facade: as nanorts_amd_env_step without the
 * auto-reset, so the state, the observation and the rewards are those of the
 * ending state (src/nanorts/adapters/jaxmarl/facade.py:130-165, transition
 * in src/nanorts/adapters/jaxmarl/env.py:170-171). */
int nanorts_amd_env_transition(void* stream, const nanorts_game* game, nanorts_state state, int64_t lanes,
                           const int32_t* actions, int32_t partial, nanorts_env_results results);

/* The JaxMARL request (src/nanorts/adapters/jaxmarl/env.py:181-184):
 * decode_actions of int32[L][2][C][7] action rows into Commands
 * (src/nanorts/adapters/jaxmarl/actions.py:61-84) and, when `episode_keys`
 * is not NULL, the episode roots fold_in(environment_root, episode_index)
 * as uint32[L][2]. */
int nanorts_amd_decode_actions(void* stream, const nanorts_game* game, nanorts_state state, int64_t lanes,
                           const int32_t* actions, nanorts_command_buffers commands, uint32_t* episode_keys);

/* The synthetic harness's integer uniform-over-legal sampler: actions
 * int32[L][2][C][7] from avail words uint32[L][2][C][3] for rollout step
 * `step`, envs numbered from env0. */
int nanorts_amd_sample_actions(void* stream, const nanorts_game* game, int64_t lanes, const uint32_t* avail_words,
                           const uint32_t* sample_key /* host [2] */, int32_t step, int64_t env0,
                           int32_t* actions);

/* Fused rollout of `steps` cycles with the state resident in LDS: per step
 * masks -> sample -> decode -> core.step -> auto-reset -> observe.  Bit-equal
 * to calling avail_actions, sample_actions and env_step once per step. */
int nanorts_amd_rollout(void* stream, const nanorts_game* game, nanorts_state state, int64_t lanes,
                    const uint32_t* sample_key /* host [2] */, int32_t step0, int32_t steps, int32_t partial,
                    int64_t env0,
                    nanorts_rollout_results results);

/* Which first pass nanorts_amd_rollout runs for `game` when the caller asks
 * for the two-pass launch (results.progress set, feature maps 8-byte
 * aligned or absent): 2 two games per wave, 1 one game per wave, 0 none (one
 * pass on the full block); < 0 an error code.  Diagnostics only: it has no
 * counterpart in the reference, whose program has no such launch. */
int nanorts_amd_rollout_first_pass(const nanorts_game* game);

/* family.act of the rush strategies: WorkerRush (NANORTS_WORKER_RUSH) or the
 * barracks rush training `trained_type` (NANORTS_BARRACKS_RUSH; LightRush
 * trains type 4).  Writes commands int32[L][6][2][C] (kind, direction,
 * none_duration, target_cell, produced_type, request_order; the other
 * player's rows empty) and updates the carry in place.  `player` is
 * [player_lanes] (1 broadcasts).  Replaces the FFI target
 * nanorts_abstraction_act (src/nanorts/bots/cuda/abstraction_act.cu:1324),
 * called through src/nanorts/bots/whole_act.py:125-162 from
 * src/nanorts/bots/family.py:34-41. */
int nanorts_amd_abstraction_act(void* stream, const nanorts_game* game, nanorts_state state, int64_t lanes,
                            int32_t strategy, int32_t trained_type, const int32_t* player, int64_t player_lanes,
                            nanorts_abstract_actions carry, int32_t* commands);

/* family.act of the rush strategies in the operand and result order of the
 * reference's FFI target nanorts_abstraction_act
 * (src/nanorts/bots/cuda/abstraction_act.cu:1231-1324, operands built by
 * src/nanorts/bots/whole_act.py:125-162): the body a handler of that name
 * calls with its buffers' device pointers.
 *   operands[24]: 0-9 the State leaves the act reads: birth s32[E],
 *     unit_type s8[E], owner s8[E], cell s16[E], carried_resources s32[E],
 *     pending_kind s8[E], pending_direction s8[E], pending_produced_type
 *     s8[E], entity_at s16[H][W], player_resources s32[2]; 10 terrain
 *     pred[H][W]; 11 the bots' unit table s32[T][6] (can_harvest,
 *     is_resource, is_stockpile, can_attack, attack_range, cost); 12 player
 *     s32; 13-23 the carry (AbstractActions: kind, unit_birth, order, target,
 *     target_birth, base, base_birth, cell, unit_type s32[L][C], trained
 *     pred[L][C], next_order s32[L]).
 *   operand_lanes[13]: the leading extents of operands 0-12, each 1 (one row
 *     shared by every lane) or `lanes`; terrain and table must be 1.
 *   results[12]: 0-10 the carry after the act (aliasing operands 13-23; an
 *     unaliased result is first filled from its operand); 11 the Commands
 *     s32[L][6][2][C].
 * `strategy` and `trained` are the target's attributes: 0 worker rush, 1
 * barracks rush training `trained`.  The defense strategies (2, 3) are
 * refused with NANORTS_INVALID_ARGUMENT: the rush bots are the ones built.
 * Index leaves are int16. */
int nanorts_amd_abstraction_act_ffi(void* stream, const void* const* operands, const int64_t* operand_lanes,
                                    void* const* results, int64_t lanes, int32_t height, int32_t width,
                                    int32_t entities, int32_t capacity, int32_t types, int64_t strategy,
                                    int64_t trained);

/* pathfinding.search per lane in the operand order of the reference's FFI
 * target nanorts_astar_search (src/nanorts/bots/cuda/pathfinding.cu:20-104,
 * called from src/nanorts/bots/pathfinding.py:102-118): free pred[*][H][W],
 * start, target and range s32[*], each with `*_lanes` rows (1 shared or
 * `lanes`); out s32[lanes][4] = found, first step, path length, pops
 * (-1, -1 for the step and length when nothing is found).  Boards of at
 * most 8192 cells. */
int nanorts_amd_astar_search_ffi(void* stream, const uint8_t* free, int64_t free_lanes, const int32_t* start,
                                 int64_t start_lanes, const int32_t* target, int64_t target_lanes,
                                 const int32_t* range, int64_t range_lanes, int32_t width, int32_t height,
                                 int32_t* out, int64_t lanes);

/* abstraction's walk in the operand order of the reference's FFI target
 * nanorts_astar_chain (src/nanorts/bots/cuda/abstraction.cu:98-301, called
 * from src/nanorts/bots/abstraction.py:1001-1033).
 *   operands[9]: free pred[*][H][W], claimed pred[*][H][W], rows
 *     s32[*][capacity][columns] (start, goal, radius, draws, options, then
 *     the desires' columns), queue s32[*][capacity], count s32[*],
 *     moves_allowed pred[*], reserved s32[*], balance s32[*], draws
 *     s32[*][draw_count]; operand_lanes[9] their leading extents (1 or
 *     `lanes`).
 *   out s32[lanes][capacity + 1][4]: per slot rank, selector, direction,
 *     drew; then kept count, draws used, 0, 0.
 * `drawing`, fallback[3] and blocked[3] (each desire's kind, claim and cost
 * columns) are the target's attributes.  Boards of at most 8192 cells. */
int nanorts_amd_astar_chain_ffi(void* stream, const void* const* operands, const int64_t* operand_lanes, int32_t* out,
                                int64_t lanes, int32_t width, int32_t height, int64_t capacity, int64_t columns,
                                int64_t draw_count, int32_t drawing, const int64_t* fallback, const int64_t* blocked);

/* seat.step_seat with a static learner seat in one launch: the bot plays
 * 1 - learner from the current state, the learner's action rows
 * int32[L][C][7] are decoded, the merged commands go through core.step under
 * the episode root, auto-reset, and the carry is emptied where done.  Results
 * as nanorts_amd_env_step, for both agents.  Replaces step_seat
 * (src/nanorts/bots/seat.py:84-149), which composes the bot's act,
 * jaxmarl.request_against (src/nanorts/adapters/jaxmarl/env.py:78-96),
 * core.step and respond. */
int nanorts_amd_seat_step(void* stream, const nanorts_game* game, nanorts_state state, int64_t lanes,
                      int32_t strategy, int32_t trained_type, int32_t learner, nanorts_abstract_actions carry,
                      const int32_t* actions, int32_t partial, nanorts_env_results results);

/* nanorts_amd_seat_step with a per-lane seat: seats int32[L] holds each lane's
 * learner (0 or 1) on entry.  With draw != 0 (the "drawn" rule) a lane whose
 * game ended takes the seat drawn from its next episode's root,
 * randint(fold_in(episode_root, 2**32 - 2), (), 0, 2); otherwise the seats
 * stay (a per-lane Player array).  Replaces step_seat with seat="drawn" or
 * an Array seat (src/nanorts/bots/seat.py:84-149, 352-366). */
int nanorts_amd_seat_step_lanes(void* stream, const nanorts_game* game, nanorts_state state, int64_t lanes,
                            int32_t strategy, int32_t trained_type, int32_t* seats, int32_t draw,
                            nanorts_abstract_actions carry, const int32_t* actions, int32_t partial,
                            nanorts_env_results results);

/* The "drawn" rule's seat of each lane's current episode:
 * randint(fold_in(fold_in(environment_root, episode_index), 2**32 - 2), (),
 * 0, 2) into seats int32[L].  Replaces _episode_seat
 * (src/nanorts/bots/seat.py:352-360) as reset_seat calls it (line 77). */
int nanorts_amd_episode_seats(void* stream, const uint32_t* environment_root /* [L][2] */,
                          const uint32_t* episode_index /* [L] */, int64_t lanes, int32_t* seats);

/* Fused learner-vs-bot rollout of `steps` cycles with the state resident in
 * LDS: per cycle the learner's rows from the synthetic harness's integer
 * uniform-over-legal sampler (its avail words, `sample_key`, step
 * step0 + t), the bot's act and the seat step as nanorts_amd_seat_step.
 * Bit-equal to calling nanorts_amd_avail_actions, nanorts_amd_sample_actions and
 * nanorts_amd_seat_step once per cycle with the learner's rows.  results.actions
 * (when set) records the learner's rows [steps][L][C][7]; rewards, dones and
 * the observation ring are those of nanorts_amd_rollout. */
int nanorts_amd_seat_rollout(void* stream, const nanorts_game* game, nanorts_state state, int64_t lanes,
                         int32_t strategy, int32_t trained_type, int32_t learner, nanorts_abstract_actions carry,
                         const uint32_t* sample_key /* host [2] */, int32_t step0, int32_t steps, int32_t partial,
                         int64_t env0, nanorts_rollout_results results);

/* nanorts_amd_seat_rollout with per-lane seats as nanorts_amd_seat_step_lanes: seats
 * int32[L] is read at the start and holds the seats after the last cycle;
 * seat_record (when set) receives the learner of every cycle [steps][L],
 * which selects the learner's reward from results.rewards [steps][L][2]. */
int nanorts_amd_seat_rollout_lanes(void* stream, const nanorts_game* game, nanorts_state state, int64_t lanes,
                               int32_t strategy, int32_t trained_type, int32_t* seats, int32_t draw,
                               int32_t* seat_record, nanorts_abstract_actions carry,
                               const uint32_t* sample_key /* host [2] */, int32_t step0, int32_t steps,
                               int32_t partial, int64_t env0, nanorts_rollout_results results);

/* GridNet decode_actions: per-cell actions int32[L][2][H][W][7] -> Commands.
 * Replaces the FFI target nanorts_gridnet_decode
 * (src/nanorts/adapters/gridnet/cuda/decode.cu, called from
 * src/nanorts/adapters/gridnet/actions.py:199-232); the legality words the
 * reference passes in are derived in the kernel. */
int nanorts_amd_gridnet_decode(void* stream, const nanorts_game* game, nanorts_state state, int64_t lanes,
                           const int32_t* actions, nanorts_command_buffers commands);

/* GridNet decode_actions in the operand and result order of the reference's
 * FFI target nanorts_gridnet_decode (src/nanorts/adapters/gridnet/cuda/decode.cu:
 * 426-540, operands built by src/nanorts/adapters/gridnet/actions.py:199-232):
 *   operands[11]: 0 actions s32[*][2][H][W][7]; 1 birth s32[*][E]; 2
 *     pending_kind s8[*][E]; 3 cell s16[*][E]; 4 pending_direction
 *     s8[*][E]; 5 pending_produced_type s8[*][E]; 6 player_resources
 *     s32[*][2]; 7 move_direction pred[*][C][4], 8 produce_direction
 *     pred[*][C][4] and 9 produce_type pred[*][C][T] (player 0's legality);
 *     10 unit_cost s32[T] (shared).  operand_lanes[11]: their leading
 *     extents, 1 or `lanes`.
 *   results[6]: the Commands fields s32[L][2][C].
 * height, width, neutral, capacity, types, costs and side are the target's
 * attributes (costs must equal types; warp_words, the reference's own
 * scratch size, plays no part).  Index leaves are int16. */
int nanorts_amd_gridnet_decode_ffi(void* stream, const void* const* operands, const int64_t* operand_lanes,
                                   void* const* results, int64_t lanes, int32_t height, int32_t width, int32_t neutral,
                                   int32_t capacity, int32_t types, int32_t costs, int32_t side);

/* GridNet observe: planes, source mask and action mask of the state
 * (src/nanorts/adapters/gridnet/observation.py:27-72). */
int nanorts_amd_gridnet_observe(void* stream, const nanorts_game* game, nanorts_state state, int64_t lanes,
                            nanorts_gridnet_obs obs);

/* GridNet step in one launch: decode, core.step keyed by the episode root,
 * reward components and reward dones, the ending state's planes, auto-reset
 * and the observation (src/nanorts/adapters/gridnet/env.py:65-118). */
int nanorts_amd_gridnet_step(void* stream, const nanorts_game* game, nanorts_state state, int64_t lanes,
                         const int32_t* actions, nanorts_gridnet_results results);

/* GridNet step_against: player 0 decoded from its per-cell actions
 * int32[L][H][W][7], player 1 plays `commands` ([L][2][C] per field; player
 * 0's rows are ignored), then as nanorts_amd_gridnet_step
 * (src/nanorts/adapters/gridnet/env.py:73-83). */
int nanorts_amd_gridnet_step_against(void* stream, const nanorts_game* game, nanorts_state state, int64_t lanes,
                                 const int32_t* actions, nanorts_commands commands, nanorts_gridnet_results results);

/* The synthetic harness's integer uniform-over-legal sampler on the GridNet
 * surface: per-cell actions int32[L][2][H][W][7] from the packed action mask
 * uint32[L][2][H][W][3] (mask_form 1), each cell drawn as
 * nanorts_amd_sample_actions draws a row, at position player * H * W + cell.
 * No reference counterpart (the reference's harness samples with
 * jax.random.categorical). */
int nanorts_amd_gridnet_sample_actions(void* stream, const nanorts_game* game, int64_t lanes, const uint32_t* mask,
                                   const uint32_t* sample_key, int32_t step, int64_t env0, int32_t* actions);

#ifdef __cplusplus
}
#endif

#endif
