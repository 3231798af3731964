// Device engine of the NanoRTS hot path for gfx950 (CDNA4, wave64).
//
// One wavefront owns one game.  The game's state rows are staged in LDS (the
// per-wave "env block"); the unit type table and the terrain are staged once
// per workgroup.  Wave-parallel phases use 64-bit ballots, mbcnt prefix counts
// and a shuffle prefix-min; the inherently sequential parts of the reference's
// semantics (requests admitted one at a time, completions applied one at a
// time) run as wave-uniform code with lane 0 writing.
//
// Semantics follow the reference JAX program (citations relative to the
// reference root, N/ = src/nanorts/); integer behaviour follows XLA: wrapping
// int32 arithmetic, floor division/modulo, gathers that wrap a negative index
// once then clamp, masked scatters that drop out-of-range indices.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/nanorts_amd.h"

#define AS3 __attribute__((address_space(3)))
#define NR_DEV __device__ __forceinline__

namespace nr {

constexpr int kWave = 64;
constexpr int32_t kAbsent = -1;
constexpr int32_t kKindNone = 0;
constexpr int32_t kKindMove = 1;
constexpr int32_t kKindHarvest = 2;
constexpr int32_t kKindReturn = 3;
constexpr int32_t kKindProduce = 4;
constexpr int32_t kKindAttack = 5;
constexpr int32_t kKindUnknown = 6;  // any issued kind outside 0..5
constexpr int32_t kNoCap = 0x7fffffff;
constexpr int32_t kCrossStride = 1 << 15;

// Unit table fields, tab[field * 8 + type] in LDS.
enum : int {
    F_COST = 0,
    F_HP,
    F_PRODUCE_TIME,
    F_MOVE_TIME,
    F_ATTACK_TIME,
    F_HARVEST_TIME,
    F_RANGE,
    F_DAMAGE,
    F_AMOUNT,
    F_SIGHT,
    F_FLAGS,
    F_PRODUCES,
    F_PACK,  // flags | produces << 8 | attack range << 16: one read for the legality rows
    F_COUNT
};
enum : int { FL_RESOURCE = 1, FL_STOCKPILE = 2, FL_HARVEST = 4, FL_MOVE = 8, FL_ATTACK = 16 };

// Per-env scalar leaves in LDS.
enum : int {
    S_TIME = 0,
    S_RES0,
    S_RES1,
    S_NEXT_BIRTH,
    S_NEXT_ORDER,
    S_ALT,
    S_GAME_OVER,
    S_WINNER,
    S_SO0,
    S_SO1,
    S_ROOT0,
    S_ROOT1,
    S_EPISODE,
    S_UNITS0,  // active units of player 0 / 1, kept by the env path for decide
    S_UNITS1,
    S_NAV,    // available units listed by summarize
    S_IRREG,  // 1 when an available unit holds a pending order
    S_NUNITS, // active owned units listed by summarize
    S_NA,     // pending MOVE / PRODUCE entries listed by summarize
    S_VISDIRTY,  // bit p: a unit of player p moved, spawned or died since its sight was last stamped
    S_COUNT = 20
};

// One row leaf of the initial State: global source, LDS destination, bytes.
struct Seg {
    const uint8_t* src;
    int32_t dst;
    int32_t bytes;
};

// Byte offsets of one env block (relative to the block) and of the
// workgroup header.  Computed on the host (see layout_for in nanorts_amd.hip).
struct Layout {
    int32_t hdr_bytes;  // tab + reset segments + terrain
    int32_t o_seg;
    int32_t env_bytes;  // one wave's block, 16-byte multiple
    int32_t o_terrain;  // in the header
    int32_t o_disk;     // in the header: sight-disk row masks [R + 1][2R + 1]
    int32_t o_walls;    // in the header: wall bitmap rows [H][seen_words] (fast_obs layouts)
    int32_t o_birth, o_carried, o_pnone, o_pissued, o_pcompl, o_porder;
    int32_t o_cell, o_hp, o_ptarget, o_entity;
    int32_t o_utype, o_owner, o_pkind, o_pdir, o_pptype;
    int32_t o_scal;
    int32_t b_events;  // admitted counts, outside the phase union
    int32_t o_bm;      // occupancy bitmaps (6 planes), outside the union
    int32_t o_lo;      // occupant word per slot (player 0's view), outside the union
    int32_t o_fl;      // occupant flags per slot: kind | resource << 4 | stockpile << 5
    int32_t o_live;    // bitmap of live slots (birth != ABSENT), 64 slots per word
    // Phase union.  Admission: commands, keys, lists.  Completion: member
    // records, keys.  Observation: seen bitmap, staging, unit list.  Masks:
    // staged words.
    int32_t c_kind, c_dir, c_ptype, c_target, c_none, c_rank;
    int32_t b_pkey, b_keys, b_tmp, b_order, b_rank;
    int32_t m_rec, m_tmp;
    int32_t v_seen, v_stage, b_units;
    int32_t v_oseen;  // observe_all's seen bitmaps (beside its staging)
    int32_t v_words;
    int32_t a_av, a_list;  // env-path admission: available list, entry list
};

// Kernel-side copy of the game (passed by value as a kernel argument).
struct KGame {
    int32_t H, W, cells, N, C, E, T, O, strategy, max_cycles;
    int32_t side, radius, rank_bits, seen_words, stage_cells, sight_max;
    int32_t fast_obs;  // 4-cell observation groups and the disk table apply
    int32_t disk_r;    // radius of the disk table: max(sight radius, attack range) <= 15
    int32_t wshift;    // log2(W) when W is a power of two, else -1
    int32_t tab[F_COUNT * 8];
    const uint8_t* terrain;
    // When set, the unit table comes from device operands in the reference's
    // layout instead of tab (see load_header); NULL otherwise.
    const int32_t* ref_table;    // [T][7 + T]
    const int32_t* ref_timings;  // [T][7]
    nanorts_state initial;
    Layout lay;
    int32_t nseg;
    Seg seg[16];
    // Slot window (the fused rollout's first pass): with shift > 0 the env
    // block stages slots [0, N + C) and [N + C + shift, N + 2C + shift) of
    // the state, whose players hold C + shift slots each; C and E here are
    // the window's.  The block's slot ls is the state's slot glob_slot(ls).
    // 0 everywhere else.
    int32_t shift;
    int32_t quick_produce;  // some produce time is below 2 or above 2^30
};

// ---------------------------------------------------------------------------
// integer helpers
// ---------------------------------------------------------------------------
NR_DEV int32_t wadd(int32_t a, int32_t b) { return (int32_t)((uint32_t)a + (uint32_t)b); }
NR_DEV int32_t wsub(int32_t a, int32_t b) { return (int32_t)((uint32_t)a - (uint32_t)b); }
NR_DEV int32_t wmul(int32_t a, int32_t b) { return (int32_t)((uint32_t)a * (uint32_t)b); }
NR_DEV int32_t clampi(int32_t v, int32_t lo, int32_t hi) { return v < lo ? lo : (v > hi ? hi : v); }
NR_DEV int32_t imin(int32_t a, int32_t b) { return a < b ? a : b; }
NR_DEV int32_t floor_div(int32_t a, int32_t b) {
    const int32_t q = a / b, r = a % b;
    return (r != 0 && ((r < 0) != (b < 0))) ? q - 1 : q;
}
NR_DEV int32_t floor_mod(int32_t a, int32_t b) {
    const int32_t r = a % b;
    return (r != 0 && ((r < 0) != (b < 0))) ? r + b : r;
}
NR_DEV int32_t gidx(int32_t i, int32_t n) { return clampi(i < 0 ? i + n : i, 0, n - 1); }
// A zero the compiler cannot see through.  Wide stores of constant zeros
// inside a loop otherwise keep a register per stored word holding zero
// across the whole loop.
NR_DEV int32_t opaque_zero() {
    int32_t z = 0;
    asm volatile("" : "+v"(z));
    return z;
}
// floor_mod / floor_div of a cell index by the board width
NR_DEV int32_t cell_x(const KGame& g, int32_t c) { return g.wshift >= 0 ? (c & (g.W - 1)) : floor_mod(c, g.W); }
NR_DEV int32_t cell_y(const KGame& g, int32_t c) { return g.wshift >= 0 ? (c >> g.wshift) : floor_div(c, g.W); }
// The state's slot and owned position of a block slot / position (the
// identity without a slot window).
NR_DEV int32_t glob_slot(const KGame& g, int32_t s) { return s < g.N + g.C ? s : s + g.shift; }
NR_DEV int32_t glob_pos(const KGame& g, int32_t p) { return p < g.C ? p : p + g.shift; }
NR_DEV int32_t dir_dx(int32_t d) { return d == 1 ? 1 : (d == 3 ? -1 : 0); }
NR_DEV int32_t dir_dy(int32_t d) { return d == 0 ? -1 : (d == 2 ? 1 : 0); }

// ---------------------------------------------------------------------------
// wave primitives
// ---------------------------------------------------------------------------
NR_DEV int lane_id() { return (int)(threadIdx.x & (kWave - 1)); }
NR_DEV uint64_t ballot(bool p) { return (uint64_t)__ballot(p); }
NR_DEV int32_t count_below(uint64_t mask) {
    return (int32_t)__builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32),
                                              __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
}
NR_DEV int32_t popc(uint64_t m) { return __popcll(m); }
NR_DEV int32_t uni(int32_t v) { return __builtin_amdgcn_readfirstlane(v); }
// LDS writes of one lane made visible to the other lanes of the wave.
NR_DEV void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}
// ---------------------------------------------------------------------------
// teams: the lanes that own one game, the whole wave (TW = 64) or one half
// of it (TW = 32, two games per wave).  Team-collective helpers act within
// the caller's team and every lane of a calling team must be active; a
// team-uniform value sits in a scalar register for a whole-wave team and in
// a vector register (one value per half) for a half-wave team.  Team masks
// are team-relative: bit i is team lane i.
// ---------------------------------------------------------------------------
template <int TW>
NR_DEV int team_lane() {
    return (int)(threadIdx.x & (TW - 1));
}
template <int TW>
NR_DEV int team_half() {
    if constexpr (TW == kWave) return 0;
    else return (int)((threadIdx.x >> 5) & 1u);
}
template <int TW>
NR_DEV uint64_t tballot(bool p) {
    const uint64_t b = (uint64_t)__ballot(p);
    if constexpr (TW == kWave) return b;
    else return team_half<TW>() ? (b >> 32) : (b & 0xFFFFFFFFull);
}
template <int TW>
NR_DEV int32_t tcount_below(uint64_t m) {
    if constexpr (TW == kWave) return count_below(m);
    else return __popc((uint32_t)m & ((1u << team_lane<TW>()) - 1u));
}
template <int TW>
NR_DEV int32_t tuni(int32_t v) {
    if constexpr (TW == kWave) return uni(v);
    else return v;
}
// team lane j's v, for j the same on every lane of the wave (a loop counter
// in a scalar register)
template <int TW>
NR_DEV int32_t tread_at(int32_t v, int32_t j) {
    if constexpr (TW == kWave) {
        return __builtin_amdgcn_readlane(v, j);
    } else {
        const int32_t lo = __builtin_amdgcn_readlane(v, j), hi = __builtin_amdgcn_readlane(v, j + 32);
        return team_half<TW>() ? hi : lo;
    }
}
// team lane j's v, for a team-uniform j
template <int TW>
NR_DEV int32_t tread(int32_t v, int32_t j) {
    if constexpr (TW == kWave) return __builtin_amdgcn_readlane(v, j);
    else return __shfl(v, j, TW);
}
// the larger of the active halves' team-uniform values (a scalar): the trip
// count of a loop both teams of a wave run, each doing its own part.  A half
// with no active lane (its game finished or stopped) counts 0: its
// registers hold nothing meaningful.
template <int TW>
NR_DEV int32_t tmax(int32_t v) {
    if constexpr (TW == kWave) {
        return v;
    } else {
        const uint64_t active = (uint64_t)__ballot(1);
        const int32_t lo = (active & 1ull) ? __builtin_amdgcn_readlane(v, 0) : 0;
        const int32_t hi = ((active >> 32) & 1ull) ? __builtin_amdgcn_readlane(v, 32) : 0;
        return lo > hi ? lo : hi;
    }
}

template <int TW = kWave>
NR_DEV int32_t wave_inclusive_min(int32_t v, int lane) {
#pragma unroll
    for (int d = 1; d < TW; d <<= 1) {
        const int32_t o = __shfl_up(v, (unsigned)d, TW);
        if (lane >= d) v = v < o ? v : o;
    }
    return v;
}

// ---------------------------------------------------------------------------
// threefry2x32 (Random123 Threefry-2x32-20) and JAX's key plumbing in
// partitionable mode: fold_in(k, d) = split(k)[d] = threefry(k, (0, d)).
// ---------------------------------------------------------------------------
NR_DEV uint32_t rotl(uint32_t x, uint32_t d) { return (x << d) | (x >> (32u - d)); }
NR_DEV void threefry(uint32_t k0, uint32_t k1, uint32_t& x0, uint32_t& x1) {
    const uint32_t k2 = k0 ^ k1 ^ 0x1BD11BDAu;
    x0 += k0;
    x1 += k1;
#define NR_R(r)          \
    x0 += x1;            \
    x1 = rotl(x1, r);    \
    x1 ^= x0;
    NR_R(13) NR_R(15) NR_R(26) NR_R(6) x0 += k1; x1 += k2 + 1u;
    NR_R(17) NR_R(29) NR_R(16) NR_R(24) x0 += k2; x1 += k0 + 2u;
    NR_R(13) NR_R(15) NR_R(26) NR_R(6) x0 += k0; x1 += k1 + 3u;
    NR_R(17) NR_R(29) NR_R(16) NR_R(24) x0 += k1; x1 += k2 + 4u;
    NR_R(13) NR_R(15) NR_R(26) NR_R(6) x0 += k2; x1 += k0 + 5u;
#undef NR_R
}
NR_DEV void fold_in(uint32_t& k0, uint32_t& k1, uint32_t data) {
    uint32_t x0 = 0u, x1 = data;
    threefry(k0, k1, x0, x1);
    k0 = x0;
    k1 = x1;
}
// jax.random.randint(k, (), 0, 2) = (b0 ^ b1) % 2 with (b0, b1) =
// threefry(split(k)[1], (0, 0)) (N/core/cuda/conflict_draw.cuh:47-55 restates it).
NR_DEV int32_t randint01(uint32_t k0, uint32_t k1) {
    uint32_t s0 = 0u, s1 = 1u;
    threefry(k0, k1, s0, s1);
    uint32_t b0 = 0u, b1 = 0u;
    threefry(s0, s1, b0, b1);
    return (int32_t)((b0 ^ b1) & 1u);
}
// The "drawn" seat rule's learner for an episode root (N/bots/seat.py:352-360):
// randint(fold_in(root, 2**32 - 2), (), 0, 2).
NR_DEV int32_t episode_seat(uint32_t k0, uint32_t k1) {
    fold_in(k0, k1, 0xFFFFFFFEu);
    return randint01(k0, k1);
}

// ---------------------------------------------------------------------------
// LDS views
// ---------------------------------------------------------------------------
struct Hdr {
    AS3 int32_t* tab;
    AS3 uint8_t* terrain;
    AS3 Seg* seg;
    AS3 uint32_t* disk;
    AS3 uint32_t* walls;
};

struct Env {
    AS3 uint8_t* base;
    AS3 int32_t* birth;
    AS3 int32_t* carried;
    AS3 int32_t* pnone;
    AS3 int32_t* pissued;
    AS3 int32_t* pcompl;
    AS3 int32_t* porder;
    AS3 int16_t* cell;
    AS3 int16_t* hp;
    AS3 int16_t* ptarget;
    AS3 int16_t* entity;
    AS3 int8_t* utype;
    AS3 int8_t* owner;
    AS3 int8_t* pkind;
    AS3 int8_t* pdir;
    AS3 int8_t* pptype;
    AS3 int32_t* sc;
};

NR_DEV Env env_view(const KGame& g, AS3 uint8_t* base) {
    const Layout& y = g.lay;
    Env e;
    e.base = base;
    e.birth = (AS3 int32_t*)(base + y.o_birth);
    e.carried = (AS3 int32_t*)(base + y.o_carried);
    e.pnone = (AS3 int32_t*)(base + y.o_pnone);
    e.pissued = (AS3 int32_t*)(base + y.o_pissued);
    e.pcompl = (AS3 int32_t*)(base + y.o_pcompl);
    e.porder = (AS3 int32_t*)(base + y.o_porder);
    e.cell = (AS3 int16_t*)(base + y.o_cell);
    e.hp = (AS3 int16_t*)(base + y.o_hp);
    e.ptarget = (AS3 int16_t*)(base + y.o_ptarget);
    e.entity = (AS3 int16_t*)(base + y.o_entity);
    e.utype = (AS3 int8_t*)(base + y.o_utype);
    e.owner = (AS3 int8_t*)(base + y.o_owner);
    e.pkind = (AS3 int8_t*)(base + y.o_pkind);
    e.pdir = (AS3 int8_t*)(base + y.o_pdir);
    e.pptype = (AS3 int8_t*)(base + y.o_pptype);
    e.sc = (AS3 int32_t*)(base + y.o_scal);
    return e;
}

// Rebuild the view from an opaque copy of the base so the per-lane
// addresses derived from it are recomputed in each phase instead of staying
// live (in registers) across the whole step.
template <int TW = kWave>
NR_DEV Env refresh(const KGame& g, const Env& e) {
    uint32_t b = (uint32_t)(uintptr_t)e.base;
    // a half-wave team's block base differs between the halves
    if constexpr (TW == kWave) asm volatile("" : "+s"(b));
    else asm volatile("" : "+v"(b));
    return env_view(g, (AS3 uint8_t*)(uintptr_t)b);
}

// The game read again from the kernel-argument segment, where a kernel that
// takes KGame as its first argument finds it at offset 0.  Fields used after
// this call are reloaded (scalar loads) instead of being kept live in scalar
// registers across a whole kernel, which would spill them to vector lanes.
typedef const __attribute__((address_space(4))) KGame* KGameArg;
NR_DEV const KGame& fresh_game() {
    KGameArg p = (KGameArg)__builtin_amdgcn_kernarg_segment_ptr();
    asm volatile("" : "+s"(p));
    return *(const KGame*)p;
}

template <typename T>
NR_DEV AS3 T* at(const Env& e, int32_t offset) {
    return (AS3 T*)(e.base + offset);
}

NR_DEV int32_t tabv(const Hdr& h, int field, int32_t type) { return h.tab[field * 8 + type]; }

// Stage the unit table and terrain for the workgroup (all threads call; a
// __syncthreads follows in the kernel).
// One entry of the LDS unit table from the reference's `table` and `timings`
// operands (src/nanorts/core/unit_tables.py:9-48): table[t] = can_move,
// can_harvest, is_resource, is_stockpile, can_attack, attack_range, cost,
// produces[T]; timings[t] = move_time, harvest_time, attack_time,
// produce_time, hit_points, attack_damage, harvest_amount.  The step reads no
// sight radius, so F_SIGHT is 0; the legality targets pass no timings, whose
// fields are then 0.
NR_DEV int32_t ref_table_entry(const KGame& g, const int32_t* table, const int32_t* timings, int field, int32_t t) {
    if (t >= g.T) return 0;
    const int32_t* row = table + t * (7 + g.T);
    const int32_t* time = timings ? timings + t * 7 : nullptr;
    switch (field) {
        case F_COST: return row[6];
        case F_HP: return time ? time[4] : 0;
        case F_PRODUCE_TIME: return time ? time[3] : 0;
        case F_MOVE_TIME: return time ? time[0] : 0;
        case F_ATTACK_TIME: return time ? time[2] : 0;
        case F_HARVEST_TIME: return time ? time[1] : 0;
        case F_RANGE: return row[5];
        case F_DAMAGE: return time ? time[5] : 0;
        case F_AMOUNT: return time ? time[6] : 0;
        case F_FLAGS:
            return (row[2] ? FL_RESOURCE : 0) | (row[3] ? FL_STOCKPILE : 0) | (row[1] ? FL_HARVEST : 0) |
                   (row[0] ? FL_MOVE : 0) | (row[4] ? FL_ATTACK : 0);
        case F_PRODUCES: {
            int32_t bits = 0;
            for (int32_t u = 0; u < g.T; ++u) bits |= row[7 + u] ? 1 << u : 0;
            return bits;
        }
        default: return 0;
    }
}

NR_DEV int32_t table_entry(const KGame& g, const int32_t* table, const int32_t* timings, int field, int32_t t) {
    return table ? ref_table_entry(g, table, timings, field, t) : g.tab[field * 8 + t];
}

// The LDS unit table from the whole-act bots' `table` operand [T][6]
// (src/nanorts/bots/whole_act.py:33-40: can_harvest, is_resource,
// is_stockpile, can_attack, attack_range, cost) or from the GridNet decode's
// `unit_cost` [T] (cols = 1): the fields those targets read, the others 0.
// Called by every thread of the workgroup after load_header and before its
// barrier; each thread rewrites the entries it wrote.
NR_DEV void load_operand_table(const KGame& g, const Hdr& h, const int32_t* rows, int32_t cols) {
    for (int i = threadIdx.x; i < F_COUNT * 8; i += blockDim.x) {
        const int field = i >> 3, t = i & 7;
        int32_t v = 0;
        if (t < g.T) {
            const int32_t* row = rows + t * cols;
            const int32_t flags = cols == 6 ? ((row[1] ? FL_RESOURCE : 0) | (row[2] ? FL_STOCKPILE : 0) |
                                               (row[0] ? FL_HARVEST : 0) | (row[3] ? FL_ATTACK : 0))
                                            : 0;
            const int32_t range = cols == 6 ? row[4] : 0;
            const int32_t cost = cols == 6 ? row[5] : row[0];
            v = field == F_COST ? cost
                : field == F_RANGE ? range
                : field == F_FLAGS ? flags
                : field == F_PACK ? ((flags & 0xFF) | (range << 16))
                : 0;
        }
        h.tab[i] = v;
    }
}

// `table` / `timings`: the reference's operands (see ref_table_entry), or
// NULL for the game's own table.
NR_DEV void load_header(const KGame& g, const Hdr& h, const uint8_t* terrain, const int32_t* table,
                        const int32_t* timings) {
    for (int i = threadIdx.x; i < F_COUNT * 8; i += blockDim.x) {
        const int field = i >> 3, t = i & 7;
        h.tab[i] = field == F_PACK ? (table_entry(g, table, timings, F_FLAGS, t) & 0xFF) |
                                         ((table_entry(g, table, timings, F_PRODUCES, t) & 0xFF) << 8) |
                                         (table_entry(g, table, timings, F_RANGE, t) << 16)
                                   : table_entry(g, table, timings, field, t);
    }
    if (threadIdx.x == 0) {
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            h.seg[k].src = g.seg[k].src;
            h.seg[k].dst = g.seg[k].dst;
            h.seg[k].bytes = g.seg[k].bytes;
        }
    }
    // (a NULL terrain, for a target that reads none, stages an open board)
    for (int i = threadIdx.x; i < g.cells; i += blockDim.x) h.terrain[i] = (terrain && terrain[i]) ? 1 : 0;
    if (g.fast_obs) {
        // the walls as bitmap rows, the blocked plane every cycle starts
        // from, packed from the terrain copy four cells per LDS read (W % 4
        // == 0 keeps every row 4-byte aligned); every thread of the block
        // calls this, so the barrier is safe
        __syncthreads();
        for (int i = threadIdx.x; i < g.H * g.seen_words; i += blockDim.x) {
            const int32_t row = i / g.seen_words, x0 = 32 * (i - row * g.seen_words);
            const int32_t n = g.W - x0 < 32 ? g.W - x0 : 32;
            AS3 const uint32_t* cells = (AS3 const uint32_t*)(h.terrain + row * g.W + x0);
            uint32_t bits = 0u;
            for (int32_t q = 0; q < (n >> 2); ++q) {
                const uint32_t v = cells[q];  // one 0/1 byte per cell
                bits |= ((v & 1u) | ((v >> 7) & 2u) | ((v >> 14) & 4u) | ((v >> 21) & 8u)) << (4 * q);
            }
            h.walls[i] = bits;
        }
        // disk[r][dy + R]: bits R - w .. R + w with w = floor(sqrt(r^2 - dy^2)),
        // 0 when |dy| > r (R = disk_r <= 15)
        const int32_t R = g.disk_r, span = 2 * R + 1;
        for (int i = threadIdx.x; i < (R + 1) * span; i += blockDim.x) {
            const int32_t r = i / span, dy = i - r * span - R;
            uint32_t m = 0u;
            if (dy * dy <= r * r) {
                int32_t w = r;
                while (w * w > r * r - dy * dy) --w;
                m = ((2u << (2 * w)) - 1u) << (R - w);
            }
            h.disk[i] = m;
        }
    }
}
NR_DEV void load_header(const KGame& g, const Hdr& h) { load_header(g, h, g.terrain, g.ref_table, g.ref_timings); }

// ---------------------------------------------------------------------------
// HBM <-> LDS row copies (16-byte, 4-byte or 1-byte granules by alignment)
// ---------------------------------------------------------------------------
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <int TW = kWave>
NR_DEV void copy_in(AS3 uint8_t* dst, const uint8_t* src, int32_t nbytes, int lane) {
    const uintptr_t a = (uintptr_t)src;
    if (((a | (uintptr_t)nbytes) & 15u) == 0) {
        const int32_t n = nbytes >> 4;
        for (int32_t i = lane; i < n; i += TW) ((AS3 u32x4*)dst)[i] = ((const u32x4*)src)[i];
    } else if (((a | (uintptr_t)nbytes) & 3u) == 0) {
        const int32_t n = nbytes >> 2;
        for (int32_t i = lane; i < n; i += TW) ((AS3 uint32_t*)dst)[i] = ((const uint32_t*)src)[i];
    } else {
        for (int32_t i = lane; i < nbytes; i += TW) dst[i] = src[i];
    }
}

template <int TW = kWave>
NR_DEV void copy_out(uint8_t* dst, const AS3 uint8_t* src, int32_t nbytes, int lane) {
    const uintptr_t a = (uintptr_t)dst;
    if (((a | (uintptr_t)nbytes) & 15u) == 0) {
        const int32_t n = nbytes >> 4;
        for (int32_t i = lane; i < n; i += TW) ((u32x4*)dst)[i] = ((const AS3 u32x4*)src)[i];
    } else if (((a | (uintptr_t)nbytes) & 3u) == 0) {
        const int32_t n = nbytes >> 2;
        for (int32_t i = lane; i < n; i += TW) ((uint32_t*)dst)[i] = ((const AS3 uint32_t*)src)[i];
    } else {
        for (int32_t i = lane; i < nbytes; i += TW) dst[i] = src[i];
    }
}

// Which leaves a kernel needs staged.
enum : uint32_t {
    LD_BIRTH = 1u << 0,
    LD_UTYPE = 1u << 1,
    LD_OWNER = 1u << 2,
    LD_CELL = 1u << 3,
    LD_HP = 1u << 4,
    LD_CARRIED = 1u << 5,
    LD_PKIND = 1u << 6,
    LD_PDIR = 1u << 7,
    LD_PNONE = 1u << 8,
    LD_PTARGET = 1u << 9,
    LD_PPTYPE = 1u << 10,
    LD_PISSUED = 1u << 11,
    LD_PCOMPL = 1u << 12,
    LD_PORDER = 1u << 13,
    LD_ENTITY = 1u << 14,
    LD_SCALARS = 1u << 15,
    LD_ALL = 0xFFFFu,
};

// The staged leaves: flag, State field, Env member, element type, count.
#define NR_LEAVES(X)                                                   \
    X(LD_BIRTH, birth, birth, int32_t, E)                              \
    X(LD_UTYPE, unit_type, utype, int8_t, E)                           \
    X(LD_OWNER, owner, owner, int8_t, E)                               \
    X(LD_CELL, cell, cell, int16_t, E)                                 \
    X(LD_HP, hit_points, hp, int16_t, E)                               \
    X(LD_CARRIED, carried_resources, carried, int32_t, E)              \
    X(LD_PKIND, pending_kind, pkind, int8_t, E)                        \
    X(LD_PDIR, pending_direction, pdir, int8_t, E)                     \
    X(LD_PNONE, pending_none_duration, pnone, int32_t, E)              \
    X(LD_PTARGET, pending_target_cell, ptarget, int16_t, E)            \
    X(LD_PPTYPE, pending_produced_type, pptype, int8_t, E)             \
    X(LD_PISSUED, pending_issued_at, pissued, int32_t, E)              \
    X(LD_PCOMPL, pending_completes_at, pcompl, int32_t, E)             \
    X(LD_PORDER, pending_order, porder, int32_t, E)                    \
    X(LD_ENTITY, entity_at, entity, int16_t, cells)

// The per-env scalars of row l into the block's scalar leaf (lanes below
// S_COUNT, one scalar each).
NR_DEV void load_scalars(const nanorts_state& s, int64_t l, const Env& e, int lane) {
    if (lane >= S_COUNT) return;
    int32_t v = 0;
    switch (lane) {
        case S_TIME: v = s.time[l]; break;
        case S_RES0: v = s.player_resources[2 * l]; break;
        case S_RES1: v = s.player_resources[2 * l + 1]; break;
        case S_NEXT_BIRTH: v = s.next_birth[l]; break;
        case S_NEXT_ORDER: v = s.next_pending_order[l]; break;
        case S_ALT: v = s.alternating_conflict_count[l]; break;
        case S_GAME_OVER: v = s.game_over[l] ? 1 : 0; break;
        case S_WINNER: v = s.winner[l]; break;
        case S_SO0: v = s.spawn_overflow[2 * l]; break;
        case S_SO1: v = s.spawn_overflow[2 * l + 1]; break;
        case S_ROOT0: v = s.environment_root ? (int32_t)s.environment_root[2 * l] : 0; break;
        case S_ROOT1: v = s.environment_root ? (int32_t)s.environment_root[2 * l + 1] : 0; break;
        case S_EPISODE: v = s.episode_index ? (int32_t)s.episode_index[l] : 0; break;
        case S_VISDIRTY: v = 3; break;
        default: break;
    }
    e.sc[lane] = v;
}

// The block's scalars into row l of the state.
NR_DEV void store_scalars(const nanorts_state& s, int64_t l, const Env& e, int lane) {
    if (lane >= S_COUNT) return;
    const int32_t v = e.sc[lane];
    switch (lane) {
        case S_TIME: s.time[l] = v; break;
        case S_RES0: s.player_resources[2 * l] = v; break;
        case S_RES1: s.player_resources[2 * l + 1] = v; break;
        case S_NEXT_BIRTH: s.next_birth[l] = v; break;
        case S_NEXT_ORDER: s.next_pending_order[l] = v; break;
        case S_ALT: s.alternating_conflict_count[l] = v; break;
        case S_GAME_OVER: s.game_over[l] = v ? 1 : 0; break;
        case S_WINNER: s.winner[l] = v; break;
        case S_SO0: s.spawn_overflow[2 * l] = v; break;
        case S_SO1: s.spawn_overflow[2 * l + 1] = v; break;
        case S_EPISODE:
            if (s.episode_index) s.episode_index[l] = (uint32_t)v;
            break;
        default: break;
    }
}

// Leaves of at most 1024 bytes (one 16-byte vector per lane), 16-byte
// aligned: every requested leaf is loaded into registers before the first
// LDS store, so the wave waits on memory once instead of once per leaf.
// False (nothing done) when a leaf does not qualify.
template <int TW = kWave>
NR_DEV bool load_leaves_batched(const KGame& g, const nanorts_state& s, int64_t l, const Env& e, uint32_t which,
                                int lane) {
    const int64_t E = g.E, cells = g.cells;
    uint64_t bad = 0u;
#define NR_CHECK(flag, field, member, type, count)                                                 \
    if (which & flag) {                                                                            \
        const int64_t bytes = count * (int64_t)sizeof(type);                                       \
        bad |= ((uint64_t)(uintptr_t)(s.field + l * count) | (uint64_t)bytes) & 15u;               \
        if (bytes > 16 * TW) bad |= 1u;                                                         \
    }
    NR_LEAVES(NR_CHECK)
#undef NR_CHECK
    if (bad != 0u) return false;
#define NR_LOAD(flag, field, member, type, count)                                                  \
    u32x4 v_##member = {0u, 0u, 0u, 0u};                                                           \
    const int32_t n_##member = (int32_t)((count * (int64_t)sizeof(type)) >> 4);                    \
    if ((which & flag) && lane < n_##member) v_##member = ((const u32x4*)(s.field + l * count))[lane];
    NR_LEAVES(NR_LOAD)
#undef NR_LOAD
#define NR_STORE(flag, field, member, type, count) \
    if ((which & flag) && lane < n_##member) ((AS3 u32x4*)e.member)[lane] = v_##member;
    NR_LEAVES(NR_STORE)
#undef NR_STORE
    return true;
}

template <int TW = kWave>
NR_DEV void load_env(const KGame& g, const nanorts_state& s, int64_t l, const Env& e, uint32_t which, int lane) {
    const int64_t E = g.E, cells = g.cells;
    if (load_leaves_batched<TW>(g, s, l, e, which, lane)) which &= ~(uint32_t)(LD_SCALARS - 1u);
#define NR_IN(flag, field, member, type) \
    if (which & flag) copy_in<TW>((AS3 uint8_t*)e.member, (const uint8_t*)(s.field + l * E), (int32_t)(E * sizeof(type)), lane);
    NR_IN(LD_BIRTH, birth, birth, int32_t)
    NR_IN(LD_UTYPE, unit_type, utype, int8_t)
    NR_IN(LD_OWNER, owner, owner, int8_t)
    NR_IN(LD_CELL, cell, cell, int16_t)
    NR_IN(LD_HP, hit_points, hp, int16_t)
    NR_IN(LD_CARRIED, carried_resources, carried, int32_t)
    NR_IN(LD_PKIND, pending_kind, pkind, int8_t)
    NR_IN(LD_PDIR, pending_direction, pdir, int8_t)
    NR_IN(LD_PNONE, pending_none_duration, pnone, int32_t)
    NR_IN(LD_PTARGET, pending_target_cell, ptarget, int16_t)
    NR_IN(LD_PPTYPE, pending_produced_type, pptype, int8_t)
    NR_IN(LD_PISSUED, pending_issued_at, pissued, int32_t)
    NR_IN(LD_PCOMPL, pending_completes_at, pcompl, int32_t)
    NR_IN(LD_PORDER, pending_order, porder, int32_t)
#undef NR_IN
    if (which & LD_ENTITY)
        copy_in<TW>((AS3 uint8_t*)e.entity, (const uint8_t*)(s.entity_at + l * cells), (int32_t)(cells * 2), lane);
    if (which & LD_SCALARS) load_scalars(s, l, e, lane);
    wave_sync();
}

// store_env's counterpart of load_leaves_batched: every leaf is read from
// LDS before the first global store.  False (nothing done) when a leaf does
// not qualify.
template <int TW = kWave>
NR_DEV bool store_leaves_batched(const KGame& g, const nanorts_state& s, int64_t l, const Env& e, int lane) {
    const int64_t E = g.E, cells = g.cells;
    uint64_t bad = 0u;
#define NR_CHECK(flag, field, member, type, count)                                                 \
    {                                                                                              \
        const int64_t bytes = count * (int64_t)sizeof(type);                                       \
        bad |= ((uint64_t)(uintptr_t)(s.field + l * count) | (uint64_t)bytes) & 15u;               \
        if (bytes > 16 * TW) bad |= 1u;                                                         \
    }
    NR_LEAVES(NR_CHECK)
#undef NR_CHECK
    if (bad != 0u) return false;
#define NR_READ(flag, field, member, type, count)                                                  \
    u32x4 v_##member = {0u, 0u, 0u, 0u};                                                           \
    const int32_t n_##member = (int32_t)((count * (int64_t)sizeof(type)) >> 4);                    \
    if (lane < n_##member) v_##member = ((const AS3 u32x4*)e.member)[lane];
    NR_LEAVES(NR_READ)
#undef NR_READ
#define NR_WRITE(flag, field, member, type, count) \
    if (lane < n_##member) ((u32x4*)(s.field + l * count))[lane] = v_##member;
    NR_LEAVES(NR_WRITE)
#undef NR_WRITE
    return true;
}

template <int TW = kWave>
NR_DEV void store_env(const KGame& g, const nanorts_state& s, int64_t l, const Env& e, int lane) {
    const int64_t E = g.E, cells = g.cells;
    const bool batched = store_leaves_batched<TW>(g, s, l, e, lane);
#define NR_OUT(field, member, type) \
    if (!batched) copy_out<TW>((uint8_t*)(s.field + l * E), (const AS3 uint8_t*)e.member, (int32_t)(E * sizeof(type)), lane);
    NR_OUT(birth, birth, int32_t)
    NR_OUT(unit_type, utype, int8_t)
    NR_OUT(owner, owner, int8_t)
    NR_OUT(cell, cell, int16_t)
    NR_OUT(hit_points, hp, int16_t)
    NR_OUT(carried_resources, carried, int32_t)
    NR_OUT(pending_kind, pkind, int8_t)
    NR_OUT(pending_direction, pdir, int8_t)
    NR_OUT(pending_none_duration, pnone, int32_t)
    NR_OUT(pending_target_cell, ptarget, int16_t)
    NR_OUT(pending_produced_type, pptype, int8_t)
    NR_OUT(pending_issued_at, pissued, int32_t)
    NR_OUT(pending_completes_at, pcompl, int32_t)
    NR_OUT(pending_order, porder, int32_t)
#undef NR_OUT
    if (!batched) copy_out<TW>((uint8_t*)(s.entity_at + l * cells), (const AS3 uint8_t*)e.entity, (int32_t)(cells * 2), lane);
    store_scalars(s, l, e, lane);
}

// ---------------------------------------------------------------------------
// Slot-window copies (KGame::shift > 0): block slot i <-> state slot
// glob_slot(i), and the occupancy grid's slot numbers mapped the same way.
// A state row holds E + 2 shift slots.
// ---------------------------------------------------------------------------
// Row l of `s` into the block (l = 0 with the initial state).  False when
// the game does not fit the window: a live slot in either gap, or an
// occupancy entry other than -1 or a slot inside the window (the block is
// then partly written and must not run).
template <int TW = kWave>
NR_DEV bool load_window_rows(const KGame& g, const nanorts_state& s, int64_t l, const Env& e, int lane) {
    const int32_t N = g.N, C = g.C, E = g.E, sh = g.shift;
    const int64_t row = l * (int64_t)(E + 2 * sh);
    bool bad = false;
    for (int32_t i = lane; i < E; i += TW) {
        // every leaf's load first, then the LDS stores
        const int64_t at = row + glob_slot(g, i);
        const int32_t birth = s.birth[at], carried = s.carried_resources[at], pnone = s.pending_none_duration[at];
        const int32_t pissued = s.pending_issued_at[at], pcompl = s.pending_completes_at[at];
        const int32_t porder = s.pending_order[at];
        const int16_t cell = s.cell[at], hp = s.hit_points[at], ptarget = s.pending_target_cell[at];
        const int8_t utype = s.unit_type[at], owner = s.owner[at], pkind = s.pending_kind[at];
        const int8_t pdir = s.pending_direction[at], pptype = s.pending_produced_type[at];
        e.birth[i] = birth;
        e.carried[i] = carried;
        e.pnone[i] = pnone;
        e.pissued[i] = pissued;
        e.pcompl[i] = pcompl;
        e.porder[i] = porder;
        e.cell[i] = cell;
        e.hp[i] = hp;
        e.ptarget[i] = ptarget;
        e.utype[i] = utype;
        e.owner[i] = owner;
        e.pkind[i] = pkind;
        e.pdir[i] = pdir;
        e.pptype[i] = pptype;
    }
    // the gaps [N + C, N + C + sh) and [E + sh, E + 2 sh) hold no live slot
    for (int32_t i = lane; i < 2 * sh; i += TW) {
        const int32_t gs = i < sh ? N + C + i : E + i;
        if (s.birth[row + gs] != kAbsent) bad = true;
    }
    for (int32_t c = lane; c < g.cells; c += TW) {
        const int32_t v = s.entity_at[l * (int64_t)g.cells + c];
        int32_t lv = v;
        if (v >= N + C + sh && v < E + sh) lv = v - sh;
        else if (v < -1 || v >= N + C) bad = true;
        e.entity[c] = (int16_t)lv;
    }
    return tballot<TW>(bad) == 0ull;
}

// Whether the initial state fits the window (load_window_rows' test alone).
template <int TW = kWave>
NR_DEV bool initial_fits_window(const KGame& g, int lane) {
    const nanorts_state& s = g.initial;
    const int32_t N = g.N, C = g.C, E = g.E, sh = g.shift;
    bool bad = false;
    for (int32_t i = lane; i < 2 * sh; i += TW) {
        const int32_t gs = i < sh ? N + C + i : E + i;
        if (s.birth[gs] != kAbsent) bad = true;
    }
    for (int32_t c = lane; c < g.cells; c += TW) {
        const int32_t v = s.entity_at[c];
        if (!(v >= N + C + sh && v < E + sh) && (v < -1 || v >= N + C)) bad = true;
    }
    return tballot<TW>(bad) == 0ull;
}

// The block into row l of the state: the window's slots and the occupancy
// grid, its slot numbers mapped back.
template <int TW = kWave>
NR_DEV void store_window_rows(const KGame& g, const nanorts_state& s, int64_t l, const Env& e, int lane) {
    const int32_t N = g.N, C = g.C, E = g.E, sh = g.shift;
    const int64_t row = l * (int64_t)(E + 2 * sh);
    for (int32_t i = lane; i < E; i += TW) {
        const int32_t birth = e.birth[i], carried = e.carried[i], pnone = e.pnone[i], pissued = e.pissued[i];
        const int32_t pcompl = e.pcompl[i], porder = e.porder[i];
        const int16_t cell = e.cell[i], hp = e.hp[i], ptarget = e.ptarget[i];
        const int8_t utype = e.utype[i], owner = e.owner[i], pkind = e.pkind[i], pdir = e.pdir[i];
        const int8_t pptype = e.pptype[i];
        const int64_t at = row + glob_slot(g, i);
        s.birth[at] = birth;
        s.carried_resources[at] = carried;
        s.pending_none_duration[at] = pnone;
        s.pending_issued_at[at] = pissued;
        s.pending_completes_at[at] = pcompl;
        s.pending_order[at] = porder;
        s.cell[at] = cell;
        s.hit_points[at] = hp;
        s.pending_target_cell[at] = ptarget;
        s.unit_type[at] = utype;
        s.owner[at] = owner;
        s.pending_kind[at] = pkind;
        s.pending_direction[at] = pdir;
        s.pending_produced_type[at] = pptype;
    }
    for (int32_t c = lane; c < g.cells; c += TW) {
        const int32_t v = e.entity[c];
        s.entity_at[l * (int64_t)g.cells + c] = (int16_t)(v >= N + C ? v + sh : v);
    }
    store_scalars(s, l, e, lane);
}

// ---------------------------------------------------------------------------
// board helpers (N/core/board.py)
// ---------------------------------------------------------------------------
struct Nb {
    bool free, occupied;
    int32_t slot, unit_type, owner;
};

// N/core/board.py:23-56
NR_DEV Nb neighbour(const KGame& g, const Hdr& h, const Env& e, int32_t cell, int32_t direction) {
    const int32_t x = cell_x(g, cell), y = cell_y(g, cell);
    const int32_t known = clampi(direction, 0, 3);
    const int32_t nx = x + dir_dx(known), ny = y + dir_dy(known);
    const bool on = direction >= 0 && direction < 4 && nx >= 0 && nx < g.W && ny >= 0 && ny < g.H;
    Nb n;
    n.free = false;
    n.occupied = false;
    n.slot = 0;
    n.unit_type = 0;
    n.owner = kAbsent;
    if (on) {
        const int32_t nc = ny * g.W + nx;
        const int32_t occ = e.entity[nc];
        n.occupied = occ != kAbsent;
        n.free = !n.occupied && h.terrain[nc] == 0;
        if (n.occupied) {
            n.slot = occ;
            const int32_t s = gidx(occ, g.E);
            n.unit_type = clampi(e.utype[s], 0, g.T - 1);
            n.owner = e.owner[s];
        }
    }
    return n;
}

// N/core/board.py:59-64 (no bounds check; may wrap rows)
NR_DEV int32_t reserved_position(const KGame& g, int32_t cell, int32_t direction) {
    const int32_t known = clampi(direction, 0, 3);
    return wadd(cell, dir_dx(known) + dir_dy(known) * g.W);
}

// N/core/admission.py:310-319 with each kind's duration.
NR_DEV int32_t action_duration(const KGame& g, const Hdr& h, int32_t actor_type, int32_t kind, int32_t none_duration,
                               int32_t produced_type) {
    const int32_t actor = clampi(actor_type, 0, g.T - 1);
    switch (kind) {
        case kKindNone: return none_duration;
        case kKindMove: return tabv(h, F_MOVE_TIME, actor);
        case kKindHarvest: return tabv(h, F_HARVEST_TIME, actor);
        case kKindReturn: return tabv(h, F_MOVE_TIME, actor);
        case kKindProduce: return tabv(h, F_PRODUCE_TIME, clampi(produced_type, 0, g.T - 1));
        case kKindAttack: return tabv(h, F_ATTACK_TIME, actor);
        default: return 0;
    }
}

NR_DEV bool claims_position(int32_t kind) { return kind == kKindMove || kind == kKindProduce; }

// ---------------------------------------------------------------------------
// Command canonical forms.  Only these properties of a command's int32
// fields are ever observed by the reference's step, so each is stored in a
// narrow form that preserves them:
//   kind: -1 absent, 0..5, or 6 for any other value (no duration, never legal)
//   direction: -1 for d < 0, 4 for d > 3 (is_direction false, clip as d)
//   produced_type: -1 below range, T above (range check false, clip as v)
//   target_cell: -1 off the board (never a legal target, never stored)
// ---------------------------------------------------------------------------
NR_DEV int32_t canon_kind(int32_t k) { return k == kAbsent ? kAbsent : ((k >= 0 && k <= 5) ? k : kKindUnknown); }
NR_DEV int32_t canon_dir(int32_t d) { return d < 0 ? -1 : (d > 3 ? 4 : d); }
NR_DEV int32_t canon_ptype(int32_t t, int32_t T) { return t < 0 ? -1 : (t >= T ? T : t); }
NR_DEV int32_t canon_target(int32_t c, int32_t cells) { return (c >= 0 && c < cells) ? c : -1; }

// N/core/kinds/*.py is_valid for one request (Request.of, action_kind.py:15-40).
NR_DEV bool can_execute(const KGame& g, const Hdr& h, const Env& e, int32_t slot, int32_t kind, int32_t dir,
                        int32_t target, int32_t ptype) {
    const int32_t actor = clampi(e.utype[slot], 0, g.T - 1);
    const int32_t owner = e.owner[slot];
    const int32_t carried = e.carried[slot];
    const int32_t cell = e.cell[slot];
    const int32_t flags = tabv(h, F_FLAGS, actor);
    switch (kind) {
        case kKindNone: return true;
        case kKindMove: {
            const Nb n = neighbour(g, h, e, cell, dir);
            return (flags & FL_MOVE) && n.free;
        }
        case kKindHarvest: {
            const Nb n = neighbour(g, h, e, cell, dir);
            return (flags & FL_HARVEST) && carried == 0 && n.occupied && (tabv(h, F_FLAGS, n.unit_type) & FL_RESOURCE);
        }
        case kKindReturn: {
            const Nb n = neighbour(g, h, e, cell, dir);
            return (flags & FL_HARVEST) && carried > 0 && n.occupied && (tabv(h, F_FLAGS, n.unit_type) & FL_STOCKPILE) &&
                   n.owner == owner;
        }
        case kKindProduce: {
            if (ptype < 0 || ptype >= g.T) return false;
            const Nb n = neighbour(g, h, e, cell, dir);
            const int32_t balance = e.sc[S_RES0 + clampi(owner, 0, 1)];
            return ((tabv(h, F_PRODUCES, actor) >> ptype) & 1) && balance >= tabv(h, F_COST, ptype) && n.free;
        }
        case kKindAttack: {
            if (target < 0 || target >= g.cells) return false;
            const int32_t occ = e.entity[target];
            if (occ == kAbsent) return false;
            const int32_t target_owner = e.owner[gidx(occ, g.E)];
            const int32_t range = tabv(h, F_RANGE, actor);
            const int32_t dx = cell_x(g, target) - cell_x(g, cell);
            const int32_t dy = cell_y(g, target) - cell_y(g, cell);
            return (flags & FL_ATTACK) && target_owner >= 0 && target_owner != owner &&
                   wadd(wmul(dx, dx), wmul(dy, dy)) <= wmul(range, range);
        }
        default: return false;
    }
}

// ---------------------------------------------------------------------------
// Admission (N/core/admission.py, N/core/pending.py:28-44,
// N/core/reservations.py)
// ---------------------------------------------------------------------------
struct Events {
    bool enabled;
};

// Request order and pending ranking for this cycle.  Returns the number of
// issued requests; region B holds `order` (owned positions in admission
// order) and `rank` (pending entries in ranking order, count in *n_rank).
NR_DEV int32_t order_requests(const KGame& g, const Env& e, int lane, int32_t* n_rank_out) {
    const Layout& y = g.lay;
    const int32_t N = g.N, C = g.C, owned = 2 * C;
    AS3 int8_t* ckind = at<int8_t>(e, y.c_kind);
    AS3 int16_t* crank = at<int16_t>(e, y.c_rank);
    AS3 uint64_t* keys = at<uint64_t>(e, y.b_keys);
    AS3 int16_t* tmp = at<int16_t>(e, y.b_tmp);
    AS3 int16_t* order = at<int16_t>(e, y.b_order);
    AS3 int16_t* rank = at<int16_t>(e, y.b_rank);
    AS3 int32_t* pkey = at<int32_t>(e, y.b_pkey);

    // issued = active & kind != ABSENT, compacted in owned-position order,
    // keyed (player, rank, birth) as in _issued_player_rank_key (:224-234).
    int32_t n = 0;
    for (int32_t base = 0; base < owned; base += kWave) {
        const int32_t p = base + lane;
        bool issued = false;
        int32_t birth = 0;
        if (p < owned) {
            birth = e.birth[N + p];
            issued = birth != kAbsent && ckind[p] != kAbsent;
        }
        const uint64_t m = ballot(issued);
        if (issued) {
            const int32_t at_ = n + count_below(m);
            const uint32_t hi = ((uint32_t)(p / C) << g.rank_bits) | (uint32_t)crank[p];
            keys[at_] = ((uint64_t)hi << 32) | (uint64_t)((uint32_t)birth ^ 0x80000000u);
            tmp[at_] = (int16_t)p;
        }
        n += popc(m);
    }
    wave_sync();
    // rank by count; ties (impossible for distinct births) by owned position
    for (int32_t i = lane; i < n; i += kWave) {
        const uint64_t ki = keys[i];
        int32_t pos = 0;
        for (int32_t j = 0; j < n; ++j) {
            const uint64_t kj = keys[j];
            pos += (kj < ki) || (kj == ki && j < i);
        }
        order[pos] = tmp[i];
    }
    wave_sync();
    // pending keys after this cycle's appends (pending.py:37-44)
    for (int32_t p = lane; p < owned; p += kWave) {
        const int32_t held = e.porder[N + p];
        pkey[p] = held == kAbsent ? kNoCap : held;
    }
    wave_sync();
    const int32_t next_order = uni(e.sc[S_NEXT_ORDER]);
    int32_t appended = 0;
    for (int32_t base = 0; base < n; base += kWave) {
        const int32_t i = base + lane;
        bool appends = false;
        int32_t p = 0;
        if (i < n) {
            p = order[i];
            appends = e.porder[N + p] == kAbsent;
        }
        const uint64_t m = ballot(appends);
        if (appends) pkey[p] = wadd(next_order, appended + count_below(m));
        appended += popc(m);
    }
    wave_sync();
    // ranking: neutral pending entries first in slot order, then owned
    // entries by (key, position); entries that cannot be pending this cycle
    // (key INT_MAX and no pending action) are left out, which does not change
    // the relative order of the others.
    int32_t nr = 0;
    for (int32_t base = 0; base < N; base += kWave) {
        const int32_t s = base + lane;
        const bool pend = s < N && e.pkind[s] != kAbsent;
        const uint64_t m = ballot(pend);
        if (pend) rank[nr + count_below(m)] = (int16_t)s;
        nr += popc(m);
    }
    int32_t no = 0;
    for (int32_t base = 0; base < owned; base += kWave) {
        const int32_t p = base + lane;
        bool inc = false;
        int32_t k = 0;
        if (p < owned) {
            k = pkey[p];
            inc = k != kNoCap || e.pkind[N + p] != kAbsent;
        }
        const uint64_t m = ballot(inc);
        if (inc) {
            const int32_t at_ = no + count_below(m);
            keys[at_] = ((uint64_t)((uint32_t)k ^ 0x80000000u) << 32) | (uint64_t)(uint32_t)p;
            tmp[at_] = (int16_t)p;
        }
        no += popc(m);
    }
    wave_sync();
    for (int32_t i = lane; i < no; i += kWave) {
        const uint64_t ki = keys[i];
        int32_t pos = 0;
        for (int32_t j = 0; j < no; ++j) pos += keys[j] < ki;
        rank[nr + pos] = (int16_t)(N + tmp[i]);
    }
    wave_sync();
    *n_rank_out = nr + no;
    return n;
}

// One request: N/core/admission.py:242-289 (_admit_one) with
// reservations.resolve (N/core/reservations.py:69-111).
NR_DEV void admit_one(const KGame& g, const Hdr& h, const Env& e, int lane, int32_t p, int32_t n_rank, uint32_t key0,
                      uint32_t key1, bool count_events) {
    const Layout& y = g.lay;
    const int32_t slot = g.N + p;
    const int32_t player = p / g.C;
    const int32_t kind0 = uni(at<int8_t>(e, y.c_kind)[p]);
    const int32_t dir = uni(at<int8_t>(e, y.c_dir)[p]);
    const int32_t ptype = uni(at<int8_t>(e, y.c_ptype)[p]);
    const int32_t target = uni(at<int16_t>(e, y.c_target)[p]);
    const int32_t none0 = uni(at<int32_t>(e, y.c_none)[p]);
    const int32_t time = uni(e.sc[S_TIME]);
    const int32_t cell = uni(e.cell[slot]);
    const int32_t unit_type = uni(e.utype[slot]);
    const int32_t owner = uni(e.owner[slot]);

    const int32_t requested = action_duration(g, h, unit_type, kind0, none0, ptype);
    // _none_if_illegal
    const bool legal = uni(can_execute(g, h, e, slot, kind0, dir, target, ptype) ? 1 : 0) != 0;
    int32_t kind = legal ? kind0 : kKindNone;
    int32_t none = legal ? none0 : requested;
    // _none_if_blocked
    if (claims_position(kind)) {
        const int32_t pos = gidx(reserved_position(g, cell, dir), g.cells);
        if (h.terrain[pos] != 0 || e.entity[pos] != kAbsent) {
            kind = kKindNone;
            none = requested;
        }
    }
    // _count_admitted (:406-429)
    if (count_events && lane == 0) {
        AS3 int32_t* ev = at<int32_t>(e, y.b_events);
        if (kind == kKindHarvest) ev[player] += 1;
        if (kind == kKindReturn) ev[2 + player] += 1;
        if (kind == kKindProduce) ev[4 + player * 8 + clampi(ptype, 0, g.T - 1)] += 1;
        if (kind == kKindAttack) {
            const int32_t occ = e.entity[clampi(target, 0, g.cells - 1)];
            const int32_t towner = occ == kAbsent ? kAbsent : e.owner[clampi(occ, 0, g.E - 1)];
            if (towner + 1 >= 0 && towner + 1 < 3) ev[20 + player * 3 + towner + 1] += 1;
        }
    }
    // _requested_reservation (:340-349) and resolve
    const bool req_claims = claims_position(kind);
    const int32_t req_cost = kind == kKindProduce ? tabv(h, F_COST, clampi(ptype, 0, g.T - 1)) : 0;
    if (req_claims || req_cost != 0) {
        const int32_t req_pos = reserved_position(g, cell, dir);
        const int32_t req_player = clampi(owner, 0, 1);
        const int32_t balance = uni(e.sc[S_RES0 + req_player]);
        const int32_t alt = uni(e.sc[S_ALT]);
        AS3 int16_t* rank = at<int16_t>(e, y.b_rank);
        int32_t same_total = 0;
        bool any_cross = false;
        int32_t cap = kNoCap;
        uint32_t ek0 = key0, ek1 = key1;
        bool have_event_key = false;
        const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
        for (int32_t base = 0; base < n_rank; base += kWave) {
            const int32_t j = base + lane;
            bool same = false, cross = false;
            int32_t dur = 0, entry = 0;
            if (j < n_rank) {
                entry = rank[j];
                const int32_t k = e.pkind[entry];
                if (k != kAbsent) {
                    const int32_t epl = clampi(e.owner[entry], 0, 1);
                    const int32_t ept = e.pptype[entry];
                    const int32_t ecost = k == kKindProduce ? tabv(h, F_COST, clampi(ept, 0, g.T - 1)) : 0;
                    const bool eclaims = claims_position(k);
                    const int32_t epos = reserved_position(g, e.cell[entry], e.pdir[entry]);
                    const bool shared = eclaims && req_claims && epos == req_pos;
                    const int32_t claimed = wadd(epl == req_player ? ecost : 0, req_cost);
                    const bool over = req_cost != 0 && claimed > 0 && claimed > balance;
                    const bool conflict = shared || over;
                    const bool crossc = e.pissued[entry] != time;
                    const int32_t d = action_duration(g, h, e.utype[entry], k, e.pnone[entry], ept);
                    const int32_t packed = wadd(wmul(d, 4), (conflict && !crossc ? 2 : 0) + (conflict && crossc ? 1 : 0));
                    dur = packed >> 2;
                    same = ((packed >> 1) & 1) != 0;
                    cross = (packed & 1) != 0;
                }
            }
            const uint64_t sm = ballot(same), cm = ballot(cross);
            if ((sm | cm) == 0ull) continue;
            const int32_t same_before = same_total + popc(sm & below);
            const bool cross_before = any_cross || (cm & below) != 0ull;
            bool cancels_req = true, cancels_pend = true;
            if (g.strategy == NANORTS_CANCEL_ALTERNATING) {
                cancels_req = floor_mod(wadd(alt, same_before), 2) == 0;
                cancels_pend = !cancels_req;
            } else if (g.strategy == NANORTS_CANCEL_RANDOM) {
                if (!have_event_key && sm != 0ull) {
                    // _event_key (N/core/reservations.py:297-300)
                    fold_in(ek0, ek1, (uint32_t)time);
                    fold_in(ek0, ek1, (uint32_t)uni(e.birth[slot]));
                    fold_in(ek0, ek1, 0u);
                    have_event_key = true;
                }
                int32_t draw = 0;
                if (same) {
                    uint32_t d0 = ek0, d1 = ek1;
                    fold_in(d0, d1, (uint32_t)same_before);
                    draw = randint01(d0, d1);
                }
                cancels_req = draw == 0;
                cancels_pend = !cancels_req;
            }
            // _settle_durations (:169-192) for this chunk
            int32_t incl = wave_inclusive_min((same && cancels_req) ? dur : kNoCap, lane);
            incl = imin(incl, cap);
            int32_t excl = __shfl_up(incl, 1u, kWave);
            if (lane == 0) excl = cap;
            const int32_t before = cross_before ? -1 : imin(requested, excl);
            if (same && cancels_pend) {
                // _cancel_pending (:207-228)
                const int32_t settled = imin(dur, before);
                const int32_t d2 = wadd(wmul(settled, 2), 1) >> 1;
                e.pkind[entry] = (int8_t)kKindNone;
                e.pdir[entry] = (int8_t)kAbsent;
                e.pnone[entry] = d2;
                e.ptarget[entry] = (int16_t)kAbsent;
                e.pptype[entry] = (int8_t)kAbsent;
                e.pcompl[entry] = wadd(e.pissued[entry], d2);
            }
            same_total += popc(sm);
            any_cross = any_cross || cm != 0ull;
            cap = __shfl(incl, kWave - 1, kWave);
        }
        if (g.strategy == NANORTS_CANCEL_ALTERNATING && lane == 0) e.sc[S_ALT] = wadd(alt, same_total);
        if (any_cross || cap != kNoCap) {
            kind = kKindNone;
            none = any_cross ? -1 : imin(requested, cap);
        }
        wave_sync();
    }
    // _assign_pending_action (:374-403)
    const int32_t duration = kind == kKindNone ? none : requested;
    if (lane == 0) {
        const int32_t held = e.porder[slot];
        const int32_t next_order = e.sc[S_NEXT_ORDER];
        e.pkind[slot] = (int8_t)kind;
        e.pdir[slot] = (int8_t)((kind == kKindMove || kind == kKindHarvest || kind == kKindReturn || kind == kKindProduce)
                                    ? dir
                                    : kAbsent);
        e.pnone[slot] = kind == kKindNone ? none : 0;
        e.ptarget[slot] = (int16_t)(kind == kKindAttack ? target : kAbsent);
        e.pptype[slot] = (int8_t)(kind == kKindProduce ? ptype : kAbsent);
        e.pissued[slot] = time;
        e.pcompl[slot] = wadd(time, duration);
        e.porder[slot] = held == kAbsent ? next_order : held;
        if (held == kAbsent) e.sc[S_NEXT_ORDER] = wadd(next_order, 1);
    }
    wave_sync();
}

// admission.admit (N/core/admission.py:181-197)
NR_DEV void admit(const KGame& g, const Hdr& h, const Env& e, int lane, uint32_t key0, uint32_t key1,
                  bool count_events) {
    const Layout& y = g.lay;
    if (count_events) {
        if (lane < 32) at<int32_t>(e, y.b_events)[lane] = 0;
        wave_sync();
    }
    int32_t n_rank = 0;
    const int32_t n = order_requests(g, e, lane, &n_rank);
    AS3 int16_t* order = at<int16_t>(e, y.b_order);
    for (int32_t i = 0; i < n; ++i) {
        const int32_t p = uni(order[i]);
        admit_one(g, h, e, lane, p, n_rank, key0, key1, count_events);
    }
}

// k-th set bit (0-based) of m by halving popcounts; m has more than k bits.
NR_DEV int32_t select_bit(uint64_t m, int32_t k) {
    int32_t pos = 0;
    uint32_t v = (uint32_t)m;
    const int32_t c32 = popc((uint64_t)v);
    if (k >= c32) {
        k -= c32;
        v = (uint32_t)(m >> 32);
        pos = 32;
    }
#pragma unroll
    for (int32_t half = 16; half >= 1; half >>= 1) {
        const uint32_t lowmask = (1u << half) - 1u;
        const int32_t c = __popc(v & lowmask);
        if (k >= c) {
            k -= c;
            v >>= half;
            pos += half;
        }
    }
    return pos;
}

// The i-th live slot (0-based, i below the live count), from the live-slot
// bitmap: each lane picks its word by the words' running counts and selects
// the bit within it, so no list goes through LDS.  Lanes with i at or past
// the count get an unused value.
NR_DEV int32_t live_slot_at(const KGame& g, const Env& e, int32_t i) {
    AS3 const uint64_t* live = at<uint64_t>(e, g.lay.o_live);
    uint64_t mine = 0ull;
    int32_t base = 0, k = 0, word = 0;
    for (int32_t w = 0; w * kWave < g.E; ++w) {
        const uint64_t m = live[w];
        const int32_t c = popc(m);
        const bool in = i >= base && i < base + c;
        mine = in ? m : mine;
        k = in ? i - base : k;
        word = in ? w : word;
        base += c;
    }
    return word * kWave + select_bit(mine, k);
}

// The live slots of the staged env: their count (wave-uniform) and, when the
// count is at most a wave, lane i's slot = the i-th live slot in slot order
// (lanes at or past the count, or every lane of a larger count, hold an
// unused value).  Each live slot's lane in its bitmap word sends the slot to
// the lane of its rank with a forward permute, which moves values between
// lanes without LDS memory; the other lanes of the word send to a lane past
// the word's ranks, and every lane keeps only what the word of its own rank
// sent.  Every lane of the wave must be active.
struct LiveLanes {
    int32_t count, slot;
    int32_t slot2;  // half-wave teams: the (TW + lane)-th live slot, for counts up to 2 TW
};
template <int TW = kWave>
NR_DEV LiveLanes live_lanes(const KGame& g, const Env& e, int lane) {
    LiveLanes out = {0, 0, 0};
    if constexpr (TW != kWave) {
        // a half-wave team: the bitmap read as 32-slot pieces, each piece's
        // live slots sent to the lanes of their ranks modulo TW within the
        // team (a piece's at most 32 ranks fall on distinct lanes); lane i
        // keeps rank i in `slot` and rank TW + i in `slot2`
        AS3 const uint32_t* live = at<uint32_t>(e, g.lay.o_live);
        const int32_t first = team_half<TW>() * TW;
        for (int32_t w = 0; w * TW < g.E; ++w) {
            const uint32_t m = live[w];
            if (m == 0u) continue;
            const int32_t base = out.count, c = __popc(m);
            out.count += c;
            if (out.count > 2 * TW) continue;
            const int32_t rank = base + __popc(m & ((1u << lane) - 1u));
            const int32_t to = ((m >> lane) & 1u) ? rank : out.count;
            const int32_t got = __builtin_amdgcn_ds_permute((first + (to & (TW - 1))) << 2, w * TW + lane);
            if (lane >= base && lane < out.count) out.slot = got;
            if (lane + TW >= base && lane + TW < out.count) out.slot2 = got;
        }
        return out;
    }
    AS3 const uint64_t* live = at<uint64_t>(e, g.lay.o_live);
    for (int32_t w = 0; w * kWave < g.E; ++w) {
        const uint64_t v = live[w];
        const uint64_t m = (uint64_t)(uint32_t)uni((int32_t)(uint32_t)v) |
                           ((uint64_t)(uint32_t)uni((int32_t)(uint32_t)(v >> 32)) << 32);
        if (m == 0ull) continue;
        const int32_t base = out.count, c = popc(m);
        out.count += c;
        if (out.count > kWave) continue;
        const uint32_t rank = __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                                        __builtin_amdgcn_mbcnt_lo((uint32_t)m, (uint32_t)base));
        const int32_t to = __builtin_amdgcn_inverse_ballot_w64(m) ? (int32_t)rank : (out.count & (kWave - 1));
        const int32_t got = __builtin_amdgcn_ds_permute(to << 2, w * kWave + lane);
        const uint64_t upto = out.count >= kWave ? ~0ull : ((1ull << out.count) - 1ull);
        const uint64_t ranks = upto & ~((1ull << base) - 1ull);
        out.slot = __builtin_amdgcn_inverse_ballot_w64(ranks) ? got : out.slot;
    }
    return out;
}

// ---------------------------------------------------------------------------
// Completion (N/core/pending.py:47-76, N/core/completion.py)
// ---------------------------------------------------------------------------
// Member record: 5 dwords.
//   [0] slot | kind << 16 | dir << 24   [1] target(16) | ptype(8) << 16 | owner(8) << 24
//   [2] unit_type(8) | cell(16) << 8    [3] birth   [4] carried
NR_DEV void remove_slot(const Env& e, int32_t s) {
    e.birth[s] = kAbsent;
    e.utype[s] = (int8_t)kAbsent;
    e.owner[s] = (int8_t)kAbsent;
    e.cell[s] = (int16_t)kAbsent;
    e.hp[s] = 0;
    e.carried[s] = 0;
    e.pkind[s] = (int8_t)kAbsent;
    e.pdir[s] = (int8_t)kAbsent;
    e.pnone[s] = 0;
    e.ptarget[s] = (int16_t)kAbsent;
    e.pptype[s] = (int8_t)kAbsent;
    e.pissued[s] = 0;
    e.pcompl[s] = 0;
    e.porder[s] = kAbsent;
}

// N/core/completion.py:134-180 (_take_turn) for the member record `r`, with
// each kind's _complete (move.py:19-27, harvest.py:24-45, return_.py:25-43,
// produce.py:47-81, attack.py:78-98).
// The member's retained values are wave-uniform arguments.
// The per-slot completion records of one env, as the step target returns them
// (results 27-30, src/nanorts/core/cycle.py:48-81, 254-300): is_member [E],
// int32 [E][6] (actor_birth, target_birth, amount, balance, spawn_birth,
// death_birth), int16 [E][4] (target_slot, spawn_slot, spawn_cell,
// death_slot), int8 [E][6] (flags, actor_owner, actor_unit_type,
// produced_type, death_owner, death_unit_type).  Flags: hit 1, death 2,
// harvest 4, depleted 8, return 16, spawn 32.  The caller zero-fills them;
// a member's turn writes its whole row.
struct StepRecords {
    uint8_t* member;
    int32_t* wide;
    int16_t* index;
    int8_t* narrow;
};
enum : int32_t { REC_HIT = 1, REC_DEATH = 2, REC_HARVEST = 4, REC_DEPLETED = 8, REC_RETURN = 16, REC_SPAWN = 32 };

// `rec` (NULL on every path but the step target's): where this member's
// records go (each kind's records, N/core/kinds/*.py, and the death of the
// unit its turn removes, N/core/completion.py:68-99).
template <int TW = kWave>
NR_DEV void take_turn(const KGame& g, const Hdr& h, const Env& e, int lane, int32_t slot, int32_t kind, int32_t dir,
                      int32_t target, int32_t ptype, int32_t owner, int32_t utype, int32_t rcell, int32_t rbirth,
                      int32_t rcarried, const StepRecords* rec = nullptr) {
    int32_t rf = 0, r_target = 0, r_tbirth = 0, r_amount = 0, r_balance = 0, r_ptype = 0, r_spawn = 0,
            r_sbirth = 0, r_scell = 0;
    const int32_t actor = clampi(utype, 0, g.T - 1);
    const int32_t player = clampi(owner, 0, 1);
    const int32_t cur_birth = tuni<TW>(e.birth[slot]);
    const bool alive = cur_birth != kAbsent && cur_birth == rbirth;
    const int32_t dest = reserved_position(g, rcell, dir);
    bool removal = false;
    int32_t removed = 0;
    if (kind == kKindMove) {
        if (alive && lane == 0) {
            if (dest >= 0 && dest < g.cells) e.entity[dest] = (int16_t)slot;
            if (rcell >= 0 && rcell < g.cells) e.entity[rcell] = (int16_t)kAbsent;
            e.cell[slot] = (int16_t)dest;
            e.sc[S_VISDIRTY] |= 1 << player;
        }
    } else if (kind == kKindHarvest) {
        const Nb n = neighbour(g, h, e, rcell, dir);
        const bool harvesting = tuni<TW>(n.occupied && (tabv(h, F_FLAGS, n.unit_type) & FL_RESOURCE) ? 1 : 0) != 0;
        if (harvesting) {
            const int32_t stack = tuni<TW>(n.slot);
            const int32_t amount = tabv(h, F_AMOUNT, actor);
            const int32_t left = wsub(tuni<TW>(e.carried[stack]), amount);
            if (rec) {
                rf |= left <= 0 ? REC_HARVEST | REC_DEPLETED : REC_HARVEST;
                r_target = stack;
                r_tbirth = tuni<TW>(e.birth[stack]);
                r_amount = amount;
            }
            if (lane == 0) {
                e.carried[stack] = left;
                if (alive) e.carried[slot] = amount;
            }
            if (left <= 0) {
                removal = true;
                removed = stack;
            }
        }
    } else if (kind == kKindReturn) {
        const Nb n = neighbour(g, h, e, rcell, dir);
        const bool returning =
            tuni<TW>(n.occupied && (tabv(h, F_FLAGS, n.unit_type) & FL_STOCKPILE) && rcarried > 0 ? 1 : 0) != 0;
        if (returning && rec) {
            rf |= REC_RETURN;
            r_target = tuni<TW>(n.slot);
            r_tbirth = tuni<TW>(e.birth[gidx(tuni<TW>(n.slot), g.E)]);
            r_amount = rcarried;
            r_balance = wadd(tuni<TW>(e.sc[S_RES0 + player]), rcarried);
        }
        if (returning && lane == 0) {
            if (alive) e.carried[slot] = 0;
            e.sc[S_RES0 + player] = wadd(e.sc[S_RES0 + player], rcarried);
        }
    } else if (kind == kKindProduce) {
        const int32_t newborn_type = clampi(ptype, 0, g.T - 1);
        const int32_t balance = wsub(tuni<TW>(e.sc[S_RES0 + player]), tabv(h, F_COST, newborn_type));
        if (balance >= 0) {
            // units.lowest_free_slot (N/core/units.py:12-18)
            const int32_t block = g.N + player * g.C;
            int32_t newborn = -1;
            for (int32_t base = 0; base < g.C && newborn < 0; base += TW) {
                const int32_t i = base + lane;
                const bool free = i < g.C && e.birth[block + i] == kAbsent;
                const uint64_t m = tballot<TW>(free);
                if (m != 0ull) newborn = block + base + (int32_t)__builtin_ctzll(m);
            }
            newborn = tuni<TW>(newborn);
            if (rec && newborn >= 0) {
                rf |= REC_SPAWN;
                r_ptype = newborn_type;
                r_spawn = newborn;
                r_sbirth = tuni<TW>(e.sc[S_NEXT_BIRTH]);
                r_scell = dest;
                r_balance = balance;
            }
            if (lane == 0) {
                if (newborn >= 0) {
                    const int32_t birth = e.sc[S_NEXT_BIRTH];
                    e.sc[S_RES0 + player] = balance;
                    if (dest >= 0 && dest < g.cells) e.entity[dest] = (int16_t)newborn;
                    e.birth[newborn] = birth;
                    at<uint64_t>(e, g.lay.o_live)[newborn >> 6] |= 1ull << (newborn & 63);
                    e.utype[newborn] = (int8_t)newborn_type;
                    e.owner[newborn] = (int8_t)player;
                    e.cell[newborn] = (int16_t)dest;
                    e.hp[newborn] = (int16_t)tabv(h, F_HP, newborn_type);
                    e.sc[S_NEXT_BIRTH] = wadd(birth, 1);
                    e.sc[S_UNITS0 + player] += 1;
                    e.sc[S_VISDIRTY] |= 1 << player;
                } else {
                    e.sc[S_SO0 + player] = wadd(e.sc[S_SO0 + player], 1);
                }
            }
        }
    } else if (kind == kKindAttack) {
        const int32_t occ = tuni<TW>(e.entity[clampi(target, 0, g.cells - 1)]);
        if (occ != kAbsent) {
            const int32_t victim = occ;
            const int32_t left = wsub(tuni<TW>(e.hp[gidx(victim, g.E)]), tabv(h, F_DAMAGE, actor));
            if (rec) {
                rf |= REC_HIT;
                r_target = victim;
                r_tbirth = tuni<TW>(e.birth[gidx(victim, g.E)]);
                r_amount = tabv(h, F_DAMAGE, actor);
            }
            if (lane == 0) e.hp[victim] = (int16_t)left;
            if (left <= 0) {
                removal = true;
                removed = victim;
            }
        }
    }
    if (rec && lane == 0) {
        // the whole row of this member: its records, the death last
        const int32_t r = gidx(removed, g.E);
        if (removal) rf |= REC_DEATH;
        const bool any = rf != 0;
        rec->member[slot] = 1;
        int32_t* w = rec->wide + (int64_t)slot * 6;
        int16_t* x = rec->index + (int64_t)slot * 4;
        int8_t* n = rec->narrow + (int64_t)slot * 6;
        w[0] = any ? rbirth : 0;
        w[1] = r_tbirth;
        w[2] = r_amount;
        w[3] = r_balance;
        w[4] = r_sbirth;
        w[5] = removal ? e.birth[r] : 0;
        x[0] = (int16_t)r_target;
        x[1] = (int16_t)r_spawn;
        x[2] = (int16_t)r_scell;
        x[3] = (int16_t)(removal ? removed : 0);
        n[0] = (int8_t)rf;
        n[1] = (int8_t)(any ? owner : 0);
        n[2] = (int8_t)(any ? utype : 0);
        n[3] = (int8_t)r_ptype;
        n[4] = (int8_t)(removal ? e.owner[r] : 0);
        n[5] = (int8_t)(removal ? e.utype[r] : 0);
    }
    if (removal) {
        wave_sync();
        if (lane == 0) {
            const int32_t c = e.cell[gidx(removed, g.E)];
            if (c >= 0 && c < g.cells) e.entity[c] = (int16_t)kAbsent;
            if (removed >= g.N && removed < g.E && e.birth[removed] != kAbsent) {
                const int32_t owner_block = (removed - g.N) / g.C;
                e.sc[S_UNITS0 + owner_block] -= 1;
                e.sc[S_VISDIRTY] |= 1 << owner_block;
            }
            if (removed >= 0 && removed < g.E) at<uint64_t>(e, g.lay.o_live)[removed >> 6] &= ~(1ull << (removed & 63));
            remove_slot(e, removed);
        }
    }
    wave_sync();
}

// pending.select + completion.apply (N/core/completion.py:106-117).  One
// pass over the slots records each acting member's retained actor (the
// pre-clear snapshot, :120-131) and clears every due pending action.
// `at_most_a_wave`: the caller guarantees at most 64 live slots, and the
// path for more (member records in the phase union) is left out.  Returns
// the new time.
// A half-wave team (TW = 32) takes the slot-per-lane paths only: one live
// slot per lane, or two (complete_two_per_lane) for 33..64; its caller
// guarantees at most 64 live slots.
template <int TW>
NR_DEV int32_t complete_two_per_lane(const KGame& g, const Hdr& h, const Env& e, int lane, int32_t time,
                                     const LiveLanes& ll, const StepRecords* records);
template <int TW = kWave>
NR_DEV int32_t complete(const KGame& g, const Hdr& h, const Env& e_in, int lane, bool at_most_a_wave = false,
                        LiveLanes known = LiveLanes{-1, 0}, const StepRecords* records = nullptr) {
    const Env e = refresh<TW>(g, e_in);
    const Layout& y = g.lay;
    const int32_t time = wadd(tuni<TW>(e.sc[S_TIME]), 1);
    if (lane == 0) e.sc[S_TIME] = time;
    AS3 int32_t* rec = at<int32_t>(e, y.m_rec);  // [2C][6] in slot order
    // only live slots hold pending actions
    // the caller's copy when it holds one for this live set (a summary of
    // the state since which no unit spawned or died)
    const LiveLanes ll = known.count >= 0 ? known : live_lanes<TW>(g, e, lane);
    const int32_t nlive = ll.count;
    if constexpr (TW != kWave) {
        if (nlive > TW) return complete_two_per_lane<TW>(g, h, e, lane, time, ll, records);
    }
    if (TW != kWave || at_most_a_wave || nlive <= kWave) {
        // one live slot per lane: the members' retained actors stay in
        // their lanes and are ranked and read from there
        const int32_t s = lane < nlive ? ll.slot : 0;
        bool acting = false;
        int32_t w0 = 0, w1 = 0, w2 = 0, rb = 0, rc = 0, ord = 0;
        if (lane < nlive) {
            const int32_t k = e.pkind[s];
            const bool due = k != kAbsent && e.pcompl[s] <= time;
            if (due) {
                acting = k != kKindNone && s >= g.N;
                if (acting) {
                    w0 = (s & 0xFFFF) | ((k & 0xFF) << 16) | ((e.pdir[s] & 0xFF) << 24);
                    w1 = (e.ptarget[s] & 0xFFFF) | ((e.pptype[s] & 0xFF) << 16) | ((e.owner[s] & 0xFF) << 24);
                    w2 = (e.utype[s] & 0xFF) | ((e.cell[s] & 0xFFFF) << 8);
                    rb = e.birth[s];
                    rc = e.carried[s];
                    ord = e.porder[s];
                }
                e.pkind[s] = (int8_t)kAbsent;
                e.pdir[s] = (int8_t)kAbsent;
                e.pnone[s] = 0;
                e.ptarget[s] = (int16_t)kAbsent;
                e.pptype[s] = (int8_t)kAbsent;
                e.pissued[s] = 0;
                e.pcompl[s] = 0;
                e.porder[s] = kAbsent;
            }
        }
        wave_sync();
        // A cycle whose members all MOVE (and no records): their turns taken
        // at once where they write distinct cells, which the grid shows: each
        // live mover's destination empty and its own cell holding it (then no
        // mover's cell is another's destination, nor two movers' cells one),
        // and, once each has written its destination, each reading itself
        // back there (no two destinations one).  A turn then writes its own
        // destination, empties its own cell and sets its own slot's cell, so
        // the turns give the same state in any order.  Admission keeps a
        // state so (a move's destination was free when the move was issued
        // and has been claimed since); a state built otherwise takes the
        // turns in order.
        if (records == nullptr && tballot<TW>(acting && ((w0 >> 16) & 0xFF) != kKindMove) == 0ull) {
            const int32_t slot = w0 & 0xFFFF;
            const int32_t rcell = (int16_t)((w2 >> 8) & 0xFFFF);
            bool alive = false;
            int32_t dest = 0;
            if (acting) {
                const int32_t cur = e.birth[slot];
                alive = cur != kAbsent && cur == rb;
                dest = reserved_position(g, rcell, (int8_t)((w0 >> 24) & 0xFF));
            }
            const bool wd = alive && dest >= 0 && dest < g.cells;     // writes its destination
            const bool wr = alive && rcell >= 0 && rcell < g.cells;  // empties its cell
            // the grid as it was (the wave reads before it writes), then the
            // destinations written and read back, and one vote on both checks
            const int16_t held = wd ? e.entity[dest] : (int16_t)kAbsent;
            const bool odd = held != kAbsent || (wr && e.entity[rcell] != slot);
            if (wd) e.entity[dest] = (int16_t)slot;
            wave_sync();
            if (tballot<TW>(odd || (wd && e.entity[dest] != slot)) == 0ull) {
                if (wr) e.entity[rcell] = (int16_t)kAbsent;
                if (alive) e.cell[slot] = (int16_t)dest;
                const int32_t mover = clampi((int8_t)((w1 >> 24) & 0xFF), 0, 1);
                const uint64_t m0 = tballot<TW>(alive && mover == 0), m1 = tballot<TW>(alive && mover == 1);
                if (lane == 0 && (m0 | m1) != 0ull)
                    e.sc[S_VISDIRTY] |= (m0 != 0ull ? 1 : 0) | (m1 != 0ull ? 2 : 0);
                wave_sync();
                return time;
            }
            // put back what the destinations held (movers sharing one read
            // the same value) and take the turns in order
            wave_sync();
            if (wd) e.entity[dest] = held;
            wave_sync();
        }
        const uint64_t members = tballot<TW>(acting);
        const int32_t n = popc(members);
        // members act in pending order (pending.batch_order :55-60), ties by slot
        int32_t rank = 0;
        if constexpr (TW == kWave) {
            for (uint64_t m = members; m != 0ull; m &= m - 1ull) {
                const int32_t j = (int32_t)__builtin_ctzll(m);
                const int32_t oj = __builtin_amdgcn_readlane(ord, j);
                rank += (oj < ord) || (oj == ord && j < lane);
            }
        } else {
            // both halves' members in one scalar loop: the lanes that are a
            // member in either half (a lane's own half counts only its own)
            const uint64_t both = (uint64_t)__ballot(acting);
            for (uint32_t m = (uint32_t)both | (uint32_t)(both >> 32); m != 0u; m &= m - 1u) {
                const int32_t j = (int32_t)__builtin_ctz(m);
                const int32_t oj = tread_at<TW>(ord, j);
                rank += ((members >> j) & 1ull) && ((oj < ord) || (oj == ord && j < lane));
            }
        }
        const int32_t turns = tmax<TW>(n);
        for (int32_t k = 0; k < turns; ++k) {
            if (TW != kWave && k >= n) continue;
            const int32_t li = (int32_t)__builtin_ctzll(tballot<TW>(acting && rank == k));
            const int32_t a = tread<TW>(w0, li), b = tread<TW>(w1, li), c = tread<TW>(w2, li);
            take_turn<TW>(g, h, e, lane, a & 0xFFFF, (int8_t)((a >> 16) & 0xFF), (int8_t)((a >> 24) & 0xFF),
                          (int16_t)(b & 0xFFFF), (int8_t)((b >> 16) & 0xFF), (int8_t)((b >> 24) & 0xFF),
                          (int8_t)(c & 0xFF), (int16_t)((c >> 8) & 0xFFFF), tread<TW>(rb, li), tread<TW>(rc, li),
                          records);
        }
        return time;
    }
    if constexpr (TW != kWave) return time;
    int32_t n = 0;
    for (int32_t base = 0; base < nlive; base += kWave) {
        const int32_t i = base + lane;
        const int32_t s = i < nlive ? live_slot_at(g, e, i) : 0;
        bool acting = false;
        int32_t r0 = 0, r1 = 0, r2 = 0, r3 = 0, r4 = 0;
        if (i < nlive) {
            const int32_t k = e.pkind[s];
            const bool due = k != kAbsent && e.pcompl[s] <= time;
            if (due) {
                acting = k != kKindNone && s >= g.N;
                if (acting) {
                    r0 = (s & 0xFFFF) | ((k & 0xFF) << 16) | ((e.pdir[s] & 0xFF) << 24);
                    r1 = (e.ptarget[s] & 0xFFFF) | ((e.pptype[s] & 0xFF) << 16) | ((e.owner[s] & 0xFF) << 24);
                    r2 = (e.utype[s] & 0xFF) | ((e.cell[s] & 0xFFFF) << 8);
                    r3 = e.birth[s];
                    r4 = e.porder[s];
                }
                e.pkind[s] = (int8_t)kAbsent;
                e.pdir[s] = (int8_t)kAbsent;
                e.pnone[s] = 0;
                e.ptarget[s] = (int16_t)kAbsent;
                e.pptype[s] = (int8_t)kAbsent;
                e.pissued[s] = 0;
                e.pcompl[s] = 0;
                e.porder[s] = kAbsent;
            }
        }
        const uint64_t m = ballot(acting);
        if (acting) {
            AS3 int32_t* r = rec + 6 * (n + count_below(m));
            r[0] = r0;
            r[1] = r1;
            r[2] = r2;
            r[3] = r3;
            r[4] = e.carried[s];
            r[5] = r4;
        }
        n += popc(m);
    }
    wave_sync();
    if (n <= kWave) {
        int32_t w0 = 0, w1 = 0, w2 = 0, rb = 0, rc = 0, ord = 0;
        if (lane < n) {
            AS3 const int32_t* r = rec + 6 * lane;
            w0 = r[0];
            w1 = r[1];
            w2 = r[2];
            rb = r[3];
            rc = r[4];
            ord = r[5];
        }
        // members act in pending order (pending.batch_order :55-60), ties by slot
        int32_t rank = 0;
        for (int32_t j = 0; j < n; ++j) {
            const int32_t oj = __builtin_amdgcn_readlane(ord, j);
            rank += (oj < ord) || (oj == ord && j < lane);
        }
        for (int32_t k = 0; k < n; ++k) {
            const int32_t li = (int32_t)__builtin_ctzll(ballot(lane < n && rank == k));
            const int32_t a = __builtin_amdgcn_readlane(w0, li), b = __builtin_amdgcn_readlane(w1, li),
                          c = __builtin_amdgcn_readlane(w2, li);
            take_turn(g, h, e, lane, a & 0xFFFF, (int8_t)((a >> 16) & 0xFF), (int8_t)((a >> 24) & 0xFF),
                      (int16_t)(b & 0xFFFF), (int8_t)((b >> 16) & 0xFF), (int8_t)((b >> 24) & 0xFF), (int8_t)(c & 0xFF),
                      (int16_t)((c >> 8) & 0xFFFF), __builtin_amdgcn_readlane(rb, li),
                      __builtin_amdgcn_readlane(rc, li), records);
        }
        return time;
    }
    // more members than lanes: rank each record by (pending order, slot)
    AS3 int16_t* pos = at<int16_t>(e, y.m_tmp);
    for (int32_t i = lane; i < n; i += kWave) {
        const int32_t oi = rec[6 * i + 5];
        int32_t r = 0;
        for (int32_t j = 0; j < n; ++j) {
            const int32_t oj = rec[6 * j + 5];
            r += (oj < oi) || (oj == oi && j < i);
        }
        pos[r] = (int16_t)i;
    }
    wave_sync();
    for (int32_t k = 0; k < n; ++k) {
        AS3 const int32_t* r = rec + 6 * uni(pos[k]);
        const int32_t a = uni(r[0]), b = uni(r[1]), c = uni(r[2]);
        take_turn(g, h, e, lane, a & 0xFFFF, (int8_t)((a >> 16) & 0xFF), (int8_t)((a >> 24) & 0xFF),
                  (int16_t)(b & 0xFFFF), (int8_t)((b >> 16) & 0xFF), (int8_t)((b >> 24) & 0xFF), (int8_t)(c & 0xFF),
                  (int16_t)((c >> 8) & 0xFFFF), uni(r[3]), uni(r[4]), records);
    }
    return time;
}

// complete() for a half-wave team with TW < nlive <= 2 TW live slots: lane i
// holds live slots i and TW + i (set 0 and set 1).  Same members, same
// order (pending order, ties by slot = by live index) as the one-per-lane
// path.
template <int TW>
NR_DEV int32_t complete_two_per_lane(const KGame& g, const Hdr& h, const Env& e, int lane, int32_t time,
                                     const LiveLanes& ll, const StepRecords* records) {
    bool acting[2] = {false, false};
    int32_t w0[2] = {0, 0}, w1[2] = {0, 0}, w2[2] = {0, 0}, rb[2] = {0, 0}, rc[2] = {0, 0}, ord[2] = {0, 0};
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int32_t i = k * TW + lane;
        if (i >= ll.count) continue;
        const int32_t s = k ? ll.slot2 : ll.slot;
        const int32_t kind = e.pkind[s];
        if (kind == kAbsent || e.pcompl[s] > time) continue;
        acting[k] = kind != kKindNone && s >= g.N;
        if (acting[k]) {
            w0[k] = (s & 0xFFFF) | ((kind & 0xFF) << 16) | ((e.pdir[s] & 0xFF) << 24);
            w1[k] = (e.ptarget[s] & 0xFFFF) | ((e.pptype[s] & 0xFF) << 16) | ((e.owner[s] & 0xFF) << 24);
            w2[k] = (e.utype[s] & 0xFF) | ((e.cell[s] & 0xFFFF) << 8);
            rb[k] = e.birth[s];
            rc[k] = e.carried[s];
            ord[k] = e.porder[s];
        }
        e.pkind[s] = (int8_t)kAbsent;
        e.pdir[s] = (int8_t)kAbsent;
        e.pnone[s] = 0;
        e.ptarget[s] = (int16_t)kAbsent;
        e.pptype[s] = (int8_t)kAbsent;
        e.pissued[s] = 0;
        e.pcompl[s] = 0;
        e.porder[s] = kAbsent;
    }
    wave_sync();
    const uint64_t members0 = tballot<TW>(acting[0]), members1 = tballot<TW>(acting[1]);
    const int32_t n = popc(members0) + popc(members1);
    // rank by (pending order, live index); live index k * TW + lane
    int32_t rank[2] = {0, 0};
#pragma unroll
    for (int kj = 0; kj < 2; ++kj) {
        for (uint64_t m = kj ? members1 : members0; m != 0ull; m &= m - 1ull) {
            const int32_t j = (int32_t)__builtin_ctzll(m);
            const int32_t oj = tread<TW>(ord[kj], j), ij = kj * TW + j;
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                const int32_t ik = k * TW + lane;
                rank[k] += (oj < ord[k]) || (oj == ord[k] && ij < ik);
            }
        }
    }
    const int32_t turns = tmax<TW>(n);
    for (int32_t t = 0; t < turns; ++t) {
        if (t >= n) continue;
        const uint64_t m0 = tballot<TW>(acting[0] && rank[0] == t);
        const bool in1 = m0 == 0ull;
        const int32_t li = (int32_t)__builtin_ctzll(in1 ? tballot<TW>(acting[1] && rank[1] == t) : m0);
        const int32_t a = tread<TW>(in1 ? w0[1] : w0[0], li), b = tread<TW>(in1 ? w1[1] : w1[0], li),
                      c = tread<TW>(in1 ? w2[1] : w2[0], li);
        const int32_t birth = tread<TW>(in1 ? rb[1] : rb[0], li), carried = tread<TW>(in1 ? rc[1] : rc[0], li);
        take_turn<TW>(g, h, e, lane, a & 0xFFFF, (int8_t)((a >> 16) & 0xFF), (int8_t)((a >> 24) & 0xFF),
                      (int16_t)(b & 0xFFFF), (int8_t)((b >> 16) & 0xFF), (int8_t)((b >> 24) & 0xFF), (int8_t)(c & 0xFF),
                      (int16_t)((c >> 8) & 0xFFFF), birth, carried, records);
    }
    return time;
}

// outcome.decide (N/core/outcome.py:11-25)
NR_DEV void decide(const KGame& g, const Env& e_in, int lane) {
    const Env e = refresh(g, e_in);
    bool alive[2] = {false, false};
    for (int32_t pl = 0; pl < 2; ++pl) {
        uint64_t any = 0;
        for (int32_t base = 0; base < g.C; base += kWave) {
            const int32_t i = base + lane;
            any |= ballot(i < g.C && e.birth[g.N + pl * g.C + i] != kAbsent);
        }
        alive[pl] = any != 0ull;
    }
    const int32_t count = (alive[0] ? 1 : 0) + (alive[1] ? 1 : 0);
    if (lane == 0) {
        e.sc[S_GAME_OVER] = count <= 1 ? 1 : 0;
        e.sc[S_WINNER] = count == 1 ? (alive[0] ? 0 : 1) : kAbsent;
    }
    wave_sync();
}

// Active units per player, for decide_counted.
// Also rebuilds the live-slot bitmap, which take_turn then keeps.
template <int TW = kWave>
NR_DEV void count_units(const KGame& g, const Env& e_in, int lane) {
    const Env e = refresh<TW>(g, e_in);
    AS3 uint64_t* live = at<uint64_t>(e, g.lay.o_live);
    int32_t count0 = 0, count1 = 0;
    // every word of the bitmap, the bits past E clear
    for (int32_t base = 0; base < ((g.E + 63) & ~63); base += TW) {
        const int32_t s = base + lane;
        const bool alive = s < g.E && e.birth[s] != kAbsent;
        const uint64_t m = tballot<TW>(alive);
        if constexpr (TW == kWave) {
            if (lane == 0) live[base >> 6] = m;
        } else {
            if (lane == 0) ((AS3 uint32_t*)live)[base >> 5] = (uint32_t)m;
        }
        count0 += popc(tballot<TW>(alive && s >= g.N && s < g.N + g.C));
        count1 += popc(tballot<TW>(alive && s >= g.N + g.C));
    }
    if (lane == 0) {
        e.sc[S_UNITS0] = count0;
        e.sc[S_UNITS1] = count1;
    }
    wave_sync();
}


// The outcome of a cycle and the scalars its observation shows, held in
// registers after decide_counted so later phases need not read them back.
struct Outcome {
    int32_t over, winner, res0, res1, alt;
};

// outcome.decide from the kept unit counts.  The balances and the
// alternating count, final once completion has run, are read in the same
// batch.
template <int TW = kWave>
NR_DEV Outcome decide_counted(const Env& e, int lane) {
    const int32_t u0 = e.sc[S_UNITS0], u1 = e.sc[S_UNITS1];
    Outcome o;
    o.res0 = tuni<TW>(e.sc[S_RES0]);
    o.res1 = tuni<TW>(e.sc[S_RES1]);
    o.alt = tuni<TW>(e.sc[S_ALT]);
    const bool a0 = tuni<TW>(u0) > 0, a1 = tuni<TW>(u1) > 0;
    const int32_t count = (a0 ? 1 : 0) + (a1 ? 1 : 0);
    o.over = count <= 1 ? 1 : 0;
    o.winner = count == 1 ? (a0 ? 0 : 1) : kAbsent;
    if (lane == 0) {
        e.sc[S_GAME_OVER] = o.over;
        e.sc[S_WINNER] = o.winner;
    }
    wave_sync();
    return o;
}

// core.step (N/core/__init__.py:99-110) on the staged env.
NR_DEV void core_step(const KGame& g, const Hdr& h, const Env& e, int lane, uint32_t key0, uint32_t key1,
                      bool count_events, const StepRecords* rec = nullptr) {
    admit(g, h, e, lane, key0, key1, count_events);
    complete(g, h, e, lane, false, LiveLanes{-1, 0}, rec);
    decide(g, e, lane);
}

// The initial State's scalars into the block, the episode counter advanced
// (lanes below S_COUNT; the roots stay).
NR_DEV void reset_scalars(const KGame& g, const Env& e, int lane, int32_t episode) {
    if (lane >= S_COUNT) return;
    const nanorts_state& s = g.initial;
    int32_t v = e.sc[lane];
    switch (lane) {
        case S_TIME: v = s.time[0]; break;
        case S_RES0: v = s.player_resources[0]; break;
        case S_RES1: v = s.player_resources[1]; break;
        case S_NEXT_BIRTH: v = s.next_birth[0]; break;
        case S_NEXT_ORDER: v = s.next_pending_order[0]; break;
        case S_ALT: v = s.alternating_conflict_count[0]; break;
        case S_GAME_OVER: v = s.game_over[0] ? 1 : 0; break;
        case S_WINNER: v = s.winner[0]; break;
        case S_SO0: v = s.spawn_overflow[0]; break;
        case S_SO1: v = s.spawn_overflow[1]; break;
        case S_EPISODE: v = (int32_t)((uint32_t)episode + 1u); break;
        case S_VISDIRTY: v = 3; break;
        default: break;
    }
    e.sc[lane] = v;
}

// Copy the initial State into the staged env: core.reset ignores its key
// (N/core/__init__.py:30-32) and lifecycle.advance takes every leaf from it
// (N/adapters/lifecycle.py:53-79).  The row leaves are copied through one
// runtime-indexed loop over g.seg so no per-leaf address stays live.
// `Window`: the block may be a slot window's (KGame::shift > 0; the fused
// rollout's first pass only).
template <int TW = kWave, bool Window = false>
NR_DEV void reset_env(const KGame& g, const Hdr& h, const Env& e_in, int lane) {
    const Env e = refresh<TW>(g, e_in);
    const int32_t episode = tuni<TW>(e.sc[S_EPISODE]);
    // a slot window's block takes the initial rows through the window (the
    // caller has checked that they fit it); its segment table is empty
    if constexpr (Window) {
        if (g.shift > 0) load_window_rows<TW>(g, g.initial, 0, e, lane);
    }
#pragma nounroll
    for (int32_t k = 0; k < g.nseg; ++k) {
        const AS3 Seg* sg = h.seg + k;
        // (the header is the workgroup's: wave-uniform for either team width)
        const uint8_t* src = (const uint8_t*)(((uint64_t)(uint32_t)uni((int32_t)(uint32_t)(uintptr_t)sg->src)) |
                                              ((uint64_t)(uint32_t)uni((int32_t)((uintptr_t)sg->src >> 32)) << 32));
        copy_in<TW>(e.base + uni(sg->dst), src, uni(sg->bytes), lane);
    }
    reset_scalars(g, e, lane, episode);
    wave_sync();
    count_units<TW>(g, e, lane);
    decide_counted<TW>(e, lane);
}


// ---------------------------------------------------------------------------
// Legality (N/core/legality.py:32-64, kinds' _legality; row layout
// N/adapters/factors.py:31-62): bit 0..5 kind, 6.. move, 10.. harvest,
// 14.. return, 18.. produce direction, 22.. produce type, 22+T.. attack.
// ---------------------------------------------------------------------------
struct Row {
    uint32_t w[3];
};

NR_DEV void set_bit(Row& r, int32_t b) {
    const uint32_t bit = 1u << (b & 31);
    const int32_t w = b >> 5;
    r.w[0] |= w == 0 ? bit : 0u;
    r.w[1] |= w == 1 ? bit : 0u;
    r.w[2] |= w == 2 ? bit : 0u;
}

NR_DEV Row legality_row(const KGame& g, const Hdr& h, const Env& e, int32_t slot) {
    Row r;
    r.w[0] = r.w[1] = r.w[2] = 0u;
    if (e.birth[slot] == kAbsent) return r;
    const int32_t actor = clampi(e.utype[slot], 0, g.T - 1);
    const int32_t owner = e.owner[slot];
    const int32_t carried = e.carried[slot];
    const int32_t cell = e.cell[slot];
    const int32_t flags = tabv(h, F_FLAGS, actor);
    const int32_t balance = e.sc[S_RES0 + clampi(owner, 0, 1)];
    uint32_t affordable = 0u;
    for (int32_t t = 0; t < g.T; ++t)
        if (balance >= tabv(h, F_COST, t)) affordable |= 1u << t;
    const uint32_t types = (uint32_t)tabv(h, F_PRODUCES, actor) & affordable;
    set_bit(r, kKindNone);
    uint32_t produce_types = 0u;
    const int32_t x = cell_x(g, cell), yy = cell_y(g, cell);
#pragma unroll
    for (int32_t d = 0; d < 4; ++d) {
        const int32_t nx = x + dir_dx(d), ny = yy + dir_dy(d);
        if (nx < 0 || nx >= g.W || ny < 0 || ny >= g.H) continue;
        const int32_t nc = ny * g.W + nx;
        const int32_t occ = e.entity[nc];
        if (occ == kAbsent) {
            if (h.terrain[nc] == 0) {
                if (flags & FL_MOVE) {
                    set_bit(r, 6 + d);
                    set_bit(r, kKindMove);
                }
                if (types != 0u) {
                    set_bit(r, 18 + d);
                    produce_types |= types;
                }
            }
        } else {
            const int32_t s = gidx(occ, g.E);
            const int32_t nflags = tabv(h, F_FLAGS, clampi(e.utype[s], 0, g.T - 1));
            if ((flags & FL_HARVEST) && carried == 0 && (nflags & FL_RESOURCE)) {
                set_bit(r, 10 + d);
                set_bit(r, kKindHarvest);
            }
            if ((flags & FL_HARVEST) && carried > 0 && (nflags & FL_STOCKPILE) && e.owner[s] == owner) {
                set_bit(r, 14 + d);
                set_bit(r, kKindReturn);
            }
        }
    }
    if (produce_types != 0u) {
        set_bit(r, kKindProduce);
        for (int32_t t = 0; t < g.T; ++t)
            if ((produce_types >> t) & 1u) set_bit(r, 22 + t);
    }
    if (flags & FL_ATTACK) {
        const int32_t range = tabv(h, F_RANGE, actor);
        const int32_t reach = imin(range, g.radius);
        const int32_t first = 22 + g.T;
        bool any = false;
        for (int32_t dy = -reach; dy <= reach; ++dy) {
            const int32_t ty = yy + dy;
            if (ty < 0 || ty >= g.H) continue;
            for (int32_t dx = -reach; dx <= reach; ++dx) {
                if (dx * dx + dy * dy > range * range) continue;
                const int32_t tx = x + dx;
                if (tx < 0 || tx >= g.W) continue;
                const int32_t occ = e.entity[ty * g.W + tx];
                if (occ == kAbsent) continue;
                const int32_t towner = e.owner[gidx(occ, g.E)];
                if (towner >= 0 && towner != owner) {
                    set_bit(r, first + (g.radius + dy) * g.side + (g.radius + dx));
                    any = true;
                }
            }
        }
        if (any) set_bit(r, kKindAttack);
    }
    return r;
}

// ---------------------------------------------------------------------------
// The synthetic harness sampler (uniform over each factor's legal values):
//   k_step = fold_in(sample_key, step);
//   (w0, w1) = threefry(k_step, (env, 2p)), (w2, w3) = threefry(k_step, (env, 2p + 1));
//   factor f draws the 16-bit half f of w0..w3 (low half first) and takes the
//   ((h * popcount) >> 16)-th set bit of its mask, or 0 when the mask is empty.
// A row whose only set bit is NONE samples all zeros.
// ---------------------------------------------------------------------------
NR_DEV uint64_t row_bits(const Row& r, int32_t lo, int32_t width) {
    const uint64_t low = (uint64_t)r.w[0] | ((uint64_t)r.w[1] << 32);
    const uint64_t high = (uint64_t)r.w[2];
    uint64_t v;
    if (lo == 0) v = low;
    else if (lo < 64) v = (low >> lo) | (high << (64 - lo));
    else v = high >> (lo - 64);
    return width >= 64 ? v : (v & ((1ull << width) - 1ull));
}

NR_DEV int32_t select_set_bit(uint64_t m, int32_t k) {
    for (int32_t i = 0; i < k; ++i) m &= m - 1ull;
    return (int32_t)__builtin_ctzll(m);
}

NR_DEV bool only_none(const Row& r) { return r.w[0] == 1u && r.w[1] == 0u && r.w[2] == 0u; }

NR_DEV void sample_row(const KGame& g, const Row& r, uint32_t ks0, uint32_t ks1, uint32_t env, int32_t p, int32_t a[7]) {
    if (only_none(r)) {
#pragma unroll
        for (int f = 0; f < 7; ++f) a[f] = 0;
        return;
    }
    uint32_t w0 = env, w1 = 2u * (uint32_t)p, w2 = env, w3 = 2u * (uint32_t)p + 1u;
    threefry(ks0, ks1, w0, w1);
    threefry(ks0, ks1, w2, w3);
    const uint32_t words[4] = {w0, w1, w2, w3};
    const int32_t lo[7] = {0, 6, 10, 14, 18, 22, 22 + g.T};
    const int32_t wid[7] = {6, 4, 4, 4, 4, g.T, g.O};
#pragma unroll
    for (int f = 0; f < 7; ++f) {
        const uint32_t hh = (words[f >> 1] >> (16 * (f & 1))) & 0xFFFFu;
        const uint64_t m = row_bits(r, lo[f], wid[f]);
        const int32_t count = popc(m);
        a[f] = count > 0 ? select_set_bit(m, (int32_t)((hh * (uint32_t)count) >> 16)) : 0;
    }
}

// decode_actions for one row (N/adapters/jaxmarl/actions.py:61-84,
// N/adapters/factors.py:117-151) of an available unit, in canonical command
// form.
NR_DEV void decode_values(const KGame& g, const Env& e, int32_t p, const int32_t a[7], int32_t* kind_out,
                          int32_t* dir_out, int32_t* ptype_out, int32_t* target_out, int32_t* none_out) {
    const int32_t kind = a[0];
    int32_t dir = kAbsent;
    if (kind == kKindMove) dir = a[1];
    else if (kind == kKindHarvest) dir = a[2];
    else if (kind == kKindReturn) dir = a[3];
    else if (kind == kKindProduce) dir = a[4];
    const int32_t ptype = kind == kKindProduce ? a[5] : kAbsent;
    int32_t target = kAbsent;
    if (kind == kKindAttack) {
        const int32_t cell = e.cell[g.N + p];
        const int32_t tx = wadd(cell_x(g, cell), floor_mod(a[6], g.side) - g.radius);
        const int32_t ty = wadd(cell_y(g, cell), floor_div(a[6], g.side) - g.radius);
        if (tx >= 0 && tx < g.W && ty >= 0 && ty < g.H) target = ty * g.W + tx;
    }
    *kind_out = canon_kind(kind);
    *dir_out = canon_dir(dir);
    *ptype_out = canon_ptype(ptype, g.T);
    *target_out = target;
    *none_out = kind == kKindNone ? 1 : 0;
}

// decode_row: the same values staged in the command arrays (ABSENT when the
// unit is not available).
NR_DEV void decode_row(const KGame& g, const Env& e, int32_t p, bool available, const int32_t a[7]) {
    const Layout& y = g.lay;
    int32_t kind, dir, ptype, target, none;
    decode_values(g, e, p, a, &kind, &dir, &ptype, &target, &none);
    at<int8_t>(e, y.c_kind)[p] = (int8_t)(available ? kind : kAbsent);
    at<int8_t>(e, y.c_dir)[p] = (int8_t)(available ? dir : kAbsent);
    at<int8_t>(e, y.c_ptype)[p] = (int8_t)(available ? ptype : kAbsent);
    at<int16_t>(e, y.c_target)[p] = (int16_t)(available ? target : kAbsent);
    at<int32_t>(e, y.c_none)[p] = available ? none : 0;
    at<int16_t>(e, y.c_rank)[p] = 0;
}

// ---------------------------------------------------------------------------
// Observations (N/observations/visibility.py:56-71, symbolic.py:130-180)
// ---------------------------------------------------------------------------
// Sight-radius visibility of `observer` as a bitmap seen[H][seen_words].
NR_DEV void stamp_visibility(const KGame& g, const Hdr& h, const Env& e, int lane, int32_t observer) {
    const Layout& y = g.lay;
    AS3 uint32_t* seen = at<uint32_t>(e, y.v_seen);
    AS3 int16_t* units = at<int16_t>(e, y.b_units);
    const int32_t nwords = g.H * g.seen_words;
    for (int32_t i = lane; i < nwords; i += kWave) seen[i] = 0u;
    const int32_t block = g.N + observer * g.C;
    int32_t n = 0;
    for (int32_t base = 0; base < g.C; base += kWave) {
        const int32_t i = base + lane;
        const bool act = i < g.C && e.birth[block + i] != kAbsent;
        const uint64_t m = ballot(act);
        if (act) units[n + count_below(m)] = (int16_t)(block + i);
        n += popc(m);
    }
    wave_sync();
    const int32_t rows = 2 * g.sight_max + 1;
    const int32_t items = n * rows;
    for (int32_t w = lane; w < items; w += kWave) {
        const int32_t u = w / rows;
        const int32_t dy = w - u * rows - g.sight_max;
        const int32_t s = units[u];
        const int32_t r = tabv(h, F_SIGHT, gidx(e.utype[s], g.T));
        if (dy < -r || dy > r) continue;
        const int32_t cell = e.cell[s];
        const int32_t cy = cell_y(g, cell) + dy;
        if (cy < 0 || cy >= g.H) continue;
        const int32_t rem = r * r - dy * dy;
        int32_t hw = r;
        while (hw * hw > rem) --hw;
        const int32_t cx = cell_x(g, cell);
        const int32_t x0 = cx - hw < 0 ? 0 : cx - hw;
        const int32_t x1 = cx + hw >= g.W ? g.W - 1 : cx + hw;
        if (x0 > x1) continue;
        for (int32_t wd = x0 >> 5; wd <= (x1 >> 5); ++wd) {
            const int32_t a = x0 > wd * 32 ? x0 - wd * 32 : 0;
            const int32_t b = x1 < wd * 32 + 31 ? x1 - wd * 32 : 31;
            const uint32_t bits = (b - a == 31) ? 0xFFFFFFFFu : (((1u << (b - a + 1)) - 1u) << a);
            __atomic_fetch_or(&seen[cy * g.seen_words + wd], bits, __ATOMIC_RELAXED);
        }
    }
    wave_sync();
}

NR_DEV bool seen_at(const KGame& g, const Env& e, int32_t c) {
    const AS3 uint32_t* seen = at<uint32_t>(e, g.lay.v_seen);
    const int32_t yy = cell_y(g, c), x = c - yy * g.W;
    return (seen[yy * g.seen_words + (x >> 5)] >> (x & 31)) & 1u;
}

}  // namespace nr
