// gfx950 kernels and the C-ABI entry points of nanorts_amd.
//
// Launch shape: one wave64 per game, WPB games per workgroup; dynamic LDS =
// workgroup header (unit table + terrain) + WPB env blocks.  No entry point
// allocates device memory; all run asynchronously on the caller's stream.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/nanorts_amd.h"
#include "engine.h"
#include "rollout.h"
#include "bots.h"
#include "gridnet.h"

using namespace nr;

#ifndef NANORTS_BUILD_ID
#define NANORTS_BUILD_ID "dev"
#endif

namespace {

thread_local std::string g_error;

int fail(int code, const std::string& message) {
    g_error = message;
    return code;
}

int32_t align16(int32_t v) { return (v + 15) & ~15; }

struct Shape {
    KGame g;
    int wpb;        // waves (games) per workgroup
    int32_t lds;    // dynamic LDS bytes per workgroup
};

bool valid_game(const nanorts_game* game, std::string* why) {
    if (!game) {
        *why = "game is NULL";
        return false;
    }
    if (game->height <= 0 || game->width <= 0 || game->cells != game->height * game->width) {
        *why = "game extents are inconsistent (cells != height * width)";
        return false;
    }
    if (game->cells > 32767 || game->entities > 32767) {
        *why = "this build lays out int16 cell and slot indices only (cells and entities <= 32767)";
        return false;
    }
    if (game->capacity <= 0 || game->neutral < 0 || game->entities != game->neutral + 2 * game->capacity) {
        *why = "entities != neutral + 2 * capacity";
        return false;
    }
    if (game->types <= 0 || game->types > NANORTS_MAX_TYPES) {
        *why = "types must be in 1..8";
        return false;
    }
    int side = 1;
    while (side * side < game->offsets) ++side;
    if (side * side != game->offsets || side % 2 == 0 || 22 + game->types + game->offsets > 96) {
        *why = "offsets must be an odd square and a mask row must fit 96 bits";
        return false;
    }
    if (game->strategy < 0 || game->strategy > 2) {
        *why = "strategy must be 0 (CANCEL_BOTH), 1 (CANCEL_RANDOM) or 2 (CANCEL_ALTERNATING)";
        return false;
    }
    if (!game->terrain) {
        *why = "terrain is NULL";
        return false;
    }
    return true;
}

// Waves per workgroup that fit the device's LDS per workgroup (at most 4).
bool fit_waves(Shape* out, std::string* why) {
    const Layout& y = out->g.lay;
    int max_lds = 65536;
    int device = 0;
    if (hipGetDevice(&device) == hipSuccess) {
        int v = 0;
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, device) == hipSuccess && v > 0)
            max_lds = v;
    }
    int wpb = 4;
    while (wpb > 1 && y.hdr_bytes + wpb * y.env_bytes > max_lds) --wpb;
    if (y.hdr_bytes + wpb * y.env_bytes > max_lds) {
        *why = "one game's LDS block (" + std::to_string(y.hdr_bytes + y.env_bytes) + " bytes) exceeds the " +
               std::to_string(max_lds) + " bytes a workgroup may allocate";
        return false;
    }
    out->wpb = wpb;
    out->lds = y.hdr_bytes + wpb * y.env_bytes;
    return true;
}

// `staging` lays out observe_all's staging in the phase union; a kernel
// that writes observations from the summary's bitmaps (the seat rollout's
// first pass) does without it.
bool shape_for(const nanorts_game* game, Shape* out, std::string* why, bool staging = true) {
    if (!valid_game(game, why)) return false;
    KGame& g = out->g;
    std::memset(&g, 0, sizeof(g));
    g.H = game->height;
    g.W = game->width;
    g.cells = game->cells;
    g.N = game->neutral;
    g.C = game->capacity;
    g.E = game->entities;
    g.T = game->types;
    g.O = game->offsets;
    g.strategy = game->strategy;
    g.max_cycles = game->max_cycles;
    int side = 1;
    while (side * side < g.O) ++side;
    g.side = side;
    g.radius = (side - 1) / 2;
    int bits = 0;
    for (int v = g.C - 1; v > 0; v >>= 1) ++bits;
    g.rank_bits = bits < 1 ? 1 : bits;
    g.seen_words = (g.W + 31) / 32;
    g.stage_cells = g.cells < 256 ? g.cells : 256;
    g.sight_max = 0;
    for (int t = 0; t < g.T; ++t) {
        g.tab[F_COST * 8 + t] = game->cost[t];
        g.tab[F_HP * 8 + t] = game->hit_points[t];
        g.tab[F_PRODUCE_TIME * 8 + t] = game->produce_time[t];
        g.tab[F_MOVE_TIME * 8 + t] = game->move_time[t];
        g.tab[F_ATTACK_TIME * 8 + t] = game->attack_time[t];
        g.tab[F_HARVEST_TIME * 8 + t] = game->harvest_time[t];
        g.tab[F_RANGE * 8 + t] = game->attack_range[t];
        g.tab[F_DAMAGE * 8 + t] = game->attack_damage[t];
        g.tab[F_AMOUNT * 8 + t] = game->harvest_amount[t];
        g.tab[F_SIGHT * 8 + t] = game->sight_radius[t];
        g.tab[F_FLAGS * 8 + t] = (game->is_resource[t] ? FL_RESOURCE : 0) | (game->is_stockpile[t] ? FL_STOCKPILE : 0) |
                                 (game->can_harvest[t] ? FL_HARVEST : 0) | (game->can_move[t] ? FL_MOVE : 0) |
                                 (game->can_attack[t] ? FL_ATTACK : 0);
        int32_t produces = 0;
        for (int u = 0; u < g.T; ++u)
            if (game->produces[t * NANORTS_MAX_TYPES + u]) produces |= 1 << u;
        g.tab[F_PRODUCES * 8 + t] = produces;
        if (game->sight_radius[t] > g.sight_max) g.sight_max = game->sight_radius[t];
        if (game->produce_time[t] < 2 || game->produce_time[t] > 0x3fffffff) g.quick_produce = 1;
        if (game->sight_radius[t] < 0 || game->sight_radius[t] > 64) {
            *why = "sight radius out of range";
            return false;
        }
    }
    g.terrain = game->terrain;
    g.initial = game->initial;

    Layout& y = g.lay;
    const int32_t E = g.E, C2 = 2 * g.C, cells = g.cells;
    g.disk_r = g.sight_max;
    for (int t = 0; t < g.T; ++t)
        if (game->attack_range[t] > g.disk_r) g.disk_r = game->attack_range[t];
    g.fast_obs = (g.W % 4 == 0 && g.disk_r <= 15) ? 1 : 0;
    g.wshift = -1;
    for (int b = 0; b < 16; ++b)
        if ((1 << b) == g.W) g.wshift = b;
    y.o_seg = F_COUNT * 8 * 4;
    y.o_terrain = y.o_seg + 16 * (int32_t)sizeof(Seg);
    y.o_disk = align16(y.o_terrain + cells);
    y.o_walls = align16(y.o_disk + (g.fast_obs ? (g.disk_r + 1) * (2 * g.disk_r + 1) * 4 : 0));
    y.hdr_bytes = align16(y.o_walls + (g.fast_obs ? g.H * g.seen_words * 4 : 0));
    int32_t o = 0;
    auto take = [&o](int32_t bytes) {
        const int32_t at = o;
        o += align16(bytes);
        return at;
    };
    y.o_birth = take(E * 4);
    y.o_carried = take(E * 4);
    y.o_pnone = take(E * 4);
    y.o_pissued = take(E * 4);
    y.o_pcompl = take(E * 4);
    y.o_porder = take(E * 4);
    y.o_cell = take(E * 2);
    y.o_hp = take(E * 2);
    y.o_ptarget = take(E * 2);
    y.o_entity = take(cells * 2);
    y.o_utype = take(E);
    y.o_owner = take(E);
    y.o_pkind = take(E);
    y.o_pdir = take(E);
    y.o_pptype = take(E);
    y.o_scal = take(S_COUNT * 4);
    y.b_events = take(32 * 4);  // admission -> finish, across completion
    y.o_live = take(((E + 63) / 64) * 8);
    // Phase union, by lifetime:
    //   persistent from sampling to admission: the command arrays at 0;
    //   persistent from the summary to sampling / admission: bitmaps,
    //     available list, entry list after them;
    //   temporaries: the summary's occupant words, unit list and seen
    //     bitmaps over the (then dead) command arrays; the general
    //     admission's keys and lists over everything but the command
    //     arrays; completion records and observation staging over all.
    const int32_t union0 = o;
    y.c_kind = take(C2);
    y.c_dir = take(C2);
    y.c_ptype = take(C2);
    y.c_target = take(C2 * 2);
    y.c_none = take(C2 * 4);
    y.c_rank = take(C2 * 2);
    const int32_t commands_end = o;
    y.o_bm = take(6 * g.H * g.seen_words * 4);
    y.a_av = take(C2 * 2);
    y.a_list = take(E * 2);
    int32_t end = o;
    // general admission
    o = commands_end;
    y.b_pkey = take(C2 * 4);
    y.b_keys = take(C2 * 8);
    y.b_tmp = take(C2 * 2);
    y.b_order = take(C2 * 2);
    y.b_rank = take(E * 2);
    if (o > end) end = o;
    // summary temporaries (the command arrays are dead then)
    o = union0;
    y.o_lo = take((E + 1) * 4);  // + the empty-cell sentinel
    y.o_fl = take(E + 1);
    y.b_units = take(C2 * 2);
    y.v_seen = take(2 * g.H * g.seen_words * 4);
    if (o > commands_end) {
        // larger boards: after the persistent lists instead
        o = end;
        y.o_lo = take((E + 1) * 4);
        y.o_fl = take(E + 1);
        y.b_units = take(C2 * 2);
        y.v_seen = take(2 * g.H * g.seen_words * 4);
    }
    if (o > end) end = o;
    // completion
    o = union0;
    y.m_rec = take(C2 * 24);
    y.m_tmp = take(C2 * 2);
    if (o > end) end = o;
    // observation staging (observe_all) with its seen bitmaps
    if (staging) {
        o = union0;
        y.v_oseen = take(2 * g.H * g.seen_words * 4);
        y.v_stage = take(2 * g.stage_cells * 6);
        if (o > end) end = o;
    } else {
        y.v_oseen = y.v_stage = -1;
    }
    // masks staging (k_legality), after the occupancy bitmaps its rows read
    o = y.o_bm;
    take(6 * g.H * g.seen_words * 4);
    y.v_words = take(C2 * 12);
    if (o > end) end = o;
    y.env_bytes = align16(end);

    // initial State rows -> env block (reset_env)
    const nanorts_state& init = game->initial;
    const struct {
        const void* src;
        int32_t dst, bytes;
    } rows[15] = {
        {init.birth, y.o_birth, E * 4}, {init.unit_type, y.o_utype, E}, {init.owner, y.o_owner, E},
        {init.cell, y.o_cell, E * 2}, {init.hit_points, y.o_hp, E * 2}, {init.carried_resources, y.o_carried, E * 4},
        {init.pending_kind, y.o_pkind, E}, {init.pending_direction, y.o_pdir, E},
        {init.pending_none_duration, y.o_pnone, E * 4}, {init.pending_target_cell, y.o_ptarget, E * 2},
        {init.pending_produced_type, y.o_pptype, E}, {init.pending_issued_at, y.o_pissued, E * 4},
        {init.pending_completes_at, y.o_pcompl, E * 4}, {init.pending_order, y.o_porder, E * 4},
        {init.entity_at, y.o_entity, cells * 2},
    };
    g.nseg = 15;
    for (int k = 0; k < 15; ++k) {
        g.seg[k].src = (const uint8_t*)rows[k].src;
        g.seg[k].dst = rows[k].dst;
        g.seg[k].bytes = rows[k].bytes;
    }

    return fit_waves(out, why);
}

// Resident waves per SIMD the first pass of the fused rollout is sized for,
// and its largest workgroup, in games.  Measured at 16x16 on the bench
// workload: workgroups of 5 or 10 games (20 games per CU) ran 17 % slower
// than workgroups of 4, whose waves fall one to a SIMD.  The hardware still
// places a fifth workgroup of 4 on a CU where LDS and registers allow it.
constexpr int kLeanWavesPerSimd = 4;
constexpr int kLeanMaxGames = 4;

// LDS bytes of one CU, and a workgroup's LDS rounded up to the allocation
// granule.
int32_t lds_per_cu() {
    int device = 0, v = 0;
    if (hipGetDevice(&device) == hipSuccess &&
        hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerMultiprocessor, device) == hipSuccess && v > 0)
        return v;
    return 160 * 1024;
}
int32_t lds_granule(int32_t bytes) { return (bytes + 511) & ~511; }

// Games one CU holds for a layout, with at most `waves_per_simd` waves per
// SIMD (4 SIMDs) and `wpb` games per workgroup.
int32_t games_per_cu(const Layout& y, int wpb, int waves_per_simd) {
    const int32_t by_lds = lds_per_cu() / lds_granule(y.hdr_bytes + wpb * y.env_bytes);
    const int32_t by_waves = (4 * waves_per_simd) / wpb;
    return (by_lds < by_waves ? by_lds : by_waves) * wpb;
}

// The layout of the fused rollout's first pass (k_rollout_lean).  The state
// rows keep their offsets; the phase union holds only what a cycle on the
// one-wave path uses: the summary's bitmaps and lists that persist into the
// next cycle's sampling and admission, and the summary's temporaries.  A
// cycle that would need more (an irregular state,
// more than 64 available units or live slots) is left to the second pass,
// on the full block.  The command arrays, the request-by-request
// admission's keys, completion's member records and the staging of the
// non-packed observation have no place in this block and are never used
// by k_rollout_lean.  The entry list keeps 64 entries: the summary writes no
// more, and more than 64 entries is an irregular state.
bool shape_for_lean(const nanorts_game* game, Shape* out, std::string* why) {
    if (!shape_for(game, out, why)) return false;
    KGame& g = out->g;
    if (!g.fast_obs) {
        *why = "the first pass needs the packed observation (width a multiple of 4)";
        return false;
    }
    Layout& y = g.lay;
    const int32_t E = g.E, C2 = 2 * g.C, plane = g.H * g.seen_words;
    int32_t o = y.o_live + align16(((E + 63) / 64) * 8);
    auto take = [&o](int32_t bytes) {
        const int32_t at = o;
        o += align16(bytes);
        return at;
    };
    y.c_kind = y.c_dir = y.c_ptype = y.c_target = y.c_none = y.c_rank = 0;
    y.b_pkey = y.b_keys = y.b_tmp = y.b_order = y.b_rank = 0;
    y.m_rec = y.m_tmp = y.v_oseen = y.v_stage = y.v_words = 0;
    y.o_bm = take(6 * plane * 4);
    y.a_av = take(C2 * 2);
    y.a_list = take(kWave * 2);
    y.o_lo = take((E + 1) * 4);
    y.o_fl = take(E + 1);
    y.b_units = take(C2 * 2);
    // the rollout keeps its sight bitmaps in the event words when both
    // planes fit there, else the summary stamps them here
    y.v_seen = 2 * plane <= 32 ? 0 : take(2 * plane * 4);
    int32_t end = o;
    y.env_bytes = align16(end);
    int best = 0, best_wpb = 0;
    for (int wpb = 1; wpb <= kLeanMaxGames; ++wpb) {
        const int32_t games = y.hdr_bytes + wpb * y.env_bytes <= lds_per_cu() ? games_per_cu(y, wpb, kLeanWavesPerSimd) : 0;
        if (games > best) {
            best = games;
            best_wpb = wpb;
        }
    }
    if (best == 0) {
        *why = "one game's first-pass block does not fit a CU";
        return false;
    }
    out->wpb = best_wpb;
    out->lds = y.hdr_bytes + best_wpb * y.env_bytes;
    return true;
}

// The first pass's slot window: with more than kSlotWindow slots per player,
// the first pass stages slots [0, N + kSlotWindow) and the first
// kSlotWindow of player 1's block only (KGame::shift).  Slots are taken
// lowest-free-first, so a player's units sit at the bottom of its block; a
// game holding a unit outside the window, or where a spawn could land
// there, goes to the second pass.  On basesWorkers16x16 (70 slots a player)
// that is 68 slots of 144: the block shrinks from 7.6 KB to about 4.6 KB.
constexpr int32_t kSlotWindow = 32;
nanorts_game windowed(const nanorts_game* game, int32_t* shift) {
    nanorts_game w = *game;
    *shift = 0;
    if (game->capacity > kSlotWindow) {
        *shift = game->capacity - kSlotWindow;
        w.capacity = kSlotWindow;
        w.entities = game->neutral + 2 * kSlotWindow;
    }
    return w;
}
// The first pass with two games per wave (k_rollout_pair, half-wave
// teams): shape_for_lean's block per game, `wpb` waves (2 * wpb games) per
// workgroup, chosen for the most games per CU.  The choice among equal
// counts falls to the smaller workgroup: a workgroup holds its LDS until its
// last game's cycles end, so a small one returns a finished game's block
// soonest (at 16x16, 32 games per CU either way, workgroups of one wave ran
// the 1000-cycle bench 5.5 % faster than workgroups of four, 454 M against
// 430 M env-steps/s, as games grow apart in their units).  Half-wave teams issue fewer
// instructions per game-cycle but wait on LDS and scalar loads as often as
// whole-wave teams do, with half as many waves per game in flight: they pay
// only where at least three waves per SIMD fit (measured with the bench
// workload's settings: 8x8 boards, 32 games per CU, +12 %; 16x16, 20 games
// per CU, -8 %; 12x12, 16 games per CU, -16 %).  `any_occupancy` takes the
// shape whatever it fits.
constexpr int kPairMaxWaves = 4;
constexpr int kPairMinGamesPerCu = 2 * 3 * 4;
bool shape_for_pair(const nanorts_game* game, Shape* out, bool any_occupancy, std::string* why) {
    if (!shape_for_lean(game, out, why)) return false;
    const Layout& y = out->g.lay;
    int best = 0, best_w = 0;
    for (int w = 1; w <= kPairMaxWaves; ++w) {
        const int32_t bytes = y.hdr_bytes + 2 * w * y.env_bytes;
        if (bytes > lds_per_cu()) continue;
        const int32_t by_lds = lds_per_cu() / lds_granule(bytes);
        const int32_t by_waves = (4 * kLeanWavesPerSimd) / w;
        const int games = (by_lds < by_waves ? by_lds : by_waves) * 2 * w;
        if (games > best) {
            best = games;
            best_w = w;
        }
    }
    if (best == 0 || (!any_occupancy && best < kPairMinGamesPerCu)) {
        *why = "two games per wave pay only with at least three waves per SIMD";
        return false;
    }
    out->wpb = best_w;
    out->lds = y.hdr_bytes + 2 * best_w * y.env_bytes;
    return true;
}

// The first pass's shape on the slot window (windowed): one game per wave
// (shape_for_lean) or two (shape_for_pair).  The reset segments are the
// window's business (reset_env's windowed path), so the table stays empty.
bool shape_for_first_pass(const nanorts_game* game, bool pair, bool any_occupancy, Shape* out, std::string* why) {
    int32_t shift = 0;
    const nanorts_game w = windowed(game, &shift);
    if (!(pair ? shape_for_pair(&w, out, any_occupancy, why) : shape_for_lean(&w, out, why))) return false;
    out->g.shift = shift;
    if (shift > 0) out->g.nseg = 0;
    return true;
}


// A smaller env block for the kernels that read a few leaves: `masks` holds
// the leaves the legality rows read, the occupancy bitmaps and the staged
// words (k_legality); otherwise the block is empty (the samplers read only
// the header).  Every other offset is 0 and unused by those kernels.  More
// games then share a CU than the full block allows.
bool shape_for_reader(const nanorts_game* game, bool masks, Shape* out, std::string* why) {
    if (!shape_for(game, out, why)) return false;
    KGame& g = out->g;
    Layout& y = g.lay;
    const Layout full = y;
    std::memset(&y, 0, sizeof(y));
    y.hdr_bytes = full.hdr_bytes;
    y.o_seg = full.o_seg;
    y.o_terrain = full.o_terrain;
    y.o_disk = full.o_disk;
    y.o_walls = full.o_walls;
    int32_t o = 0;
    auto take = [&o](int32_t bytes) {
        const int32_t at = o;
        o += align16(bytes);
        return at;
    };
    if (masks) {
        const int32_t E = g.E;
        y.o_birth = take(E * 4);
        y.o_carried = take(E * 4);
        y.o_cell = take(E * 2);
        y.o_entity = take(g.cells * 2);
        y.o_utype = take(E);
        y.o_owner = take(E);
        y.o_pkind = take(E);
        y.o_scal = take(S_COUNT * 4);
        y.o_bm = take(6 * g.H * g.seen_words * 4);
        y.v_words = take(2 * g.C * 12);
    }
    y.env_bytes = align16(o > 16 ? o : 16);
    g.nseg = 0;
    return fit_waves(out, why);
}

// GridNet decode scratch (gridnet.h) in the env block's phase union, after
// the command arrays the decode fills.
bool shape_for_gridnet(const nanorts_game* game, Shape* out, GridLayout* gy, std::string* why) {
    if (!shape_for(game, out, why)) return false;
    KGame& g = out->g;
    if (g.T != 7 || g.O != 49) {
        *why = "the GridNet surface is pinned to 7 unit types and a 49-cell attack window";
        return false;
    }
    const int32_t C = g.C, words = (g.cells + 2 * g.W + 1 + 31) / 32;
    std::memset(gy, 0, sizeof(*gy));
    int32_t o = 0;
    auto take = [&o](int32_t bytes) {
        const int32_t at = o;
        o += align16(bytes);
        return at;
    };
    gy->order = take(2 * C);
    gy->list = take(2 * C);
    gy->pos = take(2 * C);
    gy->cost = take(4 * C);
    gy->kept = take(C);
    gy->base = take(4 * words);
    gy->used = take(4 * words);
    gy->bytes = align16(o);
    gy->origin = g.lay.c_rank + align16(4 * C);
    if (gy->origin + gy->bytes > g.lay.env_bytes) g.lay.env_bytes = gy->origin + gy->bytes;
    return fit_waves(out, why);
}

// Bot region after each env block (scripted bots, bots.h): the per-wave
// stride grows by the region, the env offsets stay.
// `first_pass` is the seat rollout's first pass (half-wave teams): no
// observation staging, and the carry's target, base and cell rows as int16.
bool shape_for_bots(const nanorts_game* game, Shape* out, BotLayout* by, std::string* why, bool first_pass = false) {
    if (!shape_for(game, out, why, !first_pass)) return false;
    KGame& g = out->g;
    if (g.C > 512) {
        *why = "the scripted bots take at most 512 slots per player";
        return false;
    }
    const int32_t C = g.C, E = g.E, cells = g.cells, words = (cells + 31) / 32;
    std::memset(by, 0, sizeof(*by));
    int32_t o = 0;
    auto take = [&o](int32_t bytes) {
        const int32_t at = o;
        o += align16(bytes);
        return at;
    };
    const int32_t N = g.N;
    // per unit, alive from the plan to the commands and the settled carry:
    // kinds, directions and types as bytes, cells, radii and costs as int16
    by->u_flags = take(C);
    by->u_goal = take(2 * C);
    by->u_radius = take(2 * C);
    by->u_fkind = take(C);
    by->u_fdir = take(C);
    by->u_ftarget = take(2 * C);
    by->u_fptype = take(C);
    by->u_fclaimed = take(2 * C);
    by->u_fcost = take(2 * C);
    by->u_sel = take(C);
    by->u_dir = take(C);
    by->u_drank = take(2 * C);
    by->u_queue = take(2 * C);
    by->u_live = take(2 * C);
    by->u_lbirth = take(4 * C);
    by->u_lkey = take(4 * C);
    by->m_claimed = take(4 * words);
    by->m_free = take(4 * words);
    by->m_used = take(4 * words);
    by->m_kept = take(4 * words);
    // dead once the walk starts (ranks, nearest enemies, roles, the queue's
    // scratch list, the candidate lists, the build reservations): the walk's
    // search scratch lies over them.  Enemies and own stockpiles are units of
    // one player (at most C), resources neutral units (at most N).
    const int32_t scratch = o;
    by->u_rank = take(2 * C);
    by->u_es = take(2 * C);
    by->u_eb = take(4 * C);
    by->u_role = take(C);
    by->u_list = take(2 * C);
    by->l_enemy = take(2 * C);
    by->l_resource = take(2 * N);
    by->l_stock = take(2 * C);
    by->m_reserved = take(4 * words);
    const int32_t scratch_end = o;
    o = scratch;
    by->a_below = take(2 * cells);
    by->a_mark = take(cells);
    if (o < scratch_end) o = scratch_end;
    // the carry last, past the end of the env block's phase union (which
    // the step's phases overwrite), so that a fused rollout keeps it in LDS
    // from cycle to cycle: its int32 rows, then kind and unit_type as bytes
    // (small codes) and the trained flags
    const int32_t union_end = g.lay.env_bytes - (g.lay.c_rank + align16(4 * C));
    if (o < union_end) o = align16(union_end);
    by->k_ubirth = take(4 * C);
    by->k_order = take(4 * C);
    const int32_t slot_bytes = first_pass ? 2 : 4;
    by->k_target = take(slot_bytes * C);
    by->k_tbirth = take(4 * C);
    by->k_base = take(slot_bytes * C);
    by->k_bbirth = take(4 * C);
    by->k_cell = take(slot_bytes * C);
    by->k_kind = take(C);
    by->k_utype = take(C);
    by->k_trained = take(C);
    by->bytes = align16(o);
    // The bot runs before admission, so its region shares the env block's
    // phase union after the command arrays the bot writes; only the carry
    // lies beyond the union.
    by->origin = g.lay.c_rank + align16(4 * C);
    if (by->origin + by->bytes > g.lay.env_bytes) g.lay.env_bytes = by->origin + by->bytes;
    return fit_waves(out, why);
}

template <typename Kernel, typename... Args>
int launch(Kernel kernel, const Shape& sh, int64_t lanes, hipStream_t stream, Args... args) {
    if (lanes <= 0) return NANORTS_OK;
    const int64_t blocks = (lanes + sh.wpb - 1) / sh.wpb;
    if (blocks > 0x7fffffff) return fail(NANORTS_INVALID_ARGUMENT, "too many lanes for one launch");
    hipLaunchKernelGGL(kernel, dim3((unsigned)blocks), dim3((unsigned)(kWave * sh.wpb)), (size_t)sh.lds, stream,
                       sh.g, lanes, args...);
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) return fail(NANORTS_INTERNAL, std::string("kernel launch failed: ") + hipGetErrorString(err));
    return NANORTS_OK;
}

bool state_complete(const nanorts_state& s) {
    return s.birth && s.unit_type && s.owner && s.cell && s.hit_points && s.carried_resources && s.pending_kind &&
           s.pending_direction && s.pending_none_duration && s.pending_target_cell && s.pending_produced_type &&
           s.pending_issued_at && s.pending_completes_at && s.pending_order && s.entity_at && s.time &&
           s.player_resources && s.next_birth && s.next_pending_order && s.alternating_conflict_count && s.game_over &&
           s.winner && s.spawn_overflow;
}

}  // namespace

// ---------------------------------------------------------------------------
// kernels
// ---------------------------------------------------------------------------
#define NR_KERNEL_PROLOGUE                                                        \
    extern __shared__ __align__(16) uint8_t nr_lds[];                             \
    AS3 uint8_t* lds = (AS3 uint8_t*)nr_lds;                                      \
    Hdr hdr;                                                                      \
    hdr.tab = (AS3 int32_t*)lds;                                                  \
    hdr.terrain = lds + g.lay.o_terrain;                                          \
    hdr.seg = (AS3 Seg*)(lds + g.lay.o_seg);                                      \
    hdr.disk = (AS3 uint32_t*)(lds + g.lay.o_disk);                               \
    hdr.walls = (AS3 uint32_t*)(lds + g.lay.o_walls);                             \
    load_header(g, hdr);                                                          \
    __syncthreads();                                                              \
    const int lane = lane_id();                                                   \
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));     \
    const int64_t l = (int64_t)blockIdx.x * (blockDim.x >> 6) + wave;             \
    if (l >= lanes) return;                                                       \
    const Env e = env_view(g, lds + g.lay.hdr_bytes + wave * g.lay.env_bytes);

// The prologue with the unit table taken from a table operand of the
// reference (load_operand_table) instead of the game's own.
#define NR_KERNEL_PROLOGUE_OPERAND_TABLE(rows, cols)                              \
    extern __shared__ __align__(16) uint8_t nr_lds[];                             \
    AS3 uint8_t* lds = (AS3 uint8_t*)nr_lds;                                      \
    Hdr hdr;                                                                      \
    hdr.tab = (AS3 int32_t*)lds;                                                  \
    hdr.terrain = lds + g.lay.o_terrain;                                          \
    hdr.seg = (AS3 Seg*)(lds + g.lay.o_seg);                                      \
    hdr.disk = (AS3 uint32_t*)(lds + g.lay.o_disk);                               \
    hdr.walls = (AS3 uint32_t*)(lds + g.lay.o_walls);                             \
    load_header(g, hdr);                                                          \
    load_operand_table(g, hdr, rows, cols);                                       \
    __syncthreads();                                                              \
    const int lane = lane_id();                                                   \
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));     \
    const int64_t l = (int64_t)blockIdx.x * (blockDim.x >> 6) + wave;             \
    if (l >= lanes) return;                                                       \
    const Env e = env_view(g, lds + g.lay.hdr_bytes + wave * g.lay.env_bytes);

// Canonical commands from the reference's int32 Commands operands.
NR_DEV void stage_commands(const KGame& g, const Env& e, int64_t l, const nanorts_commands& c, int lane) {
    const Layout& y = g.lay;
    const int32_t owned = 2 * g.C;
    const int32_t top = (1 << g.rank_bits) - 1;
    for (int32_t p = lane; p < owned; p += kWave) {
        const int64_t i = l * owned + p;
        at<int8_t>(e, y.c_kind)[p] = (int8_t)canon_kind(c.kind[i]);
        at<int8_t>(e, y.c_dir)[p] = (int8_t)canon_dir(c.direction[i]);
        at<int8_t>(e, y.c_ptype)[p] = (int8_t)canon_ptype(c.produced_type[i], g.T);
        at<int16_t>(e, y.c_target)[p] = (int16_t)canon_target(c.target_cell[i], g.cells);
        at<int32_t>(e, y.c_none)[p] = c.none_duration[i];
        const int32_t ro = c.request_order[i];
        at<int16_t>(e, y.c_rank)[p] = (int16_t)clampi(ro == kAbsent ? 0 : ro, 0, top);
    }
    wave_sync();
}

NR_DEV void write_events(const KGame& g, const Env& e, int64_t l, const nanorts_step_results& r, int lane) {
    const AS3 int32_t* ev = at<int32_t>(e, g.lay.b_events);
    if (r.admitted_harvest && lane < 2) r.admitted_harvest[2 * l + lane] = ev[lane];
    if (r.admitted_return && lane < 2) r.admitted_return[2 * l + lane] = ev[2 + lane];
    if (r.admitted_produce && lane < 2 * g.T) {
        const int32_t pl = lane / g.T, t = lane % g.T;
        r.admitted_produce[(2 * l + pl) * g.T + t] = ev[4 + pl * 8 + t];
    }
    if (r.admitted_attack && lane < 6) r.admitted_attack[6 * l + lane] = ev[20 + lane];
}

// The completion records of env l when the caller asked for them: every
// row zeroed (a member's turn then writes its own).
NR_DEV bool begin_records(const KGame& g, const nanorts_step_results& r, int64_t l, StepRecords* rec, int lane) {
    if (!r.is_member || !r.records_i32 || !r.records_i16 || !r.records_i8) return false;
    const int64_t E = g.E;
    rec->member = r.is_member + l * E;
    rec->wide = r.records_i32 + l * E * 6;
    rec->index = r.records_i16 + l * E * 4;
    rec->narrow = r.records_i8 + l * E * 6;
    for (int32_t i = lane; i < g.E; i += kWave) rec->member[i] = 0;
    for (int32_t i = lane; i < 6 * g.E; i += kWave) {
        rec->wide[i] = 0;
        rec->narrow[i] = 0;
    }
    for (int32_t i = lane; i < 4 * g.E; i += kWave) rec->index[i] = 0;
    wave_sync();
    return true;
}

// core.step on Commands [cmd_lanes][2][C] (cmd_lanes 1 broadcasts one row
// to every lane, the reference's extent-1 operand) and keys [key_lanes][2].
__global__ __launch_bounds__(256) void k_step(KGame g, int64_t lanes, nanorts_state s, const uint32_t* key, int64_t key_lanes,
                       nanorts_commands c, int64_t cmd_lanes, nanorts_step_results r) {
    NR_KERNEL_PROLOGUE
    load_env(g, s, l, e, LD_ALL, lane);
    count_units(g, e, lane);
    stage_commands(g, e, cmd_lanes == 1 ? 0 : l, c, lane);
    const int64_t kl = key_lanes == 1 ? 0 : l;
    const uint32_t k0 = key[2 * kl], k1 = key[2 * kl + 1];
    const bool events = r.admitted_harvest || r.admitted_return || r.admitted_produce || r.admitted_attack;
    StepRecords rec;
    const bool records = begin_records(g, r, l, &rec, lane);
    core_step(g, hdr, e, lane, k0, k1, events, records ? &rec : nullptr);
    store_env(g, s, l, e, lane);
    if (lane == 0) {
        const bool over = e.sc[S_GAME_OVER] != 0;
        const bool trunc = !over && e.sc[S_TIME] >= g.max_cycles;
        if (r.terminated) r.terminated[l] = over ? 1 : 0;
        if (r.truncated) r.truncated[l] = trunc ? 1 : 0;
        if (r.reward) {
            const int32_t winner = e.sc[S_WINNER];
            for (int p = 0; p < 2; ++p) r.reward[2 * l + p] = (over || trunc) ? (p == winner ? 1.0f : -1.0f) : 0.0f;
        }
    }
    if (events) write_events(g, e, l, r, lane);
}

// Zero bytes [0, n) of a device buffer with 16-byte stores where the pointer
// allows (a fill kernel rather than a memset node, so a captured graph
// replays it correctly).
__global__ __launch_bounds__(256) void k_zero_bytes(uint8_t* p, int64_t n) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t to_aligned = (int64_t)((16u - ((uintptr_t)p & 15u)) & 15u);
    const int64_t head = to_aligned < n ? to_aligned : n;
    const int64_t vecs = (n - head) >> 4;
    for (int64_t k = i; k < head; k += stride) p[k] = 0;
    typedef uint32_t v4 __attribute__((ext_vector_type(4)));
    v4* body = (v4*)(p + head);
    for (int64_t k = i; k < vecs; k += stride) body[k] = v4{0u, 0u, 0u, 0u};
    for (int64_t k = head + (vecs << 4) + i; k < n; k += stride) p[k] = 0;
}

// core.step over several groups of lanes in one launch (step_groups,
// N/core/cuda/step.cu:704-808): the groups share one bucket and unit table,
// so one LDS shape serves every workgroup; each group brings its own State,
// Commands, keys, results, terrain and horizon.  Workgroups are handed out
// group after group (first_block), and every workgroup reads its group's
// slot through the kernel-argument segment pointer, which a runtime index
// into the slots needs.
constexpr int32_t kGroupsPerLaunch = 4;
struct GroupSlot {
    nanorts_state s;
    nanorts_commands c;
    nanorts_step_results r;
    const uint32_t* key;
    int64_t key_lanes;
    int64_t cmd_lanes;  // 1: one Commands row for every lane
    int64_t lanes;
    const uint8_t* terrain;
    const int32_t* table;    // the group's own table / timings operands, or NULL: the launch's table
    const int32_t* timings;
    int32_t max_cycles;
    uint32_t first_block;
};
struct GroupsArgs {
    KGame g;  // first: fresh_game() reads it at offset 0
    int32_t count;
    GroupSlot slot[kGroupsPerLaunch];
};
static_assert(sizeof(GroupsArgs) <= 4096, "the group table must fit the kernel-argument segment");
typedef const __attribute__((address_space(4))) GroupsArgs* GroupsArgsArg;

__global__ __launch_bounds__(256) void k_step_groups(GroupsArgs args) {
    (void)args;
    GroupsArgsArg ap = (GroupsArgsArg)__builtin_amdgcn_kernarg_segment_ptr();
    const GroupsArgs& a = *(const GroupsArgs*)ap;
    const KGame& g = a.g;
    int32_t gi = 0;
    for (int32_t i = 1; i < a.count; ++i)
        if (blockIdx.x >= a.slot[i].first_block) gi = i;
    const GroupSlot& sl = a.slot[gi];
    extern __shared__ __align__(16) uint8_t nr_lds[];
    AS3 uint8_t* lds = (AS3 uint8_t*)nr_lds;
    Hdr hdr;
    hdr.tab = (AS3 int32_t*)lds;
    hdr.terrain = lds + g.lay.o_terrain;
    hdr.seg = (AS3 Seg*)(lds + g.lay.o_seg);
    hdr.disk = (AS3 uint32_t*)(lds + g.lay.o_disk);
    hdr.walls = (AS3 uint32_t*)(lds + g.lay.o_walls);
    load_header(g, hdr, sl.terrain, sl.table ? sl.table : g.ref_table, sl.table ? sl.timings : g.ref_timings);
    __syncthreads();
    const int lane = lane_id();
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int64_t l = (int64_t)(blockIdx.x - sl.first_block) * (blockDim.x >> 6) + wave;
    if (l >= sl.lanes) return;
    const Env e = env_view(g, lds + g.lay.hdr_bytes + wave * g.lay.env_bytes);
    load_env(g, sl.s, l, e, LD_ALL, lane);
    count_units(g, e, lane);
    stage_commands(g, e, sl.cmd_lanes == 1 ? 0 : l, sl.c, lane);
    const int64_t kl = sl.key_lanes == 1 ? 0 : l;
    const uint32_t k0 = sl.key[2 * kl], k1 = sl.key[2 * kl + 1];
    const nanorts_step_results r = sl.r;
    const bool events = r.admitted_harvest || r.admitted_return || r.admitted_produce || r.admitted_attack;
    StepRecords rec;
    const bool records = begin_records(g, r, l, &rec, lane);
    core_step(g, hdr, e, lane, k0, k1, events, records ? &rec : nullptr);
    store_env(g, sl.s, l, e, lane);
    if (lane == 0) {
        const bool over = e.sc[S_GAME_OVER] != 0;
        const bool trunc = !over && e.sc[S_TIME] >= sl.max_cycles;
        if (r.terminated) r.terminated[l] = over ? 1 : 0;
        if (r.truncated) r.truncated[l] = trunc ? 1 : 0;
        if (r.reward) {
            const int32_t winner = e.sc[S_WINNER];
            for (int p = 0; p < 2; ++p) r.reward[2 * l + p] = (over || trunc) ? (p == winner ? 1.0f : -1.0f) : 0.0f;
        }
    }
    if (events) write_events(g, e, l, r, lane);
}

// Legality words of every owned row into the staged words area; `merge`
// applies availability (only NONE on unavailable rows).
// The rows come from the occupancy bitmaps (legality_row_w1 on boards of at
// most 32 columns, legality_row_bm otherwise), the same bits as legality_row.
NR_DEV void stage_words(const KGame& g, const Hdr& h, const Env& e, int lane, bool merge) {
    build_bitmaps(g, h, e, lane);
    const bool narrow = g.fast_obs && g.seen_words == 1;
    const Affordable aff = affordable_types(g, h, e, lane);
    AS3 uint32_t* words = at<uint32_t>(e, g.lay.v_words);
    for (int32_t p = lane; p < 2 * g.C; p += kWave) {
        const int32_t s = g.N + p;
        Row r;
        const bool available = e.birth[s] != kAbsent && e.pkind[s] == kAbsent;
        if (merge && !available) {
            r.w[0] = 1u;
            r.w[1] = r.w[2] = 0u;
        } else {
            r = narrow ? legality_row_w1(g, h, e, s, aff) : legality_row_bm(g, h, e, s);
        }
        words[3 * p] = r.w[0];
        words[3 * p + 1] = r.w[1];
        words[3 * p + 2] = r.w[2];
    }
    wave_sync();
}

NR_DEV void emit_rows(const KGame& g, const Env& e, int64_t l, uint8_t* rows, int lane) {
    const AS3 uint32_t* words = at<uint32_t>(e, g.lay.v_words);
    const int32_t width = 22 + g.T + g.O;
    const int32_t total = 2 * g.C * width;
    uint8_t* out = rows + l * (int64_t)total;
    if ((((uintptr_t)out) & 3u) == 0 && (total & 3) == 0) {
        for (int32_t d = lane; d < total / 4; d += kWave) {
            // one division a word: its four bytes step through the row,
            // into the next one past its last bit (width > 4)
            int32_t row = (4 * d) / width, bit = 4 * d - row * width;
            uint32_t v = 0u;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                v |= ((words[3 * row + (bit >> 5)] >> (bit & 31)) & 1u) << (8 * k);
                if (++bit == width) {
                    bit = 0;
                    ++row;
                }
            }
            ((uint32_t*)out)[d] = v;
        }
    } else {
        for (int32_t b = lane; b < total; b += kWave) {
            const int32_t row = b / width, bit = b - row * width;
            out[b] = (uint8_t)((words[3 * row + (bit >> 5)] >> (bit & 31)) & 1u);
        }
    }
}

__global__ __launch_bounds__(256) void k_legality(KGame g, int64_t lanes, nanorts_state s, int32_t merge, uint8_t* rows, uint32_t* words) {
    NR_KERNEL_PROLOGUE
    load_env(g, s, l, e, LD_BIRTH | LD_UTYPE | LD_OWNER | LD_CELL | LD_CARRIED | LD_PKIND | LD_ENTITY | LD_SCALARS,
             lane);
    stage_words(g, hdr, e, lane, merge != 0);
    if (words) copy_out((uint8_t*)(words + l * 2 * g.C * 3), at<uint8_t>(e, g.lay.v_words), 2 * g.C * 12, lane);
    if (rows) emit_rows(g, e, l, rows, lane);
}

__global__ __launch_bounds__(256) void k_visible(KGame g, int64_t lanes, nanorts_state s, int32_t observer, uint8_t* cells) {
    NR_KERNEL_PROLOGUE
    load_env(g, s, l, e, LD_BIRTH | LD_UTYPE | LD_CELL, lane);
    stamp_visibility(g, hdr, e, lane, observer);
    for (int32_t c = lane; c < g.cells; c += kWave) cells[l * g.cells + c] = seen_at(g, e, c) ? 1 : 0;
}

// Legality from the operands of the reference's nanorts_legality targets: the
// seven leaves the rows read (no pending leaf, no scalar but the resources).
__global__ __launch_bounds__(256) void k_legality_operands(KGame g, int64_t lanes, nanorts_state s, uint8_t* rows,
                                                           uint32_t* words) {
    NR_KERNEL_PROLOGUE
    load_env(g, s, l, e, LD_BIRTH | LD_UTYPE | LD_OWNER | LD_CELL | LD_CARRIED | LD_ENTITY, lane);
    if (lane < 2) e.sc[S_RES0 + lane] = s.player_resources[2 * l + lane];
    wave_sync();
    stage_words(g, hdr, e, lane, false);
    if (words) copy_out((uint8_t*)(words + l * 2 * g.C * 3), at<uint8_t>(e, g.lay.v_words), 2 * g.C * 12, lane);
    if (rows) emit_rows(g, e, l, rows, lane);
}

// Sight of one slot block, from the operands of the reference's
// nanorts_visible_cells target: per-slot leaves with a row per lane or one
// shared row (stride 0), a shared radius table, any board up to 48K cells.
struct VisibleArgs {
    const int32_t* birth;
    const int8_t* unit_type;
    const uint8_t* cell;  // int8, int16 or int32 elements (cell_bytes)
    const int32_t* radius;
    uint8_t* out;
    int64_t birth_stride, type_stride, cell_stride;  // elements per lane
    int64_t types, lanes, first, count;
    int32_t width, height, cell_bytes, words;  // words: bitmap words per lane
};

NR_DEV int64_t cell_element(const uint8_t* base, int32_t bytes, int64_t i) {
    if (bytes == 1) return ((const int8_t*)base)[i];
    if (bytes == 2) return ((const int16_t*)base)[i];
    return ((const int32_t*)base)[i];
}

// Sets bits [lo, hi] of an LDS bitmap.
NR_DEV void set_bit_run(AS3 uint32_t* bm, int64_t lo, int64_t hi) {
    for (int64_t w = lo >> 5; w <= (hi >> 5); ++w) {
        const int32_t a = w == (lo >> 5) ? (int32_t)(lo & 31) : 0;
        const int32_t b = w == (hi >> 5) ? (int32_t)(hi & 31) : 31;
        const uint32_t m = (b == 31 ? 0xFFFFFFFFu : ((2u << b) - 1u)) & ~((1u << a) - 1u);
        __atomic_fetch_or(&bm[w], m, __ATOMIC_RELAXED);
    }
}

// One wave per lane: each lane of the wave takes slots of the block and ORs
// its disk, row by row as runs of the flat cell bitmap, into LDS; the wave
// then writes the bitmap out as one bool per cell.
__global__ __launch_bounds__(256) void k_visible_block(VisibleArgs a) {
    extern __shared__ __align__(16) uint8_t nr_lds[];
    const int lane = lane_id();
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int64_t l = (int64_t)blockIdx.x * (blockDim.x >> 6) + wave;
    if (l >= a.lanes) return;
    AS3 uint32_t* bm = (AS3 uint32_t*)nr_lds + (int64_t)wave * a.words;
    for (int32_t i = lane; i < a.words; i += kWave) bm[i] = 0u;
    wave_sync();
    const int64_t cells = (int64_t)a.width * a.height;
    for (int64_t slot = a.first + lane; slot < a.first + a.count; slot += kWave) {
        if (a.birth[l * a.birth_stride + slot] == kAbsent) continue;
        const int64_t c = cell_element(a.cell, a.cell_bytes, l * a.cell_stride + slot);
        const int64_t t = a.unit_type[l * a.type_stride + slot];
        if (c < 0 || c >= cells || t < 0 || t >= a.types) continue;
        const int64_t r = a.radius[t];
        if (r < 0) continue;
        const int64_t x = c % a.width, y = c / a.width;
        const int64_t y0 = y - r < 0 ? 0 : y - r, y1 = y + r > a.height - 1 ? a.height - 1 : y + r;
        int64_t w = r;  // half-width of the disk's row: the largest w with w^2 + dy^2 <= r^2
        for (int64_t yy = y0; yy <= y1; ++yy) {
            const int64_t dy = yy - y, room = r * r - dy * dy;
            w = r;
            while (w * w > room) --w;
            const int64_t x0 = x - w < 0 ? 0 : x - w, x1 = x + w > a.width - 1 ? a.width - 1 : x + w;
            set_bit_run(bm, yy * a.width + x0, yy * a.width + x1);
        }
    }
    wave_sync();
    uint8_t* out = a.out + l * cells;
    const bool packed = ((((uintptr_t)out) | (uintptr_t)cells) & 3u) == 0;
    if (packed) {
        for (int64_t q = lane; q < cells / 4; q += kWave) {
            const uint32_t bits = (bm[q >> 3] >> ((q & 7) * 4)) & 0xFu;
            ((uint32_t*)out)[q] = (bits & 1u) | ((bits & 2u) << 7) | ((bits & 4u) << 14) | ((bits & 8u) << 21);
        }
    } else {
        for (int64_t c = lane; c < cells; c += kWave) out[c] = (uint8_t)((bm[c >> 5] >> (c & 31)) & 1u);
    }
}

// Masked row select of the reference's nanorts_reset_where_done and
// nanorts_reset_packed_where_done targets: result[k][l] = done[l] ?
// reset[k][row l, or the shared row] : ending[k][l].  A result that aliases
// its ending rows is written on done lanes only.  Read through the
// kernel-argument segment pointer, as the leaf index is a run-time value.
constexpr int32_t kMaxResetLeaves = 32;
struct ResetArgs {
    const uint8_t* done;
    int64_t lanes;
    int32_t leaves;
    const uint8_t* reset[kMaxResetLeaves];
    int64_t reset_stride[kMaxResetLeaves];  // bytes per lane, 0 for a shared row
    const uint8_t* ending[kMaxResetLeaves];
    uint8_t* result[kMaxResetLeaves];
    int64_t row_bytes[kMaxResetLeaves];
};
static_assert(sizeof(ResetArgs) <= 4096, "the reset table must fit the kernel-argument segment");
typedef const __attribute__((address_space(4))) ResetArgs* ResetArgsArg;

__global__ __launch_bounds__(256) void k_reset_rows(ResetArgs args) {
    (void)args;
    ResetArgsArg ap = (ResetArgsArg)__builtin_amdgcn_kernarg_segment_ptr();
    const ResetArgs& a = *(const ResetArgs*)ap;
    const int32_t k = (int32_t)blockIdx.y;
    const int lane = lane_id();
    const int64_t l = (int64_t)blockIdx.x * (blockDim.x >> 6) + __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    if (l >= a.lanes) return;
    const bool done = a.done[l] != 0;
    const int64_t rb = a.row_bytes[k];
    uint8_t* dst = a.result[k] + l * rb;
    if (!done && a.result[k] == a.ending[k]) return;
    const uint8_t* src = done ? a.reset[k] + l * a.reset_stride[k] : a.ending[k] + l * rb;
    const uintptr_t align = (uintptr_t)src | (uintptr_t)dst | (uintptr_t)rb;
    if ((align & 15u) == 0) {
        for (int64_t i = lane; i < rb / 16; i += kWave) ((u32x4*)dst)[i] = ((const u32x4*)src)[i];
    } else if ((align & 3u) == 0) {
        for (int64_t i = lane; i < rb / 4; i += kWave) ((uint32_t*)dst)[i] = ((const uint32_t*)src)[i];
    } else {
        for (int64_t i = lane; i < rb; i += kWave) dst[i] = src[i];
    }
}

NR_DEV void observe_both(const KGame& g, const Hdr& h, const Env& e, int64_t slot, int lane, bool partial,
                         uint8_t* maps, int32_t* scalars) {
    const int64_t per = (int64_t)g.cells * 6;
    observe_all(g, h, e, lane, partial, maps ? maps + (slot * 2) * per : nullptr,
                maps ? maps + (slot * 2 + 1) * per : nullptr, scalars ? scalars + slot * 8 : nullptr,
                scalars ? scalars + slot * 8 + 4 : nullptr);
}

__global__ __launch_bounds__(256) void k_observe(KGame g, int64_t lanes, nanorts_state s, int32_t partial, uint8_t* maps, int32_t* scalars) {
    NR_KERNEL_PROLOGUE
    load_env(g, s, l, e,
             LD_BIRTH | LD_UTYPE | LD_OWNER | LD_CELL | LD_HP | LD_CARRIED | LD_PKIND | LD_ENTITY | LD_SCALARS, lane);
    observe_both(g, hdr, e, l, lane, partial != 0, maps, scalars);
}

__global__ __launch_bounds__(256) void k_reset(KGame g, int64_t lanes, nanorts_state s, const uint8_t* done) {
    NR_KERNEL_PROLOGUE
    if (!done[l]) return;
    load_env(g, s, l, e, LD_SCALARS, lane);
    reset_env(g, hdr, e, lane);
    store_env(g, s, l, e, lane);
}

// After core.step: outcome, rewards, optional final observation, auto-reset.
// `known` / `known_time`: the cycle's outcome and time from decide_counted
// and complete, when the caller holds them (else read from the env).
// A half-wave team (TW = 32) writes rewards and done flags only (no event
// counts, no final observation).
template <int TW = kWave, bool Window = false>
NR_DEV bool finish_step(const KGame& g, const Hdr& h, const Env& e, int64_t l, int lane, bool partial,
                        const nanorts_env_results& r, bool events, bool fast_obs = false, bool reset = true,
                        const Outcome* known = nullptr, int32_t known_time = 0) {
    const bool over = known ? known->over != 0 : tuni<TW>(e.sc[S_GAME_OVER]) != 0;
    const int32_t time = known ? known_time : tuni<TW>(e.sc[S_TIME]);
    const int32_t winner = known ? known->winner : tuni<TW>(e.sc[S_WINNER]);
    const bool trunc = !over && time >= g.max_cycles;
    const bool done = over || trunc;
    if (lane == 0) {
        if (r.reward)
            for (int p = 0; p < 2; ++p) r.reward[2 * l + p] = done ? (p == winner ? 1.0f : -1.0f) : 0.0f;
        if (r.done) r.done[l] = done ? 1 : 0;
        if (r.terminated) r.terminated[l] = over ? 1 : 0;
        if (r.truncated) r.truncated[l] = trunc ? 1 : 0;
        if (r.winner) r.winner[l] = winner;
        if (r.spawn_overflowed) r.spawn_overflowed[l] = (e.sc[S_SO0] > 0 || e.sc[S_SO1] > 0) ? 1 : 0;
        if (r.spawn_overflow) {
            r.spawn_overflow[2 * l] = e.sc[S_SO0];
            r.spawn_overflow[2 * l + 1] = e.sc[S_SO1];
        }
    }
    if constexpr (TW == kWave) {  // the event counts and the final observation
        if (events && r.reward_components && lane < 2) {
            // N/adapters/rewards.py:47-71 (encode_components)
            const AS3 int32_t* ev = at<int32_t>(e, g.lay.b_events);
            const int p = lane, o = lane ^ 1;
            const AS3 int32_t* prod = ev + 4 + p * 8;
            float* out = r.reward_components + (2 * l + p) * 6;
            out[0] = over ? (winner == p ? 1.0f : -1.0f) : 0.0f;
            out[1] = (float)(ev[p] + ev[2 + p]);
            out[2] = (float)prod[3];
            out[3] = (float)(prod[1] + prod[2]);
            out[4] = (float)(ev[20 + p * 3 + o + 1] - ev[20 + p * 3 + p + 1]);
            out[5] = (float)(prod[4] + prod[5] + prod[6]);
        }
        if (fast_obs && (r.final_feature_maps || r.final_scalars)) {
            const int64_t per = (int64_t)g.cells * 6;
            uint8_t* m0 = r.final_feature_maps ? r.final_feature_maps + (l * 2) * per : nullptr;
            int32_t* s0 = r.final_scalars ? r.final_scalars + l * 8 : nullptr;
            summarize(g, h, e, lane, partial, m0, m0 ? m0 + per : nullptr, s0, s0 ? s0 + 4 : nullptr);
        } else if (r.final_feature_maps || r.final_scalars) {
            observe_both(g, h, e, l, lane, partial, r.final_feature_maps, r.final_scalars);
        }
    }
    if (done && reset) reset_env<TW, Window>(g, h, e, lane);
    return done;
}

__global__ __launch_bounds__(256) void k_env_step(KGame g, int64_t lanes, nanorts_state s, const int32_t* actions, int32_t partial,
                           nanorts_env_results r, int32_t reset) {
    NR_KERNEL_PROLOGUE
    load_env(g, s, l, e, LD_ALL, lane);
    count_units(g, e, lane);
    const int32_t owned = 2 * g.C;
    uint32_t k0 = (uint32_t)uni(e.sc[S_ROOT0]), k1 = (uint32_t)uni(e.sc[S_ROOT1]);
    fold_in(k0, k1, (uint32_t)uni(e.sc[S_EPISODE]));
    const bool events = r.reward_components != nullptr;
    // the summary path encodes observations with 8-byte stores
    const bool fast = g.fast_obs && ((((uintptr_t)r.feature_maps) | ((uintptr_t)r.final_feature_maps)) & 7u) == 0;
    bool fused = false;
    if (fast) {
        // lists of the summary, then decode straight into the admission's
        // request registers (no staging through the command arrays)
        summarize_slots(g, hdr, e, lane, false);
        const int32_t n = uni(e.sc[S_NAV]);
        int32_t nA = 0, posA[1] = {0}, costA[1] = {0}, playerA[1] = {0};
        fused = uni(e.sc[S_IRREG]) == 0 && n <= kWave && admit_entries(g, hdr, e, lane, true, &nA, posA, costA, playerA);
        if (fused) {
            if (events) {
                if (lane < 32) at<int32_t>(e, g.lay.b_events)[lane] = 0;
                wave_sync();
            }
            Reqs q;
            no_request(q);
            if (lane < n) {
                const int32_t p = at<int16_t>(e, g.lay.a_av)[lane];
                const int32_t* row = actions + (l * owned + p) * 7;
                int32_t a[7];
#pragma unroll
                for (int f = 0; f < 7; ++f) a[f] = row[f];
                int32_t kind, dir, ptype, target, none;
                decode_values(g, e, p, a, &kind, &dir, &ptype, &target, &none);
                request_of(g, hdr, e, p, kind, dir, ptype, target, none, false, events, q);
            }
            wave_sync();
            admit_resolve(g, hdr, e, lane, k0, k1, n, nA, posA, costA, playerA, q);
            complete(g, hdr, e, lane);
            decide_counted(e, lane);
        }
    }
    if (!fused) {
        bool irregular = false;
        const int32_t n = compact_available(g, e, lane, &irregular);
        AS3 const int16_t* av = at<int16_t>(e, g.lay.a_av);
        for (int32_t i = lane; i < n; i += kWave) {
            const int32_t p = av[i];
            const int32_t* row = actions + (l * owned + p) * 7;
            int32_t a[7];
#pragma unroll
            for (int f = 0; f < 7; ++f) a[f] = row[f];
            decode_row(g, e, p, true, a);
        }
        wave_sync();
        env_core_step(g, hdr, e, lane, k0, k1, events, n, irregular, false);
    }
    finish_step(g, hdr, e, l, lane, partial != 0, r, events, fast, reset != 0);
    store_env(g, s, l, e, lane);
    if (fast) {
        const int64_t per = (int64_t)g.cells * 6;
        uint8_t* m0 = r.feature_maps ? r.feature_maps + (l * 2) * per : nullptr;
        int32_t* s0 = r.scalars ? r.scalars + l * 8 : nullptr;
        summarize(g, hdr, e, lane, partial != 0, m0, m0 ? m0 + per : nullptr, s0, s0 ? s0 + 4 : nullptr);
    } else if (r.feature_maps || r.scalars) {
        observe_both(g, hdr, e, l, lane, partial != 0, r.feature_maps, r.scalars);
    }
}

// Scripted-bot arguments: the bot region layout, the carry and the strategy.
struct BotArgs {
    BotLayout y;
    BotCarry carry;
    int32_t strategy, trained;
};

// family.act for the rush strategies (N/bots/family.py:34-41): commands
// int32[L][6][2][C] and the carry updated in place.
NR_DEV void act_and_emit(const KGame& g, const Hdr& hdr, const Env& e, const BotArgs& a, int64_t l,
                         const int32_t* player, int64_t player_lanes, int32_t* commands, int lane) {
    Bot b;
    b.base = e.base + a.y.origin;
    b.player = clampi(player[player_lanes == 1 ? 0 : l], 0, 1);
    b.block = g.N + b.player * g.C;
    const int32_t kept = bot_act(g, hdr, e, b, a.y, l, a.carry, a.strategy, a.trained, lane);
    const int32_t owned = 2 * g.C;
    int32_t* out = commands + l * 6 * owned;
    for (int32_t p = lane; p < owned; p += kWave) {
        int32_t v[6] = {kAbsent, kAbsent, 0, kAbsent, kAbsent, kAbsent};
        if (p / g.C == b.player) unit_command(g, e, b, a.y, p - b.player * g.C, kept, v);
#pragma unroll
        for (int f = 0; f < 6; ++f) out[f * owned + p] = v[f];
    }
    settle_carry(g, b, a.y, l, a.carry, lane);
}

__global__ __launch_bounds__(256) void k_abstraction_act(KGame g, int64_t lanes, nanorts_state s, BotArgs a,
                                                         const int32_t* player, int64_t player_lanes,
                                                         int32_t* commands) {
    NR_KERNEL_PROLOGUE
    load_env(g, s, l, e, LD_ALL, lane);
    act_and_emit(g, hdr, e, a, l, player, player_lanes, commands, lane);
}

// family.act from the reference's operands: the ten State leaves the act
// reads (the bots read no others), each one row per lane or one row shared by
// every lane; `shared` holds the LD_* flags of the shared ones, LD_SCALARS
// standing for player_resources.  The balances are the only scalars set.
__global__ __launch_bounds__(256) void k_abstraction_act_operands(KGame g, int64_t lanes, nanorts_state s,
                                                                  const int32_t* table, uint32_t shared, BotArgs a,
                                                                  const int32_t* player, int64_t player_lanes,
                                                                  int32_t* commands) {
    NR_KERNEL_PROLOGUE_OPERAND_TABLE(table, 6)
    const uint32_t read = LD_BIRTH | LD_UTYPE | LD_OWNER | LD_CELL | LD_CARRIED | LD_PKIND | LD_PDIR | LD_PPTYPE | LD_ENTITY;
    load_env(g, s, l, e, read & ~shared, lane);
    if ((read & shared) != 0u) load_env(g, s, 0, e, read & shared, lane);
    if (lane < S_COUNT) {
        const int64_t row = (shared & LD_SCALARS) ? 0 : l;
        e.sc[lane] = lane == S_RES0 ? s.player_resources[2 * row] : (lane == S_RES1 ? s.player_resources[2 * row + 1] : 0);
    }
    wave_sync();
    act_and_emit(g, hdr, e, a, l, player, player_lanes, commands, lane);
}

// The A* FFI targets: one wave per lane, each wave's scratch in its own LDS
// region (mark bytes, then the below and depth int16 rows, then the chain's
// flag bytes); operands hold one row per lane or one shared row (stride 0).
struct AstarArgs {
    const uint8_t* free;      // [cells] bool
    const uint8_t* claimed;   // chain: [cells] bool
    const int32_t* start;     // search: start, target, range
    const int32_t* target;
    const int32_t* range;
    const int32_t* rows;      // chain: [capacity][columns]
    const int32_t* queue;     // chain: [capacity]
    const int32_t* count;     // chain: scalars count, may_move, reserved, balance
    const uint8_t* moves;
    const int32_t* reserved;
    const int32_t* balance;
    const int32_t* draws;     // chain: [draw_count]
    int64_t free_stride, claimed_stride, start_stride, target_stride, range_stride, rows_stride, queue_stride,
        count_stride, moves_stride, reserved_stride, balance_stride, draws_stride;
    int64_t lanes, capacity, columns, draw_count;
    int32_t W, H, waves, region, drawing;
    int32_t fallback[3], blocked[3];  // columns of each desire's kind, claim, cost
    int32_t* out;
};

NR_DEV void astar_region(const AstarArgs& a, AS3 uint8_t** mark, AS3 int16_t** below, AS3 int16_t** depth,
                         AS3 uint8_t** flags, int wave) {
    extern __shared__ __align__(16) uint8_t nr_lds[];
    const int32_t cells = a.W * a.H;
    AS3 uint8_t* base = (AS3 uint8_t*)nr_lds + (int64_t)wave * a.region;
    *mark = base;
    *below = (AS3 int16_t*)(base + ((cells + 15) & ~15));
    *depth = *below + ((cells + 7) & ~7);
    *flags = (AS3 uint8_t*)(*depth + ((cells + 7) & ~7));
}

// pathfinding.search per lane: out[l] = found, step, distance, pops.
// Replaces the FFI target nanorts_astar_search (N/bots/cuda/pathfinding.cu:20-104).
__global__ __launch_bounds__(256) void k_astar_search(AstarArgs a) {
    const int lane = lane_id();
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int64_t l = (int64_t)blockIdx.x * a.waves + wave;
    if (l >= a.lanes) return;
    AS3 uint8_t *mark, *flags;
    AS3 int16_t *below, *depth;
    astar_region(a, &mark, &below, &depth, &flags, wave);
    const int32_t cells = a.W * a.H;
    const uint8_t* free = a.free + l * a.free_stride;
    for (int32_t c = lane; c < cells; c += kWave) mark[c] = free[c] ? 0 : 1;
    wave_sync();
    if (lane == 0) {
        const AstarPath path = astar_path(a.W, a.H, below, mark, depth, a.start[l * a.start_stride],
                                          a.target[l * a.target_stride], a.range[l * a.range_stride]);
        int32_t* o = a.out + l * 4;
        o[0] = path.found;
        o[1] = path.step;
        o[2] = path.distance;
        o[3] = path.pops;
    }
}

// A neighbour cell by the chain's offsets (UP -W, RIGHT +1, DOWN +W, any
// other direction -1), in wrapping arithmetic.
NR_DEV int32_t chain_neighbour(int32_t cell, int32_t direction, int32_t W) {
    const int32_t offset = direction == 0 ? -W : (direction == 1 ? 1 : (direction == 2 ? W : -1));
    return (int32_t)((uint32_t)cell + (uint32_t)offset);
}

// The first direction from `first` (turning by +1 mod 4) that `options`
// allows, or -1.
NR_DEV int32_t chain_drawn_direction(int32_t first, int32_t options) {
    for (int32_t turn = 0; turn < 4; ++turn) {
        const int32_t d = (int32_t)(((uint32_t)first + (uint32_t)turn) & 3u);
        if ((options >> d) & 1) return d;
    }
    return kAbsent;
}

// The walk of abstraction._walked (N/bots/abstraction.py:804-952) as the FFI
// target nanorts_astar_chain runs it (N/bots/cuda/abstraction.cu:98-215): the
// queued rows in order, each searched from its start toward its goal on the
// cells still open; a unit that can step and may move claims the step's
// cell, one that can step but may not takes its blocked desire, one that
// cannot takes its fallback (or, in a drawing pass, a drawn direction); a
// desire is kept when its claim is free and its cost stays within the
// balance beside the reserve and the costs already kept.  Per slot: rank
// among the kept (or -1), selector (0 fell back, 1 blocked, 2 moved),
// direction, drew; then one totals row: kept count, draws used.
__global__ __launch_bounds__(256) void k_astar_chain(AstarArgs a) {
    const int lane = lane_id();
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int64_t l = (int64_t)blockIdx.x * a.waves + wave;
    if (l >= a.lanes) return;
    AS3 uint8_t *mark, *flags;
    AS3 int16_t *below, *depth;
    astar_region(a, &mark, &below, &depth, &flags, wave);
    const int32_t W = a.W, cells = a.W * a.H;
    constexpr uint8_t kOpen = 1, kTaken = 2;
    const uint8_t* free = a.free + l * a.free_stride;
    const uint8_t* claimed = a.claimed + l * a.claimed_stride;
    for (int32_t c = lane; c < cells; c += kWave) flags[c] = (free[c] ? kOpen : 0) | (claimed[c] ? kTaken : 0);
    const int64_t cap = a.capacity;
    int32_t* decisions = a.out + l * (cap + 1) * 4;
    for (int64_t i = lane; i < cap * 4; i += kWave) {
        const int64_t f = i & 3;
        decisions[i] = (f == 0 || f == 2) ? kAbsent : 0;
    }
    const int32_t* entries = a.rows + l * a.rows_stride;
    const int32_t* order = a.queue + l * a.queue_stride;
    const int32_t* drawn = a.draws + l * a.draws_stride;
    const bool moves = a.moves[l * a.moves_stride] != 0;
    const uint32_t reserve = (uint32_t)a.reserved[l * a.reserved_stride];
    const int32_t held = a.balance[l * a.balance_stride];
    const int32_t asked = a.count[l * a.count_stride];
    const int64_t searched = asked < 0 ? 0 : (asked > cap ? cap : (int64_t)asked);
    uint32_t spent = 0u;
    int32_t granted = 0;
    int64_t calls = 0;
    for (int64_t row = 0; row < searched; ++row) {
        wave_sync();
        const int32_t slot = order[row];
        if (slot < 0 || slot >= cap) continue;
        for (int32_t c = lane; c < cells; c += kWave) mark[c] = (flags[c] & kOpen) ? 0 : 1;
        wave_sync();
        if (lane == 0) {
            const int32_t* entry = entries + (int64_t)slot * a.columns;
            const int32_t start = entry[0];
            const AstarPath path = astar_path(W, a.H, below, mark, depth, start, entry[1], entry[2]);
            const bool stepped = path.step != kAbsent;
            int32_t selector = 0, direction = kAbsent;
            bool eligible = entry[a.fallback[0]] != kAbsent;
            int32_t claim = entry[a.fallback[1]], cost = entry[a.fallback[2]];
            if (stepped && moves) {
                selector = 2;
                direction = path.step;
                eligible = true;
                claim = chain_neighbour(start, direction, W);
                cost = 0;
            } else if (stepped) {
                selector = 1;
                eligible = entry[a.blocked[0]] != kAbsent;
                claim = entry[a.blocked[1]];
                cost = entry[a.blocked[2]];
            }
            const bool drew = a.drawing && entry[3] != 0 && !(stepped && moves);
            if (drew) {
                const int64_t at = calls < a.draw_count ? calls : a.draw_count - 1;
                selector = 2;
                direction = chain_drawn_direction(drawn[at], entry[4]);
                eligible = true;
                claim = direction == kAbsent ? kAbsent : chain_neighbour(start, direction, W);
                cost = 0;
                ++calls;
            }
            const bool on_board = claim >= 0 && claim < cells;
            const bool conflicting = on_board && (flags[claim] & kTaken) != 0;
            const bool over = cost > 0 && (int32_t)(reserve + spent + (uint32_t)cost) > held;
            const bool kept = eligible && !conflicting && !over;
            if (on_board) flags[claim] = (uint8_t)((flags[claim] & ~kOpen) | (kept ? kTaken : 0));
            int32_t* d = decisions + (int64_t)slot * 4;
            d[0] = kept ? granted : kAbsent;
            d[1] = selector;
            d[2] = direction;
            d[3] = drew ? 1 : 0;
            if (kept) {
                spent += (uint32_t)cost;
                ++granted;
            }
        }
        granted = __builtin_amdgcn_readfirstlane(granted);
        spent = (uint32_t)__builtin_amdgcn_readfirstlane((int32_t)spent);
        calls = (int64_t)__builtin_amdgcn_readfirstlane((int32_t)calls);
    }
    wave_sync();
    if (lane < 4) decisions[cap * 4 + lane] = lane == 0 ? granted : (lane == 1 ? (int32_t)calls : 0);
}

// seat.step_seat (N/bots/seat.py:84-149): the bot's commands from the current
// state, the learner's rows decoded (N/adapters/jaxmarl/env.py:78-96),
// core.step under the episode root, auto-reset, the carry emptied where done,
// observations.  The learner is `fixed` for every lane, or seats[l] when
// `seats` is set; with `draw` a lane whose game ended takes the seat drawn
// from its next episode's root (N/bots/seat.py:119-123).
__global__ __launch_bounds__(256) void k_seat_step(KGame g, int64_t lanes, nanorts_state s, BotArgs a, int32_t fixed,
                                                   int32_t* seats, int32_t draw, const int32_t* actions,
                                                   int32_t partial, nanorts_env_results r) {
    NR_KERNEL_PROLOGUE
    const int32_t learner = seats ? clampi(uni(seats[l]), 0, 1) : fixed;
    load_env(g, s, l, e, LD_ALL, lane);
    count_units(g, e, lane);
    uint32_t k0 = (uint32_t)uni(e.sc[S_ROOT0]), k1 = (uint32_t)uni(e.sc[S_ROOT1]);
    fold_in(k0, k1, (uint32_t)uni(e.sc[S_EPISODE]));
    Bot b;
    b.base = e.base + a.y.origin;
    b.player = 1 - learner;
    b.block = g.N + b.player * g.C;
    const int32_t kept = bot_act(g, hdr, e, b, a.y, l, a.carry, a.strategy, a.trained, lane);
    const Layout& y = g.lay;
    const int32_t top = (1 << g.rank_bits) - 1;
    for (int32_t p = lane; p < 2 * g.C; p += kWave) {
        const int32_t slot = g.N + p;
        if (p / g.C == b.player) {
            int32_t v[6];
            unit_command(g, e, b, a.y, p - b.player * g.C, kept, v);
            at<int8_t>(e, y.c_kind)[p] = (int8_t)canon_kind(v[0]);
            at<int8_t>(e, y.c_dir)[p] = (int8_t)canon_dir(v[1]);
            at<int32_t>(e, y.c_none)[p] = v[2];
            at<int16_t>(e, y.c_target)[p] = (int16_t)canon_target(v[3], g.cells);
            at<int8_t>(e, y.c_ptype)[p] = (int8_t)canon_ptype(v[4], g.T);
            at<int16_t>(e, y.c_rank)[p] = (int16_t)clampi(v[5] == kAbsent ? 0 : v[5], 0, top);
        } else {
            const int32_t* row = actions + (l * g.C + (p - learner * g.C)) * 7;
            int32_t act[7];
#pragma unroll
            for (int f = 0; f < 7; ++f) act[f] = row[f];
            const bool available = e.birth[slot] != kAbsent && e.pkind[slot] == kAbsent;
            decode_row(g, e, p, available, act);
        }
    }
    // the carry is written before the step, whose phases reuse the region
    settle_carry(g, b, a.y, l, a.carry, lane);
    wave_sync();
    const bool events = r.reward_components != nullptr;
    core_step(g, hdr, e, lane, k0, k1, events);
    if (finish_step(g, hdr, e, l, lane, partial != 0, r, events)) {
        clear_carry(g, l, a.carry, lane);
        if (seats && draw) {
            uint32_t n0 = (uint32_t)uni(e.sc[S_ROOT0]), n1 = (uint32_t)uni(e.sc[S_ROOT1]);
            fold_in(n0, n1, (uint32_t)uni(e.sc[S_EPISODE]));
            const int32_t next = episode_seat(n0, n1);
            if (lane == 0) seats[l] = next;
        }
    }
    store_env(g, s, l, e, lane);
    if (r.feature_maps || r.scalars) observe_both(g, hdr, e, l, lane, partial != 0, r.feature_maps, r.scalars);
}

// The "drawn" rule's learner of each lane's current episode
// (N/bots/seat.py:77, 352-360): episode_seat(fold_in(root, episode)).
__global__ __launch_bounds__(256) void k_episode_seats(int64_t lanes, const uint32_t* roots, const uint32_t* episodes,
                                                       int32_t* seats) {
    const int64_t l = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (l >= lanes) return;
    uint32_t k0 = roots[2 * l], k1 = roots[2 * l + 1];
    fold_in(k0, k1, episodes[l]);
    seats[l] = episode_seat(k0, k1);
}

__global__ __launch_bounds__(256) void k_sample(KGame g, int64_t lanes, const uint32_t* words, uint32_t key0, uint32_t key1, int32_t step,
                         int64_t env0, int32_t* actions) {
    NR_KERNEL_PROLOGUE
    uint32_t k0 = key0, k1 = key1;
    fold_in(k0, k1, (uint32_t)step);
    const uint32_t env = (uint32_t)(env0 + l);
    const int32_t owned = 2 * g.C;
    // A position's action row (28 bytes) stored at a lane's stride would make
    // each of its seven store instructions touch a cache line per two or
    // three lanes: where the host gave the wave a block for the game's rows
    // (nanorts_amd_sample_actions) and they fill whole 16-byte vectors, the
    // rows go out through LDS as 16-byte vectors, consecutive across the
    // lanes.  (Staging the 12-byte words the same way as well cost more
    // occupancy than it saved.)
    const int32_t out16 = owned * 28 / 16;
    if ((owned & 3) == 0 && g.lay.env_bytes >= owned * 28 && (((uintptr_t)actions) & 15u) == 0) {
        AS3 int32_t* rows = (AS3 int32_t*)e.base;
        for (int32_t p = lane; p < owned; p += kWave) {
            Row r;
            const uint32_t* w = words + (l * owned + p) * 3;
            r.w[0] = w[0];
            r.w[1] = w[1];
            r.w[2] = w[2];
            int32_t a[7];
            sample_row(g, r, k0, k1, env, p, a);
#pragma unroll
            for (int f = 0; f < 7; ++f) rows[7 * p + f] = a[f];
        }
        wave_sync();
        u32x4* dst = (u32x4*)(actions + l * owned * 7);
        AS3 const u32x4* rv = (AS3 const u32x4*)rows;
        for (int32_t i = lane; i < out16; i += kWave) dst[i] = rv[i];
        return;
    }
    for (int32_t p = lane; p < owned; p += kWave) {
        Row r;
        const uint32_t* w = words + (l * owned + p) * 3;
        r.w[0] = w[0];
        r.w[1] = w[1];
        r.w[2] = w[2];
        int32_t a[7];
        sample_row(g, r, k0, k1, env, p, a);
        int32_t* out = actions + (l * owned + p) * 7;
#pragma unroll
        for (int f = 0; f < 7; ++f) out[f] = a[f];
    }
}

// The harness sampler on the GridNet surface: each cell's row of the packed
// action mask (bits 0-28, 29-60, 61-77 of the 78-bit row) drawn as k_sample
// draws a row, at position player * cells + cell.  A cell without a source
// (an all-zero row) comes out as zeros, which is what the draw gives it too.
__global__ __launch_bounds__(256) void k_gridnet_sample(KGame g, int64_t lanes, const uint32_t* mask, uint32_t key0,
                                                        uint32_t key1, int32_t step, int64_t env0, int32_t* actions) {
    NR_KERNEL_PROLOGUE
    (void)e;
    uint32_t k0 = key0, k1 = key1;
    fold_in(k0, k1, (uint32_t)step);
    const uint32_t env = (uint32_t)(env0 + l);
    const int32_t rows = 2 * g.cells;
    // as k_sample, the rows go out through LDS as 16-byte vectors, here a
    // wave's 64 rows (1 792 bytes) at a time, where the host gave the wave a
    // block for them (nanorts_amd_gridnet_sample_actions) and the rows fill
    // whole vectors
    if ((rows & 3) == 0 && g.lay.env_bytes >= kWave * 28 && (((uintptr_t)actions) & 15u) == 0) {
        AS3 int32_t* stage = (AS3 int32_t*)e.base;
        AS3 const u32x4* sv = (AS3 const u32x4*)e.base;
        for (int32_t p0 = 0; p0 < rows; p0 += kWave) {
            const int32_t p = p0 + lane;
            int32_t a[7] = {0, 0, 0, 0, 0, 0, 0};
            if (p < rows) {
                const uint32_t* w = mask + (l * rows + p) * 3;
                const uint32_t q0 = w[0], q1 = w[1], q2 = w[2];
                if ((q0 | q1 | q2) != 0u) {
                    Row r;
                    r.w[0] = q0 | (q1 << 29);
                    r.w[1] = (q1 >> 3) | (q2 << 29);
                    r.w[2] = q2 >> 3;
                    sample_row(g, r, k0, k1, env, p, a);
                }
            }
#pragma unroll
            for (int f = 0; f < 7; ++f) stage[7 * lane + f] = a[f];
            wave_sync();
            // rows p0 .. p0 + n - 1, n a multiple of 4
            const int32_t n = rows - p0 < kWave ? rows - p0 : kWave;
            u32x4* dst = (u32x4*)(actions + (l * rows + p0) * 7);
            for (int32_t i = lane; i < n * 7 / 4; i += kWave) dst[i] = sv[i];
            wave_sync();
        }
        return;
    }
    for (int32_t p = lane; p < rows; p += kWave) {
        const uint32_t* w = mask + (l * rows + p) * 3;
        const uint32_t p0 = w[0], p1 = w[1], p2 = w[2];
        int32_t a[7] = {0, 0, 0, 0, 0, 0, 0};
        if ((p0 | p1 | p2) != 0u) {
            Row r;
            r.w[0] = p0 | (p1 << 29);
            r.w[1] = (p1 >> 3) | (p2 << 29);
            r.w[2] = p2 >> 3;
            sample_row(g, r, k0, k1, env, p, a);
        }
        int32_t* out = actions + (l * rows + p) * 7;
#pragma unroll
        for (int f = 0; f < 7; ++f) out[f] = a[f];
    }
}

// Fused rollout: the state stays staged in LDS across `steps` cycles.  With
// the per-cycle summary (rollout.h) each cycle is: sample from the masks of
// the summarised state -> decode -> core.step -> finish (reward, done,
// auto-reset) -> summarise the new state, which writes its observation.
//
// The kernel takes one argument struct and every phase of the cycle reads
// it again from the kernel-argument segment (fresh_rollout_args), together
// with the LDS views derived from it, so that almost nothing but the loop
// counters and keys stays live in scalar registers across the cycle.
constexpr int32_t kRolloutChunk = 128;  // cycles per launch (one step key each)
struct RolloutArgs {
    KGame g;  // first: fresh_game() reads it at offset 0
    int64_t lanes;
    nanorts_state s;
    int32_t t0, steps, partial;  // cycles t0 .. t0 + steps - 1 of the caller's rollout
    int32_t resume;              // second pass: each game starts at its out.progress cycle
    int64_t env0;
    nanorts_rollout_results out;
    uint32_t step_keys[2 * kRolloutChunk];  // fold_in(sample_key, step0 + t0 + t), host-computed
};
typedef const __attribute__((address_space(4))) RolloutArgs* RolloutArgsArg;
NR_DEV const RolloutArgs& fresh_rollout_args() {
    RolloutArgsArg p = (RolloutArgsArg)__builtin_amdgcn_kernarg_segment_ptr();
    asm volatile("" : "+s"(p));
    return *(const RolloutArgs*)p;
}
NR_DEV Hdr header_view(const KGame& g) {
    extern __shared__ __align__(16) uint8_t nr_lds[];
    AS3 uint8_t* lds = (AS3 uint8_t*)nr_lds;
    Hdr h;
    h.tab = (AS3 int32_t*)lds;
    h.terrain = lds + g.lay.o_terrain;
    h.seg = (AS3 Seg*)(lds + g.lay.o_seg);
    h.disk = (AS3 uint32_t*)(lds + g.lay.o_disk);
    h.walls = (AS3 uint32_t*)(lds + g.lay.o_walls);
    return h;
}
// The env block of the workgroup's `team`-th game (its wave for whole-wave
// teams, 2 * wave + half for half-wave teams).
NR_DEV Env team_env(const KGame& g, int team) {
    extern __shared__ __align__(16) uint8_t nr_lds[];
    return env_view(g, (AS3 uint8_t*)nr_lds + g.lay.hdr_bytes + team * g.lay.env_bytes);
}
#define NR_ROLLOUT_PHASE                              \
    const RolloutArgs& a = fresh_rollout_args();      \
    const KGame& g = a.g;                             \
    const Hdr hdr = header_view(g);                   \
    const Env e = team_env(g, team);                  \
    (void)hdr;
// The kernel prologue for teams of TW lanes: the header staged, this team's
// game l and env block.
#define NR_TEAM_PROLOGUE(TW)                                                            \
    extern __shared__ __align__(16) uint8_t nr_lds[];                                   \
    AS3 uint8_t* lds = (AS3 uint8_t*)nr_lds;                                            \
    const Hdr hdr = header_view(g);                                                     \
    load_header(g, hdr);                                                                \
    __syncthreads();                                                                    \
    const int lane = team_lane<TW>();                                                   \
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));           \
    const int team = (kWave / TW) * wave + team_half<TW>();                             \
    int64_t l = (int64_t)blockIdx.x * ((blockDim.x >> 6) * (kWave / TW)) + team;        \
    if (l >= lanes) return;                                                             \
    const Env e = env_view(g, lds + g.lay.hdr_bytes + team * g.lay.env_bytes);

// The cycles of one launch.  `Lean` is the first pass of the two-pass
// launch (k_rollout_lean, on shape_for_lean's block): before each cycle it
// checks that the cycle stays on the one-wave path (a regular state with at
// most 64 available units and at most 64 live slots); at the first cycle
// that does not, the game's state goes back to memory and out.progress
// records that cycle, from which the second pass (k_rollout with `resume`,
// on the full block) runs the rest.  Splitting a game's cycles between
// launches this way gives the same result as one launch, as the state is
// all a cycle carries.
template <bool Lean, int TW = kWave>
NR_DEV void rollout_cycles(const RolloutArgs& args) {
    static_assert(TW == kWave || Lean, "half-wave teams run the first pass only");
    const KGame& g = args.g;
    const int64_t lanes = args.lanes;
    int32_t t_begin = 0;
    if (!Lean && args.resume) {
        // a workgroup whose games the first pass finished stages nothing.
        // The waves vote through the first words of the dynamic LDS (the
        // header goes there after the second barrier): a static LDS
        // variable (as __syncthreads_or keeps) would grow every
        // workgroup's allocation past what four workgroups per CU allow.
        extern __shared__ __align__(16) uint8_t nr_lds[];
        AS3 uint32_t* votes = (AS3 uint32_t*)nr_lds;
        const int waves = (int)(blockDim.x >> 6);
        const int64_t l0 = (int64_t)blockIdx.x * waves + (threadIdx.x >> 6);
        const bool busy = l0 < lanes && args.out.progress[l0] < args.steps;
        if ((threadIdx.x & (kWave - 1)) == 0) votes[threadIdx.x >> 6] = busy ? 1u : 0u;
        __syncthreads();
        uint32_t any = 0u;
        for (int w = 0; w < waves; ++w) any |= votes[w];
        __syncthreads();
        if (any == 0u) return;
    }
    NR_TEAM_PROLOGUE(TW)
    (void)lds;
    if (!Lean && args.resume) {
        t_begin = uni(args.out.progress[l]);
        if (t_begin >= args.steps) return;
    }
    // with a slot window, a game that does not fit it (or whose initial
    // state, which an auto-reset copies in, does not) runs no cycle here
    bool fits = true;
    if (Lean && g.shift > 0) {
        fits = load_window_rows<TW>(g, args.s, l, e, lane) && initial_fits_window<TW>(g, lane);
        load_scalars(args.s, l, e, lane);
        wave_sync();
    } else {
        load_env<TW>(g, args.s, l, e, LD_ALL, lane);
    }
    if (fits) count_units<TW>(g, e, lane);
    // the first pass runs only where this holds (the host checks it)
    const bool fast = Lean || (g.fast_obs && ((((uintptr_t)args.out.feature_maps) & 7u) == 0));
    // the summary's counts stay in registers from one cycle into the next
    SlotSummary sm = {0, 0, 0, 0, false};
    if (fast && fits) sm = summarize<TW>(g, hdr, e, lane, args.partial != 0, nullptr, nullptr, nullptr, nullptr);
    if (!fits) sm.full = true;
    uint32_t ek0 = (uint32_t)tuni<TW>(e.sc[S_ROOT0]), ek1 = (uint32_t)tuni<TW>(e.sc[S_ROOT1]);
    fold_in(ek0, ek1, (uint32_t)tuni<TW>(e.sc[S_EPISODE]));
    const int32_t steps = args.steps;
    int32_t general = 0;  // cycles admitted request by request
    int32_t stop = steps;  // first pass: the first cycle left to the second
    // the output rows of the launch's first cycle and the observation ring,
    // read once into registers instead of from the argument segment every
    // cycle
    const int64_t t0l = (int64_t)args.t0 * lanes;
    float* const rew = args.out.rewards ? args.out.rewards + t0l * 2 : nullptr;
    uint8_t* const dn = args.out.dones ? args.out.dones + t0l : nullptr;
    uint8_t* const maps = args.out.feature_maps;
    int32_t* const scal = args.out.scalars;
    const uint32_t depth = (uint32_t)(args.out.depth > 0 ? args.out.depth : 1), first = (uint32_t)args.t0;
    for (int32_t t = t_begin; t < steps; ++t) {
        bool irregular = false;
        int32_t n;
        // fused: the sampled commands go straight into the admission's
        // request registers (no staging through the command arrays)
        bool fused = false, listed = false;
        Reqs q;
        no_request(q);
        // this lane's pending entries (two a lane for a half-wave team)
        int32_t nA = 0, posA[2] = {0, 0}, costA[2] = {0, 0}, playerA[2] = {0, 0};
        {
            // masks -> sample -> decode (get_avail_actions + harness + decode_actions)
            NR_ROLLOUT_PHASE
            // (a half-wave team holds up to two live slots per lane)
            if (Lean && (sm.irregular || sm.full || sm.nav > TW || sm.nlive > (TW == kWave ? kWave : 2 * TW))) {
                stop = t;
                break;
            }
            const nanorts_rollout_results& out = a.out;
            // the state's owned positions (a slot window's block holds fewer)
            const int32_t owned = 2 * (g.C + g.shift);
            const int64_t tt = (int64_t)a.t0 + t;  // cycle index within the caller's rollout
            if (fast) {
                n = sm.nav;
                irregular = sm.irregular;
                fused = Lean || (!irregular && n <= kWave);
            } else {
                n = compact_available(g, e, lane, &irregular);
                build_bitmaps(g, hdr, e, lane);
            }
            // the pending entries of the admission, loaded early so their
            // latency overlaps the sampling
            if (fused) listed = admit_entries<TW>(g, hdr, e, lane, true, &nA, posA, costA, playerA, sm.nA);
            const uint32_t ke0 = a.step_keys[2 * t], ke1 = a.step_keys[2 * t + 1];
            const uint32_t env = (uint32_t)(a.env0 + l);
            AS3 const int16_t* av = at<int16_t>(e, g.lay.a_av);
            // draw words: with n <= 32 the two threefry blocks of a position run
            // on two lanes at once; otherwise each lane computes both
            const bool paired = n <= TW / 2;
            const bool narrow = fast && g.seen_words == 1;
            // (no unit to sample: no balance read)
            const Affordable aff = n > 0 ? affordable_types<TW>(g, hdr, e, lane) : Affordable{{0u, 0u}};
            uint32_t pw0 = 0u, pw1 = 0u, pw2 = 0u, pw3 = 0u;
            if (paired && n > 0) {
                const int32_t u = lane >> 1;
                uint32_t dx0 = env, dx1 = 2u * (u < n ? (uint32_t)glob_pos(g, av[u]) : 0u) + (uint32_t)(lane & 1);
                threefry(ke0, ke1, dx0, dx1);
                // every lane active: lane u takes lanes 2u and 2u + 1
                pw0 = (uint32_t)__shfl((int)dx0, 2 * lane, TW);
                pw1 = (uint32_t)__shfl((int)dx1, 2 * lane, TW);
                pw2 = (uint32_t)__shfl((int)dx0, 2 * lane + 1, TW);
                pw3 = (uint32_t)__shfl((int)dx1, 2 * lane + 1, TW);
            }
            for (int32_t i = lane; i < n; i += TW) {
                const int32_t p = av[i];
                uint32_t words[4];
                if (paired) {
                    words[0] = pw0;
                    words[1] = pw1;
                    words[2] = pw2;
                    words[3] = pw3;
                } else {
                    const uint32_t pg = (uint32_t)glob_pos(g, p);
                    uint32_t w0 = env, w1 = 2u * pg, w2 = env, w3 = 2u * pg + 1u;
                    threefry(ke0, ke1, w0, w1);
                    threefry(ke0, ke1, w2, w3);
                    words[0] = w0;
                    words[1] = w1;
                    words[2] = w2;
                    words[3] = w3;
                }
                int32_t kind, dir, ptype, target, none;
                // unrecorded, units of attack range at most 1: the factors
                // straight from the neighbour masks, no row assembled
                if (!(narrow && !out.actions && g.T <= 8 &&
                      sample_unit_w1(g, hdr, e, p, aff, words[0], words[1], words[2], words[3], &kind, &dir, &ptype,
                                     &target, &none))) {
                    const Row r =
                        narrow ? legality_row_w1(g, hdr, e, g.N + p, aff) : legality_row_bm(g, hdr, e, g.N + p);
                    if (!out.actions && g.T <= 8) {
                        // unrecorded: only the factors decode reads are drawn
                        sample_decode8(g, e, p, r, words[0], words[1], words[2], words[3], &kind, &dir, &ptype,
                                       &target, &none);
                    } else {
                        int32_t act[7];
                        if (g.T <= 8) sample_row_words8(g, r, words, act);
                        else sample_row_words(g, r, words, act);
                        if (out.actions) {
                            int32_t* dst = out.actions + ((tt * lanes + l) * owned + glob_pos(g, p)) * 7;
#pragma unroll
                            for (int f = 0; f < 7; ++f) dst[f] = act[f];
                        }
                        decode_values(g, e, p, act, &kind, &dir, &ptype, &target, &none);
                    }
                }
                if (fused) {
                    request_of(g, hdr, e, p, kind, dir, ptype, target, none, true, false, q);
                } else {
                    const Layout& y = g.lay;
                    at<int8_t>(e, y.c_kind)[p] = (int8_t)kind;
                    at<int8_t>(e, y.c_dir)[p] = (int8_t)dir;
                    at<int8_t>(e, y.c_ptype)[p] = (int8_t)ptype;
                    at<int16_t>(e, y.c_target)[p] = (int16_t)target;
                    at<int32_t>(e, y.c_none)[p] = none;
                    at<int16_t>(e, y.c_rank)[p] = 0;
                }
            }
            if (out.actions) {
                // unavailable rows sample all zeros (a slot window's gaps
                // hold no unit)
                for (int32_t p = lane; p < owned; p += TW) {
                    // each player's last `shift` positions lie past its window
                    const bool gap = (p >= g.C && p < g.C + g.shift) || p >= 2 * g.C + g.shift;
                    const int32_t sl = g.N + (p < g.C ? p : p - g.shift);
                    if (!gap && e.birth[sl] != kAbsent && e.pkind[sl] == kAbsent) continue;
                    int32_t* dst = out.actions + ((tt * lanes + l) * owned + p) * 7;
#pragma unroll
                    for (int f = 0; f < 7; ++f) dst[f] = 0;
                }
            }
            wave_sync();
            // env.step: core.step keyed by fold_in(env root, episode)
            if (Lean || (fused && listed)) {
                // the first pass stopped before any cycle that is not both
                admit_resolve<TW>(g, hdr, e, lane, ek0, ek1, n, nA, posA, costA, playerA, q);
            } else if (fused || !admit_env(g, hdr, e, lane, ek0, ek1, false, n, irregular, true, fast)) {
                // general admission; a fused cycle (which the summary's
                // irregular flag keeps off this path) stages its requests first
                if (fused) stage_requests(g, e, lane, n, q);
                if (fast) mark_unavailable(g, e, lane);
                ++general;
                int32_t n_rank = 0;
                const int32_t issued = order_requests(g, e, lane, &n_rank);
                AS3 int16_t* order = at<int16_t>(e, g.lay.b_order);
                for (int32_t i = 0; i < issued; ++i) admit_one(g, hdr, e, lane, uni(order[i]), n_rank, ek0, ek1, false);
            }
        }
        {
            NR_ROLLOUT_PHASE
            // the summary's live lanes: sampling and admission spawn and
            // remove nothing
            const LiveLanes known = summary_live(sm);
            const int32_t held = TW == kWave ? kWave : 2 * TW;  // live slots the lanes hold
            int32_t time = complete<TW>(g, hdr, e, lane, Lean, (fast && sm.nlive <= held) ? known : LiveLanes{-1, 0, 0});
            Outcome oc = decide_counted<TW>(e, lane);
            nanorts_env_results r = {};
            if (rew) r.reward = rew + (int64_t)t * lanes * 2;
            if (dn) r.done = dn + (int64_t)t * lanes;
            const bool done = finish_step<TW, Lean>(g, hdr, e, l, lane, a.partial != 0, r, false, false, true, &oc, time);
            if (done) {
                ek0 = (uint32_t)tuni<TW>(e.sc[S_ROOT0]);
                ek1 = (uint32_t)tuni<TW>(e.sc[S_ROOT1]);
                fold_in(ek0, ek1, (uint32_t)tuni<TW>(e.sc[S_EPISODE]));
                // the published observation is the reset state's
                time = tuni<TW>(e.sc[S_TIME]);
                oc.res0 = tuni<TW>(e.sc[S_RES0]);
                oc.res1 = tuni<TW>(e.sc[S_RES1]);
                oc.alt = tuni<TW>(e.sc[S_ALT]);
            }
            const nanorts_rollout_results& out = a.out;
            const int64_t per = (int64_t)g.cells * 6;
            // ring slot (t0 + t) % depth in 32 bits (a mask for powers of two)
            const uint32_t d = depth, c = first + (uint32_t)t;
            const uint32_t ring = (d & (d - 1u)) == 0u ? (c & (d - 1u)) : c % d;
            const int64_t slot = (int64_t)ring * lanes + l;
            if (fast) {
                uint8_t* m0 = maps ? maps + (slot * 2) * per : nullptr;
                if (scal && lane < 8) {
                    // the scalars from registers: own balance, the opponent's,
                    // time, alternating count (as summarize writes them)
                    const int32_t pl = lane >> 2, f = lane & 3;
                    const int32_t own = pl == 0 ? oc.res0 : oc.res1, opp = pl == 0 ? oc.res1 : oc.res0;
                    scal[slot * 8 + lane] = f == 0 ? own : (f == 1 ? opp : (f == 2 ? time : oc.alt));
                }
                // the sight bitmaps persist in the event counters' words, which
                // the rollout does not count, when both planes fit there
                const int32_t kept = 2 * g.H * g.seen_words <= 32 ? g.lay.b_events : -1;
                sm = summarize<TW>(g, hdr, e, lane, a.partial != 0, m0, m0 ? m0 + per : nullptr, nullptr, nullptr, kept);
            } else if (out.feature_maps || out.scalars) {
                observe_both(g, hdr, e, slot, lane, a.partial != 0, out.feature_maps, out.scalars);
            }
        }
    }
    {
        NR_ROLLOUT_PHASE
        if (!Lean || stop > 0) {
            if (Lean && g.shift > 0) store_window_rows<TW>(g, a.s, l, e, lane);
            else store_env<TW>(g, a.s, l, e, lane);
        }
        if (lane == 0) {
            if (Lean) a.out.progress[l] = stop;
            else if (!a.resume && a.out.progress) a.out.progress[l] = 0;  // one pass on the full block
            // the second pass counts the cycles of a game the first stopped
            if (a.out.general_admissions && (!Lean || stop == steps)) a.out.general_admissions[l] = general;
        }
    }
}

__global__ __launch_bounds__(256, 4) void k_rollout(RolloutArgs args) { rollout_cycles<false>(args); }

// The first pass: the one-wave path alone, on a smaller LDS block per game.
// Without the request-by-request admission and completion's member records
// its code is smaller and keeps fewer scalar registers (90 VGPRs, 60 SGPRs
// spilled to VGPR lanes against k_rollout's 112 and 117), which makes a
// cycle about 2.5 % faster at the same 16 games per CU.
__global__ __launch_bounds__(kWave * kLeanMaxGames) void k_rollout_lean(RolloutArgs args) {
    rollout_cycles<true>(args);
}

// The first pass with two games per wave: each half of a wave (32 lanes)
// runs one game's cycles, so the phases whose work is narrower than a wave
// (sampling, admission, completion, the slot pass) serve two games per
// instruction.  A game leaves for the second pass at the first cycle with
// more than 32 available units or live slots.
__global__ __launch_bounds__(kWave * kPairMaxWaves, 4) void k_rollout_pair(RolloutArgs args) {
    rollout_cycles<true, 32>(args);
}

// Fused learner-vs-bot rollout: per cycle the learner's rows sampled from
// its masks (the integer uniform-over-legal sampler, as nanorts_amd_sample_actions
// on get_avail_actions words), the bot's act, the seat step and the
// observations, with the state resident in LDS across the launch.
struct SeatRolloutArgs {
    KGame g;  // first: fresh_game() reads it at offset 0
    int64_t lanes;
    nanorts_state s;
    BotArgs bot;
    int32_t learner, t0, steps, partial;  // cycles t0 .. t0 + steps - 1 of the caller's rollout
    int64_t env0;
    int32_t* seats;        // per-lane learners (or NULL: `learner` for every lane)
    int32_t* seat_record;  // [steps][lanes] learner of each cycle, or NULL
    int32_t draw;          // re-draw a lane's seat from its next episode root
    int32_t resume;        // second pass: each game starts at its out.progress cycle
    nanorts_rollout_results out;
    uint32_t step_keys[2 * kRolloutChunk];  // fold_in(sample_key, step0 + t0 + t), host-computed
};

// The carry rows of env l into the bot region through the slot window: the
// window's C units' rows (row stride C + shift), their target and base
// slots mapped to block slots.  False when the carry does not fit: a target
// or base outside [-1, E + 2 shift) or in a gap, or a row past the window
// that is not empty (kind, the int32 rows and unit_type -1, trained 0),
// which the full block would settle.
template <int TW>
NR_DEV bool load_carry_window(const KGame& g, Bot& b, const BotLayout& y, int64_t l, const BotCarry& carry, int lane) {
    const int32_t C = g.C, sh = g.shift, N = g.N, E = g.E;
    const int64_t row = l * (int64_t)(C + sh);
    bool bad = false;
    for (int32_t i = lane; i < C + sh; i += TW) {
        const int64_t at = row + i;
        int32_t v[9];
#pragma unroll
        for (int f = 0; f < 9; ++f) v[f] = carry.row[f][at];
        const uint8_t trained = carry.trained[at] ? 1 : 0;
        if (i >= C) {
            // past the window: must already be the empty row
            bool empty = trained == 0;
#pragma unroll
            for (int f = 0; f < 9; ++f) empty = empty && v[f] == kAbsent;
            if (!empty) bad = true;
            continue;
        }
#pragma unroll
        for (int f = 3; f <= 5; f += 2) {  // target (row 3) and base (row 5) are slots
            const int32_t s = v[f];
            if (s >= N + C + sh && s < E + sh) v[f] = s - sh;
            else if (s < -1 || s >= N + C) bad = true;
        }
        // the cell (row 7) is held as int16 (with the slots)
        if (v[7] < -32768 || v[7] > 32767) bad = true;
        bv<int8_t>(b, y.k_kind)[i] = (int8_t)v[0];
#pragma unroll
        for (int f = 1; f < 8; ++f) carry_put<TW>(b, y, f, i, v[f]);
        bv<int8_t>(b, y.k_utype)[i] = (int8_t)v[8];
        bv<uint8_t>(b, y.k_trained)[i] = trained;
    }
    int32_t next_order = 0;
    if (lane == 0) next_order = __builtin_nontemporal_load(carry.next_order + l);
    b.next_order = tread<TW>(next_order, 0);
    return tballot<TW>(bad) == 0ull;
}

// The window's carry rows back into env l's carry (target and base slots
// mapped back); the rows past the window stay as they are (empty).
template <int TW>
NR_DEV void store_carry_window(const KGame& g, const Bot& b, const BotLayout& y, int64_t l, const BotCarry& carry,
                               int lane) {
    const int64_t row = l * (int64_t)(g.C + g.shift);
    for (int32_t i = lane; i < g.C; i += TW) {
        const int64_t at = row + i;
        carry.row[0][at] = bv<int8_t>(b, y.k_kind)[i];
#pragma unroll
        for (int f = 1; f < 8; ++f) {
            const int32_t v = carry_at<TW>(b, y, f, i);
            carry.row[f][at] = (f == 3 || f == 5) && v >= 0 ? glob_slot(g, v) : v;
        }
        carry.row[8][at] = bv<int8_t>(b, y.k_utype)[i];
        carry.trained[at] = bv<uint8_t>(b, y.k_trained)[i];
    }
    if (lane == 0) carry.next_order[l] = b.next_order;
}

// The argument struct read in place from the kernel-argument segment (the
// step keys are indexed by the cycle, which would otherwise copy the whole
// struct into scratch memory).  The seat kernels take the struct as their
// one argument.
typedef const __attribute__((address_space(4))) SeatRolloutArgs* SeatRolloutArgsArg;
NR_DEV const SeatRolloutArgs& seat_args() {
    SeatRolloutArgsArg p = (SeatRolloutArgsArg)__builtin_amdgcn_kernarg_segment_ptr();
    return *(const SeatRolloutArgs*)p;
}
// The same through an opaque copy of the segment pointer: the fields used
// after this call are loaded again (scalar loads) rather than held in scalar
// registers from the start of the kernel.
NR_DEV const SeatRolloutArgs& seat_args_again() {
    SeatRolloutArgsArg p = (SeatRolloutArgsArg)__builtin_amdgcn_kernarg_segment_ptr();
    asm volatile("" : "+s"(p));
    return *(const SeatRolloutArgs*)p;
}

// The step key of the block's episode, fold_in(env root, episode), read
// from its scalars (which change only when the game resets).
template <int TW = kWave>
NR_DEV void episode_key(const Env& e, uint32_t& k0, uint32_t& k1) {
    k0 = (uint32_t)tuni<TW>(e.sc[S_ROOT0]);
    k1 = (uint32_t)tuni<TW>(e.sc[S_ROOT1]);
    fold_in(k0, k1, (uint32_t)tuni<TW>(e.sc[S_EPISODE]));
}

// The cycles of one seat launch.  `First` is the first pass of a two-pass
// launch (k_seat_rollout_pair): two games per wave (TW = 32) on the slot
// window (KGame::shift), each game running until a cycle would leave the
// one-team path (an irregular state, more than 32 available units, more than
// 64 live slots, a full slot window) or its state or carry does not fit the
// window; out.progress then records that cycle, and the second pass
// (k_seat_rollout with `resume`, one game per wave on the full block) runs
// the rest.  The state and the carry are all a cycle carries, so the split
// gives the one-pass result.
template <bool First, int TW = kWave>
NR_DEV void seat_cycles(const SeatRolloutArgs& args) {
    static_assert(TW == kWave || First, "half-wave teams run the first pass only");
    const KGame& g = args.g;
    const int64_t lanes = args.lanes;
    int32_t t_begin = 0;
    if (!First && args.resume) {
        // a workgroup whose games the first pass finished stages nothing
        extern __shared__ __align__(16) uint8_t nr_lds[];
        AS3 uint32_t* votes = (AS3 uint32_t*)nr_lds;
        const int waves = (int)(blockDim.x >> 6);
        const int64_t l0 = (int64_t)blockIdx.x * waves + (threadIdx.x >> 6);
        const bool busy = l0 < lanes && args.out.progress[l0] < args.steps;
        if ((threadIdx.x & (kWave - 1)) == 0) votes[threadIdx.x >> 6] = busy ? 1u : 0u;
        __syncthreads();
        uint32_t any = 0u;
        for (int w = 0; w < waves; ++w) any |= votes[w];
        __syncthreads();
        if (any == 0u) return;
    }
    NR_TEAM_PROLOGUE(TW)
    (void)lds;
    if (!First && args.resume) {
        t_begin = uni(args.out.progress[l]);
        if (t_begin >= args.steps) return;
    }
    const BotArgs& ba = args.bot;
    bool fits = true;
    if (First && g.shift > 0) {
        fits = load_window_rows<TW>(g, args.s, l, e, lane) && initial_fits_window<TW>(g, lane);
        load_scalars(args.s, l, e, lane);
        wave_sync();
    } else {
        load_env<TW>(g, args.s, l, e, LD_ALL, lane);
    }
    int32_t learner = args.seats ? clampi(tuni<TW>(args.seats[l]), 0, 1) : args.learner;
    Bot b;
    b.base = e.base + ba.y.origin;
    b.player = 1 - learner;
    b.block = g.N + b.player * g.C;
    // the carry: loaded here for the first pass (through the window, the
    // identity without one), by the bot's first act otherwise
    if (First) fits = load_carry_window<TW>(g, b, ba.y, l, ba.carry, lane) && fits;
    if (fits) count_units<TW>(g, e, lane);
    const nanorts_rollout_results& out = args.out;
    const Layout& y = g.lay;
    const uint32_t env = (uint32_t)(args.env0 + l);
    // the state's per-player positions (a slot window's block holds fewer)
    const int32_t Cg = g.C + g.shift;
    // boards of at most 32 columns: the per-cycle summary (occupancy bitmaps,
    // available list, kept sight bitmaps, packed observation stores), as in
    // the fused rollout (the first pass runs only where this holds)
    const bool fast = First || (g.fast_obs && g.seen_words == 1 && ((((uintptr_t)out.feature_maps) & 7u) == 0));
    // the summary's counts stay in registers from one cycle into the next
    SlotSummary sm = {0, 0, 0, 0, false};
    if (fast && fits) sm = summarize<TW>(g, hdr, e, lane, args.partial != 0, nullptr, nullptr, nullptr, nullptr);
    if (!fits) sm.full = true;
    int32_t stop = args.steps;  // first pass: the first cycle left to the second
    // Each part of a cycle rebuilds the block's row pointers from the block
    // base (refresh) and the game's addresses from an opaque copy of its
    // index, and the episode key and the bot's rows are derived again where
    // they are used, so that they are not held in registers across the
    // cycle: a half-wave team holds each of them in a vector register.
    const Env& e_in = e;
    for (int32_t t = t_begin; t < args.steps; ++t) {
        if (First && (sm.irregular || sm.full || sm.nav > TW || sm.nlive > (TW == kWave ? kWave : 2 * TW))) {
            stop = t;
            break;
        }
        if constexpr (TW != kWave) asm volatile("" : "+v"(l));
        // the game's fields loaded again in each cycle (scalar loads) rather
        // than held in scalar registers across the loop
        const KGame& g = fresh_game();
        const Layout& y = g.lay;
        b.player = 1 - learner;
        b.block = g.N + b.player * g.C;
        const int64_t tt = (int64_t)args.t0 + t;
        if (args.seat_record && lane == 0) args.seat_record[tt * lanes + l] = learner;
        // the learner: masks -> sample -> decode (unavailable rows absent)
        const uint32_t ke0 = args.step_keys[2 * t], ke1 = args.step_keys[2 * t + 1];
        if (fast) {
            const Env e = refresh<TW>(g, e_in);
            const AS3 int16_t* av = at<int16_t>(e, y.a_av);
            const int32_t n = sm.nav;
            mark_unavailable<TW>(g, e, lane);
            // (no unit to sample: no balance read; only the learner's units
            // are sampled, so both entries hold its types)
            const Affordable both = n > 0 ? affordable_types<TW>(g, hdr, e, lane) : Affordable{{0u, 0u}};
            const uint32_t mine = learner ? both.player[1] : both.player[0];
            const Affordable aff = {{mine, mine}};
            // both threefry blocks of a position on two lanes when n <= TW / 2
            const bool paired = n <= TW / 2;
            uint32_t pw0 = 0u, pw1 = 0u, pw2 = 0u, pw3 = 0u;
            if (paired && n > 0) {
                const int32_t u = lane >> 1;
                uint32_t dx0 = env, dx1 = 2u * (u < n ? (uint32_t)glob_pos(g, av[u]) : 0u) + (uint32_t)(lane & 1);
                threefry(ke0, ke1, dx0, dx1);
                pw0 = (uint32_t)__shfl((int)dx0, 2 * lane, TW);
                pw1 = (uint32_t)__shfl((int)dx1, 2 * lane, TW);
                pw2 = (uint32_t)__shfl((int)dx0, 2 * lane + 1, TW);
                pw3 = (uint32_t)__shfl((int)dx1, 2 * lane + 1, TW);
            }
            for (int32_t i = lane; i < n; i += TW) {
                const int32_t p = av[i];
                if ((p >= g.C ? 1 : 0) != learner) continue;  // positions below 2C
                uint32_t words[4] = {pw0, pw1, pw2, pw3};
                if (!paired) {
                    const uint32_t pg = (uint32_t)glob_pos(g, p);
                    words[0] = env;
                    words[1] = 2u * pg;
                    words[2] = env;
                    words[3] = 2u * pg + 1u;
                    threefry(ke0, ke1, words[0], words[1]);
                    threefry(ke0, ke1, words[2], words[3]);
                }
                int32_t kind, dir, ptype, target, none;
                // unrecorded, units of attack range at most 1: the factors
                // straight from the neighbour masks, no row assembled
                if (!(!out.actions && g.T <= 8 &&
                      sample_unit_w1(g, hdr, e, p, aff, words[0], words[1], words[2], words[3], &kind, &dir, &ptype,
                                     &target, &none))) {
                    const Row r = legality_row_w1(g, hdr, e, g.N + p, aff);
                    if (!out.actions && g.T <= 8) {
                        sample_decode8(g, e, p, r, words[0], words[1], words[2], words[3], &kind, &dir, &ptype,
                                       &target, &none);
                    } else {
                        int32_t act[7];
                        if (g.T <= 8) sample_row_words8(g, r, words, act);
                        else sample_row_words(g, r, words, act);
                        if (out.actions) {
                            int32_t* dst = out.actions + ((tt * lanes + l) * Cg + (p - learner * g.C)) * 7;
#pragma unroll
                            for (int f = 0; f < 7; ++f) dst[f] = act[f];
                        }
                        decode_values(g, e, p, act, &kind, &dir, &ptype, &target, &none);
                    }
                }
                at<int8_t>(e, y.c_kind)[p] = (int8_t)kind;
                at<int8_t>(e, y.c_dir)[p] = (int8_t)dir;
                at<int8_t>(e, y.c_ptype)[p] = (int8_t)ptype;
                at<int16_t>(e, y.c_target)[p] = (int16_t)target;
                at<int32_t>(e, y.c_none)[p] = none;
            }
        }
        if constexpr (!First) {
            const AS3 int16_t* av = at<int16_t>(e, y.a_av);
            bool irregular = false;
            const int32_t n = fast ? 0 : compact_available(g, e, lane, &irregular);
            if (!fast) build_bitmaps(g, hdr, e, lane);
            for (int32_t i = lane; i < n; i += kWave) {
                const int32_t p = av[i];
                if (p / g.C != learner) continue;
                const Row r = legality_row_bm(g, hdr, e, g.N + p);
                uint32_t w0 = env, w1 = 2u * (uint32_t)p, w2 = env, w3 = 2u * (uint32_t)p + 1u;
                threefry(ke0, ke1, w0, w1);
                threefry(ke0, ke1, w2, w3);
                uint32_t words[4] = {w0, w1, w2, w3};
                int32_t act[7];
                if (g.T <= 8) sample_row_words8(g, r, words, act);
                else sample_row_words(g, r, words, act);
                if (out.actions) {
                    int32_t* dst = out.actions + ((tt * lanes + l) * g.C + (p - learner * g.C)) * 7;
#pragma unroll
                    for (int f = 0; f < 7; ++f) dst[f] = act[f];
                }
                decode_row(g, e, p, true, act);
            }
        }
        if (out.actions) {
            // unavailable rows sample all zeros (a slot window's gap holds no
            // unit)
            const Env e = refresh<TW>(g, e_in);
            for (int32_t i = lane; i < Cg; i += TW) {
                const int32_t sl = g.N + learner * g.C + i;
                if (i < g.C && e.birth[sl] != kAbsent && e.pkind[sl] == kAbsent) continue;
                int32_t* dst = out.actions + ((tt * lanes + l) * Cg + i) * 7;
                const int32_t z = opaque_zero();
#pragma unroll
                for (int f = 0; f < 7; ++f) dst[f] = z;
            }
        }
        wave_sync();
        // the bot's rows
        // the carry stays in LDS between cycles: loaded once, settled in place
        const int32_t kept = bot_act<TW>(g, hdr, e_in, b, ba.y, l, ba.carry, ba.strategy, ba.trained, lane,
                                         !First && t == t_begin);
        const int32_t top = (1 << g.rank_bits) - 1;
        {
        const Env e = refresh<TW>(g, e_in);
        for (int32_t i = lane; i < g.C; i += TW) {
            const int32_t p = b.player * g.C + i;
            int32_t v[6];
            unit_command(g, e, b, ba.y, i, kept, v);
            at<int8_t>(e, y.c_kind)[p] = (int8_t)canon_kind(v[0]);
            at<int8_t>(e, y.c_dir)[p] = (int8_t)canon_dir(v[1]);
            at<int32_t>(e, y.c_none)[p] = v[2];
            at<int16_t>(e, y.c_target)[p] = (int16_t)canon_target(v[3], g.cells);
            at<int8_t>(e, y.c_ptype)[p] = (int8_t)canon_ptype(v[4], g.T);
            at<int16_t>(e, y.c_rank)[p] = (int16_t)clampi(v[5] == kAbsent ? 0 : v[5], 0, top);
        }
        }
        settle_carry<TW>(g, b, ba.y, l, ba.carry, lane, false);
        wave_sync();
        if (fast) {
            // the env-path admission: the learner and the bot command exactly
            // their available units.  The bot's region lay over the summary's
            // lists, so the available positions are listed again.
            const int32_t nav = list_available<TW>(g, e, lane);
            uint32_t ek0, ek1;
            episode_key<TW>(refresh<TW>(g, e_in), ek0, ek1);
            if constexpr (First) {
                // (the cycle's check above keeps the first pass on this path)
                admit_env<TW>(g, hdr, e, lane, ek0, ek1, false, nav, sm.irregular, false);
            } else {
                if (!admit_env(g, hdr, e, lane, ek0, ek1, false, nav, sm.irregular, false))
                    admit(g, hdr, e, lane, ek0, ek1, false);
            }
        }
        // completion's time and the outcome stay in registers into the
        // finish phase and the observation scalars
        int32_t time = 0;
        Outcome oc = {0, 0, 0, 0, 0};
        if (fast) {
            // the summary's live lanes: the bot, sampling and admission spawn
            // and remove nothing
            const LiveLanes known = summary_live(sm);
            const int32_t held = TW == kWave ? kWave : 2 * TW;
            time = complete<TW>(g, hdr, e, lane, false, sm.nlive <= held ? known : LiveLanes{-1, 0, 0});
            oc = decide_counted<TW>(refresh<TW>(g, e_in), lane);
        } else {
            if constexpr (!First) {
                uint32_t ek0, ek1;
                episode_key(e, ek0, ek1);
                core_step(g, hdr, e, lane, ek0, ek1, false);
            }
        }
        nanorts_env_results r = {};
        if (out.rewards) r.reward = out.rewards + tt * lanes * 2;
        if (out.dones) r.done = out.dones + tt * lanes;
        const bool done = finish_step<TW, First>(g, hdr, refresh<TW>(g, e_in), l, lane, args.partial != 0, r, false,
                                                 false, true, fast ? &oc : nullptr, time);
        if (done) {
            const Env e = refresh<TW>(g, e_in);
            clear_carry_rows<TW>(g, b, ba.y, lane);
            if (args.seats && args.draw) {
                uint32_t ek0, ek1;
                episode_key<TW>(e, ek0, ek1);
                learner = episode_seat(ek0, ek1);
            }
            // the published observation is the reset state's
            time = tuni<TW>(e.sc[S_TIME]);
            oc.res0 = tuni<TW>(e.sc[S_RES0]);
            oc.res1 = tuni<TW>(e.sc[S_RES1]);
            oc.alt = tuni<TW>(e.sc[S_ALT]);
        }
        const uint32_t d = (uint32_t)(out.depth > 0 ? out.depth : 1), c = (uint32_t)tt;
        const uint32_t ring = (d & (d - 1u)) == 0u ? (c & (d - 1u)) : c % d;
        const int64_t slot = (int64_t)ring * lanes + l;
        if (fast) {
            const int64_t per = (int64_t)g.cells * 6;
            uint8_t* m0 = out.feature_maps ? out.feature_maps + (slot * 2) * per : nullptr;
            if (out.scalars && lane < 8) {
                // own balance, the opponent's, time, alternating count
                const int32_t pl = lane >> 2, f = lane & 3;
                const int32_t own = pl == 0 ? oc.res0 : oc.res1, opp = pl == 0 ? oc.res1 : oc.res0;
                out.scalars[slot * 8 + lane] = f == 0 ? own : (f == 1 ? opp : (f == 2 ? time : oc.alt));
            }
            // the sight bitmaps persist in the event counters' words, which
            // the seat step does not count, when both planes fit there
            const int32_t kept_seen = 2 * g.H * g.seen_words <= 32 ? y.b_events : -1;
            sm = summarize<TW>(g, hdr, e, lane, args.partial != 0, m0, m0 ? m0 + per : nullptr, nullptr, nullptr,
                               kept_seen);
        } else if (out.feature_maps || out.scalars) {
            if constexpr (!First) observe_both(g, hdr, e, slot, lane, args.partial != 0, out.feature_maps, out.scalars);
        }
    }
    if constexpr (TW != kWave) asm volatile("" : "+v"(l));
    b.player = 1 - learner;
    b.block = g.N + b.player * g.C;
    // (the arguments of the stores read again: `args` is the kernel's
    // argument struct)
    const SeatRolloutArgs& fin = seat_args_again();
    const KGame& gf = fin.g;
    if (!First || stop > 0) {
        if (First) {
            if (gf.shift > 0) store_window_rows<TW>(gf, fin.s, l, e, lane);
            else store_env<TW>(gf, fin.s, l, e, lane);
            store_carry_window<TW>(gf, b, fin.bot.y, l, fin.bot.carry, lane);
        } else {
            // (a game resumed in its launch's last cycle has its carry loaded
            // by the bot's act; one that ran no cycle stores the state only)
            if (fin.steps > t_begin) store_carry<TW>(gf, b, fin.bot.y, l, fin.bot.carry, lane);
            store_env<TW>(gf, fin.s, l, e, lane);
        }
    }
    if (lane == 0) {
        if (fin.seats && (!First || stop > 0)) fin.seats[l] = learner;
        if (First) fin.out.progress[l] = stop;
        else if (!fin.resume && fin.out.progress) fin.out.progress[l] = 0;
    }
}

// 168 VGPRs at most: three waves per SIMD, which the bot region's LDS allows
// on boards up to 16x16
__global__ __launch_bounds__(256, 3) void k_seat_rollout(SeatRolloutArgs args) {
    (void)args;
    seat_cycles<false>(seat_args());
}

// The seat rollout's first pass: two games per wave on the slot window.
__global__ __launch_bounds__(256, 3) void k_seat_rollout_pair(SeatRolloutArgs args) {
    (void)args;
    seat_cycles<true, 32>(seat_args());
}

// GridNet decode_actions (N/adapters/gridnet/actions.py:31-52) into Commands.
__global__ __launch_bounds__(256) void k_gridnet_decode(KGame g, int64_t lanes, nanorts_state s, GridLayout gy,
                                                        const int32_t* actions, nanorts_command_buffers out) {
    NR_KERNEL_PROLOGUE
    load_env(g, s, l, e, LD_ALL, lane);
    const int32_t owned = 2 * g.C;
    gridnet_decode(g, hdr, e, gy, actions + l * 2 * g.cells * 7, 2, lane,
                   [&](int32_t p, int32_t kind, int32_t dir, int32_t none, int32_t target, int32_t ptype, int32_t order) {
                       const int64_t at = l * owned + p;
                       out.kind[at] = kind;
                       out.direction[at] = dir;
                       out.none_duration[at] = none;
                       out.target_cell[at] = target;
                       out.produced_type[at] = ptype;
                       out.request_order[at] = order;
                   });
}

// GridNet decode from the reference's operands (the FFI target
// nanorts_gridnet_decode): per-lane strides in elements, 0 for an operand
// shared by every lane; player 0's legality comes from the move_direction,
// produce_direction and produce_type operands instead of the state.
struct GridOperands {
    const int32_t* actions;
    const uint8_t* move;
    const uint8_t* pdir;
    const uint8_t* ptype;
    int64_t actions_stride, move_stride, pdir_stride, ptype_stride;
};
__global__ __launch_bounds__(256) void k_gridnet_decode_operands(KGame g, int64_t lanes, nanorts_state s,
                                                                 const int32_t* unit_cost, uint32_t shared,
                                                                 GridLayout gy, GridOperands o,
                                                                 nanorts_command_buffers out) {
    NR_KERNEL_PROLOGUE_OPERAND_TABLE(unit_cost, 1)
    const uint32_t read = LD_BIRTH | LD_PKIND | LD_CELL | LD_PDIR | LD_PPTYPE;
    load_env(g, s, l, e, read & ~shared, lane);
    if ((read & shared) != 0u) load_env(g, s, 0, e, read & shared, lane);
    if (lane < S_COUNT) {
        const int64_t row = (shared & LD_SCALARS) ? 0 : l;
        e.sc[lane] = lane == S_RES0 ? s.player_resources[2 * row] : (lane == S_RES1 ? s.player_resources[2 * row + 1] : 0);
    }
    wave_sync();
    const int32_t owned = 2 * g.C;
    const uint8_t* move = o.move + l * o.move_stride;
    const uint8_t* pdir = o.pdir + l * o.pdir_stride;
    const uint8_t* ptype = o.ptype + l * o.ptype_stride;
    gridnet_decode_by(
        g, hdr, e, gy, o.actions + l * o.actions_stride, 2, lane,
        [&](int32_t p, int32_t kind, int32_t dir, int32_t none, int32_t target, int32_t pt, int32_t order) {
            const int64_t at = l * owned + p;
            out.kind[at] = kind;
            out.direction[at] = dir;
            out.none_duration[at] = none;
            out.target_cell[at] = target;
            out.produced_type[at] = pt;
            out.request_order[at] = order;
        },
        [&](int32_t i, const GridRow& r) {
            return r.kind == kKindMove ? move[i * 4 + gidx(r.dir, 4)] != 0
                                       : (pdir[i * 4 + gidx(r.dir, 4)] != 0 && ptype[i * g.T + gidx(r.ptype, g.T)] != 0);
        });
}

// GridNet observe (N/adapters/gridnet/observation.py:27-72).
__global__ __launch_bounds__(256) void k_gridnet_observe(KGame g, int64_t lanes, nanorts_state s, nanorts_gridnet_obs o) {
    NR_KERNEL_PROLOGUE
    load_env(g, s, l, e, LD_ALL, lane);
    gridnet_observe(g, hdr, e, l, lane, o, o.planes);
}

// GridNet step (N/adapters/gridnet/env.py:65-118): decode, core.step keyed by
// the episode root, reward components and dones, the ending state's planes,
// auto-reset and the observation of the post-reset state.  With `against`,
// step_against (env.py:73-83): player 0's rows are decoded from `actions`
// ([L][H][W][7]) and player 1 plays the given Commands.
__global__ __launch_bounds__(256) void k_gridnet_step(KGame g, int64_t lanes, nanorts_state s, GridLayout gy,
                                                      const int32_t* actions, nanorts_commands given, int32_t against,
                                                      nanorts_gridnet_results r) {
    NR_KERNEL_PROLOGUE
    load_env(g, s, l, e, LD_ALL, lane);
    count_units(g, e, lane);
    uint32_t k0 = (uint32_t)uni(e.sc[S_ROOT0]), k1 = (uint32_t)uni(e.sc[S_ROOT1]);
    fold_in(k0, k1, (uint32_t)uni(e.sc[S_EPISODE]));
    const Layout& y = g.lay;
    const int32_t top = (1 << g.rank_bits) - 1;
    const int32_t players = against ? 1 : 2;
    gridnet_decode(g, hdr, e, gy, actions + l * players * g.cells * 7, players, lane,
                   [&](int32_t p, int32_t kind, int32_t dir, int32_t none, int32_t target, int32_t ptype, int32_t order) {
                       at<int8_t>(e, y.c_kind)[p] = (int8_t)canon_kind(kind);
                       at<int8_t>(e, y.c_dir)[p] = (int8_t)canon_dir(dir);
                       at<int32_t>(e, y.c_none)[p] = none;
                       at<int16_t>(e, y.c_target)[p] = (int16_t)canon_target(target, g.cells);
                       at<int8_t>(e, y.c_ptype)[p] = (int8_t)canon_ptype(ptype, g.T);
                       at<int16_t>(e, y.c_rank)[p] = (int16_t)clampi(order == kAbsent ? 0 : order, 0, top);
                   });
    if (against) {
        for (int32_t p = g.C + lane; p < 2 * g.C; p += kWave) {
            const int64_t i = l * 2 * g.C + p;
            at<int8_t>(e, y.c_kind)[p] = (int8_t)canon_kind(given.kind[i]);
            at<int8_t>(e, y.c_dir)[p] = (int8_t)canon_dir(given.direction[i]);
            at<int8_t>(e, y.c_ptype)[p] = (int8_t)canon_ptype(given.produced_type[i], g.T);
            at<int16_t>(e, y.c_target)[p] = (int16_t)canon_target(given.target_cell[i], g.cells);
            at<int32_t>(e, y.c_none)[p] = given.none_duration[i];
            const int32_t ro = given.request_order[i];
            at<int16_t>(e, y.c_rank)[p] = (int16_t)clampi(ro == kAbsent ? 0 : ro, 0, top);
        }
    }
    wave_sync();
    core_step(g, hdr, e, lane, k0, k1, true);
    // reward dones (N/adapters/rewards.py:30-44): column 0 done, column 1
    // no resource pile left carrying resources
    const bool over = uni(e.sc[S_GAME_OVER]) != 0;
    const bool done = over || uni(e.sc[S_TIME]) >= g.max_cycles;
    bool stacked = false;
    for (int32_t sl = lane; sl < g.E; sl += kWave)
        stacked |= e.birth[sl] != kAbsent && type_flag(g, hdr, e.utype[sl], FL_RESOURCE) && e.carried[sl] > 0;
    stacked = ballot(stacked) != 0ull;
    if (r.reward_dones && lane < 12) {
        const int32_t c = lane % 6;
        r.reward_dones[l * 12 + lane] = (c == 0 && done) || (c == 1 && !stacked) ? 1 : 0;
    }
    if (r.final_planes) {
        nanorts_gridnet_obs planes_only = r.observation;
        planes_only.source_mask = nullptr;
        planes_only.action_mask = nullptr;
        gridnet_observe(g, hdr, e, l, lane, planes_only, r.final_planes);
    }
    nanorts_env_results er = {};
    er.terminated = r.terminated;
    er.truncated = r.truncated;
    er.done = r.done;
    er.winner = r.winner;
    er.spawn_overflowed = r.spawn_overflowed;
    er.reward_components = r.reward_components;
    er.spawn_overflow = r.spawn_overflow;
    finish_step(g, hdr, e, l, lane, false, er, true);
    store_env(g, s, l, e, lane);
    gridnet_observe(g, hdr, e, l, lane, r.observation, r.observation.planes);
}

// The JaxMARL request (N/adapters/jaxmarl/env.py:181-184): decode_actions
// (N/adapters/jaxmarl/actions.py:61-84) into Commands, and the episode root
// fold_in(environment_root, episode_index) that keys core.step.
__global__ __launch_bounds__(256) void k_decode_actions(KGame g, int64_t lanes, nanorts_state s, const int32_t* actions,
                                                        nanorts_command_buffers out, uint32_t* keys) {
    NR_KERNEL_PROLOGUE
    load_env(g, s, l, e, LD_BIRTH | LD_CELL | LD_PKIND | LD_SCALARS, lane);
    const int32_t owned = 2 * g.C;
    for (int32_t p = lane; p < owned; p += kWave) {
        const int32_t slot = g.N + p;
        const bool available = e.birth[slot] != kAbsent && e.pkind[slot] == kAbsent;
        const int32_t* row = actions + (l * owned + p) * 7;
        const int64_t at = l * owned + p;
        int32_t kind = kAbsent, dir = kAbsent, none = 0, target = kAbsent, ptype = kAbsent;
        if (available) {
            const GridRow r = grid_row(g, row, e.cell[slot]);  // the factor helpers of factors.py:117-151
            kind = r.kind;
            dir = r.dir;
            ptype = r.ptype;
            target = r.target;
            none = kind == kKindNone ? 1 : 0;
        }
        out.kind[at] = kind;
        out.direction[at] = dir;
        out.none_duration[at] = none;
        out.target_cell[at] = target;
        out.produced_type[at] = ptype;
        out.request_order[at] = kAbsent;
    }
    if (keys && lane == 0) {
        uint32_t k0 = (uint32_t)e.sc[S_ROOT0], k1 = (uint32_t)e.sc[S_ROOT1];
        fold_in(k0, k1, (uint32_t)e.sc[S_EPISODE]);
        keys[2 * l] = k0;
        keys[2 * l + 1] = k1;
    }
}

// Pixel observations (N/observations/pixels.py:71-88; N/rendering/raster.py:53-127).
__global__ __launch_bounds__(256) void k_pixels(KGame g, int64_t lanes, nanorts_state s, int32_t partial, const uint8_t* tiles, uint8_t* image,
                         int32_t* scalars) {
    NR_KERNEL_PROLOGUE
    load_env(g, s, l, e,
             LD_BIRTH | LD_UTYPE | LD_OWNER | LD_CELL | LD_HP | LD_CARRIED | LD_PKIND | LD_ENTITY | LD_SCALARS, lane);
    const int32_t occupant_states = 1 + 3 * g.T;
    const int64_t row_bytes = (int64_t)g.W * 16 * 3;
    const int64_t per = (int64_t)g.H * 16 * row_bytes;
    for (int32_t pl = 0; pl < 2; ++pl) {
        if (partial) stamp_visibility(g, hdr, e, lane, pl);
        uint8_t* img = image + (l * 2 + pl) * per;
        // one lane writes one 4-pixel (12-byte) run of one sprite row
        const int32_t runs = g.cells * 16 * 4;
        for (int32_t w = lane; w < runs; w += kWave) {
            const int32_t c = w >> 6;
            const int32_t py = (w >> 2) & 15;
            const int32_t px0 = (w & 3) * 4;
            const int32_t occ = e.entity[c];
            bool present = occ != kAbsent;
            const int32_t sl = clampi(occ, 0, g.E - 1);
            if (present && partial) {
                const int32_t cell_of = clampi(e.cell[sl], 0, g.cells - 1);
                present = e.birth[sl] != kAbsent && (e.owner[sl] == pl || seen_at(g, e, cell_of));
            }
            int32_t owner = present ? e.owner[sl] : kAbsent;
            if (owner >= 0) owner = (owner + pl) & 1;
            const int32_t type = present ? e.utype[sl] : kAbsent;
            const int32_t pk = present ? e.pkind[sl] : 0;
            const int32_t kind = pk > 0 ? pk : 0;
            const int32_t carried = present ? e.carried[sl] : 0;
            const int32_t hp = present ? e.hp[sl] : 0;
            const int32_t occupant = present ? 1 + (owner + 1) * g.T + type : 0;
            const int32_t tile = gidx((hdr.terrain[c] ? occupant_states : 0) + occupant, 2 * occupant_states);
            const uint8_t* src = tiles + ((int64_t)tile * 256 + py * 16 + px0) * 3;
            uint8_t px[12];
#pragma unroll
            for (int k = 0; k < 12; ++k) px[k] = src[k];
            if (present && py >= 12 && py <= 14) {
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const int32_t x = px0 + k;
                    if (x < 1 || x >= 15) continue;
                    const int32_t position = x - 1;
                    bool lit;
                    if (py == 12) lit = kind == position + 1;
                    else if (py == 13) lit = ((carried >> position) & 1) != 0;
                    else lit = hp > position;
                    px[3 * k] = px[3 * k + 1] = px[3 * k + 2] = lit ? 0xFF : 0x00;
                }
            }
            const int32_t cy = cell_y(g, c), cx = c - cy * g.W;
            uint8_t* dst = img + (int64_t)(cy * 16 + py) * row_bytes + (int64_t)(cx * 16 + px0) * 3;
            if ((((uintptr_t)dst) & 3u) == 0) {
                uint32_t* d4 = (uint32_t*)dst;
                d4[0] = px[0] | (px[1] << 8) | (px[2] << 16) | ((uint32_t)px[3] << 24);
                d4[1] = px[4] | (px[5] << 8) | (px[6] << 16) | ((uint32_t)px[7] << 24);
                d4[2] = px[8] | (px[9] << 8) | (px[10] << 16) | ((uint32_t)px[11] << 24);
            } else {
                for (int k = 0; k < 12; ++k) dst[k] = px[k];
            }
        }
        wave_sync();
        if (scalars && lane < 4) {
            int32_t v;
            if (lane == 0) v = e.sc[S_RES0 + pl];
            else if (lane == 1) v = e.sc[S_RES0 + (pl ^ 1)];
            else if (lane == 2) v = e.sc[S_TIME];
            else v = e.sc[S_ALT];
            scalars[(l * 2 + pl) * 4 + lane] = v;
        }
    }
}

// Pixel observations from symbolic feature maps (pixels_from_symbolic,
// N/observations/pixels.py:91-110): the maps carry presence (type != 0),
// the observer-relative owner, type, pending kind, carried resources, hit
// points and terrain, which is all the tile pick and glyph band read.
// HBM-write-bound: 768 bytes written per cell per image.  One thread per
// cell row: 16 pixels x RGB = 48 bytes from the cell's tile row, with the
// glyph bands (rows 12-14 of an occupied cell: action, carried resources,
// hit points; N/rendering/raster.py:53-127) drawn over pixels 1-14.  A
// wave's 64 cell rows are consecutive in the image, so its 3 KB of output
// are too: the rows are staged in LDS and stored back as chunks 16 bytes
// apart across the lanes, each store instruction writing 1 KB of consecutive
// bytes.  Grid: x = 256 cell rows, y (+ 65535 z) = image.
constexpr int kPixelWaves = 4;
__global__ __launch_bounds__(kPixelWaves * 64) void k_pixels_from_maps(int32_t H, int32_t W, int32_t T, int32_t wshift,
                                                                       int64_t images, const uint8_t* maps,
                                                                       const uint8_t* tiles, uint8_t* image) {
    __shared__ u32x4 stage[kPixelWaves * kWave * 3];
    const int64_t m = (int64_t)blockIdx.z * 65535 + blockIdx.y;
    if (m >= images) return;
    const int lane = lane_id(), wave = (int)(threadIdx.x >> 6);
    const int32_t per_image = 16 * H * W;  // cell rows of one image
    const int32_t n0 = (int32_t)blockIdx.x * (kPixelWaves * kWave) + wave * kWave;  // the wave's first
    if (n0 >= per_image) return;
    const int32_t n = n0 + lane;
    AS3 u32x4* mine = (AS3 u32x4*)stage + wave * kWave * 3;
    if (n < per_image) {
        const int32_t Y = wshift >= 0 ? n >> wshift : n / W;
        const int32_t cx = n - Y * W;
        const int32_t cy = Y >> 4, py = Y & 15;
        const uint8_t* f = maps + ((m * H + cy) * W + cx) * 6;
        const int32_t hp = f[0], carried = f[1], owner = (int32_t)f[2] - 1, type = f[3], kind = f[4], terrain = f[5];
        const bool present = type != 0;
        const int32_t states = 1 + 3 * T;
        const int32_t occupant = present ? 1 + (owner + 1) * T + (type - 1) : 0;
        const int32_t tile = gidx(terrain * states + occupant, 2 * states);
        const u32x4* src = (const u32x4*)(tiles + (int64_t)tile * 768 + py * 48);
        u32x4 v[3] = {src[0], src[1], src[2]};
        if (present && py >= 12 && py <= 14) {
            // lit pixels of the band row as a bit set over pixels 1..14
            uint32_t lit = 0u;
#pragma unroll
            for (int32_t x = 1; x < 15; ++x) {
                const int32_t position = x - 1;
                bool on;
                if (py == 12) on = kind == position + 1;
                else if (py == 13) on = ((carried >> position) & 1) != 0;
                else on = hp > position;
                lit |= (on ? 1u : 0u) << x;
            }
#pragma unroll
            for (int k = 0; k < 3; ++k)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    uint32_t w = v[k][j];
#pragma unroll
                    for (int bi = 0; bi < 4; ++bi) {
                        const int32_t x = (16 * k + 4 * j + bi) / 3;  // the byte's pixel
                        if (x >= 1 && x <= 14) {
                            const uint32_t c = ((lit >> x) & 1u) ? 0xFFu : 0x00u;
                            w = (w & ~(0xFFu << (8 * bi))) | (c << (8 * bi));
                        }
                    }
                    v[k][j] = w;
                }
        }
#pragma unroll
        for (int k = 0; k < 3; ++k) mine[3 * lane + k] = v[k];
    }
    wave_sync();
    const int32_t valid = per_image - n0 < kWave ? per_image - n0 : kWave;  // cell rows in this wave
    u32x4* out = (u32x4*)(image + (m * per_image + n0) * 48);
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        const int32_t c = k * kWave + lane;  // the 16-byte chunk of the wave's run
        // the images are written once and not read back by this kernel:
        // streaming (non-temporal) stores
        if (c < 3 * valid) __builtin_nontemporal_store((u32x4)mine[c], out + c);
    }
}

// wave64 semantics probe: ballot, mbcnt prefix counts, shuffles, prefix-min.
__global__ void k_probe(int32_t* out) {
    const int lane = lane_id();
    const uint64_t m = ballot((lane % 3) == 0);
    const int32_t below = count_below(m);
    const int32_t up = __shfl_up(lane, 1u, kWave);
    const int32_t mn = wave_inclusive_min(100 - lane, lane);
    const bool ok = popc(m) == 22 && below == (lane + 2) / 3 && (lane == 0 || up == lane - 1) && mn == 100 - lane;
    const uint64_t all = ballot(ok);
    if (lane == 0) out[blockIdx.x] = all == ~0ull ? 1 : 0;  // one word per probe wave (block of 64)
}

// Probe words of nanorts_amd_self_check_no_alloc: one per probe wave, in a
// file-scope array each device holds until the process ends, so that check
// allocates no device memory.  Host code reaches it only through the address
// hipGetSymbolAddress returns on each device (probe_scratch below).
constexpr int32_t kProbeScratchWords = 1024;
static __device__ __align__(256) int32_t scratch[kProbeScratchWords];

// Host threefry2x32 (20 rounds) and fold_in(k, d) = threefry(k, (0, d)), the
// same published Random123 cipher the kernels evaluate.
static uint32_t host_rotl(uint32_t x, uint32_t d) { return (x << d) | (x >> (32u - d)); }
static void host_threefry(uint32_t k0, uint32_t k1, uint32_t& x0, uint32_t& x1) {
    static const uint32_t rot[8] = {13, 15, 26, 6, 17, 29, 16, 24};
    const uint32_t ks[3] = {k0, k1, k0 ^ k1 ^ 0x1BD11BDAu};
    x0 += ks[0];
    x1 += ks[1];
    for (uint32_t block = 0; block < 5; ++block) {
        for (uint32_t i = 0; i < 4; ++i) {
            x0 += x1;
            x1 = host_rotl(x1, rot[(block & 1u) * 4 + i]);
            x1 ^= x0;
        }
        x0 += ks[(block + 1) % 3];
        x1 += ks[(block + 2) % 3] + block + 1u;
    }
}
static void host_fold_in(uint32_t& k0, uint32_t& k1, uint32_t data) {
    uint32_t x0 = 0u, x1 = data;
    host_threefry(k0, k1, x0, x1);
    k0 = x0;
    k1 = x1;
}

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------
extern "C" {

const char* nanorts_amd_build_id(void) { return NANORTS_BUILD_ID; }

const char* nanorts_amd_entries(void) {
    return "nanorts_amd_step,nanorts_amd_step_ffi,nanorts_amd_legality,nanorts_amd_legality_words,nanorts_amd_legality_ffi,"
           "nanorts_amd_avail_actions,nanorts_amd_visible_cells,nanorts_amd_visible_cells_ffi,nanorts_amd_reset_rows_ffi,"
           "nanorts_amd_observe,nanorts_amd_pixels,nanorts_amd_pixels_from_maps,nanorts_amd_reset_where_done,nanorts_amd_env_step,nanorts_amd_sample_actions,"
           "nanorts_amd_step_groups,nanorts_amd_step_groups_ffi,nanorts_amd_env_transition,nanorts_amd_decode_actions,nanorts_amd_rollout,"
           "nanorts_amd_abstraction_act,nanorts_amd_abstraction_act_ffi,nanorts_amd_seat_step,nanorts_amd_seat_rollout,"
           "nanorts_amd_seat_step_lanes,nanorts_amd_seat_rollout_lanes,nanorts_amd_episode_seats,nanorts_amd_astar_search_ffi,"
           "nanorts_amd_astar_chain_ffi,nanorts_amd_gridnet_decode,nanorts_amd_gridnet_decode_ffi,"
           "nanorts_amd_gridnet_observe,nanorts_amd_gridnet_step,nanorts_amd_gridnet_step_against,nanorts_amd_gridnet_sample_actions";
}

const char* nanorts_amd_last_error(void) { return g_error.c_str(); }

int64_t nanorts_amd_shared_opt_in(const int32_t* devices, int64_t n) {
    int64_t least = 0;
    for (int64_t i = 0; i < n; ++i) {
        int bytes = 0;
        if (!devices || hipDeviceGetAttribute(&bytes, hipDeviceAttributeMaxSharedMemoryPerBlock, devices[i]) != hipSuccess) {
            (void)hipGetLastError();
            return 0;
        }
        least = i == 0 ? bytes : (bytes < least ? bytes : least);
    }
    return least;
}

const char* nanorts_amd_self_check(const int32_t* devices, int64_t n) {
    static thread_local std::string result;
    result.clear();
    int current = 0;
    (void)hipGetDevice(&current);
    for (int64_t i = 0; i < n; ++i) {
        if (hipSetDevice(devices[i]) != hipSuccess) {
            result = "cannot select device " + std::to_string(devices[i]);
            break;
        }
        hipDeviceProp_t prop;
        if (hipGetDeviceProperties(&prop, devices[i]) != hipSuccess || prop.warpSize != 64) {
            result = "device " + std::to_string(devices[i]) + " does not run 64-wide wavefronts";
            break;
        }
        int32_t* d = nullptr;
        if (hipMalloc(&d, sizeof(int32_t)) != hipSuccess) {
            result = "probe allocation failed";
            break;
        }
        int32_t h = 0;
        hipLaunchKernelGGL(k_probe, dim3(1), dim3(64), 0, nullptr, d);
        const bool copied = hipMemcpy(&h, d, sizeof(h), hipMemcpyDeviceToHost) == hipSuccess;
        (void)hipFree(d);
        if (!copied || h != 1) {
            result = "wave64 probe failed on device " + std::to_string(devices[i]);
            break;
        }
    }
    (void)hipSetDevice(current);
    return result.c_str();
}

}  // extern "C"

namespace {
std::mutex g_scratch_mutex;
std::vector<int32_t*> g_scratch_address;  // per device ordinal

// The device address of `scratch` on `device`, which must be current: taken
// with hipGetSymbolAddress on the first call for that device and kept.
bool probe_scratch(int device, int32_t** address, std::string* why) {
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (device < 0) {
        *why = "no current device";
        return false;
    }
    if ((int)g_scratch_address.size() <= device) g_scratch_address.resize((size_t)device + 1, nullptr);
    if (!g_scratch_address[(size_t)device]) {
        void* p = nullptr;
        const hipError_t err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (err != hipSuccess || !p) {
            *why = std::string("hipGetSymbolAddress of the probe scratch failed: ") + hipGetErrorString(err);
            return false;
        }
        g_scratch_address[(size_t)device] = (int32_t*)p;
    }
    *address = g_scratch_address[(size_t)device];
    return true;
}
}  // namespace

extern "C" {

const char* nanorts_amd_self_check_no_alloc(const int32_t* devices, int64_t n, int32_t waves, int32_t* probe_words) {
    static thread_local std::string result;
    static thread_local int32_t words[kProbeScratchWords];
    result.clear();
    if (waves < 1 || waves > kProbeScratchWords) {
        result = "waves is " + std::to_string(waves) + "; the probe scratch holds 1 to " +
                 std::to_string(kProbeScratchWords) + " waves";
        return result.c_str();
    }
    if (n > 0 && !devices) {
        result = "devices is NULL";
        return result.c_str();
    }
    int current = 0;
    (void)hipGetDevice(&current);
    for (int64_t i = 0; i < n; ++i) {
        if (hipSetDevice(devices[i]) != hipSuccess) {
            result = "cannot select device " + std::to_string(devices[i]);
            break;
        }
        hipDeviceProp_t prop;
        if (hipGetDeviceProperties(&prop, devices[i]) != hipSuccess || prop.warpSize != 64) {
            result = "device " + std::to_string(devices[i]) + " does not run 64-wide wavefronts";
            break;
        }
        int32_t* address = nullptr;
        std::string why;
        if (!probe_scratch(devices[i], &address, &why)) {
            result = why;
            break;
        }
        // the scratch keeps the last call's words: clear the ones this call reads
        hipLaunchKernelGGL(k_zero_bytes, dim3(1), dim3(256), 0, nullptr, (uint8_t*)address, (int64_t)waves * 4);
        hipLaunchKernelGGL(k_probe, dim3((unsigned)waves), dim3(64), 0, nullptr, address);
        if (hipGetLastError() != hipSuccess ||
            hipMemcpy(words, address, sizeof(int32_t) * (size_t)waves, hipMemcpyDeviceToHost) != hipSuccess) {
            result = "the probe launch or its read-back failed on device " + std::to_string(devices[i]);
            break;
        }
        if (probe_words) std::memcpy(probe_words, words, sizeof(int32_t) * (size_t)waves);
        for (int32_t w = 0; w < waves; ++w) {
            if (words[w] != 1) {
                result = "wave64 probe failed on device " + std::to_string(devices[i]) + " (wave " +
                         std::to_string(w) + ")";
                break;
            }
        }
        if (!result.empty()) break;
    }
    (void)hipSetDevice(current);
    return result.c_str();
}

#define NR_SHAPE(game)                                                   \
    Shape sh;                                                            \
    {                                                                    \
        std::string why;                                                 \
        if (!shape_for(game, &sh, &why)) return fail(NANORTS_INVALID_ARGUMENT, why); \
    }

#define NR_READER_SHAPE(game, masks)                                                  \
    Shape sh;                                                                         \
    {                                                                                 \
        std::string why;                                                              \
        if (!shape_for_reader(game, masks, &sh, &why)) return fail(NANORTS_INVALID_ARGUMENT, why); \
    }

#define NR_STATE(state)                                                                      \
    if (!state_complete(state)) return fail(NANORTS_INVALID_ARGUMENT, "a State leaf pointer is NULL");

int nanorts_amd_step(void* stream, const nanorts_game* game, nanorts_state state, int64_t lanes, const uint32_t* key,
                 int64_t key_lanes, nanorts_commands commands, nanorts_step_results results) {
    NR_SHAPE(game)
    NR_STATE(state)
    if (!key || (key_lanes != 1 && key_lanes != lanes))
        return fail(NANORTS_INVALID_ARGUMENT, "key must be [1][2] or [lanes][2]");
    if (!commands.kind || !commands.direction || !commands.none_duration || !commands.target_cell ||
        !commands.produced_type || !commands.request_order)
        return fail(NANORTS_INVALID_ARGUMENT, "a Commands field pointer is NULL");
    return launch(k_step, sh, lanes, (hipStream_t)stream, state, key, key_lanes, commands, lanes, results);
}

// One group of the step target's operands and results (nanorts_amd_step_ffi's
// order) as the kernel's State, Commands and results.  A result that does not
// alias its state operand is first filled from it, so the step runs in the
// result buffers.  The per-slot completion records (results 27-30) are the
// kernel's.
static int step_operands(hipStream_t st, const char* target, const void* const* operands, void* const* results,
                         int64_t lanes, int64_t E, int64_t cells, nanorts_state* s, nanorts_commands* c,
                         nanorts_step_results* r) {
    for (int i = 0; i < 33; ++i)
        if (!operands[i]) return fail(NANORTS_INVALID_ARGUMENT, std::string(target) + ": operand " + std::to_string(i) + " is NULL");
    for (int i = 0; i < 31; ++i)
        if (!results[i]) return fail(NANORTS_INVALID_ARGUMENT, std::string(target) + ": result " + std::to_string(i) + " is NULL");
    // Bytes per lane of the 23 state leaves in the reference's order.
    const int64_t leaf_bytes[23] = {E * 4, E, E, E * 2, E * 2, E * 4, E, E, E * 4, E * 2, E, E * 4, E * 4, E * 4,
                                    cells * 2, 4, 8, 4, 4, 4, 1, 4, 8};
    void* leaf[23];
    for (int i = 0; i < 23; ++i) {
        leaf[i] = results[i];
        if (results[i] != operands[10 + i] && lanes > 0 &&
            hipMemcpyAsync(results[i], operands[10 + i], (size_t)(leaf_bytes[i] * lanes), hipMemcpyDeviceToDevice, st) !=
                hipSuccess)
            return fail(NANORTS_INTERNAL, std::string(target) + ": copying an unaliased state leaf failed");
    }
    std::memset(s, 0, sizeof(*s));
    s->birth = (int32_t*)leaf[0];
    s->unit_type = (int8_t*)leaf[1];
    s->owner = (int8_t*)leaf[2];
    s->cell = (int16_t*)leaf[3];
    s->hit_points = (int16_t*)leaf[4];
    s->carried_resources = (int32_t*)leaf[5];
    s->pending_kind = (int8_t*)leaf[6];
    s->pending_direction = (int8_t*)leaf[7];
    s->pending_none_duration = (int32_t*)leaf[8];
    s->pending_target_cell = (int16_t*)leaf[9];
    s->pending_produced_type = (int8_t*)leaf[10];
    s->pending_issued_at = (int32_t*)leaf[11];
    s->pending_completes_at = (int32_t*)leaf[12];
    s->pending_order = (int32_t*)leaf[13];
    s->entity_at = (int16_t*)leaf[14];
    s->time = (int32_t*)leaf[15];
    s->player_resources = (int32_t*)leaf[16];
    s->next_birth = (int32_t*)leaf[17];
    s->next_pending_order = (int32_t*)leaf[18];
    s->alternating_conflict_count = (int32_t*)leaf[19];
    s->game_over = (uint8_t*)leaf[20];
    s->winner = (int32_t*)leaf[21];
    s->spawn_overflow = (int32_t*)leaf[22];
    c->kind = (const int32_t*)operands[1];
    c->direction = (const int32_t*)operands[2];
    c->none_duration = (const int32_t*)operands[3];
    c->target_cell = (const int32_t*)operands[4];
    c->produced_type = (const int32_t*)operands[5];
    c->request_order = (const int32_t*)operands[6];
    std::memset(r, 0, sizeof(*r));
    r->admitted_harvest = (int32_t*)results[23];
    r->admitted_return = (int32_t*)results[24];
    r->admitted_produce = (int32_t*)results[25];
    r->admitted_attack = (int32_t*)results[26];
    r->is_member = (uint8_t*)results[27];
    r->records_i32 = (int32_t*)results[28];
    r->records_i16 = (int16_t*)results[29];
    r->records_i8 = (int8_t*)results[30];
    return NANORTS_OK;
}

// The bucket a step target's extents describe; the unit table columns stay
// zero and come from the table / timings operands in the kernel.
static nanorts_game step_bucket(int32_t height, int32_t width, int32_t neutral, int32_t capacity, int32_t types,
                                int64_t strategy, const void* terrain) {
    nanorts_game game;
    std::memset(&game, 0, sizeof(game));
    game.height = height;
    game.width = width;
    game.cells = height * width;
    game.neutral = neutral;
    game.capacity = capacity;
    game.entities = neutral + 2 * capacity;
    game.types = types;
    game.offsets = 1;  // a step decodes no legality rows: one target offset is a valid window
    game.strategy = (int32_t)strategy;
    game.max_cycles = 0x7fffffff;  // truncation is not a result of these targets
    game.terrain = (const uint8_t*)terrain;
    return game;
}

int nanorts_amd_step_ffi(void* stream, const void* const* operands, void* const* results, int64_t lanes,
                         int64_t key_lanes, int64_t command_lanes, int32_t height, int32_t width, int32_t neutral,
                         int32_t capacity, int32_t types, int64_t strategy) {
    if (!operands || !results) return fail(NANORTS_INVALID_ARGUMENT, "nanorts_amd_step_ffi: operands or results is NULL");
    if (strategy < NANORTS_CANCEL_BOTH || strategy > NANORTS_CANCEL_ALTERNATING)
        return fail(NANORTS_INVALID_ARGUMENT, "nanorts_amd_step_ffi: strategy must be 0, 1 or 2");
    if (lanes < 0 || (lanes > 0 && (key_lanes != 1 && key_lanes != lanes)))
        return fail(NANORTS_INVALID_ARGUMENT, "nanorts_amd_step_ffi: the key operand holds 1 or `lanes` rows");
    if (lanes > 0 && command_lanes != 1 && command_lanes != lanes)
        return fail(NANORTS_INVALID_ARGUMENT, "nanorts_amd_step_ffi: the Commands operands hold 1 or `lanes` rows");
    nanorts_game game = step_bucket(height, width, neutral, capacity, types, strategy, operands[7]);
    NR_SHAPE(&game)
    sh.g.ref_table = (const int32_t*)operands[8];
    sh.g.ref_timings = (const int32_t*)operands[9];
    const hipStream_t st = (hipStream_t)stream;
    nanorts_state s;
    nanorts_commands c;
    nanorts_step_results r;
    const int code = step_operands(st, "nanorts_amd_step_ffi", operands, results, lanes, game.entities, game.cells, &s,
                                   &c, &r);
    if (code != NANORTS_OK) return code;
    return launch(k_step, sh, lanes, st, s, (const uint32_t*)operands[0], key_lanes, c, command_lanes, r);
}

int nanorts_amd_step_groups_ffi(void* stream, int32_t groups, const void* const* operands, void* const* results,
                                const int64_t* lanes, const int64_t* key_lanes, const int64_t* command_lanes,
                                int32_t height, int32_t width, int32_t neutral, int32_t capacity, int32_t types,
                                int64_t strategy) {
    const char* target = "nanorts_amd_step_groups_ffi";
    if (groups < 1 || groups > 16) return fail(NANORTS_INVALID_ARGUMENT, std::string(target) + ": groups must be in [1, 16]");
    if (!operands || !results || !lanes || !key_lanes || !command_lanes)
        return fail(NANORTS_INVALID_ARGUMENT, std::string(target) + ": NULL argument");
    if (strategy < NANORTS_CANCEL_BOTH || strategy > NANORTS_CANCEL_ALTERNATING)
        return fail(NANORTS_INVALID_ARGUMENT, std::string(target) + ": strategy must be 0, 1 or 2");
    for (int32_t k = 0; k < groups; ++k) {
        if (lanes[k] < 0) return fail(NANORTS_INVALID_ARGUMENT, std::string(target) + ": lanes must be >= 0");
        if (lanes[k] > 0 && ((key_lanes[k] != 1 && key_lanes[k] != lanes[k]) ||
                             (command_lanes[k] != 1 && command_lanes[k] != lanes[k])))
            return fail(NANORTS_INVALID_ARGUMENT, std::string(target) + ": group " + std::to_string(k) +
                                                      "'s key and Commands operands hold 1 or `lanes` rows");
        if (!operands[33 * k + 7])
            return fail(NANORTS_INVALID_ARGUMENT, std::string(target) + ": group " + std::to_string(k) + "'s terrain is NULL");
    }
    // one LDS shape for every group: the bucket is shared, the terrain and
    // tables are each group's own
    nanorts_game game = step_bucket(height, width, neutral, capacity, types, strategy, operands[7]);
    NR_SHAPE(&game)
    const hipStream_t st = (hipStream_t)stream;
    for (int32_t c0 = 0; c0 < groups; c0 += kGroupsPerLaunch) {
        GroupsArgs args;
        std::memset(&args, 0, sizeof(args));
        args.g = sh.g;
        int64_t blocks = 0;
        for (int32_t k = c0; k < groups && k < c0 + kGroupsPerLaunch; ++k) {
            const void* const* ops = operands + 33 * k;
            void* const* rets = results + 31 * k;
            nanorts_state s;
            nanorts_commands c;
            nanorts_step_results r;
            const int code = step_operands(st, target, ops, rets, lanes[k], game.entities, game.cells, &s, &c, &r);
            if (code != NANORTS_OK) return code;
            if (lanes[k] == 0) continue;
            GroupSlot& slot = args.slot[args.count++];
            slot.s = s;
            slot.c = c;
            slot.r = r;
            slot.key = (const uint32_t*)ops[0];
            slot.key_lanes = key_lanes[k];
            slot.cmd_lanes = command_lanes[k];
            slot.lanes = lanes[k];
            slot.terrain = (const uint8_t*)ops[7];
            slot.table = (const int32_t*)ops[8];
            slot.timings = (const int32_t*)ops[9];
            slot.max_cycles = 0x7fffffff;
            slot.first_block = (uint32_t)blocks;
            blocks += (lanes[k] + sh.wpb - 1) / sh.wpb;
            if (blocks > 0x7fffffff) return fail(NANORTS_INVALID_ARGUMENT, std::string(target) + ": too many lanes for one launch");
        }
        if (blocks == 0) continue;
        hipLaunchKernelGGL(k_step_groups, dim3((unsigned)blocks), dim3((unsigned)(kWave * sh.wpb)), (size_t)sh.lds, st,
                           args);
        const hipError_t err = hipGetLastError();
        if (err != hipSuccess) return fail(NANORTS_INTERNAL, std::string("kernel launch failed: ") + hipGetErrorString(err));
    }
    return NANORTS_OK;
}

int nanorts_amd_step_groups(void* stream, int32_t groups, const nanorts_game* const* games, const nanorts_state* states,
                        const int64_t* lanes, const uint32_t* const* keys, const int64_t* key_lanes,
                        const nanorts_commands* commands, const nanorts_step_results* results) {
    if (groups < 1 || groups > 16) return fail(NANORTS_INVALID_ARGUMENT, "groups must be in [1, 16]");
    if (!games || !states || !lanes || !keys || !key_lanes || !commands || !results)
        return fail(NANORTS_INVALID_ARGUMENT, "NULL argument");
    std::vector<Shape> shapes((size_t)groups);
    for (int32_t i = 0; i < groups; ++i) {
        std::string why;
        if (!games[i] || !shape_for(games[i], &shapes[(size_t)i], &why))
            return fail(NANORTS_INVALID_ARGUMENT, "group " + std::to_string(i) + ": " + why);
        const KGame& a = shapes[0].g;
        const KGame& b = shapes[(size_t)i].g;
        if (a.H != b.H || a.W != b.W || a.N != b.N || a.C != b.C || a.T != b.T || a.O != b.O ||
            a.strategy != b.strategy || std::memcmp(a.tab, b.tab, sizeof(a.tab)) != 0)
            return fail(NANORTS_INVALID_ARGUMENT,
                        "nanorts_amd_step_groups: group " + std::to_string(i) + "'s bucket or unit table disagrees with group 0's");
        if (!state_complete(states[i])) return fail(NANORTS_INVALID_ARGUMENT, "a State leaf pointer is NULL");
        const nanorts_commands& c = commands[i];
        if (!c.kind || !c.direction || !c.none_duration || !c.target_cell || !c.produced_type || !c.request_order)
            return fail(NANORTS_INVALID_ARGUMENT, "a Commands field pointer is NULL");
        if (lanes[i] < 0) return fail(NANORTS_INVALID_ARGUMENT, "lanes must be >= 0");
        if (lanes[i] > 0 && (!keys[i] || (key_lanes[i] != 1 && key_lanes[i] != lanes[i])))
            return fail(NANORTS_INVALID_ARGUMENT, "each group's key must be [1][2] or [lanes][2]");
    }
    const Shape& sh = shapes[0];
    for (int32_t c0 = 0; c0 < groups; c0 += kGroupsPerLaunch) {
        GroupsArgs args;
        std::memset(&args, 0, sizeof(args));
        args.g = sh.g;
        int64_t blocks = 0;
        for (int32_t i = c0; i < groups && i < c0 + kGroupsPerLaunch; ++i) {
            if (lanes[i] == 0) continue;
            GroupSlot& s = args.slot[args.count++];
            s.s = states[i];
            s.c = commands[i];
            s.r = results[i];
            s.key = keys[i];
            s.key_lanes = key_lanes[i];
            s.cmd_lanes = lanes[i];
            s.lanes = lanes[i];
            s.terrain = games[i]->terrain;
            s.max_cycles = games[i]->max_cycles;
            s.first_block = (uint32_t)blocks;
            blocks += (lanes[i] + sh.wpb - 1) / sh.wpb;
            if (blocks > 0x7fffffff) return fail(NANORTS_INVALID_ARGUMENT, "too many lanes for one launch");
        }
        if (blocks == 0) continue;
        hipLaunchKernelGGL(k_step_groups, dim3((unsigned)blocks), dim3((unsigned)(kWave * sh.wpb)), (size_t)sh.lds,
                           (hipStream_t)stream, args);
        const hipError_t err = hipGetLastError();
        if (err != hipSuccess) return fail(NANORTS_INTERNAL, std::string("kernel launch failed: ") + hipGetErrorString(err));
    }
    return NANORTS_OK;
}

int nanorts_amd_legality_ffi(void* stream, const void* const* operands, void* result, int32_t words, int64_t lanes,
                             int32_t height, int32_t width, int32_t entities, int32_t capacity, int32_t types,
                             int32_t offsets) {
    if (!operands || !result) return fail(NANORTS_INVALID_ARGUMENT, "nanorts_amd_legality_ffi: operands or result is NULL");
    for (int i = 0; i < 9; ++i)
        if (!operands[i])
            return fail(NANORTS_INVALID_ARGUMENT, "nanorts_amd_legality_ffi: operand " + std::to_string(i) + " is NULL");
    if (lanes < 0) return fail(NANORTS_INVALID_ARGUMENT, "nanorts_amd_legality_ffi: lanes is negative");
    nanorts_game game;
    std::memset(&game, 0, sizeof(game));
    game.height = height;
    game.width = width;
    game.cells = height * width;
    game.capacity = capacity;
    game.neutral = entities - 2 * capacity;
    game.entities = entities;
    game.types = types;
    game.offsets = offsets;
    game.max_cycles = 0x7fffffff;
    game.terrain = (const uint8_t*)operands[7];
    NR_READER_SHAPE(&game, true)
    sh.g.ref_table = (const int32_t*)operands[8];
    nanorts_state s;
    std::memset(&s, 0, sizeof(s));
    s.birth = (int32_t*)operands[0];
    s.unit_type = (int8_t*)operands[1];
    s.owner = (int8_t*)operands[2];
    s.carried_resources = (int32_t*)operands[3];
    s.cell = (int16_t*)operands[4];
    s.entity_at = (int16_t*)operands[5];
    s.player_resources = (int32_t*)operands[6];
    if (words) return launch(k_legality_operands, sh, lanes, (hipStream_t)stream, s, (uint8_t*)nullptr, (uint32_t*)result);
    return launch(k_legality_operands, sh, lanes, (hipStream_t)stream, s, (uint8_t*)result, (uint32_t*)nullptr);
}

int nanorts_amd_visible_cells_ffi(void* stream, const int32_t* birth, int64_t birth_lanes, const int8_t* unit_type,
                                  int64_t unit_type_lanes, const void* cell, int32_t cell_bytes, int64_t cell_lanes,
                                  int64_t slots, const int32_t* radius, int64_t types, uint8_t* out, int64_t lanes,
                                  int64_t first, int64_t count, int32_t width, int32_t height) {
    const std::string who = "nanorts_amd_visible_cells_ffi: ";
    if (!birth || !unit_type || !cell || !radius || !out) return fail(NANORTS_INVALID_ARGUMENT, who + "a buffer is NULL");
    if (cell_bytes != 1 && cell_bytes != 2 && cell_bytes != 4)
        return fail(NANORTS_INVALID_ARGUMENT, who + "cell elements are 1, 2 or 4 bytes");
    const int64_t cells = (int64_t)width * height;
    if (width <= 0 || height <= 0 || cells > 48 * 1024)
        return fail(NANORTS_INVALID_ARGUMENT, who + "the board is 1 to 48K cells");
    if (lanes < 0) return fail(NANORTS_INVALID_ARGUMENT, who + "lanes is negative");
    if (lanes == 0) return NANORTS_OK;
    const auto shared_or_per_lane = [lanes](int64_t n) { return n == 1 || n == lanes; };
    if (!shared_or_per_lane(birth_lanes) || !shared_or_per_lane(unit_type_lanes) || !shared_or_per_lane(cell_lanes))
        return fail(NANORTS_INVALID_ARGUMENT, who + "each per-slot leaf holds a row per lane or one shared row");
    if (first < 0 || count < 0 || first + count > slots || types <= 0)
        return fail(NANORTS_INVALID_ARGUMENT, who + "the block lies inside the per-slot rows and the radius table is not empty");
    VisibleArgs a;
    a.birth = birth;
    a.unit_type = unit_type;
    a.cell = (const uint8_t*)cell;
    a.radius = radius;
    a.out = out;
    a.birth_stride = birth_lanes == 1 ? 0 : slots;
    a.type_stride = unit_type_lanes == 1 ? 0 : slots;
    a.cell_stride = cell_lanes == 1 ? 0 : slots;
    a.types = types;
    a.lanes = lanes;
    a.first = first;
    a.count = count;
    a.width = width;
    a.height = height;
    a.cell_bytes = cell_bytes;
    a.words = (int32_t)((cells + 31) / 32);
    const int32_t wpb = 4;
    const int64_t blocks = (lanes + wpb - 1) / wpb;
    if (blocks > 0x7fffffff) return fail(NANORTS_INVALID_ARGUMENT, who + "too many lanes for one launch");
    hipLaunchKernelGGL(k_visible_block, dim3((unsigned)blocks), dim3(kWave * wpb), (size_t)(wpb * a.words * 4),
                       (hipStream_t)stream, a);
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) return fail(NANORTS_INTERNAL, std::string("kernel launch failed: ") + hipGetErrorString(err));
    return NANORTS_OK;
}

int nanorts_amd_reset_rows_ffi(void* stream, const uint8_t* done, int64_t lanes, int32_t leaves,
                               const void* const* reset_rows, const int64_t* reset_lanes, const void* const* ending,
                               void* const* results, const int64_t* row_bytes) {
    const std::string who = "nanorts_amd_reset_rows_ffi: ";
    if (leaves < 0 || leaves > kMaxResetLeaves)
        return fail(NANORTS_INVALID_ARGUMENT, who + "leaves is 0 to " + std::to_string(kMaxResetLeaves));
    if (lanes < 0) return fail(NANORTS_INVALID_ARGUMENT, who + "lanes is negative");
    if (leaves == 0 || lanes == 0) return NANORTS_OK;
    if (!done || !reset_rows || !reset_lanes || !ending || !results || !row_bytes)
        return fail(NANORTS_INVALID_ARGUMENT, who + "an array is NULL");
    ResetArgs a;
    std::memset(&a, 0, sizeof(a));
    a.done = done;
    a.lanes = lanes;
    a.leaves = leaves;
    for (int32_t k = 0; k < leaves; ++k) {
        if (!reset_rows[k] || !ending[k] || !results[k])
            return fail(NANORTS_INVALID_ARGUMENT, who + "leaf " + std::to_string(k) + " has a NULL buffer");
        if (row_bytes[k] < 0) return fail(NANORTS_INVALID_ARGUMENT, who + "a row has negative bytes");
        if (reset_lanes[k] != 1 && reset_lanes[k] != lanes)
            return fail(NANORTS_INVALID_ARGUMENT, who + "a reset leaf holds one row per lane or one shared row");
        a.reset[k] = (const uint8_t*)reset_rows[k];
        a.reset_stride[k] = reset_lanes[k] == 1 ? 0 : row_bytes[k];
        a.ending[k] = (const uint8_t*)ending[k];
        a.result[k] = (uint8_t*)results[k];
        a.row_bytes[k] = row_bytes[k];
    }
    const int32_t wpb = 4;
    const int64_t blocks = (lanes + wpb - 1) / wpb;
    if (blocks > 0x7fffffff) return fail(NANORTS_INVALID_ARGUMENT, who + "too many lanes for one launch");
    hipLaunchKernelGGL(k_reset_rows, dim3((unsigned)blocks, (unsigned)leaves), dim3(kWave * wpb), 0,
                       (hipStream_t)stream, a);
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) return fail(NANORTS_INTERNAL, std::string("kernel launch failed: ") + hipGetErrorString(err));
    return NANORTS_OK;
}

int nanorts_amd_legality(void* stream, const nanorts_game* game, nanorts_state state, int64_t lanes, uint8_t* rows) {
    NR_READER_SHAPE(game, true)
    NR_STATE(state)
    if (!rows) return fail(NANORTS_INVALID_ARGUMENT, "rows is NULL");
    return launch(k_legality, sh, lanes, (hipStream_t)stream, state, 0, rows, (uint32_t*)nullptr);
}

int nanorts_amd_legality_words(void* stream, const nanorts_game* game, nanorts_state state, int64_t lanes,
                           uint32_t* words) {
    NR_READER_SHAPE(game, true)
    NR_STATE(state)
    if (!words) return fail(NANORTS_INVALID_ARGUMENT, "words is NULL");
    return launch(k_legality, sh, lanes, (hipStream_t)stream, state, 0, (uint8_t*)nullptr, words);
}

int nanorts_amd_avail_actions(void* stream, const nanorts_game* game, nanorts_state state, int64_t lanes, uint8_t* rows,
                          uint32_t* words) {
    NR_READER_SHAPE(game, true)
    NR_STATE(state)
    if (!rows && !words) return fail(NANORTS_INVALID_ARGUMENT, "rows and words are both NULL");
    return launch(k_legality, sh, lanes, (hipStream_t)stream, state, 1, rows, words);
}

int nanorts_amd_visible_cells(void* stream, const nanorts_game* game, nanorts_state state, int64_t lanes, int32_t observer,
                          uint8_t* cells) {
    NR_SHAPE(game)
    NR_STATE(state)
    if (observer < 0 || observer > 1) return fail(NANORTS_INVALID_ARGUMENT, "observer must be 0 or 1");
    if (!cells) return fail(NANORTS_INVALID_ARGUMENT, "cells is NULL");
    return launch(k_visible, sh, lanes, (hipStream_t)stream, state, observer, cells);
}

int nanorts_amd_observe(void* stream, const nanorts_game* game, nanorts_state state, int64_t lanes, int32_t partial,
                    uint8_t* feature_maps, int32_t* scalars) {
    NR_SHAPE(game)
    NR_STATE(state)
    if (!feature_maps && !scalars) return fail(NANORTS_INVALID_ARGUMENT, "no output requested");
    return launch(k_observe, sh, lanes, (hipStream_t)stream, state, partial, feature_maps, scalars);
}

int nanorts_amd_pixels(void* stream, const nanorts_game* game, nanorts_state state, int64_t lanes, int32_t partial,
                   const uint8_t* tiles, uint8_t* image, int32_t* scalars) {
    NR_SHAPE(game)
    NR_STATE(state)
    if (!tiles || !image) return fail(NANORTS_INVALID_ARGUMENT, "tiles and image are required");
    return launch(k_pixels, sh, lanes, (hipStream_t)stream, state, partial, tiles, image, scalars);
}

int nanorts_amd_pixels_from_maps(void* stream, const nanorts_game* game, int64_t images, const uint8_t* feature_maps,
                             const uint8_t* tiles, uint8_t* image) {
    NR_SHAPE(game)
    (void)sh;
    if (images < 0) return fail(NANORTS_INVALID_ARGUMENT, "images must be >= 0");
    if (images == 0) return NANORTS_OK;
    if (!feature_maps || !tiles || !image) return fail(NANORTS_INVALID_ARGUMENT, "feature_maps, tiles and image are required");
    if ((((uintptr_t)tiles) & 15u) != 0 || (((uintptr_t)image) & 15u) != 0)
        return fail(NANORTS_INVALID_ARGUMENT, "tiles and image must be 16-byte aligned");
    const int64_t rows = (int64_t)game->height * 16 * game->width;  // cell rows of one image
    const int64_t per_block = kPixelWaves * kWave;
    const int64_t zs = (images + 65534) / 65535;
    if (zs > 65535) return fail(NANORTS_INVALID_ARGUMENT, "too many images for one launch");
    int32_t wshift = -1;
    for (int32_t b = 0; b < 16; ++b)
        if ((1 << b) == game->width) wshift = b;
    const dim3 grid((unsigned)((rows + per_block - 1) / per_block), (unsigned)(images < 65535 ? images : 65535),
                    (unsigned)zs);
    hipLaunchKernelGGL(k_pixels_from_maps, grid, dim3((unsigned)per_block), 0, (hipStream_t)stream, game->height,
                       game->width, game->types, wshift, images, feature_maps, tiles, image);
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) return fail(NANORTS_INTERNAL, std::string("k_pixels_from_maps launch: ") + hipGetErrorString(err));
    return NANORTS_OK;
}

int nanorts_amd_reset_where_done(void* stream, const nanorts_game* game, nanorts_state state, int64_t lanes,
                             const uint8_t* done) {
    NR_SHAPE(game)
    NR_STATE(state)
    if (!done) return fail(NANORTS_INVALID_ARGUMENT, "done is NULL");
    if (!state_complete(game->initial)) return fail(NANORTS_INVALID_ARGUMENT, "game->initial is incomplete");
    return launch(k_reset, sh, lanes, (hipStream_t)stream, state, done);
}

int nanorts_amd_env_step(void* stream, const nanorts_game* game, nanorts_state state, int64_t lanes, const int32_t* actions,
                     int32_t partial, nanorts_env_results results) {
    NR_SHAPE(game)
    NR_STATE(state)
    if (!actions) return fail(NANORTS_INVALID_ARGUMENT, "actions is NULL");
    if (!state.environment_root || !state.episode_index)
        return fail(NANORTS_INVALID_ARGUMENT, "env.step needs environment_root and episode_index");
    if (!state_complete(game->initial)) return fail(NANORTS_INVALID_ARGUMENT, "game->initial is incomplete");
    return launch(k_env_step, sh, lanes, (hipStream_t)stream, state, actions, partial, results, 1);
}

int nanorts_amd_env_transition(void* stream, const nanorts_game* game, nanorts_state state, int64_t lanes,
                           const int32_t* actions, int32_t partial, nanorts_env_results results) {
    NR_SHAPE(game)
    NR_STATE(state)
    if (!actions) return fail(NANORTS_INVALID_ARGUMENT, "actions is NULL");
    if (!state.environment_root || !state.episode_index)
        return fail(NANORTS_INVALID_ARGUMENT, "env.step_env needs environment_root and episode_index");
    return launch(k_env_step, sh, lanes, (hipStream_t)stream, state, actions, partial, results, 0);
}

int nanorts_amd_decode_actions(void* stream, const nanorts_game* game, nanorts_state state, int64_t lanes,
                           const int32_t* actions, nanorts_command_buffers commands, uint32_t* episode_keys) {
    NR_SHAPE(game)
    NR_STATE(state)
    if (!actions) return fail(NANORTS_INVALID_ARGUMENT, "actions is NULL");
    if (!commands.kind || !commands.direction || !commands.none_duration || !commands.target_cell ||
        !commands.produced_type || !commands.request_order)
        return fail(NANORTS_INVALID_ARGUMENT, "a Commands buffer pointer is NULL");
    if (episode_keys && (!state.environment_root || !state.episode_index))
        return fail(NANORTS_INVALID_ARGUMENT, "episode keys need environment_root and episode_index");
    return launch(k_decode_actions, sh, lanes, (hipStream_t)stream, state, actions, commands, episode_keys);
}

static bool bot_args(const nanorts_game* game, Shape* sh, BotArgs* a, int32_t strategy, int32_t trained_type,
                     const nanorts_abstract_actions& carry, std::string* why, bool first_pass = false) {
    if (strategy != NANORTS_WORKER_RUSH && strategy != NANORTS_BARRACKS_RUSH) {
        *why = "strategy must be NANORTS_WORKER_RUSH or NANORTS_BARRACKS_RUSH";
        return false;
    }
    if (!carry.kind || !carry.unit_birth || !carry.order || !carry.target || !carry.target_birth || !carry.base ||
        !carry.base_birth || !carry.cell || !carry.unit_type || !carry.trained || !carry.next_order) {
        *why = "a carry (AbstractActions) pointer is NULL";
        return false;
    }
    if (!shape_for_bots(game, sh, &a->y, why, first_pass)) return false;
    int32_t* rows[9] = {carry.kind, carry.unit_birth, carry.order, carry.target, carry.target_birth,
                        carry.base, carry.base_birth, carry.cell, carry.unit_type};
    for (int f = 0; f < 9; ++f) a->carry.row[f] = rows[f];
    a->carry.trained = carry.trained;
    a->carry.next_order = carry.next_order;
    a->strategy = strategy;
    a->trained = trained_type;
    return true;
}

int nanorts_amd_abstraction_act(void* stream, const nanorts_game* game, nanorts_state state, int64_t lanes,
                            int32_t strategy, int32_t trained_type, const int32_t* player, int64_t player_lanes,
                            nanorts_abstract_actions carry, int32_t* commands) {
    NR_STATE(state)
    if (!player || (player_lanes != 1 && player_lanes != lanes))
        return fail(NANORTS_INVALID_ARGUMENT, "player must be [1] or [lanes]");
    if (!commands) return fail(NANORTS_INVALID_ARGUMENT, "commands is NULL");
    Shape sh;
    BotArgs a;
    std::string why;
    if (!bot_args(game, &sh, &a, strategy, trained_type, carry, &why)) return fail(NANORTS_INVALID_ARGUMENT, why);
    return launch(k_abstraction_act, sh, lanes, (hipStream_t)stream, state, a, player, player_lanes, commands);
}

int nanorts_amd_abstraction_act_ffi(void* stream, const void* const* operands, const int64_t* operand_lanes,
                                    void* const* results, int64_t lanes, int32_t height, int32_t width,
                                    int32_t entities, int32_t capacity, int32_t types, int64_t strategy,
                                    int64_t trained) {
    const std::string target = "nanorts_amd_abstraction_act_ffi";
    if (!operands || !operand_lanes || !results) return fail(NANORTS_INVALID_ARGUMENT, target + ": NULL argument");
    for (int i = 0; i < 24; ++i)
        if (!operands[i]) return fail(NANORTS_INVALID_ARGUMENT, target + ": operand " + std::to_string(i) + " is NULL");
    for (int i = 0; i < 12; ++i)
        if (!results[i]) return fail(NANORTS_INVALID_ARGUMENT, target + ": result " + std::to_string(i) + " is NULL");
    if (lanes < 0) return fail(NANORTS_INVALID_ARGUMENT, target + ": lanes is negative");
    for (int i = 0; i < 13; ++i)
        if (operand_lanes[i] != 1 && operand_lanes[i] != lanes)
            return fail(NANORTS_INVALID_ARGUMENT, target + ": operand " + std::to_string(i) +
                                                      " is not one row per lane or one shared row");
    if (operand_lanes[10] != 1 || operand_lanes[11] != 1)
        return fail(NANORTS_INVALID_ARGUMENT, target + ": the terrain and the unit table must be one shared row");
    if (strategy == 2 || strategy == 3)
        return fail(NANORTS_INVALID_ARGUMENT, target + ": the defense strategies (2, 3) are not built; "
                                                       "0 (worker rush) and 1 (barracks rush) are");
    if (strategy != NANORTS_WORKER_RUSH && strategy != NANORTS_BARRACKS_RUSH)
        return fail(NANORTS_INVALID_ARGUMENT, target + ": strategy must be 0 (worker rush) or 1 (barracks rush)");
    if (types <= 3 || (strategy == NANORTS_BARRACKS_RUSH && (trained < 0 || trained >= types)))
        return fail(NANORTS_INVALID_ARGUMENT, target + ": the table must hold the Worker type and the trained type");
    if (entities - 2 * capacity < 0 || capacity <= 0)
        return fail(NANORTS_INVALID_ARGUMENT, target + ": entities must hold both players' capacity");
    const hipStream_t st = (hipStream_t)stream;
    // the carry in place: an unaliased result is first filled from its operand
    const int64_t C = capacity;
    const int64_t carry_bytes[11] = {C * 4, C * 4, C * 4, C * 4, C * 4, C * 4, C * 4, C * 4, C * 4, C, 4};
    for (int i = 0; i < 11; ++i)
        if (results[i] != operands[13 + i] && lanes > 0 &&
            hipMemcpyAsync(results[i], operands[13 + i], (size_t)(carry_bytes[i] * lanes), hipMemcpyDeviceToDevice, st) !=
                hipSuccess)
            return fail(NANORTS_INTERNAL, target + ": copying an unaliased carry leaf failed");
    nanorts_game game;
    std::memset(&game, 0, sizeof(game));
    game.height = height;
    game.width = width;
    game.cells = height * width;
    game.neutral = entities - 2 * capacity;
    game.capacity = capacity;
    game.entities = entities;
    game.types = types;
    game.offsets = 1;  // the act reads no legality rows
    game.max_cycles = 0x7fffffff;
    game.terrain = (const uint8_t*)operands[10];
    Shape sh;
    BotArgs a;
    std::string why;
    if (!shape_for_bots(&game, &sh, &a.y, &why)) return fail(NANORTS_INVALID_ARGUMENT, target + ": " + why);
    for (int f = 0; f < 9; ++f) a.carry.row[f] = (int32_t*)results[f];
    a.carry.trained = (uint8_t*)results[9];
    a.carry.next_order = (int32_t*)results[10];
    a.strategy = (int32_t)strategy;
    a.trained = (int32_t)trained;
    nanorts_state s;
    std::memset(&s, 0, sizeof(s));
    s.birth = (int32_t*)operands[0];
    s.unit_type = (int8_t*)operands[1];
    s.owner = (int8_t*)operands[2];
    s.cell = (int16_t*)operands[3];
    s.carried_resources = (int32_t*)operands[4];
    s.pending_kind = (int8_t*)operands[5];
    s.pending_direction = (int8_t*)operands[6];
    s.pending_produced_type = (int8_t*)operands[7];
    s.entity_at = (int16_t*)operands[8];
    s.player_resources = (int32_t*)operands[9];
    const uint32_t flags[10] = {LD_BIRTH, LD_UTYPE, LD_OWNER, LD_CELL, LD_CARRIED,
                                LD_PKIND, LD_PDIR, LD_PPTYPE, LD_ENTITY, LD_SCALARS};
    uint32_t shared = 0u;
    for (int i = 0; i < 10; ++i)
        if (operand_lanes[i] == 1) shared |= flags[i];
    return launch(k_abstraction_act_operands, sh, lanes, st, s, (const int32_t*)operands[11], shared, a,
                  (const int32_t*)operands[12], operand_lanes[12], (int32_t*)results[11]);
}

// Waves per workgroup and per-wave LDS bytes of the A* kernels on a W x H
// board (at most 8192 cells).
static bool astar_shape(const std::string& target, int32_t width, int32_t height, int64_t lanes, AstarArgs* a) {
    if (width <= 0 || height <= 0 || (int64_t)width * height > 8192)
        return fail(NANORTS_INVALID_ARGUMENT, target + ": the board must hold 1 to 8192 cells"), false;
    if (lanes < 0) return fail(NANORTS_INVALID_ARGUMENT, target + ": lanes is negative"), false;
    const int32_t cells = width * height;
    a->W = width;
    a->H = height;
    a->lanes = lanes;
    a->region = ((cells + 15) & ~15) + 2 * 2 * ((cells + 7) & ~7) + ((cells + 15) & ~15);
    a->waves = 4;
    while (a->waves > 1 && a->waves * a->region > 65536) --a->waves;
    return true;
}

static int launch_astar(void (*kernel)(AstarArgs), const AstarArgs& a, hipStream_t stream) {
    if (a.lanes == 0) return NANORTS_OK;
    const int64_t blocks = (a.lanes + a.waves - 1) / a.waves;
    if (blocks > 0x7fffffff) return fail(NANORTS_INVALID_ARGUMENT, "too many lanes for one launch");
    hipLaunchKernelGGL(kernel, dim3((unsigned)blocks), dim3((unsigned)(kWave * a.waves)), (size_t)(a.waves * a.region),
                       stream, a);
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) return fail(NANORTS_INTERNAL, std::string("kernel launch failed: ") + hipGetErrorString(err));
    return NANORTS_OK;
}

static int64_t row_stride(int64_t extent, int64_t lanes, int64_t row) { return extent == 1 && lanes != 1 ? 0 : row; }

int nanorts_amd_astar_search_ffi(void* stream, const uint8_t* free, int64_t free_lanes, const int32_t* start,
                                 int64_t start_lanes, const int32_t* target, int64_t target_lanes, const int32_t* range,
                                 int64_t range_lanes, int32_t width, int32_t height, int32_t* out, int64_t lanes) {
    const std::string name = "nanorts_amd_astar_search_ffi";
    AstarArgs a;
    std::memset(&a, 0, sizeof(a));
    if (!astar_shape(name, width, height, lanes, &a)) return NANORTS_INVALID_ARGUMENT;
    if (!free || !start || !target || !range || !out) return fail(NANORTS_INVALID_ARGUMENT, name + ": NULL argument");
    const int64_t extents[4] = {free_lanes, start_lanes, target_lanes, range_lanes};
    for (int i = 0; i < 4; ++i)
        if (extents[i] != 1 && extents[i] != lanes)
            return fail(NANORTS_INVALID_ARGUMENT, name + ": operand " + std::to_string(i) +
                                                      " is not one row per lane or one shared row");
    a.free = free;
    a.start = start;
    a.target = target;
    a.range = range;
    a.free_stride = row_stride(free_lanes, lanes, (int64_t)width * height);
    a.start_stride = row_stride(start_lanes, lanes, 1);
    a.target_stride = row_stride(target_lanes, lanes, 1);
    a.range_stride = row_stride(range_lanes, lanes, 1);
    a.out = out;
    return launch_astar(k_astar_search, a, (hipStream_t)stream);
}

int nanorts_amd_astar_chain_ffi(void* stream, const void* const* operands, const int64_t* operand_lanes, int32_t* out,
                                int64_t lanes, int32_t width, int32_t height, int64_t capacity, int64_t columns,
                                int64_t draw_count, int32_t drawing, const int64_t* fallback, const int64_t* blocked) {
    const std::string name = "nanorts_amd_astar_chain_ffi";
    AstarArgs a;
    std::memset(&a, 0, sizeof(a));
    if (!astar_shape(name, width, height, lanes, &a)) return NANORTS_INVALID_ARGUMENT;
    if (!operands || !operand_lanes || !out || !fallback || !blocked)
        return fail(NANORTS_INVALID_ARGUMENT, name + ": NULL argument");
    for (int i = 0; i < 9; ++i) {
        if (!operands[i]) return fail(NANORTS_INVALID_ARGUMENT, name + ": operand " + std::to_string(i) + " is NULL");
        if (operand_lanes[i] != 1 && operand_lanes[i] != lanes)
            return fail(NANORTS_INVALID_ARGUMENT, name + ": operand " + std::to_string(i) +
                                                      " is not one row per lane or one shared row");
    }
    if (capacity < 0 || capacity > (1 << 20) || columns < 5 || draw_count < 0 || (drawing && draw_count == 0))
        return fail(NANORTS_INVALID_ARGUMENT, name + ": each row holds the five search columns, and a drawing pass "
                                                     "has draws");
    for (int k = 0; k < 3; ++k)
        if (fallback[k] < 5 || fallback[k] >= columns || blocked[k] < 5 || blocked[k] >= columns)
            return fail(NANORTS_INVALID_ARGUMENT, name + ": the desires' kind, claim and cost columns lie past the "
                                                         "search columns, within the row");
    const int64_t cells = (int64_t)width * height;
    a.free = (const uint8_t*)operands[0];
    a.claimed = (const uint8_t*)operands[1];
    a.rows = (const int32_t*)operands[2];
    a.queue = (const int32_t*)operands[3];
    a.count = (const int32_t*)operands[4];
    a.moves = (const uint8_t*)operands[5];
    a.reserved = (const int32_t*)operands[6];
    a.balance = (const int32_t*)operands[7];
    a.draws = (const int32_t*)operands[8];
    a.free_stride = row_stride(operand_lanes[0], lanes, cells);
    a.claimed_stride = row_stride(operand_lanes[1], lanes, cells);
    a.rows_stride = row_stride(operand_lanes[2], lanes, capacity * columns);
    a.queue_stride = row_stride(operand_lanes[3], lanes, capacity);
    a.count_stride = row_stride(operand_lanes[4], lanes, 1);
    a.moves_stride = row_stride(operand_lanes[5], lanes, 1);
    a.reserved_stride = row_stride(operand_lanes[6], lanes, 1);
    a.balance_stride = row_stride(operand_lanes[7], lanes, 1);
    a.draws_stride = row_stride(operand_lanes[8], lanes, draw_count);
    a.capacity = capacity;
    a.columns = columns;
    a.draw_count = draw_count;
    a.drawing = drawing ? 1 : 0;
    for (int k = 0; k < 3; ++k) {
        a.fallback[k] = (int32_t)fallback[k];
        a.blocked[k] = (int32_t)blocked[k];
    }
    a.out = out;
    return launch_astar(k_astar_chain, a, (hipStream_t)stream);
}

static int seat_step(void* stream, const nanorts_game* game, nanorts_state state, int64_t lanes, int32_t strategy,
                     int32_t trained_type, int32_t learner, int32_t* seats, int32_t draw,
                     nanorts_abstract_actions carry, const int32_t* actions, int32_t partial,
                     nanorts_env_results results) {
    if (!actions) return fail(NANORTS_INVALID_ARGUMENT, "actions is NULL");
    if (!state.environment_root || !state.episode_index)
        return fail(NANORTS_INVALID_ARGUMENT, "the seat step needs environment_root and episode_index");
    if (!state_complete(game->initial)) return fail(NANORTS_INVALID_ARGUMENT, "game->initial is incomplete");
    Shape sh;
    BotArgs a;
    std::string why;
    if (!bot_args(game, &sh, &a, strategy, trained_type, carry, &why)) return fail(NANORTS_INVALID_ARGUMENT, why);
    return launch(k_seat_step, sh, lanes, (hipStream_t)stream, state, a, learner, seats, draw, actions, partial,
                  results);
}

int nanorts_amd_seat_step(void* stream, const nanorts_game* game, nanorts_state state, int64_t lanes, int32_t strategy,
                      int32_t trained_type, int32_t learner, nanorts_abstract_actions carry, const int32_t* actions,
                      int32_t partial, nanorts_env_results results) {
    NR_STATE(state)
    if (learner != 0 && learner != 1) return fail(NANORTS_INVALID_ARGUMENT, "learner must be 0 or 1");
    return seat_step(stream, game, state, lanes, strategy, trained_type, learner, nullptr, 0, carry, actions, partial,
                     results);
}

int nanorts_amd_seat_step_lanes(void* stream, const nanorts_game* game, nanorts_state state, int64_t lanes,
                            int32_t strategy, int32_t trained_type, int32_t* seats, int32_t draw,
                            nanorts_abstract_actions carry, const int32_t* actions, int32_t partial,
                            nanorts_env_results results) {
    NR_STATE(state)
    if (!seats) return fail(NANORTS_INVALID_ARGUMENT, "seats is NULL");
    return seat_step(stream, game, state, lanes, strategy, trained_type, 0, seats, draw != 0, carry, actions, partial,
                     results);
}

int nanorts_amd_episode_seats(void* stream, const uint32_t* environment_root, const uint32_t* episode_index, int64_t lanes,
                          int32_t* seats) {
    if (!environment_root || !episode_index || !seats) return fail(NANORTS_INVALID_ARGUMENT, "NULL argument");
    if (lanes < 0) return fail(NANORTS_INVALID_ARGUMENT, "lanes must be >= 0");
    if (lanes == 0) return NANORTS_OK;
    const int64_t blocks = (lanes + 255) / 256;
    if (blocks > 0x7fffffff) return fail(NANORTS_INVALID_ARGUMENT, "too many lanes for one launch");
    hipLaunchKernelGGL(k_episode_seats, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, lanes,
                       environment_root, episode_index, seats);
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) return fail(NANORTS_INTERNAL, std::string("kernel launch failed: ") + hipGetErrorString(err));
    return NANORTS_OK;
}

int nanorts_amd_sample_actions(void* stream, const nanorts_game* game, int64_t lanes, const uint32_t* avail_words,
                           const uint32_t* sample_key, int32_t step, int64_t env0, int32_t* actions) {
    NR_READER_SHAPE(game, false)
    if (!avail_words || !sample_key || !actions) return fail(NANORTS_INVALID_ARGUMENT, "NULL argument");
    {
        // each wave's block holds its game's action rows (k_sample)
        Shape staged = sh;
        staged.g.lay.env_bytes = align16(2 * sh.g.C * 28);
        std::string why;
        if (fit_waves(&staged, &why)) sh = staged;
    }
    return launch(k_sample, sh, lanes, (hipStream_t)stream, avail_words, sample_key[0], sample_key[1], step, env0,
                  actions);
}

int nanorts_amd_gridnet_sample_actions(void* stream, const nanorts_game* game, int64_t lanes, const uint32_t* mask,
                                   const uint32_t* sample_key, int32_t step, int64_t env0, int32_t* actions) {
    NR_READER_SHAPE(game, false)
    if (!mask || !sample_key || !actions) return fail(NANORTS_INVALID_ARGUMENT, "NULL argument");
    if (sh.g.T != 7 || sh.g.O != 49)
        return fail(NANORTS_INVALID_ARGUMENT, "the GridNet surface is pinned to 7 unit types and a 49-cell attack window");
    {
        // each wave's block holds 64 action rows (k_gridnet_sample)
        Shape staged = sh;
        staged.g.lay.env_bytes = align16(kWave * 28);
        std::string why;
        if (fit_waves(&staged, &why)) sh = staged;
    }
    return launch(k_gridnet_sample, sh, lanes, (hipStream_t)stream, mask, sample_key[0], sample_key[1], step, env0,
                  actions);
}

// The rollout's first pass for a two-pass launch: 2 two games per wave
// (`pair` shaped), 1 one game per wave (`lean`), 0 none.  Two games per wave
// where that pays (shape_for_pair); the environment variable
// NANORTS_AMD_FIRST_PASS set to "lean" or "pair" takes one game or two games
// per wave whatever the board.
static int choose_first_pass(const nanorts_game* game, const Shape& full, Shape* lean, Shape* pair) {
    std::string why;
    if (!full.g.fast_obs || !shape_for_first_pass(game, false, false, lean, &why) ||
        games_per_cu(lean->g.lay, lean->wpb, kLeanWavesPerSimd) < games_per_cu(full.g.lay, full.wpb, 4))
        return 0;
    const char* mode = std::getenv("NANORTS_AMD_FIRST_PASS");
    const bool want_lean = mode && std::strcmp(mode, "lean") == 0;
    const bool want_pair = mode && std::strcmp(mode, "pair") == 0;
    return !want_lean && shape_for_first_pass(game, true, want_pair, pair, &why) ? 2 : 1;
}

int nanorts_amd_rollout_first_pass(const nanorts_game* game) {
    NR_SHAPE(game)
    Shape lean, pair;
    return choose_first_pass(game, sh, &lean, &pair);
}

int nanorts_amd_rollout(void* stream, const nanorts_game* game, nanorts_state state, int64_t lanes,
                    const uint32_t* sample_key, int32_t step0, int32_t steps, int32_t partial, int64_t env0,
                    nanorts_rollout_results results) {
    NR_SHAPE(game)
    NR_STATE(state)
    if (!sample_key) return fail(NANORTS_INVALID_ARGUMENT, "sample_key is NULL");
    if (!state.environment_root || !state.episode_index)
        return fail(NANORTS_INVALID_ARGUMENT, "a rollout needs environment_root and episode_index");
    if (!state_complete(game->initial)) return fail(NANORTS_INVALID_ARGUMENT, "game->initial is incomplete");
    if (steps < 0) return fail(NANORTS_INVALID_ARGUMENT, "steps must be >= 0");
    if ((results.feature_maps || results.scalars) && results.depth < 1)
        return fail(NANORTS_INVALID_ARGUMENT, "depth must be >= 1");
    if (lanes <= 0 || steps == 0) return NANORTS_OK;
    const int64_t blocks = (lanes + sh.wpb - 1) / sh.wpb;
    if (blocks > 0x7fffffff) return fail(NANORTS_INVALID_ARGUMENT, "too many lanes for one launch");
    // Two passes when the caller gives the work words, the packed
    // observation applies and the first pass's block holds at least as many
    // games per CU as the full block.
    Shape lean, pair;
    const int first = results.progress != nullptr && (((uintptr_t)results.feature_maps) & 7u) == 0
                          ? choose_first_pass(game, sh, &lean, &pair)
                          : 0;
    const bool two_pass = first > 0, paired = first == 2;
    const int64_t games_per_block = paired ? 2 * pair.wpb : lean.wpb;
    const int64_t lean_blocks = two_pass ? (lanes + games_per_block - 1) / games_per_block : 0;
    if (lean_blocks > 0x7fffffff) return fail(NANORTS_INVALID_ARGUMENT, "too many lanes for one launch");
    // launches of at most kRolloutChunk cycles; the state stays in HBM
    // between them, so the result does not depend on the split
    for (int32_t t0 = 0; t0 < steps; t0 += kRolloutChunk) {
        RolloutArgs args;
        std::memset(&args, 0, sizeof(args));
        args.g = sh.g;
        args.lanes = lanes;
        args.s = state;
        args.t0 = t0;
        args.steps = steps - t0 < kRolloutChunk ? steps - t0 : kRolloutChunk;
        args.partial = partial;
        args.env0 = env0;
        args.out = results;
        for (int32_t t = 0; t < args.steps; ++t) {
            // the sampler's per-cycle key: fold_in(sample_key, step)
            uint32_t k0 = sample_key[0], k1 = sample_key[1];
            host_fold_in(k0, k1, (uint32_t)(step0 + t0 + t));
            args.step_keys[2 * t] = k0;
            args.step_keys[2 * t + 1] = k1;
        }
        if (paired) {
            args.g = pair.g;
            hipLaunchKernelGGL(k_rollout_pair, dim3((unsigned)lean_blocks), dim3((unsigned)(kWave * pair.wpb)),
                               (size_t)pair.lds, (hipStream_t)stream, args);
            args.g = sh.g;
            args.resume = 1;
        } else if (two_pass) {
            args.g = lean.g;
            hipLaunchKernelGGL(k_rollout_lean, dim3((unsigned)lean_blocks), dim3((unsigned)(kWave * lean.wpb)),
                               (size_t)lean.lds, (hipStream_t)stream, args);
            args.g = sh.g;
            args.resume = 1;
        }
        hipLaunchKernelGGL(k_rollout, dim3((unsigned)blocks), dim3((unsigned)(kWave * sh.wpb)), (size_t)sh.lds,
                           (hipStream_t)stream, args);
        const hipError_t err = hipGetLastError();
        if (err != hipSuccess)
            return fail(NANORTS_INTERNAL, std::string("kernel launch failed: ") + hipGetErrorString(err));
    }
    return NANORTS_OK;
}

static bool gridnet_obs_valid(const nanorts_gridnet_obs& o, std::string* why) {
    if (o.planes && !(o.planes_form == 1 || (o.planes_form == 0 && (o.planes_bytes == 1 || o.planes_bytes == 4)))) {
        *why = "planes_form must be 0 (one-hot, 1 or 4 bytes) or 1 (indices)";
        return false;
    }
    if (o.action_mask && !(o.mask_form == 1 || (o.mask_form == 0 && (o.mask_bytes == 1 || o.mask_bytes == 4)))) {
        *why = "mask_form must be 0 (rows, 1 or 4 bytes) or 1 (packed words)";
        return false;
    }
    return true;
}

int nanorts_amd_gridnet_decode(void* stream, const nanorts_game* game, nanorts_state state, int64_t lanes,
                           const int32_t* actions, nanorts_command_buffers commands) {
    NR_STATE(state)
    if (!actions) return fail(NANORTS_INVALID_ARGUMENT, "actions is NULL");
    if (!commands.kind || !commands.direction || !commands.none_duration || !commands.target_cell ||
        !commands.produced_type || !commands.request_order)
        return fail(NANORTS_INVALID_ARGUMENT, "a Commands buffer pointer is NULL");
    Shape sh;
    GridLayout gy;
    std::string why;
    if (!shape_for_gridnet(game, &sh, &gy, &why)) return fail(NANORTS_INVALID_ARGUMENT, why);
    return launch(k_gridnet_decode, sh, lanes, (hipStream_t)stream, state, gy, actions, commands);
}

int nanorts_amd_gridnet_decode_ffi(void* stream, const void* const* operands, const int64_t* operand_lanes,
                                   void* const* results, int64_t lanes, int32_t height, int32_t width, int32_t neutral,
                                   int32_t capacity, int32_t types, int32_t costs, int32_t side) {
    const std::string target = "nanorts_amd_gridnet_decode_ffi";
    if (!operands || !operand_lanes || !results) return fail(NANORTS_INVALID_ARGUMENT, target + ": NULL argument");
    for (int i = 0; i < 11; ++i)
        if (!operands[i]) return fail(NANORTS_INVALID_ARGUMENT, target + ": operand " + std::to_string(i) + " is NULL");
    for (int i = 0; i < 6; ++i)
        if (!results[i]) return fail(NANORTS_INVALID_ARGUMENT, target + ": result " + std::to_string(i) + " is NULL");
    if (lanes < 0) return fail(NANORTS_INVALID_ARGUMENT, target + ": lanes is negative");
    for (int i = 0; i < 11; ++i)
        if (operand_lanes[i] != 1 && operand_lanes[i] != lanes)
            return fail(NANORTS_INVALID_ARGUMENT, target + ": operand " + std::to_string(i) +
                                                      " is not one row per lane or one shared row");
    if (operand_lanes[10] != 1) return fail(NANORTS_INVALID_ARGUMENT, target + ": unit_cost must be one shared row");
    if (costs != types)
        return fail(NANORTS_INVALID_ARGUMENT, target + ": unit_cost must hold one cost per unit type (costs = types)");
    if (side <= 0 || side % 2 == 0) return fail(NANORTS_INVALID_ARGUMENT, target + ": side must be odd and positive");
    nanorts_game game;
    std::memset(&game, 0, sizeof(game));
    game.height = height;
    game.width = width;
    game.cells = height * width;
    game.neutral = neutral;
    game.capacity = capacity;
    game.entities = neutral + 2 * capacity;
    game.types = types;
    game.offsets = side * side;
    game.max_cycles = 0x7fffffff;
    // the decode reads no terrain (no operand carries it): the shape is
    // checked with a stand-in pointer, and the kernel's header stages an
    // open board for a NULL terrain
    game.terrain = (const uint8_t*)operands[1];
    Shape sh;
    GridLayout gy;
    std::string why;
    if (!shape_for_gridnet(&game, &sh, &gy, &why)) return fail(NANORTS_INVALID_ARGUMENT, target + ": " + why);
    sh.g.terrain = nullptr;
    const int64_t C = capacity, cells = game.cells;
    GridOperands o;
    o.actions = (const int32_t*)operands[0];
    o.move = (const uint8_t*)operands[7];
    o.pdir = (const uint8_t*)operands[8];
    o.ptype = (const uint8_t*)operands[9];
    o.actions_stride = operand_lanes[0] == 1 ? 0 : 2 * cells * 7;
    o.move_stride = operand_lanes[7] == 1 ? 0 : C * 4;
    o.pdir_stride = operand_lanes[8] == 1 ? 0 : C * 4;
    o.ptype_stride = operand_lanes[9] == 1 ? 0 : C * types;
    nanorts_state s;
    std::memset(&s, 0, sizeof(s));
    s.birth = (int32_t*)operands[1];
    s.pending_kind = (int8_t*)operands[2];
    s.cell = (int16_t*)operands[3];
    s.pending_direction = (int8_t*)operands[4];
    s.pending_produced_type = (int8_t*)operands[5];
    s.player_resources = (int32_t*)operands[6];
    const uint32_t flags[6] = {LD_BIRTH, LD_PKIND, LD_CELL, LD_PDIR, LD_PPTYPE, LD_SCALARS};
    uint32_t shared = 0u;
    for (int i = 0; i < 6; ++i)
        if (operand_lanes[1 + i] == 1) shared |= flags[i];
    nanorts_command_buffers out;
    out.kind = (int32_t*)results[0];
    out.direction = (int32_t*)results[1];
    out.none_duration = (int32_t*)results[2];
    out.target_cell = (int32_t*)results[3];
    out.produced_type = (int32_t*)results[4];
    out.request_order = (int32_t*)results[5];
    return launch(k_gridnet_decode_operands, sh, lanes, (hipStream_t)stream, s, (const int32_t*)operands[10], shared,
                  gy, o, out);
}

int nanorts_amd_gridnet_observe(void* stream, const nanorts_game* game, nanorts_state state, int64_t lanes,
                            nanorts_gridnet_obs obs) {
    NR_STATE(state)
    Shape sh;
    GridLayout gy;
    std::string why;
    if (!shape_for_gridnet(game, &sh, &gy, &why) || !gridnet_obs_valid(obs, &why))
        return fail(NANORTS_INVALID_ARGUMENT, why);
    return launch(k_gridnet_observe, sh, lanes, (hipStream_t)stream, state, obs);
}

int nanorts_amd_gridnet_step(void* stream, const nanorts_game* game, nanorts_state state, int64_t lanes,
                         const int32_t* actions, nanorts_gridnet_results results) {
    NR_STATE(state)
    if (!actions) return fail(NANORTS_INVALID_ARGUMENT, "actions is NULL");
    if (!state.environment_root || !state.episode_index)
        return fail(NANORTS_INVALID_ARGUMENT, "the GridNet step needs environment_root and episode_index");
    if (!state_complete(game->initial)) return fail(NANORTS_INVALID_ARGUMENT, "game->initial is incomplete");
    Shape sh;
    GridLayout gy;
    std::string why;
    if (!shape_for_gridnet(game, &sh, &gy, &why) || !gridnet_obs_valid(results.observation, &why))
        return fail(NANORTS_INVALID_ARGUMENT, why);
    const nanorts_commands none = {};
    return launch(k_gridnet_step, sh, lanes, (hipStream_t)stream, state, gy, actions, none, 0, results);
}

int nanorts_amd_gridnet_step_against(void* stream, const nanorts_game* game, nanorts_state state, int64_t lanes,
                                 const int32_t* actions, nanorts_commands commands, nanorts_gridnet_results results) {
    NR_STATE(state)
    if (!actions) return fail(NANORTS_INVALID_ARGUMENT, "actions is NULL");
    if (!commands.kind || !commands.direction || !commands.none_duration || !commands.target_cell ||
        !commands.produced_type || !commands.request_order)
        return fail(NANORTS_INVALID_ARGUMENT, "a Commands operand is NULL");
    if (!state.environment_root || !state.episode_index)
        return fail(NANORTS_INVALID_ARGUMENT, "the GridNet step needs environment_root and episode_index");
    if (!state_complete(game->initial)) return fail(NANORTS_INVALID_ARGUMENT, "game->initial is incomplete");
    Shape sh;
    GridLayout gy;
    std::string why;
    if (!shape_for_gridnet(game, &sh, &gy, &why) || !gridnet_obs_valid(results.observation, &why))
        return fail(NANORTS_INVALID_ARGUMENT, why);
    return launch(k_gridnet_step, sh, lanes, (hipStream_t)stream, state, gy, actions, commands, 1, results);
}

// The seat rollout's first pass (k_seat_rollout_pair): the bot's layout on
// the slot-window game, two games per wave, `wpb` waves per workgroup chosen
// for the most games per CU at three waves per SIMD (the kernel's register
// bound).  False where it would hold no more games per CU than the full
// block's one-game-per-wave pass, or the board has no packed observation.
static bool seat_pair_shape(const nanorts_game* game, int32_t strategy, int32_t trained_type,
                            const nanorts_abstract_actions& carry, const Shape& full, Shape* out, BotArgs* a) {
    std::string why;
    int32_t shift = 0;
    const nanorts_game w = windowed(game, &shift);
    // (the first pass writes observations from the summary's bitmaps: no
    // observation staging in its union; its carry rows of slots and cells
    // are int16)
    if (!bot_args(&w, out, a, strategy, trained_type, carry, &why, true)) return false;
    KGame& g = out->g;
    if (!g.fast_obs || g.seen_words != 1) return false;
    g.shift = shift;
    if (shift > 0) g.nseg = 0;
    const Layout& y = g.lay;
    int best = 0, best_w = 0;
    for (int wv = 1; wv <= 4; ++wv) {
        const int32_t bytes = y.hdr_bytes + 2 * wv * y.env_bytes;
        if (bytes > lds_per_cu()) continue;
        const int32_t by_lds = lds_per_cu() / lds_granule(bytes);
        const int32_t by_waves = (4 * 3) / wv;
        const int games = (by_lds < by_waves ? by_lds : by_waves) * 2 * wv;
        if (games >= best) {
            best = games;
            best_w = wv;
        }
    }
    const int32_t full_games = games_per_cu(full.g.lay, full.wpb, 3);
    if (best_w == 0 || best <= full_games) return false;
    out->wpb = best_w;
    out->lds = y.hdr_bytes + 2 * best_w * y.env_bytes;
    return true;
}

static int seat_rollout(void* stream, const nanorts_game* game, nanorts_state state, int64_t lanes, int32_t strategy,
                        int32_t trained_type, int32_t learner, int32_t* seats, int32_t draw, int32_t* seat_record,
                        nanorts_abstract_actions carry, const uint32_t* sample_key, int32_t step0, int32_t steps,
                        int32_t partial, int64_t env0, nanorts_rollout_results results) {
    if (!sample_key) return fail(NANORTS_INVALID_ARGUMENT, "sample_key is NULL");
    if (!state.environment_root || !state.episode_index)
        return fail(NANORTS_INVALID_ARGUMENT, "a rollout needs environment_root and episode_index");
    if (!state_complete(game->initial)) return fail(NANORTS_INVALID_ARGUMENT, "game->initial is incomplete");
    if (steps < 0) return fail(NANORTS_INVALID_ARGUMENT, "steps must be >= 0");
    if ((results.feature_maps || results.scalars) && results.depth < 1)
        return fail(NANORTS_INVALID_ARGUMENT, "depth must be >= 1");
    Shape sh;
    BotArgs a;
    std::string why;
    if (!bot_args(game, &sh, &a, strategy, trained_type, carry, &why)) return fail(NANORTS_INVALID_ARGUMENT, why);
    if (lanes <= 0 || steps == 0) return NANORTS_OK;
    const int64_t blocks = (lanes + sh.wpb - 1) / sh.wpb;
    if (blocks > 0x7fffffff) return fail(NANORTS_INVALID_ARGUMENT, "too many lanes for one launch");
    // two passes when the caller gives the work words (results.progress) and
    // the first pass holds more games per CU; NANORTS_AMD_FIRST_PASS=lean
    // keeps the one pass
    Shape ps;
    BotArgs pa;
    const char* mode = std::getenv("NANORTS_AMD_FIRST_PASS");
    const bool paired = results.progress != nullptr && (((uintptr_t)results.feature_maps) & 7u) == 0 &&
                        !(mode && std::strcmp(mode, "lean") == 0) &&
                        seat_pair_shape(game, strategy, trained_type, carry, sh, &ps, &pa);
    const int64_t pair_blocks = paired ? (lanes + 2 * ps.wpb - 1) / (2 * ps.wpb) : 0;
    for (int32_t t0 = 0; t0 < steps; t0 += kRolloutChunk) {
        SeatRolloutArgs args;
        std::memset(&args, 0, sizeof(args));
        args.g = sh.g;
        args.lanes = lanes;
        args.s = state;
        args.bot = a;
        args.learner = learner;
        args.seats = seats;
        args.seat_record = seat_record;
        args.draw = draw;
        args.t0 = t0;
        args.steps = steps - t0 < kRolloutChunk ? steps - t0 : kRolloutChunk;
        args.partial = partial;
        args.env0 = env0;
        args.out = results;
        for (int32_t t = 0; t < args.steps; ++t) {
            uint32_t k0 = sample_key[0], k1 = sample_key[1];
            host_fold_in(k0, k1, (uint32_t)(step0 + t0 + t));
            args.step_keys[2 * t] = k0;
            args.step_keys[2 * t + 1] = k1;
        }
        if (paired) {
            args.g = ps.g;
            args.bot = pa;
            hipLaunchKernelGGL(k_seat_rollout_pair, dim3((unsigned)pair_blocks), dim3((unsigned)(kWave * ps.wpb)),
                               (size_t)ps.lds, (hipStream_t)stream, args);
            args.g = sh.g;
            args.bot = a;
            args.resume = 1;
        }
        hipLaunchKernelGGL(k_seat_rollout, dim3((unsigned)blocks), dim3((unsigned)(kWave * sh.wpb)), (size_t)sh.lds,
                           (hipStream_t)stream, args);
        const hipError_t err = hipGetLastError();
        if (err != hipSuccess)
            return fail(NANORTS_INTERNAL, std::string("kernel launch failed: ") + hipGetErrorString(err));
    }
    return NANORTS_OK;
}

int nanorts_amd_seat_rollout(void* stream, const nanorts_game* game, nanorts_state state, int64_t lanes, int32_t strategy,
                         int32_t trained_type, int32_t learner, nanorts_abstract_actions carry,
                         const uint32_t* sample_key, int32_t step0, int32_t steps, int32_t partial, int64_t env0,
                         nanorts_rollout_results results) {
    NR_STATE(state)
    if (learner != 0 && learner != 1) return fail(NANORTS_INVALID_ARGUMENT, "learner must be 0 or 1");
    return seat_rollout(stream, game, state, lanes, strategy, trained_type, learner, nullptr, 0, nullptr, carry,
                        sample_key, step0, steps, partial, env0, results);
}

int nanorts_amd_seat_rollout_lanes(void* stream, const nanorts_game* game, nanorts_state state, int64_t lanes,
                               int32_t strategy, int32_t trained_type, int32_t* seats, int32_t draw,
                               int32_t* seat_record, nanorts_abstract_actions carry, const uint32_t* sample_key,
                               int32_t step0, int32_t steps, int32_t partial, int64_t env0,
                               nanorts_rollout_results results) {
    NR_STATE(state)
    if (!seats) return fail(NANORTS_INVALID_ARGUMENT, "seats is NULL");
    return seat_rollout(stream, game, state, lanes, strategy, trained_type, 0, seats, draw != 0, seat_record, carry,
                        sample_key, step0, steps, partial, env0, results);
}

}  // extern "C"
