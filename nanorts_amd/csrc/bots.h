// Scripted bots of the abstraction family on one wave per game: WorkerRush
// and the barracks rush that LightRush runs (N/bots/rush.py), their
// translation into Commands (N/bots/abstraction.py with the rush kinds
// ATTACK / HARVEST / TRAIN / BUILD), and the A* search it calls
// (N/bots/pathfinding.py).
//
// The game state is the wave's LDS env block.  The bot's own per-wave region
// (after the env block) holds the carry (AbstractActions rows), the plan of
// each unit, candidate lists and the search scratch.  Decisions are per unit,
// one lane per own slot; the walk over the queued units is sequential as in
// the reference (each search sees the cells claimed before it), and each
// search runs on lane 0 over LDS stacks.
#pragma once

#include "engine.h"

namespace nr {

constexpr int32_t kLast = 0x7fffffff;
constexpr int32_t kAbNone = -1;
constexpr int32_t kAbAttack = 1;
constexpr int32_t kAbHarvest = 2;
constexpr int32_t kAbTrain = 3;
constexpr int32_t kAbBuild = 4;
constexpr int32_t kAbTrainDirection = 6;
constexpr int32_t kTypeBase = 1;
constexpr int32_t kTypeBarracks = 2;
constexpr int32_t kTypeWorker = 3;
constexpr int32_t kFillerDuration = 10;
constexpr int32_t kWorkerRush = 0;
constexpr int32_t kBarracksRush = 1;

// Offsets in the bot region of one wave (computed on the host).
struct BotLayout {
    int32_t bytes;   // region size per wave
    int32_t origin;  // region offset from the env block
    // carry rows [C]
    int32_t k_kind, k_ubirth, k_order, k_target, k_tbirth, k_base, k_bbirth, k_cell, k_utype, k_trained;
    // per unit [C]
    int32_t u_flags, u_role, u_rank, u_es, u_eb, u_goal, u_radius;
    int32_t u_fkind, u_fdir, u_ftarget, u_fptype, u_fclaimed, u_fcost;
    int32_t u_sel, u_dir, u_drank, u_queue;
    int32_t u_live, u_lbirth, u_list, u_lkey;  // live units and their births; a scratch list with keys
    // candidate slot lists [E]
    int32_t l_enemy, l_resource, l_stock;
    // search scratch [cells]
    int32_t a_below, a_mark;
    // cell bitmaps [ceil(cells / 32)] words
    int32_t m_claimed, m_free, m_used, m_kept, m_reserved;
};

// Device view of the carry (AbstractActions) of all lanes, [L][C] rows.
struct BotCarry {
    int32_t* row[9];  // kind, unit_birth, order, target, target_birth, base, base_birth, cell, unit_type
    uint8_t* trained;
    int32_t* next_order;
};

enum : int32_t { U_STANDING = 1, U_EXECUTES = 2 };
enum : int32_t { SEL_NONE = 0, SEL_FALLBACK = 1, SEL_MOVED = 2 };

struct Bot {
    AS3 uint8_t* base;
    int32_t player, block;
    int32_t n_enemy, n_resource, n_stock;
    int32_t n_live;  // own units present, listed in u_live
    int32_t next_order;
    int32_t reserved0, reserved1;  // pending production cost per player
};

template <typename T>
NR_DEV AS3 T* bv(const Bot& b, int32_t offset) {
    return (AS3 T*)(b.base + offset);
}

// The LDS offset of carry row f (1..7: unit_birth, order, target,
// target_birth, base, base_birth, cell); rows 0 (kind) and 8 (unit_type)
// are bytes.
NR_DEV int32_t carry_row32(const BotLayout& y, int f) {
    switch (f) {
        case 1: return y.k_ubirth;
        case 2: return y.k_order;
        case 3: return y.k_target;
        case 4: return y.k_tbirth;
        case 5: return y.k_base;
        case 6: return y.k_bbirth;
        default: return y.k_cell;
    }
}

// Carry rows 3, 5 and 7 (target, base, cell: slots and cells, below 2^15)
// are int16 in the half-wave teams' layout (the seat rollout's first pass,
// whose load checks that they fit), int32 otherwise.
template <int TW>
NR_DEV constexpr bool narrow_row(int f) {
    return TW != kWave && (f == 3 || f == 5 || f == 7);
}
template <int TW = kWave>
NR_DEV int32_t carry_at(const Bot& b, const BotLayout& y, int f, int32_t i) {
    if (narrow_row<TW>(f)) return bv<int16_t>(b, carry_row32(y, f))[i];
    return bv<int32_t>(b, carry_row32(y, f))[i];
}
template <int TW = kWave>
NR_DEV void carry_put(const Bot& b, const BotLayout& y, int f, int32_t i, int32_t v) {
    if (narrow_row<TW>(f)) bv<int16_t>(b, carry_row32(y, f))[i] = (int16_t)v;
    else bv<int32_t>(b, carry_row32(y, f))[i] = v;
}

template <int TW = kWave>
NR_DEV int32_t team_min(int32_t v) {
#pragma unroll
    for (int d = TW / 2; d >= 1; d >>= 1) {
        const int32_t o = __shfl_xor(v, d, TW);
        v = o < v ? o : v;
    }
    return v;
}

template <int TW = kWave>
NR_DEV int32_t team_sum(int32_t v) {
#pragma unroll
    for (int d = TW / 2; d >= 1; d >>= 1) v += __shfl_xor(v, d, TW);
    return v;
}

NR_DEV int32_t bit_of(const AS3 uint32_t* m, int32_t c) { return (int32_t)((m[c >> 5] >> (c & 31)) & 1u); }
NR_DEV void set_bit(AS3 uint32_t* m, int32_t c) { __atomic_fetch_or(&m[c >> 5], 1u << (c & 31), __ATOMIC_RELAXED); }

NR_DEV int32_t type_flag(const KGame& g, const Hdr& h, int32_t t, int32_t flag) {
    return (tabv(h, F_FLAGS, clampi(t, 0, g.T - 1)) & flag) != 0;
}

// ---------------------------------------------------------------------------
// own_units (N/bots/abstraction.py:136-160)
// ---------------------------------------------------------------------------
struct Unit {
    int32_t slot, birth, cell, type, carried;
    bool present, available;
};

NR_DEV Unit unit_at(const KGame& g, const Env& e, const Bot& b, int32_t i) {
    Unit u;
    u.slot = b.block + i;
    u.birth = e.birth[u.slot];
    u.cell = e.cell[u.slot];
    u.type = clampi(e.utype[u.slot], 0, g.T - 1);
    u.carried = e.carried[u.slot];
    u.present = u.birth != kAbsent;
    u.available = u.present && e.pkind[u.slot] == kAbsent;
    return u;
}

// Manhattan-nearest slot of a candidate list, ties by the lowest birth then
// the lowest slot (rush._closest, N/bots/rush.py:30-45).
NR_DEV void closest(const KGame& g, const Env& e, int32_t origin, const AS3 int16_t* list, int32_t n, int32_t* slot,
                    int32_t* birth) {
    const int32_t ox = floor_mod(origin, g.W), oy = floor_div(origin, g.W);
    int32_t best = kAbsent, bd = kLast, bb = kLast;
#pragma unroll 4
    for (int32_t k = 0; k < n; ++k) {
        const int32_t j = list[k];
        const int32_t c = e.cell[j];
        const int32_t d = abs(ox - cell_x(g, c)) + abs(oy - cell_y(g, c));
        const int32_t bj = e.birth[j];
        if (d < bd || (d == bd && bj < bb)) {
            bd = d;
            bb = bj;
            best = j;
        }
    }
    *slot = best;
    *birth = best == kAbsent ? kAbsent : bb;
}

// abstraction.put / _written (N/bots/abstraction.py:172-227) for unit i of
// this lane; the caller advances next_order by C + 1 once per put.
template <int TW = kWave>
NR_DEV void put_unit(const KGame& g, const Bot& b, const Unit& u, int32_t i, bool last, int32_t kind, int32_t target,
                     int32_t tbirth, int32_t base, int32_t bbirth, int32_t cell, int32_t utype, const BotLayout& y) {
    AS3 int8_t* kk = bv<int8_t>(b, y.k_kind);
    AS3 int32_t* ub = bv<int32_t>(b, y.k_ubirth);
    const bool known = kk[i] != kAbNone && ub[i] == u.birth;
    if (!known) bv<int32_t>(b, y.k_order)[i] = wadd(b.next_order, last ? g.C : (int32_t)bv<int16_t>(b, y.u_rank)[i]);
    kk[i] = (int8_t)kind;
    ub[i] = u.birth;
    carry_put<TW>(b, y, 3, i, target);
    bv<int32_t>(b, y.k_tbirth)[i] = tbirth;
    carry_put<TW>(b, y, 5, i, base);
    bv<int32_t>(b, y.k_bbirth)[i] = bbirth;
    carry_put<TW>(b, y, 7, i, cell);
    bv<int8_t>(b, y.k_utype)[i] = (int8_t)utype;
    bv<uint8_t>(b, y.k_trained)[i] = 0;
}

NR_DEV bool is_entry(const Bot& b, const BotLayout& y, int32_t i, int32_t birth, int32_t kind) {
    return bv<int8_t>(b, y.k_kind)[i] == kind && bv<int32_t>(b, y.k_ubirth)[i] == birth;
}

// ---------------------------------------------------------------------------
// Setup: units, carry, candidate lists
// ---------------------------------------------------------------------------
// With `load_carry` false the carry rows in LDS and b.next_order are the
// ones the last settle_carry left (a fused rollout keeps them there).
template <int TW = kWave>
NR_DEV void bot_begin(const KGame& g, const Hdr& h, const Env& e, Bot& b, const BotLayout& y, int64_t l,
                      const BotCarry& carry, int lane, bool load_carry = true) {
    const int32_t C = g.C;
    // live own units in slot order, with their births
    AS3 int16_t* live = bv<int16_t>(b, y.u_live);
    AS3 int32_t* lbirth = bv<int32_t>(b, y.u_lbirth);
    int32_t n = 0;
    for (int32_t i0 = 0; i0 < C; i0 += TW) {
        const int32_t i = i0 + lane;
        const int32_t bi = i < C ? e.birth[b.block + i] : kAbsent;
        const bool present = bi != kAbsent;
        const uint64_t m = tballot<TW>(present);
        if (present) {
            live[n + tcount_below<TW>(m)] = (int16_t)i;
            lbirth[n + tcount_below<TW>(m)] = bi;
        }
        n += popc(m);
    }
    b.n_live = n;
    for (int32_t i = lane; i < (load_carry ? C : 0); i += TW) {
        const int64_t at = l * C + i;
        bv<int8_t>(b, y.k_kind)[i] = (int8_t)carry.row[0][at];
#pragma unroll
        for (int f = 1; f < 8; ++f) carry_put<TW>(b, y, f, i, carry.row[f][at]);
        bv<int8_t>(b, y.k_utype)[i] = (int8_t)carry.row[8][at];
        bv<uint8_t>(b, y.k_trained)[i] = carry.trained[at] ? 1 : 0;
    }
    // a vector load on one lane: in a fused rollout this word was written by
    // the previous cycle's vector store, which the scalar cache does not see
    if (load_carry) {
        int32_t next_order = 0;
        if (lane == 0) next_order = __builtin_nontemporal_load(carry.next_order + l);
        b.next_order = tuni<TW>(next_order);
    }
    // candidate lists in slot order: enemies (abstraction.enemies), resources
    // and own stockpiles (rush.harvest_sites)
    AS3 int16_t* le = bv<int16_t>(b, y.l_enemy);
    AS3 int16_t* lr = bv<int16_t>(b, y.l_resource);
    AS3 int16_t* ls = bv<int16_t>(b, y.l_stock);
    int32_t ne = 0, nr_ = 0, ns = 0;
    for (int32_t s0 = 0; s0 < g.E; s0 += TW) {
        const int32_t s = s0 + lane;
        bool en = false, re = false, st = false;
        if (s < g.E && e.birth[s] != kAbsent) {
            const int32_t owner = e.owner[s], t = e.utype[s];
            en = owner != kAbsent && owner != b.player;
            re = type_flag(g, h, t, FL_RESOURCE);
            st = type_flag(g, h, t, FL_STOCKPILE) && owner == b.player;
        }
        const uint64_t me = tballot<TW>(en), mr = tballot<TW>(re), ms = tballot<TW>(st);
        // the lists hold what a valid state can put in them: the opponent's
        // units, neutral resources, own stockpiles
        if (en && ne + tcount_below<TW>(me) < C) le[ne + tcount_below<TW>(me)] = (int16_t)s;
        if (re && nr_ + tcount_below<TW>(mr) < g.N) lr[nr_ + tcount_below<TW>(mr)] = (int16_t)s;
        if (st && ns + tcount_below<TW>(ms) < C) ls[ns + tcount_below<TW>(ms)] = (int16_t)s;
        ne += popc(me);
        nr_ += popc(mr);
        ns += popc(ms);
    }
    b.n_enemy = ne < C ? ne : C;
    b.n_resource = nr_ < g.N ? nr_ : g.N;
    b.n_stock = ns < C ? ns : C;
    wave_sync();
    // birth rank among the present units (abstraction._rank) and the
    // nearest enemy of every live unit
    for (int32_t k = lane; k < n; k += TW) {
        const int32_t i = live[k], bi = lbirth[k];
        int32_t r = 0;
#pragma unroll 4
        for (int32_t q = 0; q < n; ++q) r += lbirth[q] < bi ? 1 : 0;
        bv<int16_t>(b, y.u_rank)[i] = (int16_t)r;
        int32_t es, eb;
        closest(g, e, e.cell[b.block + i], le, ne, &es, &eb);
        bv<int16_t>(b, y.u_es)[i] = (int16_t)es;
        bv<int32_t>(b, y.u_eb)[i] = eb;
    }
    wave_sync();
}

// ---------------------------------------------------------------------------
// Rush decisions (N/bots/rush.py)
// ---------------------------------------------------------------------------
// abstraction._building_site (N/bots/abstraction.py:247-283): the open cell
// first in the ring walk around `desired`.
template <int TW = kWave>
NR_DEV int32_t building_site(const KGame& g, const Hdr& h, const Env& e, const Bot& b, const BotLayout& y,
                             int32_t desired, int lane) {
    const AS3 uint32_t* reserved = bv<uint32_t>(b, y.m_reserved);
    const int32_t longest = g.W > g.H ? g.W : g.H;
    const int32_t x0 = floor_mod(desired, g.W), y0 = floor_div(desired, g.W);
    int32_t best = kLast, site = kAbsent;
    for (int32_t c = lane; c < g.cells; c += TW) {
        const int32_t dx = cell_x(g, c) - x0, dy = cell_y(g, c) - y0;
        const int32_t ax = abs(dx), ay = abs(dy);
        const int32_t ring = ax > ay ? ax : ay;
        if (ring == 0) continue;
        const int32_t side = dy == -ring ? 0 : (dx == ring ? 1 : (dy == ring ? 2 : 3));
        const int32_t along = ((side == 0 || side == 2) ? dx : dy) + ring;
        const int32_t visit = (ring * 4 + side) * (2 * longest + 1) + along;
        const bool open = h.terrain[c] == 0 && e.entity[c] == kAbsent && !bit_of(reserved, c);
        if (open && visit < best) {
            best = visit;
            site = c;
        }
    }
    const int32_t m = team_min<TW>(best);
    const uint64_t at = tballot<TW>(site != kAbsent && best == m);
    return at == 0ull ? kAbsent : tread<TW>(site, (int32_t)__builtin_ctzll(at));
}

// Per-unit role bits of the rush decisions (u_role, one byte per own slot).
enum : uint8_t { R_WORKER = 1, R_PICK = 2, R_IDLE = 4, R_LAST = 8 };

NR_DEV AS3 uint8_t* roles(const Bot& b, const BotLayout& y) { return bv<uint8_t>(b, y.u_role); }

// The unit of least birth among those whose role byte has any of `bits`
// (rush.first_in_unit_order, N/bots/rush.py:56-58), excluding `skip0` and
// `skip1`; -1 when there is none.
template <int TW = kWave>
NR_DEV int32_t first_of(const KGame& g, const Env& e, const Bot& b, const BotLayout& y, uint8_t bits, int32_t skip0,
                        int32_t skip1, int lane) {
    const AS3 uint8_t* r = roles(b, y);
    int32_t best = kLast, who = -1;
    for (int32_t k = lane; k < b.n_live; k += TW) {
        const int32_t i = bv<int16_t>(b, y.u_live)[k];
        if (!(r[i] & bits) || i == skip0 || i == skip1) continue;
        const int32_t bi = e.birth[b.block + i];
        if (bi < best) {
            best = bi;
            who = i;
        }
    }
    const int32_t mn = team_min<TW>(best);
    const uint64_t at = tballot<TW>(who >= 0 && best == mn);
    return at == 0ull ? -1 : tread<TW>(who, (int32_t)__builtin_ctzll(at));
}

// abstraction.build_if_not_already_building (N/bots/abstraction.py:286-297)
// for a one-unit builder (or none); marks the site in the reserved bitmap.
template <int TW = kWave>
NR_DEV void build_unless_building(const KGame& g, const Hdr& h, const Env& e, Bot& b, const BotLayout& y,
                                  int32_t builder, int32_t unit_type, int lane) {
    bool builds = false;
    if (builder >= 0) {
        const int32_t bb = e.birth[b.block + builder];
        builds = !(is_entry(b, y, builder, bb, kAbBuild) && bv<int8_t>(b, y.k_utype)[builder] == unit_type);
    }
    builds = tuni<TW>(builds ? 1 : 0) != 0;
    if (builds) {
        const int32_t site = building_site<TW>(g, h, e, b, y, e.cell[b.block + builder], lane);
        if (lane == 0) {
            const Unit u = unit_at(g, e, b, builder);
            put_unit<TW>(g, b, u, builder, false, kAbBuild, kAbsent, kAbsent, kAbsent, kAbsent, site, unit_type, y);
            if (site >= 0 && site < g.cells) set_bit(bv<uint32_t>(b, y.m_reserved), site);
        }
        wave_sync();
    }
    b.next_order = wadd(b.next_order, g.C + 1);
}

// rush.build_base (N/bots/rush.py:88-104) over the R_WORKER units: clears the
// reserved bitmap, returns the builder or -1.
template <int TW = kWave>
NR_DEV int32_t build_base(const KGame& g, const Hdr& h, const Env& e, Bot& b, const BotLayout& y, int lane) {
    AS3 uint32_t* reserved = bv<uint32_t>(b, y.m_reserved);
    for (int32_t w = lane; w < (g.cells + 31) / 32; w += TW) reserved[w] = 0u;
    bool any_base = false;
    for (int32_t k = lane; k < b.n_live; k += TW) {
        const int32_t i = bv<int16_t>(b, y.u_live)[k];
        const Unit u = unit_at(g, e, b, i);
        any_base |= u.present && u.type == kTypeBase;
    }
    any_base = tballot<TW>(any_base) != 0ull;
    const int32_t res = tuni<TW>(e.sc[S_RES0 + b.player]);
    const bool builds = !any_base && res >= tabv(h, F_COST, kTypeBase);
    const int32_t builder = builds ? first_of<TW>(g, e, b, y, R_WORKER, -1, -1, lane) : -1;
    wave_sync();
    build_unless_building<TW>(g, h, e, b, y, builder, kTypeBase, lane);
    return builder;
}

// rush._harvest (N/bots/rush.py:156-181) for the R_PICK units; marks the
// idle ones (no site to harvest) R_IDLE.
template <int TW = kWave>
NR_DEV void harvest(const KGame& g, const Env& e, Bot& b, const BotLayout& y, int lane) {
    AS3 uint8_t* r = roles(b, y);
    const AS3 int16_t* lr = bv<int16_t>(b, y.l_resource);
    const AS3 int16_t* ls = bv<int16_t>(b, y.l_stock);
    for (int32_t k = lane; k < b.n_live; k += TW) {
        const int32_t i = bv<int16_t>(b, y.u_live)[k];
        const uint8_t role = r[i];
        if (!(role & R_PICK)) continue;
        const Unit u = unit_at(g, e, b, i);
        int32_t rs, rb, ss, sb;
        closest(g, e, u.cell, lr, b.n_resource, &rs, &rb);
        closest(g, e, u.cell, ls, b.n_stock, &ss, &sb);
        const bool carrying = u.carried > 0;
        const bool harvesting = is_entry(b, y, i, u.birth, kAbHarvest);
        const bool same_base = carry_at<TW>(b, y, 5, i) == ss && bv<int32_t>(b, y.k_bbirth)[i] == sb;
        const bool same_target = carry_at<TW>(b, y, 3, i) == rs && bv<int32_t>(b, y.k_tbirth)[i] == rb;
        const bool occupied = carrying ? ss != kAbsent : (ss != kAbsent && rs != kAbsent);
        const bool unchanged = harvesting && same_base && (carrying || same_target);
        if (occupied && !unchanged)
            put_unit<TW>(g, b, u, i, false, kAbHarvest, carrying ? kAbsent : rs, carrying ? kAbsent : rb, ss, sb, kAbsent,
                     kAbsent, y);
        if (!occupied) r[i] = (uint8_t)(role | R_IDLE);
    }
    b.next_order = wadd(b.next_order, g.C + 1);
    wave_sync();
}

// rush._attack_nearest (N/bots/rush.py:61-70) for the units whose role has
// any of `bits`; R_LAST units are stamped last.
template <int TW = kWave>
NR_DEV void attack_nearest(const KGame& g, const Env& e, Bot& b, const BotLayout& y, uint8_t bits, int lane) {
    const AS3 uint8_t* r = roles(b, y);
    for (int32_t k = lane; k < b.n_live; k += TW) {
        const int32_t i = bv<int16_t>(b, y.u_live)[k];
        const uint8_t role = r[i];
        if (!(role & bits)) continue;
        const int32_t es = bv<int16_t>(b, y.u_es)[i];
        if (es == kAbsent) continue;
        const Unit u = unit_at(g, e, b, i);
        put_unit<TW>(g, b, u, i, (role & R_LAST) != 0, kAbAttack, es, bv<int32_t>(b, y.u_eb)[i], kAbsent, kAbsent,
                 kAbsent, kAbsent, y);
    }
    b.next_order = wadd(b.next_order, g.C + 1);
    wave_sync();
}

// A put of TRAIN for the units `pick` selects.
template <int TW, typename Pick>
NR_DEV void train_where(const KGame& g, const Env& e, Bot& b, const BotLayout& y, int32_t unit_type, Pick pick,
                        int lane) {
    for (int32_t k = lane; k < b.n_live; k += TW) {
        const int32_t i = bv<int16_t>(b, y.u_live)[k];
        const Unit u = unit_at(g, e, b, i);
        if (pick(u)) put_unit<TW>(g, b, u, i, false, kAbTrain, kAbsent, kAbsent, kAbsent, kAbsent, kAbsent, unit_type, y);
    }
    b.next_order = wadd(b.next_order, g.C + 1);
    wave_sync();
}

// rush._melee_units_attack with available_melee (N/bots/rush.py:73-85); also
// marks the workers (present units that can harvest) R_WORKER.
template <int TW = kWave>
NR_DEV void melee_attack(const KGame& g, const Hdr& h, const Env& e, Bot& b, const BotLayout& y, int lane) {
    AS3 uint8_t* r = roles(b, y);
    for (int32_t k = lane; k < b.n_live; k += TW) {
        const int32_t i = bv<int16_t>(b, y.u_live)[k];
        const Unit u = unit_at(g, e, b, i);
        const bool harvests = type_flag(g, h, u.type, FL_HARVEST);
        const bool melee = u.present && type_flag(g, h, u.type, FL_ATTACK) && !harvests && u.available;
        r[i] = (uint8_t)((melee ? R_PICK : 0) | ((u.present && harvests) ? R_WORKER : 0));
    }
    wave_sync();
    attack_nearest<TW>(g, e, b, y, R_PICK, lane);
}

// Role bytes for a new decision: R_WORKER kept, `pick` units get R_PICK,
// others lose R_PICK / R_IDLE / R_LAST.
template <int TW = kWave>
NR_DEV void mark_picks(const KGame& g, const Bot& b, const BotLayout& y, int32_t skip0, int32_t skip1, int32_t only,
                       int lane) {
    AS3 uint8_t* r = roles(b, y);
    for (int32_t k = lane; k < b.n_live; k += TW) {
        const int32_t i = bv<int16_t>(b, y.u_live)[k];
        const uint8_t w = r[i] & R_WORKER;
        const bool pick = only >= 0 ? i == only : (w && i != skip0 && i != skip1);
        r[i] = (uint8_t)(w | (pick ? R_PICK : 0));
    }
    wave_sync();
}

// rush.worker_rush (N/bots/rush.py:213-220) with _rushing_workers (:204-210).
template <int TW = kWave>
NR_DEV void worker_rush(const KGame& g, const Hdr& h, const Env& e, Bot& b, const BotLayout& y, int lane) {
    const int32_t res = tuni<TW>(e.sc[S_RES0 + b.player]);
    const int32_t worker_cost = tabv(h, F_COST, kTypeWorker);
    train_where<TW>(g, e, b, y, kTypeWorker,
                [&](const Unit& u) { return u.present && u.type == kTypeBase && u.available && res >= worker_cost; },
                lane);
    melee_attack<TW>(g, h, e, b, y, lane);
    const int32_t builder = build_base<TW>(g, h, e, b, y, lane);
    const int32_t harvester = first_of<TW>(g, e, b, y, R_WORKER, builder, -1, lane);
    mark_picks<TW>(g, b, y, -1, -1, harvester < 0 ? g.C : harvester, lane);
    harvest<TW>(g, e, b, y, lane);
    // free = (workers - builder - harvester) | idle harvester; the idle
    // harvester is stamped last
    AS3 uint8_t* r = roles(b, y);
    for (int32_t k = lane; k < b.n_live; k += TW) {
        const int32_t i = bv<int16_t>(b, y.u_live)[k];
        const uint8_t role = r[i];
        const bool idle = (role & R_IDLE) != 0;
        const bool free = ((role & R_WORKER) && i != builder && i != harvester) || idle;
        r[i] = (uint8_t)((role & R_WORKER) | (free ? R_PICK : 0) | (idle ? R_LAST : 0));
    }
    wave_sync();
    attack_nearest<TW>(g, e, b, y, R_PICK, lane);
}

// rush.barracks_rush (N/bots/rush.py:229-236) with train_at_base_and_barracks
// (:107-133), build_base_and_barracks (:184-201) and _workers_behavior
// (:223-226).
template <int TW = kWave>
NR_DEV void barracks_rush(const KGame& g, const Hdr& h, const Env& e, Bot& b, const BotLayout& y,
                          int32_t trained_type, int lane) {
    const int32_t res = tuni<TW>(e.sc[S_RES0 + b.player]);
    int32_t held = 0;
    bool any_barracks = false;
    for (int32_t k = lane; k < b.n_live; k += TW) {
        const int32_t i = bv<int16_t>(b, y.u_live)[k];
        const Unit u = unit_at(g, e, b, i);
        held += (u.present && u.type == kTypeWorker) ? 1 : 0;
        any_barracks |= u.present && u.type == kTypeBarracks;
    }
    held = team_sum<TW>(held);
    any_barracks = tballot<TW>(any_barracks) != 0ull;
    const int32_t worker_cost = tabv(h, F_COST, kTypeWorker);
    train_where<TW>(g, e, b, y, kTypeWorker,
                [&](const Unit& u) {
                    return u.present && u.type == kTypeBase && u.available && held < 1 && res >= worker_cost;
                },
                lane);
    const int32_t trained_cost = tabv(h, F_COST, clampi(trained_type, 0, g.T - 1));
    train_where<TW>(g, e, b, y, trained_type,
                [&](const Unit& u) { return u.present && u.type == kTypeBarracks && u.available && res >= trained_cost; },
                lane);
    melee_attack<TW>(g, h, e, b, y, lane);
    const int32_t base_builder = build_base<TW>(g, h, e, b, y, lane);
    const int32_t used = base_builder >= 0 ? tabv(h, F_COST, kTypeBase) : 0;
    const bool builds_barracks = !any_barracks && res >= wadd(tabv(h, F_COST, kTypeBarracks), used);
    const int32_t barracks_builder = builds_barracks ? first_of<TW>(g, e, b, y, R_WORKER, base_builder, -1, lane) : -1;
    build_unless_building<TW>(g, h, e, b, y, barracks_builder, kTypeBarracks, lane);
    mark_picks<TW>(g, b, y, base_builder, barracks_builder, -1, lane);
    harvest<TW>(g, e, b, y, lane);
    attack_nearest<TW>(g, e, b, y, R_IDLE, lane);
}

// ---------------------------------------------------------------------------
// pathfinding.search (N/bots/pathfinding.py:170-245) on lane 0.
// Open cells pop by least f = g + Manhattan(cell, target), the most recently
// inserted first among equal f; neighbours are inserted up, right, down,
// left; each cell once.  A neighbour's f is the popped cell's f or f + 2,
// and every open cell has f_low or f_low + 2 (f_low = f of the last pop), so
// the open list is two LIFO stacks linked through below[]: `cur` (f_low)
// and `nxt` (f_low + 2).  mark[c]: 0 open, 1 blocked, 2 + d inserted with
// first step d from the start.  Returns the first step's direction, or -1
// when no cell within `range` of the target is reachable or the start is
// already within it.
// ---------------------------------------------------------------------------
NR_DEV int32_t astar_first_step(const KGame& g, AS3 int16_t* below, AS3 uint8_t* mark, int32_t start, int32_t target,
                                int32_t range) {
    const int32_t W = g.W, H = g.H;
    const int32_t tx = floor_mod(target, W), ty = floor_div(target, W);
    const int32_t r2 = (int32_t)((uint32_t)range * (uint32_t)range);
    mark[start] = 2;
    int32_t cur = start, nxt = -1;
    below[start] = -1;
    while (true) {
        if (cur < 0) {
            if (nxt < 0) return kAbsent;
            cur = nxt;
            nxt = -1;
        }
        const int32_t pos = cur;
        const int32_t py = cell_y(g, pos), px = pos - py * W;
        // every read of this pop is issued before its first write: the four
        // neighbours are distinct cells and only this pop writes them
        int32_t nbs[4];
        bool on[4];
#pragma unroll
        for (int32_t d = 0; d < 4; ++d) {
            const int32_t nx = px + dir_dx(d), ny = py + dir_dy(d);
            on[d] = nx >= 0 && nx < W && ny >= 0 && ny < H;
            nbs[d] = on[d] ? ny * W + nx : pos;
        }
        cur = below[pos];
        const int32_t first = (int32_t)mark[pos] - 3;  // -1 at the start
        int32_t seen[4];
#pragma unroll
        for (int32_t d = 0; d < 4; ++d) seen[d] = mark[nbs[d]];
        const int32_t dx = px - tx, dy = py - ty;
        if (dx * dx + dy * dy <= r2) {
            // the reference maps the step offset +W, -1, -W, +1 in that order:
            // on a one-wide board an upward step (-W = -1) reads as LEFT
            return (first == 0 && W == 1) ? 3 : first;
        }
        const int32_t hcur = abs(dx) + abs(dy);
#pragma unroll
        for (int32_t d = 0; d < 4; ++d) {
            if (!on[d] || seen[d] != 0) continue;
            const int32_t nx = px + dir_dx(d), ny = py + dir_dy(d);
            const int32_t nb = nbs[d];
            mark[nb] = (uint8_t)(3 + (first < 0 ? d : first));
            if (abs(nx - tx) + abs(ny - ty) < hcur) {
                below[nb] = (int16_t)cur;
                cur = nb;
            } else {
                below[nb] = (int16_t)nxt;
                nxt = nb;
            }
        }
    }
}

// The whole answer of pathfinding.search (N/bots/pathfinding.py:72-130): found,
// the first step, the path's length and the number of pops, for the FFI
// targets nanorts_astar_search and nanorts_astar_chain.  The same search as
// astar_first_step (same stacks, same pop order); depth[] holds each
// inserted cell's distance from the start.  mark[] comes in with 0 for open
// and 1 for blocked cells; a start off the board finds nothing and pops
// nothing.  The step of a path of length 0 is -1.
struct AstarPath {
    int32_t found, step, distance, pops;
};
NR_DEV AstarPath astar_path(int32_t W, int32_t H, AS3 int16_t* below, AS3 uint8_t* mark, AS3 int16_t* depth,
                            int32_t start, int32_t target, int32_t range) {
    AstarPath out = {0, kAbsent, kAbsent, 0};
    if (start < 0 || start >= W * H) return out;
    const int32_t tx = floor_mod(target, W), ty = floor_div(target, W);
    const int32_t r2 = (int32_t)((uint32_t)range * (uint32_t)range);
    mark[start] = 2;
    depth[start] = 0;
    int32_t cur = start, nxt = -1;
    below[start] = -1;
    while (true) {
        if (cur < 0) {
            if (nxt < 0) return out;
            cur = nxt;
            nxt = -1;
        }
        const int32_t pos = cur;
        ++out.pops;
        const int32_t py = pos / W, px = pos - py * W;
        cur = below[pos];
        const int32_t first = (int32_t)mark[pos] - 3;  // -1 at the start
        const int32_t dx = px - tx, dy = py - ty;
        if (dx * dx + dy * dy <= r2) {
            out.found = 1;
            out.distance = depth[pos];
            // the offsets +W, -1, -W, +1 are told apart in that order: on a
            // one-wide board an upward step (-W = -1) reads as LEFT
            out.step = first < 0 ? kAbsent : ((first == 0 && W == 1) ? 3 : first);
            return out;
        }
        const int32_t hcur = abs(dx) + abs(dy);
        const int32_t dnext = depth[pos] + 1;
        for (int32_t d = 0; d < 4; ++d) {
            const int32_t nx = px + dir_dx(d), ny = py + dir_dy(d);
            if (nx < 0 || nx >= W || ny < 0 || ny >= H) continue;
            const int32_t nb = ny * W + nx;
            if (mark[nb] != 0) continue;
            mark[nb] = (uint8_t)(3 + (first < 0 ? d : first));
            depth[nb] = (int16_t)dnext;
            if (abs(nx - tx) + abs(ny - ty) < hcur) {
                below[nb] = (int16_t)cur;
                cur = nb;
            } else {
                below[nb] = (int16_t)nxt;
                nxt = nb;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// abstraction.translate with the rush kinds and filler duration 10
// (N/bots/abstraction.py:300-319 and the helpers cited below).
// ---------------------------------------------------------------------------
NR_DEV int32_t sq_distance(const KGame& g, int32_t a, int32_t c) {
    const int32_t dx = floor_mod(a, g.W) - floor_mod(c, g.W), dy = floor_div(a, g.W) - floor_div(c, g.W);
    return wadd(wmul(dx, dx), wmul(dy, dy));
}

NR_DEV int32_t step_cell(const KGame& g, int32_t cell, int32_t direction) {
    const int32_t d = clampi(direction, 0, 3);
    return wadd(cell, dir_dy(d) * g.W + dir_dx(d));
}

// _adjacent_direction (N/bots/abstraction.py:399-407)
NR_DEV int32_t adjacent_direction(const KGame& g, int32_t origin, int32_t goal) {
    if (goal == kAbsent) return kAbsent;
    const int32_t dx = floor_mod(goal, g.W) - floor_mod(origin, g.W), dy = floor_div(goal, g.W) - floor_div(origin, g.W);
    for (int32_t d = 0; d < 4; ++d)
        if (dx == dir_dx(d) && dy == dir_dy(d)) return d;
    return kAbsent;
}

struct Desire {
    int32_t kind, dir, target, ptype, claimed, cost;
};

NR_DEV Desire no_desire() { return Desire{kAbsent, kAbsent, kAbsent, kAbsent, kAbsent, 0}; }

NR_DEV bool within_balance(const Env& e, const Bot& b, int32_t p) {
    const int32_t r = p == 0 ? b.reserved0 : b.reserved1;
    return r == 0 || r <= e.sc[S_RES0 + p];
}

// _production with _produce_allowed (N/bots/abstraction.py:440-462, 368-380)
NR_DEV Desire production(const KGame& g, const Hdr& h, const Env& e, const Bot& b, const BotLayout& y,
                         int32_t direction, int32_t ptype, int32_t cell) {
    const int32_t own = b.player;
    const int32_t claimed = direction != kAbsent ? step_cell(g, cell, direction) : kAbsent;
    const int32_t cost = tabv(h, F_COST, clampi(ptype, 0, g.T - 1));
    const int32_t reserved = own == 0 ? b.reserved0 : b.reserved1;
    const bool allowed = direction != kAbsent && !bit_of(bv<uint32_t>(b, y.m_claimed), clampi(claimed, 0, g.cells - 1)) &&
                         (reserved == 0 || wadd(cost, reserved) <= e.sc[S_RES0 + own]) && within_balance(e, b, 1 - own);
    if (!allowed) return no_desire();
    return Desire{kKindProduce, direction, kAbsent, ptype, claimed, cost};
}

// _training_direction (N/bots/abstraction.py:465-489)
NR_DEV int32_t training_direction(const KGame& g, const Hdr& h, const Env& e, const Bot& b, const BotLayout& y,
                                  int32_t cell, int32_t produced) {
    const bool harvests = type_flag(g, h, produced, FL_HARVEST);
    const AS3 int16_t* near = harvests ? bv<int16_t>(b, y.l_resource) : bv<int16_t>(b, y.l_enemy);
    const int32_t n = harvests ? b.n_resource : b.n_enemy;
    const AS3 uint32_t* freem = bv<uint32_t>(b, y.m_free);
    const int32_t cx = floor_mod(cell, g.W), cy = floor_div(cell, g.W);
    int32_t best = kAbsent, best_score = 0;
    for (int32_t d = 0; d < 4; ++d) {
        const int32_t x = cx + dir_dx(d), yy = cy + dir_dy(d);
        if (x < 0 || x >= g.W || yy < 0 || yy >= g.H || !bit_of(freem, yy * g.W + x)) continue;
        int32_t nearest = kLast;
#pragma unroll 4
        for (int32_t k = 0; k < n; ++k) {
            const int32_t c = e.cell[near[k]];
            const int32_t dist = abs(x - cell_x(g, c)) + abs(yy - cell_y(g, c));
            nearest = dist < nearest ? dist : nearest;
        }
        const int32_t score = n > 0 ? -nearest : 0;
        if (best == kAbsent || score > best_score) {
            best = d;
            best_score = score;
        }
    }
    return best;
}

NR_DEV bool exists_slot(const KGame& g, const Env& e, int32_t slot, int32_t birth) {
    return slot != kAbsent && e.birth[clampi(slot, 0, g.E - 1)] == birth;
}

NR_DEV int32_t cell_of_slot(const KGame& g, const Env& e, int32_t slot) {
    return slot != kAbsent ? (int32_t)e.cell[clampi(slot, 0, g.E - 1)] : kAbsent;
}

// Usage, standing, plan and queue; returns the number of queued units.
template <int TW = kWave>
NR_DEV int32_t translate_plan(const KGame& g, const Hdr& h, const Env& e, Bot& b, const BotLayout& y, int lane) {
    const int32_t C = g.C, words = (g.cells + 31) / 32;
    AS3 uint32_t* claimed = bv<uint32_t>(b, y.m_claimed);
    AS3 uint32_t* freem = bv<uint32_t>(b, y.m_free);
    for (int32_t w = lane; w < words; w += TW) {
        claimed[w] = 0u;
        freem[w] = 0u;
        bv<uint32_t>(b, y.m_used)[w] = 0u;
        bv<uint32_t>(b, y.m_kept)[w] = 0u;
    }
    wave_sync();
    // _pending_usage (N/bots/abstraction.py:331-359)
    int32_t cost0 = 0, cost1 = 0;
    for (int32_t s = lane; s < g.E; s += TW) {
        if (e.birth[s] == kAbsent) continue;
        const int32_t kind = e.pkind[s];
        if (kind == kKindMove || kind == kKindProduce) {
            int32_t t = step_cell(g, e.cell[s], e.pdir[s]);
            if (t < 0) t += g.cells;
            if (t >= 0 && t < g.cells) set_bit(claimed, t);
        }
        if (kind == kKindProduce && s >= g.N) {
            const int32_t c = tabv(h, F_COST, clampi(e.pptype[s], 0, g.T - 1));
            if ((s - g.N) / C == 0) cost0 = wadd(cost0, c);
            else cost1 = wadd(cost1, c);
        }
    }
    b.reserved0 = team_sum<TW>(cost0);
    b.reserved1 = team_sum<TW>(cost1);
    wave_sync();
    // _free_cells (:362-365)
    for (int32_t c = lane; c < g.cells; c += TW)
        if (h.terrain[c] == 0 && e.entity[c] == kAbsent && !bit_of(claimed, c)) set_bit(freem, c);
    wave_sync();
    // _standing (:383-423) and _plan (:653-715) with _fallback (:575-650)
    for (int32_t i = lane; i < C; i += TW) {
        const Unit u = unit_at(g, e, b, i);
        const int32_t kind = bv<int8_t>(b, y.k_kind)[i];
        const bool alive = kind != kAbNone && bv<int32_t>(b, y.k_ubirth)[i] == u.birth;
        const bool carrying = u.carried > 0;
        const int32_t kcell = carry_at<TW>(b, y, 7, i);
        const int32_t target = carry_at<TW>(b, y, 3, i);
        const int32_t base = carry_at<TW>(b, y, 5, i);
        const bool built_on = kcell != kAbsent && e.entity[clampi(kcell, 0, g.cells - 1)] != kAbsent;
        const bool target_gone = !exists_slot(g, e, target, bv<int32_t>(b, y.k_tbirth)[i]);
        bool completed = false;
        if (kind == kAbAttack) completed = target_gone;
        else if (kind == kAbHarvest) completed = carrying ? !exists_slot(g, e, base, bv<int32_t>(b, y.k_bbirth)[i]) : target_gone;
        else if (kind == kAbTrain) completed = bv<uint8_t>(b, y.k_trained)[i] != 0;
        else if (kind == kAbBuild) completed = built_on;
        const bool standing = alive && !completed;
        const bool executes = standing && u.available;
        bv<uint8_t>(b, y.u_flags)[i] = (uint8_t)((standing ? U_STANDING : 0) | (executes ? U_EXECUTES : 0));
        if (!executes) continue;
        const int32_t target_cell = cell_of_slot(g, e, target);
        const int32_t range = tabv(h, F_RANGE, u.type);
        const bool in_range = sq_distance(g, u.cell, target_cell) <= wmul(range, range);
        const int32_t harvest_goal = carrying ? cell_of_slot(g, e, base) : target_cell;
        int32_t goal = kAbsent, radius = 0;
        Desire fb = no_desire();
        const int32_t utype = bv<int8_t>(b, y.k_utype)[i];
        if (kind == kAbAttack) {
            goal = target_cell;
            radius = range;
            if (in_range && target_cell != kAbsent) fb = Desire{kKindAttack, kAbsent, target_cell, kAbsent, kAbsent, 0};
        } else if (kind == kAbHarvest) {
            goal = harvest_goal;
            radius = 1;
            const int32_t d = adjacent_direction(g, u.cell, harvest_goal);
            if (d != kAbsent) fb = Desire{carrying ? kKindReturn : kKindHarvest, d, kAbsent, kAbsent, kAbsent, 0};
        } else if (kind == kAbTrain) {
            fb = production(g, h, e, b, y, training_direction(g, h, e, b, y, u.cell, utype), utype, u.cell);
        } else if (kind == kAbBuild) {
            goal = kcell;
            radius = 1;
            fb = production(g, h, e, b, y, adjacent_direction(g, u.cell, kcell), utype, u.cell);
        }
        const bool searches = goal != kAbsent && !(kind == kAbAttack && in_range);
        bv<int16_t>(b, y.u_goal)[i] = (int16_t)(searches ? goal : u.cell);
        bv<int16_t>(b, y.u_radius)[i] = (int16_t)(searches ? radius : 0);
        bv<int8_t>(b, y.u_fkind)[i] = (int8_t)fb.kind;
        bv<int8_t>(b, y.u_fdir)[i] = (int8_t)fb.dir;
        bv<int16_t>(b, y.u_ftarget)[i] = (int16_t)fb.target;
        bv<int8_t>(b, y.u_fptype)[i] = (int8_t)fb.ptype;
        bv<int16_t>(b, y.u_fclaimed)[i] = (int16_t)fb.claimed;
        bv<int16_t>(b, y.u_fcost)[i] = (int16_t)fb.cost;
    }
    wave_sync();
    // _queue (:800-801): executing units by order, ties by unit index
    AS3 int16_t* list = bv<int16_t>(b, y.u_list);
    AS3 int32_t* key = bv<int32_t>(b, y.u_lkey);
    int32_t queued = 0;
    for (int32_t i0 = 0; i0 < C; i0 += TW) {
        const int32_t i = i0 + lane;
        const bool ex = i < C && (bv<uint8_t>(b, y.u_flags)[i] & U_EXECUTES);
        const uint64_t m = tballot<TW>(ex);
        if (ex) {
            list[queued + tcount_below<TW>(m)] = (int16_t)i;
            key[queued + tcount_below<TW>(m)] = bv<int32_t>(b, y.k_order)[i];
        }
        queued += popc(m);
    }
    wave_sync();
    for (int32_t k = lane; k < queued; k += TW) {
        const int32_t oi = key[k];
        int32_t r = 0;
#pragma unroll 4
        for (int32_t q = 0; q < queued; ++q) {
            const int32_t oq = key[q];
            r += (oq < oi || (oq == oi && q < k)) ? 1 : 0;
        }
        bv<int16_t>(b, y.u_queue)[r] = list[k];
    }
    for (int32_t i = lane; i < C; i += TW) {
        bv<uint8_t>(b, y.u_sel)[i] = SEL_NONE;
        bv<int16_t>(b, y.u_drank)[i] = (int16_t)kAbsent;
    }
    wave_sync();
    return queued;
}

// _walked / _walk_step with _answer and _kept (N/bots/abstraction.py:718-797,
// 904-952): returns how many desires it keeps.
template <int TW = kWave>
NR_DEV int32_t translate_walk(const KGame& g, const Hdr& h, const Env& e, Bot& b, const BotLayout& y, int32_t queued,
                              int lane) {
    (void)h;
    AS3 uint32_t* claimed = bv<uint32_t>(b, y.m_claimed);
    AS3 uint32_t* freem = bv<uint32_t>(b, y.m_free);
    AS3 uint32_t* used = bv<uint32_t>(b, y.m_used);
    AS3 uint32_t* kept_m = bv<uint32_t>(b, y.m_kept);
    AS3 int16_t* below = bv<int16_t>(b, y.a_below);
    AS3 uint8_t* mark = bv<uint8_t>(b, y.a_mark);
    const int32_t own = b.player;
    const bool may_move = within_balance(e, b, 0) && within_balance(e, b, 1);
    const int32_t reserved_own = own == 0 ? b.reserved0 : b.reserved1;
    const int32_t balance = tuni<TW>(e.sc[S_RES0 + own]);
    int32_t spent = 0, granted = 0;
    for (int32_t q = 0; q < queued; ++q) {
        const int32_t i = tuni<TW>(bv<int16_t>(b, y.u_queue)[q]);
        const int32_t start = tuni<TW>(e.cell[b.block + i]);
        const int32_t goal = tuni<TW>(bv<int16_t>(b, y.u_goal)[i]);
        const int32_t radius = tuni<TW>(bv<int16_t>(b, y.u_radius)[i]);
        int32_t step = kAbsent;
        // the first pop is the start: already within range means no step
        if (start >= 0 && start < g.cells && sq_distance(g, start, goal) > wmul(radius, radius)) {
            if ((g.cells & 3) == 0) {
                // four cells per lane: their open bits to four mark bytes
                for (int32_t q = lane; q < g.cells / 4; q += TW) {
                    const int32_t c0 = 4 * q;
                    const uint32_t shut = ~((freem[c0 >> 5] & ~used[c0 >> 5]) >> (c0 & 31)) & 15u;
                    ((AS3 uint32_t*)mark)[q] = (shut & 1u) | ((shut & 2u) << 7) | ((shut & 4u) << 14) | ((shut & 8u) << 21);
                }
            } else {
                for (int32_t c = lane; c < g.cells; c += TW) mark[c] = (bit_of(freem, c) && !bit_of(used, c)) ? 0 : 1;
            }
            wave_sync();
            int32_t s = kAbsent;
            if (lane == 0) s = astar_first_step(g, below, mark, start, goal, radius);
            step = tread<TW>(s, 0);
            wave_sync();
        }
        int32_t sel, kind, claim, cost;
        if (step != kAbsent) {
            sel = may_move ? SEL_MOVED : SEL_NONE;
            kind = may_move ? kKindMove : kAbsent;
            claim = may_move ? step_cell(g, start, step) : kAbsent;
            cost = 0;
        } else {
            sel = SEL_FALLBACK;
            kind = tuni<TW>(bv<int8_t>(b, y.u_fkind)[i]);
            claim = tuni<TW>(bv<int16_t>(b, y.u_fclaimed)[i]);
            cost = tuni<TW>(bv<int16_t>(b, y.u_fcost)[i]);
        }
        const bool has_cell = claim != kAbsent && claim >= 0 && claim < g.cells;
        const bool conflicting = has_cell && (bit_of(claimed, claim) || bit_of(kept_m, claim));
        const bool over_budget = cost > 0 && wadd(wadd(reserved_own, spent), cost) > balance;
        const bool kept = kind != kAbsent && !conflicting && !over_budget;
        if (lane == 0) {
            if (has_cell) {
                used[claim >> 5] |= 1u << (claim & 31);
                if (kept) kept_m[claim >> 5] |= 1u << (claim & 31);
            }
            if (kept) {
                bv<uint8_t>(b, y.u_sel)[i] = (uint8_t)sel;
                bv<int8_t>(b, y.u_dir)[i] = (int8_t)step;
                bv<int16_t>(b, y.u_drank)[i] = (int16_t)granted;
            }
        }
        if (kept) {
            spent = wadd(spent, cost);
            ++granted;
        }
        wave_sync();
    }
    return granted;
}

// The decided command of unit i (_commands, N/bots/abstraction.py:1063-1096):
// {kind, direction, none_duration, target_cell, produced_type, request_order}.
NR_DEV void unit_command(const KGame& g, const Env& e, const Bot& b, const BotLayout& y, int32_t i, int32_t granted,
                         int32_t out[6]) {
    const Unit u = unit_at(g, e, b, i);
    const int32_t sel = bv<uint8_t>(b, y.u_sel)[i];
    int32_t kind = kAbsent, dir = kAbsent, target = kAbsent, ptype = kAbsent;
    if (sel == SEL_MOVED) {
        kind = kKindMove;
        dir = bv<int8_t>(b, y.u_dir)[i];
    } else if (sel == SEL_FALLBACK) {
        kind = bv<int8_t>(b, y.u_fkind)[i];
        dir = bv<int8_t>(b, y.u_fdir)[i];
        target = bv<int16_t>(b, y.u_ftarget)[i];
        ptype = bv<int8_t>(b, y.u_fptype)[i];
    }
    const bool kept = sel != SEL_NONE;
    const bool filler = u.available && !kept;
    int32_t filler_rank = 0;
    if (filler) {
        const AS3 int16_t* live = bv<int16_t>(b, y.u_live);
        const AS3 int32_t* lbirth = bv<int32_t>(b, y.u_lbirth);
#pragma unroll 4
        for (int32_t q = 0; q < b.n_live; ++q) {
            const int32_t j = live[q];
            filler_rank += (e.pkind[b.block + j] == kAbsent && bv<uint8_t>(b, y.u_sel)[j] == SEL_NONE &&
                            lbirth[q] < u.birth) ? 1 : 0;
        }
    }
    out[0] = kept ? kind : (filler ? kKindNone : kAbsent);
    out[1] = kept ? dir : kAbsent;
    out[2] = filler ? kFillerDuration : 0;  // no rush desire waits
    out[3] = kept ? target : kAbsent;
    out[4] = kept ? ptype : kAbsent;
    out[5] = kept ? (int32_t)bv<int16_t>(b, y.u_drank)[i] : (filler ? wadd(granted, filler_rank) : kAbsent);
}

// The carry rows in LDS and b.next_order into the carry of env l.
template <int TW = kWave>
NR_DEV void store_carry(const KGame& g, const Bot& b, const BotLayout& y, int64_t l, const BotCarry& carry, int lane) {
    for (int32_t i = lane; i < g.C; i += TW) {
        const int64_t at = l * g.C + i;
        carry.row[0][at] = bv<int8_t>(b, y.k_kind)[i];
#pragma unroll
        for (int f = 1; f < 8; ++f) carry.row[f][at] = carry_at<TW>(b, y, f, i);
        carry.row[8][at] = bv<int8_t>(b, y.k_utype)[i];
        carry.trained[at] = bv<uint8_t>(b, y.k_trained)[i];
    }
    if (lane == 0) carry.next_order[l] = b.next_order;
}

// _settled (N/bots/abstraction.py:1099-1119): the carry rows in LDS become
// the settled carry (the standing units, their orders ranked; the others
// emptied) and b.next_order the standing count; with `to_memory` they are
// also written to the carry rows of env l.
template <int TW = kWave>
NR_DEV void settle_carry(const KGame& g, Bot& b, const BotLayout& y, int64_t l, const BotCarry& carry, int lane,
                         bool to_memory = true) {
    const int32_t C = g.C;
    // the standing units with their orders
    AS3 int32_t* key = bv<int32_t>(b, y.u_lkey);
    int32_t standing = 0;
    for (int32_t i0 = 0; i0 < C; i0 += TW) {
        const int32_t i = i0 + lane;
        const bool st = i < C && (bv<uint8_t>(b, y.u_flags)[i] & U_STANDING);
        const uint64_t m = tballot<TW>(st);
        if (st) key[standing + tcount_below<TW>(m)] = bv<int32_t>(b, y.k_order)[i];
        standing += popc(m);
    }
    wave_sync();
    for (int32_t i = lane; i < C; i += TW) {
        const int32_t fl = bv<uint8_t>(b, y.u_flags)[i];
        const bool st = (fl & U_STANDING) != 0;
        const int32_t oi = bv<int32_t>(b, y.k_order)[i];
        int32_t r = 0;
#pragma unroll 4
        for (int32_t q = 0; q < standing; ++q) r += key[q] < oi ? 1 : 0;
        const int32_t kind = bv<int8_t>(b, y.k_kind)[i];
        const bool trained = st && (bv<uint8_t>(b, y.k_trained)[i] != 0 ||
                                    ((fl & U_EXECUTES) && (kind == kAbTrain || kind == kAbTrainDirection)));
        if (st) {
            bv<int32_t>(b, y.k_order)[i] = r;
        } else {
            bv<int8_t>(b, y.k_kind)[i] = (int8_t)kAbsent;
#pragma unroll
            for (int f = 1; f < 8; ++f) carry_put<TW>(b, y, f, i, kAbsent);
            bv<int8_t>(b, y.k_utype)[i] = (int8_t)kAbsent;
        }
        bv<uint8_t>(b, y.k_trained)[i] = trained ? 1 : 0;
    }
    b.next_order = standing;
    wave_sync();
    if (to_memory) store_carry<TW>(g, b, y, l, carry, lane);
}

// abstraction.empty_actions into the carry rows of env l (a new episode).
template <int TW = kWave>
NR_DEV void clear_carry(const KGame& g, int64_t l, const BotCarry& carry, int lane) {
    for (int32_t i = lane; i < g.C; i += TW) {
        const int64_t at = l * g.C + i;
#pragma unroll
        for (int f = 0; f < 9; ++f) carry.row[f][at] = kAbsent;
        carry.trained[at] = 0;
    }
    if (lane == 0) carry.next_order[l] = 0;
}

// The same in LDS, for a fused rollout that keeps the carry there.
template <int TW = kWave>
NR_DEV void clear_carry_rows(const KGame& g, Bot& b, const BotLayout& y, int lane) {
    for (int32_t i = lane; i < g.C; i += TW) {
        bv<int8_t>(b, y.k_kind)[i] = (int8_t)kAbsent;
#pragma unroll
        for (int f = 1; f < 8; ++f) carry_put<TW>(b, y, f, i, kAbsent);
        bv<int8_t>(b, y.k_utype)[i] = (int8_t)kAbsent;
        bv<uint8_t>(b, y.k_trained)[i] = 0;
    }
    b.next_order = 0;
    wave_sync();
}

// family.act (N/bots/family.py:34-41): the rush decisions on the carry, then
// translate's plan and walk.  Returns how many desires the walk keeps; commands come from
// unit_command and the carry from settle_carry.
template <int TW = kWave>
NR_DEV int32_t bot_act(const KGame& g, const Hdr& h, const Env& e_in, Bot& b, const BotLayout& y, int64_t l,
                       const BotCarry& carry, int32_t strategy, int32_t trained_type, int lane,
                       bool load_carry = true) {
    // the block's pointers rebuilt here rather than held across the caller's
    // phases
    const Env e = refresh<TW>(g, e_in);
    b.base = e.base + y.origin;
    bot_begin<TW>(g, h, e, b, y, l, carry, lane, load_carry);
    if (strategy == kWorkerRush) worker_rush<TW>(g, h, e, b, y, lane);
    else barracks_rush<TW>(g, h, e, b, y, trained_type, lane);
    const int32_t queued = translate_plan<TW>(g, h, e, b, y, lane);
    return translate_walk<TW>(g, h, e, b, y, queued, lane);
}

}  // namespace nr
