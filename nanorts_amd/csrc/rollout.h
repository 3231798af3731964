// The per-cycle summary of the fused env path and the sampling phase that
// reads it.
//
// `summarize` runs once after every cycle (and once after the state is
// loaded).  In three passes it derives everything the next cycle's masks,
// admission and this cycle's observation need from the post-step state:
//   slots: the occupant word and flags of every live slot, the list of
//          available owned positions and of active owned units;
//   units: the sight disks of both players, stamped row by row from a
//          precomputed disk table (N/observations/visibility.py:56-71);
//   cells: four consecutive cells per lane -> the six occupancy bitmaps of
//          the masks, and both agents' symbolic feature maps
//          (N/observations/symbolic.py:130-180) packed into dwords and
//          stored straight to HBM.
#pragma once

#include "envstep.h"

namespace nr {

// sample_row with select_bit (same draws, same result), given the
// position's four draw words threefry(k_step, (env, 2p)) ++ threefry(k_step, (env, 2p + 1)).
NR_DEV void sample_row_words(const KGame& g, const Row& r, const uint32_t words[4], int32_t a[7]) {
    if (only_none(r)) {
#pragma unroll
        for (int f = 0; f < 7; ++f) a[f] = 0;
        return;
    }
    const int32_t lo[7] = {0, 6, 10, 14, 18, 22, 22 + g.T};
    const int32_t wid[7] = {6, 4, 4, 4, 4, g.T, g.O};
#pragma unroll
    for (int f = 0; f < 7; ++f) {
        const uint32_t hh = (words[f >> 1] >> (16 * (f & 1))) & 0xFFFFu;
        const uint64_t m = row_bits(r, lo[f], wid[f]);
        const int32_t count = popc(m);
        a[f] = count > 0 ? select_bit(m, (int32_t)((hh * (uint32_t)count) >> 16)) : 0;
    }
}

// k-th set bit of an 8-bit mask (more than k bits set), by halving.
NR_DEV int32_t select_bit8(uint32_t v, int32_t k) {
    int32_t pos = 0;
    int32_t c = __popc(v & 15u);
    if (k >= c) {
        k -= c;
        v >>= 4;
        pos = 4;
    }
    c = __popc(v & 3u);
    if (k >= c) {
        k -= c;
        v >>= 2;
        pos += 2;
    }
    return pos + ((k >= (int32_t)(v & 1u)) ? 1 : 0);
}

// sample_row_words for T <= 8 and 22 + T <= 32: the first six factors lie
// in word 0 and select within 8 bits.
NR_DEV void sample_row_words8(const KGame& g, const Row& r, const uint32_t words[4], int32_t a[7]) {
    if (only_none(r)) {
#pragma unroll
        for (int f = 0; f < 7; ++f) a[f] = 0;
        return;
    }
    const int32_t lo[6] = {0, 6, 10, 14, 18, 22};
#pragma unroll
    for (int f = 0; f < 6; ++f) {
        const int32_t wid = f == 0 ? 6 : (f == 5 ? g.T : 4);
        const uint32_t hh = (words[f >> 1] >> (16 * (f & 1))) & 0xFFFFu;
        const uint32_t m = (r.w[0] >> lo[f]) & ((1u << wid) - 1u);
        const int32_t count = __popc(m);
        a[f] = count > 0 ? select_bit8(m, (int32_t)((hh * (uint32_t)count) >> 16)) : 0;
    }
    const uint32_t hh = words[3] & 0xFFFFu;  // factor 6: low half of word 3
    const uint64_t m = row_bits(r, 22 + g.T, g.O);
    const int32_t count = popc(m);
    a[6] = count > 0 ? select_bit(m, (int32_t)((hh * (uint32_t)count) >> 16)) : 0;
}

// The sampled kind and what decode_values reads of the other factors, with
// sample_row_words8's draws: the factor of the sampled kind alone (and the
// produced type for PRODUCE) is selected, the others are not needed.  Same
// results as sample_row_words8 followed by decode_values.
NR_DEV void sample_decode8(const KGame& g, const Env& e, int32_t p, const Row& r, uint32_t w0, uint32_t w1,
                           uint32_t w2, uint32_t w3, int32_t* kind_out, int32_t* dir_out, int32_t* ptype_out,
                           int32_t* target_out, int32_t* none_out) {
    int32_t kind = kKindNone, dir = kAbsent, ptype = kAbsent, target = kAbsent;
    if (!only_none(r)) {
        const uint32_t mk = r.w[0] & 63u;
        kind = select_bit8(mk, (int32_t)(((w0 & 0xFFFFu) * (uint32_t)__popc(mk)) >> 16));
        if (kind >= kKindMove && kind <= kKindProduce) {
            // factor f = kind: bits 2 + 4f .. 5 + 4f, draw half f & 1 of word f >> 1
            const uint32_t m = (r.w[0] >> (2 + 4 * kind)) & 15u;
            uint32_t w = w1;
            if (kind == kKindMove) w = w0;
            if (kind == kKindProduce) w = w2;
            const uint32_t hh = (kind & 1) ? (w >> 16) : (w & 0xFFFFu);
            const int32_t c = __popc(m);
            dir = c > 0 ? select_bit8(m, (int32_t)((hh * (uint32_t)c) >> 16)) : 0;
            if (kind == kKindProduce) {
                const uint32_t mt = (r.w[0] >> 22) & ((1u << g.T) - 1u);
                const int32_t ct = __popc(mt);
                ptype = ct > 0 ? select_bit8(mt, (int32_t)(((w2 >> 16) * (uint32_t)ct) >> 16)) : 0;
            }
        } else if (kind == kKindAttack) {
            const uint64_t m = row_bits(r, 22 + g.T, g.O);
            const int32_t c = popc(m);
            const int32_t off = c > 0 ? select_bit(m, (int32_t)(((w3 & 0xFFFFu) * (uint32_t)c) >> 16)) : 0;
            const int32_t cell = e.cell[g.N + p];
            const int32_t tx = wadd(cell_x(g, cell), floor_mod(off, g.side) - g.radius);
            const int32_t ty = wadd(cell_y(g, cell), floor_div(off, g.side) - g.radius);
            if (tx >= 0 && tx < g.W && ty >= 0 && ty < g.H) target = ty * g.W + tx;
        }
    }
    *kind_out = kind;
    *dir_out = canon_dir(dir);
    *ptype_out = canon_ptype(ptype, g.T);
    *target_out = target;
    *none_out = kind == kKindNone ? 1 : 0;
}

// legality_row_bm for boards of at most 32 columns (one bitmap word per
// row) with the disk table: the four neighbours and the attack window come
// from whole-row words.  Same bits as legality_row_bm.
// The unit types each player can afford at its current balance, bit t for
// type t (the produce factor's validity, N/core/kinds/produce.py:25-35):
// one compare per type on the first lanes, wave-uniform results.
struct Affordable {
    uint32_t player[2];
};
template <int TW = kWave>
NR_DEV Affordable affordable_types(const KGame& g, const Hdr& h, const Env& e, int lane) {
    const int32_t cost = lane < g.T ? tabv(h, F_COST, lane) : 0x7fffffff;
    Affordable a;
    a.player[0] = (uint32_t)tballot<TW>(lane < g.T && tuni<TW>(e.sc[S_RES0]) >= cost);
    a.player[1] = (uint32_t)tballot<TW>(lane < g.T && tuni<TW>(e.sc[S_RES1]) >= cost);
    return a;
}

// Columns x - 1 .. x + 1 (0 <= x < W <= 32) of a board row as bits 0 .. 2;
// with `fill` the columns off the board read as set (blocked).  Up to 30
// columns the shifted row and its fill fit one word: one bitfield extract.
NR_DEV uint32_t window3(const KGame& g, uint32_t row, uint32_t x, bool fill) {
    if (g.W <= 30) return __builtin_amdgcn_ubfe((row << 1) | (fill ? 1u | (~0u << (g.W + 1)) : 0u), x, 3u);
    const uint64_t v = ((uint64_t)row << 1) | (fill ? 1ull | (~0ull << (g.W + 1)) : 0ull);
    return (uint32_t)((v >> x) & 7ull);
}

NR_DEV Row legality_row_w1(const KGame& g, const Hdr& h, const Env& e, int32_t slot, const Affordable& aff) {
    Row r;
    r.w[0] = r.w[1] = r.w[2] = 0u;
    if (e.birth[slot] == kAbsent) return r;
    const int32_t owner = e.owner[slot];
    if (owner != 0 && owner != 1) return legality_row(g, h, e, slot);
    const int32_t actor = clampi(e.utype[slot], 0, g.T - 1);
    const int32_t carried = e.carried[slot];
    const int32_t cell = e.cell[slot];
    const int32_t info = tabv(h, F_PACK, actor);
    const int32_t flags = info & 0xFF;
    const uint32_t types = ((uint32_t)info >> 8) & 0xFFu & (owner ? aff.player[1] : aff.player[0]);
    const int32_t x = cell_x(g, cell), yy = cell_y(g, cell);
    const int32_t H = g.H;
    AS3 const uint32_t* bm = at<uint32_t>(e, g.lay.o_bm);
    AS3 const uint32_t* blk = bm;
    AS3 const uint32_t* res = bm + 3 * H;
    AS3 const uint32_t* stk = bm + (4 + owner) * H;
    const bool has_up = yy - 1 >= 0 && yy - 1 < H, has_dn = yy + 1 >= 0 && yy + 1 < H;
    const bool has_mid = yy >= 0 && yy < H;
    const int32_t ru = has_up ? yy - 1 : 0, rd = has_dn ? yy + 1 : 0, rm = has_mid ? yy : 0;
    const uint32_t b_up = has_up ? blk[ru] : 0xFFFFFFFFu, b_dn = has_dn ? blk[rd] : 0xFFFFFFFFu;
    const uint32_t b_mid = has_mid ? blk[rm] : 0xFFFFFFFFu;
    const uint32_t r_up = has_up ? res[ru] : 0u, r_dn = has_dn ? res[rd] : 0u, r_mid = has_mid ? res[rm] : 0u;
    const uint32_t s_up = has_up ? stk[ru] : 0u, s_dn = has_dn ? stk[rd] : 0u, s_mid = has_mid ? stk[rm] : 0u;
    // x - 1 .. x + 1 of the middle rows: bit 0 left, bit 2 right; off the
    // board is blocked and holds nothing
    const bool inx = x >= 0 && x < g.W;
    const uint32_t xb = inx ? (uint32_t)x : 0u;
    const uint32_t bw = inx ? window3(g, b_mid, xb, true) : 7u;
    const uint32_t rw = inx ? window3(g, r_mid, xb, false) : 0u;
    const uint32_t sw = inx ? window3(g, s_mid, xb, false) : 0u;
    const uint32_t bu = inx ? (b_up >> xb) & 1u : 1u, bd = inx ? (b_dn >> xb) & 1u : 1u;
    const uint32_t blocked4 = bu | (((bw >> 2) & 1u) << 1) | (bd << 2) | ((bw & 1u) << 3);
    const uint32_t free4 = ~blocked4 & 15u;
    const uint32_t res4 = inx ? (((r_up >> xb) & 1u) | (((rw >> 2) & 1u) << 1) | (((r_dn >> xb) & 1u) << 2) |
                                 ((rw & 1u) << 3))
                              : 0u;
    const uint32_t stk4 = inx ? (((s_up >> xb) & 1u) | (((sw >> 2) & 1u) << 1) | (((s_dn >> xb) & 1u) << 2) |
                                 ((sw & 1u) << 3))
                              : 0u;
    r.w[0] = 1u;  // NONE
    if (flags & FL_MOVE) r.w[0] |= free4 << 6;
    if ((flags & FL_HARVEST) && carried == 0) r.w[0] |= res4 << 10;
    if ((flags & FL_HARVEST) && carried > 0) r.w[0] |= stk4 << 14;
    if (types != 0u) r.w[0] |= free4 << 18;
    const uint32_t produce_types = free4 != 0u ? types : 0u;
    r.w[0] |= produce_types << 22;
    r.w[0] |= ((r.w[0] >> 6) & 15u ? 1u : 0u) << kKindMove;
    r.w[0] |= ((r.w[0] >> 10) & 15u ? 1u : 0u) << kKindHarvest;
    r.w[0] |= ((r.w[0] >> 14) & 15u ? 1u : 0u) << kKindReturn;
    r.w[0] |= (produce_types ? 1u : 0u) << kKindProduce;
    if (flags & FL_ATTACK) {
        const int32_t range = info >> 16;
        const int32_t reach = imin(range, g.radius);
        AS3 const uint32_t* enemy = bm + (2 - owner) * H;
        uint64_t att = 0;
        if (range == 1 && g.radius >= 1 && inx) {
            // range 1: the four neighbours (the unit's own cell never holds
            // an enemy), read like the move directions
            const uint32_t e_up = has_up ? enemy[ru] : 0u, e_dn = has_dn ? enemy[rd] : 0u;
            const uint32_t ew = window3(g, has_mid ? enemy[rm] : 0u, xb, false);
            const int32_t c0 = g.radius * g.side + g.radius;
            att = ((uint64_t)((e_up >> xb) & 1u) << (c0 - g.side)) | ((uint64_t)(ew & 1u) << (c0 - 1)) |
                  ((uint64_t)((ew >> 2) & 1u) << (c0 + 1)) | ((uint64_t)((e_dn >> xb) & 1u) << (c0 + g.side));
        } else if (range >= 0 && range <= g.disk_r && inx) {
            AS3 const uint32_t* disk = h.disk + range * (2 * g.disk_r + 1) + g.disk_r;
            const uint32_t window = (2u << (2 * reach)) - 1u;
            const int32_t left = x - reach;
            for (int32_t dy = -g.radius; dy <= g.radius; ++dy) {
                const int32_t ty = yy + dy;
                if (dy < -reach || dy > reach || ty < 0 || ty >= H) continue;
                const uint32_t row = enemy[ty];
                const uint32_t span = (disk[dy] >> (g.disk_r - reach)) & window;
                const uint32_t bits = (left >= 0 ? (row >> left) : (row << (-left))) & span;
                att |= (uint64_t)bits << ((g.radius + dy) * g.side + g.radius - reach);
            }
        } else {
            // general window (never taken for the shipped unit tables)
            return legality_row_bm(g, h, e, slot);
        }
        if (att != 0ull) {
            r.w[0] |= 1u << kKindAttack;
            const int32_t first = 22 + g.T;  // < 32
            r.w[0] |= (uint32_t)(att << first);
            r.w[1] |= (uint32_t)(att >> (32 - first));
            r.w[2] |= (uint32_t)(att >> (64 - first));
        }
    }
    return r;
}

// k-th set bit (0-based, below the count) of a 4-bit mask from a table of
// each mask's set-bit positions in increasing order, two bits apiece: byte m
// of the 128-bit table, masks 0-7 in the low word, 8-15 in the high word.
constexpr uint64_t select4_table(int half) {
    uint64_t t = 0;
    for (int i = 0; i < 8; ++i) {
        const int m = half * 8 + i;
        uint64_t byte = 0;
        int j = 0;
        for (int b = 0; b < 4; ++b)
            if ((m >> b) & 1) byte |= (uint64_t)b << (2 * j++);
        t |= byte << (8 * i);
    }
    return t;
}
NR_DEV int32_t select4(uint32_t m, int32_t k) {
    const uint64_t t = (m & 8u) ? select4_table(1) : select4_table(0);
    return (int32_t)((t >> (((m & 7u) << 3) | ((uint32_t)k << 1))) & 3u);
}

// legality_row_w1 and sample_decode8 in one pass, for a unit of player 0 or
// 1 on the board whose attack range is 1 (or that cannot attack), on boards
// of at most 32 columns with T <= 8: every factor it can sample is a 4-bit
// mask over the four neighbours, so the row is never assembled and the
// attack target follows from the neighbour drawn.  Same draws and results as
// the two functions; returns false, writing nothing, for any other unit.
// The range-1 attack window holds the four neighbours at offsets
// c0 - side, c0 - 1, c0 + 1, c0 + side (c0 its centre): in offset order up,
// left, right, down.
NR_DEV bool sample_unit_w1(const KGame& g, const Hdr& h, const Env& e, int32_t p, const Affordable& aff, uint32_t w0,
                           uint32_t w1, uint32_t w2, uint32_t w3, int32_t* kind_out, int32_t* dir_out,
                           int32_t* ptype_out, int32_t* target_out, int32_t* none_out) {
    const int32_t slot = g.N + p;
    if (e.birth[slot] == kAbsent) return false;
    const int32_t owner = e.owner[slot];
    if (owner != 0 && owner != 1) return false;
    const int32_t actor = clampi(e.utype[slot], 0, g.T - 1);
    const int32_t info = tabv(h, F_PACK, actor);
    const int32_t flags = info & 0xFF;
    if ((flags & FL_ATTACK) && !((info >> 16) == 1 && g.radius >= 1)) return false;
    const int32_t cell = e.cell[slot];
    const int32_t x = cell_x(g, cell), yy = cell_y(g, cell);
    const int32_t H = g.H;
    if (x < 0 || x >= g.W || yy < 0 || yy >= H) return false;
    const int32_t carried = e.carried[slot];
    const uint32_t types = ((uint32_t)info >> 8) & 0xFFu & (owner ? aff.player[1] : aff.player[0]);
    AS3 const uint32_t* bm = at<uint32_t>(e, g.lay.o_bm);
    AS3 const uint32_t* res = bm + 3 * H;
    AS3 const uint32_t* stk = bm + (4 + owner) * H;
    AS3 const uint32_t* enemy = bm + (2 - owner) * H;
    const bool has_up = yy >= 1, has_dn = yy + 1 < H;
    const int32_t ru = has_up ? yy - 1 : 0, rd = has_dn ? yy + 1 : 0;
    // rows above and below: the unit's column; off the board is blocked and
    // holds nothing
    const uint32_t b_up = has_up ? bm[ru] : 0xFFFFFFFFu, b_dn = has_dn ? bm[rd] : 0xFFFFFFFFu;
    const uint32_t r_up = has_up ? res[ru] : 0u, r_dn = has_dn ? res[rd] : 0u;
    const uint32_t s_up = has_up ? stk[ru] : 0u, s_dn = has_dn ? stk[rd] : 0u;
    const uint32_t e_up = has_up ? enemy[ru] : 0u, e_dn = has_dn ? enemy[rd] : 0u;
    // the unit's row: columns x - 1 .. x + 1 as bits 0 .. 2
    const uint32_t xb = (uint32_t)x;
    const uint32_t bw = window3(g, bm[yy], xb, true), rw = window3(g, res[yy], xb, false);
    const uint32_t sw = window3(g, stk[yy], xb, false), ew = window3(g, enemy[yy], xb, false);
    // directions 0 up, 1 right, 2 down, 3 left
    const uint32_t blocked4 = ((b_up >> xb) & 1u) | (((bw >> 2) & 1u) << 1) | (((b_dn >> xb) & 1u) << 2) | ((bw & 1u) << 3);
    const uint32_t free4 = ~blocked4 & 15u;
    const uint32_t res4 = ((r_up >> xb) & 1u) | (((rw >> 2) & 1u) << 1) | (((r_dn >> xb) & 1u) << 2) | ((rw & 1u) << 3);
    const uint32_t stk4 = ((s_up >> xb) & 1u) | (((sw >> 2) & 1u) << 1) | (((s_dn >> xb) & 1u) << 2) | ((sw & 1u) << 3);
    // attack offsets in window order: up, left, right, down
    const uint32_t att4 = (flags & FL_ATTACK) ? (((e_up >> xb) & 1u) | ((ew & 1u) << 1) | (((ew >> 2) & 1u) << 2) |
                                                 (((e_dn >> xb) & 1u) << 3))
                                              : 0u;
    const uint32_t mk = 1u | (((flags & FL_MOVE) && free4) ? 2u : 0u) |
                        (((flags & FL_HARVEST) && carried == 0 && res4) ? 4u : 0u) |
                        (((flags & FL_HARVEST) && carried > 0 && stk4) ? 8u : 0u) | ((types && free4) ? 16u : 0u) |
                        (att4 ? 32u : 0u);
    int32_t kind = kKindNone, dir = kAbsent, ptype = kAbsent, target = kAbsent;
    if (mk != 1u) {
        kind = select_bit8(mk, (int32_t)(((w0 & 0xFFFFu) * (uint32_t)__popc(mk)) >> 16));
        if (kind >= kKindMove && kind <= kKindProduce) {
            const uint32_t m = kind == kKindHarvest ? res4 : (kind == kKindReturn ? stk4 : free4);
            uint32_t w = w1;
            if (kind == kKindMove) w = w0;
            if (kind == kKindProduce) w = w2;
            const uint32_t hh = (kind & 1) ? (w >> 16) : (w & 0xFFFFu);
            dir = select4(m, (int32_t)((hh * (uint32_t)__popc(m)) >> 16));
            if (kind == kKindProduce)
                ptype = select_bit8(types, (int32_t)(((w2 >> 16) * (uint32_t)__popc(types)) >> 16));
        } else if (kind == kKindAttack) {
            const int32_t j = select4(att4, (int32_t)(((w3 & 0xFFFFu) * (uint32_t)__popc(att4)) >> 16));
            const int32_t tx = x + (j == 1 ? -1 : (j == 2 ? 1 : 0)), ty = yy + (j == 0 ? -1 : (j == 3 ? 1 : 0));
            if (tx >= 0 && tx < g.W && ty >= 0 && ty < H) target = ty * g.W + tx;
        }
    }
    *kind_out = kind;
    *dir_out = dir;
    *ptype_out = ptype;
    *target_out = target;
    *none_out = kind == kKindNone ? 1 : 0;
    return true;
}

// Pass over the slots: occupant words, available list, unit list, and (with
// `bitmaps`) the six occupancy bitmaps of the next cycle's masks, stamped per
// live slot over the wall rows: 0 blocked (occupied or wall), 1 / 2 units of
// player 0 / 1, 3 resources, 4 / 5 stockpiles of player 0 / 1.
// What the slot pass lists, wave-uniform, for callers that keep it in
// registers into the next cycle rather than reading it back from the env.
struct SlotSummary {
    int32_t nav, nunits, nA, nlive;
    bool irregular;
    // this lane's live slot (live_lanes) for at most a wave of them in the
    // low half, and, for half-wave teams, its second for at most two halves
    // of them in the high half (slots are below 2^15): one register to carry
    // into the next cycle
    int32_t live_slots;
    // slot window (KGame::shift > 0): a unit spawned in the next cycle could
    // land past a player's window (its units plus the units that may spawn
    // one in that cycle exceed C: a pending PRODUCE due then, and, where a
    // PRODUCE can complete in the cycle it is issued, every available unit
    // that produces)
    bool full;
};

// The live lanes a summary carries (its count and this lane's slots).
NR_DEV LiveLanes summary_live(const SlotSummary& sm) {
    return LiveLanes{sm.nlive, (int32_t)(int16_t)(sm.live_slots & 0xffff), sm.live_slots >> 16};
}

template <int TW = kWave>
NR_DEV SlotSummary summarize_slots(const KGame& g, const Hdr& h, const Env& e_in, int lane, bool bitmaps = true) {
    const Env e = refresh<TW>(g, e_in);
    const Layout& y = g.lay;
    const int32_t words = g.seen_words, plane = g.H * words;
    AS3 uint32_t* bm = at<uint32_t>(e, y.o_bm);
    if (bitmaps) {
        // the blocked plane starts from the wall rows, the other five empty
        if ((plane & 3) == 0) {
            // 16 bytes a lane (both regions are 16-byte aligned)
            const int32_t n4 = (6 * plane) >> 2, w4 = plane >> 2;
            for (int32_t i = lane; i < n4; i += TW) {
                u32x4 v = {0u, 0u, 0u, 0u};
                if (i < w4) v = ((AS3 const u32x4*)h.walls)[i];
                ((AS3 u32x4*)bm)[i] = v;
            }
        } else {
            for (int32_t i = lane; i < 6 * plane; i += TW) bm[i] = i < plane ? h.walls[i] : 0u;
        }
        wave_sync();
    }
    AS3 uint32_t* olo = at<uint32_t>(e, y.o_lo);
    AS3 uint8_t* ofl = at<uint8_t>(e, y.o_fl);
    AS3 int16_t* av = at<int16_t>(e, y.a_av);
    AS3 int16_t* units = at<int16_t>(e, y.b_units);
    AS3 int16_t* entries = at<int16_t>(e, y.a_list);
    const int32_t time = tuni<TW>(e.sc[S_TIME]);
    const int32_t next_order = tuni<TW>(e.sc[S_NEXT_ORDER]);
    // only live slots hold units or pending actions
    const LiveLanes ll = live_lanes<TW>(g, e, lane);
    const int32_t nlive = ll.count;
    int32_t nav = 0, nunits = 0, nA = 0, reach0 = 0, reach1 = 0;
    // a PRODUCE issued in a cycle can complete in it (a produce time below 2,
    // or a completion time that wraps)
    const bool quick = g.quick_produce || time > 0x3fffffff;
    bool odd = false;
    for (int32_t base = 0; base < nlive; base += TW) {
        const int32_t i = base + lane;
        // (a half-wave team takes up to two live slots a lane from live_lanes)
        const int32_t s = i < nlive ? (nlive <= TW ? ll.slot
                                                   : (TW != kWave && nlive <= 2 * TW ? (base == 0 ? ll.slot : ll.slot2)
                                                                                     : live_slot_at(g, e, i)))
                                    : 0;
        bool alive = false, available = false, entry = false, grows = false;
        if (i < nlive) {
            // pending entries for the env-path admission: MOVE / PRODUCE
            // pending from earlier cycles, in slot order (see admit_env)
            const int32_t k = e.pkind[s];
            if (k != kAbsent) {
                const int32_t ord = e.porder[s];
                if (s < g.N || ord == kAbsent || ord >= next_order) odd = true;
                if (k == kKindMove || k == kKindProduce) {
                    entry = true;
                    if (e.pissued[s] == time) odd = true;
                }
            }
            alive = e.birth[s] != kAbsent;
            if (g.shift > 0 && alive && s >= g.N) {
                // completion in the next cycle takes pending actions due by
                // time + 1; spawning into the lowest free slot of a block of
                // u units lands at most at index u
                if (k == kKindProduce) grows = e.pcompl[s] <= wadd(time, 1);
                else if (k == kAbsent && quick)
                    grows = tabv(h, F_PRODUCES, clampi(e.utype[s], 0, g.T - 1)) != 0;
            }
            if (alive) {
                // occupant word: hp | carried << 8 | owner' << 16 | pending
                // kind << 18 | (type + 1) << 24, owner' = 1 player 0, 2
                // player 1, 0 neutral; plane flags: bit 0 occupied, 1 / 2
                // unit of player 0 / 1, 3 resource, 4 / 5 stockpile of player
                // 0 / 1 (the rows of the occupancy bitmaps)
                const int32_t ty = e.utype[s];
                const int32_t ow = e.owner[s];
                const uint32_t rel0 = ow == 0 ? 1u : (ow == 1 ? 2u : 0u);
                const int32_t pk = e.pkind[s];
                olo[s] = ((uint32_t)(int32_t)e.hp[s] & 0xFFu) | (((uint32_t)e.carried[s] & 0xFFu) << 8) |
                         (rel0 << 16) | ((uint32_t)((pk > 0 ? pk : 0) & 7) << 18) |
                         (((uint32_t)(ty + 1) & 0xFFu) << 24);
                const int32_t fl = tabv(h, F_FLAGS, clampi(ty, 0, g.T - 1));
                const uint32_t stk = (fl & FL_STOCKPILE) ? 1u : 0u;
                const uint32_t planes = 1u | (rel0 << 1) | ((fl & FL_RESOURCE) ? 8u : 0u) | ((stk & (rel0 & 1u)) << 4) |
                                        ((stk & (rel0 >> 1)) << 5);
                ofl[s] = (uint8_t)planes;
                if (bitmaps) {
                    const int32_t c = e.cell[s];
                    const int32_t cy = cell_y(g, c), cx = c - cy * g.W;
                    AS3 uint32_t* at_ = bm + cy * words + (cx >> 5);
                    const uint32_t bit = 1u << (cx & 31);
                    // the planes it names, at most one of each pair: occupied,
                    // its player's units (1 or 2), resource (3), its
                    // player's stockpiles (4 or 5); an OR of 0 where a
                    // plane is not named
                    __atomic_fetch_or(at_, bit, __ATOMIC_RELAXED);
                    __atomic_fetch_or(at_ + (rel0 == 2u ? 2 : 1) * plane, rel0 != 0u ? bit : 0u, __ATOMIC_RELAXED);
                    __atomic_fetch_or(at_ + 3 * plane, (planes & 8u) ? bit : 0u, __ATOMIC_RELAXED);
                    __atomic_fetch_or(at_ + (rel0 == 2u ? 5 : 4) * plane, (planes & 48u) ? bit : 0u,
                                      __ATOMIC_RELAXED);
                }
                available = s >= g.N && pk == kAbsent;
                if (available && e.porder[s] != kAbsent) odd = true;
            }
        }
        const bool unit = alive && s >= g.N;
        const uint64_t me = tballot<TW>(entry);
        if (entry && nA + tcount_below<TW>(me) < kWave) entries[nA + tcount_below<TW>(me)] = (int16_t)s;
        nA += popc(me);
        const uint64_t ma = tballot<TW>(available);
        if (available) av[nav + tcount_below<TW>(ma)] = (int16_t)(s - g.N);
        nav += popc(ma);
        const uint64_t mu = tballot<TW>(unit);
        if (unit) {
            int32_t item = s;
            if (g.H <= 32 && g.seen_words == 1) {
                // what the sight pass reads, packed (boards of at most 32
                // columns and rows, sight radii below 31): column, row,
                // radius + 1 (0: none) and player
                const int32_t c = e.cell[s];
                const int32_t cy = cell_y(g, c), cx = c - cy * g.W;
                const int32_t r = tabv(h, F_SIGHT, gidx(e.utype[s], g.T));
                const int32_t r1 = r < 0 ? 0 : r + 1;
                item = (int32_t)((uint32_t)cx | ((uint32_t)cy << 5) | ((uint32_t)r1 << 10) |
                                 ((s - g.N) >= g.C ? 0x8000u : 0u));
            }
            units[nunits + tcount_below<TW>(mu)] = (int16_t)item;
        }
        nunits += popc(mu);
        if (g.shift > 0) {
            // each unit, and once more each that may spawn one this cycle
            const bool p1 = s >= g.N + g.C;
            reach0 += popc(tballot<TW>(unit && !p1)) + popc(tballot<TW>(grows && !p1));
            reach1 += popc(tballot<TW>(unit && p1)) + popc(tballot<TW>(grows && p1));
        }
    }
    // irregular: the env-path admission does not apply (admit_env)
    // (a half-wave team holds up to two entries a lane)
    const bool irregular = tballot<TW>(odd) != 0ull || nA > (TW == kWave ? TW : 2 * TW) ||
                           next_order > 0x7fffffff - kWave;
    if (lane == 0) {
        // the empty cell's sentinel (index E) of the occupant arrays
        olo[g.E] = 0u;
        ofl[g.E] = 0u;
        e.sc[S_NAV] = nav;
        e.sc[S_NUNITS] = nunits;
        e.sc[S_NA] = nA;
        e.sc[S_IRREG] = irregular ? 1 : 0;
    }
    wave_sync();
    SlotSummary out;
    out.nav = tuni<TW>(nav);
    out.nunits = tuni<TW>(nunits);
    out.nA = tuni<TW>(nA);
    out.nlive = nlive;
    out.irregular = irregular;
    out.live_slots = (int32_t)(((uint32_t)ll.slot & 0xffffu) | ((uint32_t)ll.slot2 << 16));
    out.full = reach0 > g.C || reach1 > g.C;
    return out;
}

// Sight disks of both players into seen[2][H][words].  With H <= 32 a lane
// takes (unit k, row) for U = 64 / H units at a time and ORs the unit's disk
// row into a per-lane accumulator of its player; the U partial rows are
// OR-ed across lanes at the end, so the bitmap is written once, without
// atomics.  Taller boards stamp (unit, dy) rows with LDS atomics.
// Sight bitmaps of the players whose bit is set in `which` (the others'
// planes are left as they are).
template <int TW = kWave>
NR_DEV void summarize_visibility(const KGame& g, const Hdr& h, const Env& e_in, int lane, int32_t seen_at,
                                 int32_t which, int32_t nunits) {
    const Env e = refresh<TW>(g, e_in);
    const Layout& y = g.lay;
    AS3 uint32_t* seen = at<uint32_t>(e, seen_at);
    const int32_t words = g.seen_words, plane = g.H * words;
    AS3 const int16_t* units = at<int16_t>(e, y.b_units);
    const int32_t R = g.disk_r, span = 2 * R + 1;
    if (g.H <= 32 && words == 1) {
        const int32_t U = TW / g.H;
        // lane / H by a 16-bit reciprocal (exact for lane < 64, H <= 32)
        const int32_t k = (int32_t)(((uint32_t)lane * ((65536u + (uint32_t)g.H - 1u) / (uint32_t)g.H)) >> 16);
        const int32_t row = lane - k * g.H;
        const uint32_t rowmask = g.W >= 32 ? 0xFFFFFFFFu : ((1u << g.W) - 1u);
        uint32_t acc0 = 0u, acc1 = 0u;
        // the listed units are player 0's, then player 1's
        const int32_t n0 = tuni<TW>(e.sc[S_UNITS0]);
        const int32_t first = (which & 1) ? 0 : n0, last = (which & 2) ? nunits : n0;
        for (int32_t base = first; base < last; base += U) {
            const int32_t i = base + k;
            if (k >= U || i >= nunits) continue;
            // the unit's column, row, sight radius and player, as the slot
            // pass packed them
            const uint32_t v = (uint16_t)units[i];
            const int32_t r = (int32_t)((v >> 10) & 31u) - 1;
            const int32_t dy = row - (int32_t)((v >> 5) & 31u);
            if (dy < -r || dy > r) continue;
            const uint32_t m = h.disk[r * span + dy + R];
            const int32_t x0 = (int32_t)(v & 31u) - R;  // in [-R, W - 1]: 32-bit shifts
            const uint32_t bits = (x0 >= 0 ? m << x0 : m >> (-x0)) & rowmask;
            if (v & 0x8000u) acc1 |= bits;
            else acc0 |= bits;
        }
        for (int32_t j = 1; j < U; ++j) {
            acc0 |= (uint32_t)__shfl((int)acc0, lane + j * g.H, TW);
            acc1 |= (uint32_t)__shfl((int)acc1, lane + j * g.H, TW);
        }
        if (lane < g.H) {
            if (which & 1) seen[lane] = acc0;
            if (which & 2) seen[plane + lane] = acc1;
        }
        wave_sync();
        return;
    }
    for (int32_t i = lane; i < 2 * plane; i += TW) seen[i] = 0u;
    wave_sync();
    for (int32_t base = 0; base < nunits; base += TW) {
        const int32_t i = base + lane;
        int32_t r = -1, cx = 0, cy = 0;
        AS3 uint32_t* mine = seen;
        if (i < nunits) {
            const int32_t s = units[i];
            r = tabv(h, F_SIGHT, gidx(e.utype[s], g.T));
            const int32_t cell = e.cell[s];
            cx = cell_x(g, cell);
            cy = cell_y(g, cell);
            mine = seen + ((s - g.N) >= g.C ? plane : 0);
        }
        AS3 const uint32_t* disk = h.disk + (r < 0 ? 0 : r) * span;
        for (int32_t dy = -R; dy <= R; ++dy) {
            const int32_t row = cy + dy;
            if (r < 0 || dy < -r || dy > r || row < 0 || row >= g.H) continue;
            const uint64_t m = disk[dy + R];
            const int32_t x0 = cx - R;
            for (int32_t wd = 0; wd < words; ++wd) {
                const int32_t sh = x0 - 32 * wd;
                uint64_t bits = sh >= 0 ? (sh < 64 ? m << sh : 0ull) : (-sh < 64 ? m >> (-sh) : 0ull);
                uint32_t b32 = (uint32_t)bits;
                const int32_t valid = g.W - 32 * wd;
                if (valid < 32) b32 &= (1u << valid) - 1u;
                if (b32 != 0u) __atomic_fetch_or(&mine[row * words + wd], b32, __ATOMIC_RELAXED);
            }
        }
    }
    wave_sync();
}

// Pass over the cells, four per lane (W % 4 == 0): bitmaps for the masks and
// both agents' feature maps.  maps0/maps1 may be null (no observation).
template <int TW = kWave>
NR_DEV void summarize_cells(const KGame& g, const Hdr& h, const Env& e_in, int lane, bool partial, bool bitmaps,
                            uint8_t* maps0, uint8_t* maps1, int32_t seen_at) {
    const Env e = refresh<TW>(g, e_in);
    const Layout& y = g.lay;
    const int32_t words = g.seen_words, plane = g.H * words;
    AS3 uint32_t* bm = at<uint32_t>(e, y.o_bm);
    if (bitmaps) {
        for (int32_t i = lane; i < 6 * plane; i += TW) bm[i] = 0u;
        wave_sync();
    }
    AS3 const uint32_t* olo = at<uint32_t>(e, y.o_lo);
    AS3 const uint8_t* ofl = at<uint8_t>(e, y.o_fl);
    AS3 const uint32_t* seen = at<uint32_t>(e, seen_at);
    const bool obs = maps0 != nullptr;
    // bits 0, 8, 16, 24 of x -> bits 0..3
    auto nibble = [](uint32_t x) {
        x |= x >> 7;
        x |= x >> 14;
        return x & 15u;
    };
    for (int32_t base = 0; base < g.cells; base += 4 * TW) {
        const int32_t c0 = base + 4 * lane;
        if (c0 >= g.cells) continue;
        const uint64_t ent = *(AS3 const uint64_t*)(e.entity + c0);
        const uint32_t ter = *(AS3 const uint32_t*)(h.terrain + c0);  // one 0/1 byte per cell
        const int32_t yy = cell_y(g, c0), x = c0 - yy * g.W;
        const int32_t word = yy * words + (x >> 5), shift = x & 31;
        // the occupants' words and flags; an empty cell reads the zero
        // sentinel at index E (ABSENT -> 0xFFFFFFFF -> min E)
        uint32_t lo[4], F = 0u;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t idx = __builtin_elementwise_min((uint32_t)(int32_t)(int16_t)(uint16_t)(ent >> (16 * k)),
                                                           (uint32_t)g.E);
            lo[k] = olo[idx];
            F |= (uint32_t)ofl[idx] << (8 * k);
        }
        const uint32_t occ_n = nibble((F & 0x01010101u) | ter);
        const uint32_t p0_n = nibble((F >> 1) & 0x01010101u), p1_n = nibble((F >> 2) & 0x01010101u);
        if (bitmaps) {
            const uint32_t res_n = nibble((F >> 3) & 0x01010101u);
            const uint32_t stk0_n = nibble((F >> 4) & 0x01010101u), stk1_n = nibble((F >> 5) & 0x01010101u);
            if (occ_n) __atomic_fetch_or(&bm[word], occ_n << shift, __ATOMIC_RELAXED);
            if (p0_n) __atomic_fetch_or(&bm[plane + word], p0_n << shift, __ATOMIC_RELAXED);
            if (p1_n) __atomic_fetch_or(&bm[2 * plane + word], p1_n << shift, __ATOMIC_RELAXED);
            if (res_n) __atomic_fetch_or(&bm[3 * plane + word], res_n << shift, __ATOMIC_RELAXED);
            if (stk0_n) __atomic_fetch_or(&bm[4 * plane + word], stk0_n << shift, __ATOMIC_RELAXED);
            if (stk1_n) __atomic_fetch_or(&bm[5 * plane + word], stk1_n << shift, __ATOMIC_RELAXED);
        }
        if (!obs) continue;
        // per cell: the word without the kind bits, the kind byte and the
        // terrain byte (shown to both players)
        uint32_t clean[4], kindb[4], terb[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            clean[k] = lo[k] & ~(7u << 18);
            kindb[k] = (lo[k] >> 18) & 7u;
            terb[k] = ((ter >> (8 * k)) & 0xFFu) << 8;
        }
        const uint32_t owned_n = p0_n | p1_n;
#pragma unroll
        for (int32_t pl = 0; pl < 2; ++pl) {
            const uint32_t own = pl == 0 ? p0_n : p1_n;
            const uint32_t vis = partial ? ((seen[pl * plane + word] >> shift) & 15u) | own : 15u;
            uint32_t l4[4], h4[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const bool shown = (vis >> k) & 1u;
                // player 1 sees owners 1 <-> 2 swapped (neutral stays 0)
                const uint32_t v = pl == 1 ? clean[k] ^ (((owned_n >> k) & 1u) ? (3u << 16) : 0u) : clean[k];
                l4[k] = shown ? v : 0u;
                h4[k] = (shown ? kindb[k] : 0u) | terb[k];
            }
            uint64_t* dst = (uint64_t*)((pl == 0 ? maps0 : maps1) + (int64_t)c0 * 6);
            dst[0] = (uint64_t)l4[0] | ((uint64_t)(h4[0] | (l4[1] << 16)) << 32);
            dst[1] = (uint64_t)((l4[1] >> 16) | (h4[1] << 16)) | ((uint64_t)l4[2] << 32);
            dst[2] = (uint64_t)(h4[2] | (l4[3] << 16)) | ((uint64_t)((l4[3] >> 16) | (h4[3] << 16)) << 32);
        }
    }
    wave_sync();
}

// The summary of the current state; the observation is written when
// maps0/maps1 are given (8-byte aligned), scalars when scalars0/1 are.
// `kept_seen` >= 0 is the LDS offset of sight bitmaps kept from the last
// summary: they are stamped again only for a state whose units moved,
// spawned or died since (S_VISDIRTY).
template <int TW = kWave>
NR_DEV SlotSummary summarize(const KGame& g, const Hdr& h, const Env& e, int lane, bool partial, uint8_t* maps0,
                             uint8_t* maps1, int32_t* scalars0, int32_t* scalars1, int32_t kept_seen = -1) {
    const SlotSummary sm = summarize_slots<TW>(g, h, e, lane);
    const int32_t seen_at = kept_seen >= 0 ? kept_seen : g.lay.v_seen;
    const int32_t which = kept_seen >= 0 ? tuni<TW>(e.sc[S_VISDIRTY]) & 3 : 3;
    if (partial && maps0 && which != 0) {
        summarize_visibility<TW>(g, h, e, lane, seen_at, which, sm.nunits);
        if (kept_seen >= 0 && lane == 0) e.sc[S_VISDIRTY] = 0;
    }
    if (maps0) summarize_cells<TW>(g, h, e, lane, partial, false, maps0, maps1, seen_at);
    if (scalars0 && lane < 8) {
        const int32_t pl = lane >> 2, f = lane & 3;
        int32_t v;
        if (f == 0) v = e.sc[S_RES0 + pl];
        else if (f == 1) v = e.sc[S_RES0 + (pl ^ 1)];
        else if (f == 2) v = e.sc[S_TIME];
        else v = e.sc[S_ALT];
        (pl == 0 ? scalars0 : scalars1)[f] = v;
    }
    return sm;
}

// The available owned positions in slot order (the summary's list, again,
// for a state the summary already saw); returns their count.
template <int TW = kWave>
NR_DEV int32_t list_available(const KGame& g, const Env& e_in, int lane) {
    const Env e = refresh<TW>(g, e_in);
    AS3 int16_t* av = at<int16_t>(e, g.lay.a_av);
    int32_t n = 0;
    for (int32_t base = 0; base < 2 * g.C; base += TW) {
        const int32_t p = base + lane;
        const bool available = p < 2 * g.C && e.birth[g.N + p] != kAbsent && e.pkind[g.N + p] == kAbsent;
        const uint64_t m = tballot<TW>(available);
        if (available) av[n + tcount_below<TW>(m)] = (int16_t)p;
        n += popc(m);
    }
    wave_sync();
    return n;
}

// Commands of the positions the summary did not list as available.
template <int TW = kWave>
NR_DEV void mark_unavailable(const KGame& g, const Env& e_in, int lane) {
    const Env e = refresh<TW>(g, e_in);
    const Layout& y = g.lay;
    AS3 int8_t* ckind = at<int8_t>(e, y.c_kind);
    AS3 int16_t* crank = at<int16_t>(e, y.c_rank);
    for (int32_t p = lane; p < 2 * g.C; p += TW) {
        const int32_t s = g.N + p;
        if (!(e.birth[s] != kAbsent && e.pkind[s] == kAbsent)) ckind[p] = (int8_t)kAbsent;
        crank[p] = 0;
    }
    wave_sync();
}

}  // namespace nr
