// The GridNet surface (MicroRTS-Py's per-cell interface) for one wave per
// game: per-cell action decode with the source filter
// (N/adapters/gridnet/actions.py, source_filter.py) and the observation
// planes, source mask and action mask (N/adapters/gridnet/observation.py).
//
// The decode keeps, per player and in cell order, the rows whose claimed
// position is still free and whose cost does not overdraw a player already
// spending; the walk is sequential, as the reference's lax.while_loop is.
// Its scratch lies in the env block's phase union after the command arrays.
#pragma once

#include "engine.h"

namespace nr {

// Offsets of the decode scratch (from the env block), computed on the host.
struct GridLayout {
    int32_t origin, bytes;
    int32_t order;  // int16 [C]: available own units by cell
    int32_t list;   // int16 [C]: the same units in slot order
    int32_t pos;    // int16 [C]: claimed position + W, -1 for none
    int32_t cost;   // int32 [C]
    int32_t kept;   // uint8 [C]
    int32_t base;   // uint32 [words]: pending claims (+ player 0's issued ones)
    int32_t used;   // uint32 [words]: the filter's working copy
};

// Observation buffers (see nanorts_gridnet_obs in the C header).
constexpr int32_t kPlaneCount = 29;  // one-hot widths 5, 5, 3, 8, 6, 2
constexpr int32_t kMaskWidth = 78;

template <typename T>
NR_DEV AS3 T* gat(const Env& e, const GridLayout& y, int32_t offset) {
    return (AS3 T*)(e.base + y.origin + offset);
}

// The word is chosen by selects: an index into the row's array, different in
// each lane, would put the row in private memory.
NR_DEV bool row_bit(const Row& r, int32_t b) {
    const int32_t w = b >> 5;
    const uint32_t word = w == 0 ? r.w[0] : (w == 1 ? r.w[1] : r.w[2]);
    return (word >> (b & 31)) & 1u;
}

// source_filter.direction_delta (N/adapters/gridnet/source_filter.py:51-58)
NR_DEV int32_t grid_delta(int32_t direction, int32_t W) {
    if (direction < 0 || direction > 3) return 0;
    return dir_dx(direction) + dir_dy(direction) * W;
}

// One decoded row (factors.direction / produced_type / attack_target,
// N/adapters/factors.py:117-151; none -1 for NONE, actions.py:115).
struct GridRow {
    int32_t kind, dir, none, target, ptype;
};

NR_DEV GridRow grid_row(const KGame& g, const int32_t* row, int32_t at_cell) {
    GridRow r;
    r.kind = row[0];
    r.dir = r.kind == kKindMove      ? row[1]
            : r.kind == kKindHarvest ? row[2]
            : r.kind == kKindReturn  ? row[3]
            : r.kind == kKindProduce ? row[4]
                                     : kAbsent;
    r.ptype = r.kind == kKindProduce ? row[5] : kAbsent;
    const int32_t tx = wadd(floor_mod(at_cell, g.W), floor_mod(row[6], g.side) - g.radius);
    const int32_t ty = wadd(floor_div(at_cell, g.W), floor_div(row[6], g.side) - g.radius);
    r.target = (r.kind == kKindAttack && tx >= 0 && tx < g.W && ty >= 0 && ty < g.H) ? ty * g.W + tx : kAbsent;
    r.none = r.kind == kKindNone ? -1 : 0;
    return r;
}

// decode_actions (N/adapters/gridnet/actions.py:31-52, 91-184;
// source_filter.py:61-139) of one env.  `acts` is the env's
// [players][cells][7] block; `sink(p, kind, dir, none, target, ptype, order)`
// receives every owned position p of the first `players` players once
// (players 1: player 0 alone, whose decode never reads player 1's rows).
// `legal(i, r)` tells whether player 0's kept row r of its unit at position
// i (slot N + i) is legal, the issued usage's filter (:124-139).
template <typename Sink, typename Legal>
NR_DEV void gridnet_decode_by(const KGame& g, const Hdr& h, const Env& e, const GridLayout& y, const int32_t* acts,
                              int32_t players, int lane, Sink sink, Legal legal) {
    const int32_t W = g.W, cells = g.cells, C = g.C, T = g.T;
    const int32_t domain = cells + 2 * W + 1, words = (domain + 31) / 32, margin = W;
    AS3 uint32_t* base = gat<uint32_t>(e, y, y.base);
    AS3 uint32_t* used = gat<uint32_t>(e, y, y.used);
    AS3 int16_t* order = gat<int16_t>(e, y, y.order);
    AS3 int16_t* list = gat<int16_t>(e, y, y.list);
    AS3 int16_t* pos = gat<int16_t>(e, y, y.pos);
    AS3 int32_t* cost = gat<int32_t>(e, y, y.cost);
    // kept[k]: 0 dropped, 1 kept, 2 kept but submitted no kind (an ABSENT
    // kind survives the filter, counts as a survivor and still waits as an
    // idle filler, actions.py:154-157)
    AS3 uint8_t* kept = gat<uint8_t>(e, y, y.kept);
    for (int32_t w = lane; w < words; w += kWave) base[w] = 0u;
    wave_sync();
    // pending_usage (:61-85)
    int32_t p0 = 0, p1 = 0;
    for (int32_t s = lane; s < g.E; s += kWave) {
        if (e.birth[s] == kAbsent) continue;
        const int32_t k = e.pkind[s];
        if (k == kKindMove || k == kKindProduce) {
            const int32_t idx = e.cell[s] + grid_delta(e.pdir[s], W) + margin;
            if (idx >= 0 && idx < domain - 1) __atomic_fetch_or(&base[idx >> 5], 1u << (idx & 31), __ATOMIC_RELAXED);
        }
        if (k == kKindProduce && s >= g.N) {
            const int32_t c = tabv(h, F_COST, gidx(e.pptype[s], T));
            if (s < g.N + C) p0 = wadd(p0, c);
            else p1 = wadd(p1, c);
        }
    }
    int32_t base0 = 0, base1 = 0;
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) {
        p0 = wadd(p0, __shfl_xor(p0, d, kWave));
        p1 = wadd(p1, __shfl_xor(p1, d, kWave));
    }
    base0 = p0;
    base1 = p1;
    const int32_t res0 = uni(e.sc[S_RES0]), res1 = uni(e.sc[S_RES1]);
    wave_sync();
    for (int32_t player = 0; player < players; ++player) {
        const int32_t first = g.N + player * C;
        // _decode_rows: the available units, sorted by cell
        int32_t n = 0;
        for (int32_t i0 = 0; i0 < C; i0 += kWave) {
            const int32_t i = i0 + lane;
            const bool av = i < C && e.birth[first + i] != kAbsent && e.pkind[first + i] == kAbsent;
            const uint64_t m = ballot(av);
            if (av) list[n + count_below(m)] = (int16_t)i;
            n += popc(m);
        }
        wave_sync();
        for (int32_t k = lane; k < n; k += kWave) {
            const int32_t ck = e.cell[first + list[k]];
            int32_t r = 0;
            for (int32_t q = 0; q < n; ++q) r += e.cell[first + list[q]] < ck ? 1 : 0;
            order[r] = list[k];
        }
        wave_sync();
        for (int32_t k = lane; k < n; k += kWave) {
            const int32_t at = e.cell[first + order[k]];
            const GridRow r = grid_row(g, acts + ((int64_t)player * cells + clampi(at, 0, cells - 1)) * 7, at);
            const bool claims = r.kind == kKindMove || r.kind == kKindProduce;
            pos[k] = (int16_t)(claims ? wadd(wadd(at, grid_delta(r.dir, W)), margin) : -1);
            cost[k] = r.kind == kKindProduce ? tabv(h, F_COST, gidx(r.ptype, T)) : 0;
            kept[k] = r.kind == kAbsent ? 2 : 0;
        }
        for (int32_t w = lane; w < words; w += kWave) used[w] = base[w];
        wave_sync();
        // keep (:88-121), in cell order
        int32_t s0 = base0, s1 = base1;
        for (int32_t k = 0; k < n; ++k) {
            const int32_t pk = uni(pos[k]), ck = uni(cost[k]);
            const int32_t t0 = wadd(s0, player == 0 ? ck : 0), t1 = wadd(s1, player == 1 ? ck : 0);
            const bool over = (s0 != 0 && t0 > 0 && t0 > res0) || (s1 != 0 && t1 > 0 && t1 > res1);
            const bool taken = pk >= 0 && ((used[pk >> 5] >> (pk & 31)) & 1u);
            const bool consistent = !taken && !over;
            if (lane == 0) {
                kept[k] = consistent ? (kept[k] == 2 ? 2 : 1) : 0;
                if (consistent && pk >= 0) used[pk >> 5] |= 1u << (pk & 31);
            }
            if (consistent) {
                s0 = t0;
                s1 = t1;
            }
            wave_sync();
        }
        // issued_usage (:124-139): player 0's kept legal claims seed player 1
        if (player == 0 && players > 1) {
            int32_t produced = 0;
            for (int32_t k = lane; k < n; k += kWave) {
                const int32_t pk = pos[k];
                if (!kept[k] || pk < 0) continue;
                const int32_t i = order[k];
                const int32_t at = e.cell[first + i];
                const int32_t* row = acts + ((int64_t)player * cells + clampi(at, 0, cells - 1)) * 7;
                const GridRow r = grid_row(g, row, at);
                if (!legal(i, r)) continue;
                if (pk < domain - 1) __atomic_fetch_or(&base[pk >> 5], 1u << (pk & 31), __ATOMIC_RELAXED);
                if (r.kind == kKindProduce) produced = wadd(produced, cost[k]);
            }
#pragma unroll
            for (int d = 32; d >= 1; d >>= 1) produced = wadd(produced, __shfl_xor(produced, d, kWave));
            base0 = wadd(base0, produced);
            wave_sync();
        }
        // _player_commands: unavailable rows absent; kept rows ranked in cell
        // order; the others wait as NONE fillers ranked by birth after them
        for (int32_t i = lane; i < C; i += kWave) {
            const int32_t s = first + i;
            if (e.birth[s] != kAbsent && e.pkind[s] == kAbsent) continue;
            sink(player * C + i, kAbsent, kAbsent, 0, kAbsent, kAbsent, kAbsent);
        }
        int32_t survivors = 0;
        for (int32_t k0 = 0; k0 < n; k0 += kWave) survivors += popc(ballot(k0 + lane < n && kept[k0 + lane] != 0));
        for (int32_t k = lane; k < n; k += kWave) {
            const int32_t i = order[k], slot = first + i;
            if (kept[k] == 1) {
                int32_t rank = 0;
                for (int32_t q = 0; q < k; ++q) rank += kept[q] != 0 ? 1 : 0;
                const int32_t at = e.cell[slot];
                const GridRow r = grid_row(g, acts + ((int64_t)player * cells + clampi(at, 0, cells - 1)) * 7, at);
                sink(player * C + i, r.kind, r.dir, r.none, r.target, r.ptype, rank);
            } else {
                const int32_t bi = e.birth[slot];
                int32_t below = 0;
                for (int32_t q = 0; q < n; ++q) {
                    if (kept[q] == 1) continue;
                    const int32_t iq = order[q];
                    const int32_t bq = e.birth[first + iq];
                    below += (bq < bi || (bq == bi && iq < i)) ? 1 : 0;
                }
                sink(player * C + i, kKindNone, kAbsent, 1, kAbsent, kAbsent, wadd(below, survivors));
            }
        }
        wave_sync();
    }
}

// The decode with player 0's legality from the state (legality_row).
template <typename Sink>
NR_DEV void gridnet_decode(const KGame& g, const Hdr& h, const Env& e, const GridLayout& y, const int32_t* acts,
                           int32_t players, int lane, Sink sink) {
    gridnet_decode_by(g, h, e, y, acts, players, lane, sink, [&](int32_t i, const GridRow& r) {
        const Row lr = legality_row(g, h, e, g.N + i);
        return r.kind == kKindMove ? row_bit(lr, 6 + gidx(r.dir, 4))
                                   : (row_bit(lr, 18 + gidx(r.dir, 4)) && row_bit(lr, 22 + gidx(r.ptype, g.T)));
    });
}

// Wave-cooperative writers for 64-cell chunks: lane i holds the words of
// cell c0 + i, and element j of the chunk's contiguous run is written by lane
// j % 64 after fetching its cell's words from lane j / width with a shuffle,
// so each store instruction covers one contiguous span.  Every lane runs the
// same iterations, which keeps the shuffles' source lanes active.
NR_DEV uint32_t lane_word(uint32_t v, int32_t src) { return (uint32_t)__shfl((int)v, src, kWave); }

// n rows of Width 0/1 elements: bit b of the cell's row is bit b of w0..w2.
template <typename T, int Width, int Words>
NR_DEV void put_bit_rows(T* dst, int32_t n, uint32_t w0, uint32_t w1, uint32_t w2, int lane) {
    const int32_t total = n * Width;
    for (int32_t j0 = 0; j0 < total; j0 += kWave) {
        const int32_t j = j0 + lane;
        const int32_t jj = j < total ? j : total - 1;
        const int32_t cell = jj / Width, bit = jj - cell * Width;
        uint32_t w = lane_word(w0, cell);
        if (Words > 1) {
            const uint32_t b = lane_word(w1, cell), c = lane_word(w2, cell);
            w = bit < 32 ? w : (bit < 64 ? b : c);
        }
        if (j < total) dst[j] = (T)((w >> (bit & 31)) & 1u);
    }
}

// The same rows, four elements per store: int32 elements as 16-byte stores,
// bytes packed four to a dword.  A run whose start or length does not fit
// the wider store takes the element path.
template <int Width, int Words>
NR_DEV uint32_t row_bit_of(int32_t bit, uint32_t a0, uint32_t a1, uint32_t a2) {
    uint32_t w = a0;
    if (Words > 1) w = bit < 32 ? a0 : (bit < 64 ? a1 : a2);
    return (w >> (bit & 31)) & 1u;
}

template <typename T, int Width, int Words>
NR_DEV void put_bit_rows4(T* dst, int32_t n, uint32_t w0, uint32_t w1, uint32_t w2, int lane) {
    const int32_t total = n * Width;
    const uintptr_t align = sizeof(T) == 4 ? 15u : 3u;
    if ((((uintptr_t)dst) & align) != 0u || (total & 3) != 0) {
        put_bit_rows<T, Width, Words>(dst, n, w0, w1, w2, lane);
        return;
    }
    const int32_t quads = total >> 2;
    for (int32_t q0 = 0; q0 < quads; q0 += kWave) {
        const int32_t q = q0 + lane;
        const int32_t e0 = (q < quads ? q : quads - 1) * 4;
        const int32_t ca = e0 / Width, cb = (e0 + 3) / Width;  // Width >= 4: at most two cells
        const uint32_t a0 = lane_word(w0, ca), b0 = lane_word(w0, cb);
        uint32_t a1 = 0u, a2 = 0u, b1 = 0u, b2 = 0u;
        if (Words > 1) {
            a1 = lane_word(w1, ca);
            a2 = lane_word(w2, ca);
            b1 = lane_word(w1, cb);
            b2 = lane_word(w2, cb);
        }
        uint32_t v[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int32_t b = e0 + k;
            const bool first = b < (ca + 1) * Width;
            const int32_t bit = b - (first ? ca : cb) * Width;
            v[k] = first ? row_bit_of<Width, Words>(bit, a0, a1, a2) : row_bit_of<Width, Words>(bit, b0, b1, b2);
        }
        if (q < quads) {
            if (sizeof(T) == 4) {
                uint4 x;
                x.x = v[0];
                x.y = v[1];
                x.z = v[2];
                x.w = v[3];
                ((uint4*)dst)[q] = x;
            } else {
                ((uint32_t*)dst)[q] = v[0] | (v[1] << 8) | (v[2] << 16) | (v[3] << 24);
            }
        }
    }
}

// GridNet observation of one env (N/adapters/gridnet/observation.py:27-72):
// planes = one-hot of the full-observation feature maps clipped to the widths
// 5, 5, 3, 8, 6, 2 (or the six clipped values), the source mask (cells of an
// available unit of the player) and its legality row as the action mask
// (rows, or packed into three words: bits 0-28, 29-60, 61-77).  The wave
// walks the board in 64-cell chunks, one cell per lane; the wide rows
// (one-hot planes, mask rows) go out as contiguous runs, the narrow ones
// (plane indices, packed words, the source mask) from each cell's lane.
NR_DEV void gridnet_observe(const KGame& g, const Hdr& h, const Env& e, int64_t l, int lane,
                            const nanorts_gridnet_obs& o, void* planes_out) {
    const int32_t cells = g.cells;
    const int32_t widths[6] = {5, 5, 3, 8, 6, 2};
    const int32_t offsets[6] = {0, 5, 10, 13, 21, 27};
    const bool rows_needed = o.source_mask || o.action_mask;
    for (int32_t c0 = 0; c0 < cells; c0 += kWave) {
        const int32_t c = c0 + lane, n = imin(kWave, cells - c0);
        uint32_t word = 0u, terrain = 0u;
        int32_t owner = kAbsent, slot = 0;
        bool available = false;
        if (c < cells) {
            const int32_t occ = e.entity[c];
            if (occ != kAbsent) {
                slot = clampi(occ, 0, g.E - 1);
                const uint32_t hp = (uint32_t)(int32_t)e.hp[slot] & 0xFFu;
                const uint32_t carried = (uint32_t)e.carried[slot] & 0xFFu;
                const uint32_t type = (uint32_t)((int32_t)e.utype[slot] + 1) & 0xFFu;
                const int32_t pk = e.pkind[slot];
                const uint32_t kind = (uint32_t)(pk > 0 ? pk : 0) & 0xFu;
                owner = e.owner[slot];
                const uint32_t own = (uint32_t)(owner + 1) & 0x3u;
                word = hp | (carried << 8) | (type << 16) | (kind << 24) | (own << 28);
                available = owner >= 0 && pk == kAbsent;  // board_view.available
            }
            terrain = h.terrain[c] ? 1u : 0u;
        }
        Row lr;
        lr.w[0] = lr.w[1] = lr.w[2] = 0u;
        if (available && rows_needed) lr = legality_row(g, h, e, slot);
#pragma unroll
        for (int32_t p = 0; p < 2; ++p) {
            const int64_t at0 = (l * 2 + p) * cells + c0;
            const uint32_t own = (word >> 28) & 3u;
            const uint32_t relabelled = own > 0 ? (uint32_t)(((int32_t)own - 1 + p) % 2 + 1) : 0u;
            const uint32_t fm[6] = {word & 0xFFu, (word >> 8) & 0xFFu, relabelled, (word >> 16) & 0xFFu,
                                    (word >> 24) & 0xFu, terrain};
            if (planes_out) {
                if (o.planes_form == 1) {
                    uint32_t packed = 0u;  // six 3-bit clipped values
#pragma unroll
                    for (int f = 0; f < 6; ++f) packed |= (uint32_t)imin((int32_t)fm[f], widths[f] - 1) << (3 * f);
                    // six bytes per cell are written by their own lane, as
                    // three 2-byte stores (a shuffle per element costs more
                    // than it saves for so narrow a row)
                    if (c < cells) {
                        int16_t* dst = (int16_t*)((int8_t*)planes_out + (at0 + lane) * 6);
#pragma unroll
                        for (int k = 0; k < 3; ++k)
                            dst[k] = (int16_t)(((packed >> (6 * k)) & 7u) | (((packed >> (6 * k + 3)) & 7u) << 8));
                    }
                } else {
                    uint32_t hot = 0u;  // 29 plane bits
#pragma unroll
                    for (int f = 0; f < 6; ++f) hot |= 1u << (offsets[f] + imin((int32_t)fm[f], widths[f] - 1));
                    if (o.planes_bytes == 4)
                        put_bit_rows4<int32_t, kPlaneCount, 1>((int32_t*)planes_out + at0 * kPlaneCount, n, hot, 0u,
                                                              0u, lane);
                    else
                        put_bit_rows4<uint8_t, kPlaneCount, 1>((uint8_t*)planes_out + at0 * kPlaneCount, n, hot, 0u,
                                                              0u, lane);
                }
            }
            const bool source = available && owner == p;
            if (o.source_mask && c < cells) o.source_mask[at0 + lane] = source ? 1 : 0;
            if (o.action_mask) {
                const uint32_t w0 = source ? lr.w[0] : 0u, w1 = source ? lr.w[1] : 0u, w2 = source ? lr.w[2] : 0u;
                if (o.mask_form == 1) {
                    if (c < cells) {
                        uint32_t* dst = (uint32_t*)o.action_mask + (at0 + lane) * 3;
                        dst[0] = w0 & 0x1FFFFFFFu;
                        dst[1] = (w0 >> 29) | (w1 << 3);
                        dst[2] = ((w1 >> 29) | (w2 << 3)) & 0x1FFFFu;
                    }
                } else if (o.mask_bytes == 4)
                    put_bit_rows4<int32_t, kMaskWidth, 3>((int32_t*)o.action_mask + at0 * kMaskWidth, n, w0, w1, w2,
                                                         lane);
                else
                    put_bit_rows4<uint8_t, kMaskWidth, 3>((uint8_t*)o.action_mask + at0 * kMaskWidth, n, w0, w1, w2,
                                                         lane);
            }
        }
    }
}

}  // namespace nr
