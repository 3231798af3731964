// The env path of one cycle (get_avail_actions -> decode -> core.step ->
// observe) with the requests held in lanes.
//
// Through the JaxMARL surface, decode_actions issues a command to every
// available unit and to nothing else (src/nanorts/adapters/jaxmarl/actions.py
// :61-84), so the issued requests are the available units.  That lets the
// admission below compute every request's legality, blocking, duration and
// reservation in parallel (they read only the board, which admission never
// changes) and run the sequential conflict resolution only over the requests
// that claim a position or cost resources, against claim lists held in
// registers.  When a precondition of this formulation does not hold, it
// returns false untouched and the general admission (engine.h) runs instead.
#pragma once

#include "engine.h"

namespace nr {

// Availability compaction: lists available owned positions in order, marks
// the commands of unavailable positions absent, and reports states whose
// available units hold a pending order (then the parallel admission does
// not apply).
NR_DEV int32_t compact_available(const KGame& g, const Env& e_in, int lane, bool* irregular) {
    const Env e = refresh(g, e_in);
    const Layout& y = g.lay;
    AS3 int16_t* av = at<int16_t>(e, y.a_av);
    AS3 int8_t* ckind = at<int8_t>(e, y.c_kind);
    AS3 int16_t* crank = at<int16_t>(e, y.c_rank);
    int32_t n = 0;
    bool odd = false;
    for (int32_t base = 0; base < 2 * g.C; base += kWave) {
        const int32_t p = base + lane;
        bool available = false;
        if (p < 2 * g.C) {
            const int32_t s = g.N + p;
            available = e.birth[s] != kAbsent && e.pkind[s] == kAbsent;
            if (available && e.porder[s] != kAbsent) odd = true;
            if (!available) ckind[p] = (int8_t)kAbsent;
            crank[p] = 0;
        }
        const uint64_t m = ballot(available);
        if (available) av[n + count_below(m)] = (int16_t)p;
        n += popc(m);
    }
    *irregular = ballot(odd) != 0ull;
    wave_sync();
    return n;
}

// Admission over the n available units listed by compact_available, whose
// canonical commands are staged in the command arrays.
NR_DEV bool admit_env(const KGame& g, const Hdr& h, const Env& e_in, int lane, uint32_t key0, uint32_t key1,
                      bool count_events, int32_t n, bool irregular) {
    const Env e = refresh(g, e_in);
    const Layout& y = g.lay;
    if (irregular || n > kWave) return false;
    const int32_t time = uni(e.sc[S_TIME]);
    const int32_t next_order = uni(e.sc[S_NEXT_ORDER]);
    if (next_order > 0x7fffffff - kWave) return false;
    // Entries that can conflict: pending MOVE / PRODUCE (the only kinds that
    // claim a position or cost resources).  Those pending at the start of
    // the cycle were issued earlier, so every conflict with them is
    // cross-cycle and they all rank before this cycle's appends; their order
    // among themselves then does not matter (N/core/reservations.py:154-192).
    AS3 int16_t* list = at<int16_t>(e, y.a_list);
    int32_t nA = 0;
    bool bad = false;
    for (int32_t base = 0; base < g.E; base += kWave) {
        const int32_t s = base + lane;
        bool entry = false;
        if (s < g.E) {
            const int32_t k = e.pkind[s];
            if (k != kAbsent) {
                const int32_t ord = e.porder[s];
                if (s < g.N || ord == kAbsent || ord >= next_order) bad = true;
                if (k == kKindMove || k == kKindProduce) {
                    entry = true;
                    if (e.pissued[s] == time) bad = true;
                }
            }
        }
        const uint64_t m = ballot(entry);
        if (entry) list[nA + count_below(m)] = (int16_t)s;
        nA += popc(m);
    }
    if (ballot(bad) != 0ull || nA > kWave) return false;
    wave_sync();
    int32_t posA = 0, costA = 0, playerA = 0;
    if (lane < nA) {
        const int32_t s = list[lane];
        const int32_t k = e.pkind[s];
        playerA = clampi(e.owner[s], 0, 1);
        costA = k == kKindProduce ? tabv(h, F_COST, clampi(e.pptype[s], 0, g.T - 1)) : 0;
        posA = reserved_position(g, e.cell[s], e.pdir[s]);
    }
    // Requests, lane i = i-th available unit: _admit_one up to the
    // reservation (N/core/admission.py:242-289), in parallel.
    int32_t p = 0, slot = 0, kind1 = kAbsent, none1 = 0, req = 0, dir = kAbsent, ptype = kAbsent, target = kAbsent;
    int32_t pos1 = 0, cost1 = 0, player1 = 0, birth = 0, pl = 0;
    bool conflicting = false;
    if (lane < n) {
        p = at<int16_t>(e, y.a_av)[lane];
        slot = g.N + p;
        pl = p / g.C;
        const int32_t kind0 = at<int8_t>(e, y.c_kind)[p];
        dir = at<int8_t>(e, y.c_dir)[p];
        ptype = at<int8_t>(e, y.c_ptype)[p];
        target = at<int16_t>(e, y.c_target)[p];
        const int32_t none0 = at<int32_t>(e, y.c_none)[p];
        const int32_t cell = e.cell[slot];
        const int32_t owner = e.owner[slot];
        birth = e.birth[slot];
        req = action_duration(g, h, e.utype[slot], kind0, none0, ptype);
        const bool legal = can_execute(g, h, e, slot, kind0, dir, target, ptype);
        kind1 = legal ? kind0 : kKindNone;
        none1 = legal ? none0 : req;
        if (claims_position(kind1)) {
            const int32_t at_ = gidx(reserved_position(g, cell, dir), g.cells);
            if (h.terrain[at_] != 0 || e.entity[at_] != kAbsent) {
                kind1 = kKindNone;
                none1 = req;
            }
        }
        if (count_events) {
            // _count_admitted (:406-429)
            AS3 uint32_t* ev = at<uint32_t>(e, y.b_events);
            int32_t idx = -1;
            if (kind1 == kKindHarvest) idx = pl;
            else if (kind1 == kKindReturn) idx = 2 + pl;
            else if (kind1 == kKindProduce) idx = 4 + pl * 8 + clampi(ptype, 0, g.T - 1);
            else if (kind1 == kKindAttack) {
                const int32_t occ = e.entity[clampi(target, 0, g.cells - 1)];
                const int32_t towner = occ == kAbsent ? kAbsent : e.owner[clampi(occ, 0, g.E - 1)];
                if (towner + 1 >= 0 && towner + 1 < 3) idx = 20 + pl * 3 + towner + 1;
            }
            if (idx >= 0) __atomic_fetch_add(&ev[idx], 1u, __ATOMIC_RELAXED);
        }
        cost1 = kind1 == kKindProduce ? tabv(h, F_COST, clampi(ptype, 0, g.T - 1)) : 0;
        pos1 = reserved_position(g, cell, dir);
        player1 = clampi(owner, 0, 1);
        conflicting = claims_position(kind1) || cost1 != 0;
    }
    // Java admission order (_ordered_requests :200-221): player, then birth.
    int32_t rank = 0;
    for (int32_t j = 0; j < n; ++j) {
        const int32_t plj = __builtin_amdgcn_readlane(pl, j);
        const int32_t bj = __builtin_amdgcn_readlane(birth, j);
        rank += (plj < pl) || (plj == pl && (bj < birth || (bj == birth && j < lane)));
    }
    // Sequential conflict resolution over the requests that can conflict.
    const int32_t bal0 = uni(e.sc[S_RES0]), bal1 = uni(e.sc[S_RES1]);
    int32_t alt = uni(e.sc[S_ALT]);
    AS3 int32_t* fk = at<int32_t>(e, y.a_fk);
    AS3 int32_t* fn = at<int32_t>(e, y.a_fn);
    int32_t posB = 0, costB = 0, playerB = 0, durB = 0, rlB = 0, nB = 0;
    bool liveB = false;
    const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
    const uint64_t conflicting_lanes = ballot(conflicting);
    for (int32_t k = 0; k < n && conflicting_lanes != 0ull; ++k) {
        const int32_t li = (int32_t)__builtin_ctzll(ballot(lane < n && rank == k));
        if (((conflicting_lanes >> li) & 1ull) == 0ull) continue;
        const int32_t rkind = __builtin_amdgcn_readlane(kind1, li);
        const int32_t rnone = __builtin_amdgcn_readlane(none1, li);
        const int32_t rreq = __builtin_amdgcn_readlane(req, li);
        const int32_t rpos = __builtin_amdgcn_readlane(pos1, li);
        const int32_t rcost = __builtin_amdgcn_readlane(cost1, li);
        const int32_t rplayer = __builtin_amdgcn_readlane(player1, li);
        const bool rclaims = claims_position(rkind);
        const int32_t bal = rplayer ? bal1 : bal0;
        // _reservations_conflict (N/core/reservations.py:122-135)
        const int32_t clA = wadd(playerA == rplayer ? costA : 0, rcost);
        const bool cA = lane < nA && ((rclaims && posA == rpos) || (rcost != 0 && clA > 0 && clA > bal));
        const bool anyA = ballot(cA) != 0ull;
        const int32_t clB = wadd(playerB == rplayer ? costB : 0, rcost);
        const bool cB = liveB && ((rclaims && posB == rpos) || (rcost != 0 && clB > 0 && clB > bal));
        const uint64_t sm = ballot(cB);
        int32_t fkind = rkind, fnone = rnone;
        if (anyA || sm != 0ull) {
            const int32_t same_before = popc(sm & below);
            bool cancels_req = true, cancels_pend = true;
            if (g.strategy == NANORTS_CANCEL_ALTERNATING) {
                cancels_req = floor_mod(wadd(alt, same_before), 2) == 0;
                cancels_pend = !cancels_req;
            } else if (g.strategy == NANORTS_CANCEL_RANDOM) {
                int32_t draw = 0;
                if (sm != 0ull) {
                    uint32_t ek0 = key0, ek1 = key1;
                    fold_in(ek0, ek1, (uint32_t)time);
                    fold_in(ek0, ek1, (uint32_t)__builtin_amdgcn_readlane(birth, li));
                    fold_in(ek0, ek1, 0u);
                    if (cB) {
                        fold_in(ek0, ek1, (uint32_t)same_before);
                        draw = randint01(ek0, ek1);
                    }
                }
                cancels_req = draw == 0;
                cancels_pend = !cancels_req;
            }
            const int32_t incl = wave_inclusive_min((cB && cancels_req) ? durB : kNoCap, lane);
            const int32_t cap = __shfl(incl, kWave - 1, kWave);
            int32_t excl = __shfl_up(incl, 1u, kWave);
            if (lane == 0) excl = kNoCap;
            const int32_t before = anyA ? -1 : imin(rreq, excl);
            if (cB && cancels_pend) {
                const int32_t settled = wadd(wmul(imin(durB, before), 2), 1) >> 1;
                liveB = false;
                fk[rlB] = kKindNone;
                fn[rlB] = settled;
            }
            if (g.strategy == NANORTS_CANCEL_ALTERNATING) alt = wadd(alt, popc(sm));
            if (anyA || cap != kNoCap) {
                fkind = kKindNone;
                fnone = anyA ? -1 : imin(rreq, cap);
            }
        }
        if (lane == 0) {
            fk[li] = fkind;
            fn[li] = fnone;
        }
        if (fkind != kKindNone) {
            // admitted as MOVE / PRODUCE: a same-cycle entry from now on
            if (lane == nB) {
                posB = rpos;
                costB = rcost;
                playerB = rplayer;
                durB = wmul(rreq, 4) >> 2;
                rlB = li;
                liveB = true;
            }
            ++nB;
        }
        wave_sync();
    }
    // _assign_pending_action (:374-403) for every request, in parallel.
    if (lane < n) {
        int32_t fkind = kind1, fnone = none1;
        if (conflicting) {
            fkind = fk[lane];
            fnone = fn[lane];
        }
        const int32_t duration = fkind == kKindNone ? fnone : req;
        e.pkind[slot] = (int8_t)fkind;
        e.pdir[slot] = (int8_t)((fkind == kKindMove || fkind == kKindHarvest || fkind == kKindReturn ||
                                 fkind == kKindProduce)
                                    ? dir
                                    : kAbsent);
        e.pnone[slot] = fkind == kKindNone ? fnone : 0;
        e.ptarget[slot] = (int16_t)(fkind == kKindAttack ? target : kAbsent);
        e.pptype[slot] = (int8_t)(fkind == kKindProduce ? ptype : kAbsent);
        e.pissued[slot] = time;
        e.pcompl[slot] = wadd(time, duration);
        e.porder[slot] = wadd(next_order, rank);
    }
    if (lane == 0) {
        e.sc[S_NEXT_ORDER] = wadd(next_order, n);
        if (g.strategy == NANORTS_CANCEL_ALTERNATING) e.sc[S_ALT] = alt;
    }
    wave_sync();
    return true;
}

// core.step of the env path.
NR_DEV void env_core_step(const KGame& g, const Hdr& h, const Env& e, int lane, uint32_t key0, uint32_t key1,
                          bool count_events, int32_t n, bool irregular) {
    if (count_events) {
        if (lane < 32) at<int32_t>(e, g.lay.b_events)[lane] = 0;
        wave_sync();
    }
    if (!admit_env(g, h, e, lane, key0, key1, count_events, n, irregular)) {
        int32_t n_rank = 0;
        const int32_t issued = order_requests(g, e, lane, &n_rank);
        AS3 int16_t* order = at<int16_t>(e, g.lay.b_order);
        for (int32_t i = 0; i < issued; ++i) admit_one(g, h, e, lane, uni(order[i]), n_rank, key0, key1, count_events);
    }
    complete(g, h, e, lane);
    decide(g, e, lane);
}

// Symbolic observations of both agents in one pass over the cells
// (N/observations/symbolic.py:130-180, visibility.py:56-71).
NR_DEV void observe_all(const KGame& g, const Hdr& h, const Env& e_in, int lane, bool partial, uint8_t* maps0,
                        uint8_t* maps1, int32_t* scalars0, int32_t* scalars1) {
    const Env e = refresh(g, e_in);
    const Layout& y = g.lay;
    AS3 uint32_t* seen = at<uint32_t>(e, y.v_seen);  // [2][H][seen_words]
    const int32_t plane = g.H * g.seen_words;
    if (partial) {
        AS3 int16_t* units = at<int16_t>(e, y.b_units);
        for (int32_t i = lane; i < 2 * plane; i += kWave) seen[i] = 0u;
        int32_t n = 0;
        for (int32_t base = 0; base < 2 * g.C; base += kWave) {
            const int32_t i = base + lane;
            const bool act = i < 2 * g.C && e.birth[g.N + i] != kAbsent;
            const uint64_t m = ballot(act);
            if (act) units[n + count_below(m)] = (int16_t)(g.N + i);
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
            const int32_t cy = floor_div(cell, g.W) + dy;
            if (cy < 0 || cy >= g.H) continue;
            const int32_t rem = r * r - dy * dy;
            int32_t hw = r;
            while (hw * hw > rem) --hw;
            const int32_t cx = floor_mod(cell, g.W);
            const int32_t x0 = cx - hw < 0 ? 0 : cx - hw;
            const int32_t x1 = cx + hw >= g.W ? g.W - 1 : cx + hw;
            if (x0 > x1) continue;
            AS3 uint32_t* row = seen + ((s - g.N) / g.C) * plane + cy * g.seen_words;
            for (int32_t wd = x0 >> 5; wd <= (x1 >> 5); ++wd) {
                const int32_t a = x0 > wd * 32 ? x0 - wd * 32 : 0;
                const int32_t b = x1 < wd * 32 + 31 ? x1 - wd * 32 : 31;
                const uint32_t bits = (b - a == 31) ? 0xFFFFFFFFu : (((1u << (b - a + 1)) - 1u) << a);
                __atomic_fetch_or(&row[wd], bits, __ATOMIC_RELAXED);
            }
        }
        wave_sync();
    }
    AS3 uint8_t* stage0 = at<uint8_t>(e, y.v_stage);
    AS3 uint8_t* stage1 = stage0 + g.stage_cells * 6;
    for (int32_t c0 = 0; c0 < g.cells; c0 += g.stage_cells) {
        const int32_t nc = imin(g.stage_cells, g.cells - c0);
        for (int32_t i = lane; i < nc; i += kWave) {
            const int32_t c = c0 + i;
            const int32_t occ = e.entity[c];
            uint32_t hp = 0, carried = 0, type = 0, kind = 0, owner = 0;
            if (occ != kAbsent) {
                const int32_t s = clampi(occ, 0, g.E - 1);
                hp = (uint32_t)(int32_t)e.hp[s] & 0xFFu;
                carried = (uint32_t)e.carried[s] & 0xFFu;
                type = (uint32_t)((int32_t)e.utype[s] + 1) & 0xFFu;
                const int32_t pk = e.pkind[s];
                kind = (uint32_t)(pk > 0 ? pk : 0) & 0xFu;
                owner = (uint32_t)((int32_t)e.owner[s] + 1) & 0x3u;
            }
            const uint32_t terrain = (uint32_t)h.terrain[c] << 8;
            const int32_t yy = c / g.W, x = c - yy * g.W;
#pragma unroll
            for (int32_t pl = 0; pl < 2; ++pl) {
                bool shown = true;
                if (partial) {
                    const uint32_t word = seen[pl * plane + yy * g.seen_words + (x >> 5)];
                    shown = owner == (uint32_t)(pl + 1) || ((word >> (x & 31)) & 1u);
                }
                AS3 uint16_t* out = (AS3 uint16_t*)((pl == 0 ? stage0 : stage1) + i * 6);
                if (shown) {
                    const uint32_t rel = owner > 0 ? (uint32_t)((((int32_t)owner - 1 + pl) & 1) + 1) : 0u;
                    out[0] = (uint16_t)(hp | (carried << 8));
                    out[1] = (uint16_t)(rel | (type << 8));
                    out[2] = (uint16_t)(kind | terrain);
                } else {
                    out[0] = 0;
                    out[1] = 0;
                    out[2] = (uint16_t)terrain;
                }
            }
        }
        wave_sync();
        if (maps0) copy_out(maps0 + (size_t)c0 * 6, stage0, nc * 6, lane);
        if (maps1) copy_out(maps1 + (size_t)c0 * 6, stage1, nc * 6, lane);
        wave_sync();
    }
    if (lane < 8) {
        const int32_t pl = lane >> 2, f = lane & 3;
        int32_t v;
        if (f == 0) v = e.sc[S_RES0 + pl];
        else if (f == 1) v = e.sc[S_RES0 + (pl ^ 1)];
        else if (f == 2) v = e.sc[S_TIME];
        else v = e.sc[S_ALT];
        int32_t* dst = pl == 0 ? scalars0 : scalars1;
        if (dst) dst[f] = v;
    }
}

}  // namespace nr
