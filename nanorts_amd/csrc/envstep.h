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

// One request per lane (lane i = the i-th available unit): _admit_one up to
// the reservation (N/core/admission.py:242-289).
struct Reqs {
    int32_t p, slot, kind1, none1, req, dir, ptype, target, pos1, cost1, player1, birth, pl;
    int32_t order_rank;  // the command's request_order rank (0 through the JaxMARL surface)
    bool conflicting;
};

// The request fields that follow from a canonical command of slot N + p.
NR_DEV void request_of(const KGame& g, const Hdr& h, const Env& e, int32_t p, int32_t kind0, int32_t dir, int32_t ptype,
                       int32_t target, int32_t none0, bool known_legal, bool count_events, Reqs& q) {
    const Layout& y = g.lay;
    q.p = p;
    q.slot = g.N + p;
    q.pl = p >= g.C ? 1 : 0;
    q.dir = dir;
    q.ptype = ptype;
    q.target = target;
    const int32_t slot = q.slot;
    const int32_t cell = e.cell[slot];
    const int32_t owner = e.owner[slot];
    q.birth = e.birth[slot];
    q.req = action_duration(g, h, e.utype[slot], kind0, none0, ptype);
    // A command sampled from this cycle's masks is legal and unblocked:
    // every mask factor is legal for some value of the others, and the
    // produce factors are independent (free direction and affordable
    // type), so the sampled combination passes is_valid.
    const bool legal = known_legal || can_execute(g, h, e, slot, kind0, dir, target, ptype);
    int32_t kind1 = legal ? kind0 : kKindNone;
    int32_t none1 = legal ? none0 : q.req;
    if (!known_legal && claims_position(kind1)) {
        const int32_t at_ = gidx(reserved_position(g, cell, dir), g.cells);
        if (h.terrain[at_] != 0 || e.entity[at_] != kAbsent) {
            kind1 = kKindNone;
            none1 = q.req;
        }
    }
    if (count_events) {
        // _count_admitted (:406-429)
        AS3 uint32_t* ev = at<uint32_t>(e, y.b_events);
        const int32_t pl = q.pl;
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
    q.kind1 = kind1;
    q.none1 = none1;
    q.cost1 = kind1 == kKindProduce ? tabv(h, F_COST, clampi(ptype, 0, g.T - 1)) : 0;
    q.pos1 = reserved_position(g, cell, dir);
    q.player1 = clampi(owner, 0, 1);
    q.conflicting = claims_position(kind1) || q.cost1 != 0;
}

NR_DEV void no_request(Reqs& q) {
    q.p = q.slot = 0;
    q.kind1 = kAbsent;
    q.none1 = q.req = 0;
    q.dir = q.ptype = q.target = kAbsent;
    q.pos1 = q.cost1 = q.player1 = q.birth = q.pl = 0;
    q.order_rank = 0;
    q.conflicting = false;
}

// Entries that can conflict: pending MOVE / PRODUCE (the only kinds that
// claim a position or cost resources).  Those pending at the start of the
// cycle were issued earlier, so every conflict with them is cross-cycle and
// they all rank before this cycle's appends; their order among themselves
// then does not matter (N/core/reservations.py:154-192).  With `listed`, the
// summary of the state (rollout.h) already listed them and folded their
// preconditions into `irregular`.  Lane i < nA receives entry i.
// A half-wave team (TW = 32) takes up to 64 entries: lane i receives entries
// i and TW + i (the second into posA[1], costA[1], playerA[1]).
template <int TW = kWave>
NR_DEV bool admit_entries(const KGame& g, const Hdr& h, const Env& e, int lane, bool listed, int32_t* nA_out,
                          int32_t* posA, int32_t* costA, int32_t* playerA, int32_t listed_count = -1) {
    constexpr int32_t kHeld = TW == kWave ? TW : 2 * TW;
    const Layout& y = g.lay;
    const int32_t time = tuni<TW>(e.sc[S_TIME]);
    const int32_t next_order = tuni<TW>(e.sc[S_NEXT_ORDER]);
    if (next_order > 0x7fffffff - kWave) return false;
    AS3 int16_t* list = at<int16_t>(e, y.a_list);
    int32_t nA = 0;
    bool bad = false;
    // the summary's count, from the caller's registers when it holds it
    if (listed) nA = listed_count >= 0 ? listed_count : tuni<TW>(e.sc[S_NA]);
    for (int32_t base = 0; base < (listed ? 0 : g.E); base += TW) {
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
        const uint64_t m = tballot<TW>(entry);
        if (entry) list[nA + tcount_below<TW>(m)] = (int16_t)s;
        nA += popc(m);
    }
    if (tballot<TW>(bad) != 0ull || nA > kHeld) return false;
    wave_sync();
#pragma unroll
    for (int k = 0; k < kHeld / TW; ++k) {
        posA[k] = 0;
        costA[k] = 0;
        playerA[k] = 0;
        if (k * TW + lane < nA) {
            const int32_t s = list[k * TW + lane];
            const int32_t kind = e.pkind[s];
            playerA[k] = clampi(e.owner[s], 0, 1);
            costA[k] = kind == kKindProduce ? tabv(h, F_COST, clampi(e.pptype[s], 0, g.T - 1)) : 0;
            posA[k] = reserved_position(g, e.cell[s], e.pdir[s]);
        }
    }
    *nA_out = nA;
    return true;
}

template <int TW = kWave>
NR_DEV void admit_resolve(const KGame& g, const Hdr& h, const Env& e, int lane, uint32_t key0, uint32_t key1, int32_t n,
                          int32_t nA, const int32_t* posA, const int32_t* costA, const int32_t* playerA, const Reqs& q);
// The requests of q (built from sampled, known-legal commands) staged in
// the command arrays for the general admission.
NR_DEV void stage_requests(const KGame& g, const Env& e_in, int lane, int32_t n, const Reqs& q) {
    const Env e = refresh(g, e_in);
    const Layout& y = g.lay;
    if (lane < n) {
        at<int8_t>(e, y.c_kind)[q.p] = (int8_t)q.kind1;
        at<int8_t>(e, y.c_dir)[q.p] = (int8_t)q.dir;
        at<int8_t>(e, y.c_ptype)[q.p] = (int8_t)q.ptype;
        at<int16_t>(e, y.c_target)[q.p] = (int16_t)q.target;
        at<int32_t>(e, y.c_none)[q.p] = q.none1;
        at<int16_t>(e, y.c_rank)[q.p] = 0;
    }
    wave_sync();
}

// Admission over the n available units listed by compact_available, whose
// canonical commands are staged in the command arrays.
template <int TW = kWave>
NR_DEV bool admit_env(const KGame& g, const Hdr& h, const Env& e_in, int lane, uint32_t key0, uint32_t key1,
                      bool count_events, int32_t n, bool irregular, bool known_legal, bool listed = false) {
    const Env e = refresh<TW>(g, e_in);
    const Layout& y = g.lay;
    if (irregular || n > TW) return false;
    int32_t nA = 0, posA[2] = {0, 0}, costA[2] = {0, 0}, playerA[2] = {0, 0};
    if (!admit_entries<TW>(g, h, e, lane, listed, &nA, posA, costA, playerA)) return false;
    Reqs q;
    no_request(q);
    if (lane < n) {
        const int32_t p = at<int16_t>(e, y.a_av)[lane];
        request_of(g, h, e, p, at<int8_t>(e, y.c_kind)[p], at<int8_t>(e, y.c_dir)[p], at<int8_t>(e, y.c_ptype)[p],
                   at<int16_t>(e, y.c_target)[p], at<int32_t>(e, y.c_none)[p], known_legal, count_events, q);
        q.order_rank = at<int16_t>(e, y.c_rank)[p];
    }
    admit_resolve<TW>(g, h, e, lane, key0, key1, n, nA, posA, costA, playerA, q);
    return true;
}

// Rank, conflict resolution and pending assignment of the requests in q.
// posA / costA / playerA: this lane's entries, as admit_entries gives them
// (two for a half-wave team).
template <int TW>
NR_DEV void admit_resolve(const KGame& g, const Hdr& h, const Env& e, int lane, uint32_t key0, uint32_t key1, int32_t n,
                          int32_t nA, const int32_t* posA, const int32_t* costA, const int32_t* playerA, const Reqs& q) {
    const Layout& y = g.lay;
    const int32_t time = tuni<TW>(e.sc[S_TIME]);
    const int32_t next_order = tuni<TW>(e.sc[S_NEXT_ORDER]);
    const int32_t slot = q.slot, kind1 = q.kind1, none1 = q.none1, req = q.req, dir = q.dir, ptype = q.ptype;
    const int32_t target = q.target, pos1 = q.pos1, cost1 = q.cost1, player1 = q.player1, birth = q.birth, pl = q.pl;
    const bool conflicting = q.conflicting;
    // Java admission order (_ordered_requests :200-221): player, then the
    // request_order rank, then birth.  crank orders the requests that can
    // conflict among themselves.
    const uint64_t conflicting_lanes = tballot<TW>(conflicting);
    const int32_t orank = q.order_rank;
    int32_t rank = 0, crank = 0;
    // (a half-wave team's loops run to the larger of the halves' counts:
    // a lane j at or past its own team's count holds no request)
    const int32_t nmax = tmax<TW>(n);
    if (tballot<TW>(lane < n && (birth < 0 || birth >= (1 << 24) || orank != 0)) == 0ull) {
        // one 32-bit key per request: player, birth, lane
        const uint32_t key = lane < n ? ((uint32_t)pl << 31) | ((uint32_t)birth << 6) | (uint32_t)lane : 0xFFFFFFFFu;
        for (int32_t j = 0; j < nmax; ++j) {
            const uint32_t kj = (uint32_t)tread_at<TW>((int32_t)key, j);
            const int32_t before = kj < key ? 1 : 0;
            rank += before;
            crank += ((conflicting_lanes >> j) & 1ull) ? before : 0;
        }
    } else {
        for (int32_t j = 0; j < nmax; ++j) {
            const int32_t plj = tread_at<TW>(pl, j);
            const int32_t oj = tread_at<TW>(orank, j);
            const int32_t bj = tread_at<TW>(birth, j);
            const bool before = j < n && ((plj < pl) ||
                                          (plj == pl && (oj < orank || (oj == orank && (bj < birth || (bj == birth && j < lane))))));
            rank += before;
            crank += before && ((conflicting_lanes >> j) & 1ull);
        }
    }
    // Sequential conflict resolution over the requests that can conflict.
    int32_t alt = tuni<TW>(e.sc[S_ALT]);
    // each request's final kind and duration, held in its own lane
    int32_t my_kind = kind1, my_none = none1;
    int32_t posB = 0, costB = 0, playerB = 0, durB = 0, rlB = 0, nB = 0;
    bool liveB = false;
    const int32_t nconf = popc(conflicting_lanes);
    const int32_t kmax = tmax<TW>(nconf);
    for (int32_t k = 0; k < kmax; ++k) {
        if (TW != kWave && k >= nconf) continue;
        const int32_t li = (int32_t)__builtin_ctzll(tballot<TW>(conflicting && crank == k));
        const int32_t rkind = tread<TW>(kind1, li);
        const int32_t rnone = tread<TW>(none1, li);
        const int32_t rreq = tread<TW>(req, li);
        const int32_t rpos = tread<TW>(pos1, li);
        const int32_t rcost = tread<TW>(cost1, li);
        const int32_t rplayer = tread<TW>(player1, li);
        const bool rclaims = claims_position(rkind);
        // (the balances are read here, at the conflict, rather than held in
        // registers through the loop; admission writes them only after it)
        const int32_t bal = tuni<TW>(e.sc[S_RES0 + rplayer]);
        // _reservations_conflict (N/core/reservations.py:122-135)
        bool cA = false;
#pragma unroll
        for (int k = 0; k < (TW == kWave ? 1 : 2); ++k) {
            const int32_t clA = wadd(playerA[k] == rplayer ? costA[k] : 0, rcost);
            cA = cA || (k * TW + lane < nA &&
                        ((rclaims && posA[k] == rpos) || (rcost != 0 && clA > 0 && clA > bal)));
        }
        const bool anyA = tballot<TW>(cA) != 0ull;
        const int32_t clB = wadd(playerB == rplayer ? costB : 0, rcost);
        const bool cB = liveB && ((rclaims && posB == rpos) || (rcost != 0 && clB > 0 && clB > bal));
        const uint64_t sm = tballot<TW>(cB);
        int32_t fkind = rkind, fnone = rnone;
        if (anyA || sm != 0ull) {
            const int32_t same_before = tcount_below<TW>(sm);
            bool cancels_req = true, cancels_pend = true;
            if (g.strategy == NANORTS_CANCEL_ALTERNATING) {
                cancels_req = floor_mod(wadd(alt, same_before), 2) == 0;
                cancels_pend = !cancels_req;
            } else if (g.strategy == NANORTS_CANCEL_RANDOM) {
                int32_t draw = 0;
                if (sm != 0ull) {
                    uint32_t ek0 = key0, ek1 = key1;
                    fold_in(ek0, ek1, (uint32_t)time);
                    fold_in(ek0, ek1, (uint32_t)tread<TW>(birth, li));
                    fold_in(ek0, ek1, 0u);
                    if (cB) {
                        fold_in(ek0, ek1, (uint32_t)same_before);
                        draw = randint01(ek0, ek1);
                    }
                }
                cancels_req = draw == 0;
                cancels_pend = !cancels_req;
            }
            const int32_t incl = wave_inclusive_min<TW>((cB && cancels_req) ? durB : kNoCap, lane);
            const int32_t cap = __shfl(incl, TW - 1, TW);
            int32_t excl = __shfl_up(incl, 1u, TW);
            if (lane == 0) excl = kNoCap;
            const int32_t before = anyA ? -1 : imin(rreq, excl);
            const bool cancelled = cB && cancels_pend;
            const int32_t settled = wadd(wmul(imin(durB, before), 2), 1) >> 1;
            // each cancelled same-cycle entry settles its request's lane
            for (uint64_t m = tballot<TW>(cancelled); m != 0ull; m &= m - 1ull) {
                const int32_t b = (int32_t)__builtin_ctzll(m);
                const int32_t to = tread<TW>(rlB, b), settles = tread<TW>(settled, b);
                if (lane == to) {
                    my_kind = kKindNone;
                    my_none = settles;
                }
            }
            if (cancelled) liveB = false;
            if (g.strategy == NANORTS_CANCEL_ALTERNATING) alt = wadd(alt, popc(sm));
            if (anyA || cap != kNoCap) {
                fkind = kKindNone;
                fnone = anyA ? -1 : imin(rreq, cap);
            }
        }
        if (lane == li) {
            my_kind = fkind;
            my_none = fnone;
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
    }
    // _assign_pending_action (:374-403) for every request, in parallel.
    if (lane < n) {
        const int32_t fkind = my_kind, fnone = my_none;
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
}

// core.step of the env path.
NR_DEV void env_core_step(const KGame& g, const Hdr& h, const Env& e, int lane, uint32_t key0, uint32_t key1,
                          bool count_events, int32_t n, bool irregular, bool known_legal) {
    if (count_events) {
        if (lane < 32) at<int32_t>(e, g.lay.b_events)[lane] = 0;
        wave_sync();
    }
    if (!admit_env(g, h, e, lane, key0, key1, count_events, n, irregular, known_legal)) {
        int32_t n_rank = 0;
        const int32_t issued = order_requests(g, e, lane, &n_rank);
        AS3 int16_t* order = at<int16_t>(e, g.lay.b_order);
        for (int32_t i = 0; i < issued; ++i) admit_one(g, h, e, lane, uni(order[i]), n_rank, key0, key1, count_events);
    }
    complete(g, h, e, lane);
    decide_counted(e, lane);
}

// Per-cycle occupancy bitmaps, rows of g.seen_words 32-bit words:
//   0 blocked (occupied or wall), 1/2 units of player 0/1, 3 resources,
//   4/5 stockpiles of player 0/1.
NR_DEV void build_bitmaps(const KGame& g, const Hdr& h, const Env& e_in, int lane) {
    const Env e = refresh(g, e_in);
    AS3 uint32_t* bm = at<uint32_t>(e, g.lay.o_bm);
    const int32_t plane = g.H * g.seen_words;
    for (int32_t i = lane; i < 6 * plane; i += kWave) bm[i] = 0u;
    wave_sync();
    for (int32_t c = lane; c < g.cells; c += kWave) {
        const int32_t occ = e.entity[c];
        const bool wall = h.terrain[c] != 0;
        if (occ == kAbsent && !wall) continue;
        const int32_t yy = cell_y(g, c), x = c - yy * g.W;
        const int32_t word = yy * g.seen_words + (x >> 5);
        const uint32_t bit = 1u << (x & 31);
        __atomic_fetch_or(&bm[word], bit, __ATOMIC_RELAXED);
        if (occ == kAbsent) continue;
        const int32_t s = gidx(occ, g.E);
        const int32_t o = e.owner[s];
        const int32_t fl = tabv(h, F_FLAGS, clampi(e.utype[s], 0, g.T - 1));
        if (o == 0 || o == 1) {
            __atomic_fetch_or(&bm[(1 + o) * plane + word], bit, __ATOMIC_RELAXED);
            if (fl & FL_STOCKPILE) __atomic_fetch_or(&bm[(4 + o) * plane + word], bit, __ATOMIC_RELAXED);
        }
        if (fl & FL_RESOURCE) __atomic_fetch_or(&bm[3 * plane + word], bit, __ATOMIC_RELAXED);
    }
    wave_sync();
}

// Bits [x0, x0 + nbits) of a bitmap row; positions off the row read 0.
NR_DEV uint32_t row_window(AS3 const uint32_t* row, int32_t words, int32_t x0, int32_t nbits) {
    int32_t lead = 0;
    if (x0 < 0) {
        lead = -x0;
        x0 = 0;
    }
    const int32_t w = x0 >> 5;
    uint64_t v = 0;
    if (w < words) v = row[w];
    if (w + 1 < words) v |= (uint64_t)row[w + 1] << 32;
    v = (v >> (x0 & 31)) << lead;
    return (uint32_t)v & ((1u << nbits) - 1u);
}

// legality_row from the bitmaps (same bits; owners of owned slots are 0/1).
NR_DEV Row legality_row_bm(const KGame& g, const Hdr& h, const Env& e, int32_t slot) {
    Row r;
    r.w[0] = r.w[1] = r.w[2] = 0u;
    if (e.birth[slot] == kAbsent) return r;
    const int32_t owner = e.owner[slot];
    if (owner != 0 && owner != 1) return legality_row(g, h, e, slot);
    const int32_t actor = clampi(e.utype[slot], 0, g.T - 1);
    const int32_t carried = e.carried[slot];
    const int32_t cell = e.cell[slot];
    const int32_t flags = tabv(h, F_FLAGS, actor);
    const int32_t balance = e.sc[S_RES0 + owner];
    uint32_t affordable = 0u;
    for (int32_t t = 0; t < g.T; ++t)
        if (balance >= tabv(h, F_COST, t)) affordable |= 1u << t;
    const uint32_t types = (uint32_t)tabv(h, F_PRODUCES, actor) & affordable;
    const int32_t x = cell_x(g, cell), yy = cell_y(g, cell);
    const int32_t words = g.seen_words, plane = g.H * words;
    AS3 const uint32_t* bm = at<uint32_t>(e, g.lay.o_bm);
    // 3-bit windows (x-1 .. x+1) of the rows above, at and below the unit
    uint32_t blk[3] = {7u, 7u, 7u}, res[3] = {0u, 0u, 0u}, stk[3] = {0u, 0u, 0u};
#pragma unroll
    for (int32_t k = 0; k < 3; ++k) {
        const int32_t ry = yy - 1 + k;
        if (ry < 0 || ry >= g.H) continue;
        AS3 const uint32_t* row = bm + ry * words;
        blk[k] = row_window(row, words, x - 1, 3);
        res[k] = row_window(row + 3 * plane, words, x - 1, 3);
        stk[k] = row_window(row + (4 + owner) * plane, words, x - 1, 3);
        if (x - 1 < 0) blk[k] |= 1u;
        if (x + 1 >= g.W) blk[k] |= 4u;
    }
    // direction d -> (row k, bit b): up (0,1) right (1,2) down (2,1) left (1,0)
    uint32_t free4 = 0u, res4 = 0u, stk4 = 0u;
    const int32_t dk[4] = {0, 1, 2, 1}, db[4] = {1, 2, 1, 0};
#pragma unroll
    for (int32_t d = 0; d < 4; ++d) {
        free4 |= (((blk[dk[d]] >> db[d]) & 1u) ^ 1u) << d;
        res4 |= ((res[dk[d]] >> db[d]) & 1u) << d;
        stk4 |= ((stk[dk[d]] >> db[d]) & 1u) << d;
    }
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
        const int32_t range = tabv(h, F_RANGE, actor);
        const int32_t reach = imin(range, g.radius);
        AS3 const uint32_t* enemy = bm + (2 - owner) * plane;
        uint64_t att = 0;
        if (g.fast_obs && range >= 0 && range <= g.disk_r) {
            // rows of the attack disk from the disk table, clipped to the window
            AS3 const uint32_t* disk = h.disk + range * (2 * g.disk_r + 1) + g.disk_r;
            const uint32_t window = (2u << (2 * reach)) - 1u;
            for (int32_t dy = -g.radius; dy <= g.radius; ++dy) {
                const int32_t ty = yy + dy;
                if (dy < -reach || dy > reach || ty < 0 || ty >= g.H) continue;
                const uint32_t span = (disk[dy] >> (g.disk_r - reach)) & window;
                const uint32_t bits = row_window(enemy + ty * words, words, x - reach, 2 * reach + 1) & span;
                att |= (uint64_t)bits << ((g.radius + dy) * g.side + g.radius - reach);
            }
        } else {
            for (int32_t dy = -reach; dy <= reach; ++dy) {
                const int32_t ty = yy + dy;
                if (ty < 0 || ty >= g.H) continue;
                const int32_t rem = range * range - dy * dy;
                int32_t hw = reach;
                while (hw * hw > rem) --hw;
                const uint32_t span = ((1u << (2 * hw + 1)) - 1u) << (reach - hw);
                const uint32_t bits = row_window(enemy + ty * words, words, x - reach, 2 * reach + 1) & span;
                att |= (uint64_t)bits << ((g.radius + dy) * g.side + g.radius - reach);
            }
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

// Symbolic observations of both agents in one pass over the cells
// (N/observations/symbolic.py:130-180, visibility.py:56-71).
NR_DEV void observe_all(const KGame& g, const Hdr& h, const Env& e_in, int lane, bool partial, uint8_t* maps0,
                        uint8_t* maps1, int32_t* scalars0, int32_t* scalars1) {
    const Env e = refresh(g, e_in);
    const Layout& y = g.lay;
    AS3 uint32_t* seen = at<uint32_t>(e, y.v_oseen);  // [2][H][seen_words]
    const int32_t plane = g.H * g.seen_words;
    if (partial) {
        for (int32_t i = lane; i < 2 * plane; i += kWave) seen[i] = 0u;
        wave_sync();
        // each lane stamps the sight disk of one active unit, row by row
        for (int32_t base = 0; base < 2 * g.C; base += kWave) {
            const int32_t i = base + lane;
            if (i >= 2 * g.C) continue;
            const int32_t s = g.N + i;
            if (e.birth[s] == kAbsent) continue;
            const int32_t r = tabv(h, F_SIGHT, gidx(e.utype[s], g.T));
            const int32_t cell = e.cell[s];
            const int32_t cx = cell_x(g, cell), cy = cell_y(g, cell);
            AS3 uint32_t* mine = seen + (i / g.C) * plane;
            int32_t hw = r;
            for (int32_t dy = 0; dy <= r; ++dy) {
                const int32_t rem = r * r - dy * dy;
                while (hw * hw > rem) --hw;
                const int32_t x0 = cx - hw < 0 ? 0 : cx - hw;
                const int32_t x1 = cx + hw >= g.W ? g.W - 1 : cx + hw;
                if (x0 > x1) continue;
                for (int32_t side = 0; side < (dy == 0 ? 1 : 2); ++side) {
                    const int32_t ry = side == 0 ? cy - dy : cy + dy;
                    if (ry < 0 || ry >= g.H) continue;
                    for (int32_t wd = x0 >> 5; wd <= (x1 >> 5); ++wd) {
                        const int32_t a = x0 > wd * 32 ? x0 - wd * 32 : 0;
                        const int32_t b = x1 < wd * 32 + 31 ? x1 - wd * 32 : 31;
                        const uint32_t bits = (b - a == 31) ? 0xFFFFFFFFu : (((1u << (b - a + 1)) - 1u) << a);
                        __atomic_fetch_or(&mine[ry * g.seen_words + wd], bits, __ATOMIC_RELAXED);
                    }
                }
            }
        }
        wave_sync();
    }
    AS3 uint8_t* stage0 = at<uint8_t>(e, y.v_stage);
    AS3 uint8_t* stage1 = stage0 + g.stage_cells * 6;
    constexpr int kPer = 4;  // cells per lane per staging block (stage_cells <= 256)
    for (int32_t c0 = 0; c0 < g.cells; c0 += g.stage_cells) {
        const int32_t nc = imin(g.stage_cells, g.cells - c0);
        // gather first (independent loads), then encode and stage
        int32_t occ[kPer];
#pragma unroll
        for (int k = 0; k < kPer; ++k) {
            const int32_t i = lane + k * kWave;
            occ[k] = i < nc ? (int32_t)e.entity[c0 + i] : kAbsent;
        }
        uint32_t word[kPer];
#pragma unroll
        for (int k = 0; k < kPer; ++k) {
            word[k] = 0u;
            if (occ[k] != kAbsent) {
                const int32_t s = clampi(occ[k], 0, g.E - 1);
                const uint32_t hp = (uint32_t)(int32_t)e.hp[s] & 0xFFu;
                const uint32_t carried = (uint32_t)e.carried[s] & 0xFFu;
                const uint32_t type = (uint32_t)((int32_t)e.utype[s] + 1) & 0xFFu;
                const int32_t pk = e.pkind[s];
                const uint32_t kind = (uint32_t)(pk > 0 ? pk : 0) & 0xFu;
                const uint32_t owner = (uint32_t)((int32_t)e.owner[s] + 1) & 0x3u;
                word[k] = hp | (carried << 8) | (type << 16) | (kind << 24) | (owner << 28);
            }
        }
#pragma unroll
        for (int k = 0; k < kPer; ++k) {
            const int32_t i = lane + k * kWave;
            if (i >= nc) continue;
            const int32_t c = c0 + i;
            const uint32_t terrain = (uint32_t)h.terrain[c] << 8;
            const uint32_t w = word[k];
            const uint32_t owner = w >> 28;
            const int32_t yy = cell_y(g, c), x = c - yy * g.W;
#pragma unroll
            for (int32_t pl = 0; pl < 2; ++pl) {
                bool shown = true;
                if (partial) {
                    const uint32_t sw = seen[pl * plane + yy * g.seen_words + (x >> 5)];
                    shown = owner == (uint32_t)(pl + 1) || ((sw >> (x & 31)) & 1u);
                }
                AS3 uint16_t* out = (AS3 uint16_t*)((pl == 0 ? stage0 : stage1) + i * 6);
                if (shown) {
                    const uint32_t rel = owner > 0 ? (uint32_t)((((int32_t)owner - 1 + pl) & 1) + 1) : 0u;
                    out[0] = (uint16_t)(w & 0xFFFFu);
                    out[1] = (uint16_t)(rel | (((w >> 16) & 0xFFu) << 8));
                    out[2] = (uint16_t)(((w >> 24) & 0xFu) | terrain);
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
