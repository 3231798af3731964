/*
 * GridNet action decode (the MicroRTS-Py per-cell action surface).
 * TEST INFRASTRUCTURE ONLY (part of the CPU oracle; nanorts_oracle.c
 * includes this file so it shares the env view and legality rows).
 *
 * Restates N/adapters/gridnet/actions.py:31-52 (_decode), :91-125
 * (_decode_rows), :139-184 (_player_commands, _idle_fillers, _filler_ranks)
 * and N/adapters/gridnet/source_filter.py:51-139 (direction_delta,
 * pending_usage, keep, issued_usage, position_domain), with the factor
 * helpers of N/adapters/factors.py:117-151.
 */

static inline int32_t grid_delta(int32_t direction, int32_t W) {
    /* source_filter.direction_delta: codes 0..3 move by their offset, any
       other value by 0 */
    if (direction < 0 || direction > 3) return 0;
    return DIRECTION_DX[direction] + DIRECTION_DY[direction] * W;
}

/* A gather from a [n] table: a negative index wraps once, then clamps. */
static inline int32_t gather_i32(const int32_t* table, int32_t n, int32_t index) {
    return table[gidx(index, n)];
}

typedef struct grid_row_t {
    int32_t slot, cell, kind, direction, none_duration, target_cell, produced_type, position, has_position, cost;
    int survived;
} grid_row_t;

static void gridnet_decode_one(const nro_game* g, const env_t* e, const int32_t* actions /* [2][cells][7] */,
                               cmd_t* cmds, grid_row_t* rows, uint8_t* base, uint8_t* used, uint8_t* legal_row) {
    const int32_t N = g->neutral, C = g->capacity, W = g->width, H = g->height, cells = g->cells, T = g->types;
    const int32_t domain = cells + 2 * W + 1, margin = W;
    int32_t side = 1;
    while (side * side < g->offsets) ++side;
    const int32_t radius = (side - 1) / 2;
    /* pending_usage (:65-85): claimed positions and pending production cost;
       each player's filter starts from these (plus player 0's issued usage
       for player 1) on a copy */
    memset(base, 0, (size_t)domain);
    int32_t base_spent[2] = {0, 0};
    for (int32_t s = 0; s < g->entities; ++s) {
        if (!active(e, s)) continue;
        const int32_t kind = e->pending_kind[s];
        if (kind == KIND_MOVE || kind == KIND_PRODUCE) {
            const int32_t idx = e->cell[s] + grid_delta(e->pending_direction[s], W) + margin;
            if (idx >= 0 && idx < domain - 1) base[idx] = 1;
        }
        if (kind == KIND_PRODUCE && s >= N)
            base_spent[(s - N) / C] = wadd(base_spent[(s - N) / C], gather_i32(g->cost, T, e->pending_produced_type[s]));
    }
    for (int32_t player = 0; player < 2; ++player) {
        const int32_t first = N + player * C;
        /* _decode_rows: available units by cell (stable), then the rest */
        int32_t count = 0;
        for (int32_t i = 0; i < C; ++i) {
            const int32_t s = first + i;
            if (active(e, s) && e->pending_kind[s] == KIND_ABSENT) rows[count++].slot = i;
        }
        for (int32_t x = 1; x < count; ++x) {
            const grid_row_t v = rows[x];
            int32_t y = x - 1;
            while (y >= 0 && e->cell[first + rows[y].slot] > e->cell[first + v.slot]) {
                rows[y + 1] = rows[y];
                --y;
            }
            rows[y + 1] = v;
        }
        for (int32_t k = 0; k < count; ++k) {
            grid_row_t* r = &rows[k];
            const int32_t at_cell = e->cell[first + r->slot];
            const int32_t* row = actions + ((size_t)player * cells + clampi(at_cell, 0, cells - 1)) * 7;
            const int32_t kind = row[0];
            r->cell = at_cell;
            r->kind = kind;
            r->direction = kind == KIND_MOVE ? row[1]
                           : kind == KIND_HARVEST ? row[2]
                           : kind == KIND_RETURN ? row[3]
                           : kind == KIND_PRODUCE ? row[4]
                           : ABSENT;
            r->produced_type = kind == KIND_PRODUCE ? row[5] : ABSENT;
            const int32_t tx = wadd(floor_mod(at_cell, W), floor_mod(row[6], side) - radius);
            const int32_t ty = wadd(floor_div(at_cell, W), floor_div(row[6], side) - radius);
            const int on_board = tx >= 0 && tx < W && ty >= 0 && ty < H;
            r->target_cell = (kind == KIND_ATTACK && on_board) ? ty * W + tx : ABSENT;
            r->none_duration = kind == KIND_NONE ? -1 : 0;
            r->position = wadd(at_cell, grid_delta(r->direction, W));
            r->has_position = kind == KIND_MOVE || kind == KIND_PRODUCE;
            r->cost = kind == KIND_PRODUCE ? gather_i32(g->cost, T, row[5]) : 0;
            r->survived = 0;
        }
        /* keep (:88-121): in cell order, a claim on a used position or a
           cost that overdraws a player already spending is dropped */
        memcpy(used, base, (size_t)domain);
        int32_t spent[2] = {base_spent[0], base_spent[1]};
        for (int32_t k = 0; k < count; ++k) {
            grid_row_t* r = &rows[k];
            const int32_t index = r->has_position ? wadd(r->position, margin) : domain - 1;
            const int32_t idx = gidx(index, domain);
            int32_t total[2];
            int over = 0;
            for (int32_t q = 0; q < 2; ++q) {
                total[q] = wadd(spent[q], q == player ? r->cost : 0);
                over |= spent[q] != 0 && total[q] > 0 && total[q] > e->resources[q];
            }
            const int consistent = !(r->has_position && used[idx]) && !over;
            if (consistent) {
                if (r->has_position) used[idx] = 1;
                spent[0] = total[0];
                spent[1] = total[1];
                r->survived = 1;
            }
        }
        /* issued_usage (:124-139): player 0's kept legal claims and costs
           seed player 1's filter */
        if (player == 0) {
            int32_t produced = 0;
            for (int32_t k = 0; k < count; ++k) {
                const grid_row_t* r = &rows[k];
                if (!r->survived || !r->has_position) continue;
                legality_row(g, e, first + r->slot, legal_row);
                int legal;
                if (r->kind == KIND_MOVE) {
                    legal = legal_row[6 + gidx(r->direction, 4)];
                } else {
                    legal = legal_row[18 + gidx(r->direction, 4)] && legal_row[22 + gidx(r->produced_type, T)];
                }
                if (!legal) continue;
                const int32_t idx = wadd(r->position, margin);
                if (idx >= 0 && idx < domain - 1) base[idx] = 1;
                if (r->kind == KIND_PRODUCE) produced = wadd(produced, r->cost);
            }
            base_spent[0] = wadd(base_spent[0], produced);
        }
        /* _player_commands: survivors in cell order, then idle fillers by birth */
        int32_t survivors = 0;
        for (int32_t k = 0; k < count; ++k) survivors += rows[k].survived;
        for (int32_t i = 0; i < C; ++i) {
            cmd_t x = {KIND_ABSENT, ABSENT, 0, ABSENT, ABSENT, ABSENT};
            cmds[player * C + i] = x;
        }
        int32_t rank = 0;
        for (int32_t k = 0; k < count; ++k) {
            const grid_row_t* r = &rows[k];
            if (!r->survived) continue;
            cmd_t* c = &cmds[player * C + r->slot];
            c->kind = r->kind;
            c->direction = r->direction;
            c->none_duration = r->none_duration;
            c->target_cell = r->target_cell;
            c->produced_type = r->produced_type;
            c->request_order = rank++;
        }
        /* idle fillers: available units without a kept row (marked first,
           then ranked by birth, stable on the slot) */
        for (int32_t i = 0; i < C; ++i) {
            const int32_t s = first + i;
            rows[i].has_position = active(e, s) && e->pending_kind[s] == KIND_ABSENT &&
                                   cmds[player * C + i].kind == KIND_ABSENT;
        }
        for (int32_t i = 0; i < C; ++i) {
            if (!rows[i].has_position) continue;
            const int32_t s = first + i;
            int32_t below = 0;
            for (int32_t j = 0; j < C; ++j) {
                const int32_t t = first + j;
                if (rows[j].has_position && (e->birth[t] < e->birth[s] || (e->birth[t] == e->birth[s] && j < i)))
                    ++below;
            }
            cmd_t* c = &cmds[player * C + i];
            c->kind = KIND_NONE;
            c->none_duration = 1;
            c->request_order = wadd(below, survivors);
        }
    }
}

void nro_gridnet_decode(const nro_game* g, const nro_state* s, const int32_t* actions, int64_t L,
                        nro_commands* out) {
    const int32_t C = g->capacity, owned = 2 * C, cells = g->cells;
    cmd_t* cmds = (cmd_t*)malloc(sizeof(cmd_t) * (size_t)owned);
    grid_row_t* rows = (grid_row_t*)malloc(sizeof(grid_row_t) * (size_t)C);
    uint8_t* base = (uint8_t*)malloc((size_t)(cells + 2 * g->width + 1));
    uint8_t* used = (uint8_t*)malloc((size_t)(cells + 2 * g->width + 1));
    uint8_t* legal = (uint8_t*)malloc((size_t)row_width(g));
    for (int64_t l = 0; l < L; ++l) {
        env_t e = env_of(g, s, l);
        gridnet_decode_one(g, &e, actions + (size_t)l * 2 * cells * 7, cmds, rows, base, used, legal);
        for (int32_t p = 0; p < owned; ++p) {
            const int64_t at = l * owned + p;
            out->kind[at] = cmds[p].kind;
            out->direction[at] = cmds[p].direction;
            out->none_duration[at] = cmds[p].none_duration;
            out->target_cell[at] = cmds[p].target_cell;
            out->produced_type[at] = cmds[p].produced_type;
            out->request_order[at] = cmds[p].request_order;
        }
    }
    free(legal);
    free(base);
    free(used);
    free(rows);
    free(cmds);
}
