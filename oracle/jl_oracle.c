/*
 * jl_oracle.c - CPU oracle for the JointLoom hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file restates, in plain sequential C, the
 * algorithms of the reference implementation so that the HIP kernels in
 * iclr_2027_jointoom_amd/csrc can be checked bit for bit.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it, and
 * only as a checker; the product path never calls it.
 *
 * The descriptor structs of include/jointloom.h are reused with HOST
 * pointers.  Every function cites the reference file:line it follows
 * (paths relative to /root/reference/src).
 *
 * Pinning (what fixes each function independently of this text):
 *   jlo_encode_map          closed form bit layout, grid_world_cuda.h:17-23
 *   jlo_step / resolvers    9 DIRECTED_FIXTURES KATs, stateful-standard KATs,
 *                           512-agent chain, naive-vs-event brute force,
 *                           invariants (no shared cell, no swap)
 *   jlo_bfs_u16             corridor KAT (distance 256), Manhattan closed form
 *                           on empty grids, brute-force Bellman-Ford
 *   jlo_energy_u8           goal cell 255 KAT, closed form 255-d / cap at 254
 *   jlo_mapfgpt_*           tokenizer KATs (vocabulary, sentinels, top-13
 *                           ordering), closed-form cost/greedy tokens on
 *                           empty grids, history roll KAT
 *   jlo_magat_*             cell-level FOV KATs, edge closed forms,
 *                           integer goal-projection identity
 *   jlo_splitmix64          published outputs of SplitMix64 from state 0
 *   jlo_xorshift64s         an independent pure-Python restatement of the
 *                           published generator, period structure checks
 *   jlo_free_cells, jlo_init_agents, random lifelong goals
 *                           hand-derived known answers, a set-based
 *                           Python restatement on seeded rollouts, and the
 *                           rule's invariants (distinct cells, free cells
 *                           inside the real extent, reserved goals skipped)
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "../include/jointloom.h"

#define JLO_UNREACHABLE 0xFFFFu
#define JLO_CONTEXT 256
#define JLO_RADIUS 5
#define JLO_DIAM 11
#define JLO_COST_TOKENS 121
#define JLO_VISIBLE 13
#define JLO_AGENT_TOKENS 10
#define JLO_COST_LIMIT 20
#define JLO_TOK_UNREACHABLE 41
#define JLO_TOK_NEG_CLIP 42
#define JLO_TOK_POS_CLIP 43
#define JLO_TOK_EMPTY_ACTION 44
#define JLO_TOK_WAIT 45
#define JLO_TOK_GREEDY 50
#define JLO_TOK_PAD 66
#define JLO_MAX_FRONTIER 4096
#define JLO_PYG_DIAM 13
#define JLO_PYG_AREA 169
#define JLO_COMM_RADIUS_SQ 49

/* Squared distance in 32-bit int arithmetic as the reference computes it
 * (stateless_step.cu:513-520, :889): for int16 positions near opposite
 * extremes the products and sum wrap modulo 2^32; done in unsigned so the
 * wrap is defined. */
static inline int jlo_dist2(int dx, int dy) {
    return (int)((uint32_t)dx * (uint32_t)dx + (uint32_t)dy * (uint32_t)dy);
}

static const int ACT_DX[5] = {0, -1, 1, 0, 0};
static const int ACT_DY[5] = {0, 0, 0, -1, 1};

/* ------------------------------------------------------------------ */
/* Map encoding: grid_world_cuda.cu:112-146 (32 consecutive int32 cells */
/* of the flat [E, W, H] array per uint32 word, bit i = cell i).        */
/* ------------------------------------------------------------------ */
void jlo_encode_map(const int32_t* grids, uint32_t* bits, int n_envs, int W, int H) {
    const int64_t cells = (int64_t)n_envs * W * H;
    for (int64_t w = 0; w < cells / 32; ++w) {
        uint32_t v = 0;
        for (int i = 0; i < 32; ++i) {
            if (grids[w * 32 + i] != 0) v |= 1u << i;
        }
        bits[w] = v;
    }
}

static inline int bit_at(const uint32_t* env_bits, int cell) {
    return (int)((env_bits[cell >> 5] >> (cell & 31)) & 1u);
}

/* is_wall, 128_agents_map_step.cu:12-16: out of [0,W)x[0,H) is a wall. */
static inline int is_wall(const uint32_t* env_bits, int W, int H, int x, int y) {
    if (x < 0 || x >= W || y < 0 || y >= H) return 1;
    return bit_at(env_bits, x * H + y);
}

/* ------------------------------------------------------------------ */
/* Conflict resolution for one env.                                     */
/* Inputs: current cells cx/cy, proposal nx/ny (already wall-checked).  */
/* Outputs: final nx/ny and per-agent category (only filled where 0).   */
/* ------------------------------------------------------------------ */

/* Literal restatement of the Jacobi scan of step_kernel,
 * 128_agents_map_step.cu:91-169: each round decides every moving agent
 * against the previous round's proposals of all other agents (Manhattan
 * prefilter <= 2), rejections apply together, stop at a round without
 * rejections or after A rounds.  The category of a rejection is that of the
 * first colliding k in ascending order, swap before vertex before chain,
 * as in the CPU restatement transition_adapters.py:414-445. */
static void resolve_naive(int A, const int* cx, const int* cy, int* nx, int* ny,
                          uint8_t* cat) {
    int* tx = (int*)malloc(sizeof(int) * (size_t)A * 2);
    int* ty = tx + A;
    for (int iter = 0; iter < A; ++iter) {
        int changed = 0;
        for (int i = 0; i < A; ++i) {
            tx[i] = nx[i];
            ty[i] = ny[i];
            if (nx[i] == cx[i] && ny[i] == cy[i]) continue;
            int c = 0;
            for (int k = 0; k < A && !c; ++k) {
                if (k == i) continue;
                if (abs(cx[i] - cx[k]) + abs(cy[i] - cy[k]) > 2) continue;
                if (nx[i] == cx[k] && ny[i] == cy[k] && nx[k] == cx[i] && ny[k] == cy[i]) {
                    c = JL_OUTCOME_SWAP;
                } else if (nx[i] == nx[k] && ny[i] == ny[k] && i > k) {
                    c = JL_OUTCOME_VERTEX;
                } else if (nx[i] == cx[k] && ny[i] == cy[k] && nx[k] == cx[k] && ny[k] == cy[k]) {
                    c = JL_OUTCOME_CHAIN;
                }
            }
            if (c) {
                tx[i] = cx[i];
                ty[i] = cy[i];
                if (cat[i] == 0) cat[i] = (uint8_t)c;
                changed = 1;
            }
        }
        for (int i = 0; i < A; ++i) {
            nx[i] = tx[i];
            ny[i] = ty[i];
        }
        if (!changed) break;
    }
    free(tx);
}

/* Event-indexed formulation, transition_adapters.py:392-449: the only
 * agents that can reject mover i are the current occupant of i's
 * destination and the smallest-id agent proposing that destination.  Uses
 * dense per-cell tables of the env (W*H entries). */
static void resolve_event(int A, int W, int H, const int* cx, const int* cy, int* nx,
                          int* ny, uint8_t* cat) {
    const int cells = W * H;
    int* owner = (int*)malloc(sizeof(int) * (size_t)cells * 2);
    int* minid = owner + cells;
    int* rej = (int*)malloc(sizeof(int) * (size_t)A);
    for (int c = 0; c < cells; ++c) owner[c] = -1;
    /* current_owner dict: last agent wins on a shared cell (:390-392) */
    for (int k = 0; k < A; ++k) owner[cx[k] * H + cy[k]] = k;
    for (int iter = 0; iter < A; ++iter) {
        for (int k = 0; k < A; ++k) minid[nx[k] * H + ny[k]] = A;
        for (int k = 0; k < A; ++k) {
            int c = nx[k] * H + ny[k];
            if (k < minid[c]) minid[c] = k;
        }
        int nrej = 0;
        for (int i = 0; i < A; ++i) {
            rej[i] = 0;
            if (nx[i] == cx[i] && ny[i] == cy[i]) continue;
            const int dest = nx[i] * H + ny[i];
            int cand[2];
            int nc = 0;
            const int o = owner[dest];
            if (o >= 0 && o != i) cand[nc++] = o;
            const int m = minid[dest];
            if (m < i && !(nc == 1 && cand[0] == m)) cand[nc++] = m;
            if (nc == 2 && cand[1] < cand[0]) {
                int t = cand[0];
                cand[0] = cand[1];
                cand[1] = t;
            }
            int c = 0;
            for (int j = 0; j < nc && !c; ++j) {
                const int k = cand[j];
                if (nx[i] == cx[k] && ny[i] == cy[k] && nx[k] == cx[i] && ny[k] == cy[i]) {
                    c = JL_OUTCOME_SWAP;
                } else if (i > k && nx[i] == nx[k] && ny[i] == ny[k]) {
                    c = JL_OUTCOME_VERTEX;
                } else if (nx[i] == cx[k] && ny[i] == cy[k] && nx[k] == cx[k] && ny[k] == cy[k]) {
                    c = JL_OUTCOME_CHAIN;
                }
            }
            if (c) {
                rej[i] = c;
                ++nrej;
            }
        }
        if (!nrej) break;
        for (int i = 0; i < A; ++i) {
            if (!rej[i]) continue;
            nx[i] = cx[i];
            ny[i] = cy[i];
            if (cat[i] == 0) cat[i] = (uint8_t)rej[i];
        }
    }
    free(rej);
    free(owner);
}

/* One-env conflict resolution on raw inputs, for brute-force tests.
 * cur: int32 [A,2]; arrived/actions: [A]; out_pos: int32 [A,2];
 * out_cat: [A].  Proposal + wall rule: 128_agents_map_step.cu:54-82 and
 * transition_adapters.py:367-388 (requested = active and action in 1..4). */
void jlo_resolve_env(const uint32_t* env_bits, int W, int H, int A, const int32_t* cur,
                     const uint8_t* arrived, const uint8_t* actions, int32_t* out_pos,
                     uint8_t* out_cat, int naive) {
    int* buf = (int*)malloc(sizeof(int) * (size_t)A * 4);
    int *cx = buf, *cy = buf + A, *nx = buf + 2 * A, *ny = buf + 3 * A;
    for (int i = 0; i < A; ++i) {
        cx[i] = cur[2 * i];
        cy[i] = cur[2 * i + 1];
        int act = actions[i];
        if (act > 4) act = 0;
        out_cat[i] = 0;
        if (arrived && arrived[i]) {
            nx[i] = cx[i];
            ny[i] = cy[i];
            continue;
        }
        const int tx = cx[i] + ACT_DX[act], ty = cy[i] + ACT_DY[act];
        if (is_wall(env_bits, W, H, tx, ty)) {
            nx[i] = cx[i];
            ny[i] = cy[i];
            if (act != 0) out_cat[i] = JL_OUTCOME_WALL;
        } else {
            nx[i] = tx;
            ny[i] = ty;
        }
    }
    if (naive) {
        resolve_naive(A, cx, cy, nx, ny, out_cat);
    } else {
        resolve_event(A, W, H, cx, cy, nx, ny, out_cat);
    }
    for (int i = 0; i < A; ++i) {
        out_pos[2 * i] = nx[i];
        out_pos[2 * i + 1] = ny[i];
    }
    free(buf);
}

static void write_state_row(uint16_t* row, int env, int agent, int px, int py, int gx, int gy,
                            int action, int reset) {
    row[0] = (uint16_t)env;
    row[1] = (uint16_t)agent;
    row[2] = (uint16_t)px;
    row[3] = (uint16_t)py;
    row[4] = (uint16_t)gx;
    row[5] = (uint16_t)gy;
    row[6] = (uint16_t)action;
    row[7] = (uint16_t)reset;
}

/* Deterministic lifelong goals of one env after its move: the canonical
 * agent order of assign_goals (rebuttal/online-il/tasks.py:51-65), the CPU
 * twin of the candidate branch of 128_agents_map_step.cu:303-330 in
 * rebuttal/online-rl/native/src/cuda_backend.  Goals held by agents off
 * their goal are reserved; each agent on its goal, in id order, takes the
 * first cell of the env's list, from candidates[cursor % K] on, that is not
 * its own cell and not reserved, and reserves it.  Returns the number of
 * agents that found no cell (the CPU twin raises for them; the device leaves
 * their goal). */
static int assign_candidate_goals(const jl_sim_t* s, int e, const int32_t* fin) {
    const int A = s->n_agents, W = s->map_w, H = s->map_h;
    const int K = s->candidate_length;
    int count = s->candidate_counts[e];
    if (count > s->candidate_stride) count = s->candidate_stride;
    const uint16_t* cells = s->candidate_cells + (size_t)e * s->candidate_stride * 2;
    uint8_t* reserved = (uint8_t*)calloc((size_t)W * H, 1);
    uint8_t* reached = (uint8_t*)malloc((size_t)A);
    for (int i = 0; i < A; ++i) {
        const size_t g = (size_t)e * A + i;
        reached[i] = fin[2 * i] == s->goal_x[g] && fin[2 * i + 1] == s->goal_y[g];
        if (!reached[i]) reserved[s->goal_x[g] * H + s->goal_y[g]] = 1;
    }
    int failed = 0;
    for (int i = 0; i < A && count > 0; ++i) {
        if (!reached[i]) continue;
        const size_t g = (size_t)e * A + i;
        const int cursor = s->goal_cursors[g];
        int ci = cursor % K;
        if (ci < 0) ci += K;
        int begin = s->goal_candidates[g * K + ci] % count;
        if (begin < 0) begin += count;
        int done = 0;
        for (int off = 0; off < count && !done; ++off) {
            const int k = (int)(((int64_t)begin + off) % count);
            const int x = cells[2 * k], y = cells[2 * k + 1];
            if (x < 0 || x >= W || y < 0 || y >= H) continue;
            if (x == fin[2 * i] && y == fin[2 * i + 1]) continue;
            if (reserved[x * H + y]) continue;
            reserved[x * H + y] = 1;
            s->goal_x[g] = (uint16_t)x;
            s->goal_y[g] = (uint16_t)y;
            s->goal_changed[g] = 1;
            s->goal_cursors[g] = cursor + 1;
            done = 1;
        }
        failed += !done;
    }
    free(reached);
    free(reserved);
    return failed;
}

/* ---- generator-drawn lifelong goals and random placement ----------------
 * The reference draws from one cuRAND XORWOW stream per agent
 * (curand_init(seed, id, 0), grid_world_cuda.cu:458-479) with one thread per
 * agent racing on atomicOr (128_agents_map_step.cu:265-343,
 * grid_world_cuda.cu:405-436, utils_cuda.h:39-61), so its result depends on
 * thread timing and cannot be restated.  This build's device rule, restated
 * here, keeps the reference's search (a random start index into the env's
 * free-cell list, then a linear probe with wrap-around) and makes it
 * deterministic: one xorshift64* generator per agent (Marsaglia 2003, with
 * the output multiplier of Vigna 2016, "An experimental exploration of
 * Marsaglia's xorshift generators, scrambled") seeded through splitmix64
 * (Steele, Lea and Flood 2014), start index = (output >> 32) mod count, and
 * agents settled one after the other in id order. */
uint64_t jlo_splitmix64(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

uint64_t jlo_xorshift64s(uint64_t* state) {
    uint64_t x = *state;
    x ^= x >> 12;
    x ^= x << 25;
    x ^= x >> 27;
    *state = x;
    return x * 0x2545F4914F6CDD1Dull;
}

/* Per-agent generator states for init_rng(seed) (setup_rng_kernel,
 * grid_world_cuda.cu:458-470): state i = splitmix64(seed ^ splitmix64(i)),
 * a zero state replaced by the golden-ratio constant (xorshift states must
 * be nonzero). */
void jlo_seed_rng(uint64_t* state, int64_t count, uint64_t seed) {
    for (int64_t i = 0; i < count; ++i) {
        const uint64_t v = jlo_splitmix64(seed ^ jlo_splitmix64((uint64_t)i));
        state[i] = v ? v : 0x9E3779B97F4A7C15ull;
    }
}

/* Free cells of each env inside its real extent (cache_map_free_cells_kernel,
 * grid_world_cuda.cu:225-320): cells (x, y) with x < rw, y < rh and no
 * obstacle, packed x << 16 | y, in cell order (x major), at offset e*W*H of
 * free_cells; offsets[e] = e*W*H, or -1 for an env without a free cell. */
void jlo_free_cells(const jl_sim_t* s, const int32_t* extents, uint32_t* free_cells, int32_t* offsets,
                    int32_t* counts) {
    const int E = s->n_envs, W = s->map_w, H = s->map_h;
    const int words = W * H / 32;
    for (int e = 0; e < E; ++e) {
        const int rw = extents[2 * e], rh = extents[2 * e + 1];
        const uint32_t* bits = s->grid_bits + (size_t)e * words;
        uint32_t* out = free_cells + (size_t)e * W * H;
        int n = 0;
        for (int x = 0; x < W && x < rw; ++x)
            for (int y = 0; y < H && y < rh; ++y) {
                const int cell = x * H + y;
                if (!((bits[cell >> 5] >> (cell & 31)) & 1u)) out[n++] = ((uint32_t)x << 16) | (uint32_t)y;
            }
        counts[e] = n;
        offsets[e] = n > 0 ? e * W * H : -1;
    }
}

/* Random distinct starts and goals (init_agents_kernel,
 * grid_world_cuda.cu:405-436, with find_unique_slot utils_cuda.h:39-61):
 * agents in id order, each drawing a start and then a goal: a start index
 * into the env's list, then the first list entry at or after it (with
 * wrap-around) not taken by an earlier draw of the env.  A draw that finds
 * no entry (more than count draws) leaves 0xFFFF coordinates, where the
 * reference would search forever. */
void jlo_init_agents(const jl_sim_t* s, const uint32_t* free_cells, const int32_t* offsets,
                     const int32_t* counts) {
    const int E = s->n_envs, A = s->n_agents;
    for (int e = 0; e < E; ++e) {
        const int count = counts[e], offset = offsets[e];
        uint8_t* used = (uint8_t*)calloc((size_t)(count > 0 ? count : 1), 1);
        for (int a = 0; a < A; ++a) {
            const size_t g = (size_t)e * A + a;
            uint64_t st = s->rng_state[g];
            uint32_t picked[2] = {0xFFFFFFFFu, 0xFFFFFFFFu};
            for (int which = 0; which < 2 && count > 0; ++which) {
                int k = (int)((jlo_xorshift64s(&st) >> 32) % (uint64_t)count);
                for (int attempt = 0; attempt < count; ++attempt) {
                    if (!used[k]) {
                        used[k] = 1;
                        picked[which] = free_cells[offset + k];
                        break;
                    }
                    if (++k >= count) k = 0;
                }
            }
            s->rng_state[g] = st;
            s->cur_x[g] = (uint16_t)(picked[0] >> 16);
            s->cur_y[g] = (uint16_t)(picked[0] & 0xFFFFu);
            s->goal_x[g] = (uint16_t)(picked[1] >> 16);
            s->goal_y[g] = (uint16_t)(picked[1] & 0xFFFFu);
        }
        free(used);
    }
}

/* Generator-drawn lifelong goals of one env after its move
 * (128_agents_map_step.cu:265-343, made deterministic as above): goals of
 * agents off their goal are reserved; each agent on its goal, in id order,
 * draws a start index into the env's free-cell list and takes the first
 * entry at or after it (with wrap-around) whose cell is not reserved, and
 * reserves it.  Its own cell is not reserved, so it may draw it again (the
 * goal is then unchanged but still flagged, as in the reference).  The
 * generator advances once per agent on its goal, whether or not a cell is
 * found.  Goals outside the map reserve nothing. */
static void assign_random_goals(const jl_sim_t* s, int e, const int32_t* fin) {
    const int A = s->n_agents, W = s->map_w, H = s->map_h;
    const int count = s->env_counts[e], offset = s->env_offsets[e];
    uint8_t* reserved = (uint8_t*)calloc((size_t)W * H, 1);
    for (int i = 0; i < A; ++i) {
        const size_t g = (size_t)e * A + i;
        const int gx = s->goal_x[g], gy = s->goal_y[g];
        if (fin[2 * i] == gx && fin[2 * i + 1] == gy) continue;
        if (gx < W && gy < H) reserved[gx * H + gy] = 1;
    }
    for (int i = 0; i < A && count > 0; ++i) {
        const size_t g = (size_t)e * A + i;
        if (fin[2 * i] != s->goal_x[g] || fin[2 * i + 1] != s->goal_y[g]) continue;
        uint64_t st = s->rng_state[g];
        int k = (int)((jlo_xorshift64s(&st) >> 32) % (uint64_t)count);
        for (int attempt = 0; attempt < count; ++attempt) {
            const uint32_t packed = s->free_cells[offset + k];
            const int x = (int)(packed >> 16), y = (int)(packed & 0xFFFFu);
            if (x < W && y < H && !reserved[x * H + y]) {
                reserved[x * H + y] = 1;
                s->goal_x[g] = (uint16_t)x;
                s->goal_y[g] = (uint16_t)y;
                s->goal_changed[g] = 1;
                break;
            }
            if (++k >= count) k = 0;
        }
        s->rng_state[g] = st;
    }
    free(reserved);
}

/* Batched step, step_kernel 128_agents_map_step.cu:25-262 (positions are
 * cached as uint8 there, :39-43; supported maps are at most 256 wide so the
 * cache is exact).  CostTracer steps (task mode 2, rebuttal/online-rl/native/
 * src/cuda_backend/128_agents_map_step.cu:219-222) count the step and stop
 * before the packed rows.  Lifelong steps with candidate lists take new goals
 * in canonical order (assign_candidate_goals) and count the step; without
 * them, given the generator states and free-cell lists, goals are drawn by
 * assign_random_goals (the reference's :265-343 rule made deterministic; no
 * step count, as there), and with neither goals stay as a step without
 * arrivals would leave them. */
void jlo_step(const jl_sim_t* s, int naive) {
    const int E = s->n_envs, A = s->n_agents, W = s->map_w, H = s->map_h;
    const int words = W * H / 32;
    const int standard = s->task_mode == JL_TASK_STANDARD_MAPF;
    const int costtracer = s->task_mode == JL_TASK_COSTTRACER;
    const int by_candidates = s->task_mode == JL_TASK_LIFELONG && s->goal_candidates != NULL;
    const int by_draws = s->task_mode == JL_TASK_LIFELONG && !by_candidates && s->rng_state != NULL &&
                         s->free_cells != NULL && s->env_offsets != NULL && s->env_counts != NULL;
    int32_t* cur = (int32_t*)malloc(sizeof(int32_t) * (size_t)A * 4);
    int32_t* fin = cur + 2 * A;
    uint8_t* cat = (uint8_t*)malloc((size_t)A);
    uint8_t* was_arrived = (uint8_t*)malloc((size_t)A);
    for (int e = 0; e < E; ++e) {
        /* done envs do not advance (:31-34) */
        if (standard && (s->terminated[e] || s->truncated[e])) {
            if (s->outcomes) memset(s->outcomes + (size_t)e * A, 0, (size_t)A);
            continue;
        }
        const uint32_t* env_bits = s->grid_bits + (size_t)e * words;
        for (int i = 0; i < A; ++i) {
            const size_t g = (size_t)e * A + i;
            cur[2 * i] = s->cur_x[g];
            cur[2 * i + 1] = s->cur_y[g];
            was_arrived[i] = (uint8_t)(standard && s->arrived[g] != 0);
        }
        jlo_resolve_env(env_bits, W, H, A, cur, was_arrived, s->actions + (size_t)e * A, fin, cat,
                        naive);
        uint32_t* ocp = s->grid_ocp + (size_t)e * words;
        memset(ocp, 0, sizeof(uint32_t) * (size_t)words);
        for (int i = 0; i < A; ++i) {
            const size_t g = (size_t)e * A + i;
            const int fx = fin[2 * i], fy = fin[2 * i + 1];
            s->cur_x[g] = (uint16_t)fx;
            s->cur_y[g] = (uint16_t)fy;
            const int on_goal = fx == s->goal_x[g] && fy == s->goal_y[g];
            s->rewards[g] = on_goal ? 1.0f : 0.0f; /* :188 */
            s->goal_changed[g] = 0;                 /* :192 */
            const int cell = fx * H + fy;
            ocp[cell >> 5] |= 1u << (cell & 31); /* :202-210 */
            if (s->outcomes) s->outcomes[g] = cat[i];
        }
        if (costtracer) {
            s->step_counts[e] += 1;
            continue;
        }
        if (by_candidates) {
            assign_candidate_goals(s, e, fin);
            s->step_counts[e] += 1;
        } else if (by_draws) {
            assign_random_goals(s, e, fin);
        }
        if (standard) {
            int all = 1;
            for (int i = 0; i < A; ++i) {
                const size_t g = (size_t)e * A + i;
                if (fin[2 * i] == s->goal_x[g] && fin[2 * i + 1] == s->goal_y[g]) s->arrived[g] = 1;
                if (!s->arrived[g]) all = 0;
            }
            /* :228-244 */
            const int next = s->step_counts[e] + 1;
            s->step_counts[e] = next;
            if (all) {
                s->terminated[e] = 1;
                s->truncated[e] = 0;
            } else if (next >= s->max_episode_steps) {
                s->truncated[e] = 1;
            }
        }
        for (int i = 0; i < A; ++i) {
            const size_t g = (size_t)e * A + i;
            const int action = (standard && was_arrived[i]) ? 0 : s->actions[g]; /* :257-259 */
            write_state_row(s->state_packed + g * 8, e, i, fin[2 * i], fin[2 * i + 1], s->goal_x[g],
                            s->goal_y[g], action, standard ? 0 : s->goal_changed[g]);
        }
    }
    free(was_arrived);
    free(cat);
    free(cur);
}

/* load_state: grid_world_simulator.cpp:573-589 (host part) and
 * load_state_kernel 128_agents_map_step.cu:379-416.  Validation lives in the
 * Python layer. */
void jlo_load_state(const jl_sim_t* s, const int16_t* positions, const int16_t* goals,
                    const uint8_t* arrived, const int32_t* step_counts) {
    const int E = s->n_envs, A = s->n_agents, W = s->map_w, H = s->map_h;
    const int words = W * H / 32;
    for (int e = 0; e < E; ++e) {
        int all = 1;
        for (int i = 0; i < A; ++i) {
            s->arrived[(size_t)e * A + i] = arrived[(size_t)e * A + i];
            if (!arrived[(size_t)e * A + i]) all = 0;
        }
        s->step_counts[e] = step_counts[e];
        s->terminated[e] = (uint8_t)all;
        s->truncated[e] = (uint8_t)(!all && step_counts[e] >= s->max_episode_steps);
        uint32_t* ocp = s->grid_ocp + (size_t)e * words;
        memset(ocp, 0, sizeof(uint32_t) * (size_t)words);
        for (int i = 0; i < A; ++i) {
            const size_t g = (size_t)e * A + i;
            const uint16_t x = (uint16_t)positions[2 * g], y = (uint16_t)positions[2 * g + 1];
            const uint16_t gx = (uint16_t)goals[2 * g], gy = (uint16_t)goals[2 * g + 1];
            s->cur_x[g] = x;
            s->cur_y[g] = y;
            s->goal_x[g] = gx;
            s->goal_y[g] = gy;
            s->goal_changed[g] = 1;
            s->rewards[g] = 0.0f;
            s->actions[g] = 0;
            write_state_row(s->state_packed + g * 8, e, i, x, y, gx, gy, 0, 1);
            const int cell = x * H + y;
            ocp[cell >> 5] |= 1u << (cell & 31);
        }
    }
}

/* ------------------------------------------------------------------ */
/* BFS fields                                                           */
/* ------------------------------------------------------------------ */

/* Exact uint16 distance to the goal over free 4-neighbour cells;
 * 0xFFFF unreachable.  A goal outside the map or on an obstacle gives an
 * all-0xFFFF field and returns 1 (diagnostics[3]).  Follows
 * mapf_gpt_cost_to_go_kernel, mapf_gpt_cuda.cu:181-325, and the CPU form
 * _bfs_cost_to_go, expert/mapf_gpt_schema.py:172-193.  Distances are
 * canonical (independent of queue order), so a FIFO gives the same field as
 * the level-synchronous GPU frontier.  *overflow receives the number of
 * nodes the reference's 4096-entry frontier would drop (sum over levels of
 * max(0, level_size - 4096)). */
int jlo_bfs_u16(const uint32_t* env_bits, int W, int H, int gx, int gy, uint16_t* out,
                int* overflow) {
    const int cells = W * H;
    for (int c = 0; c < cells; ++c) out[c] = JLO_UNREACHABLE;
    if (overflow) *overflow = 0;
    if (gx < 0 || gx >= W || gy < 0 || gy >= H) return 1;
    if (bit_at(env_bits, gx * H + gy)) return 1;
    int* queue = (int*)malloc(sizeof(int) * (size_t)cells);
    int head = 0, tail = 0;
    queue[tail++] = gx * H + gy;
    out[gx * H + gy] = 0;
    int level_end = tail, level_count = 0;
    while (head < tail) {
        const int c = queue[head++];
        const int x = c / H, y = c % H;
        const int d = out[c];
        static const int DX[4] = {-1, 1, 0, 0};
        static const int DY[4] = {0, 0, -1, 1};
        for (int k = 0; k < 4; ++k) {
            const int nx = x + DX[k], ny = y + DY[k];
            if (nx < 0 || nx >= W || ny < 0 || ny >= H) continue;
            const int n = nx * H + ny;
            if (bit_at(env_bits, n) || out[n] != JLO_UNREACHABLE) continue;
            out[n] = (uint16_t)(d + 1);
            queue[tail++] = n;
            ++level_count;
        }
        if (head == level_end) {
            if (overflow && level_count > JLO_MAX_FRONTIER) *overflow += level_count - JLO_MAX_FRONTIER;
            level_end = tail;
            level_count = 0;
        }
    }
    free(queue);
    return 0;
}

/* uint8 energy field, generate_energy_map_kernel energy_map.cu:80-253:
 * BFS from the target (no obstacle test on the target itself) over free
 * cells, stopped after distance 254; energy = 255 - d for visited cells,
 * 0 otherwise. */
void jlo_energy_u8(const uint32_t* env_bits, int W, int H, int gx, int gy, uint8_t* out) {
    const int cells = W * H;
    uint8_t* dist = (uint8_t*)malloc((size_t)cells);
    for (int c = 0; c < cells; ++c) dist[c] = 255;
    int* queue = (int*)malloc(sizeof(int) * (size_t)cells);
    int head = 0, tail = 0;
    queue[tail++] = gx * H + gy;
    dist[gx * H + gy] = 0;
    while (head < tail) {
        const int c = queue[head++];
        const int d = dist[c];
        if (d >= 254) continue; /* loop guard current_dist < 254, :174 */
        const int x = c / H, y = c % H;
        static const int DX[4] = {0, 0, -1, 1};
        static const int DY[4] = {-1, 1, 0, 0};
        for (int k = 0; k < 4; ++k) {
            const int nx = x + DX[k], ny = y + DY[k];
            if (nx < 0 || nx >= W || ny < 0 || ny >= H) continue;
            const int n = nx * H + ny;
            if (bit_at(env_bits, n) || dist[n] != 255) continue;
            dist[n] = (uint8_t)(d + 1);
            queue[tail++] = n;
        }
    }
    for (int c = 0; c < cells; ++c) out[c] = dist[c] == 255 ? 0 : (uint8_t)(255 - dist[c]);
    free(queue);
    free(dist);
}

/* Energy fields for a batch of state rows (launch_energy_map_kernel,
 * energy_map.cu:255-272).  Rows with env/agent out of range or a target off
 * the map are skipped (the reference indexes out of bounds there). */
void jlo_energy_maps(const uint32_t* grid_bits, uint8_t* energy, const uint16_t* states,
                     int length, int E, int A, int W, int H, int incremental_only) {
    const int words = W * H / 32;
    for (int b = 0; b < length; ++b) {
        const uint16_t* r = states + (size_t)b * 8;
        if (incremental_only && r[7] == 0) continue;
        if (r[0] >= E || r[1] >= A || r[4] >= W || r[5] >= H) continue;
        const size_t g = (size_t)r[0] * A + r[1];
        jlo_energy_u8(grid_bits + (size_t)r[0] * words, W, H, r[4], r[5],
                      energy + g * (size_t)W * H);
    }
}

/* ------------------------------------------------------------------ */
/* MAPF-GPT builder                                                     */
/* ------------------------------------------------------------------ */

static inline int coord_token(int v) { /* mapf_gpt_cuda.cu:40-44 */
    if (v < -JLO_COST_LIMIT) v = -JLO_COST_LIMIT;
    if (v > JLO_COST_LIMIT) v = JLO_COST_LIMIT;
    return v + JLO_COST_LIMIT;
}

static inline int cost_token(uint16_t v, uint16_t center) { /* :47-61 */
    if (v == JLO_UNREACHABLE) return JLO_TOK_UNREACHABLE;
    const int d = (int)v - (int)center;
    if (d > JLO_COST_LIMIT) return JLO_TOK_POS_CLIP;
    if (d < -JLO_COST_LIMIT) return JLO_TOK_NEG_CLIP;
    return d + JLO_COST_LIMIT;
}

/* mapf_gpt_unpack_kernel, mapf_gpt_cuda.cu:75-118.  A row whose env/agent
 * columns disagree with its position leaves every output of that agent
 * untouched and counts in diagnostics[1]. */
void jlo_mapfgpt_unpack_rows(const jl_mapfgpt_t* b, const int16_t* raw_rows) {
    const int N = b->n_envs * b->n_agents;
    for (int i = 0; i < N; ++i) {
        const uint16_t* row = (const uint16_t*)raw_rows + (size_t)i * 13;
        if (row[0] >= b->n_envs || row[1] >= b->n_agents || i != row[0] * b->n_agents + row[1]) {
            b->diagnostics[1] += 1;
            continue;
        }
        uint16_t* gc = b->goal_cache + (size_t)i * 2;
        const int changed = gc[0] != row[4] || gc[1] != row[5];
        const int reset = (row[7] != 0 || changed) ? 1 : 0;
        gc[0] = row[4];
        gc[1] = row[5];
        write_state_row(b->state_packed + (size_t)i * 8, row[0], row[1], row[2], row[3], row[4],
                        row[5], row[6], reset);
        for (int k = 0; k < 5; ++k) b->histories[(size_t)i * 5 + k] = row[8 + k];
        b->labels[i] = (int64_t)row[6];
    }
}

/* mapf_gpt_state_unpack_kernel, mapf_gpt_cuda.cu:121-152. */
void jlo_mapfgpt_unpack_state(const jl_mapfgpt_t* b, const int16_t* cx, const int16_t* cy,
                              const int16_t* gx, const int16_t* gy) {
    const int N = b->n_envs * b->n_agents;
    for (int i = 0; i < N; ++i) {
        const int env = i / b->n_agents, agent = i % b->n_agents;
        uint16_t* gc = b->goal_cache + (size_t)i * 2;
        const uint16_t tx = (uint16_t)gx[i], ty = (uint16_t)gy[i];
        const int changed = gc[0] != tx || gc[1] != ty;
        gc[0] = tx;
        gc[1] = ty;
        write_state_row(b->state_packed + (size_t)i * 8, env, agent, (uint16_t)cx[i],
                        (uint16_t)cy[i], tx, ty, 0, changed);
        b->labels[i] = 0;
    }
}

/* Refresh the field of every agent whose state row has reset_flag set
 * (mapf_gpt_cost_to_go_kernel, :181-325, launched over all agents). */
void jlo_mapfgpt_bfs(const jl_mapfgpt_t* b) {
    const int N = b->n_envs * b->n_agents;
    const int W = b->map_w, H = b->map_h, words = W * H / 32;
    for (int i = 0; i < N; ++i) {
        const uint16_t* st = b->state_packed + (size_t)i * 8;
        if (st[7] == 0) continue;
        if (st[0] >= b->n_envs) { /* a row this builder never wrote: no field to refresh */
            b->diagnostics[1] += 1;
            continue;
        }
        int overflow = 0;
        const int bad = jlo_bfs_u16(b->grid_bits + (size_t)st[0] * words, W, H, st[4], st[5],
                                    b->cost_to_go + (size_t)i * W * H, &overflow);
        if (bad) b->diagnostics[3] += 1;
        b->diagnostics[0] += overflow;
    }
}

/* agent_at_cell scatter (:328-347; the first agent in index order keeps a
 * shared cell) followed by mapf_gpt_materialize_tokens_kernel (:350-497).
 * agent_at_cell is the caller's [E, W, H] int32 buffer. */
void jlo_mapfgpt_tokens(const jl_mapfgpt_t* b) {
    const int E = b->n_envs, A = b->n_agents, W = b->map_w, H = b->map_h;
    const int N = E * A;
    const size_t cells = (size_t)W * H;
    for (size_t c = 0; c < (size_t)E * cells; ++c) b->agent_at_cell[c] = -1;
    for (int i = 0; i < N; ++i) {
        const uint16_t* st = b->state_packed + (size_t)i * 8;
        if (st[0] >= E) continue; /* no env to scatter into (rows written by this builder never have one) */
        if (st[2] >= W || st[3] >= H) {
            b->diagnostics[3] += 1;
            continue;
        }
        int32_t* cell = b->agent_at_cell + (size_t)st[0] * cells + (size_t)st[2] * H + st[3];
        if (*cell != -1) {
            b->diagnostics[2] += 1;
        } else {
            *cell = st[1];
        }
    }
    for (int ego_i = 0; ego_i < N; ++ego_i) {
        int32_t* out = b->tokens + (size_t)ego_i * JLO_CONTEXT;
        for (int t = 0; t < JLO_CONTEXT; ++t) out[t] = JLO_TOK_PAD;
        const uint16_t* ego = b->state_packed + (size_t)ego_i * 8;
        b->active_mask[ego_i] = (uint8_t)(ego[2] != ego[4] || ego[3] != ego[5]);
        if (ego[2] >= W || ego[3] >= H || ego[0] >= E) continue;
        const uint16_t* cost = b->cost_to_go + (size_t)ego_i * cells;
        const uint16_t center = cost[ego[2] * H + ego[3]];
        for (int t = 0; t < JLO_COST_TOKENS; ++t) {
            const int x = ego[2] + t / JLO_DIAM - JLO_RADIUS;
            const int y = ego[3] + t % JLO_DIAM - JLO_RADIUS;
            uint16_t v = JLO_UNREACHABLE;
            if (x >= 0 && x < W && y >= 0 && y < H) v = cost[x * H + y];
            out[t] = cost_token(v, center);
        }
        /* top-13 visible agents by (Manhattan distance, id), ego included */
        int sel_id[JLO_VISIBLE], sel_d[JLO_VISIBLE], nsel = 0;
        const int32_t* env_agents = b->agent_at_cell + (size_t)ego[0] * cells;
        for (int dx = -JLO_RADIUS; dx <= JLO_RADIUS; ++dx) {
            for (int dy = -JLO_RADIUS; dy <= JLO_RADIUS; ++dy) {
                const int x = ego[2] + dx, y = ego[3] + dy;
                if (x < 0 || x >= W || y < 0 || y >= H) continue;
                const int id = env_agents[x * H + y];
                if (id < 0) continue;
                const int d = abs(dx) + abs(dy);
                int pos = nsel;
                if (nsel == JLO_VISIBLE) {
                    const int ld = sel_d[JLO_VISIBLE - 1], li = sel_id[JLO_VISIBLE - 1];
                    if (!(d < ld || (d == ld && id < li))) continue;
                    pos = JLO_VISIBLE - 1;
                } else {
                    ++nsel;
                }
                while (pos > 0 && (d < sel_d[pos - 1] || (d == sel_d[pos - 1] && id < sel_id[pos - 1]))) {
                    sel_d[pos] = sel_d[pos - 1];
                    sel_id[pos] = sel_id[pos - 1];
                    --pos;
                }
                sel_d[pos] = d;
                sel_id[pos] = id;
            }
        }
        for (int s = 0; s < nsel; ++s) {
            const size_t j = (size_t)ego[0] * A + sel_id[s];
            const uint16_t* o = b->state_packed + j * 8;
            int32_t* rec = out + JLO_COST_TOKENS + s * JLO_AGENT_TOKENS;
            rec[0] = coord_token((int)o[2] - ego[2]);
            rec[1] = coord_token((int)o[3] - ego[3]);
            rec[2] = coord_token((int)o[4] - ego[2]);
            rec[3] = coord_token((int)o[5] - ego[3]);
            for (int k = 0; k < 5; ++k) {
                const int a = b->histories[j * 5 + k];
                rec[4 + k] = a == 5 ? JLO_TOK_EMPTY_ACTION : JLO_TOK_WAIT + a;
            }
            const uint16_t* oc = b->cost_to_go + j * cells;
            const uint16_t c0 = oc[o[2] * H + o[3]];
            static const int MX[4] = {-1, 1, 0, 0};
            static const int MY[4] = {0, 0, -1, 1};
            int mask = 0;
            for (int dir = 0; dir < 4; ++dir) {
                const int x = o[2] + MX[dir], y = o[3] + MY[dir];
                uint16_t nb = JLO_UNREACHABLE;
                if (x >= 0 && x < W && y >= 0 && y < H) nb = oc[x * H + y];
                if (nb != JLO_UNREACHABLE && c0 > nb) mask |= 1 << (3 - dir);
            }
            rec[9] = JLO_TOK_GREEDY + mask;
        }
    }
}

/* build_tokens (mapf_gpt_builder.cpp:89-114): zero diagnostics, unpack,
 * refresh fields, scatter + tokens. */
void jlo_mapfgpt_build_rows(const jl_mapfgpt_t* b, const int16_t* raw_rows) {
    memset(b->diagnostics, 0, 4 * sizeof(int32_t));
    jlo_mapfgpt_unpack_rows(b, raw_rows);
    jlo_mapfgpt_bfs(b);
    jlo_mapfgpt_tokens(b);
}

/* build_tokens_from_state (mapf_gpt_builder.cpp:140-167). */
void jlo_mapfgpt_build_state(const jl_mapfgpt_t* b, const int16_t* cx, const int16_t* cy,
                             const int16_t* gx, const int16_t* gy) {
    memset(b->diagnostics, 0, 4 * sizeof(int32_t));
    jlo_mapfgpt_unpack_state(b, cx, cy, gx, gy);
    jlo_mapfgpt_bfs(b);
    jlo_mapfgpt_tokens(b);
}

/* mapf_gpt_append_actions_kernel, mapf_gpt_cuda.cu:155-178. */
void jlo_mapfgpt_append(const jl_mapfgpt_t* b, const uint8_t* actions) {
    const int N = b->n_envs * b->n_agents;
    for (int i = 0; i < N; ++i) {
        uint16_t a = b->active_mask[i] ? actions[i] : 0;
        if (a >= 5) {
            b->diagnostics[1] += 1;
            a = 0;
        }
        uint16_t* h = b->histories + (size_t)i * 5;
        for (int k = 0; k < 4; ++k) h[k] = h[k + 1];
        h[4] = a;
    }
}

/* ------------------------------------------------------------------ */
/* MAGAT builder                                                        */
/* ------------------------------------------------------------------ */

/* refresh_occ_bitmap_from_packed_states_kernel, stateless_step.cu:140-173:
 * block j covers rows [j*A, (j+1)*A); the env of its first row is cleared
 * and the cells of rows with a valid env id are set.  A position off the map
 * sets no bit (the reference's word index would fall outside the env's
 * bitmap, :168-170; the device kernel skips it the same way). */
void jlo_magat_occupancy(const jl_magat_t* m) {
    const int E = m->n_envs, A = m->n_agents, W = m->map_w, H = m->map_h;
    const int words = W * H / 32;
    for (int j = 0; j < E; ++j) {
        const uint16_t env = m->states[(size_t)j * A * 8];
        if (env >= E) continue;
        uint32_t* occ = m->grid_ocp + (size_t)env * words;
        memset(occ, 0, sizeof(uint32_t) * (size_t)words);
        for (int i = 0; i < A; ++i) {
            const uint16_t* r = m->states + ((size_t)j * A + i) * 8;
            if (r[0] >= E) continue;
            if (r[2] >= W || r[3] >= H) continue;  /* uint16: negative positions are large */
            const int cell = r[2] * H + r[3];
            occ[cell >> 5] |= 1u << (cell & 31);
        }
    }
}

/* Exact round-half-even of num/den (den > 0), stateless_step.cu:120-138. */
static int round_ratio_half_even(long long num, int den) {
    const int neg = num < 0;
    unsigned long long mag = neg ? (unsigned long long)(-num) : (unsigned long long)num;
    unsigned long long q = mag / (unsigned long long)den, r = mag % (unsigned long long)den;
    if (2 * r > (unsigned long long)den || (2 * r == (unsigned long long)den && (q & 1ull))) ++q;
    return neg ? -(int)q : (int)q;
}

static inline float clampf(float v, float lo, float hi) { return v < lo ? lo : (v > hi ? hi : v); }

/* Node features, materialize_pyg_nodes_and_count_edges_local_gather_kernel
 * stateless_step.cu:368-525.  Channel order {obstacle, agents, goal, ctg}
 * over a 13x13 patch whose 11x11 window sits at offset (1,1).  The goal
 * branch tests |dy| >= |dx| where the reference compares atan2f against
 * pi/4 (:489-505); for integer offsets the two agree, and on the diagonal
 * both branches give the same corner.  ctg is (E_c - E_cell) / 10 in IEEE
 * float32, clamped to [-1, 1]. */
void jlo_magat_nodes(const jl_magat_t* m) {
    const int E = m->n_envs, A = m->n_agents, W = m->map_w, H = m->map_h;
    const int words = W * H / 32;
    const size_t cells = (size_t)W * H;
    for (int e = 0; e < E; ++e) {
        const uint16_t* rows = m->states + (size_t)e * A * 8;
        const uint32_t* st = m->grid_bits + (size_t)e * words;
        const uint32_t* oc = m->grid_ocp + (size_t)e * words;
        for (int a = 0; a < A; ++a) {
            const uint16_t* r = rows + (size_t)a * 8;
            if (r[0] >= E) continue;
            const size_t g = (size_t)e * A + a;
            float* x = m->pyg_x + g * 4 * JLO_PYG_AREA;
            for (int k = 0; k < 4 * JLO_PYG_AREA; ++k) x[k] = 0.0f;
            const int cx = (int16_t)r[2], cy = (int16_t)r[3];
            const int gx = (int16_t)r[4], gy = (int16_t)r[5];
            const uint8_t* en = m->energy + g * cells;
            float center = 0.0f;
            if (cx >= 0 && cx < W && cy >= 0 && cy < H) center = (float)en[cx * H + cy];
            for (int dx = -JLO_RADIUS; dx <= JLO_RADIUS; ++dx) {
                const int tx = cx + dx;
                for (int lc = 0; lc < JLO_DIAM; ++lc) {
                    const int ty = cy - JLO_RADIUS + lc;
                    const int li = (dx + JLO_RADIUS + 1) * JLO_PYG_DIAM + lc + 1;
                    float obs = 0.0f, occ = 0.0f, ctg = 0.0f;
                    if (tx < -1 || tx > W || ty < -1 || ty > H) {
                        ctg = 1.0f;
                    } else if (tx == -1 || tx == W || ty == -1 || ty == H) {
                        obs = 1.0f;
                        ctg = 1.0f;
                    } else {
                        const int cell = tx * H + ty;
                        const int wall = bit_at(st, cell);
                        if (wall) {
                            obs = 1.0f;
                            ctg = 1.0f;
                        } else {
                            if (bit_at(oc, cell)) occ = 1.0f;
                            ctg = clampf((center - (float)en[cell]) / 10.0f, -1.0f, 1.0f);
                        }
                    }
                    x[li] = obs;
                    x[JLO_PYG_AREA + li] = occ;
                    x[3 * JLO_PYG_AREA + li] = ctg;
                }
            }
            const int rx = gx - cx, ry = gy - cy;
            if (abs(rx) <= JLO_RADIUS && abs(ry) <= JLO_RADIUS) {
                x[2 * JLO_PYG_AREA + (rx + 6) * JLO_PYG_DIAM + (ry + 6)] = 1.0f;
            } else {
                int fx, fy;
                if (abs(ry) >= abs(rx)) {
                    fy = 6 * ((ry > 0) - (ry < 0) + 1);
                    fx = 6 + round_ratio_half_even(6LL * rx, abs(ry));
                } else {
                    fx = 6 * ((rx > 0) - (rx < 0) + 1);
                    fy = 6 + round_ratio_half_even(6LL * ry, abs(rx));
                }
                fx = fx < 0 ? 0 : (fx > 12 ? 12 : fx);
                fy = fy < 0 ? 0 : (fy > 12 ? 12 : fy);
                x[2 * JLO_PYG_AREA + fx * JLO_PYG_DIAM + fy] = 1.0f;
            }
            int count = 0;
            for (int o = 0; o < A; ++o) {
                if (o == a) continue;
                const int dx = cx - (int16_t)rows[(size_t)o * 8 + 2];
                const int dy = cy - (int16_t)rows[(size_t)o * 8 + 3];
                if (jlo_dist2(dx, dy) <= JLO_COMM_RADIUS_SQ) ++count;
            }
            m->pyg_pos[g * 2] = (float)cx;
            m->pyg_pos[g * 2 + 1] = (float)cy;
            m->edge_counts[g] = count;
        }
    }
}

/* Exclusive scan (grid_world_cuda.cu:17-110) and COO edge writer
 * (generate_pyg_edges_kernel, stateless_step.cu:854-901): per source in
 * node order, destinations in id order within the env, attr (dx, dy,
 * |dx|+|dy|) with d = source - destination, positions read from pyg_pos. */
void jlo_magat_edges(const jl_magat_t* m) {
    const int E = m->n_envs, A = m->n_agents;
    const int N = E * A;
    int64_t acc = 0;
    for (int i = 0; i < N; ++i) {
        m->edge_prefix[i] = acc;
        acc += m->edge_counts[i];
    }
    m->edge_prefix[N] = acc;
    m->num_edges[0] = acc;
    const int64_t cap = m->edge_capacity;
    for (int e = 0; e < E; ++e) {
        for (int a = 0; a < A; ++a) {
            const int node = e * A + a;
            const int cx = (int16_t)m->pyg_pos[(size_t)node * 2];
            const int cy = (int16_t)m->pyg_pos[(size_t)node * 2 + 1];
            int64_t out = m->edge_prefix[node];
            for (int o = 0; o < A; ++o) {
                if (o == a) continue;
                const int ox = (int16_t)m->pyg_pos[((size_t)e * A + o) * 2];
                const int oy = (int16_t)m->pyg_pos[((size_t)e * A + o) * 2 + 1];
                const int dx = cx - ox, dy = cy - oy;
                if (jlo_dist2(dx, dy) > JLO_COMM_RADIUS_SQ) continue;
                m->edge_index[out] = node;
                m->edge_index[cap + out] = (int64_t)e * A + o;
                m->edge_attr[out * 3] = (float)dx;
                m->edge_attr[out * 3 + 1] = (float)dy;
                m->edge_attr[out * 3 + 2] = (float)(abs(dx) + abs(dy));
                ++out;
            }
        }
    }
}
