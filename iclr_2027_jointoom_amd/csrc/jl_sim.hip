// jl_sim.hip - batched MAPF grid simulator for gfx950.
//
// step: one workgroup per env.  The reference resolves conflicts with an
// O(A^2) pair scan per Jacobi round and three barriers per round
// (128_agents_map_step.cu:91-169).  Here every cell an agent can occupy or
// enter this step (its current cell and its proposal) gets one slot in LDS
// tables, so a round is O(1) per agent: the only agents that can reject mover
// i are the current occupant of i's destination and the smallest id
// proposing it (the event-indexed form of transition_adapters.py:392-449).
// Maps of up to 4096 cells index the tables by cell; larger ones insert the
// cells into an open-addressing hash (at most 2A keys, independent of the map
// size).  The smallest proposer per cell and round is found with one LDS
// atomicMax of (round << 16 | ~id), so no table reset is needed between
// rounds: two barriers per round.  Rejections are never undone and the round
// structure is the reference's, so positions are identical.
#include <vector>

#include "jl_common.h"

namespace jl {
namespace {

constexpr int kStepThreads = 1024;  // workgroup size cap of a step
constexpr uint32_t kEmpty = 0xFFFFFFFFu;

__device__ __forceinline__ uint32_t hslot(uint32_t cell, uint32_t mask) {
    return (cell * 2654435761u >> 7) & mask;
}

__device__ __forceinline__ uint32_t hinsert(uint32_t* keys, uint32_t mask, uint32_t cell) {
    uint32_t h = hslot(cell, mask);
    while (true) {
        const uint32_t old = atomicCAS(&keys[h], kEmpty, cell);
        if (old == kEmpty || old == cell) return h;
        h = (h + 1) & mask;
    }
}

struct StepLayout {
    int slots;
    size_t keys_off, owner_off, tag_off, ocp_off, bits_off, cur_off, prop_off, goal_off, sc_off,
        sp_off, flag_off, mv_off, cat_off, any_off, life_off, total;
};

// Step modes (JL_TASK_*) as a template argument.
constexpr int kModeLifelong = JL_TASK_LIFELONG;
constexpr int kModeStandard = JL_TASK_STANDARD_MAPF;
constexpr int kModeCost = JL_TASK_COSTTRACER;

// Words of the lifelong candidate pass: reached list, start index, cursor,
// two prefetched candidates per reached agent, the reached count and one
// count per 64-agent chunk.
__host__ __device__ inline int life_words(int A) { return 5 * A + 1 + (A + 63) / 64; }

__host__ __device__ inline size_t a16(size_t v) { return (v + 15) & ~(size_t)15; }

// Maps of at most kDenseStepCells cells index the owner and round-tag tables
// by cell directly; larger maps go through the LDS hash.
constexpr int kDenseStepCells = 4096;

__host__ __device__ inline bool step_dense(int W, int H) { return W * H <= kDenseStepCells; }

// Dynamic LDS budget of a step workgroup: the CU's LDS less 1 KB for the
// kernel's own (256 bytes: the workgroup reduction of __syncthreads_and),
// which jl_step checks at launch.
constexpr size_t kStepLdsBytes = 159 * 1024;

// The tables of one step workgroup with s hash slots (maps of more than
// kDenseStepCells cells).
__host__ __device__ inline StepLayout step_layout_slots(int A, int W, int H, bool life, int s) {
    StepLayout L;
    const bool dense = step_dense(W, H);
    L.slots = dense ? W * H : s;
    size_t o = 0;
    L.keys_off = o;
    o = a16(o + (dense ? 0 : (size_t)s * 4));
    L.owner_off = o;
    o = a16(o + (size_t)L.slots * 4);
    L.tag_off = o;
    o = a16(o + (size_t)L.slots * 4);
    L.ocp_off = o;
    o = a16(o + (size_t)W * H / 8);
    L.bits_off = o;  // + one spare 16-byte word (the load pass's sink)
    o = a16(o + (size_t)W * H / 8 + 16);
    L.cur_off = o;  // cur, goal and flag have a spare entry [A]
    o = a16(o + (size_t)(A + 1) * 4);
    L.prop_off = o;
    o = a16(o + (size_t)A * 4);
    L.goal_off = o;
    o = a16(o + (size_t)(A + 1) * 4);
    L.sc_off = o;
    o = a16(o + (size_t)A * 2);
    L.sp_off = o;
    o = a16(o + (size_t)A * 2);
    L.flag_off = o;
    o = a16(o + (size_t)(A + 1) * 2);
    L.mv_off = o;
    o = a16(o + (size_t)A * 2);
    L.cat_off = o;
    o = a16(o + (size_t)A);
    L.any_off = o;
    o = a16(o + 3 * 4);
    L.life_off = o;
    o = a16(o + (life ? (size_t)life_words(A) * 4 : 0));
    L.total = o;
    return L;
}

// Hash slots: the smallest power of two of at least 4A (a load factor of at
// most 1/2 for the at most 2A distinct cells of a step), or, where those
// tables would not fit in LDS, the smallest one above 2A (a probe still
// always finds a free slot); 2,048 agents per env fit the first way on a
// 256 x 256 map in the standard mode, about 2,280 the second.
__host__ __device__ inline StepLayout step_layout(int A, int W, int H, bool life) {
    int s = 64;
    while (s < 4 * A) s <<= 1;
    StepLayout L = step_layout_slots(A, W, H, life, s);
    if (!step_dense(W, H) && L.total > kStepLdsBytes) {
        s = 64;
        while (s <= 2 * A) s <<= 1;
        L = step_layout_slots(A, W, H, life, s);
    }
    return L;
}

// Workgroup size of a step: whole wavefronts covering the agents, at most
// kStepThreads.
inline int step_threads(int A) {
    return A >= kStepThreads ? kStepThreads : (A + kWave - 1) / kWave * kWave;
}

__device__ __forceinline__ void store_row(uint16_t* dst, uint32_t env, uint32_t agent,
                                          uint32_t pos, uint32_t gx, uint32_t gy,
                                          uint32_t action, uint32_t reset) {
    uint4 v;
    v.x = (env & 0xFFFFu) | (agent << 16);
    v.y = pos;
    v.z = (gx & 0xFFFFu) | (gy << 16);
    v.w = (action & 0xFFFFu) | (reset << 16);
    *reinterpret_cast<uint4*>(dst) = v;
}

__device__ __forceinline__ uint64_t rng_next(uint64_t* state) {
    // xorshift64* (Vigna 2016)
    uint64_t x = *state;
    x ^= x >> 12;
    x ^= x << 25;
    x ^= x >> 27;
    *state = x;
    return x * 0x2545F4914F6CDD1Dull;
}

// s_flag: the action as given (low byte) and the arrival latch.
constexpr uint16_t kFlagArrived = 0x100;
// Agents (and bitmap words) a thread holds in registers: 1 up to
// kStepThreads agents (one thread per agent), else 4; agents past
// 4 * kStepThreads go through LDS.
inline int step_per(int A) { return A <= kStepThreads ? 1 : 4; }

// Everything the step reads from HBM is requested at its start (the env's
// obstacle bitmap and each agent's position, goal, action and arrival latch
// into LDS, the done flags and the step count into registers), so a step
// costs one memory round trip and the Jacobi rounds run in LDS.
template <int H, int kMode, bool kDense, int kStepPer>
__global__ __launch_bounds__(kStepThreads) void step_kernel(jl_sim_t s) {
    constexpr bool kStandard = kMode == kModeStandard;
    extern __shared__ __align__(16) uint8_t smem[];
    const int env = blockIdx.x;
    const int A = s.n_agents, W = s.map_w;
    const int tid = threadIdx.x, nt = blockDim.x;
    const size_t base = (size_t)env * A;
    const StepLayout L = step_layout(A, W, H, kMode == kModeLifelong);
    uint32_t* keys = reinterpret_cast<uint32_t*>(smem + L.keys_off);
    uint32_t* owner = reinterpret_cast<uint32_t*>(smem + L.owner_off);
    uint32_t* tag = reinterpret_cast<uint32_t*>(smem + L.tag_off);
    uint32_t* ocp = reinterpret_cast<uint32_t*>(smem + L.ocp_off);
    uint32_t* s_bits = reinterpret_cast<uint32_t*>(smem + L.bits_off);
    uint32_t* s_cur = reinterpret_cast<uint32_t*>(smem + L.cur_off);
    uint32_t* s_prop = reinterpret_cast<uint32_t*>(smem + L.prop_off);
    uint32_t* s_goal = reinterpret_cast<uint32_t*>(smem + L.goal_off);
    uint16_t* s_sc = reinterpret_cast<uint16_t*>(smem + L.sc_off);
    uint16_t* s_sp = reinterpret_cast<uint16_t*>(smem + L.sp_off);
    uint16_t* s_flag = reinterpret_cast<uint16_t*>(smem + L.flag_off);
    uint8_t* s_mv = smem + L.mv_off;  // [2][A] moving flags, ping-pong by round
    uint8_t* s_cat = smem + L.cat_off;
    uint32_t* s_any = reinterpret_cast<uint32_t*>(smem + L.any_off);  // [3] rotating round flags
    const uint32_t mask = (uint32_t)L.slots - 1;
    const int words = W * H / 32;
    // every env's bitmap starts 16-byte aligned when its word count is a multiple of 4
    const bool vec_words = (words & 3) == 0;

    // First pass: every load is issued (at clamped indices, without a
    // branch) before the first LDS store, so they share one round trip.
    const uint8_t term = kStandard ? s.terminated[env] : 0;
    const uint8_t trunc = kStandard ? s.truncated[env] : 0;
    const int steps = s.step_counts[env];
    const bool by_candidates = kMode == kModeLifelong && s.goal_candidates != nullptr;
    const int cand_count = by_candidates ? min(s.candidate_counts[env], s.candidate_stride) : 0;
    const uint4* bits4 = reinterpret_cast<const uint4*>(s.grid_bits + (size_t)env * words);
    const int nvec = vec_words ? words / 4 : 0;
    // the bitmap words as four scalar arrays: an array of uint4 was left in
    // scratch memory (not promoted to registers) when kStepPer > 1
    uint32_t rbx[kStepPer], rby[kStepPer], rbz[kStepPer], rbw[kStepPer];
    uint32_t rc[kStepPer], rg[kStepPer], rf[kStepPer];
#pragma unroll
    for (int j = 0; j < kStepPer; ++j) {
        const int k = tid + j * nt;
        const uint4 v = bits4[k < nvec ? k : 0];
        rbx[j] = v.x;
        rby[j] = v.y;
        rbz[j] = v.z;
        rbw[j] = v.w;
    }
#pragma unroll
    for (int j = 0; j < kStepPer; ++j) {
        const int a = tid + j * nt;
        const size_t g = base + (a < A ? a : A - 1);
        rc[j] = (uint32_t)s.cur_x[g] | ((uint32_t)s.cur_y[g] << 16);
        rg[j] = (uint32_t)s.goal_x[g] | ((uint32_t)s.goal_y[g] << 16);
        const bool arrived = kStandard && s.arrived[g] != 0;
        rf[j] = (uint32_t)s.actions[g] | (arrived ? kFlagArrived : 0u);
    }
    // out-of-range items land in the spare slot past each array: no branch
    // for the compiler to sink the loads into
#pragma unroll
    for (int j = 0; j < kStepPer; ++j) {
        const int k = tid + j * nt;
        reinterpret_cast<uint4*>(s_bits)[k < nvec ? k : nvec] = make_uint4(rbx[j], rby[j], rbz[j], rbw[j]);
    }
#pragma unroll
    for (int j = 0; j < kStepPer; ++j) {
        const int a = tid + j * nt;
        const int d = a < A ? a : A;
        s_cur[d] = rc[j];
        s_goal[d] = rg[j];
        s_flag[d] = (uint16_t)rf[j];
    }
    // the rest: larger maps and agent counts, and bitmaps not 16-byte aligned
    if (vec_words) {
        for (int k = tid + kStepPer * nt; k < nvec; k += nt)
            reinterpret_cast<uint4*>(s_bits)[k] = bits4[k];
    } else {
        const uint32_t* src = s.grid_bits + (size_t)env * words;
        for (int k = tid; k < words; k += nt) s_bits[k] = src[k];
    }
    for (int a = tid + kStepPer * nt; a < A; a += nt) {
        const size_t g = base + a;
        s_cur[a] = (uint32_t)s.cur_x[g] | ((uint32_t)s.cur_y[g] << 16);
        s_goal[a] = (uint32_t)s.goal_x[g] | ((uint32_t)s.goal_y[g] << 16);
        const bool arrived = kStandard && s.arrived[g] != 0;
        s_flag[a] = (uint16_t)(s.actions[g] | (arrived ? kFlagArrived : 0));
    }
    const bool done = (term | trunc) != 0;

    // Tables.  Dense: only the entries of cells the agents stand on or may
    // enter are read, so each agent clears those (its cell and, when in the
    // map, its tentative destination) instead of the whole map.
    auto target_of = [&](uint32_t cur, uint32_t f, int& tx, int& ty) __attribute__((always_inline)) {
        int act = (int)(f & 0xFFu);
        if (act > 4) act = 0;
        tx = (int)(cur & 0xFFFFu) + (act == 1 ? -1 : (act == 2 ? 1 : 0));
        ty = (int)(cur >> 16) + (act == 3 ? -1 : (act == 4 ? 1 : 0));
    };
    if (kDense) {
        for (int a = tid; a < A; a += nt) {
            const uint32_t cur = s_cur[a];
            int tx, ty;
            target_of(cur, s_flag[a], tx, ty);
            const uint32_t cc = (cur & 0xFFFFu) * H + (cur >> 16);
            owner[cc] = 0;
            tag[cc] = 0;
            if (tx >= 0 && tx < W && ty >= 0 && ty < H) {
                owner[tx * H + ty] = 0;
                tag[tx * H + ty] = 0;
            }
        }
    } else {
        for (int k = tid; k < L.slots; k += nt) {
            keys[k] = kEmpty;
            owner[k] = 0;
            tag[k] = 0;
        }
    }
    for (int k = tid; k < words; k += nt) ocp[k] = 0;
    if (tid < 3) s_any[tid] = 0;
    __syncthreads();
    if (done) {
        // done envs do not advance (128_agents_map_step.cu:31-34)
        if (s.outcomes)
            for (int a = tid; a < A; a += nt) s.outcomes[base + a] = 0;
        return;
    }

    // Proposals (:54-82): arrived agents stay; walls and the map edge stay.
    // Agents a = tid + j * nt, j < kStepPer, keep their own state in
    // registers for the rounds; the moving flags and slots other agents read
    // are also in LDS.
    uint32_t r_sc[kStepPer], r_sp[kStepPer], r_cat[kStepPer];
    bool r_mv[kStepPer];
    auto propose = [&](int a, uint32_t& sc_out, uint32_t& sp_out, bool& mv_out,
                       uint32_t& cat_out) __attribute__((always_inline)) {
        const uint32_t cur = s_cur[a];
        const uint32_t f = s_flag[a];
        int tx, ty;
        target_of(cur, f, tx, ty);
        const bool was_arrived = (f & kFlagArrived) != 0;
        bool move = !was_arrived && (tx != (int)(cur & 0xFFFFu) || ty != (int)(cur >> 16));
        uint32_t cat = 0;
        if (move) {
            const bool wall = tx < 0 || tx >= W || ty < 0 || ty >= H || bit_at(s_bits, tx * H + ty);
            if (wall) {
                move = false;
                cat = JL_OUTCOME_WALL;
            }
        }
        s_prop[a] = move ? ((uint32_t)tx | ((uint32_t)ty << 16)) : cur;
        s_mv[a] = move ? 1 : 0;
        // slot of a cell: the cell itself, or its hash entry
        const uint32_t ccell = (cur & 0xFFFFu) * H + (cur >> 16), tcell = (uint32_t)(tx * H + ty);
        const uint32_t sc = kDense ? ccell : hinsert(keys, mask, ccell);
        // a cell shared by several agents keeps the highest id as occupant,
        // as the CPU restatement's dict does (transition_adapters.py:389-392)
        atomicMax(&owner[sc], (uint32_t)a + 1);
        const uint32_t sp = move ? (kDense ? tcell : hinsert(keys, mask, tcell)) : sc;
        s_sc[a] = (uint16_t)sc;
        s_sp[a] = (uint16_t)sp;
        sc_out = sc;
        sp_out = sp;
        mv_out = move;
        cat_out = cat;
    };
#pragma unroll
    for (int j = 0; j < kStepPer; ++j) {
        const int a = tid + j * nt;
        r_mv[j] = false;
        r_sc[j] = r_sp[j] = r_cat[j] = 0;
        if (a < A) propose(a, r_sc[j], r_sp[j], r_mv[j], r_cat[j]);
    }
    for (int a = tid + kStepPer * nt; a < A; a += nt) {
        uint32_t sc, sp, cat;
        bool mv;
        propose(a, sc, sp, mv, cat);
        s_cat[a] = (uint8_t)cat;
    }
    __syncthreads();

    // Jacobi rounds (:91-169).  Mover a is rejected by the occupant o of its
    // destination d (swap if o moves into a's cell; vertex if o stays and
    // a > o, else chain) or by the smallest id proposing d this round
    // (vertex if smaller than a); the earlier of the two in id order gives
    // the category.
    auto decide = [&](int a, bool mv_a, uint32_t sc_a, uint32_t sp_a,
                      const uint8_t* mv) __attribute__((always_inline)) -> uint32_t {
        const uint32_t own = owner[sp_a], tg = tag[sp_a];
        const int o = (int)own - 1;
        const int oc = o >= 0 ? o : 0;
        const bool mv_o = mv[oc] != 0;
        const uint32_t sp_o = s_sp[oc];
        const int mid = (int)(0xFFFFu - (tg & 0xFFFFu));
        int cat_o = 0;
        if (o >= 0) cat_o = mv_o ? (sp_o == sc_a ? JL_OUTCOME_SWAP : 0)
                                 : (a > o ? JL_OUTCOME_VERTEX : JL_OUTCOME_CHAIN);
        const int cat_m = (mid < a && mid != o) ? JL_OUTCOME_VERTEX : 0;
        const int c = (cat_o && cat_m) ? (o < mid ? cat_o : cat_m) : (cat_o ? cat_o : cat_m);
        return mv_a ? (uint32_t)c : 0u;
    };
    int cur = 0;
    for (int iter = 0; iter < A; ++iter) {
        const uint8_t* mv = s_mv + cur * A;
        uint8_t* mv_next = s_mv + (cur ^ 1) * A;
        const uint32_t stamp = (uint32_t)(iter + 1) << 16;
        // the flag of the next round: its previous readers have all passed
        // the first barrier of the round before this one
        if (tid == 0) s_any[(iter + 1) % 3] = 0;
#pragma unroll
        for (int j = 0; j < kStepPer; ++j) {
            const int a = tid + j * nt;
            if (a < A) atomicMax(&tag[r_mv[j] ? r_sp[j] : r_sc[j]], stamp | (0xFFFFu - (uint32_t)a));
        }
        for (int a = tid + kStepPer * nt; a < A; a += nt) {
            const uint32_t slot = mv[a] ? s_sp[a] : s_sc[a];
            atomicMax(&tag[slot], stamp | (0xFFFFu - (uint32_t)a));
        }
        __syncthreads();
        bool rejected = false;
#pragma unroll
        for (int j = 0; j < kStepPer; ++j) {
            const int a = tid + j * nt;
            if (a < A) {
                const uint32_t c = decide(a, r_mv[j], r_sc[j], r_sp[j], mv);
                if (c) {
                    r_mv[j] = false;
                    r_cat[j] = r_cat[j] ? r_cat[j] : c;
                    rejected = true;
                }
                mv_next[a] = r_mv[j] ? 1 : 0;
            }
        }
        for (int a = tid + kStepPer * nt; a < A; a += nt) {
            const bool m = mv[a] != 0;
            const uint32_t c = decide(a, m, s_sc[a], s_sp[a], mv);
            if (c) {
                if (s_cat[a] == 0) s_cat[a] = (uint8_t)c;
                rejected = true;
            }
            mv_next[a] = (m && !c) ? 1 : 0;
        }
        if (rejected) s_any[iter % 3] = 1;
        __syncthreads();
        const bool any = s_any[iter % 3] != 0;
        cur ^= 1;
        if (!any) break;
    }
    const uint8_t* mv = s_mv + cur * A;
#pragma unroll
    for (int j = 0; j < kStepPer; ++j) {
        const int a = tid + j * nt;
        if (a < A) s_cat[a] = (uint8_t)r_cat[j];
    }

    // Outputs (:171-217): positions, rewards, occupancy, arrival latch.
    int all_arrived = 1;
    for (int a = tid; a < A; a += nt) {
        const size_t g = base + a;
        const uint32_t fin = mv[a] ? s_prop[a] : s_cur[a];
        const uint32_t fx = fin & 0xFFFFu, fy = fin >> 16;
        s.cur_x[g] = (uint16_t)fx;
        s.cur_y[g] = (uint16_t)fy;
        const uint32_t goal = s_goal[a];
        const bool on_goal = fin == goal;
        s.rewards[g] = on_goal ? 1.0f : 0.0f;
        s.goal_changed[g] = 0;
        const uint32_t cell = fx * H + fy;
        atomicOr(&ocp[cell >> 5], 1u << (cell & 31));
        if (s.outcomes) s.outcomes[g] = s_cat[a];
        if (kStandard) {
            const uint32_t f = s_flag[a];
            const bool was = (f & kFlagArrived) != 0;
            const bool now = was || on_goal;
            if (now != was) s.arrived[g] = 1;
            if (!now) all_arrived = 0;
            // packed state: arrived agents report the stay action (:257-259)
            store_row(s.state_packed + g * 8, env, a, fin, goal & 0xFFFFu, goal >> 16,
                      was ? 0u : (f & 0xFFu), 0);
        }
        s_cur[a] = fin;  // keep the final cell for the lifelong pass
    }
    all_arrived = __syncthreads_and(all_arrived);
    if (vec_words) {
        uint4* gocp = reinterpret_cast<uint4*>(s.grid_ocp + (size_t)env * words);
        const uint4* src = reinterpret_cast<const uint4*>(ocp);
        for (int k = tid; k < words / 4; k += nt) gocp[k] = src[k];
    } else {
        uint32_t* gocp = s.grid_ocp + (size_t)env * words;
        for (int k = tid; k < words; k += nt) gocp[k] = ocp[k];
    }

    if (kMode == kModeCost) {
        // CostTracer steps move agents and count steps only (the goal stream
        // is advanced by the reward pass), 128_agents_map_step.cu:219-222 of
        // rebuttal/online-rl/native/src/cuda_backend
        if (tid == 0) s.step_counts[env] = steps + 1;
        return;
    }
    if (kStandard) {
        if (tid == 0) {
            const int next = steps + 1;
            s.step_counts[env] = next;
            if (all_arrived) {
                s.terminated[env] = 1;
                s.truncated[env] = 0;
            } else if (next >= s.max_episode_steps) {
                s.truncated[env] = 1;
            }
        }
        return;
    }

    // Lifelong (:265-361): agents standing on their goal draw a new goal
    // among the env's free cells not used as a goal by an agent off its goal.
    // Draws are made in agent order by one thread, so the result depends only
    // on the generator state.
    uint32_t* goal_bits = ocp;  // reuse: goals of agents not on their goal
    __syncthreads();
    for (int k = tid; k < words; k += nt) goal_bits[k] = 0;
    __syncthreads();
    for (int a = tid; a < A; a += nt) {
        const uint32_t goal = s_goal[a];
        const uint32_t gx = goal & 0xFFFFu, gy = goal >> 16;
        if (s_cur[a] != goal && gx < (uint32_t)W && gy < (uint32_t)H) {  // goals off the map reserve nothing
            const uint32_t cell = gx * H + gy;
            atomicOr(&goal_bits[cell >> 5], 1u << (cell & 31));
        }
    }
    __syncthreads();
    // The agents on their goal, listed in id order (ballots per chunk of 64
    // agents and the chunks' counts); both rules settle them in that order.
    uint32_t* life = reinterpret_cast<uint32_t*>(smem + L.life_off);
    uint32_t* r_list = life;
    int32_t* r_start = reinterpret_cast<int32_t*>(life + A);
    int32_t* r_cursor = reinterpret_cast<int32_t*>(life + 2 * A);
    uint32_t* r_pref = life + 3 * A;  // [2A]: first two cells, then the chosen cell
    uint32_t* r_meta = life + 5 * A;  // [0] reached count, [1 + c] count of chunk c
    {
        const int lane = tid & (kWave - 1);
        const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
        const int nwaves = nt / kWave;
        const int nchunks = (A + kWave - 1) / kWave;
        for (int c = wave; c < nchunks; c += nwaves) {
            const int a = c * kWave + lane;
            const uint64_t m = __ballot(a < A && s_cur[a] == s_goal[a]);
            if (lane == 0) r_meta[1 + c] = (uint32_t)__popcll(m);
        }
        __syncthreads();
        for (int c = wave; c < nchunks; c += nwaves) {
            uint32_t before = 0;
            for (int k = 0; k < c; ++k) before += r_meta[1 + k];
            const int a = c * kWave + lane;
            const bool hit = a < A && s_cur[a] == s_goal[a];
            const uint64_t m = __ballot(hit);
            if (hit) r_list[before + __popcll(m & ((1ull << lane) - 1ull))] = (uint32_t)a;
            if (c == nchunks - 1 && lane == 0) r_meta[0] = before + (uint32_t)__popcll(m);
        }
        __syncthreads();
    }
    const int nr = (int)r_meta[0];
    if (by_candidates) {
        // Canonical agent order over per-agent candidate lists
        // (128_agents_map_step.cu:303-330 of rebuttal/online-rl/native/src/
        // cuda_backend; its CPU twin assign_goals, rebuttal/online-il/
        // tasks.py:51-65): agent i on its goal takes the first cell of its
        // env's list, from candidates[i][cursor % length] on, that is neither
        // its own cell nor the goal of an agent off its goal or of an agent
        // before it.  The reached agents' first two candidates are fetched in
        // parallel, and one thread settles them in order against the goal
        // bitmap.
        const int count = cand_count;
        const int clen = s.candidate_length;
        const uint16_t* cells = s.candidate_cells + (size_t)env * s.candidate_stride * 2;
        auto cand = [&](int64_t k) -> uint32_t {
            const int64_t i = k % count;
            return (uint32_t)cells[2 * i] | ((uint32_t)cells[2 * i + 1] << 16);
        };
        if (count > 0) {
            for (int j = tid; j < nr; j += nt) {
                const size_t g = base + r_list[j];
                const int cursor = s.goal_cursors[g];
                int ci = cursor % clen;
                ci += ci < 0 ? clen : 0;
                int start = s.goal_candidates[g * clen + ci] % count;
                start += start < 0 ? count : 0;
                r_cursor[j] = cursor;
                r_start[j] = start;
                r_pref[2 * j] = cand(start);
                r_pref[2 * j + 1] = cand((int64_t)start + 1);
            }
        }
        __syncthreads();
        if (tid == 0) {
            for (int j = 0; j < nr && count > 0; ++j) {
                const int a = (int)r_list[j];
                const uint32_t cur = s_cur[a];
                uint32_t chosen = kEmpty;
                for (int attempt = 0; attempt < count; ++attempt) {
                    const uint32_t c = attempt < 2 ? r_pref[2 * j + attempt]
                                                   : cand((int64_t)r_start[j] + attempt);
                    const uint32_t x = c & 0xFFFFu, y = c >> 16;
                    if (c == cur || x >= (uint32_t)W || y >= (uint32_t)H) continue;
                    const uint32_t cell = x * H + y;
                    if ((goal_bits[cell >> 5] >> (cell & 31)) & 1u) continue;
                    goal_bits[cell >> 5] |= 1u << (cell & 31);
                    chosen = c;
                    break;
                }
                r_pref[2 * j] = chosen;
                if (chosen != kEmpty) {
                    s_goal[a] = chosen;
                    s_flag[a] |= 0x8000;  // goal changed this step
                }
            }
            s.step_counts[env] = steps + 1;
        }
        __syncthreads();
        for (int j = tid; j < nr && count > 0; j += nt) {
            const uint32_t c = r_pref[2 * j];
            if (c == kEmpty) continue;
            const size_t g = base + r_list[j];
            s.goal_x[g] = (uint16_t)(c & 0xFFFFu);
            s.goal_y[g] = (uint16_t)(c >> 16);
            s.goal_changed[g] = 1;
            s.goal_cursors[g] = r_cursor[j] + 1;
        }
    } else {
        // Generator draws (128_agents_map_step.cu:265-343): agent i on its
        // goal draws a start index into the env's free-cell list from its own
        // generator (one draw per reached agent) and takes the first cell from
        // there on, wrapping, that is not the goal of an agent off its goal or
        // of an agent before it.  Each reached agent draws and fetches its
        // first two cells in parallel; one thread settles them in id order
        // against the goal bitmap, reading further cells of the list only when
        // both are taken.
        const int count = s.env_counts[env];
        const int offset = s.env_offsets[env];
        if (count > 0) {
            for (int j = tid; j < nr; j += nt) {
                const size_t g = base + r_list[j];
                uint64_t st = s.rng_state[g];
                const int k = (int)((rng_next(&st) >> 32) % (uint64_t)count);
                s.rng_state[g] = st;
                r_start[j] = k;
                r_pref[2 * j] = s.free_cells[offset + k];
                r_pref[2 * j + 1] = s.free_cells[offset + (k + 1 < count ? k + 1 : 0)];
            }
        }
        __syncthreads();
        if (tid == 0 && count > 0) {
            for (int j = 0; j < nr; ++j) {
                int k = r_start[j];
                uint32_t chosen = kEmpty;
                for (int attempt = 0; attempt < count; ++attempt) {
                    // free-cell list entries are x << 16 | y
                    const uint32_t packed = attempt < 2 ? r_pref[2 * j + attempt] : s.free_cells[offset + k];
                    const uint32_t x = packed >> 16, y = packed & 0xFFFFu;
                    const uint32_t cell = x * H + y;
                    if (!((goal_bits[cell >> 5] >> (cell & 31)) & 1u)) {
                        goal_bits[cell >> 5] |= 1u << (cell & 31);
                        chosen = x | (y << 16);
                        break;
                    }
                    if (++k >= count) k = 0;
                }
                r_pref[2 * j] = chosen;
            }
        }
        __syncthreads();
        for (int j = tid; j < nr && count > 0; j += nt) {
            const uint32_t c = r_pref[2 * j];
            if (c == kEmpty) continue;
            const int a = (int)r_list[j];
            const size_t g = base + a;
            s_goal[a] = c;
            s_flag[a] |= 0x8000;  // goal changed this step
            s.goal_x[g] = (uint16_t)(c & 0xFFFFu);
            s.goal_y[g] = (uint16_t)(c >> 16);
            s.goal_changed[g] = 1;
        }
    }
    __syncthreads();
    for (int a = tid; a < A; a += nt) {
        const size_t g = base + a;
        const uint32_t goal = s_goal[a];
        const uint32_t f = s_flag[a];
        store_row(s.state_packed + g * 8, env, a, s_cur[a], goal & 0xFFFFu, goal >> 16, f & 0xFFu,
                  (f & 0x8000) ? 1u : 0u);
    }
}

template <int H>
__global__ __launch_bounds__(256) void load_state_kernel(jl_sim_t s,
                                                         const int16_t* __restrict__ positions,
                                                         const int16_t* __restrict__ goals,
                                                         const uint8_t* __restrict__ arrived,
                                                         const int32_t* __restrict__ step_counts) {
    extern __shared__ __align__(16) uint32_t s_ocp[];
    const int env = blockIdx.x, A = s.n_agents, W = s.map_w;
    const int words = W * H / 32;
    const size_t base = (size_t)env * A;
    for (int k = threadIdx.x; k < words; k += blockDim.x) s_ocp[k] = 0;
    __syncthreads();
    int all = 1;
    for (int a = threadIdx.x; a < A; a += blockDim.x) {
        const size_t g = base + a;
        const uint32_t x = (uint16_t)positions[2 * g], y = (uint16_t)positions[2 * g + 1];
        const uint32_t gx = (uint16_t)goals[2 * g], gy = (uint16_t)goals[2 * g + 1];
        s.cur_x[g] = (uint16_t)x;
        s.cur_y[g] = (uint16_t)y;
        s.goal_x[g] = (uint16_t)gx;
        s.goal_y[g] = (uint16_t)gy;
        s.goal_changed[g] = 1;
        s.rewards[g] = 0.0f;
        s.actions[g] = 0;
        const uint8_t arr = arrived[g];
        s.arrived[g] = arr;
        if (!arr) all = 0;
        store_row(s.state_packed + g * 8, env, a, x | (y << 16), gx, gy, 0, 1);
        const uint32_t cell = x * H + y;
        atomicOr(&s_ocp[cell >> 5], 1u << (cell & 31));
    }
    all = __syncthreads_and(all);
    uint32_t* gocp = s.grid_ocp + (size_t)env * words;
    for (int k = threadIdx.x; k < words; k += blockDim.x) gocp[k] = s_ocp[k];
    if (threadIdx.x == 0) {
        const int steps = step_counts[env];
        s.step_counts[env] = steps;
        s.terminated[env] = (uint8_t)all;
        s.truncated[env] = (uint8_t)(!all && steps >= s.max_episode_steps);
    }
}

// Wavefront ballot packs 64 consecutive cells into two words: coalesced reads.
__global__ void encode_map_kernel(const int32_t* __restrict__ grids, uint32_t* __restrict__ bits,
                                  size_t cells) {
    const size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
    const int v = i < cells ? grids[i] : 0;
    const uint64_t m = __ballot(v != 0);
    const int lane = threadIdx.x & (kWave - 1);
    const size_t w0 = (i - lane) / 32;
    if (lane == 0 && i < cells) bits[w0] = (uint32_t)m;
    if (lane == 32 && i < cells) bits[w0 + 1] = (uint32_t)(m >> 32);
}

__global__ void decode_kernel(const uint16_t* __restrict__ obs, uint8_t* __restrict__ out,
                              size_t total, int diam) {
    const size_t t = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
    if (t >= total) return;
    const size_t col = t % diam;
    size_t rest = t / diam;
    const size_t row = rest % diam;
    rest /= diam;
    const size_t ch = rest % 2;
    const size_t agent = rest / 2;
    out[t] = (uint8_t)((obs[agent * 2 * diam + ch * diam + row] >> col) & 1u);
}

__device__ __forceinline__ uint64_t splitmix64(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

__global__ void seed_kernel(uint64_t* state, int64_t count, uint64_t seed) {
    const int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (i >= count) return;
    uint64_t v = splitmix64(seed ^ splitmix64((uint64_t)i));
    state[i] = v ? v : 0x9E3779B97F4A7C15ull;  // xorshift state must be nonzero
}

// Free cells of each env inside its real extent, row-major, at offset e*W*H.
template <int H>
__global__ __launch_bounds__(256) void free_cells_kernel(jl_sim_t s, const int32_t* extents,
                                                         uint32_t* free_cells, int32_t* offsets,
                                                         int32_t* counts) {
    __shared__ int s_wave_sum[4];
    __shared__ int s_running;
    const int env = blockIdx.x, W = s.map_w;
    const int words = W * H / 32;
    const int rw = extents[2 * env], rh = extents[2 * env + 1];
    const uint32_t* bits = s.grid_bits + (size_t)env * words;
    uint32_t* out = free_cells + (size_t)env * W * H;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (tid == 0) s_running = 0;
    __syncthreads();
    for (int w0 = 0; w0 < words; w0 += 256) {
        const int w = w0 + tid;
        uint32_t m = 0;
        int x = 0, ybase = 0;
        if (w < words) {
            x = (w * 32) / H;
            ybase = (w * 32) % H;
            if (x < rw) {
                m = ~bits[w];
                const int rem = rh - ybase;
                m &= rem >= 32 ? 0xFFFFFFFFu : (rem <= 0 ? 0u : ((1u << rem) - 1u));
            }
        }
        const int c = __popc(m);
        int incl = c;
        for (int off = 1; off < 64; off <<= 1) {
            const int v = __shfl_up(incl, off, 64);
            if (lane >= off) incl += v;
        }
        if (lane == 63) s_wave_sum[wave] = incl;
        __syncthreads();
        int before = s_running;
        for (int k = 0; k < wave; ++k) before += s_wave_sum[k];
        int pos = before + incl - c;
        while (m) {
            const int b = __ffs(m) - 1;
            m &= m - 1;
            out[pos++] = ((uint32_t)x << 16) | (uint32_t)(ybase + b);
        }
        __syncthreads();
        if (tid == 0) s_running += s_wave_sum[0] + s_wave_sum[1] + s_wave_sum[2] + s_wave_sum[3];
        __syncthreads();
    }
    if (tid == 0) {
        counts[env] = s_running;
        offsets[env] = s_running > 0 ? env * W * H : -1;
    }
}

// Distinct random start and goal cells for every agent of an env
// (init_agents_kernel, grid_world_cuda.cu:405-450): draws in agent order,
// start then goal, linear probing over the env's free-cell list.
__global__ void init_agents_kernel(jl_sim_t s, const uint32_t* free_cells, const int32_t* offsets,
                                   const int32_t* counts) {
    extern __shared__ uint32_t s_used[];
    const int env = blockIdx.x, A = s.n_agents;
    const int count = counts[env];
    const int used_words = (s.map_w * s.map_h + 31) / 32;
    for (int k = threadIdx.x; k < used_words; k += blockDim.x) s_used[k] = 0;
    __syncthreads();
    if (threadIdx.x != 0) return;
    const int offset = offsets[env];
    for (int a = 0; a < A; ++a) {
        const size_t g = (size_t)env * A + a;
        uint64_t st = s.rng_state[g];
        uint32_t picked[2] = {0xFFFFFFFFu, 0xFFFFFFFFu};
        for (int which = 0; which < 2 && count > 0; ++which) {
            int k = (int)((rng_next(&st) >> 32) % (uint64_t)count);
            for (int attempt = 0; attempt < count; ++attempt) {
                if (!((s_used[k >> 5] >> (k & 31)) & 1u)) {
                    s_used[k >> 5] |= 1u << (k & 31);
                    picked[which] = free_cells[offset + k];
                    break;
                }
                if (++k >= count) k = 0;
            }
        }
        s.rng_state[g] = st;
        s.cur_x[g] = (uint16_t)(picked[0] >> 16);
        s.cur_y[g] = (uint16_t)(picked[0] & 0xFFFFu);
        s.goal_x[g] = (uint16_t)(picked[1] >> 16);
        s.goal_y[g] = (uint16_t)(picked[1] & 0xFFFFu);
    }
}

// Copy of the caller's actions into the simulator's buffer, one thread per
// 16 bytes: a 16-byte word when both ends are 16-byte aligned, else the same
// 16 bytes one by one (decided on the device from the pointers, so a copy
// captured into a graph stays right when its source is pointed at a buffer
// of another alignment); the last n % 16 bytes go to the first threads (a
// grid has at least 256).
__global__ __launch_bounds__(256) void copy_actions_kernel(uint8_t* __restrict__ dst,
                                                           const uint8_t* __restrict__ src, size_t n) {
    const size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
    const size_t words = n / 16;
    if (i < words) {
        if (((reinterpret_cast<uintptr_t>(dst) | reinterpret_cast<uintptr_t>(src)) & 15u) == 0) {
            reinterpret_cast<uint4*>(dst)[i] = reinterpret_cast<const uint4*>(src)[i];
        } else {
#pragma unroll
            for (int k = 0; k < 16; ++k) dst[i * 16 + k] = src[i * 16 + k];
        }
    }
    if (i < n - words * 16) dst[words * 16 + i] = src[words * 16 + i];
}

// Inclusive int64 prefix sum of the goal_changed values and its last value
// (the int64 cast, cumsum and count of GridWorldSimulator::
// update_derived_state, grid_world_simulator.cpp:709-717).  Workgroup w
// scans values [w * chunk, (w + 1) * chunk), chunk = kScanThreads * PER: it
// sums every value before its range itself (16 bytes per load, from the L2),
// so workgroups never wait for each other, scans its own range (through LDS
// when a thread holds more than one value) and writes the prefixes with
// consecutive lanes on consecutive values.  PER grows with N only past 128
// workgroups of one value per thread, so that small batches spread over as
// many CUs as the chunks allow.
constexpr int kScanThreads = 1024;
constexpr int kScanWorkgroups = 128;  // PER = 1 up to this many workgroups, then 2, then 4

template <int PER>
__global__ __launch_bounds__(kScanThreads) void goal_changed_scan_kernel(jl_sim_t s, int64_t* prefix,
                                                                         int64_t* count,
                                                                         uint16_t* changed) {
    constexpr int kChunk = kScanThreads * PER;
    __shared__ int64_t s_wave[kScanThreads / kWave];
    __shared__ int64_t s_out[PER > 1 ? kChunk : 1];
    const int tid = threadIdx.x, lane = tid & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);  // uniform per wavefront
    const int64_t N = (int64_t)s.n_envs * s.n_agents;
    const int64_t c0 = (int64_t)blockIdx.x * kChunk;
    const uint8_t* f = s.goal_changed;
    // this thread's PER consecutive values, loaded first so that they travel
    // with the loads of the values before the chunk
    const int64_t e0 = c0 + (int64_t)tid * PER;
    uint32_t v[PER];
#pragma unroll
    for (int j = 0; j < PER; ++j) v[j] = e0 + j < N ? f[e0 + j] : 0u;
    // the changed-row buffer is cleared before the energy pass packs into it
    // (the reference zero-fills it, grid_world_simulator.cpp:724-733)
    if (changed) {
        const uint4 zero = make_uint4(0, 0, 0, 0);
#pragma unroll
        for (int j = 0; j < PER; ++j) {
            const int64_t e = c0 + tid + j * kScanThreads;
            if (e < N) reinterpret_cast<uint4*>(changed)[e] = zero;
        }
    }
    // values before this chunk: 16-byte words up to c0, bytes for the rest
    const bool vec = (reinterpret_cast<uintptr_t>(f) & 15u) == 0;
    const int64_t words = vec ? c0 / 16 : 0;
    uint64_t before = 0;
#pragma unroll 8
    for (int64_t k = tid; k < words; k += kScanThreads) {
        const uint4 w = reinterpret_cast<const uint4*>(f)[k];
        before += byte_sum(w.x) + byte_sum(w.y) + byte_sum(w.z) + byte_sum(w.w);
    }
    for (int64_t k = words * 16 + tid; k < c0; k += kScanThreads) before += f[k];
    for (int off = kWave / 2; off > 0; off >>= 1) before += __shfl_xor(before, off, kWave);
    if (lane == 0) s_wave[wave] = (int64_t)before;
    __syncthreads();
    int64_t base = 0;
    for (int k = 0; k < kScanThreads / kWave; ++k) base += s_wave[k];
    __syncthreads();
    // this thread's values, scanned across the workgroup: a wavefront's sum
    // is at most 64 * PER * 255, so 32 bits hold it
    uint32_t local = 0;
#pragma unroll
    for (int j = 0; j < PER; ++j) local += v[j];
    uint32_t incl = local;
    for (int off = 1; off < kWave; off <<= 1) {
        const uint32_t t = __shfl_up(incl, off, kWave);
        if (lane >= off) incl += t;
    }
    if (lane == kWave - 1) s_wave[wave] = incl;
    __syncthreads();
    int64_t run = base + (int64_t)(incl - local);
    for (int k = 0; k < wave; ++k) run += s_wave[k];
    if constexpr (PER == 1) {
        run += v[0];
        if (e0 < N) prefix[e0] = run;
        if (e0 == N - 1) count[0] = run;
    } else {
#pragma unroll
        for (int j = 0; j < PER; ++j) {
            run += v[j];
            s_out[tid * PER + j] = run;
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < PER; ++j) {
            const int64_t e = c0 + tid + j * kScanThreads;
            if (e < N) prefix[e] = s_out[tid + j * kScanThreads];
            if (e == N - 1) count[0] = s_out[tid + j * kScanThreads];
        }
    }
}

int check_sim(const jl_sim_t* s) {
    if (!s || s->n_envs <= 0 || s->n_agents <= 0) return JL_ERR_ARG;
    if (!profile_ok(s->map_w, s->map_h)) return JL_ERR_PROFILE;
    if (s->n_agents > 16384 || s->n_envs > 65535) return JL_ERR_ARG;
    if (!s->grid_bits || !s->grid_ocp || !s->cur_x || !s->cur_y || !s->goal_x || !s->goal_y ||
        !s->actions || !s->arrived || !s->goal_changed || !s->rewards || !s->terminated ||
        !s->truncated || !s->step_counts || !s->state_packed)
        return JL_ERR_ARG;
    if (s->task_mode != JL_TASK_LIFELONG && s->task_mode != JL_TASK_STANDARD_MAPF &&
        s->task_mode != JL_TASK_COSTTRACER)
        return JL_ERR_ARG;
    if (s->task_mode == JL_TASK_LIFELONG) {
        if (s->goal_candidates) {
            if (!s->candidate_cells || !s->candidate_counts || !s->goal_cursors ||
                s->candidate_length <= 0 || s->candidate_stride <= 0)
                return JL_ERR_ARG;
        } else if (!s->free_cells || !s->env_offsets || !s->env_counts || !s->rng_state) {
            return JL_ERR_ARG;
        }
    }
    return JL_OK;
}

}  // namespace
}  // namespace jl

using namespace jl;

extern "C" int jl_encode_map(const int32_t* grids, uint32_t* grid_bits, int32_t n_envs,
                             int32_t map_w, int32_t map_h, jl_stream_t stream) {
    if (!grids || !grid_bits || n_envs <= 0) return JL_ERR_ARG;
    if (!profile_ok(map_w, map_h)) return JL_ERR_PROFILE;
    const size_t cells = (size_t)n_envs * map_w * map_h;
    hipLaunchKernelGGL(encode_map_kernel, dim3((unsigned)((cells + 255) / 256)), dim3(256), 0,
                       (hipStream_t)stream, grids, grid_bits, cells);
    return launch_status();
}

extern "C" int jl_step(const jl_sim_t* s, jl_stream_t stream) {
    int rc = check_sim(s);
    if (rc) return rc;
    const StepLayout L =
        step_layout(s->n_agents, s->map_w, s->map_h, s->task_mode == JL_TASK_LIFELONG);
    if (L.total > kStepLdsBytes) return JL_ERR_AGENTS;
    const int nt = step_threads(s->n_agents);
    const bool dense = step_dense(s->map_w, s->map_h);
    const bool one = step_per(s->n_agents) == 1;
#define JL_STEP_LAUNCH(MODE, DENSE, PER)                                                           \
    do {                                                                                           \
        if (!lds_fits<&step_kernel<H, MODE, DENSE, PER>>(L.total)) return JL_ERR_AGENTS;          \
        hipLaunchKernelGGL((step_kernel<H, MODE, DENSE, PER>), dim3(s->n_envs), dim3(nt), L.total, \
                           (hipStream_t)stream, *s);                                              \
    } while (0)
#define JL_STEP_SHAPES(MODE)                                                            \
    if (dense) {                                                                        \
        if (one) JL_STEP_LAUNCH(MODE, true, 1); else JL_STEP_LAUNCH(MODE, true, 4);     \
    } else {                                                                            \
        if (one) JL_STEP_LAUNCH(MODE, false, 1); else JL_STEP_LAUNCH(MODE, false, 4);   \
    }
    JL_DISPATCH_H(s->map_h, {
        if (s->task_mode == JL_TASK_STANDARD_MAPF) {
            JL_STEP_SHAPES(kModeStandard)
        } else if (s->task_mode == JL_TASK_COSTTRACER) {
            JL_STEP_SHAPES(kModeCost)
        } else {
            JL_STEP_SHAPES(kModeLifelong)
        }
    });
#undef JL_STEP_SHAPES
#undef JL_STEP_LAUNCH
    return launch_status();
}

extern "C" int jl_update_actions(const jl_sim_t* s, const uint8_t* actions, jl_stream_t stream) {
    int rc = check_sim(s);
    if (rc) return rc;
    if (!actions) return JL_ERR_ARG;
    const size_t n = (size_t)s->n_envs * s->n_agents;
    const dim3 grid((unsigned)(((n + 15) / 16 + 255) / 256));
    hipLaunchKernelGGL(copy_actions_kernel, grid, dim3(256), 0, (hipStream_t)stream, s->actions, actions, n);
    return launch_status();
}

// The action-reading nodes of a captured graph: the history append (the
// builder, actions at argument 1 of 2) and the action copy (update_actions,
// source at argument 1 of 3).  Every node is checked before any is changed.
extern "C" int jl_graph_retarget_actions(void* graph, void* graph_exec, const void* captured,
                                         const void* actions, int32_t* n_nodes) {
    if (!graph || !graph_exec || !captured || !actions) return JL_ERR_ARG;
    size_t count = 0;
    int rc = status(hipGraphGetNodes(static_cast<hipGraph_t>(graph), nullptr, &count));
    if (rc) return rc;
    std::vector<hipGraphNode_t> nodes(count);
    if (count) {
        rc = status(hipGraphGetNodes(static_cast<hipGraph_t>(graph), nodes.data(), &count));
        if (rc) return rc;
    }
    const void* append = append_actions_kernel_address();
    const void* copy = reinterpret_cast<const void*>(&copy_actions_kernel);
    struct Hit {
        hipGraphNode_t node;
        hipKernelNodeParams params;
        int nargs;
    };
    std::vector<Hit> hits;
    for (hipGraphNode_t node : nodes) {
        hipGraphNodeType type;
        rc = status(hipGraphNodeGetType(node, &type));
        if (rc) return rc;
        if (type != hipGraphNodeTypeKernel) continue;
        hipKernelNodeParams p;
        rc = status(hipGraphKernelNodeGetParams(node, &p));
        if (rc) return rc;
        const int nargs = p.func == append ? 2 : (p.func == copy ? 3 : 0);
        if (!nargs) continue;
        if (!p.kernelParams || !p.kernelParams[1]) return JL_ERR_ARG;
        if (*static_cast<const void* const*>(p.kernelParams[1]) != captured) continue;
        hits.push_back({node, p, nargs});
    }
    for (Hit& h : hits) {
        void* args[3];
        for (int k = 0; k < h.nargs; ++k) args[k] = h.params.kernelParams[k];
        const void* moved = actions;
        args[1] = &moved;
        h.params.kernelParams = args;
        rc = status(hipGraphExecKernelNodeSetParams(static_cast<hipGraphExec_t>(graph_exec), h.node, &h.params));
        if (rc) return rc;
    }
    if (n_nodes) *n_nodes = (int32_t)hits.size();
    return JL_OK;
}

extern "C" int jl_goal_changed_scan(const jl_sim_t* s, int64_t* prefix, int64_t* count,
                                    uint16_t* changed_states, jl_stream_t stream) {
    int rc = check_sim(s);
    if (rc) return rc;
    if (!prefix || !count) return JL_ERR_ARG;
    const int64_t N = (int64_t)s->n_envs * s->n_agents;
    const int64_t one = (int64_t)kScanThreads * kScanWorkgroups;
    if (N <= one) {
        hipLaunchKernelGGL(goal_changed_scan_kernel<1>, dim3((unsigned)((N + kScanThreads - 1) / kScanThreads)),
                           dim3(kScanThreads), 0, (hipStream_t)stream, *s, prefix, count, changed_states);
    } else if (N <= 2 * one) {
        hipLaunchKernelGGL(goal_changed_scan_kernel<2>,
                           dim3((unsigned)((N + 2 * kScanThreads - 1) / (2 * kScanThreads))), dim3(kScanThreads), 0,
                           (hipStream_t)stream, *s, prefix, count, changed_states);
    } else {
        hipLaunchKernelGGL(goal_changed_scan_kernel<4>,
                           dim3((unsigned)((N + 4 * kScanThreads - 1) / (4 * kScanThreads))), dim3(kScanThreads), 0,
                           (hipStream_t)stream, *s, prefix, count, changed_states);
    }
    return launch_status();
}

extern "C" int jl_load_state(const jl_sim_t* s, const int16_t* positions, const int16_t* goals,
                             const uint8_t* arrived, const int32_t* step_counts,
                             jl_stream_t stream) {
    int rc = check_sim(s);
    if (rc) return rc;
    if (!positions || !goals || !arrived || !step_counts) return JL_ERR_ARG;
    const size_t lds = (size_t)s->map_w * s->map_h / 8;
    JL_DISPATCH_H(s->map_h, {
        hipLaunchKernelGGL((load_state_kernel<H>), dim3(s->n_envs), dim3(256), lds,
                           (hipStream_t)stream, *s, positions, goals, arrived, step_counts);
    });
    return launch_status();
}

extern "C" int jl_lifelong_init(const jl_sim_t* s, const int32_t* real_extents,
                                uint32_t* free_cells, int32_t* env_offsets, int32_t* env_counts,
                                jl_stream_t stream) {
    if (!s || !real_extents || !free_cells || !env_offsets || !env_counts || !s->rng_state)
        return JL_ERR_ARG;
    if (!profile_ok(s->map_w, s->map_h)) return JL_ERR_PROFILE;
    if (s->n_envs <= 0 || s->n_agents <= 0 || !s->grid_bits) return JL_ERR_ARG;
    JL_DISPATCH_H(s->map_h, {
        hipLaunchKernelGGL((free_cells_kernel<H>), dim3(s->n_envs), dim3(256), 0,
                           (hipStream_t)stream, *s, real_extents, free_cells, env_offsets,
                           env_counts);
    });
    const int rc = launch_status();
    if (rc) return rc;
    const size_t lds = (size_t)(s->map_w * s->map_h + 31) / 32 * 4;
    hipLaunchKernelGGL(init_agents_kernel, dim3(s->n_envs), dim3(256), lds, (hipStream_t)stream, *s,
                       free_cells, env_offsets, env_counts);
    return launch_status();
}

extern "C" int jl_seed_rng(uint64_t* rng_state, int64_t count, uint64_t seed, jl_stream_t stream) {
    if (!rng_state || count <= 0) return JL_ERR_ARG;
    hipLaunchKernelGGL(seed_kernel, dim3((unsigned)((count + 255) / 256)), dim3(256), 0,
                       (hipStream_t)stream, rng_state, count, seed);
    return launch_status();
}

extern "C" int jl_decode_to_uint8(const uint16_t* obs, uint8_t* out, int64_t n_batch,
                                  int32_t diameter, jl_stream_t stream) {
    if (!obs || !out || n_batch <= 0 || diameter <= 0 || diameter > 16) return JL_ERR_ARG;
    const size_t total = (size_t)n_batch * 2 * diameter * diameter;
    hipLaunchKernelGGL(decode_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                       (hipStream_t)stream, obs, out, total, diameter);
    return launch_status();
}

extern "C" const char* jl_error_string(int code) {
    switch (code) {
        case JL_OK: return "success";
        case JL_ERR_ARG: return "invalid argument (null pointer or size out of range)";
        case JL_ERR_PROFILE: return "unsupported map profile (map_h a multiple of 32 up to 256, 1 <= map_w <= 256)";
        case JL_ERR_CAPACITY: return "edge buffer smaller than the worst case";
        case JL_ERR_AGENTS:
            return "too many agents per env for this map: the kernel's per-env LDS tables exceed 160 KB";
        default: return code > 0 ? hipGetErrorString((hipError_t)code) : "unknown error";
    }
}

extern "C" const char* jl_version(void) { return "jointloom-gfx950 0.1.0"; }
