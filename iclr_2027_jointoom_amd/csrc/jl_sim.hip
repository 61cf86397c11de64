// jl_sim.hip - batched MAPF grid simulator for gfx950.
//
// step: one workgroup per env.  The reference resolves conflicts with an
// O(A^2) pair scan per Jacobi round and three barriers per round
// (128_agents_map_step.cu:91-169).  Here every cell an agent can occupy or
// enter this step (its current cell and its proposal) is inserted once into
// an LDS open-addressing hash, so a round is O(1) per agent: the only agents
// that can reject mover i are the current occupant of i's destination and
// the smallest id proposing it (the event-indexed form of
// transition_adapters.py:392-449).  The smallest proposer per cell and round
// is found with one LDS atomicMax of (round << 16 | ~id), so no table reset
// is needed between rounds: two barriers per round.  Rejections are never
// undone and the round structure is the reference's, so positions are
// identical.  The table holds at most 2A keys, independent of the map size.
#include "jl_common.h"

namespace jl {
namespace {

constexpr int kStepThreads = 256;
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
    size_t keys_off, owner_off, tag_off, ocp_off, cur_off, prop_off, sc_off, sp_off, mv_off, cat_off,
        total;
};

__host__ __device__ inline size_t a16(size_t v) { return (v + 15) & ~(size_t)15; }

__host__ __device__ inline StepLayout step_layout(int A, int W, int H) {
    StepLayout L;
    int s = 64;
    while (s < 4 * A) s <<= 1;  // load factor <= 1/2 for the <= 2A distinct cells
    L.slots = s;
    size_t o = 0;
    L.keys_off = o;
    o = a16(o + (size_t)s * 4);
    L.owner_off = o;
    o = a16(o + (size_t)s * 4);
    L.tag_off = o;
    o = a16(o + (size_t)s * 4);
    L.ocp_off = o;
    o = a16(o + (size_t)W * H / 8);
    L.cur_off = o;
    o = a16(o + (size_t)A * 4);
    L.prop_off = o;
    o = a16(o + (size_t)A * 4);
    L.sc_off = o;
    o = a16(o + (size_t)A * 2);
    L.sp_off = o;
    o = a16(o + (size_t)A * 2);
    L.mv_off = o;
    o = a16(o + (size_t)A * 2);
    L.cat_off = o;
    o = a16(o + (size_t)A);
    L.total = o;
    return L;
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

template <int H, bool kStandard>
__global__ __launch_bounds__(kStepThreads) void step_kernel(jl_sim_t s) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int env = blockIdx.x;
    const int A = s.n_agents, W = s.map_w;
    const int tid = threadIdx.x;
    const size_t base = (size_t)env * A;
    if (kStandard && (s.terminated[env] != 0 || s.truncated[env] != 0)) {
        // done envs do not advance (128_agents_map_step.cu:31-34)
        if (s.outcomes)
            for (int a = tid; a < A; a += kStepThreads) s.outcomes[base + a] = 0;
        return;
    }
    const StepLayout L = step_layout(A, W, H);
    uint32_t* keys = reinterpret_cast<uint32_t*>(smem + L.keys_off);
    uint32_t* owner = reinterpret_cast<uint32_t*>(smem + L.owner_off);
    uint32_t* tag = reinterpret_cast<uint32_t*>(smem + L.tag_off);
    uint32_t* ocp = reinterpret_cast<uint32_t*>(smem + L.ocp_off);
    uint32_t* s_cur = reinterpret_cast<uint32_t*>(smem + L.cur_off);
    uint32_t* s_prop = reinterpret_cast<uint32_t*>(smem + L.prop_off);
    uint16_t* s_sc = reinterpret_cast<uint16_t*>(smem + L.sc_off);
    uint16_t* s_sp = reinterpret_cast<uint16_t*>(smem + L.sp_off);
    uint8_t* s_mv = smem + L.mv_off;  // [2][A] moving flags, ping-pong by round
    uint8_t* s_cat = smem + L.cat_off;
    const uint32_t mask = (uint32_t)L.slots - 1;
    const int words = W * H / 32;
    const uint32_t* env_bits = s.grid_bits + (size_t)env * words;

    for (int k = tid; k < L.slots; k += kStepThreads) {
        keys[k] = kEmpty;
        owner[k] = 0;
        tag[k] = 0;
    }
    for (int k = tid; k < words; k += kStepThreads) ocp[k] = 0;
    __syncthreads();

    // Proposals (:54-82): arrived agents stay; walls and the map edge stay.
    for (int a = tid; a < A; a += kStepThreads) {
        const size_t g = base + a;
        const int cx = s.cur_x[g], cy = s.cur_y[g];
        int act = s.actions[g];
        if (act > 4) act = 0;
        const bool was_arrived = kStandard && s.arrived[g] != 0;
        const int dx = act == 1 ? -1 : (act == 2 ? 1 : 0);
        const int dy = act == 3 ? -1 : (act == 4 ? 1 : 0);
        const int tx = cx + dx, ty = cy + dy;
        bool move = !was_arrived && act != 0;
        uint8_t cat = 0;
        if (move) {
            const bool wall = tx < 0 || tx >= W || ty < 0 || ty >= H || bit_at(env_bits, tx * H + ty);
            if (wall) {
                move = false;
                cat = JL_OUTCOME_WALL;
            }
        }
        const uint32_t cur = (uint32_t)cx | ((uint32_t)cy << 16);
        const uint32_t prop = move ? ((uint32_t)tx | ((uint32_t)ty << 16)) : cur;
        s_cur[a] = cur;
        s_prop[a] = prop;
        s_cat[a] = cat;
        s_mv[a] = move ? 1 : 0;
        const uint32_t sc = hinsert(keys, mask, (uint32_t)(cx * H + cy));
        s_sc[a] = (uint16_t)sc;
        // a cell shared by several agents keeps the highest id as occupant,
        // as the CPU restatement's dict does (transition_adapters.py:389-392)
        atomicMax(&owner[sc], (uint32_t)a + 1);
        s_sp[a] = move ? (uint16_t)hinsert(keys, mask, (uint32_t)(tx * H + ty)) : (uint16_t)sc;
    }
    __syncthreads();

    // Jacobi rounds (:91-169).
    int cur = 0;
    for (int iter = 0; iter < A; ++iter) {
        const uint8_t* mv = s_mv + cur * A;
        uint8_t* mv_next = s_mv + (cur ^ 1) * A;
        const uint32_t stamp = (uint32_t)(iter + 1) << 16;
        for (int a = tid; a < A; a += kStepThreads) {
            const uint32_t slot = mv[a] ? s_sp[a] : s_sc[a];
            atomicMax(&tag[slot], stamp | (0xFFFFu - (uint32_t)a));
        }
        __syncthreads();
        int rejected = 0;
        for (int a = tid; a < A; a += kStepThreads) {
            uint8_t m = mv[a];
            if (m) {
                const uint32_t d = s_sp[a];
                const int o = (int)owner[d] - 1;
                const int mid = (int)(0xFFFFu - (tag[d] & 0xFFFFu));
                int cat_o = 0;
                if (o >= 0) {
                    if (mv[o]) {
                        if (s_sp[o] == s_sc[a]) cat_o = JL_OUTCOME_SWAP;
                    } else {
                        cat_o = a > o ? JL_OUTCOME_VERTEX : JL_OUTCOME_CHAIN;
                    }
                }
                const int cat_m = (mid < a && mid != o) ? JL_OUTCOME_VERTEX : 0;
                int c;
                if (cat_o && cat_m) {
                    c = o < mid ? cat_o : cat_m;
                } else {
                    c = cat_o ? cat_o : cat_m;
                }
                if (c) {
                    m = 0;
                    if (s_cat[a] == 0) s_cat[a] = (uint8_t)c;
                    rejected = 1;
                }
            }
            mv_next[a] = m;
        }
        const int any = __syncthreads_or(rejected);
        cur ^= 1;
        if (!any) break;
    }
    const uint8_t* mv = s_mv + cur * A;

    // Outputs (:171-217): positions, rewards, occupancy, arrival latch.
    int all_arrived = 1;
    for (int a = tid; a < A; a += kStepThreads) {
        const size_t g = base + a;
        const uint32_t fin = mv[a] ? s_prop[a] : s_cur[a];
        const uint32_t fx = fin & 0xFFFFu, fy = fin >> 16;
        s.cur_x[g] = (uint16_t)fx;
        s.cur_y[g] = (uint16_t)fy;
        const uint32_t gx = s.goal_x[g], gy = s.goal_y[g];
        const bool on_goal = fx == gx && fy == gy;
        s.rewards[g] = on_goal ? 1.0f : 0.0f;
        s.goal_changed[g] = 0;
        const uint32_t cell = fx * H + fy;
        atomicOr(&ocp[cell >> 5], 1u << (cell & 31));
        if (s.outcomes) s.outcomes[g] = s_cat[a];
        if (kStandard) {
            const uint8_t was = s.arrived[g];
            const uint8_t now = (was != 0 || on_goal) ? 1 : 0;
            if (now != was) s.arrived[g] = now;
            if (!now) all_arrived = 0;
            // packed state: arrived agents report the stay action (:257-259)
            const uint32_t action = was ? 0u : (uint32_t)s.actions[g];
            store_row(s.state_packed + g * 8, env, a, fin, gx, gy, action, 0);
        }
        s_cur[a] = fin;  // keep the final cell for the lifelong pass
    }
    all_arrived = __syncthreads_and(all_arrived);
    uint32_t* gocp = s.grid_ocp + (size_t)env * words;
    for (int k = tid; k < words; k += kStepThreads) gocp[k] = ocp[k];

    if (kStandard) {
        if (tid == 0) {
            const int next = s.step_counts[env] + 1;
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
    for (int k = tid; k < words; k += kStepThreads) goal_bits[k] = 0;
    __syncthreads();
    for (int a = tid; a < A; a += kStepThreads) {
        const size_t g = base + a;
        const uint32_t fin = s_cur[a];
        const uint32_t gx = s.goal_x[g], gy = s.goal_y[g];
        if (!((fin & 0xFFFFu) == gx && (fin >> 16) == gy)) {
            const uint32_t cell = gx * H + gy;
            atomicOr(&goal_bits[cell >> 5], 1u << (cell & 31));
        }
    }
    __syncthreads();
    if (tid == 0) {
        const int count = s.env_counts[env];
        const int offset = s.env_offsets[env];
        for (int a = 0; a < A; ++a) {
            const size_t g = base + a;
            const uint32_t fin = s_cur[a];
            if (!((fin & 0xFFFFu) == s.goal_x[g] && (fin >> 16) == s.goal_y[g])) continue;
            if (count <= 0) continue;
            uint64_t st = s.rng_state[g];
            int k = (int)((rng_next(&st) >> 32) % (uint64_t)count);
            for (int attempt = 0; attempt < count; ++attempt) {
                const uint32_t packed = s.free_cells[offset + k];
                const uint32_t x = packed >> 16, y = packed & 0xFFFFu;
                const uint32_t cell = x * H + y;
                if (!((goal_bits[cell >> 5] >> (cell & 31)) & 1u)) {
                    goal_bits[cell >> 5] |= 1u << (cell & 31);
                    s.goal_x[g] = (uint16_t)x;
                    s.goal_y[g] = (uint16_t)y;
                    s.goal_changed[g] = 1;
                    break;
                }
                if (++k >= count) k = 0;
            }
            s.rng_state[g] = st;
        }
    }
    __syncthreads();
    for (int a = tid; a < A; a += kStepThreads) {
        const size_t g = base + a;
        store_row(s.state_packed + g * 8, env, a, s_cur[a], s.goal_x[g], s.goal_y[g],
                  s.actions[g], s.goal_changed[g]);
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

int check_sim(const jl_sim_t* s) {
    if (!s || s->n_envs <= 0 || s->n_agents <= 0) return JL_ERR_ARG;
    if (!profile_ok(s->map_w, s->map_h)) return JL_ERR_PROFILE;
    if (s->n_agents > 16384 || s->n_envs > 65535) return JL_ERR_ARG;
    if (!s->grid_bits || !s->grid_ocp || !s->cur_x || !s->cur_y || !s->goal_x || !s->goal_y ||
        !s->actions || !s->arrived || !s->goal_changed || !s->rewards || !s->terminated ||
        !s->truncated || !s->step_counts || !s->state_packed)
        return JL_ERR_ARG;
    if (s->task_mode != JL_TASK_LIFELONG && s->task_mode != JL_TASK_STANDARD_MAPF) return JL_ERR_ARG;
    if (s->task_mode == JL_TASK_LIFELONG &&
        (!s->free_cells || !s->env_offsets || !s->env_counts || !s->rng_state))
        return JL_ERR_ARG;
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
    const StepLayout L = step_layout(s->n_agents, s->map_w, s->map_h);
    if (L.total > 160 * 1024) return JL_ERR_ARG;
    JL_DISPATCH_H(s->map_h, {
        if (s->task_mode == JL_TASK_STANDARD_MAPF) {
            hipLaunchKernelGGL((step_kernel<H, true>), dim3(s->n_envs), dim3(kStepThreads), L.total,
                               (hipStream_t)stream, *s);
        } else {
            hipLaunchKernelGGL((step_kernel<H, false>), dim3(s->n_envs), dim3(kStepThreads),
                               L.total, (hipStream_t)stream, *s);
        }
    });
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
        case JL_ERR_PROFILE: return "unsupported map profile (map_h in {32,64,128,256}, map_w <= 256)";
        case JL_ERR_CAPACITY: return "edge buffer smaller than the worst case";
        default: return code > 0 ? hipGetErrorString((hipError_t)code) : "unknown error";
    }
}

extern "C" const char* jl_version(void) { return "jointloom-gfx950 0.1.0"; }
