// jl_mapfgpt.hip - MAPF-GPT observation builder for gfx950.
//
// A build is two launches:
//   1. unpack_bfs: one wavefront per 64 agents unpacks the state (raw rows or
//      resident split arrays), refreshes the goal cache, and runs the
//      bit-parallel BFS (jl_bfs.h) for each agent whose reset flag is set,
//      staging the field in LDS and storing it with coalesced 16-byte writes.
//   2. tokens: one workgroup per env.  Agent positions, goals, histories and
//      greedy masks of the env live in LDS together with an occupancy bitmap
//      and a cell->agent hash, so the visible-agent search never touches HBM;
//      the 11x11 cost windows of a chunk of egos are gathered into LDS with
//      many independent loads in flight; each ego's 1 KB token row is then
//      written by one wavefront as 64 x 16-byte stores.
// The reference runs four kernels plus a 16 KB/env memset per build
// (mapf_gpt_builder.cpp:108-110, mapf_gpt_cuda.cu:544-610) with the
// top-13 search done serially by one lane per ego (:395-496).
#include "jl_bfs.h"
#include "jl_common.h"

namespace jl {
namespace {

constexpr int kTokThreads = 256;
constexpr uint32_t kEmptyKey = 0xFFFFFFFFu;
constexpr uint32_t kNoAgent = 0xFFFFFFFFu;

__device__ __forceinline__ uint32_t hash_cell(uint32_t cell, uint32_t mask) {
    return (cell * 2654435761u >> 7) & mask;
}

// Insert `cell` (once per distinct cell) and return its slot.
__device__ __forceinline__ uint32_t hash_insert(uint32_t* keys, uint32_t mask, uint32_t cell) {
    uint32_t h = hash_cell(cell, mask);
    while (true) {
        const uint32_t old = atomicCAS(&keys[h], kEmptyKey, cell);
        if (old == kEmptyKey || old == cell) return h;
        h = (h + 1) & mask;
    }
}

__device__ __forceinline__ uint32_t hash_find(const uint32_t* keys, uint32_t mask, uint32_t cell) {
    uint32_t h = hash_cell(cell, mask);
    while (true) {
        const uint32_t k = keys[h];
        if (k == cell) return h;
        if (k == kEmptyKey) return kEmptyKey;
        h = (h + 1) & mask;
    }
}

__device__ __forceinline__ void store_state_row(uint16_t* dst, uint32_t env, uint32_t agent,
                                                uint32_t px, uint32_t py, uint32_t gx,
                                                uint32_t gy, uint32_t action, uint32_t reset) {
    uint4 v;
    v.x = (env & 0xFFFFu) | (agent << 16);
    v.y = (px & 0xFFFFu) | (py << 16);
    v.z = (gx & 0xFFFFu) | (gy << 16);
    v.w = (action & 0xFFFFu) | (reset << 16);
    *reinterpret_cast<uint4*>(dst) = v;
}

// ---------------------------------------------------------------------------
// Launch 1: unpack + goal-cache refresh + BFS of refreshed goals.
// kRows: raw 13-column rows (mapf_gpt_unpack_kernel, mapf_gpt_cuda.cu:75-118);
// otherwise resident split arrays (mapf_gpt_state_unpack_kernel, :121-152).
// ---------------------------------------------------------------------------
template <int H, int R, bool kRows>
__global__ __launch_bounds__(kWave) void unpack_bfs_kernel(jl_mapfgpt_t b,
                                                            const int16_t* __restrict__ raw_rows,
                                                            const int16_t* __restrict__ cur_x,
                                                            const int16_t* __restrict__ cur_y,
                                                            const int16_t* __restrict__ goal_x,
                                                            const int16_t* __restrict__ goal_y) {
    extern __shared__ uint16_t s_dist[];
    const int A = b.n_agents, W = b.map_w;
    const int N = b.n_envs * A;
    const int lane = threadIdx.x;
    const int i = blockIdx.x * kWave + lane;
    int32_t* accum = b.scratch + kScratchAccum;

    bool reset = false;
    uint32_t env = 0, tx = 0, ty = 0;
    bool bad_row = false;
    if (i < N) {
        uint16_t* st = b.state_packed + (size_t)i * 8;
        if (kRows) {
            const uint16_t* row = reinterpret_cast<const uint16_t*>(raw_rows) + (size_t)i * 13;
            uint16_t c[13];
#pragma unroll
            for (int k = 0; k < 13; ++k) c[k] = row[k];
            if (c[0] >= b.n_envs || c[1] >= A || i != (int)c[0] * A + c[1]) {
                // rejected row: every output of this agent keeps its old value,
                // including the reset flag the BFS pass reads (:90-92, :186-189)
                bad_row = true;
                const uint4 old = *reinterpret_cast<const uint4*>(st);
                env = old.x & 0xFFFFu;
                tx = old.z & 0xFFFFu;
                ty = old.z >> 16;
                reset = (old.w >> 16) != 0;
            } else {
                uint16_t* gc = b.goal_cache + (size_t)i * 2;
                const uint32_t cache = *reinterpret_cast<const uint32_t*>(gc);
                const uint32_t goal = (uint32_t)c[4] | ((uint32_t)c[5] << 16);
                const bool changed = cache != goal;
                if (changed) *reinterpret_cast<uint32_t*>(gc) = goal;
                reset = c[7] != 0 || changed;
                env = c[0];
                tx = c[4];
                ty = c[5];
                store_state_row(st, c[0], c[1], c[2], c[3], c[4], c[5], c[6], reset ? 1u : 0u);
                uint16_t* h = b.histories + (size_t)i * 5;
#pragma unroll
                for (int k = 0; k < 5; ++k) h[k] = c[8 + k];
                b.labels[i] = (int64_t)c[6];
            }
        } else {
            env = (uint32_t)(i / A);
            const uint32_t agent = (uint32_t)(i - (int)env * A);
            tx = (uint16_t)goal_x[i];
            ty = (uint16_t)goal_y[i];
            uint16_t* gc = b.goal_cache + (size_t)i * 2;
            const uint32_t cache = *reinterpret_cast<const uint32_t*>(gc);
            const uint32_t goal = tx | (ty << 16);
            reset = cache != goal;
            if (reset) *reinterpret_cast<uint32_t*>(gc) = goal;
            store_state_row(st, env, agent, (uint16_t)cur_x[i], (uint16_t)cur_y[i], tx, ty, 0u,
                            reset ? 1u : 0u);
            b.labels[i] = 0;
        }
    }
    const uint64_t bad_mask = __ballot(bad_row);
    if (lane == 0 && bad_mask) atomicAdd(accum + 1, (int)__popcll(bad_mask));

    uint64_t todo = __ballot(reset);
    if (!todo) return;

    constexpr int HW = RowWords<H>::HW;
    const int cells = W * H;
    const int words = cells / 32;
    while (todo) {
        const int src = __ffsll((unsigned long long)todo) - 1;
        todo &= todo - 1;
        const uint32_t e = (uint32_t)__shfl((int)env, src, kWave);
        const int gx = __shfl((int)tx, src, kWave);
        const int gy = __shfl((int)ty, src, kWave);
        const size_t agent_index = (size_t)blockIdx.x * kWave + src;
        for (int c = lane; c < cells; c += kWave) s_dist[c] = kUnreachable;
        __syncthreads();
        bool ok = e < (uint32_t)b.n_envs && gx < W && gy < H;
        const uint32_t* env_bits = b.grid_bits + (size_t)(ok ? e : 0) * words;
        if (ok && bit_at(env_bits, gx * H + gy)) ok = false;
        if (ok) {
            uint64_t fr[R][HW];
            load_free_rows<H, R>(env_bits, W, fr);
            if (lane == 0) s_dist[gx * H + gy] = 0;
            __syncthreads();
            int overflow;
            if (W * H > kMaxFrontier + 1) {
                overflow = wave_bfs<H, R, uint16_t, true>(fr, gx, gy, 0x7FFFFFFF, s_dist);
            } else {
                overflow = wave_bfs<H, R, uint16_t, false>(fr, gx, gy, 0x7FFFFFFF, s_dist);
            }
            if (lane == 0 && overflow) atomicAdd(accum + 0, overflow);
        } else if (lane == 0) {
            atomicAdd(accum + 3, 1);  // goal off the map or on an obstacle (:224-236)
        }
        __syncthreads();
        uint4* out = reinterpret_cast<uint4*>(b.cost_to_go + agent_index * (size_t)cells);
        const uint4* src_lds = reinterpret_cast<const uint4*>(s_dist);
        for (int c = lane; c < cells / 8; c += kWave) out[c] = src_lds[c];
        __syncthreads();
    }
}

// ---------------------------------------------------------------------------
// Launch 2: tokens (mapf_gpt_materialize_tokens_kernel, :350-497) plus the
// agent scatter and its diagnostics (:328-347).
// ---------------------------------------------------------------------------
struct TokLayout {
    int hash_slots;  // power of two >= 2A
    int chunk;       // egos per window pass
    size_t occ_off, keys_off, vals_off, pos_off, goal_off, hist_off, greedy_off, win_off, sel_off,
        nsel_off, total;
};

__host__ __device__ inline size_t align16(size_t v) { return (v + 15) & ~(size_t)15; }

__host__ __device__ inline TokLayout tok_layout(int A, int W, int H) {
    TokLayout L;
    int s = 64;
    while (s < 2 * A) s <<= 1;
    L.hash_slots = s;
    L.chunk = A < 128 ? A : 128;
    size_t off = 0;
    L.occ_off = off;
    off = align16(off + (size_t)W * H / 8);
    L.keys_off = off;
    off = align16(off + (size_t)s * 4);
    L.vals_off = off;
    off = align16(off + (size_t)s * 4);
    L.pos_off = off;
    off = align16(off + (size_t)A * 4);
    L.goal_off = off;
    off = align16(off + (size_t)A * 4);
    L.hist_off = off;
    off = align16(off + (size_t)A * 10);
    L.greedy_off = off;
    off = align16(off + (size_t)A);
    L.win_off = off;
    off = align16(off + (size_t)L.chunk * kCostTokens * 2);
    L.sel_off = off;
    off = align16(off + (size_t)L.chunk * kVisible * 2);
    L.nsel_off = off;
    off = align16(off + (size_t)L.chunk);
    L.total = off;
    return L;
}

// 11-bit occupancy of columns y0..y0+10 of row x (bits outside the map are 0).
template <int H>
__device__ __forceinline__ uint32_t occ_window_row(const uint32_t* occ, int x, int y0) {
    uint32_t bits = 0;
#pragma unroll
    for (int c = 0; c < kDiam; ++c) {
        const int y = y0 + c;
        if (y >= 0 && y < H) bits |= ((occ[(x * H + y) >> 5] >> ((x * H + y) & 31)) & 1u) << c;
    }
    return bits;
}

template <int H>
__global__ __launch_bounds__(kTokThreads) void tokens_kernel(jl_mapfgpt_t b) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int A = b.n_agents, W = b.map_w;
    const int env = blockIdx.x;
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = tid / kWave;
    const int nwaves = kTokThreads / kWave;
    const TokLayout L = tok_layout(A, W, H);
    uint32_t* s_occ = reinterpret_cast<uint32_t*>(smem + L.occ_off);
    uint32_t* s_keys = reinterpret_cast<uint32_t*>(smem + L.keys_off);
    uint32_t* s_vals = reinterpret_cast<uint32_t*>(smem + L.vals_off);
    uint32_t* s_pos = reinterpret_cast<uint32_t*>(smem + L.pos_off);
    uint32_t* s_goal = reinterpret_cast<uint32_t*>(smem + L.goal_off);
    uint16_t* s_hist = reinterpret_cast<uint16_t*>(smem + L.hist_off);
    uint8_t* s_greedy = smem + L.greedy_off;
    uint16_t* s_win = reinterpret_cast<uint16_t*>(smem + L.win_off);
    uint16_t* s_sel = reinterpret_cast<uint16_t*>(smem + L.sel_off);
    uint8_t* s_nsel = smem + L.nsel_off;
    const uint32_t hmask = (uint32_t)L.hash_slots - 1;
    const int occ_words = W * H / 32;
    const size_t cells = (size_t)W * H;

    for (int k = tid; k < occ_words; k += kTokThreads) s_occ[k] = 0;
    for (int k = tid; k < L.hash_slots; k += kTokThreads) {
        s_keys[k] = kEmptyKey;
        s_vals[k] = kNoAgent;
    }
    __syncthreads();

    // Agents of this env: LDS state, greedy masks, active mask, scatter.
    int dup = 0, oob = 0;
    for (int a = tid; a < A; a += kTokThreads) {
        const size_t g = (size_t)env * A + a;
        const uint4 st = *reinterpret_cast<const uint4*>(b.state_packed + g * 8);
        const uint32_t px = st.y & 0xFFFFu, py = st.y >> 16;
        const uint32_t gx = st.z & 0xFFFFu, gy = st.z >> 16;
        b.active_mask[g] = (px != gx || py != gy) ? 1 : 0;
        const bool valid = px < (uint32_t)W && py < (uint32_t)H;
        s_pos[a] = valid ? (px | (py << 16)) : kNoAgent;
        s_goal[a] = st.z;
        const uint16_t* h = b.histories + g * 5;
#pragma unroll
        for (int k = 0; k < 5; ++k) s_hist[a * 5 + k] = h[k];
        uint32_t greedy = 0;
        if (valid) {
            const uint16_t* f = b.cost_to_go + g * cells;
            const int x = (int)px, y = (int)py;
            const uint32_t c0 = f[x * H + y];
            const uint32_t n0 = x > 0 ? f[(x - 1) * H + y] : kUnreachable;
            const uint32_t n1 = x + 1 < W ? f[(x + 1) * H + y] : kUnreachable;
            const uint32_t n2 = y > 0 ? f[x * H + y - 1] : kUnreachable;
            const uint32_t n3 = y + 1 < H ? f[x * H + y + 1] : kUnreachable;
            // bit (3 - dir), dir order (-1,0), (+1,0), (0,-1), (0,+1) (:465-479)
            if (n0 != kUnreachable && c0 > n0) greedy |= 8u;
            if (n1 != kUnreachable && c0 > n1) greedy |= 4u;
            if (n2 != kUnreachable && c0 > n2) greedy |= 2u;
            if (n3 != kUnreachable && c0 > n3) greedy |= 1u;
            const uint32_t cell = px * H + py;
            atomicOr(&s_occ[cell >> 5], 1u << (cell & 31));
            const uint32_t slot = hash_insert(s_keys, hmask, cell);
            // lowest id keeps a shared cell; each extra agent counts once
            const uint32_t prev = atomicMin(&s_vals[slot], (uint32_t)a);
            if (prev != kNoAgent) ++dup;
        } else {
            ++oob;
        }
        s_greedy[a] = (uint8_t)greedy;
    }
    {
        const int d = __syncthreads_count(dup);
        const int o = __syncthreads_count(oob);
        if (tid == 0) {
            if (d) atomicAdd(b.scratch + kScratchAccum + 2, d);
            if (o) atomicAdd(b.scratch + kScratchAccum + 3, o);
        }
    }
    // __syncthreads_count are barriers: LDS tables are complete here.

    for (int c0 = 0; c0 < A; c0 += L.chunk) {
        const int nch = (A - c0) < L.chunk ? (A - c0) : L.chunk;
        // Gather the cost windows of the chunk: (ego, cell) pairs spread over
        // the workgroup so every thread keeps many independent loads in flight.
        const int pairs = nch * kCostTokens;
#pragma unroll 4
        for (int p = tid; p < pairs; p += kTokThreads) {
            const int el = p / kCostTokens;
            const int c = p - el * kCostTokens;
            const int e = c0 + el;
            const uint32_t pos = s_pos[e];
            uint16_t v = kUnreachable;
            if (pos != kNoAgent) {
                const int x = (int)(pos & 0xFFFFu) + c / kDiam - kRadius;
                const int y = (int)(pos >> 16) + c % kDiam - kRadius;
                if (x >= 0 && x < W && y >= 0 && y < H) {
                    v = b.cost_to_go[((size_t)env * A + e) * cells + (size_t)(x * H + y)];
                }
            }
            s_win[el * kCostTokens + c] = v;
        }
        // Visible agents of each ego: top 13 by (Manhattan distance, id),
        // ego included (:383-431), from the LDS occupancy bitmap + hash.
        for (int el = tid; el < nch; el += kTokThreads) {
            const int e = c0 + el;
            const uint32_t pos = s_pos[e];
            int n = 0;
            int sd[kVisible];
            int sid[kVisible];
            if (pos != kNoAgent) {
                const int ex = (int)(pos & 0xFFFFu), ey = (int)(pos >> 16);
                for (int dx = -kRadius; dx <= kRadius; ++dx) {
                    const int x = ex + dx;
                    if (x < 0 || x >= W) continue;
                    uint32_t bits = occ_window_row<H>(s_occ, x, ey - kRadius);
                    while (bits) {
                        const int c = __ffs(bits) - 1;
                        bits &= bits - 1;
                        const int dy = c - kRadius;
                        const uint32_t cell = (uint32_t)(x * H + ey + dy);
                        const uint32_t slot = hash_find(s_keys, hmask, cell);
                        const int id = (int)s_vals[slot];
                        const int d = (dx < 0 ? -dx : dx) + (dy < 0 ? -dy : dy);
                        int at = n;
                        if (n == kVisible) {
                            const int ld = sd[kVisible - 1], li = sid[kVisible - 1];
                            if (!(d < ld || (d == ld && id < li))) continue;
                            at = kVisible - 1;
                        } else {
                            ++n;
                        }
                        while (at > 0 && (d < sd[at - 1] || (d == sd[at - 1] && id < sid[at - 1]))) {
                            sd[at] = sd[at - 1];
                            sid[at] = sid[at - 1];
                            --at;
                        }
                        sd[at] = d;
                        sid[at] = id;
                    }
                }
            }
            for (int s = 0; s < n; ++s) s_sel[el * kVisible + s] = (uint16_t)sid[s];
            s_nsel[el] = (uint8_t)n;
        }
        __syncthreads();

        // One wavefront per ego row: lane l builds tokens 4l..4l+3.
        for (int el = wave; el < nch; el += nwaves) {
            const int e = c0 + el;
            const uint32_t pos = s_pos[e];
            int tok[4];
            if (pos == kNoAgent) {
                tok[0] = tok[1] = tok[2] = tok[3] = kTokPad;
            } else {
                const int ex = (int)(pos & 0xFFFFu), ey = (int)(pos >> 16);
                const uint16_t* win = s_win + el * kCostTokens;
                const uint32_t center = win[kRadius * kDiam + kRadius];
                const int nsel = s_nsel[el];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int t = 4 * lane + j;
                    int v = kTokPad;
                    if (t < kCostTokens) {
                        v = cost_token(win[t], center);
                    } else if (t < kCostTokens + kVisible * kAgentTokens) {
                        const int s = (t - kCostTokens) / kAgentTokens;
                        const int f = (t - kCostTokens) - s * kAgentTokens;
                        if (s < nsel) {
                            const int o = s_sel[el * kVisible + s];
                            const uint32_t op = s_pos[o];
                            const uint32_t og = s_goal[o];
                            switch (f) {
                                case 0: v = coord_token((int)(op & 0xFFFFu) - ex); break;
                                case 1: v = coord_token((int)(op >> 16) - ey); break;
                                case 2: v = coord_token((int)(og & 0xFFFFu) - ex); break;
                                case 3: v = coord_token((int)(og >> 16) - ey); break;
                                case 9: v = kTokGreedy + s_greedy[o]; break;
                                default: {
                                    const int act = s_hist[o * 5 + (f - 4)];
                                    v = act == 5 ? kTokEmptyAction : kTokWait + act;
                                }
                            }
                        }
                    }
                    tok[j] = v;
                }
            }
            int4 out;
            out.x = tok[0];
            out.y = tok[1];
            out.z = tok[2];
            out.w = tok[3];
            reinterpret_cast<int4*>(b.tokens + ((size_t)env * A + e) * kContext)[lane] = out;
        }
        __syncthreads();
    }

    // Publish the build's diagnostics once every workgroup is done.
    if (tid == 0) {
        __threadfence();
        const int ticket = atomicAdd(b.scratch + kScratchTicket, 1);
        if (ticket == (int)gridDim.x - 1) {
            __threadfence();
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                b.diagnostics[k] = atomicExch(b.scratch + kScratchAccum + k, 0);
            }
            atomicExch(b.scratch + kScratchTicket, 0);
        }
    }
}

__global__ void append_actions_kernel(jl_mapfgpt_t b, const uint8_t* __restrict__ actions) {
    const int N = b.n_envs * b.n_agents;
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    bool bad = false;
    if (i < N) {
        uint16_t a = b.active_mask[i] ? (uint16_t)actions[i] : (uint16_t)0;
        if (a >= 5) {
            bad = true;
            a = 0;
        }
        uint16_t* h = b.histories + (size_t)i * 5;
        const uint16_t h1 = h[1], h2 = h[2], h3 = h[3], h4 = h[4];
        h[0] = h1;
        h[1] = h2;
        h[2] = h3;
        h[3] = h4;
        h[4] = a;
    }
    const uint64_t m = __ballot(bad);
    if ((threadIdx.x & (kWave - 1)) == 0 && m) atomicAdd(b.diagnostics + 1, (int)__popcll(m));
}

__global__ void fill_u16_kernel(uint16_t* p, size_t n, uint16_t v) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
         i += (size_t)gridDim.x * blockDim.x)
        p[i] = v;
}

// agent_at_cell on request: per env, lowest id keeps a shared cell.
template <int H>
__global__ __launch_bounds__(256) void agent_at_cell_kernel(jl_mapfgpt_t b) {
    const int env = blockIdx.x, A = b.n_agents, W = b.map_w;
    const size_t cells = (size_t)W * H;
    int32_t* map = b.agent_at_cell + (size_t)env * cells;
    for (size_t c = threadIdx.x; c < cells; c += blockDim.x) map[c] = 0x7FFFFFFF;
    __syncthreads();
    for (int a = threadIdx.x; a < A; a += blockDim.x) {
        const uint16_t* st = b.state_packed + ((size_t)env * A + a) * 8;
        if (st[2] < W && st[3] < H) atomicMin(&map[st[2] * H + st[3]], st[1]);
    }
    __syncthreads();
    for (size_t c = threadIdx.x; c < cells; c += blockDim.x)
        if (map[c] == 0x7FFFFFFF) map[c] = -1;
}

int check_builder(const jl_mapfgpt_t* b) {
    if (!b || b->n_envs <= 0 || b->n_agents <= 0) return JL_ERR_ARG;
    if (!profile_ok(b->map_w, b->map_h)) return JL_ERR_PROFILE;
    if ((int64_t)b->n_envs * b->n_agents > 0x7FFFFFFF) return JL_ERR_ARG;
    if (b->n_agents > 65535 || b->n_envs > 65535) return JL_ERR_ARG;
    if (!b->grid_bits || !b->state_packed || !b->histories || !b->labels || !b->cost_to_go ||
        !b->goal_cache || !b->tokens || !b->active_mask || !b->diagnostics || !b->scratch)
        return JL_ERR_ARG;
    return JL_OK;
}

template <bool kRows>
int build(const jl_mapfgpt_t* b, const int16_t* rows, const int16_t* cx, const int16_t* cy,
          const int16_t* gx, const int16_t* gy, hipStream_t stream) {
    int rc = check_builder(b);
    if (rc) return rc;
    const int N = b->n_envs * b->n_agents;
    const int W = b->map_w;
    const int grid1 = (N + kWave - 1) / kWave;
    const size_t bfs_lds = (size_t)W * b->map_h * sizeof(uint16_t);
    const TokLayout L = tok_layout(b->n_agents, W, b->map_h);
    if (L.total > 160 * 1024 || bfs_lds > 160 * 1024) return JL_ERR_PROFILE;
    JL_DISPATCH_H(b->map_h, {
        if (W <= 64) {
            hipLaunchKernelGGL((unpack_bfs_kernel<H, 1, kRows>), dim3(grid1), dim3(kWave), bfs_lds,
                               stream, *b, rows, cx, cy, gx, gy);
        } else if (W <= 128) {
            hipLaunchKernelGGL((unpack_bfs_kernel<H, 2, kRows>), dim3(grid1), dim3(kWave), bfs_lds,
                               stream, *b, rows, cx, cy, gx, gy);
        } else {
            hipLaunchKernelGGL((unpack_bfs_kernel<H, 4, kRows>), dim3(grid1), dim3(kWave), bfs_lds,
                               stream, *b, rows, cx, cy, gx, gy);
        }
        rc = launch_status();
        if (rc) return rc;
        if (b->token_events[0]) {
            rc = status(hipEventRecord((hipEvent_t)b->token_events[0], stream));
            if (rc) return rc;
        }
        hipLaunchKernelGGL((tokens_kernel<H>), dim3(b->n_envs), dim3(kTokThreads), L.total, stream,
                           *b);
        rc = launch_status();
        if (rc) return rc;
        if (b->token_events[1]) {
            rc = status(hipEventRecord((hipEvent_t)b->token_events[1], stream));
            if (rc) return rc;
        }
    });
    return JL_OK;
}

}  // namespace
}  // namespace jl

using namespace jl;

extern "C" int jl_mapfgpt_build_rows(const jl_mapfgpt_t* b, const int16_t* raw_rows,
                                     jl_stream_t stream) {
    if (!raw_rows) return JL_ERR_ARG;
    return build<true>(b, raw_rows, nullptr, nullptr, nullptr, nullptr, (hipStream_t)stream);
}

extern "C" int jl_mapfgpt_build_state(const jl_mapfgpt_t* b, const int16_t* cur_x,
                                      const int16_t* cur_y, const int16_t* goal_x,
                                      const int16_t* goal_y, jl_stream_t stream) {
    if (!cur_x || !cur_y || !goal_x || !goal_y) return JL_ERR_ARG;
    return build<false>(b, nullptr, cur_x, cur_y, goal_x, goal_y, (hipStream_t)stream);
}

extern "C" int jl_mapfgpt_append_actions(const jl_mapfgpt_t* b, const uint8_t* actions,
                                         jl_stream_t stream) {
    int rc = check_builder(b);
    if (rc) return rc;
    if (!actions) return JL_ERR_ARG;
    const int N = b->n_envs * b->n_agents;
    hipLaunchKernelGGL(append_actions_kernel, dim3((N + 255) / 256), dim3(256), 0,
                       (hipStream_t)stream, *b, actions);
    return launch_status();
}

extern "C" int jl_mapfgpt_reset_histories(const jl_mapfgpt_t* b, jl_stream_t stream) {
    int rc = check_builder(b);
    if (rc) return rc;
    const size_t n = (size_t)b->n_envs * b->n_agents * 5;
    const int blocks = (int)((n + 255) / 256 < 4096 ? (n + 255) / 256 : 4096);
    hipLaunchKernelGGL(fill_u16_kernel, dim3(blocks), dim3(256), 0, (hipStream_t)stream,
                       b->histories, n, (uint16_t)5);
    return launch_status();
}

extern "C" int jl_mapfgpt_agent_at_cell(const jl_mapfgpt_t* b, jl_stream_t stream) {
    int rc = check_builder(b);
    if (rc) return rc;
    if (!b->agent_at_cell) return JL_ERR_ARG;
    JL_DISPATCH_H(b->map_h, {
        hipLaunchKernelGGL((agent_at_cell_kernel<H>), dim3(b->n_envs), dim3(256), 0,
                           (hipStream_t)stream, *b);
    });
    return launch_status();
}
