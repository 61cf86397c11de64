// jl_costtracer.hip - CostTracer reward, observation and episode reset on gfx950.
//
// CostTracer (rebuttal/online-rl/native/src/cuda_backend/costtracer.cu) is the
// RL consumer of the simulator and the MAPF-GPT builder's distance fields: per
// agent and step a progress reward and the next goal of a fixed goal stream,
// a 2 x 11 x 11 float observation (occupancy and a normalised distance
// window, with a progress feature at the centre), and per env a reset from a
// bank of episodes when the horizon is reached.
//
// Distances are read from the builder's tiled fields (8 x 8 tiles of uint16,
// one 128-byte line each), which hold what the builder last wrote into
// cost_to_go (plus, on small maps, greedy marks that field_distance strips):
// an 11 x 11 window touches 4 to 9 lines instead of 11 to 22 row-major ones.  The observation runs four agents per wavefront (two
// window cells per lane and agent, all loads of the four in flight together,
// the window reductions as DPP steps); the 16 agents of a workgroup assemble
// their floats in LDS, which leave as one contiguous run of 16-byte stores.
#include "jl_common.h"

namespace jl {
namespace {

typedef float v4f __attribute__((ext_vector_type(4)));
constexpr int kObsWaves = 4;  // wavefronts per workgroup of the observation
constexpr int kObsPer = 4;    // agents per wavefront
constexpr int kObsAgents = kObsWaves * kObsPer;
constexpr int kObsCells = kCostTokens;       // 121
constexpr int kObsFloats = 2 * kObsCells;    // 242
constexpr int kObsCentre = kRadius * kDiam + kRadius;  // 60

// Wavefront max / min, wavefront-uniform result: DPP steps within quads,
// half-rows and rows, then row 0 into row 1 and row 2 into row 3 (bcast15,
// rows 1 and 3 written) and rows 0-1 into rows 2-3 (bcast31, rows 2 and 3
// written), which leaves the result in lane 63.  Lanes a step does not
// write keep their own value (old = v), the identity of max and min.
template <bool kMax>
__device__ __forceinline__ int wave_reduce(int v) {
    auto op = [](int a, int b) { return kMax ? max(a, b) : min(a, b); };
    v = op(v, __builtin_amdgcn_update_dpp(v, v, 0xB1, 0xF, 0xF, false));  // quad_perm [1,0,3,2]
    v = op(v, __builtin_amdgcn_update_dpp(v, v, 0x4E, 0xF, 0xF, false));  // quad_perm [2,3,0,1]
    v = op(v, __builtin_amdgcn_update_dpp(v, v, 0x141, 0xF, 0xF, false)); // row_half_mirror
    v = op(v, __builtin_amdgcn_update_dpp(v, v, 0x140, 0xF, 0xF, false)); // row_mirror
    v = op(v, __builtin_amdgcn_update_dpp(v, v, 0x142, 0xA, 0xF, false)); // row_bcast15
    v = op(v, __builtin_amdgcn_update_dpp(v, v, 0x143, 0xC, 0xF, false)); // row_bcast31
    return __builtin_amdgcn_readlane(v, kWave - 1);
}

__device__ __forceinline__ int wave_max(int v) { return wave_reduce<true>(v); }
__device__ __forceinline__ int wave_min(int v) { return wave_reduce<false>(v); }

// progress_goals, costtracer.cu:5-23: reward 0.1 when the distance to the goal
// fell below the best so far, the goal hit flag, and on a hit the next goal of
// the agent's stream (best reset to -1 so the next observation re-anchors it).
template <int H>
__global__ __launch_bounds__(256) void reward_goals_kernel(jl_sim_t s, const uint16_t* __restrict__ tiles,
                                                           int32_t* __restrict__ best,
                                                           const int16_t* __restrict__ targets,
                                                           int length, int32_t* __restrict__ cursor,
                                                           float* __restrict__ rewards,
                                                           float* __restrict__ reached, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const int W = s.map_w;
    const int x = s.cur_x[i], y = s.cur_y[i];
    const int gx = s.goal_x[i], gy = s.goal_y[i];
    const int b0 = best[i];
    const int k = cursor[i];
    const int xc = x < W ? x : W - 1, yc = y < H ? y : H - 1;
    const int d = (int)field_distance(tiles[(size_t)i * tiled_cells(W, H) + tile_offset(xc, yc, W)],
                                      field_mask(W, H));
    rewards[i] = d < b0 ? 0.1f : 0.0f;
    int bn = min(b0, d);
    const bool hit = x == gx && y == gy;
    reached[i] = hit ? 1.0f : 0.0f;
    if (hit) {
        cursor[i] = k + 1;
        // the stream outlasts the horizon (length > horizon, checked by the
        // caller); a cursor past its end keeps the goal
        if (k >= 0 && k < length) {
            const int16_t* t = targets + ((size_t)i * length + k) * 2;
            s.goal_x[i] = (uint16_t)t[0];
            s.goal_y[i] = (uint16_t)t[1];
        }
        bn = -1;  // even when the next target equals the old one
    }
    if (bn != b0) best[i] = bn;
}

// The observations of kObsPer consecutive agents i0.. (nvalid of them real)
// into o[k * 242 ..] (LDS), by one wavefront: every load of the group is in
// flight at once (their positions in one round trip, then the windows and
// the occupancy words of all of them in a second), and the per-agent
// reductions interleave.
template <int H>
__device__ __forceinline__ void observe_agents(const jl_sim_t& s, const jl_mapfgpt_t& b,
                                               int32_t* __restrict__ best, float* o, int i0,
                                               int nvalid, int lane) {
    const int W = s.map_w, A = s.n_agents;
    const size_t tcells = tiled_cells(W, H);
    const uint32_t fmask = field_mask(W, H);
    const int words = W * H / 32;
    // lane k < nvalid fetches agent i0 + k's position, best and refresh flag
    const int il = i0 + (lane < nvalid ? lane : 0);
    const int pxl = s.cur_x[il], pyl = s.cur_y[il];
    const int32_t bestl = best[il];
    const int resetl = b.state_packed[(size_t)il * 8 + 7];
    // window cells t0 = lane, t1 = lane + 64 (a cell when < 121); t = r*11 + c
    // is (cx + r - 5, cy + c - 5)
    const int t0 = lane, t1 = lane + kWave;
    const bool has1 = t1 < kObsCells;
    const int r0 = t0 / kDiam - kRadius, q0 = t0 % kDiam - kRadius;
    const int r1 = t1 / kDiam - kRadius, q1 = t1 % kDiam - kRadius;
    int cxk[kObsPer], cyk[kObsPer];
    bool in0[kObsPer], in1[kObsPer];
    uint32_t raw0[kObsPer], raw1[kObsPer], w0[kObsPer], w1[kObsPer], c0[kObsPer], c1[kObsPer];
#pragma unroll
    for (int k = 0; k < kObsPer; ++k) {
        const int i = i0 + (k < nvalid ? k : 0);
        cxk[k] = __builtin_amdgcn_readlane(pxl, k);
        cyk[k] = __builtin_amdgcn_readlane(pyl, k);
        const int x0 = cxk[k] + r0, y0 = cyk[k] + q0, x1 = cxk[k] + r1, y1 = cyk[k] + q1;
        in0[k] = x0 >= 0 && x0 < W && y0 >= 0 && y0 < H;
        in1[k] = has1 && x1 >= 0 && x1 < W && y1 >= 0 && y1 < H;
        // reads at clamped cells, unconditionally
        const int xa = in0[k] ? x0 : 0, ya = in0[k] ? y0 : 0;
        const int xb = in1[k] ? x1 : 0, yb = in1[k] ? y1 : 0;
        const uint16_t* f = b.cost_tiles + (size_t)i * tcells;
        const uint32_t* ocp = s.grid_ocp + (size_t)(i / A) * words;
        c0[k] = (uint32_t)(xa * H + ya);
        c1[k] = (uint32_t)(xb * H + yb);
        raw0[k] = f[tile_offset(xa, ya, W)];  // marks stripped where the distance is taken
        raw1[k] = f[tile_offset(xb, yb, W)];
        w0[k] = ocp[c0[k] >> 5];
        w1[k] = ocp[c1[k] >> 5];
    }
#pragma unroll
    for (int k = 0; k < kObsPer; ++k) {
        if (k >= nvalid) break;  // wavefront-uniform
        const int d0 = (in0[k] && raw0[k] != kUnreachable) ? (int)(raw0[k] & fmask) : -1;
        const int d1 = (in1[k] && raw1[k] != kUnreachable) ? (int)(raw1[k] & fmask) : -1;
        // largest reachable distance in the window (0 if none)
        const int M = wave_max(max(max(0, d0), has1 ? max(0, d1) : 0));
        // cells without a distance sit 4 past the largest one
        int v0 = d0 < 0 ? d0 + 5 + M : d0;
        int v1 = d1 < 0 ? d1 + 5 + M : d1;
        const int m = wave_min(has1 ? min(v0, v1) : v0);
        v0 -= m;
        v1 -= m;
        const int V = wave_max(has1 ? max(v0, v1) : v0);
        // the distance at the agent's cell is the window centre (t = 60, lane 60)
        const int current =
            (int)field_distance((uint32_t)__builtin_amdgcn_readlane((int)raw0[k], kObsCentre), fmask);
        int bi = __builtin_amdgcn_readlane(bestl, k);
        if (bi < 0 || __builtin_amdgcn_readlane(resetl, k) != 0) {
            bi = current;
            if (lane == 0) best[i0 + k] = bi;
        }
        float* ok = o + k * kObsFloats;
        ok[t0] = (in0[k] && ((w0[k] >> (c0[k] & 31)) & 1u)) ? 1.0f : 0.0f;
        const float fv = (float)V;
        float n0 = V > 0 ? (float)(V - v0) / fv : 0.0f;
        if (t0 == kObsCentre) n0 = -fminf(1.0f, (float)(current - bi + 1) / 64.0f);
        ok[kObsCells + t0] = n0;
        if (has1) {
            ok[t1] = (in1[k] && ((w1[k] >> (c1[k] & 31)) & 1u)) ? 1.0f : 0.0f;
            ok[kObsCells + t1] = V > 0 ? (float)(V - v1) / fv : 0.0f;
        }
    }
}

// observe, costtracer.cu:25-64 (one 128-thread block per agent there).
template <int H>
__global__ __launch_bounds__(kWave * kObsWaves) void observe_kernel(jl_sim_t s, jl_mapfgpt_t b,
                                                                    int32_t* __restrict__ best,
                                                                    float* __restrict__ out, int n,
                                                                    int vec_store) {
    __shared__ __align__(16) float s_out[kObsAgents * kObsFloats];
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int first = blockIdx.x * kObsAgents;
    const int i0 = first + wave * kObsPer;
    const int nvalid = min(kObsPer, n - i0);
    if (nvalid > 0) observe_agents<H>(s, b, best, s_out + wave * kObsPer * kObsFloats, i0, nvalid, lane);
    __syncthreads();
    // the workgroup's agents are one contiguous run of floats (121 whole
    // 128-byte lines for 16 agents), stored non-temporally: the 127 MB of
    // observations of a C2-shaped step then stay out of the caches, whose
    // window lines the next step reads again (observe 45.5 -> 40.7 us)
    float* o = out + (size_t)first * kObsFloats;
    const int count = min(kObsAgents, n - first) * kObsFloats;
    int k0 = 0;
    if (vec_store) {
        const v4f* src = reinterpret_cast<const v4f*>(s_out);
        v4f* dst = reinterpret_cast<v4f*>(o);
        for (int k = threadIdx.x; k < count / 4; k += kWave * kObsWaves) __builtin_nontemporal_store(src[k], dst + k);
        k0 = count / 4 * 4;
    }
    for (int k = k0 + threadIdx.x; k < count; k += kWave * kObsWaves) o[k] = s_out[k];
}

// reset_selected, costtracer.cu:66-85: envs at the horizon start the next
// episode of the bank (positions and goals), with cursors 0, best -1, step
// count 0 and the occupancy of the new positions.
template <int H>
__global__ __launch_bounds__(256) void reset_kernel(jl_sim_t s, const int16_t* __restrict__ pos,
                                                    const int16_t* __restrict__ goal, int bank,
                                                    int32_t* __restrict__ episodes,
                                                    int32_t* __restrict__ cursors,
                                                    int32_t* __restrict__ best, int horizon) {
    extern __shared__ __align__(16) uint32_t s_ocp[];
    __shared__ int s_episode;
    const int e = blockIdx.x, tid = threadIdx.x;
    const int A = s.n_agents, W = s.map_w, E = s.n_envs;
    if (s.step_counts[e] < horizon) return;  // uniform per workgroup
    const int words = W * H / 32;
    for (int k = tid; k < words; k += blockDim.x) s_ocp[k] = 0;
    if (tid == 0) {
        const int next = episodes[e] + 1;
        episodes[e] = next;
        int ep = next % bank;
        s_episode = ep < 0 ? ep + bank : ep;
        s.step_counts[e] = 0;
    }
    __syncthreads();
    const size_t bank_base = (size_t)s_episode * E * A;
    for (int a = tid; a < A; a += blockDim.x) {
        const size_t g = (size_t)e * A + a;
        const size_t k = (bank_base + g) * 2;
        const int x = pos[k], y = pos[k + 1];
        s.cur_x[g] = (uint16_t)x;
        s.cur_y[g] = (uint16_t)y;
        s.goal_x[g] = (uint16_t)goal[k];
        s.goal_y[g] = (uint16_t)goal[k + 1];
        cursors[g] = 0;
        best[g] = -1;
        if (x >= 0 && x < W && y >= 0 && y < H) {
            const uint32_t cell = (uint32_t)(x * H + y);
            atomicOr(&s_ocp[cell >> 5], 1u << (cell & 31));
        }
    }
    __syncthreads();
    uint32_t* gocp = s.grid_ocp + (size_t)e * words;
    for (int k = tid; k < words; k += blockDim.x) gocp[k] = s_ocp[k];
}

int check_pair(const jl_sim_t* s, const jl_mapfgpt_t* b) {
    if (!s || !b || s->n_envs <= 0 || s->n_agents <= 0) return JL_ERR_ARG;
    if (!profile_ok(s->map_w, s->map_h)) return JL_ERR_PROFILE;
    if (b->n_envs != s->n_envs || b->n_agents != s->n_agents || b->map_w != s->map_w ||
        b->map_h != s->map_h)
        return JL_ERR_ARG;
    if ((int64_t)s->n_envs * s->n_agents > 0x7FFFFFFF) return JL_ERR_ARG;
    if (!s->cur_x || !s->cur_y || !s->goal_x || !s->goal_y || !s->grid_ocp || !b->cost_tiles ||
        !b->state_packed)
        return JL_ERR_ARG;
    return JL_OK;
}

}  // namespace
}  // namespace jl

using namespace jl;

extern "C" int jl_costtracer_reward_goals(const jl_sim_t* s, const jl_mapfgpt_t* b, int32_t* best,
                                          const int16_t* targets, int32_t target_length,
                                          int32_t* cursor, float* rewards, float* reached,
                                          jl_stream_t stream) {
    int rc = check_pair(s, b);
    if (rc) return rc;
    if (!best || !targets || target_length <= 0 || !cursor || !rewards || !reached) return JL_ERR_ARG;
    const int n = s->n_envs * s->n_agents;
    JL_DISPATCH_H(s->map_h, {
        hipLaunchKernelGGL((reward_goals_kernel<H>), dim3((n + 255) / 256), dim3(256), 0,
                           (hipStream_t)stream, *s, b->cost_tiles, best, targets, target_length,
                           cursor, rewards, reached, n);
    });
    return launch_status();
}

extern "C" int jl_costtracer_observe(const jl_sim_t* s, const jl_mapfgpt_t* b, int32_t* best,
                                     float* output, jl_stream_t stream) {
    int rc = check_pair(s, b);
    if (rc) return rc;
    if (!best || !output) return JL_ERR_ARG;
    const int n = s->n_envs * s->n_agents;
    JL_DISPATCH_H(s->map_h, {
        hipLaunchKernelGGL((observe_kernel<H>), dim3((n + kObsAgents - 1) / kObsAgents),
                           dim3(kWave * kObsWaves), 0, (hipStream_t)stream, *s, *b, best, output, n,
                           ((uintptr_t)output & 15) == 0 ? 1 : 0);
    });
    return launch_status();
}

extern "C" int jl_costtracer_reset(const jl_sim_t* s, const int16_t* bank_positions,
                                   const int16_t* bank_goals, int32_t bank_episodes,
                                   int32_t* episodes, int32_t* cursors, int32_t* best,
                                   int32_t horizon, jl_stream_t stream) {
    if (!s || s->n_envs <= 0 || s->n_agents <= 0) return JL_ERR_ARG;
    if (!profile_ok(s->map_w, s->map_h)) return JL_ERR_PROFILE;
    if (!bank_positions || !bank_goals || bank_episodes <= 0 || !episodes || !cursors || !best ||
        !s->step_counts || !s->grid_ocp || !s->cur_x || !s->cur_y || !s->goal_x || !s->goal_y)
        return JL_ERR_ARG;
    const size_t lds = (size_t)s->map_w * s->map_h / 8;
    JL_DISPATCH_H(s->map_h, {
        hipLaunchKernelGGL((reset_kernel<H>), dim3(s->n_envs), dim3(256), lds, (hipStream_t)stream,
                           *s, bank_positions, bank_goals, bank_episodes, episodes, cursors, best,
                           horizon);
    });
    return launch_status();
}
