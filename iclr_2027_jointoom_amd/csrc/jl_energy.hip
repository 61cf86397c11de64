// jl_energy.hip - uint8 "energy" BFS fields for the MAGAT builder on gfx950.
//
// One wavefront serves 64 consecutive jobs: it ballots the jobs that need a
// field and runs the bit-parallel BFS (jl_bfs.h) for each, capped at 254
// levels like generate_energy_map_kernel (energy_map.cu:174), staging the
// distances in LDS and storing 255-d with 16-byte coalesced writes.  The
// reference launches one 128-thread block per row whether or not its row
// needs a refresh (energy_map.cu:262-271) and finds the changed rows with a
// host-synchronised cumsum (grid_world_simulator.cpp:707-753).
#include "jl_bfs.h"
#include "jl_common.h"

namespace jl {
namespace {

constexpr int kEnergyCap = 254;

template <int H, int R>
__device__ void energy_field(const uint32_t* __restrict__ env_bits, int W, int gx, int gy,
                             uint8_t* s_dist, uint8_t* __restrict__ out) {
    constexpr int HW = RowWords<H>::HW;
    const int lane = threadIdx.x;
    const int cells = W * H;
    for (int c = lane; c < cells; c += kWave) s_dist[c] = 255;
    __syncthreads();
    uint64_t fr[R][HW];
    load_free_rows<H, R>(env_bits, W, fr);
    if (lane == 0) s_dist[gx * H + gy] = 0;
    __syncthreads();
    wave_bfs<H, R, uint8_t, false>(fr, gx, gy, kEnergyCap, s_dist);
    __syncthreads();
    const uint4* src = reinterpret_cast<const uint4*>(s_dist);
    uint4* dst = reinterpret_cast<uint4*>(out);
    for (int c = lane; c < cells / 16; c += kWave) {
        uint4 v = src[c];
        uint32_t* w = reinterpret_cast<uint32_t*>(&v);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            uint32_t o = 0;
#pragma unroll
            for (int byte = 0; byte < 4; ++byte) {
                const uint32_t d = (w[k] >> (8 * byte)) & 0xFFu;
                o |= (d == 255u ? 0u : 255u - d) << (8 * byte);
            }
            w[k] = o;
        }
        dst[c] = v;
    }
    __syncthreads();
}

// Jobs are state rows (launch_energy_map_kernel semantics).
template <int H, int R>
__global__ __launch_bounds__(kWave) void energy_rows_kernel(const uint32_t* __restrict__ grid_bits,
                                                             uint8_t* __restrict__ energy,
                                                             const uint16_t* __restrict__ states,
                                                             int length, int E, int A, int W,
                                                             int incremental_only) {
    extern __shared__ uint8_t s_dist[];
    const int lane = threadIdx.x;
    const int b = blockIdx.x * kWave + lane;
    bool run = false;
    uint32_t env = 0, agent = 0, gx = 0, gy = 0;
    if (b < length) {
        const uint4 r = *reinterpret_cast<const uint4*>(states + (size_t)b * 8);
        env = r.x & 0xFFFFu;
        agent = r.x >> 16;
        gx = r.z & 0xFFFFu;
        gy = r.z >> 16;
        const uint32_t reset = r.w >> 16;
        run = !(incremental_only && reset == 0) && env < (uint32_t)E && agent < (uint32_t)A &&
              gx < (uint32_t)W && gy < (uint32_t)H;
    }
    uint64_t todo = __ballot(run);
    const size_t cells = (size_t)W * H;
    const int words = W * H / 32;
    while (todo) {
        const int src = __ffsll((unsigned long long)todo) - 1;
        todo &= todo - 1;
        const int e = __shfl((int)env, src, kWave);
        const int a = __shfl((int)agent, src, kWave);
        const int x = __shfl((int)gx, src, kWave);
        const int y = __shfl((int)gy, src, kWave);
        energy_field<H, R>(grid_bits + (size_t)e * words, W, x, y, s_dist,
                           energy + ((size_t)e * A + a) * cells);
    }
}

// Jobs are simulator agents whose goal_changed flag is set (or all).
template <int H, int R>
__global__ __launch_bounds__(kWave) void energy_flagged_kernel(jl_sim_t s, uint8_t* __restrict__ energy,
                                                                int all_agents,
                                                                const int64_t* __restrict__ prefix,
                                                                uint16_t* __restrict__ changed) {
    extern __shared__ uint8_t s_dist[];
    const int lane = threadIdx.x;
    const int A = s.n_agents, W = s.map_w;
    const int N = s.n_envs * A;
    const int g = blockIdx.x * kWave + lane;
    bool run = false;
    uint32_t gx = 0, gy = 0;
    if (g < N) {
        gx = s.goal_x[g];
        gy = s.goal_y[g];
        const bool flagged = s.goal_changed[g] != 0;
        run = (all_agents || flagged) && gx < (uint32_t)W && gy < (uint32_t)H;
        if (!all_agents && flagged && prefix && changed) {
            const int64_t slot = prefix[g] - 1;
            const uint32_t e = (uint32_t)(g / A), a = (uint32_t)(g - (int)e * A);
            uint4 v;
            v.x = (e & 0xFFFFu) | (a << 16);
            v.y = (uint32_t)s.cur_x[g] | ((uint32_t)s.cur_y[g] << 16);
            v.z = gx | (gy << 16);
            v.w = (uint32_t)s.actions[g] | (1u << 16);
            *reinterpret_cast<uint4*>(changed + slot * 8) = v;
        }
    }
    uint64_t todo = __ballot(run);
    const size_t cells = (size_t)W * H;
    const int words = W * H / 32;
    while (todo) {
        const int src = __ffsll((unsigned long long)todo) - 1;
        todo &= todo - 1;
        const int x = __shfl((int)gx, src, kWave);
        const int y = __shfl((int)gy, src, kWave);
        const int gi = blockIdx.x * kWave + src;
        const int e = gi / A;
        energy_field<H, R>(s.grid_bits + (size_t)e * words, W, x, y, s_dist,
                           energy + (size_t)gi * cells);
    }
}

}  // namespace
}  // namespace jl

using namespace jl;

extern "C" int jl_energy_maps(const uint32_t* grid_bits, uint8_t* energy, const uint16_t* states,
                              int32_t length, int32_t n_envs, int32_t n_agents, int32_t map_w,
                              int32_t map_h, int32_t incremental_only, jl_stream_t stream) {
    if (!grid_bits || !energy || n_envs <= 0 || n_agents <= 0 || length < 0) return JL_ERR_ARG;
    if (length == 0) return JL_OK;
    if (!states) return JL_ERR_ARG;
    if (!profile_ok(map_w, map_h)) return JL_ERR_PROFILE;
    const int grid = (length + kWave - 1) / kWave;
    const size_t lds = (size_t)map_w * map_h;
    JL_DISPATCH_H(map_h, {
        if (map_w <= 64) {
            hipLaunchKernelGGL((energy_rows_kernel<H, 1>), dim3(grid), dim3(kWave), lds,
                               (hipStream_t)stream, grid_bits, energy, states, length, n_envs,
                               n_agents, map_w, incremental_only);
        } else if (map_w <= 128) {
            hipLaunchKernelGGL((energy_rows_kernel<H, 2>), dim3(grid), dim3(kWave), lds,
                               (hipStream_t)stream, grid_bits, energy, states, length, n_envs,
                               n_agents, map_w, incremental_only);
        } else {
            hipLaunchKernelGGL((energy_rows_kernel<H, 4>), dim3(grid), dim3(kWave), lds,
                               (hipStream_t)stream, grid_bits, energy, states, length, n_envs,
                               n_agents, map_w, incremental_only);
        }
    });
    return launch_status();
}

extern "C" int jl_energy_maps_flagged(const jl_sim_t* s, uint8_t* energy, int32_t all_agents,
                                      const int64_t* changed_prefix, uint16_t* changed_states,
                                      jl_stream_t stream) {
    if (!s || !energy || !s->grid_bits || !s->goal_x || !s->goal_y || !s->goal_changed)
        return JL_ERR_ARG;
    if (s->n_envs <= 0 || s->n_agents <= 0) return JL_ERR_ARG;
    if (!profile_ok(s->map_w, s->map_h)) return JL_ERR_PROFILE;
    const int N = s->n_envs * s->n_agents;
    const int grid = (N + kWave - 1) / kWave;
    const size_t lds = (size_t)s->map_w * s->map_h;
    JL_DISPATCH_H(s->map_h, {
        if (s->map_w <= 64) {
            hipLaunchKernelGGL((energy_flagged_kernel<H, 1>), dim3(grid), dim3(kWave), lds,
                               (hipStream_t)stream, *s, energy, all_agents, changed_prefix,
                               changed_states);
        } else if (s->map_w <= 128) {
            hipLaunchKernelGGL((energy_flagged_kernel<H, 2>), dim3(grid), dim3(kWave), lds,
                               (hipStream_t)stream, *s, energy, all_agents, changed_prefix,
                               changed_states);
        } else {
            hipLaunchKernelGGL((energy_flagged_kernel<H, 4>), dim3(grid), dim3(kWave), lds,
                               (hipStream_t)stream, *s, energy, all_agents, changed_prefix,
                               changed_states);
        }
    });
    return launch_status();
}
