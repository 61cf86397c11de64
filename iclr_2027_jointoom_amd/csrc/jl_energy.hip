// jl_energy.hip - uint8 "energy" BFS fields for the MAGAT builder on gfx950.
//
// One wavefront serves 64 consecutive jobs: it ballots the jobs that need a
// field and runs the bit-parallel BFS (jl_bfs.h) for each, capped at 254
// levels like generate_energy_map_kernel (energy_map.cu:174), staging the
// distances in LDS and storing 255-d with 16-byte coalesced writes.  The
// reference launches one 128-thread block per row whether or not its row
// needs a refresh (energy_map.cu:262-271) and finds the changed rows with a
// host-synchronised cumsum (grid_world_simulator.cpp:707-753); here the
// incremental derived state is one launch on small maps (the scan, the
// packed rows and the fields of changed goals: goal_changed_refresh_kernel).
#include "jl_bfs.h"
#include "jl_common.h"

namespace jl {
namespace {

constexpr int kEnergyCap = 254;

// One field by one wavefront (its LDS orderings are the wavefront's own, so
// several wavefronts of a workgroup may run fields side by side).
template <int H, int R>
__device__ void energy_field(const uint32_t* __restrict__ env_bits, int W, int gx, int gy,
                             uint8_t* s_dist, uint8_t* __restrict__ out) {
    constexpr int HW = RowWords<H>::HW;
    const int lane = threadIdx.x & (kWave - 1);
    const int cells = W * H;
    for (int c = lane; c < cells; c += kWave) s_dist[c] = 255;
    wave_sync();
    uint64_t fr[R][HW];
    load_free_rows<H, R>(env_bits, W, fr);
    if (lane == 0) s_dist[gx * H + gy] = 0;
    wave_sync();
    wave_bfs<H, R, uint8_t, false>(fr, gx, gy, kEnergyCap, s_dist);
    wave_sync();
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
    wave_sync();
}

// Jobs are state rows (launch_energy_map_kernel semantics).
template <int H, int R>
__global__ __launch_bounds__(kWave) void energy_rows_kernel(const uint32_t* __restrict__ grid_bits,
                                                             uint8_t* __restrict__ energy,
                                                             const uint16_t* __restrict__ states,
                                                             int length, int E, int A, int W,
                                                             int incremental_only) {
    extern __shared__ uint8_t s_dist[];
    const int lane = threadIdx.x & (kWave - 1);
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
    const int lane = threadIdx.x & (kWave - 1);
    const int A = s.n_agents, W = s.map_w;
    const int N = s.n_envs * A;
    // the scan's total: no goal changed, no field and no row to write
    if (!all_agents && prefix && prefix[N - 1] == 0) return;
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

// Incremental derived state in one launch: goal_changed_scan_kernel and
// energy_flagged_kernel together, for at most kRefreshGroups * 1,024 agents
// on maps of at most 4,096 cells and 64 rows.  Workgroup w owns agents
// [w * 1024, (w + 1) * 1024): it sums the values before its range and all of
// them (16-byte words from the L2), scans its range and writes the prefixes;
// each changed agent writes its state row at prefix - 1 (and zero rows over
// the gap that a value above 1 leaves below it), and the rows of the range
// at or past the total are cleared, so every row is written once without
// ordering between workgroups (grid_world_simulator.cpp:709-733,
// pack_changed_agent_state_kernel, 128_agents_map_step.cu:469-511).  Then
// each wavefront runs the energy BFS of its changed agents in its own LDS
// field (energy_map.cu:80-272).
constexpr int kRefreshThreads = 1024;
constexpr int kRefreshWaves = kRefreshThreads / kWave;
constexpr int kRefreshGroups = 128;

template <int H>
__global__ __launch_bounds__(kRefreshThreads) void goal_changed_refresh_kernel(jl_sim_t s, uint8_t* __restrict__ energy,
                                                                            int64_t* __restrict__ prefix,
                                                                            int64_t* __restrict__ count,
                                                                            uint16_t* __restrict__ changed) {
    extern __shared__ uint8_t s_fields[];  // one W*H field per wavefront
    __shared__ int64_t s_before[kRefreshWaves];
    __shared__ int64_t s_all[kRefreshWaves];
    __shared__ uint32_t s_scan[kRefreshWaves];
    const int tid = threadIdx.x, lane = tid & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);  // uniform per wavefront
    const int A = s.n_agents, W = s.map_w;
    const int N = s.n_envs * A;
    const int c0 = blockIdx.x * kRefreshThreads;
    const int g = c0 + tid;
    const uint8_t* f = s.goal_changed;
    const uint32_t v = g < N ? f[g] : 0u;
    uint32_t gx = 0, gy = 0;
    if (g < N) {
        gx = s.goal_x[g];
        gy = s.goal_y[g];
    }
    // the values before the range and all of them (c0 is a multiple of 16)
    uint64_t before = 0, all = 0;
    const bool vec = (reinterpret_cast<uintptr_t>(f) & 15u) == 0;
    const int words = vec ? N / 16 : 0;
#pragma unroll 8
    for (int k = tid; k < words; k += kRefreshThreads) {
        const uint4 w = reinterpret_cast<const uint4*>(f)[k];
        const uint32_t t = byte_sum(w.x) + byte_sum(w.y) + byte_sum(w.z) + byte_sum(w.w);
        all += t;
        before += k * 16 < c0 ? t : 0u;
    }
    for (int k = words * 16 + tid; k < N; k += kRefreshThreads) {
        all += f[k];
        before += k < c0 ? f[k] : 0u;
    }
    for (int off = kWave / 2; off > 0; off >>= 1) {
        before += __shfl_xor(before, off, kWave);
        all += __shfl_xor(all, off, kWave);
    }
    // this thread's value scanned across the workgroup (a wavefront's sum is
    // at most 64 * 255)
    uint32_t incl = v;
    for (int off = 1; off < kWave; off <<= 1) {
        const uint32_t t = __shfl_up(incl, off, kWave);
        if (lane >= off) incl += t;
    }
    if (lane == 0) {
        s_before[wave] = (int64_t)before;
        s_all[wave] = (int64_t)all;
    }
    if (lane == kWave - 1) s_scan[wave] = incl;
    __syncthreads();
    int64_t run = incl, total = 0;
#pragma unroll
    for (int k = 0; k < kRefreshWaves; ++k) {
        run += s_before[k] + (k < wave ? s_scan[k] : 0u);
        total += s_all[k];
    }
    if (g < N) {
        prefix[g] = run;
        if (g == N - 1) count[0] = run;
    }
    if (changed && g < N) {
        const uint4 zero = make_uint4(0, 0, 0, 0);
        uint4* rows = reinterpret_cast<uint4*>(changed);
        if (g >= total) rows[g] = zero;
        if (v) {
            for (int64_t r = run - v; r < run - 1; ++r) rows[r] = zero;
            const uint32_t e = (uint32_t)(g / A), a = (uint32_t)(g - (int)e * A);
            uint4 row;
            row.x = (e & 0xFFFFu) | (a << 16);
            row.y = (uint32_t)s.cur_x[g] | ((uint32_t)s.cur_y[g] << 16);
            row.z = gx | (gy << 16);
            row.w = (uint32_t)s.actions[g] | (1u << 16);
            rows[run - 1] = row;
        }
    }
    // the energy fields of this wavefront's changed agents
    const int cells = W * H;
    uint64_t todo = __ballot(v != 0 && gx < (uint32_t)W && gy < (uint32_t)H);
    uint8_t* s_dist = s_fields + (size_t)wave * cells;
    while (todo) {
        const int src = __ffsll((unsigned long long)todo) - 1;
        todo &= todo - 1;
        const int x = __shfl((int)gx, src, kWave);
        const int y = __shfl((int)gy, src, kWave);
        const int gi = c0 + wave * kWave + src;
        const int e = gi / A;
        energy_field<H, 1>(s.grid_bits + (size_t)e * (cells / 32), W, x, y, s_dist,
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

extern "C" int jl_goal_changed_refresh(const jl_sim_t* s, uint8_t* energy, int64_t* prefix, int64_t* count,
                                       uint16_t* changed_states, jl_stream_t stream) {
    if (!s || !energy || !prefix || !count || !s->grid_bits || !s->goal_x || !s->goal_y ||
        !s->goal_changed)
        return JL_ERR_ARG;
    if (s->n_envs <= 0 || s->n_agents <= 0) return JL_ERR_ARG;
    if (!profile_ok(s->map_w, s->map_h)) return JL_ERR_PROFILE;
    if (changed_states && (!s->cur_x || !s->cur_y || !s->actions)) return JL_ERR_ARG;
    const int64_t N = (int64_t)s->n_envs * s->n_agents;
    const int cells = s->map_w * s->map_h;
    if (N <= (int64_t)kRefreshThreads * kRefreshGroups && s->map_w <= kWave && cells <= 4096) {
        const unsigned grid = (unsigned)((N + kRefreshThreads - 1) / kRefreshThreads);
        const size_t lds = (size_t)kRefreshWaves * cells;
        JL_DISPATCH_H(s->map_h, {
            hipLaunchKernelGGL(goal_changed_refresh_kernel<H>, dim3(grid), dim3(kRefreshThreads), lds,
                               (hipStream_t)stream, *s, energy, prefix, count, changed_states);
        });
        return launch_status();
    }
    const int rc = jl_goal_changed_scan(s, prefix, count, changed_states, stream);
    if (rc) return rc;
    return jl_energy_maps_flagged(s, energy, 0, prefix, changed_states, stream);
}
