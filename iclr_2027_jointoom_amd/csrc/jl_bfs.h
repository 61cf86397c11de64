// jl_bfs.h - wavefront-level bit-parallel BFS over one map.
//
// One 64-lane wavefront runs one BFS.  Lane l owns map rows x = l + 64*r
// (r < R, so W <= 64*R); a row is held as HW 64-bit masks over its H
// columns.  A level expands the frontier with shifts inside the row
// (y +- 1, carrying across words) and with the frontier rows of the lanes
// above/below (x +- 1, via DPP whole-wavefront shifts by one lane, and
// readlane across the 64-row groups), masks with free & ~visited, and
// stops when no lane found a new cell.  Newly reached cells get their level
// written into an LDS distance array; every other access is a register op,
// so a level costs O(R*HW) VALU work instead of one thread per frontier
// node with two workgroup barriers (energy_map.cu:174-245,
// mapf_gpt_cuda.cu:255-318).  BFS distances are unique, so the field
// equals the reference's level-synchronous queue BFS.
#pragma once

#include "jl_common.h"

namespace jl {

// Value of lane - 1 (lane 0 reads 0) and of lane + 1 (lane 63 reads 0): DPP
// wave_shr:1 / wave_shl:1 on both halves, no LDS round trip.  Every lane of
// the wavefront must be active.
__device__ __forceinline__ uint64_t from_lane_below(uint64_t v) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)v, 0x138, 0xF, 0xF, false);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(v >> 32), 0x138, 0xF, 0xF, false);
    return ((uint64_t)hi << 32) | lo;
}

__device__ __forceinline__ uint64_t from_lane_above(uint64_t v) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)v, 0x130, 0xF, 0xF, false);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(v >> 32), 0x130, 0xF, 0xF, false);
    return ((uint64_t)hi << 32) | lo;
}

// Value of a fixed lane, wavefront-uniform.
__device__ __forceinline__ uint64_t lane_value(uint64_t v, int lane) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, lane);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), lane);
    return ((uint64_t)hi << 32) | lo;
}

template <int H>
struct RowWords {
    static constexpr int HW = (H + 63) / 64;
    static constexpr uint64_t kLastMask = (H % 64 == 0) ? ~0ull : ((1ull << (H % 64)) - 1ull);
};

// Free-cell masks of the rows owned by this lane (0 for rows >= W).
template <int H, int R>
__device__ __forceinline__ void load_free_rows(const uint32_t* __restrict__ env_bits, int W,
                                               uint64_t (&fr)[R][RowWords<H>::HW]) {
    constexpr int HW = RowWords<H>::HW;
    const int lane = threadIdx.x & (kWave - 1);
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int x = lane + kWave * r;
#pragma unroll
        for (int k = 0; k < HW; ++k) {
            uint64_t v = 0;
            if (x < W) {
                const uint32_t* row = env_bits + (size_t)x * (H / 32);
                if (H == 32) {
                    v = (uint64_t)(~row[0]) & 0xFFFFFFFFull;
                } else {
                    const uint64_t lo = row[2 * k], hi = row[2 * k + 1];
                    v = ~(lo | (hi << 32));
                }
                if (k == HW - 1) v &= RowWords<H>::kLastMask;
            }
            fr[r][k] = v;
        }
    }
}

// Runs the BFS from (gx, gy) (which must be inside the map; it is visited
// even when it is an obstacle, as the energy BFS does) and writes
// dist[x*H+y] = level for every reached cell except the start, for levels
// 1..cap.  dist must already hold the "unreached" value and the start cell
// its 0.  Returns the sum over levels of max(0, level_size - 4096) when
// kCountOverflow (the nodes the reference's 4096-entry frontier would drop).
template <int H, int R, typename T, bool kCountOverflow>
__device__ int wave_bfs(const uint64_t (&fr)[R][RowWords<H>::HW], int gx, int gy, int cap,
                        T* dist) {
    constexpr int HW = RowWords<H>::HW;
    const int lane = threadIdx.x & (kWave - 1);
    uint64_t front[R][HW];
    uint64_t vis[R][HW];
#pragma unroll
    for (int r = 0; r < R; ++r) {
#pragma unroll
        for (int k = 0; k < HW; ++k) {
            front[r][k] = 0;
            vis[r][k] = 0;
        }
    }
    {
        const int owner_lane = gx & (kWave - 1);
        const int owner_r = gx / kWave;
        const uint64_t bit = 1ull << (gy & 63);
#pragma unroll
        for (int r = 0; r < R; ++r) {
#pragma unroll
            for (int k = 0; k < HW; ++k) {
                if (lane == owner_lane && r == owner_r && k == (gy >> 6)) {
                    front[r][k] = bit;
                    vis[r][k] = bit;
                }
            }
        }
    }
    int overflow = 0;
    for (int level = 1; level <= cap; ++level) {
        uint64_t nf[R][HW];
        bool any_new = false;
#pragma unroll
        for (int r = 0; r < R; ++r) {
#pragma unroll
            for (int k = 0; k < HW; ++k) {
                // vertical neighbours: row x-1 and x+1 of the same column word
                uint64_t up = from_lane_below(front[r][k]);
                uint64_t down = from_lane_above(front[r][k]);
                if (r > 0) {
                    const uint64_t wrap = lane_value(front[r - 1][k], kWave - 1);
                    if (lane == 0) up = wrap;
                }
                if (r + 1 < R) {
                    const uint64_t wrap = lane_value(front[r + 1][k], 0);
                    if (lane == kWave - 1) down = wrap;
                }
                // horizontal neighbours inside the row (y+1: <<1, y-1: >>1)
                uint64_t left = front[r][k] << 1;
                uint64_t right = front[r][k] >> 1;
                if (k > 0) left |= front[r][k - 1] >> 63;
                if (k + 1 < HW) right |= front[r][k + 1] << 63;
                const uint64_t n = (left | right | up | down) & fr[r][k] & ~vis[r][k];
                nf[r][k] = n;
                any_new |= (n != 0);
            }
        }
        if (!__any(any_new)) break;
        int local = 0;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int x = lane + kWave * r;
#pragma unroll
            for (int k = 0; k < HW; ++k) {
                vis[r][k] |= nf[r][k];
                front[r][k] = nf[r][k];
                uint64_t m = nf[r][k];
                if (kCountOverflow) local += __popcll(m);
                // two new cells per pass, the lowest and the highest (the same
                // cell twice when one is left)
                T* row_dist = dist + x * H + k * 64;
                while (m) {
                    const int lo = __ffsll((unsigned long long)m) - 1;
                    const int hi = 63 - __clzll((long long)m);
                    row_dist[lo] = (T)level;
                    row_dist[hi] = (T)level;
                    m &= ~((1ull << lo) | (1ull << hi));
                }
            }
        }
        // a level of more than kMaxFrontier = 64 * 64 cells has a lane with
        // more than 64 of them, so the sum is only needed then
        if (kCountOverflow && __any(local > kMaxFrontier / kWave)) {
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) local += __shfl_xor(local, off, kWave);
            if (local > kMaxFrontier) overflow += local - kMaxFrontier;
        }
    }
    return overflow;
}

}  // namespace jl
