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
// wave_shr:1 / wave_shl:1 on both halves, no LDS round trip; bound_ctrl
// writes the 0 of the lane without a source.  Every lane of the wavefront
// must be active.
__device__ __forceinline__ uint64_t from_lane_below(uint64_t v) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)v, 0x138, 0xF, 0xF, true);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(v >> 32), 0x138, 0xF, 0xF, true);
    return ((uint64_t)hi << 32) | lo;
}

__device__ __forceinline__ uint64_t from_lane_above(uint64_t v) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)v, 0x130, 0xF, 0xF, true);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(v >> 32), 0x130, 0xF, 0xF, true);
    return ((uint64_t)hi << 32) | lo;
}

// One level of a row held in 64 bits: the new frontier (the cells of `avail`
// that neighbour the frontier: `up` / `down` its rows of the lanes below
// and above, `left` / `right` its own row shifted by one column) is returned
// and removed from `avail`.  Per 32-bit half: a = up | right and
// b = down | left (a DPP lane move folded into each OR), then gfx950's
// three-input bit operation twice, (a | b) & avail (truth table 0xA8 with
// a, b, avail as its first, second and third input) and avail & ~(a | b)
// (0x02): four VALU instructions per half instead of the six of an OR3, an
// AND and an XOR after the two ORs.
__device__ __forceinline__ uint64_t level_step(uint64_t up, uint64_t down, uint64_t left, uint64_t right,
                                               uint64_t& avail) {
    const uint32_t a_lo = (uint32_t)up | (uint32_t)right, a_hi = (uint32_t)(up >> 32) | (uint32_t)(right >> 32);
    const uint32_t b_lo = (uint32_t)down | (uint32_t)left, b_hi = (uint32_t)(down >> 32) | (uint32_t)(left >> 32);
    const uint32_t v_lo = (uint32_t)avail, v_hi = (uint32_t)(avail >> 32);
    // (the builtin returns a signed int: each half is taken as uint32_t
    // before it is widened, so no sign bit reaches the high half)
    const uint32_t n_lo = (uint32_t)__builtin_amdgcn_bitop3_b32(a_lo, b_lo, v_lo, 0xA8);
    const uint32_t n_hi = (uint32_t)__builtin_amdgcn_bitop3_b32(a_hi, b_hi, v_hi, 0xA8);
    const uint32_t r_lo = (uint32_t)__builtin_amdgcn_bitop3_b32(a_lo, b_lo, v_lo, 0x02);
    const uint32_t r_hi = (uint32_t)__builtin_amdgcn_bitop3_b32(a_hi, b_hi, v_hi, 0x02);
    avail = ((uint64_t)r_hi << 32) | r_lo;
    return ((uint64_t)n_hi << 32) | n_lo;
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
                    // a row of H % 64 == 32 columns ends in half a word: its
                    // upper half is not read (it would be the next row's)
                    const uint64_t lo = row[2 * k];
                    const uint64_t hi = 2 * k + 1 < H / 32 ? row[2 * k + 1] : 0xFFFFFFFFu;
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
    uint64_t avail[R][HW];  // free cells not reached yet
#pragma unroll
    for (int r = 0; r < R; ++r) {
#pragma unroll
        for (int k = 0; k < HW; ++k) {
            front[r][k] = 0;
            avail[r][k] = fr[r][k];
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
                    avail[r][k] &= ~bit;
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
                const uint64_t n = level_step(up, down, left, right, avail[r][k]);
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

// wave_bfs for one row per lane (R = 1) without the frontier overflow count
// and without a level cap, in batches of 16 levels: the levels of a batch
// are unrolled into straight-line code (expansion, then the new cells ORed
// into the batch mask and into the planes of the level's 4 low bits, chosen
// at compile time), and only after the batch are its cells' distances
// L0 + (plane bits) written, one pass over the batch mask.  The search stops
// after the first batch whose last level reached no cell (levels past the
// last reach nothing, so the field is wave_bfs's).  The single wavefront's
// search is a chain of dependent instructions; the batch keeps the writes
// off that chain and lets the plane and mask updates fill its gaps.
template <int H, typename T>
__device__ void wave_bfs_batched(const uint64_t (&fr)[RowWords<H>::HW], int gx, int gy, T* dist) {
    constexpr int HW = RowWords<H>::HW;
    constexpr int kBatch = 16;
    const int lane = threadIdx.x & (kWave - 1);
    uint64_t front[HW], avail[HW];  // avail: free cells not reached yet
#pragma unroll
    for (int k = 0; k < HW; ++k) {
        front[k] = 0;
        avail[k] = fr[k];
        if (lane == gx && k == (gy >> 6)) {
            front[k] = 1ull << (gy & 63);
            avail[k] &= ~front[k];
        }
    }
    T* row_dist = dist + lane * H;
    for (int L0 = 1;; L0 += kBatch) {
        uint64_t bm[HW], p0[HW], p1[HW], p2[HW], p3[HW];
#pragma unroll
        for (int k = 0; k < HW; ++k) bm[k] = p0[k] = p1[k] = p2[k] = p3[k] = 0;
#pragma unroll
        for (int j = 0; j < kBatch; ++j) {
            uint64_t nf[HW];
#pragma unroll
            for (int k = 0; k < HW; ++k) {
                const uint64_t up = from_lane_below(front[k]);
                const uint64_t down = from_lane_above(front[k]);
                uint64_t left = front[k] << 1;
                uint64_t right = front[k] >> 1;
                if (k > 0) left |= front[k - 1] >> 63;
                if (k + 1 < HW) right |= front[k + 1] << 63;
                nf[k] = level_step(up, down, left, right, avail[k]);
            }
#pragma unroll
            for (int k = 0; k < HW; ++k) {
                front[k] = nf[k];
                bm[k] |= nf[k];
                if (j & 1) p0[k] |= nf[k];
                if (j & 2) p1[k] |= nf[k];
                if (j & 4) p2[k] |= nf[k];
                if (j & 8) p3[k] |= nf[k];
            }
        }
#pragma unroll
        for (int k = 0; k < HW; ++k) {
            uint64_t m = bm[k];
            while (m) {
                const int c = __ffsll((unsigned long long)m) - 1;
                const uint32_t j = (uint32_t)((p0[k] >> c) & 1u) | (uint32_t)((p1[k] >> c) & 1u) << 1 |
                                   (uint32_t)((p2[k] >> c) & 1u) << 2 | (uint32_t)((p3[k] >> c) & 1u) << 3;
                row_dist[k * 64 + c] = (T)(L0 + (int)j);
                m &= m - 1;
            }
        }
        bool more = false;
#pragma unroll
        for (int k = 0; k < HW; ++k) more |= front[k] != 0;
        if (!__any(more)) break;
    }
}

// Planes of the levels of a search on a map of at most 4,096 cells (levels
// stay below 4,096): four low planes in registers, eight high ones in LDS.
constexpr int kFieldPlanes = 12;
constexpr int kHighPlanes = kFieldPlanes - 4;
// LDS of one wavefront's high planes: [plane][lane] 64-bit words.
constexpr int kHighPlaneBytes = kHighPlanes * kWave * 8;

// wave_bfs_batched without a distance array: the level of every reached cell
// of this lane's row is left bit-sliced, bits 0-3 in lowp (lowp[b] bit y =
// bit b of the level of cell (lane, y)) and bits 4-11 in s_high[b - 4][lane]
// (this wavefront's kHighPlaneBytes of LDS), and the reached cells in vis
// (the start included, at level 0).  One wavefront, one map row per lane,
// rows of at most 64 columns.  Batch b runs levels 16 b + 1 .. 16 b + 16
// unrolled; with a[j] the free cells not reached before batch level j, the
// cells of level 16 b + 1 + j are a[j] ^ a[j + 1], so the low level bits of
// the batch come from a few of those snapshots (bit 1: levels 16 b + 2, 3,
// 6, 7, 10, 11, 14, 15 = (a1 ^ a3) | (a5 ^ a7) | (a9 ^ a11) | (a13 ^ a15);
// bit 2: (a3 ^ a7) | (a11 ^ a15); bit 3: a7 ^ a15), the high bits are b for
// a0 ^ a15 and b + 1 for a15 ^ a16 (level 16 b + 16), ORed into the LDS
// planes by LDS atomics once per batch, and bit 0 is no work at all: a grid
// is bipartite, so a level's parity is that of the Manhattan distance,
// x + y + gx + gy.  Per level only the expansion and the update of the free
// cells remain.  The search stops after the first batch whose last level
// reached nothing (levels past the last reach nothing).
template <int H>
__device__ void wave_bfs_levels(uint64_t fr, int gx, int gy, uint64_t& vis, uint64_t (&lowp)[4],
                                uint64_t* s_high) {
    static_assert(RowWords<H>::HW == 1, "one 64-bit word per row");
    const int lane = threadIdx.x & (kWave - 1);
    uint64_t front = lane == gx ? 1ull << gy : 0ull;
    uint64_t avail = fr & ~front;
#pragma unroll
    for (int p = 0; p < 4; ++p) lowp[p] = 0;
#pragma unroll
    for (int p = 0; p < kHighPlanes; ++p) s_high[p * kWave + lane] = 0;
    for (int b = 0;; ++b) {
        // snapshots are folded into the planes as soon as their partner
        // exists, so that few of them are live at once
        const uint64_t a0 = avail;
        uint64_t s1 = 0, s3 = 0, s5 = 0, s7 = 0, s9 = 0, s11 = 0, s13 = 0, most = 0, last = 0;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            front = level_step(from_lane_below(front), from_lane_above(front), front << 1, front >> 1, avail);
            switch (j + 1) {  // avail is now a[j + 1]
                case 1: s1 = avail; break;
                case 3: lowp[1] |= s1 ^ avail; s3 = avail; break;
                case 5: s5 = avail; break;
                case 7: lowp[1] |= s5 ^ avail; lowp[2] |= s3 ^ avail; s7 = avail; break;
                case 9: s9 = avail; break;
                case 11: lowp[1] |= s9 ^ avail; s11 = avail; break;
                case 13: s13 = avail; break;
                case 15:
                    lowp[1] |= s13 ^ avail;
                    lowp[2] |= s11 ^ avail;
                    lowp[3] |= s7 ^ avail;
                    most = a0 ^ avail;
                    last = avail;
                    break;
                case 16: last ^= avail; break;
                default: break;
            }
        }
        const int hb = __builtin_amdgcn_readfirstlane(b), hn = hb + 1;
#pragma unroll
        for (int k = 0; k < kHighPlanes; ++k) {
            const uint64_t m = (((hb >> k) & 1) ? most : 0ull) | (((hn >> k) & 1) ? last : 0ull);
            if (((hb | hn) >> k) & 1) atomicOr(reinterpret_cast<unsigned long long*>(s_high + k * kWave + lane), m);
        }
        if (!__any(front != 0)) break;
    }
    vis = fr & ~avail;
    const uint64_t odd_cols = ((lane + gx + gy) & 1) ? 0x5555555555555555ull : 0xAAAAAAAAAAAAAAAAull;
    lowp[0] = vis & odd_cols;
}

// Free-cell masks of map row x (0 for x >= W), for the group BFS.
template <int H>
__device__ __forceinline__ void load_free_row(const uint32_t* __restrict__ env_bits, int W, int x,
                                              uint64_t (&fr)[RowWords<H>::HW]) {
    constexpr int HW = RowWords<H>::HW;
#pragma unroll
    for (int k = 0; k < HW; ++k) {
        uint64_t v = 0;
        if (x < W) {
            const uint32_t* row = env_bits + (size_t)x * (H / 32);
            if (H == 32) {
                v = (uint64_t)(~row[0]) & 0xFFFFFFFFull;
            } else {
                const uint64_t hi = 2 * k + 1 < H / 32 ? row[2 * k + 1] : 0xFFFFFFFFu;  // half a word (H % 64 == 32)
                v = ~((uint64_t)row[2 * k] | (hi << 32));
            }
            if (k == HW - 1) v &= RowWords<H>::kLastMask;
        }
        fr[k] = v;
    }
}

// LDS words the group BFS needs besides the distance array (64-bit words):
// the boundary rows [2 parities][R wavefronts][top, bottom][HW], then the
// per-wavefront flags [2][R] and counts [R] (one word each).
template <int H, int R>
__host__ __device__ constexpr int group_bfs_words() {
    return 2 * R * 2 * RowWords<H>::HW + 2 * R + R;
}

// wave_bfs over a workgroup of R wavefronts (R > 1; every wavefront of the
// workgroup calls it with the same arguments and all lanes active):
// wavefront w owns map rows x = 64 w + lane, each held as HW 64-bit masks
// (fr: this lane's row).  A level is wave_bfs's on the wavefront's rows; the
// frontier rows at a wavefront boundary (64 w - 1 and 64 w + 64) travel
// through LDS, written at the end of the level before and read by this one,
// in slots alternating with the level's parity, with one workgroup barrier
// per level.  Each wavefront publishes with its boundary rows whether it
// found a new cell, and every wavefront stops at the first level at which
// none did.  The frontier overflow count needs the level's total over the
// workgroup, taken (with a second barrier) only at levels where some row
// holds more than kMaxFrontier / (64 R) new cells, as a level of more than
// kMaxFrontier cells must have one.  Same result as wave_bfs with R rows per
// lane.
template <int H, int R, typename T, bool kCountOverflow>
__device__ int group_bfs(const uint64_t (&fr)[RowWords<H>::HW], int gx, int gy, int cap, T* dist,
                         uint64_t* s_words) {
    constexpr int HW = RowWords<H>::HW;
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x / kWave));
    const int x = wave * kWave + lane;
    uint64_t* s_edge = s_words;                                      // [2][R][2][HW]
    int* s_flag = reinterpret_cast<int*>(s_words + 2 * R * 2 * HW);  // [2][R], one word apart
    int* s_count = s_flag + 2 * 2 * R;                               // [R]
    uint64_t front[HW], vis[HW];
#pragma unroll
    for (int k = 0; k < HW; ++k) {
        front[k] = 0;
        vis[k] = 0;
    }
    if (x == gx) {
#pragma unroll
        for (int k = 0; k < HW; ++k) {
            if (k == (gy >> 6)) {
                front[k] = 1ull << (gy & 63);
                vis[k] = front[k];
            }
        }
    }
    // boundary rows of slot `slot`: lane 0 stores the top row, lane 63 the bottom one
    auto publish = [&](int slot, const uint64_t (&f)[HW], int flag) {
        uint64_t* e = s_edge + (size_t)((slot * R + wave) * 2) * HW;
        if (lane == 0) {
#pragma unroll
            for (int k = 0; k < HW; ++k) e[k] = f[k];
            s_flag[2 * (slot * R + wave)] = flag;
        }
        if (lane == kWave - 1) {
#pragma unroll
            for (int k = 0; k < HW; ++k) e[HW + k] = f[k];
        }
    };
    publish(1, front, 1);  // level 1 reads the start's rows from slot 1
    __syncthreads();
    constexpr int kBigRow = kMaxFrontier / (kWave * R);
    int overflow = 0;
    for (int level = 1; level <= cap; ++level) {
        const int rd = level & 1, wr = rd ^ 1;
        uint64_t nf[HW];
        bool any_new = false;
        int local = 0;
#pragma unroll
        for (int k = 0; k < HW; ++k) {
            uint64_t up = from_lane_below(front[k]);
            uint64_t down = from_lane_above(front[k]);
            if (lane == 0 && wave > 0) up = s_edge[(size_t)((rd * R + wave - 1) * 2 + 1) * HW + k];
            if (lane == kWave - 1 && wave + 1 < R) down = s_edge[(size_t)((rd * R + wave + 1) * 2) * HW + k];
            uint64_t left = front[k] << 1;
            uint64_t right = front[k] >> 1;
            if (k > 0) left |= front[k - 1] >> 63;
            if (k + 1 < HW) right |= front[k + 1] << 63;
            const uint64_t n = (left | right | up | down) & fr[k] & ~vis[k];
            nf[k] = n;
            any_new |= (n != 0);
            if (kCountOverflow) local += __popcll(n);
        }
        const bool wave_new = __any(any_new);
        const bool big = kCountOverflow && __any(local > kBigRow);
        publish(wr, nf, (wave_new ? 1 : 0) | (big ? 2 : 0));
#pragma unroll
        for (int k = 0; k < HW; ++k) {
            vis[k] |= nf[k];
            front[k] = nf[k];
            uint64_t m = nf[k];
            T* row_dist = dist + x * H + k * 64;
            while (m) {
                const int lo = __ffsll((unsigned long long)m) - 1;
                const int hi = 63 - __clzll((long long)m);
                row_dist[lo] = (T)level;
                row_dist[hi] = (T)level;
                m &= ~((1ull << lo) | (1ull << hi));
            }
        }
        __syncthreads();
        int flags = 0;
#pragma unroll
        for (int w = 0; w < R; ++w) flags |= s_flag[2 * (wr * R + w)];
        flags = __builtin_amdgcn_readfirstlane(flags);
        if (kCountOverflow && (flags & 2)) {
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) local += __shfl_xor(local, off, kWave);
            if (lane == 0) s_count[wave] = local;
            __syncthreads();
            int total = 0;
#pragma unroll
            for (int w = 0; w < R; ++w) total += s_count[w];
            total = __builtin_amdgcn_readfirstlane(total);
            if (total > kMaxFrontier) overflow += total - kMaxFrontier;
            __syncthreads();  // s_count is rewritten at a later level
        }
        if (!(flags & 1)) break;
    }
    return overflow;
}

// Bit-planes of BFS levels: a reached cell's level (below 2^kLevelPlanes)
// is held bit-sliced, plane b holding bit b of the levels of a row's cells.
constexpr int kLevelPlanes = 16;

// 8x8 bit-matrix transpose: bit c of byte b moves to bit b of byte c.
__device__ __forceinline__ uint64_t transpose8x8(uint64_t x) {
    uint64_t t = (x ^ (x >> 7)) & 0x00AA00AA00AA00AAull;
    x = x ^ t ^ (t << 7);
    t = (x ^ (x >> 14)) & 0x0000CCCC0000CCCCull;
    x = x ^ t ^ (t << 14);
    t = (x ^ (x >> 28)) & 0x00000000F0F0F0F0ull;
    x = x ^ t ^ (t << 28);
    return x;
}

// group_bfs keeping each reached cell's level in registers instead of an LDS
// distance array: at level L the new frontier is ORed into the planes of
// L's set bits, so no per-cell write happens during the search.  On return
// vis holds the reached cells of this lane's row (the start included, at
// level 0) and `top` the last level that reached a cell.  s_words as for
// group_bfs.
template <int H, int R, bool kCountOverflow>
__device__ int group_bfs_planes(const uint64_t (&fr)[RowWords<H>::HW], int gx, int gy,
                                uint64_t (&vis)[RowWords<H>::HW],
                                uint64_t (&pl)[kLevelPlanes][RowWords<H>::HW], int& top, uint64_t* s_words) {
    constexpr int HW = RowWords<H>::HW;
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x / kWave));
    const int x = wave * kWave + lane;
    uint64_t* s_edge = s_words;
    int* s_flag = reinterpret_cast<int*>(s_words + 2 * R * 2 * HW);
    int* s_count = s_flag + 2 * 2 * R;
    uint64_t front[HW], avail[HW];  // avail: free cells not reached yet
#pragma unroll
    for (int k = 0; k < HW; ++k) {
        front[k] = 0;
        avail[k] = fr[k];
#pragma unroll
        for (int b = 0; b < kLevelPlanes; ++b) pl[b][k] = 0;
    }
    if (x == gx) {
#pragma unroll
        for (int k = 0; k < HW; ++k) {
            if (k == (gy >> 6)) {
                front[k] = 1ull << (gy & 63);
                avail[k] &= ~front[k];
            }
        }
    }
#pragma unroll
    for (int k = 0; k < HW; ++k) vis[k] = front[k];  // the start, obstacle or not
    auto publish = [&](int slot, const uint64_t (&f)[HW], int flag) {
        uint64_t* e = s_edge + (size_t)((slot * R + wave) * 2) * HW;
        if (lane == 0) {
#pragma unroll
            for (int k = 0; k < HW; ++k) e[k] = f[k];
            s_flag[2 * (slot * R + wave)] = flag;
        }
        if (lane == kWave - 1) {
#pragma unroll
            for (int k = 0; k < HW; ++k) e[HW + k] = f[k];
        }
    };
    publish(1, front, 1);
    __syncthreads();
    constexpr int kBigRow = kMaxFrontier / (kWave * R);
    constexpr int kCap = (1 << kLevelPlanes) - 2;  // levels stay below the unreachable value
    int overflow = 0;
    top = 0;
    for (int level = 1; level <= kCap; ++level) {
        const int rd = level & 1, wr = rd ^ 1;
        uint64_t nf[HW];
        bool any_new = false;
        int local = 0;
#pragma unroll
        for (int k = 0; k < HW; ++k) {
            uint64_t up = from_lane_below(front[k]);
            uint64_t down = from_lane_above(front[k]);
            if (lane == 0 && wave > 0) up = s_edge[(size_t)((rd * R + wave - 1) * 2 + 1) * HW + k];
            if (lane == kWave - 1 && wave + 1 < R) down = s_edge[(size_t)((rd * R + wave + 1) * 2) * HW + k];
            uint64_t left = front[k] << 1;
            uint64_t right = front[k] >> 1;
            if (k > 0) left |= front[k - 1] >> 63;
            if (k + 1 < HW) right |= front[k + 1] << 63;
            const uint64_t n = level_step(up, down, left, right, avail[k]);
            nf[k] = n;
            any_new |= (n != 0);
            if (kCountOverflow) local += __popcll(n);
        }
        const bool wave_new = __any(any_new);
        const bool big = kCountOverflow && __any(local > kBigRow);
        publish(wr, nf, (wave_new ? 1 : 0) | (big ? 2 : 0));
#pragma unroll
        for (int k = 0; k < HW; ++k) front[k] = nf[k];
#pragma unroll
        for (int b = 0; b < kLevelPlanes; ++b) {
            if ((level >> b) & 1) {
#pragma unroll
                for (int k = 0; k < HW; ++k) pl[b][k] |= nf[k];
            }
        }
        __syncthreads();
        int flags = 0;
#pragma unroll
        for (int w = 0; w < R; ++w) flags |= s_flag[2 * (wr * R + w)];
        flags = __builtin_amdgcn_readfirstlane(flags);
        if (kCountOverflow && (flags & 2)) {
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) local += __shfl_xor(local, off, kWave);
            if (lane == 0) s_count[wave] = local;
            __syncthreads();
            int total = 0;
#pragma unroll
            for (int w = 0; w < R; ++w) total += s_count[w];
            total = __builtin_amdgcn_readfirstlane(total);
            if (total > kMaxFrontier) overflow += total - kMaxFrontier;
            __syncthreads();
        }
        if (!(flags & 1)) break;
        top = level;
    }
#pragma unroll
    for (int k = 0; k < HW; ++k) vis[k] |= fr[k] & ~avail[k];
    return overflow;
}

// Level of this lane's cell at column y from the planes (kUnreachable when
// the cell was not reached).
template <int H>
__device__ __forceinline__ uint32_t plane_level(const uint64_t (&vis)[RowWords<H>::HW],
                                                const uint64_t (&pl)[kLevelPlanes][RowWords<H>::HW], int y) {
    constexpr int HW = RowWords<H>::HW;
    uint32_t d = 0;
    bool reached = false;
#pragma unroll
    for (int k = 0; k < HW; ++k) {
        if (k == (y >> 6)) {
            const int bit = y & 63;
            reached = (vis[k] >> bit) & 1;
#pragma unroll
            for (int b = 0; b < kLevelPlanes; ++b) d |= (uint32_t)((pl[b][k] >> bit) & 1) << b;
        }
    }
    return reached ? d : kUnreachable;
}

}  // namespace jl
