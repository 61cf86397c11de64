// jl_common.h - shared definitions of the gfx950 kernels behind include/jointloom.h.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/jointloom.h"

namespace jl {

constexpr int kWave = 64;            // CDNA wavefront width
constexpr uint16_t kUnreachable = 0xFFFFu;
constexpr int kContext = 256;        // MAPF-GPT tokens per agent
constexpr int kRadius = 5;
constexpr int kDiam = 11;
constexpr int kCostTokens = 121;
constexpr int kVisible = 13;
constexpr int kAgentTokens = 10;
constexpr int kCostLimit = 20;
constexpr int kTokUnreachable = 41;
constexpr int kTokNegClip = 42;
constexpr int kTokPosClip = 43;
constexpr int kTokEmptyAction = 44;
constexpr int kTokWait = 45;
constexpr int kTokGreedy = 50;
constexpr int kTokPad = 66;
constexpr int kMaxFrontier = 4096;   // reference BFS frontier capacity (diagnostics[0])
constexpr int kPygDiam = 13;
constexpr int kPygArea = 169;
constexpr int kPygFeatures = 4 * kPygArea;
constexpr int kCommRadiusSq = 49;

// Squared distance as the reference's 32-bit int arithmetic yields it for
// any int16 positions: products and sum wrap modulo 2^32 (done in unsigned,
// where the wrap is defined), so two agents near opposite int16 extremes can
// test as neighbours there too (stateless_step.cu:513-520, :889).
__device__ __forceinline__ int wrap_dist2(int dx, int dy) {
    return (int)((uint32_t)dx * (uint32_t)dx + (uint32_t)dy * (uint32_t)dy);
}

// Scratch layout of jl_mapfgpt_t::scratch: diagnostics accumulated by a
// build, then published by the last workgroup of the token kernel.
constexpr int kScratchAccum = 0;     // [0..3]
constexpr int kScratchTicket = 4;

// The builder's tiled copies of the distance fields (cost_tiles) of maps of
// at most 4096 cells carry each reachable cell's greedy-move mask in bits
// 12-15: a distance there is below 4095 (at most the number of free cells
// minus one, and a map with every cell free has a far smaller diameter), so
// it fits in bits 0-11 and a marked value never equals kUnreachable, which
// unreachable cells keep.  Readers take the distance as field_distance(v,
// field_mask(W, H)).  cost_to_go, the API tensor, holds plain distances.
constexpr int kMarkedCells = 4096;
__host__ __device__ inline bool marked_fields(int W, int H) { return W * H <= kMarkedCells; }
__host__ __device__ inline uint32_t field_mask(int W, int H) {
    return marked_fields(W, H) ? 0x0FFFu : 0xFFFFu;
}
__device__ __forceinline__ uint32_t field_distance(uint32_t v, uint32_t mask) {
    return v == kUnreachable ? v : (v & mask);
}

// The builder's tiled copies of the distance fields (cost_tiles): 8x8 tiles
// of uint16 (128 bytes, one cache line each) over a grid of
// TR = ceil(W/8) + 2 tile rows by H/8 + 2 tile columns, stored column-major:
// the tiles of one 8-cell column strip are consecutive, so the strip's
// 16-byte rows (8 cells each) follow one another for x = -8 .. 8 * TR - 9 and
// a window's row segments lie at offsets linear in the row.  The outer ring
// of tiles is a border of unreachable cells (set at allocation, never
// written), so a window of radius 5 around any cell of the map reads whole
// tile rows without clamping; tile (1, 1) holds cells (0..7, 0..7).  Rows
// past W inside the last tile row of the map are unreachable as well.
__host__ __device__ inline int tile_grid_rows(int W) { return (W + 7) / 8 + 2; }
__host__ __device__ inline int tile_grid_cols(int H) { return H / 8 + 2; }
__host__ __device__ inline size_t tiled_cells(int W, int H) {
    return (size_t)tile_grid_rows(W) * tile_grid_cols(H) * 64;
}
// Cells of one column strip (its TR tiles).
__host__ __device__ inline uint32_t strip_cells(int W) { return (uint32_t)tile_grid_rows(W) * 64u; }
// Offset of cell (x, y) in a tiled field, for -8 <= x < W + 8, -8 <= y < H + 8.
__device__ __forceinline__ uint32_t tile_offset(int x, int y, int W) {
    return (uint32_t)((y >> 3) + 1) * strip_cells(W) + (uint32_t)(x + 8) * 8u + (uint32_t)(y & 7);
}

// Map profiles: H a multiple of 32 (whole bitmap words per row, as
// setup.py:34-38 requires) up to 256, 1 <= W <= 256.
inline bool profile_ok(int w, int h) {
    return h >= 32 && h <= 256 && h % 32 == 0 && w >= 1 && w <= 256;
}

inline int status(hipError_t e) { return e == hipSuccess ? JL_OK : (int)e; }

inline int launch_status() { return status(hipGetLastError()); }

// Sum of the four bytes of a word.
__device__ __forceinline__ uint32_t byte_sum(uint32_t w) {
    return (w & 0xFFu) + ((w >> 8) & 0xFFu) + ((w >> 16) & 0xFFu) + (w >> 24);
}

// Compute units of the current device (grids of looping kernels are sized to them).
inline int device_cus() {
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 256;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        return 256;
    return cus > 0 ? cus : 256;
}

// Map-profile dispatch on the column count H (a compile-time divisor).
// LDS of a gfx950 CU, the most one workgroup can hold: a launch's dynamic
// LDS plus the kernel's static LDS must fit in it.
constexpr size_t kLdsBytes = 160 * 1024;

// A kernel's static LDS (its __shared__ variables and what the compiler adds,
// such as the reduction buffer behind __syncthreads_and), looked up once per
// kernel; taken as 1 KB if the lookup fails.
template <auto Kernel>
inline size_t static_lds() {
    static const size_t bytes = [] {
        hipFuncAttributes a;
        return hipFuncGetAttributes(&a, reinterpret_cast<const void*>(Kernel)) == hipSuccess
                   ? (size_t)a.sharedSizeBytes
                   : (size_t)1024;
    }();
    return bytes;
}

// Whether `dynamic` bytes of LDS fit beside the kernel's own.
template <auto Kernel>
inline bool lds_fits(size_t dynamic) {
    return dynamic + static_lds<Kernel>() <= kLdsBytes;
}

#define JL_DISPATCH_H(h, ...)                                   \
    switch (h) {                                               \
        case 32: { constexpr int H = 32; __VA_ARGS__; break; } \
        case 64: { constexpr int H = 64; __VA_ARGS__; break; } \
        case 96: { constexpr int H = 96; __VA_ARGS__; break; } \
        case 128: { constexpr int H = 128; __VA_ARGS__; break; } \
        case 160: { constexpr int H = 160; __VA_ARGS__; break; } \
        case 192: { constexpr int H = 192; __VA_ARGS__; break; } \
        case 224: { constexpr int H = 224; __VA_ARGS__; break; } \
        case 256: { constexpr int H = 256; __VA_ARGS__; break; } \
        default: return JL_ERR_PROFILE;                        \
    }

__device__ __forceinline__ bool bit_at(const uint32_t* bits, int cell) {
    return (bits[cell >> 5] >> (cell & 31)) & 1u;
}

// Orders one wavefront's LDS accesses around this point: the compiler keeps
// LDS reads and writes on their side of it, and since a wavefront's LDS
// operations execute in issue order, writes made before it by any lane of
// the wavefront are seen by reads after it.
__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Workgroup barrier that orders LDS only: LDS writes before it are seen by
// LDS reads after it in every wavefront of the workgroup, while outstanding
// global loads and stores stay in flight (__syncthreads() also waits for
// those, which would drain a prefetch issued before the barrier).
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// 64-bit cross-lane read (ds_bpermute); lanes outside [0,64) wrap.
__device__ __forceinline__ uint64_t shfl64(uint64_t v, int src_lane) {
    const int lo = __shfl((int)(uint32_t)v, src_lane, kWave);
    const int hi = __shfl((int)(uint32_t)(v >> 32), src_lane, kWave);
    return ((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo;
}

__device__ __forceinline__ int coord_token(int v) {
    v = v < -kCostLimit ? -kCostLimit : v;
    v = v > kCostLimit ? kCostLimit : v;
    return v + kCostLimit;
}

__device__ __forceinline__ int cost_token(uint32_t v, uint32_t center) {
    if (v == kUnreachable) return kTokUnreachable;
    const int d = (int)v - (int)center;
    if (d > kCostLimit) return kTokPosClip;
    if (d < -kCostLimit) return kTokNegClip;
    return d + kCostLimit;
}

// Host address of the builder's history-append kernel (jl_mapfgpt.hip), by
// which jl_graph_retarget_actions (jl_sim.hip) finds its nodes in a graph.
const void* append_actions_kernel_address();

}  // namespace jl
