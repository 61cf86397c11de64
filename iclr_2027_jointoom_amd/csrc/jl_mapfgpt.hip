// jl_mapfgpt.hip - MAPF-GPT observation builder for gfx950.
//
// On maps of at most 4096 cells with at most 1024 agents per env an eager
// build is one launch of the token kernel, one workgroup per env: its phase 0
// unpacks the env's agents and refreshes their changed fields (the work of
// 1a and 1b below), then phases 1 and 2 follow.  Otherwise a build is three
// launches (two on maps of up to 4096 cells, where 1a and 1b are one kernel):
//   1a. unpack: one lane per agent, no LDS.  Unpacks the state (raw rows or
//      resident split arrays), refreshes the goal cache and writes every
//      agent's info word: the greedy-move mask from the kept tiled field, or a
//      mark when the reset flag is set.  It also clears `diagnostics`.
//   1b. bfs: a grid sized to the CUs; each wavefront scans a range of info
//      words and runs the bit-parallel BFS (jl_bfs.h) for the marked agents
//      in its own LDS field, stores it in 8x8 tiles (cost_tiles; the API
//      tensor cost_to_go is filled from them on request) and completes the
//      info word.
//   2. tokens: one 1024-thread workgroup per env (per 512 egos of a larger
//      env).  Phase 1
//      stages the env's agents (position, goal, the six ego-independent
//      tokens) and a cell -> agent map in LDS and sums the env's diagnostics.
//      Phase 2: every wavefront on its own gathers the 11x11 windows of its
//      next ego pair from the tiled fields while it turns the current pair
//      into tokens (visible agents ranked with ballots), each row assembled
//      in LDS and written as 64 x 16-byte stores.
// The reference runs four kernels plus a 16 KB/env memset per build
// (mapf_gpt_builder.cpp:108-110, mapf_gpt_cuda.cu:544-610) with the
// top-13 search done serially by one lane per ego (:395-496) and every
// window row read from the row-major field (one 128-byte line per row).

#include <mutex>

#include "jl_bfs.h"
#include "jl_common.h"

namespace jl {
namespace {

constexpr uint32_t kNoAgent = 0xFFFFFFFFu;

// agent_info word, written for every agent by pass 1, read by pass 2.
constexpr uint32_t kInfoGreedy = 0xFu;        // greedy-move mask
constexpr uint32_t kInfoBadRow = 1u << 4;     // raw row rejected (diagnostics[1])
constexpr uint32_t kInfoBadGoal = 1u << 5;    // refresh with goal off map / on obstacle ([3])
constexpr int kInfoOverflowShift = 8;         // BFS frontier overflow count ([0]), 24 bits

// Greedy-move mask of one agent (mapf_gpt_cuda.cu:459-480): bit (3 - dir)
// is set when the neighbour in direction dir, order (-1,0), (+1,0), (0,-1),
// (0,+1), is reachable and strictly closer to the goal than the agent's cell.
// The five reads are issued unconditionally (a neighbour off the map reads a
// clamped cell and is then taken as unreachable), so a field in HBM costs one
// round trip, not one per branch.
template <int H, typename Field>
__device__ __forceinline__ uint32_t greedy_mask(Field f, int x, int y, int W) {
    const uint32_t c0 = f(x, y);
    const uint32_t r0 = f(x > 0 ? x - 1 : x, y);
    const uint32_t r1 = f(x + 1 < W ? x + 1 : x, y);
    const uint32_t r2 = f(x, y > 0 ? y - 1 : y);
    const uint32_t r3 = f(x, y + 1 < H ? y + 1 : y);
    const uint32_t n0 = x > 0 ? r0 : kUnreachable;
    const uint32_t n1 = x + 1 < W ? r1 : kUnreachable;
    const uint32_t n2 = y > 0 ? r2 : kUnreachable;
    const uint32_t n3 = y + 1 < H ? r3 : kUnreachable;
    uint32_t m = 0;
    if (n0 != kUnreachable && c0 > n0) m |= 8u;
    if (n1 != kUnreachable && c0 > n1) m |= 4u;
    if (n2 != kUnreachable && c0 > n2) m |= 2u;
    if (n3 != kUnreachable && c0 > n3) m |= 1u;
    return m;
}

// One 8-cell tile row (x, y0 .. y0 + 7) of a field in LDS (row-major, H
// columns, x < W), every reachable cell marked in bits 12-15 with its
// greedy-move mask (greedy_mask's rule: a neighbour off the map or
// unreachable is never closer, since a reachable distance is below
// kUnreachable).
template <int H>
__device__ __forceinline__ uint4 marked_segment(const uint16_t* f, int W, int x, int y0) {
    const uint4* f4 = reinterpret_cast<const uint4*>(f);
    constexpr uint32_t kNone = 0xFFFFFFFFu;
    const uint4 mid = f4[(x * H + y0) >> 3];
    const uint4 up = x > 0 ? f4[((x - 1) * H + y0) >> 3] : make_uint4(kNone, kNone, kNone, kNone);
    const uint4 dn = x + 1 < W ? f4[((x + 1) * H + y0) >> 3] : make_uint4(kNone, kNone, kNone, kNone);
    const uint32_t left = y0 > 0 ? f[x * H + y0 - 1] : kUnreachable;
    const uint32_t right = y0 + 8 < H ? f[x * H + y0 + 8] : kUnreachable;
    const uint32_t cw[4] = {mid.x, mid.y, mid.z, mid.w};
    const uint32_t uw[4] = {up.x, up.y, up.z, up.w};
    const uint32_t dw[4] = {dn.x, dn.y, dn.z, dn.w};
    uint32_t c[8], u[8], d[8];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        c[2 * k] = cw[k] & 0xFFFFu;
        c[2 * k + 1] = cw[k] >> 16;
        u[2 * k] = uw[k] & 0xFFFFu;
        u[2 * k + 1] = uw[k] >> 16;
        d[2 * k] = dw[k] & 0xFFFFu;
        d[2 * k + 1] = dw[k] >> 16;
    }
    uint32_t o[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const uint32_t v = c[k];
        const uint32_t l = k > 0 ? c[k - 1] : left;
        const uint32_t r = k < 7 ? c[k + 1] : right;
        const uint32_t m = (v > u[k] ? 8u : 0u) | (v > d[k] ? 4u : 0u) | (v > l ? 2u : 0u) | (v > r ? 1u : 0u);
        o[k] = v == kUnreachable ? v : (v | (m << 12));
    }
    return make_uint4(o[0] | (o[1] << 16), o[2] | (o[3] << 16), o[4] | (o[5] << 16), o[6] | (o[7] << 16));
}

// ---------------------------------------------------------------------------
// Per-agent steps shared by the launches of a build.
// ---------------------------------------------------------------------------
constexpr uint32_t kInfoNeedsBfs = 1u << 6;  // agent_info: field to refresh in pass 1b

__device__ __forceinline__ uint4 state_row(uint32_t env, uint32_t agent, uint32_t px, uint32_t py,
                                           uint32_t gx, uint32_t gy, uint32_t action,
                                           uint32_t reset) {
    return make_uint4((env & 0xFFFFu) | (agent << 16), (px & 0xFFFFu) | (py << 16),
                      (gx & 0xFFFFu) | (gy << 16), (action & 0xFFFFu) | (reset << 16));
}

// One agent's unpack: state row, goal cache, label and (raw rows) history.
// kRows: raw 13-column rows (mapf_gpt_unpack_kernel, mapf_gpt_cuda.cu:75-118);
// otherwise resident split arrays (mapf_gpt_state_unpack_kernel, :121-152).
// Returns the agent's state row as it now stands in state_packed (a
// rejected raw row keeps the old one, reset flag included, :90-92, :186-189)
// and sets info to kInfoBadRow for such a row, else 0.
template <bool kRows>
__device__ __forceinline__ uint4 unpack_agent(const jl_mapfgpt_t& b, int i,
                                              const int16_t* __restrict__ raw_rows,
                                              const int16_t* __restrict__ cur_x,
                                              const int16_t* __restrict__ cur_y,
                                              const int16_t* __restrict__ goal_x,
                                              const int16_t* __restrict__ goal_y, uint32_t& info) {
    const int A = b.n_agents;
    uint4* st = reinterpret_cast<uint4*>(b.state_packed + (size_t)i * 8);
    uint32_t* gc = reinterpret_cast<uint32_t*>(b.goal_cache + (size_t)i * 2);
    info = 0;
    if (kRows) {
        const uint16_t* row = reinterpret_cast<const uint16_t*>(raw_rows) + (size_t)i * 13;
        uint16_t c[13];
#pragma unroll
        for (int k = 0; k < 13; ++k) c[k] = row[k];
        if (c[0] >= b.n_envs || c[1] >= A || i != (int)c[0] * A + c[1]) {
            info = kInfoBadRow;
            return *st;
        }
        const uint32_t goal = (uint32_t)c[4] | ((uint32_t)c[5] << 16);
        const bool changed = *gc != goal;
        if (changed) *gc = goal;
        const uint4 v = state_row(c[0], c[1], c[2], c[3], c[4], c[5], c[6], (c[7] != 0 || changed) ? 1u : 0u);
        *st = v;
        uint16_t* h = b.histories + (size_t)i * 5;
#pragma unroll
        for (int k = 0; k < 5; ++k) h[k] = c[8 + k];
        b.labels[i] = (int64_t)c[6];
        return v;
    }
    const uint32_t env = (uint32_t)(i / A);
    const uint32_t agent = (uint32_t)(i - (int)env * A);
    const uint32_t tx = (uint16_t)goal_x[i], ty = (uint16_t)goal_y[i];
    const uint32_t goal = tx | (ty << 16);
    const bool changed = *gc != goal;
    if (changed) *gc = goal;
    const uint4 v = state_row(env, agent, (uint16_t)cur_x[i], (uint16_t)cur_y[i], tx, ty, 0u, changed ? 1u : 0u);
    *st = v;
    b.labels[i] = 0;
    return v;
}

// Greedy mask of an agent at (px, py) on the map whose field this build
// keeps, from the tiled copy written by an earlier build.  kMarked (maps of
// at most kMarkedCells cells): the mark of the agent's own cell, one read;
// an agent on an unreachable cell (an obstacle, or a component without its
// goal) and unmarked maps read the cross of five cells (1-3 lines).
template <int H, bool kMarked>
__device__ __forceinline__ uint32_t kept_greedy(const jl_mapfgpt_t& b, size_t i, int px, int py) {
    const int W = b.map_w;
    const uint16_t* f = b.cost_tiles + i * tiled_cells(W, H);
    if (kMarked) {
        const uint32_t c = f[tile_offset(px, py, W)];
        if (c != kUnreachable) return c >> 12;
    }
    return greedy_mask<H>([f, W](int x, int y) { return (uint32_t)f[tile_offset(x, y, W)]; }, px, py, W);
}

// Refresh of one agent's field (mapf_gpt_cost_to_go_kernel, :181-325) by the
// calling wavefront (every lane, wavefront-uniform arguments): the
// bit-parallel BFS (jl_bfs.h) from the goal (gx, gy) over env e's free cells
// in the wavefront's LDS field s_dist (W * H uint16), then the field in 8x8
// tiles into cost_tiles (with greedy marks when kMarked), 16-byte stores; the
// row-major cost_to_go is filled from the tiles on request.  Returns the
// agent's info bits: the frontier overflow count, or kInfoBadGoal for a goal
// off the map or on an obstacle (an all-unreachable field, :224-236), and the
// greedy mask at its position (spx, spy) when that is on the map.
// The map's tiles of the LDS field s_dist (W * H uint16, with greedy marks
// when kMarked) into agent agent_index's tiled field, 16-byte row segments
// first, first + stride, ... (the border ring keeps its unreachable cells).
template <int H, bool kMarked>
__device__ void store_field_tiles(const jl_mapfgpt_t& b, size_t agent_index, const uint16_t* s_dist,
                                  int first, int stride) {
    const int W = b.map_w;
    const uint4* lds4 = reinterpret_cast<const uint4*>(s_dist);
    uint4* tout = reinterpret_cast<uint4*>(b.cost_tiles + agent_index * tiled_cells(W, H));
    const int map_tile_rows = (W + 7) / 8;
    for (int c = first; c < map_tile_rows * H; c += stride) {
        const int t = c >> 3, r = c & 7;  // map tile, row inside the tile
        const int tr = t / (H / 8), tc = t - (t / (H / 8)) * (H / 8);
        const int x = tr * 8 + r, y0 = tc * 8;
        const int dst = (tc + 1) * (int)(strip_cells(W) / 8u) + x + 8;  // 16-byte row of strip tc + 1
        const bool in = x < W;  // rows past the map in the last tile row: unreachable
        uint4 v = kMarked ? marked_segment<H>(s_dist, W, in ? x : 0, y0) : lds4[((in ? x : 0) * H + y0) >> 3];
        v.x = in ? v.x : 0xFFFFFFFFu;
        v.y = in ? v.y : 0xFFFFFFFFu;
        v.z = in ? v.z : 0xFFFFFFFFu;
        v.w = in ? v.w : 0xFFFFFFFFu;
        tout[dst] = v;
    }
}

// refresh_field on a marked map of at most 64 rows of at most 64 columns,
// with no LDS field: wave_bfs_levels leaves every reached cell's level in
// bit planes (the high ones in s_high, this wavefront's kHighPlaneBytes of
// LDS); the greedy marks come from the two low planes without any
// comparison of distances (two reachable neighbours' levels differ by
// exactly one, the grid being bipartite, so a reachable neighbour is closer
// iff a0 ^ a1 ^ b1, with a0, a1 the cell's level bits 0-1 and b1 the
// neighbour's bit 1); and each lane turns its map row into the field's
// 8-cell tile-row segments, two 8x8 bit transposes per segment (level bits
// 0-7, then level bits 8-11 and the four mark bits), stored as 16-byte words
// (consecutive lanes, consecutive rows of a strip).  Same tiles and info
// bits as refresh_field<H, 1, true> (no level of such a map can overflow the
// frontier).  Every lane calls it with wavefront-uniform arguments.
template <int H>
__device__ uint32_t refresh_field_levels(const jl_mapfgpt_t& b, size_t agent_index, uint32_t e, int gx, int gy,
                                         int spx, int spy, uint64_t* s_high) {
    const int W = b.map_w;
    const int x = threadIdx.x & (kWave - 1);  // this lane's map row
    const int words = W * H / 32;
    bool ok = e < (uint32_t)b.n_envs && (uint32_t)gx < (uint32_t)W && (uint32_t)gy < (uint32_t)H;
    const uint32_t* env_bits = b.grid_bits + (size_t)(ok ? e : 0) * words;
    if (ok && bit_at(env_bits, gx * H + gy)) ok = false;
    uint64_t vis = 0, pl[4] = {0, 0, 0, 0};
    if (ok) {
        uint64_t fr[1][1];
        load_free_rows<H, 1>(env_bits, W, fr);
        wave_bfs_levels<H>(fr[0][0], gx, gy, vis, pl, s_high);
    } else {
#pragma unroll
        for (int p = 0; p < kHighPlanes; ++p) s_high[p * kWave + x] = 0;
    }
    // neighbours' reached cells aligned with this row's columns (off the
    // map: none), and the closer reachable neighbours
    const uint64_t v_up = from_lane_below(vis), v_dn = from_lane_above(vis);
    const uint64_t v_lf = vis << 1, v_rt = vis >> 1;
    const uint64_t a01 = pl[0] ^ pl[1];
    const uint64_t m_up = vis & v_up & (a01 ^ from_lane_below(pl[1]));
    const uint64_t m_dn = vis & v_dn & (a01 ^ from_lane_above(pl[1]));
    const uint64_t m_lf = vis & v_lf & (a01 ^ (pl[1] << 1));
    const uint64_t m_rt = vis & v_rt & (a01 ^ (pl[1] >> 1));
    uint32_t info = ok ? 0u : kInfoBadGoal;
    if ((uint32_t)spx < (uint32_t)W && (uint32_t)spy < (uint32_t)H) {
        // greedy_mask at (spx, spy): a reachable cell's closer neighbours;
        // an unreachable one is farther than each reachable neighbour
        const bool reached = (lane_value(vis, spx) >> spy) & 1;
        const uint64_t q0 = lane_value(reached ? m_up : v_up, spx), q1 = lane_value(reached ? m_dn : v_dn, spx);
        const uint64_t q2 = lane_value(reached ? m_lf : v_lf, spx), q3 = lane_value(reached ? m_rt : v_rt, spx);
        info |= (uint32_t)((q0 >> spy) & 1) << 3 | (uint32_t)((q1 >> spy) & 1) << 2 |
                (uint32_t)((q2 >> spy) & 1) << 1 | (uint32_t)((q3 >> spy) & 1);
    }
    // the 16 bits of every cell's tile value: level bits 0-11, then the
    // marks (bit 12 right, 13 left, 14 down, 15 up); every bit of an
    // unreachable cell set (its byte of ~vis ORed into all 16)
    if (x < (W + 7) / 8 * 8) {
        uint4* tout = reinterpret_cast<uint4*>(b.cost_tiles + agent_index * tiled_cells(W, H));
        const int strip_words = (int)(strip_cells(W) / 8u);
        const uint32_t* s_high32 = reinterpret_cast<const uint32_t*>(s_high);
#pragma unroll 1
        for (int half = 0; half < (H + 31) / 32; ++half) {
            // groups 4 half .. 4 half + 3: this 32-bit half of the high planes
            uint32_t hp[kHighPlanes];
#pragma unroll
            for (int p = 0; p < kHighPlanes; ++p) hp[p] = s_high32[(p * kWave + x) * 2 + half];
#pragma unroll 1
            for (int q = 0; q < 4; ++q) {
                const int k = 4 * half + q;  // segment: columns 8 k .. 8 k + 7
                const uint64_t unr = (uint64_t)((uint32_t)(~vis >> (8 * k)) & 0xFFu) * 0x0101010101010101ull;
                uint64_t lo = 0, hi = 0;
#pragma unroll
                for (int p = 0; p < 4; ++p) lo |= ((pl[p] >> (8 * k)) & 0xFFull) << (8 * p);
#pragma unroll
                for (int p = 0; p < 4; ++p) lo |= (uint64_t)((hp[p] >> (8 * q)) & 0xFFu) << (8 * (4 + p));
#pragma unroll
                for (int p = 0; p < 4; ++p) hi |= (uint64_t)((hp[4 + p] >> (8 * q)) & 0xFFu) << (8 * p);
                hi |= ((m_rt >> (8 * k)) & 0xFFull) << 32 | ((m_lf >> (8 * k)) & 0xFFull) << 40 |
                      ((m_dn >> (8 * k)) & 0xFFull) << 48 | ((m_up >> (8 * k)) & 0xFFull) << 56;
                lo = transpose8x8(lo | unr);  // byte c: bits 0-7 of cell 8 k + c
                hi = transpose8x8(hi | unr);  // byte c: bits 8-15
                uint32_t w[4];
#pragma unroll
                for (int c = 0; c < 8; c += 2) {
                    w[c / 2] = (uint32_t)((lo >> (8 * c)) & 0xFF) | (uint32_t)((hi >> (8 * c)) & 0xFF) << 8 |
                               (uint32_t)((lo >> (8 * c + 8)) & 0xFF) << 16 |
                               (uint32_t)((hi >> (8 * c + 8)) & 0xFF) << 24;
                }
                if (k < H / 8) tout[(k + 1) * strip_words + x + 8] = make_uint4(w[0], w[1], w[2], w[3]);
            }
        }
    }
    return info;
}

template <int H, int R, bool kMarked, bool kTiles = true>
__device__ uint32_t refresh_field(const jl_mapfgpt_t& b, size_t agent_index, uint32_t e, int gx,
                                  int gy, int spx, int spy, uint16_t* s_dist) {
    constexpr int HW = RowWords<H>::HW;
    if constexpr (R == 1 && HW == 1 && kMarked && kTiles) {
        // no LDS field on this path: the caller's s_dist (at least
        // kHighPlaneBytes, marked_wave_lds) holds the high level planes
        return refresh_field_levels<H>(b, agent_index, e, gx, gy, spx, spy, reinterpret_cast<uint64_t*>(s_dist));
    }
    const int W = b.map_w;
    const int lane = threadIdx.x & (kWave - 1);
    const int cells = W * H;
    const int words = cells / 32;
    {
        // W * H is a multiple of 8 cells (H >= 32): 16-byte stores
        const uint32_t u2 = (uint32_t)kUnreachable * 0x10001u;
        uint4* d4 = reinterpret_cast<uint4*>(s_dist);
        for (int c = lane; c < cells / 8; c += kWave) d4[c] = make_uint4(u2, u2, u2, u2);
    }
    wave_sync();
    bool ok = e < (uint32_t)b.n_envs && (uint32_t)gx < (uint32_t)W && (uint32_t)gy < (uint32_t)H;
    const uint32_t* env_bits = b.grid_bits + (size_t)(ok ? e : 0) * words;
    if (ok && bit_at(env_bits, gx * H + gy)) ok = false;
    int overflow = 0;
    if (ok) {
        uint64_t fr[R][HW];
        load_free_rows<H, R>(env_bits, W, fr);
        if (lane == 0) s_dist[gx * H + gy] = 0;
        wave_sync();
        if (W * H > kMaxFrontier + 1) {
            overflow = wave_bfs<H, R, uint16_t, true>(fr, gx, gy, 0x7FFFFFFF, s_dist);
        } else if constexpr (R == 1) {
            // no level of a map this small can overflow the frontier
            wave_bfs_batched<H, uint16_t>(fr[0], gx, gy, s_dist);
        } else {
            overflow = wave_bfs<H, R, uint16_t, false>(fr, gx, gy, 0x7FFFFFFF, s_dist);
        }
    }
    wave_sync();
    uint32_t info = ok ? (uint32_t)(overflow < 0xFFFFFF ? overflow : 0xFFFFFF) << kInfoOverflowShift
                       : kInfoBadGoal;
    if ((uint32_t)spx < (uint32_t)W && (uint32_t)spy < (uint32_t)H)
        info |= greedy_mask<H>([s_dist](int x, int y) { return (uint32_t)s_dist[x * H + y]; }, spx, spy, W);
    if (kTiles) {
        store_field_tiles<H, kMarked>(b, agent_index, s_dist, lane, kWave);
        wave_sync();  // the LDS field is rewritten by the next refresh
    }
    return info;
}

// refresh_field (unmarked fields) by a workgroup of R wavefronts on maps of
// more than 64 rows, without an LDS distance array: the group BFS with
// bit-sliced levels (jl_bfs.h, wavefront w on rows 64 w .. 64 w + 63), then
// every lane turns its row into 8-cell tile-row segments (one 8x8 bit
// transpose per 8 planes and segment) and stores them into the tiled field.
// The five cells of the greedy mask at (spx, spy) travel through s_gm.  Every
// thread calls it with the same arguments.  Same tiles and info bits as
// refresh_field.
template <int H, int R>
__device__ uint32_t refresh_field_group(const jl_mapfgpt_t& b, size_t agent_index, uint32_t e, int gx, int gy,
                                        int spx, int spy, uint64_t* s_words, uint32_t* s_gm) {
    constexpr int HW = RowWords<H>::HW;
    const int W = b.map_w;
    const int tid = threadIdx.x;
    const int x = tid;  // this lane's map row
    const int words = W * H / 32;
    const size_t tcells = tiled_cells(W, H);
    bool ok = e < (uint32_t)b.n_envs && (uint32_t)gx < (uint32_t)W && (uint32_t)gy < (uint32_t)H;
    const uint32_t* env_bits = b.grid_bits + (size_t)(ok ? e : 0) * words;
    if (ok && bit_at(env_bits, gx * H + gy)) ok = false;
    uint64_t vis[HW], pl[kLevelPlanes][HW];
    int top = 0, overflow = 0;
#pragma unroll
    for (int k = 0; k < HW; ++k) {
        vis[k] = 0;
#pragma unroll
        for (int p = 0; p < kLevelPlanes; ++p) pl[p][k] = 0;
    }
    if (ok) {
        uint64_t fr[HW];
        load_free_row<H>(env_bits, W, x, fr);
        if (W * H > kMaxFrontier + 1) {
            overflow = group_bfs_planes<H, R, true>(fr, gx, gy, vis, pl, top, s_words);
        } else {
            overflow = group_bfs_planes<H, R, false>(fr, gx, gy, vis, pl, top, s_words);
        }
    }
    // greedy mask at (spx, spy): the owners of the cell and of its four
    // neighbours publish their levels (slots: cell, x - 1, x + 1, y - 1, y + 1)
    const bool on_map = (uint32_t)spx < (uint32_t)W && (uint32_t)spy < (uint32_t)H;
    if (on_map) {
        if (x == spx) {
            s_gm[0] = plane_level<H>(vis, pl, spy);
            s_gm[3] = spy > 0 ? plane_level<H>(vis, pl, spy - 1) : kUnreachable;
            s_gm[4] = spy + 1 < H ? plane_level<H>(vis, pl, spy + 1) : kUnreachable;
        }
        if (x == spx - 1) s_gm[1] = plane_level<H>(vis, pl, spy);
        if (x == spx + 1 && x < W) s_gm[2] = plane_level<H>(vis, pl, spy);
        // neighbours off the map have no owner
        if (tid == 0 && spx == 0) s_gm[1] = kUnreachable;
        if (tid == 0 && spx + 1 >= W) s_gm[2] = kUnreachable;
    }
    __syncthreads();
    uint32_t info = ok ? (uint32_t)(overflow < 0xFFFFFF ? overflow : 0xFFFFFF) << kInfoOverflowShift
                       : kInfoBadGoal;
    if (on_map) {
        const uint32_t c0 = s_gm[0];
        const uint32_t n[4] = {s_gm[1], s_gm[2], s_gm[3], s_gm[4]};
        uint32_t m = 0;
#pragma unroll
        for (int d = 0; d < 4; ++d)
            if (n[d] != kUnreachable && c0 > n[d]) m |= 8u >> d;
        info |= m;
    }
    // the map's tiles: this lane's row, 8 cells per segment (the border ring
    // keeps its unreachable cells; rows past W hold no reached cell)
    const int nplanes = top == 0 ? 0 : 32 - __clz(top);
    uint4* tout = reinterpret_cast<uint4*>(b.cost_tiles + agent_index * tcells);
    const int strip_words = (int)(strip_cells(W) / 8u);
    if (x < (W + 7) / 8 * 8) {
#pragma unroll
        for (int k = 0; k < HW; ++k) {
            const int groups = (H - k * 64) < 64 ? (H - k * 64) / 8 : 8;
            for (int jj = 0; jj < groups; ++jj) {
                const int sh = jj * 8;
                uint64_t lo = 0, hi = 0;
#pragma unroll
                for (int p = 0; p < 8; ++p) lo |= ((pl[p][k] >> sh) & 0xFFull) << (8 * p);
                lo = transpose8x8(lo);
                if (nplanes > 8) {
#pragma unroll
                    for (int p = 0; p < 8; ++p) hi |= ((pl[8 + p][k] >> sh) & 0xFFull) << (8 * p);
                    hi = transpose8x8(hi);
                }
                const uint32_t reached = (uint32_t)(vis[k] >> sh) & 0xFFu;
                uint32_t w[4];
#pragma unroll
                for (int c = 0; c < 8; c += 2) {
                    uint32_t d0 = (uint32_t)((lo >> (8 * c)) & 0xFF) | ((uint32_t)((hi >> (8 * c)) & 0xFF) << 8);
                    uint32_t d1 = (uint32_t)((lo >> (8 * c + 8)) & 0xFF) | ((uint32_t)((hi >> (8 * c + 8)) & 0xFF) << 8);
                    d0 = ((reached >> c) & 1) ? d0 : kUnreachable;
                    d1 = ((reached >> (c + 1)) & 1) ? d1 : kUnreachable;
                    w[c / 2] = d0 | (d1 << 16);
                }
                const int strip = k * 8 + jj;  // columns 8 strip .. 8 strip + 7
                tout[(strip + 1) * strip_words + x + 8] = make_uint4(w[0], w[1], w[2], w[3]);
            }
        }
    }
    __syncthreads();  // s_words and s_gm are rewritten by the next refresh
    return info;
}

// ---------------------------------------------------------------------------
// Pass 1a (maps of more than kMarkedCells cells): unpack + goal-cache refresh
// + agent info, one lane per agent, no LDS.  An agent whose field is kept
// gets its greedy mask from the tiled field; one whose reset flag is set is
// marked for pass 1b.
// ---------------------------------------------------------------------------
constexpr int kUnpackThreads = 256;

template <int H, bool kRows>
__global__ __launch_bounds__(kUnpackThreads) void unpack_kernel(
    jl_mapfgpt_t b, const int16_t* __restrict__ raw_rows, const int16_t* __restrict__ cur_x,
    const int16_t* __restrict__ cur_y, const int16_t* __restrict__ goal_x,
    const int16_t* __restrict__ goal_y) {
    const int N = b.n_envs * b.n_agents;
    const int i = blockIdx.x * kUnpackThreads + threadIdx.x;
    // the build's diagnostics start from zero; pass 2 and append_actions add
    if (blockIdx.x == 0 && threadIdx.x < 4) b.diagnostics[threadIdx.x] = 0;
    if (i >= N) return;
    uint32_t info;
    const uint4 st = unpack_agent<kRows>(b, i, raw_rows, cur_x, cur_y, goal_x, goal_y, info);
    const uint32_t px = st.y & 0xFFFFu, py = st.y >> 16;
    if ((st.w >> 16) != 0) {
        info |= kInfoNeedsBfs;
    } else if (px < (uint32_t)b.map_w && py < (uint32_t)H) {
        info |= kept_greedy<H, false>(b, (size_t)i, (int)px, (int)py);
    }
    b.agent_info[i] = info;
}

// ---------------------------------------------------------------------------
// Pass 1b: BFS of the marked agents.  A fixed grid sized to the CUs the LDS
// fields allow; wavefront g scans agents [g * per_wave, (g + 1) * per_wave)
// for the mark, so a build without a changed goal costs one scan of
// agent_info.  Each refresh completes the agent's info word.
// ---------------------------------------------------------------------------
template <int H, int R, int kWaves>
__global__ __launch_bounds__(kWave* kWaves) void bfs_kernel(jl_mapfgpt_t b, int per_wave) {
    extern __shared__ __align__(16) uint16_t s_dist_all[];
    const int N = b.n_envs * b.n_agents;
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    uint16_t* s_dist = s_dist_all + (size_t)wave * b.map_w * H;  // this wavefront's field
    const int begin = (blockIdx.x * kWaves + wave) * per_wave;
    const int end = (begin + per_wave) < N ? (begin + per_wave) : N;
    for (int c0 = begin; c0 < end; c0 += kWave) {
        const int i = c0 + lane;
        const uint32_t mine = i < end ? b.agent_info[i] : 0u;
        uint64_t todo = __ballot((mine & kInfoNeedsBfs) != 0);
        while (todo) {
            const int src = __ffsll((unsigned long long)todo) - 1;
            todo &= todo - 1;
            const size_t agent_index = (size_t)c0 + src;
            // the agent's state row as pass 1a left it
            const uint4 row = *reinterpret_cast<const uint4*>(b.state_packed + agent_index * 8);
            const uint32_t bits = refresh_field<H, R, false>(
                b, agent_index, row.x & 0xFFFFu, (int)(row.z & 0xFFFFu), (int)(row.z >> 16),
                (int)(row.y & 0xFFFFu), (int)(row.y >> 16), s_dist);
            if (lane == src) b.agent_info[agent_index] = (mine & ~(kInfoNeedsBfs | kInfoGreedy)) | bits;
        }
    }
}

// Pass 1 as one launch on maps of more than 64 rows (and more than
// kMarkedCells cells): unpack_kernel's work and the BFS of the changed goals.
// Workgroup g of R wavefronts unpacks agents [g * per_group, (g + 1) *
// per_group), one thread per agent and pass, and lists those whose goal
// changed (reset flag) in LDS; then the whole workgroup refreshes their
// fields one after the other (refresh_field_group), and each agent's thread
// completes its info word.  A build without a changed goal is the unpack
// alone.  The grid is sized to the workgroups resident at once (the group
// BFS's registers allow two per CU), so the unpack's round trips overlap.
template <int H, int R, bool kRows>
__global__ __launch_bounds__(kWave* R) void unpack_group_bfs_kernel(
    jl_mapfgpt_t b, const int16_t* __restrict__ raw_rows, const int16_t* __restrict__ cur_x,
    const int16_t* __restrict__ cur_y, const int16_t* __restrict__ goal_x,
    const int16_t* __restrict__ goal_y, int per_group) {
    constexpr int kThreads = kWave * R;
    __shared__ uint64_t s_words[group_bfs_words<H, R>()];
    __shared__ uint32_t s_gm[8];
    __shared__ int s_n;
    extern __shared__ __align__(16) uint4 s_list[];  // [per_group]: agent, state row words y, z
    const int N = b.n_envs * b.n_agents;
    const int tid = threadIdx.x;
    const int begin = blockIdx.x * per_group;
    const int end = (begin + per_group) < N ? (begin + per_group) : N;
    // the build's diagnostics start from zero; pass 2 and append_actions add
    if (blockIdx.x == 0 && tid < 4) b.diagnostics[tid] = 0;
    if (tid == 0) s_n = 0;
    __syncthreads();
    for (int i = begin + tid; i < end; i += kThreads) {
        uint32_t info;
        const uint4 st = unpack_agent<kRows>(b, i, raw_rows, cur_x, cur_y, goal_x, goal_y, info);
        const uint32_t px = st.y & 0xFFFFu, py = st.y >> 16;
        if ((st.w >> 16) != 0) {
            // info of a listed agent: completed after its refresh
            s_list[atomicAdd(&s_n, 1)] = make_uint4((uint32_t)i, info | (st.x << 16), st.y, st.z);
            continue;
        }
        if (px < (uint32_t)b.map_w && py < (uint32_t)H) info |= kept_greedy<H, false>(b, (size_t)i, (int)px, (int)py);
        b.agent_info[i] = info;
    }
    __syncthreads();
    const int n = __builtin_amdgcn_readfirstlane(s_n);
    for (int k = 0; k < n; ++k) {
        const uint4 it = s_list[k];
        const uint32_t agent = (uint32_t)__builtin_amdgcn_readfirstlane((int)it.x);
        const uint32_t head = (uint32_t)__builtin_amdgcn_readfirstlane((int)it.y);
        const uint32_t pos = (uint32_t)__builtin_amdgcn_readfirstlane((int)it.z);
        const uint32_t goal = (uint32_t)__builtin_amdgcn_readfirstlane((int)it.w);
        const uint32_t bits = refresh_field_group<H, R>(b, agent, head >> 16, (int)(goal & 0xFFFFu), (int)(goal >> 16),
                                                        (int)(pos & 0xFFFFu), (int)(pos >> 16), s_words, s_gm);
        if (tid == 0) b.agent_info[agent] = (head & 0xFFFFu) | bits;
    }
}

// LDS bytes of one wavefront of unpack_bfs_kernel: its field, or the high
// level planes of refresh_field_levels where that is the path (W <= 64,
// H <= 64) and they are larger.
__host__ __device__ inline size_t marked_wave_lds(int W, int H) {
    const size_t field = (size_t)W * H * 2;
    return (W <= kWave && H <= 64 && field < (size_t)kHighPlaneBytes) ? (size_t)kHighPlaneBytes : field;
}

// ---------------------------------------------------------------------------
// Pass 1 for maps of at most kMarkedCells cells (8 KB fields) when the
// single-launch build does not apply: 1a and 1b in one launch, one lane per
// agent and 4 wavefronts per workgroup, each wavefront refreshing the fields
// of its own agents whose goal changed in its LDS field.  The tiled copies
// it writes carry the greedy marks (jl_common.h, marked_fields).
// ---------------------------------------------------------------------------
template <int H, int R, bool kRows, int kWaves>
__global__ __launch_bounds__(kWave* kWaves) void unpack_bfs_kernel(
    jl_mapfgpt_t b, const int16_t* __restrict__ raw_rows, const int16_t* __restrict__ cur_x,
    const int16_t* __restrict__ cur_y, const int16_t* __restrict__ goal_x,
    const int16_t* __restrict__ goal_y) {
    extern __shared__ __align__(16) uint16_t s_dist_all[];
    const int W = b.map_w;
    const int N = b.n_envs * b.n_agents;
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int i = blockIdx.x * (kWave * kWaves) + threadIdx.x;
    uint16_t* s_dist = s_dist_all + (size_t)wave * (marked_wave_lds(W, H) / 2);  // this wavefront's field
    // the build's diagnostics start from zero; pass 2 and append_actions add
    if (blockIdx.x == 0 && threadIdx.x < 4) b.diagnostics[threadIdx.x] = 0;

    uint4 st = make_uint4(0u, 0u, 0u, 0u);
    uint32_t info = 0;
    if (i < N) st = unpack_agent<kRows>(b, i, raw_rows, cur_x, cur_y, goal_x, goal_y, info);
    const bool reset = i < N && (st.w >> 16) != 0;
    const uint32_t px = st.y & 0xFFFFu, py = st.y >> 16;
    if (i < N && !reset && px < (uint32_t)W && py < (uint32_t)H)
        info |= kept_greedy<H, true>(b, (size_t)i, (int)px, (int)py);

    uint64_t todo = __ballot(reset);
    while (todo) {
        const int src = __ffsll((unsigned long long)todo) - 1;
        todo &= todo - 1;
        const uint32_t sx = (uint32_t)__shfl((int)st.x, src, kWave);
        const uint32_t sy = (uint32_t)__shfl((int)st.y, src, kWave);
        const uint32_t sz = (uint32_t)__shfl((int)st.z, src, kWave);
        const uint32_t bits = refresh_field<H, R, true>(
            b, (size_t)(i - lane) + src, sx & 0xFFFFu, (int)(sz & 0xFFFFu), (int)(sz >> 16),
            (int)(sy & 0xFFFFu), (int)(sy >> 16), s_dist);
        if (lane == src) info |= bits;
    }
    if (i < N) b.agent_info[i] = info;
}

// ---------------------------------------------------------------------------
// Pass 2: tokens (mapf_gpt_materialize_tokens_kernel, :350-497) plus the
// agent scatter and its diagnostics (:328-347).
//
// Phase 1 (whole workgroup, one env): per agent a template of ten uint16
// (position, goal, and codes of its five history values and greedy mask,
// :437-456, from which a row's tokens follow in two operations) and the
// offset of its window in its tiled field, and a cell -> agent map, in LDS.  The map is dense (one int32 per cell of the map
// grown by a kRadius border of empty cells, so a window probe needs no bounds
// test) while it fits; beyond, it is sparse: the ids of the occupied cells in
// cell order, and per 32 cells of the same bordered map their occupancy bits
// beside the count of occupied cells before them, so a probe is one 8-byte
// read, a bit test, a rank (a bit-field extract and a population count) and
// one read.
// Phase 2 (each wavefront on its own, no workgroup barrier): a wavefront
// produces its egos two at a time.  Lanes 0..32 load the 33 tile-row
// segments of both egos' 11x11 windows (cells outside the map staged as
// unreachable) for the next pair while the current pair is turned into
// tokens.  Visible agents: lane l probes window cells l and l + 64 in the
// map.  The window centre holds the ego's cell, whose agent has the only
// distance-0 key and takes slot 0; every other candidate's rank under the key
// (Manhattan distance, id) is 1 + the number of smaller keys, counted by
// walking the ballot of candidates with uniform readlanes; ranks 0..12 are
// the reference's sorted top 13 because keys are unique.  Every token of the
// row is computed by exactly one lane (two cost tokens per lane through an
// LDS table; agent-section token t = slot * 10 + field on lane t % 64, from
// the slot's template) into the wavefront's LDS row, which keeps the previous
// ego's agent section, so only the slots in use now or then are rewritten
// (one pass of the lanes for up to six); the row is then stored as 64 x
// 16-byte writes.
// ---------------------------------------------------------------------------
constexpr int kTokThreads = 1024;
// Bound of a single-launch workgroup's wait for its launch's cleared totals
// (each try is a device-scope load and a ~128-cycle sleep, about a
// microsecond, so the bound is tens of milliseconds; workgroup 0, dispatched
// first, clears them at its start, so a healthy launch never reaches it).
constexpr int kDiagSpinLimit = 1 << 16;
constexpr int kTokWaves = kTokThreads / kWave;
// Egos per workgroup of a two-launch build: every workgroup stages its whole
// env, so a workgroup takes the whole env (in steps of 128) up to 512 egos;
// larger envs span ceil(A / 512) workgroups, whose LDS (under 80 KB up to
// 1024 agents on any map) lets two share a CU (a single launch takes its
// whole env).
__host__ __device__ inline int ego_slice(int A) { return A > 512 ? 512 : (A + 127) / 128 * 128; }
constexpr int kDenseCellLimit = 16384;     // map cells up to which the agent map is dense
// A window is read as 11 rows x 3 tile columns of 16-byte tile-row segments
// (8 cells each): the 11 columns of a row span 2 or 3 tile columns.
constexpr int kSegPerEgo = kDiam * 3;
constexpr int kRegionCols = 24;            // cells per region row (3 tile columns)
constexpr int kSlotStride = 16;            // per-wave top-13 slot array (words)
constexpr int kCopyTokens = 6;             // per-agent tokens independent of the ego: five history
                                           // tokens and the greedy token
// Per-agent template of the token pass: uint16 half f is the value behind
// agent-section field f (position x, y, goal x, y, the codes of the five
// history values, the greedy mask); an agent off the map has position
// 0xFFFF, 0xFFFF (its first word is kNoAgent).
constexpr int kTmplBytes = kAgentTokens * 2;
static_assert(kAgentTokens == 4 + kCopyTokens, "template: four coordinates and the copied values");
// Code of a history value v (any uint16) from which its token, 44 for the
// empty action v = 5 and 45 + v otherwise (:437-451), follows as code + 44 +
// (code >= 6): 0 for v = 5, v + 1 for v <= 4, v itself from 6 on.  The
// greedy mask is its own code (token 50 + mask, :452-456).
constexpr uint32_t kHistCodeStep = 6;
__device__ __forceinline__ uint32_t history_code(uint32_t v) { return v == 5 ? 0u : (v < 5 ? v + 1 : v); }
static_assert(kTokWait == kTokEmptyAction + 1, "history codes: 45 + v = code + 44 for v <= 4");

// per-wavefront LDS: two egos' windows, the token row, the slot array
constexpr int kWinBytes = 2 * kSegPerEgo * 16;
constexpr int kRowBytes = kContext * 4;
constexpr int kWaveBytes = kWinBytes + kRowBytes + kSlotStride * 4;
static_assert(kWinBytes % 16 == 0 && kWaveBytes % 16 == 0, "16-byte LDS alignment");
static_assert(kSegPerEgo <= kWave, "one window segment per lane");
static_assert(kCostTokens + kVisible * kAgentTokens <= kContext, "row layout");
static_assert(kVisible * kAgentTokens > 2 * kWave && kVisible * kAgentTokens <= 3 * kWave,
              "agent-section tokens: two per lane and a few on a third pass");
typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kCentreCell = kRadius * kDiam + kRadius;  // 60: the ego's own cell
static_assert(kCentreCell < kWave, "the centre is a first-cell probe");
// Cost-token table: entry i in [0, 42] is the token of d - c = i - 21 (42
// below -20, 0..40 between, 43 above +20); entry 43 is an unreachable cell's.
constexpr int kLutEntries = 2 * kCostLimit + 4;
constexpr int kLutUnreachable = 2 * kCostLimit + 3;
__device__ __forceinline__ int cost_lut_entry(int i) {
    return i == kLutUnreachable ? kTokUnreachable
                                : (i == 0 ? kTokNegClip : (i > 2 * kCostLimit + 1 ? kTokPosClip : i - 1));
}

struct TokLayout {
    bool dense;
    int occ_words;  // occupancy words of a sparse map with its kRadius border (0 on dense maps)
    size_t map_off, occ_off, ids_off, tmpl_off, seg_off, lut_off, wave_off, diag_off, total;
};

__host__ __device__ inline size_t align16(size_t v) { return (v + 15) & ~(size_t)15; }

__host__ __device__ inline TokLayout tok_layout(int A, int W, int H) {
    TokLayout L;
    const size_t cells = (size_t)W * H;
    L.dense = cells <= (size_t)kDenseCellLimit;
    L.occ_words = L.dense ? 0 : (int)(((size_t)(W + 2 * kRadius) * (H + 2 * kRadius) + 31) / 32);
    size_t off = 0;
    L.map_off = off;
    if (L.dense) off = align16(off + (size_t)(W + 2 * kRadius) * (H + 2 * kRadius) * 4);
    L.occ_off = off;  // uint2 per 32 bordered cells: occupancy bits, occupied cells before them
    off = align16(off + (size_t)L.occ_words * 8);
    L.ids_off = off;  // per occupied cell in cell order: the lowest id on it (+ a spare entry)
    if (!L.dense) off = align16(off + (size_t)(A + 1) * 4);
    L.tmpl_off = off;
    off = align16(off + (size_t)A * kTmplBytes);
    L.seg_off = off;  // per agent: its window's first segment offset | three strips (see the kernel)
    off = align16(off + (size_t)A * 4);
    L.lut_off = off;
    off = align16(off + (size_t)kLutEntries * 4);
    L.wave_off = off;
    off = align16(off + (size_t)kTokWaves * kWaveBytes);
    L.diag_off = off;
    off = align16(off + 4 * 4);
    L.total = off;
    return L;
}

// Token of a copied per-agent value: a raw history value v (5 = empty,
// else kTokWait + v, any uint16, mapf_gpt_cuda.cu:437-451) or, for k = 5, the
// greedy mask (:452-456).
__device__ __forceinline__ int copy_token(uint32_t v, int k) {
    return k == kCopyTokens - 1 ? kTokGreedy + (int)v : (v == 5 ? kTokEmptyAction : kTokWait + (int)v);
}

// Lanes of an agent-section pass whose token t = base + lane is a
// coordinate field (t % 10 < 4), and of those the y fields (odd).
__host__ __device__ constexpr uint64_t coord_lanes(int base, bool y_only) {
    uint64_t m = 0;
    for (int l = 0; l < kWave; ++l) {
        const int f = (base + l) % kAgentTokens;
        if (f < 4 && (!y_only || (f & 1))) m |= 1ull << l;
    }
    return m;
}

// build_scratch of the single-launch build (JL_BUILD_SCRATCH_WORDS int32):
// at byte 0 the uint64 number of the last launch whose diagnostics were
// cleared; at byte 8 (word kGaveUpWord) a uint32 count of workgroups whose
// wait for that number gave up (sticky: only the host clears it); from byte
// 128, kArriveClasses uint64 arrival counters, one 128-byte line each.  Workgroup g belongs to class g % kArriveClasses and
// adds 1 to its class's counter once, so every launch (n_envs workgroups,
// the builder's fixed env count) adds the same per-class count.
constexpr int kArriveClasses = 64;
constexpr int kGaveUpWord = JL_BUILD_SCRATCH_GAVE_UP_WORD;
constexpr int kArriveBaseWords = 32;
constexpr int kArriveStrideWords = 32;
static_assert(kArriveBaseWords + kArriveClasses * kArriveStrideWords == JL_BUILD_SCRATCH_WORDS,
              "build_scratch layout");

__device__ __forceinline__ unsigned long long* arrival_counter(const jl_mapfgpt_t& b) {
    return reinterpret_cast<unsigned long long*>(
        b.build_scratch + kArriveBaseWords + (blockIdx.x % kArriveClasses) * kArriveStrideWords);
}

// The workgroup's arrival, returning the number of this launch on this
// builder (1, 2, ...), the same in every workgroup: no workgroup of an
// earlier launch is still running, so the counter's value before the add
// is (launches so far) x (class count) plus the fewer than one class count
// of this launch's arrivals that came first.  Derived on the device, it
// stays right in builds captured into a graph and replayed.  Called once
// per workgroup, by one lane.
__device__ __forceinline__ unsigned long long single_launch_number(const jl_mapfgpt_t& b) {
    const unsigned cls = blockIdx.x % kArriveClasses;
    const unsigned long long per = (gridDim.x - 1 - cls) / kArriveClasses + 1;
    return __hip_atomic_fetch_add(arrival_counter(b), 1ull, __ATOMIC_RELAXED,
                                  __HIP_MEMORY_SCOPE_AGENT) / per + 1;
}

// Diagnostics of a single-launch build.  No earlier launch of the build
// cleared them: workgroup 0 clears them at its start and then stores the
// launch's number (single_launch_number) in build_scratch; a workgroup with
// counts to add (d, its env's sums) waits (bounded) for that number, then
// adds.  Totals, the number and the arrival counters move only through
// device-scope atomics, performed where every XCD sees them.  Workgroups
// without counts, the usual case, touch neither.  A wait that reaches its
// bound (the number never came: the builder's arrival counters or launches
// out of order) still adds its counts, which a clear may then have wiped or
// not, and counts itself in the sticky kGaveUpWord for the host to report.
__device__ __forceinline__ void publish_single_diagnostics(const jl_mapfgpt_t& b, const int* d,
                                                           unsigned long long launch) {
    if ((d[0] | d[1] | d[2] | d[3]) == 0) return;
    const unsigned long long* cleared = reinterpret_cast<const unsigned long long*>(b.build_scratch);
    bool seen = false;
    for (int spin = 0; spin < kDiagSpinLimit; ++spin) {
        if (__hip_atomic_load(cleared, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= launch) {
            seen = true;
            break;
        }
        __builtin_amdgcn_s_sleep(2);
    }
    if (!seen) atomicAdd(reinterpret_cast<unsigned int*>(b.build_scratch) + kGaveUpWord, 1u);
    for (int k = 0; k < 4; ++k)
        if (d[k]) atomicAdd(b.diagnostics + k, d[k]);
}

// The token pass of a two-launch build (pass 1 has written the state rows and
// agent info words).
template <int H, bool kDense>
__global__ __launch_bounds__(kTokThreads) void tokens_kernel(jl_mapfgpt_t b) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int A = b.n_agents, W = b.map_w;
    // workgroup = (env, slice of egos); every slice stages the whole env
    const int slice = ego_slice(A);
    const int parts = (A + slice - 1) / slice;
    const int env = blockIdx.x / parts;
    const int part = blockIdx.x - env * parts;
    const int e_begin = part * slice;
    const int e_end = (e_begin + slice) < A ? (e_begin + slice) : A;
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);  // uniform per wavefront
    const TokLayout L = tok_layout(A, W, H);
    constexpr int MH = H + 2 * kRadius;  // bordered map columns
    uint32_t* s_map = reinterpret_cast<uint32_t*>(smem + L.map_off);
    uint2* s_occ = reinterpret_cast<uint2*>(smem + L.occ_off);
    uint32_t* s_ids = reinterpret_cast<uint32_t*>(smem + L.ids_off);
    uint32_t* s_tmpl = reinterpret_cast<uint32_t*>(smem + L.tmpl_off);  // kTmplBytes / 4 words per agent
    uint32_t* s_seg = reinterpret_cast<uint32_t*>(smem + L.seg_off);
    int* s_lut = reinterpret_cast<int*>(smem + L.lut_off);
    int* s_diag = reinterpret_cast<int*>(smem + L.diag_off);
    uint8_t* my_lds = smem + L.wave_off + (size_t)wave * kWaveBytes;
    uint4* my_win = reinterpret_cast<uint4*>(my_lds);                  // [2 egos][11 rows][3 segments]
    int* my_row = reinterpret_cast<int*>(my_lds + kWinBytes);           // [kContext]
    uint32_t* my_slots = reinterpret_cast<uint32_t*>(my_lds + kWinBytes + kRowBytes);
    constexpr int kTmplWords = kTmplBytes / 4;
    static_assert(kTmplBytes % 4 == 0, "template words");
    // distance bits of a tiled field value: only maps of at most
    // kMarkedCells cells, all of them dense here, carry greedy marks
    const uint32_t fmask = kDense ? field_mask(W, H) : 0xFFFFu;
    // phase 1 at the highest priority; the ego loop lowers it as each
    // wavefront advances
    __builtin_amdgcn_s_setprio(3);

    // ---- phase 1 -----------------------------------------------------------
    if (kDense) {
        const int mcells = (W + 2 * kRadius) * MH;  // even: MH is
        uint2* m2 = reinterpret_cast<uint2*>(s_map);
        for (int k = tid; k < mcells / 2; k += kTokThreads) m2[k] = make_uint2(kNoAgent, kNoAgent);
    } else {
        for (int k = tid; k < L.occ_words; k += kTokThreads) s_occ[k] = make_uint2(0u, 0u);
        for (int k = tid; k <= A; k += kTokThreads) s_ids[k] = kNoAgent;
    }
    // slot arrays only ever hold agent ids (stale entries stay readable);
    // row tokens past the agent section are always padding
    if (lane < kSlotStride) my_slots[lane] = 0;
    if (lane < kContext - (kCostTokens + kVisible * kAgentTokens))
        my_row[kCostTokens + kVisible * kAgentTokens + lane] = kTokPad;
    if (tid < kLutEntries) s_lut[tid] = cost_lut_entry(tid);
    if (tid < 4) s_diag[tid] = 0;
    lds_barrier();
    int d_over = 0, d_row = 0, d_dup = 0, d_bad = 0;
    for (int a = tid; a < A; a += kTokThreads) {
        const size_t g = (size_t)env * A + a;
        const uint4 st = *reinterpret_cast<const uint4*>(b.state_packed + g * 8);
        const uint32_t info = b.agent_info[g];
        const uint16_t* h = b.histories + g * 5;
        uint32_t hist[5];
#pragma unroll
        for (int k = 0; k < 5; ++k) hist[k] = h[k];  // any uint16 is legal in a raw row (:442-451)
        const uint32_t px = st.y & 0xFFFFu, py = st.y >> 16;
        const uint32_t gx = st.z & 0xFFFFu, gy = st.z >> 16;
        if (a >= e_begin && a < e_end) b.active_mask[g] = (px != gx || py != gy) ? 1 : 0;
        const bool valid = px < (uint32_t)W && py < (uint32_t)H;
        // the byte offset of the first tile-row segment of the agent's
        // window from the env's first tiled field, bit 0 set when the window
        // spans three column strips (an agent off the map: cell 0's window)
        {
            const int ex = valid ? (int)px : 0, ey = valid ? (int)py : 0;
            const int tyl = ((ey - kRadius + 64) >> 3) - 8;  // floor((ey - 5) / 8)
            const bool third = (tyl + 2) * 8 <= ey + kRadius;
            s_seg[a] = (uint32_t)a * (uint32_t)tiled_cells(W, H) * 2u + (uint32_t)(tyl + 1) * strip_cells(W) * 2u +
                       (uint32_t)(ex - kRadius + 8) * 16u + (third ? 1u : 0u);
        }
        // the template: position (kNoAgent off the map: such an ego's row is
        // padding, and no window holds it), goal, history codes, greedy mask
        uint32_t* tp = s_tmpl + a * kTmplWords;
        tp[0] = valid ? st.y : kNoAgent;
        tp[1] = st.z;
        tp[2] = history_code(hist[0]) | (history_code(hist[1]) << 16);
        tp[3] = history_code(hist[2]) | (history_code(hist[3]) << 16);
        tp[4] = history_code(hist[4]) | ((info & kInfoGreedy) << 16);
        d_over += (int)(info >> kInfoOverflowShift);
        d_row += (info & kInfoBadRow) ? 1 : 0;
        d_bad += (info & kInfoBadGoal) ? 1 : 0;
        if (valid) {
            const uint32_t cell = (px + kRadius) * MH + py + kRadius;
            if (kDense) {
                // lowest id keeps a shared cell; each extra agent counts once
                if (atomicMin(&s_map[cell], (uint32_t)a) != kNoAgent) ++d_dup;
            } else {
                atomicOr(&s_occ[cell >> 5].x, 1u << (cell & 31));
            }
        } else {
            ++d_bad;  // position off the map (scatter, :336-339)
        }
    }
    if (!kDense) {
        // Sparse map (the map grown by a kRadius border of empty cells, so a
        // window probe needs no bounds test): the occupied cells are ranked
        // in cell order (the count of occupied cells before each occupancy
        // word plus the set bits below the cell's own) and the lowest id on
        // each occupied cell is kept at its rank.  The wave sums of the scan use wavefront 0's
        // window area, which phase 2 fills later.
        uint32_t* s_wsum = reinterpret_cast<uint32_t*>(smem + L.wave_off);
        lds_barrier();
        const int per = (L.occ_words + kTokThreads - 1) / kTokThreads;
        const int w0 = tid * per;
        const int w1 = (w0 + per) < L.occ_words ? (w0 + per) : L.occ_words;
        uint32_t sum = 0;
        for (int w = w0; w < w1; ++w) sum += __popc(s_occ[w].x);
        uint32_t incl = sum;
        for (int off = 1; off < kWave; off <<= 1) {
            const uint32_t t = __shfl_up(incl, off, kWave);
            if (lane >= off) incl += t;
        }
        if (lane == kWave - 1) s_wsum[wave] = incl;
        lds_barrier();
        uint32_t run = incl - sum;
        for (int k = 0; k < wave; ++k) run += s_wsum[k];
        for (int w = w0; w < w1; ++w) {
            s_occ[w].y = run;
            run += __popc(s_occ[w].x);
        }
        lds_barrier();
        for (int a = tid; a < A; a += kTokThreads) {
            const uint32_t pos = s_tmpl[a * kTmplWords];
            if (pos == kNoAgent) continue;
            const uint32_t cell = ((pos & 0xFFFFu) + kRadius) * (uint32_t)MH + (pos >> 16) + kRadius;
            const uint2 ow = s_occ[cell >> 5];
            const uint32_t rank = ow.y + __popc(ow.x & ((1u << (cell & 31)) - 1u));
            // lowest id keeps a shared cell; each extra agent counts once
            if (atomicMin(&s_ids[rank], (uint32_t)a) != kNoAgent) ++d_dup;
        }
    }
    if (part != 0) d_over = d_row = d_dup = d_bad = 0;  // the env's counts come from its first slice
    if (d_over) atomicAdd(&s_diag[0], d_over);
    if (d_row) atomicAdd(&s_diag[1], d_row);
    if (d_dup) atomicAdd(&s_diag[2], d_dup);
    if (d_bad) atomicAdd(&s_diag[3], d_bad);
    lds_barrier();
    if (tid < 4 && s_diag[tid]) {
        // relaxed device-scope adds: the build's totals are complete when
        // the kernel is, and pass 1 of the build cleared them
        atomicAdd(b.diagnostics + tid, s_diag[tid]);
    }

    // ---- phase 2: lane constants ---------------------------------------------
    // Window cells q0 = lane and q1 = lane + 64 (row-major over the 11x11
    // window; lanes 57..63 repeat cell 120, whose probe they leave out):
    // probed for agents and turned into cost tokens q0, q1.
    const bool own_q1 = lane + kWave < kCostTokens;
    const int q0 = lane, q1 = own_q1 ? lane + kWave : kCostTokens - 1;
    const int di0 = q0 / kDiam, dj0 = q0 % kDiam, di1 = q1 / kDiam, dj1 = q1 % kDiam;
    const int win0 = di0 * kRegionCols + dj0, win1 = di1 * kRegionCols + dj1;
    const int map0 = (di0 - kRadius) * MH + (dj0 - kRadius);
    const int map1 = (di1 - kRadius) * MH + (dj1 - kRadius);
    const uint32_t qd0 = (uint32_t)(abs(di0 - kRadius) + abs(dj0 - kRadius)) << 16;
    const uint32_t qd1 = (uint32_t)(abs(di1 - kRadius) + abs(dj1 - kRadius)) << 16;
    // probe lanes whose cell can hold a candidate other than the centre's
    // agent: every q0 but the centre, q1 on lanes 0..56
    constexpr uint64_t kProbe0 = ~(1ull << kCentreCell);
    constexpr uint64_t kProbe1 = (1ull << (kCostTokens - kWave)) - 1;
    // agent-section passes: token 121 + t, t = lane (pass 0), lane + 64 (pass
    // 1), lane + 128 (pass 2, lanes 0..1: slot 12's fields 8 and 9); field f
    // of slot s is half f of the template of the slot's agent
    const int a_slot0 = lane / kAgentTokens, a_f0 = lane % kAgentTokens;
    const int a_slot1 = (lane + kWave) / kAgentTokens, a_f1 = (lane + kWave) % kAgentTokens;
    const int a_f2 = (lane & 1) + 8;
    const uint32_t toff0 = (uint32_t)L.tmpl_off + (uint32_t)a_f0 * 2u;
    const uint32_t toff1 = (uint32_t)L.tmpl_off + (uint32_t)a_f1 * 2u;
    const uint32_t toff2 = (uint32_t)L.tmpl_off + (uint32_t)a_f2 * 2u;
    constexpr uint64_t kCoord0 = coord_lanes(0, false), kCoordY0 = coord_lanes(0, true);
    constexpr uint64_t kCoord1 = coord_lanes(kWave, false), kCoordY1 = coord_lanes(kWave, true);
    const bool coord0 = (kCoord0 >> lane) & 1, coord1 = (kCoord1 >> lane) & 1;
    // all ones on lanes of a y coordinate (selects ey over ex)
    const int ysel0 = ((kCoordY0 >> lane) & 1) ? -1 : 0, ysel1 = ((kCoordY1 >> lane) & 1) ? -1 : 0;
    // copied fields: token = code + base + (code >= step); the greedy
    // field's step is past every code
    const int cbase0 = a_f0 == kAgentTokens - 1 ? kTokGreedy : kTokEmptyAction;
    const int cbase1 = a_f1 == kAgentTokens - 1 ? kTokGreedy : kTokEmptyAction;
    const int cbase2 = a_f2 == kAgentTokens - 1 ? kTokGreedy : kTokEmptyAction;
    const uint32_t cstep0 = a_f0 == kAgentTokens - 1 ? 0x10000u : kHistCodeStep;
    const uint32_t cstep1 = a_f1 == kAgentTokens - 1 ? 0x10000u : kHistCodeStep;
    const uint32_t cstep2 = a_f2 == kAgentTokens - 1 ? 0x10000u : kHistCodeStep;
    uint32_t* const sink = my_slots + kSlotStride - 1;  // writes of lanes with nothing to write
    int* const row_sink = reinterpret_cast<int*>(sink);
    // the previous ego's slots in use on this wavefront: the row keeps that
    // ego's agent section (all of it is padding before the first ego)
    int prev_n = kVisible;

    // Agent on bordered cell `cell` of this env (sparse map): the id at the
    // occupied cell's rank.  The rank is read unconditionally (an empty
    // cell's rank is at most the occupied-cell count, the spare entry) and
    // the caller keeps the id of an occupied cell only.
    // (Bit-field extracts take the low five bits of their offset and width.
    // The word index and the rank are formed in assembly: the compiler would
    // otherwise fold the shift into the index scaling as a shift and a mask,
    // and distribute the rank's scaling over its two terms.)
    auto probe_sparse = [&](uint32_t cell, uint32_t& id) -> bool {
        uint32_t w, rank;
        asm("v_lshrrev_b32 %0, 5, %1" : "=v"(w) : "v"(cell));
        const uint2 ow = s_occ[w];
        // rank: the occupied cells below this cell in its word (the field
        // of width cell & 31 from bit 0) plus those before the word
        asm("v_bcnt_u32_b32 %0, %1, %2" : "=v"(rank) : "v"(__builtin_amdgcn_ubfe(ow.x, 0u, cell)), "v"(ow.y));
        id = s_ids[rank];
        return __builtin_amdgcn_ubfe(ow.x, cell, 1u) != 0u;
    };

    // Window gather.  Lane l < 33 loads segment l = (row i, tile column j) of
    // an ego's window: cells (ex - 5 + i, 8 * (tyl + j) .. 8 * (tyl + j) + 7)
    // with tyl = floor((ey - 5) / 8), one 16-byte load from the tiled field.
    // Rows and tile columns outside the map fall in the field's border of
    // unreachable cells, a third tile column the window does not reach
    // re-reads the second, and lanes 33..63 repeat segments 0..30, so every
    // load is issued without a branch and touches only the window's lines.
    // Offsets are 32-bit bytes from the env's first tiled field (the host
    // checks that they fit).
    const size_t tcells = tiled_cells(W, H);
    const uint8_t* env_tiles =
        reinterpret_cast<const uint8_t*>(b.cost_tiles + (size_t)env * A * tcells);
    const uint32_t strip_bytes = strip_cells(W) * 2u;
    const int g_seg = lane < kSegPerEgo ? lane : lane - kSegPerEgo;
    const int g_i = g_seg / 3, g_j = g_seg - (g_seg / 3) * 3;
    // lane part of a segment's offset: row g_i of the window, strip g_j (a
    // window of two strips re-reads the second for its third)
    const uint32_t lane_seg3 = (uint32_t)g_i * 16u + (uint32_t)g_j * strip_bytes;
    const uint32_t lane_seg2 = (uint32_t)g_i * 16u + (uint32_t)(g_j < 1 ? g_j : 1) * strip_bytes;
    // Plain loads: they leave the agents' own-cell lines in the caches for
    // the next build's unpack, which reads them first (non-temporal loads
    // here took the token pass from 91.0 to 86.7 us at C5 and the unpack
    // from 11 to 14 us, the step unchanged).
    auto seg_load = [&](uint32_t seg) -> uint4 {
        const uint32_t off = (seg & ~15u) + ((seg & 1u) ? lane_seg3 : lane_seg2);
        return *reinterpret_cast<const uint4*>(env_tiles + off);
    };

    // One agent-section token from template half w of a slot's agent: a
    // coordinate relative to the ego, clip(w - e, -20, 20) + 20 with e = ex,
    // or ey on lanes of a y field, computed as clamp(w + (20 - ex) + (ysel &
    // (ex - ey)), 0, 40); a copied value's token from its code.
    auto agent_token = [&](uint32_t o, uint32_t toff, bool coord, int ysel, int x20, int dxy, int cbase,
                           uint32_t cstep) -> int {
        const uint32_t w = *reinterpret_cast<const uint16_t*>(smem + (__umul24(o, (uint32_t)kTmplBytes) + toff));
        const int c = (int)w + x20 + (ysel & dxy);
        const int ct = c < 0 ? 0 : (c > 2 * kCostLimit ? 2 * kCostLimit : c);
        const int kt = (int)w + cbase + (w >= cstep ? 1 : 0);
        return coord ? ct : kt;
    };
    // Cost token of a window value through the LDS table: index clamp(d - c +
    // 21, 0, 42) (42 below -20, 43 above +20) or 43 for an unreachable cell.
    auto cost_token_lut = [&](uint32_t v, int c_minus_21) {
        const int t = (int)(v & fmask) - c_minus_21;
        const int i = t < 0 ? 0 : (t > 2 * kCostLimit + 2 ? 2 * kCostLimit + 2 : t);
        return s_lut[v == kUnreachable ? kLutUnreachable : i];
    };

    // One ego's row: tokens into my_row, then the 16-byte store.
    auto produce = [&](const uint4 rec, int e, const uint16_t* win_base) {
        v4i out = {kTokPad, kTokPad, kTokPad, kTokPad};
        const uint32_t pos = rec.x;
        if (pos != kNoAgent) {
            const int ex = (int)(pos & 0xFFFFu), ey = (int)(pos >> 16);
            // region row = dx + 5, column = dy + 5 + ((ey + 3) & 7) (see seg_load)
            const uint16_t* win = win_base + (rec.w >> 24);
            const uint32_t craw = win[kRadius * kRegionCols + kRadius];
            const uint32_t center = field_distance((uint32_t)__builtin_amdgcn_readfirstlane((int)craw), fmask);
            const uint32_t v0 = win[win0];  // raw tiled values: the table index strips the marks
            const uint32_t v1 = win[win1];
            uint32_t id0, id1;
            bool occ0, occ1;
            const uint32_t mcell = rec.w & 0xFFFFFFu;
            if (kDense) {
                const uint32_t* mrow = s_map + mcell;
                id0 = mrow[map0];
                id1 = mrow[map1];
                occ0 = id0 != kNoAgent;
                occ1 = id1 != kNoAgent;
            } else {
                occ0 = probe_sparse(mcell + (uint32_t)map0, id0);
                occ1 = probe_sparse(mcell + (uint32_t)map1, id1);
            }
            // the centre's agent (an ego on the map stands there) is slot 0
            const uint32_t centre_id = (uint32_t)__builtin_amdgcn_readlane((int)id0, kCentreCell);
            // other candidates: (distance << 16 | id), ranked among themselves
            const uint32_t key0 = qd0 | id0, key1 = qd1 | id1;
            const uint64_t m0 = __ballot(occ0) & kProbe0;
            const uint64_t m1 = __ballot(occ1) & kProbe1;
            int r0 = 1, r1 = 1;
            for (uint64_t m = m0; m;) {
                const int l = __builtin_ctzll(m);
                m &= ~(1ull << l);
                const uint32_t k = (uint32_t)__builtin_amdgcn_readlane((int)key0, l);
                r0 += k < key0;
                r1 += k < key1;
            }
            for (uint64_t m = m1; m;) {
                const int l = __builtin_ctzll(m);
                m &= ~(1ull << l);
                const uint32_t k = (uint32_t)__builtin_amdgcn_readlane((int)key1, l);
                r0 += k < key0;
                r1 += k < key1;
            }
            const int others = __popcll(m0) + __popcll(m1);
            const int nsel = others + 1 < kVisible ? others + 1 : kVisible;
            // the selected ids move through the wave's slot array
            if (occ0 && lane != kCentreCell && r0 < kVisible) my_slots[r0] = id0;
            if (occ1 && own_q1 && r1 < kVisible) my_slots[r1] = id1;
            my_slots[0] = centre_id;
            // cost tokens
            const int c21 = (int)center - (kCostLimit + 1);
            my_row[q0] = cost_token_lut(v0, c21);
            my_row[q1] = cost_token_lut(v1, c21);
            wave_sync();
            // agent section: slots in use now or for the previous ego; a
            // slot at or past nsel is padding.  Up to six slots (tokens
            // 0..59, padding at 60..63) take one pass of the lanes.
            const int span = (nsel > prev_n ? nsel : prev_n) * kAgentTokens;
            const int live = nsel * kAgentTokens;
            const int x20 = kCostLimit - ex, dxy = ex - ey;
            {
                const uint32_t o = my_slots[a_slot0];
                const int t = agent_token(o, toff0, coord0, ysel0, x20, dxy, cbase0, cstep0);
                my_row[kCostTokens + lane] = lane < live ? t : kTokPad;
            }
            if (span > kWave) {
                const uint32_t o = my_slots[a_slot1];
                const int t = agent_token(o, toff1, coord1, ysel1, x20, dxy, cbase1, cstep1);
                my_row[kCostTokens + kWave + lane] = lane + kWave < live ? t : kTokPad;
                if (span > 2 * kWave) {
                    const uint32_t o2 = my_slots[kVisible - 1];
                    const int t2 = agent_token(o2, toff2, false, 0, 0, 0, cbase2, cstep2);
                    *(lane < 2 ? my_row + kCostTokens + 2 * kWave + lane : row_sink) =
                        nsel == kVisible ? t2 : kTokPad;
                }
            }
            prev_n = nsel;
            wave_sync();
            out = reinterpret_cast<const v4i*>(my_row)[lane];
            wave_sync();  // row and slot reads done before the next ego's writes
        }
        // streaming store: the row is not read again by this build
        __builtin_nontemporal_store(
            out, reinterpret_cast<v4i*>(b.tokens + ((size_t)env * A + e) * kContext) + lane);
    };

    // ---- phase 2: pairs of egos, pair p on wavefront p % kTokWaves ----------
    // Vector-memory stores count in the same in-order counter as the window
    // loads.  Every step stores exactly two rows (an odd slice's last pair
    // repeats its ego: the same tokens into the same row) and commits the
    // next pair's windows after those stores in straight-line code, so
    // waiting for the loads does not wait for the stores.
    const int npairs = (e_end - e_begin + 1) >> 1;
    if (wave >= npairs) return;
    const uint16_t* win_a = reinterpret_cast<const uint16_t*>(my_win);
    const uint16_t* win_b = reinterpret_cast<const uint16_t*>(my_win + kSegPerEgo);
    auto ego_a = [&](int p) { return e_begin + 2 * p; };
    auto ego_b = [&](int p) { return (e_begin + 2 * p + 1) < e_end ? e_begin + 2 * p + 1 : e_begin + 2 * p; };
    // An ego's record, wavefront-uniform: its position word; its window
    // segment offset; its cell in the bordered map | the window's first
    // column inside its first strip << 24 (used for an ego on the map only).
    auto record = [&](int e) {
        const uint32_t pos = (uint32_t)__builtin_amdgcn_readfirstlane((int)s_tmpl[e * kTmplWords]);
        const uint32_t seg = (uint32_t)__builtin_amdgcn_readfirstlane((int)s_seg[e]);
        const uint32_t ex = pos & 0xFFFFu, ey = pos >> 16;
        const uint32_t mcell = (ex + kRadius) * (uint32_t)MH + ey + kRadius;
        return make_uint4(pos, 0u, seg, mcell | (((ey + 3) & 7) << 24));
    };
    uint4 ga, gb;
    uint4 rec_a, rec_b;  // records of the pair whose windows are staged
    auto stage = [&](int p) {
        rec_a = record(ego_a(p));
        rec_b = record(ego_b(p));
        ga = seg_load(rec_a.z);
        gb = seg_load(rec_b.z);
    };
    auto commit = [&]() {
        // every use of the loaded values stays here, so that the loads stay
        // in flight across the current pair's token work
        asm volatile("" : "+v"(ga.x), "+v"(ga.y), "+v"(ga.z), "+v"(ga.w));
        asm volatile("" : "+v"(gb.x), "+v"(gb.y), "+v"(gb.z), "+v"(gb.w));
        if (lane < kSegPerEgo) {
            my_win[lane] = ga;
            my_win[kSegPerEgo + lane] = gb;
        }
        wave_sync();
    };
    stage(wave);
    commit();
    // The hardware issues the oldest wavefront first, which lets the first
    // workgroup of a CU race ahead and leaves the last one alone at the end;
    // wavefronts further along yield instead: priority 3 for the first
    // quarter of this wavefront's pairs, 2, 1, then 0 for the last.
    const int iters = (npairs - wave + kTokWaves - 1) / kTokWaves;
    int p = wave, it = 0;
    for (int quarter = 0; quarter < 4; ++quarter) {
        switch (quarter) {
            case 0: __builtin_amdgcn_s_setprio(3); break;
            case 1: __builtin_amdgcn_s_setprio(2); break;
            case 2: __builtin_amdgcn_s_setprio(1); break;
            default: __builtin_amdgcn_s_setprio(0); break;
        }
        const int it_end = ((quarter + 1) * iters + 3) / 4;  // the first pair of the next quarter
        for (; it < it_end; ++it, p += kTokWaves) {
            const uint4 cur_a = rec_a, cur_b = rec_b;
            const int pn = p + kTokWaves;
            // always staged (no branch around the loads, which would make the
            // compiler wait for them early); after the last pair it repeats this one
            stage(pn < npairs ? pn : p);
            produce(cur_a, ego_a(p), win_a);
            produce(cur_b, ego_b(p), win_b);
            commit();
        }
    }
}

// ---------------------------------------------------------------------------
// Single-launch build (maps of at most kMarkedCells cells, A <= 1024): one
// workgroup per env does the whole build of build_tokens / build_tokens_from_state
// (mapf_gpt_builder.cpp:89-114, 140-167): unpack and goal-cache refresh, BFS of
// the env's changed goals, scatter, tokens.  512-thread workgroups (1024 when
// A > 512) whose LDS stays under 40 KB at the C2/C3 shape, so four share a CU
// and a grid of up to 4 x CUs envs runs in one round: each workgroup's start
// (two dependent HBM round trips) is paid once per launch, not once per round.
//
// Start: thread t unpacks agent t (state, goal cache, history in one round
// trip); the env's changed goals are listed and refreshed by up to
// L.bfs_waves wavefronts, whose BFS fields overlay the token area.  Then, in
// one second round trip, every agent's own tiled cell (its greedy-move mark)
// and every wavefront's first ego pair of windows are loaded while the cell
// -> agent map (uint16 ids, a 5-cell empty border so that window probes need
// no bounds test) and a 10-word slot template per agent (position, goal, the
// six copied tokens) are laid out in LDS.
//
// Egos (pairs per wavefront, no workgroup barrier, the next pair's windows in
// flight while the current pair is turned into tokens), per ego:
//  * visible agents: lane l probes window cells l and l + 64 in the map.  The
//    window centre holds the ego's cell, whose agent has the only distance-0
//    key and takes slot 0; the other candidates' keys (distance << 16 | id)
//    are compacted into LDS by ballot position and each compacted lane counts
//    the smaller keys, four per broadcast read, which gives its slot;
//  * cost tokens: two cells per lane from the window staged in LDS;
//  * agent section: token 121 + l on lane l (and l + 64 when more than six
//    slots are in use): the slot's template word, made relative to the ego for
//    the four coordinates.  The row buffer keeps the previous ego's agent
//    section, so only slots in use now or then are rewritten, which is one
//    pass for up to six visible agents;
//  * the row leaves as 64 x 16-byte streaming stores.
// ---------------------------------------------------------------------------
constexpr uint16_t kNoAgent16 = 0xFFFFu;
constexpr int kTmplWords = 10;  // slot template: x, y, goal x, goal y, 5 history tokens, greedy token
// LDS the BFS fields of a refresh may overlay: at least this much, so that
// four 64x64 fields refresh at once in each workgroup
constexpr size_t kBuildFieldRoom = 32768;
// Visible-agent keys of the single-launch build, 16 bits: (Manhattan
// distance << 10) | id, below 2^15 (distance <= 10, id < 1024), so a 16-bit
// difference of two keys is negative exactly when the first is smaller.  The
// pad of the compacted key list is above every key.
constexpr uint32_t kKeyPad16 = 0x7FFFu;
constexpr int kKeyDistShift = 10;
typedef short v2s __attribute__((ext_vector_type(2)));

// Per-agent record of the single-launch build: position word (kNoAgent off
// the map), goal word, the byte offset of its window's first tile-row segment
// from the env's first tiled field with bit 0 set when the window spans three
// column strips, and the byte offset of its cell in the LDS agent map with
// the window's first column inside its strip ((y + 3) & 7) in bits 16..18.
constexpr int kBuildRecWords = 4;

struct BuildLayout {
    int bfs_waves;
    size_t map_off, tmpl_off, wave_off, lut_off, overlay;  // token area, overlaid by BFS fields
    size_t rec_off, info_off, list_off, nlist_off, diag_off, total;
};

__host__ __device__ inline BuildLayout build_layout(int A, int W, int H, int waves) {
    BuildLayout L;
    const size_t cells = (size_t)W * H;
    size_t off = 0;
    L.map_off = off;
    off = align16(off + (size_t)(W + 2 * kRadius) * (H + 2 * kRadius) * 2);
    L.tmpl_off = off;
    off = align16(off + (size_t)A * kTmplWords * 4);
    L.wave_off = off;
    off = align16(off + (size_t)waves * kWaveBytes);
    L.lut_off = off;
    off = align16(off + (size_t)kLutEntries * 4);
    const size_t field = cells * 2;
    const size_t room = off > kBuildFieldRoom ? off : kBuildFieldRoom;
    const size_t fit = room / field;
    L.bfs_waves = (int)(fit < (size_t)waves ? fit : (size_t)waves);
    size_t fields = (size_t)L.bfs_waves * field;
    // builds whose fields stay in registers keep their high level planes
    // in the overlay instead (refresh_field_levels)
    if (W <= kWave && H <= 64 && fields < (size_t)waves * kHighPlaneBytes) fields = (size_t)waves * kHighPlaneBytes;
    L.overlay = align16(off > fields ? off : fields);
    off = L.overlay;
    L.rec_off = off;
    off = align16(off + (size_t)A * kBuildRecWords * 4);
    L.info_off = off;
    off = align16(off + (size_t)A * 4);
    L.list_off = off;
    off = align16(off + (size_t)A * 8);
    L.nlist_off = off;
    off = align16(off + 4);
    L.diag_off = off;
    off = align16(off + 4 * 4);
    L.total = off;
    return L;
}

// Workgroup size of the single-launch build: one thread per agent.
__host__ __device__ inline int build_threads(int A) { return A <= 512 ? 512 : 1024; }

// Lowest agent id keeps a shared cell of the uint16 map: min of the 16-bit
// half of its dword by compare-and-swap (LDS has no 16-bit atomic min).
// Returns the id the cell held before.
__device__ __forceinline__ uint32_t map16_min(uint16_t* map, uint32_t cell, uint32_t id) {
    uint32_t* word = reinterpret_cast<uint32_t*>(map) + (cell >> 1);
    const uint32_t shift = (cell & 1u) * 16u;
    uint32_t cur = *word;
    while (true) {
        const uint32_t held = (cur >> shift) & 0xFFFFu;
        if (held <= id) return held;
        const uint32_t next = (cur & ~(0xFFFFu << shift)) | (id << shift);
        const uint32_t seen = atomicCAS(word, cur, next);
        if (seen == cur) return held;
        cur = seen;
    }
}

template <int H, bool kRows, int R, int kThreads>
// Held to 8 wavefronts per SIMD (4 workgroups of 512 threads per CU); not
// for H = 256 (16-row maps), whose BFS registers would then spill.
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(H <= 128 ? 8 : 1))) void build_kernel(
    jl_mapfgpt_t b, const int16_t* __restrict__ raw_rows, const int16_t* __restrict__ cur_x,
    const int16_t* __restrict__ cur_y, const int16_t* __restrict__ goal_x,
    const int16_t* __restrict__ goal_y) {
    constexpr int kWaves = kThreads / kWave;
    constexpr int MH = H + 2 * kRadius;  // map columns
    extern __shared__ __align__(16) uint8_t smem[];
    const int A = b.n_agents, W = b.map_w;
    const int env = blockIdx.x;
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const BuildLayout L = build_layout(A, W, H, kWaves);
    const size_t cells = (size_t)W * H;
    const size_t tcells = tiled_cells(W, H);
    const uint32_t fmask = field_mask(W, H);
    uint16_t* s_map = reinterpret_cast<uint16_t*>(smem + L.map_off);
    int* s_tmpl = reinterpret_cast<int*>(smem + L.tmpl_off);
    int* s_lut = reinterpret_cast<int*>(smem + L.lut_off);
    uint32_t* s_rec = reinterpret_cast<uint32_t*>(smem + L.rec_off);
    uint32_t* s_info = reinterpret_cast<uint32_t*>(smem + L.info_off);
    uint2* s_list = reinterpret_cast<uint2*>(smem + L.list_off);
    int* s_nlist = reinterpret_cast<int*>(smem + L.nlist_off);
    int* s_diag = reinterpret_cast<int*>(smem + L.diag_off);
    uint8_t* my_lds = smem + L.wave_off + (size_t)wave * kWaveBytes;
    uint4* my_win = reinterpret_cast<uint4*>(my_lds);
    int* my_row = reinterpret_cast<int*>(my_lds + kWinBytes);
    uint32_t* my_slots = reinterpret_cast<uint32_t*>(my_lds + kWinBytes + kRowBytes);

    // the start (round trips and staging) at the highest priority; the ego
    // loop lowers it as each wavefront advances
    __builtin_amdgcn_s_setprio(3);
    unsigned long long launch = 0;  // lane 0 of thread 0: this launch's number
    if (tid == 0) {
        *s_nlist = 0;
        s_diag[0] = s_diag[1] = s_diag[2] = s_diag[3] = 0;
    }
    if (blockIdx.x == 0 && tid == 0) {
        // this launch's diagnostics start from zero, then its number is
        // published (publish_single_diagnostics, at the end)
        launch = single_launch_number(b);
        int z = 0;
        for (int k = 0; k < 4; ++k) z |= atomicExch(b.diagnostics + k, 0);
        asm volatile("" ::"v"(z));  // cleared before the launch is published
        atomicExch(reinterpret_cast<unsigned long long*>(b.build_scratch), launch);
    }

    // ---- start: unpack (one round trip) ---------------------------------------
    const bool mine = tid < A;
    const size_t g = (size_t)env * A + (mine ? tid : 0);
    uint4 st = make_uint4(0u, 0u, 0u, 0u);
    uint32_t hist[5] = {5u, 5u, 5u, 5u, 5u};
    uint32_t info = 0;
    if (mine) {
        const uint16_t* h = b.histories + g * 5;
#pragma unroll
        for (int k = 0; k < 5; ++k) hist[k] = h[k];  // the kept history (a rejected raw row's too)
        st = unpack_agent<kRows>(b, (int)g, raw_rows, cur_x, cur_y, goal_x, goal_y, info);
        if (kRows && !(info & kInfoBadRow)) {
            const uint16_t* row = reinterpret_cast<const uint16_t*>(raw_rows) + g * 13;
#pragma unroll
            for (int k = 0; k < 5; ++k) hist[k] = row[8 + k];
        }
    }
    const uint32_t px = st.y & 0xFFFFu, py = st.y >> 16;
    const bool valid = mine && px < (uint32_t)W && py < (uint32_t)H;
    const bool reset = mine && (st.w >> 16) != 0;
    lds_barrier();  // s_nlist and s_diag cleared
    const uint32_t strip_bytes = strip_cells(W) * 2u;
    const uint32_t field_bytes = (uint32_t)tcells * 2u;
    if (mine) {
        const uint32_t ex = valid ? px : 0u, ey = valid ? py : 0u;  // windows of agents off the map: cell 0
        const uint32_t y8 = ey + (8 - kRadius);                        // bordered first column
        const uint32_t seg = (uint32_t)tid * field_bytes + (y8 >> 3) * strip_bytes + (ex + (8 - kRadius)) * 16u;
        uint4 rec;
        rec.x = valid ? st.y : kNoAgent;
        rec.y = st.z;
        rec.z = seg | ((y8 & 7u) >= 6u ? 1u : 0u);
        rec.w = ((ex + kRadius) * MH + ey + kRadius) * 2u | ((y8 & 7u) << 16);
        reinterpret_cast<uint4*>(s_rec)[tid] = rec;
        s_info[tid] = info;
        if (reset) s_list[atomicAdd(s_nlist, 1)] = make_uint2((uint32_t)tid, st.x);
    }
    lds_barrier();

    // ---- changed goals: BFS fields --------------------------------------------
    const int nlist = __builtin_amdgcn_readfirstlane(*s_nlist);
    if constexpr (R == 1 && RowWords<H>::HW == 1) {
        // fields in registers (refresh_field_levels): wavefront w refreshes
        // list entries w, w + kWaves, ... and stores their tiles itself
        for (int k = wave; k < nlist; k += kWaves) {
            const uint2 it = s_list[k];
            const uint32_t a = (uint32_t)__builtin_amdgcn_readfirstlane((int)it.x);
            const uint32_t sx = (uint32_t)__builtin_amdgcn_readfirstlane((int)it.y);
            const uint32_t pos = (uint32_t)__builtin_amdgcn_readfirstlane((int)s_rec[a * kBuildRecWords]);
            const uint32_t goal = (uint32_t)__builtin_amdgcn_readfirstlane((int)s_rec[a * kBuildRecWords + 1]);
            const uint32_t bits = refresh_field_levels<H>(
                b, (size_t)env * A + a, sx & 0xFFFFu, (int)(goal & 0xFFFFu), (int)(goal >> 16), (int)(pos & 0xFFFFu),
                (int)(pos >> 16), reinterpret_cast<uint64_t*>(smem + (size_t)wave * kHighPlaneBytes));
            if (lane == 0) s_info[a] |= bits;
        }
        // the refreshed tiles are stored before any window load of this
        // workgroup
        if (nlist > 0) __syncthreads();
    } else
    // rounds of up to bfs_waves fields overlaying the token area: each
    // wavefront searches one into its LDS field, then the whole workgroup
    // stores the round's tiles
    for (int r0 = 0; r0 < nlist; r0 += L.bfs_waves) {
        if (wave < L.bfs_waves && r0 + wave < nlist) {
            uint16_t* s_dist = reinterpret_cast<uint16_t*>(smem) + (size_t)wave * cells;
            const uint2 it = s_list[r0 + wave];
            const uint32_t a = (uint32_t)__builtin_amdgcn_readfirstlane((int)it.x);
            const uint32_t sx = (uint32_t)__builtin_amdgcn_readfirstlane((int)it.y);
            const uint32_t pos = (uint32_t)__builtin_amdgcn_readfirstlane((int)s_rec[a * kBuildRecWords]);
            const uint32_t goal = (uint32_t)__builtin_amdgcn_readfirstlane((int)s_rec[a * kBuildRecWords + 1]);
            const uint32_t bits = refresh_field<H, R, true, false>(
                b, (size_t)env * A + a, sx & 0xFFFFu, (int)(goal & 0xFFFFu), (int)(goal >> 16),
                (int)(pos & 0xFFFFu), (int)(pos >> 16), s_dist);
            if (lane == 0) s_info[a] |= bits;
        }
        __syncthreads();
        const int nround = (nlist - r0) < L.bfs_waves ? (nlist - r0) : L.bfs_waves;
        for (int f = 0; f < nround; ++f) {
            const uint32_t a = s_list[r0 + f].x;
            store_field_tiles<H, true>(b, (size_t)env * A + a, reinterpret_cast<uint16_t*>(smem) + (size_t)f * cells,
                                       tid, kThreads);
        }
        // the refreshed fields are stored before any window load of this
        // workgroup, and the LDS fields are free for the next round or the
        // token area
        __syncthreads();
    }

    // ---- second round trip: own cells' marks and the first windows ------------
    uint32_t f_center = kUnreachable;
    if (valid && !reset) f_center = b.cost_tiles[g * tcells + tile_offset((int)px, (int)py, W)];

    // Window segment of this lane: lane l < 33 loads segment (row i, column
    // strip j) = l of an ego's 11 x 3 segments of 8 cells: row ex - 5 + i of
    // the strips from that of column ey - 5 on (a third strip the window does
    // not reach re-reads the second); lanes 33..63 repeat segments 0..30.
    // Cells off the map are the tiled field's unreachable border.  A strip's
    // rows are consecutive 16-byte words, so a segment lies at the ego's
    // record offset (32-bit bytes from the env's first tiled field; the host
    // checks that they fit) plus a per-lane constant.
    const uint8_t* env_tiles = reinterpret_cast<const uint8_t*>(b.cost_tiles + (size_t)env * A * tcells);
    const int g_seg = lane < kSegPerEgo ? lane : lane - kSegPerEgo;
    const int g_i = g_seg / 3, g_j = g_seg - (g_seg / 3) * 3;
    const uint32_t lane_seg3 = (uint32_t)g_i * 16u + (uint32_t)g_j * strip_bytes;
    const uint32_t lane_seg2 = (uint32_t)g_i * 16u + (uint32_t)(g_j < 1 ? g_j : 1) * strip_bytes;
    auto seg_load = [&](uint32_t seg) -> uint4 {
        const uint32_t off = (seg & ~15u) + ((seg & 1u) ? lane_seg3 : lane_seg2);
        return *reinterpret_cast<const uint4*>(env_tiles + off);
    };
    const int npairs = (A + 1) >> 1;
    auto ego_a = [&](int p) { return 2 * p; };
    auto ego_b = [&](int p) { return (2 * p + 1) < A ? 2 * p + 1 : 2 * p; };
    // an ego's record, wavefront-uniform
    auto record = [&](int e) {
        const uint4 r = reinterpret_cast<const uint4*>(s_rec)[e];
        return make_uint4((uint32_t)__builtin_amdgcn_readfirstlane((int)r.x), 0u,
                          (uint32_t)__builtin_amdgcn_readfirstlane((int)r.z),
                          (uint32_t)__builtin_amdgcn_readfirstlane((int)r.w));
    };
    uint4 ga = make_uint4(0u, 0u, 0u, 0u), gb = ga;
    uint4 rec_a = ga, rec_b = ga;  // records of the pair whose windows are staged
    auto stage = [&](int p) {
        rec_a = record(ego_a(p));
        rec_b = record(ego_b(p));
        ga = seg_load(rec_a.z);
        gb = seg_load(rec_b.z);
    };
    const bool has_pairs = wave < npairs;
    if (has_pairs) stage(wave);

    // ---- token area: map, slot templates, wavefront buffers ------------------
    {
        const int mwords = ((W + 2 * kRadius) * MH * 2 + 15) / 16;  // the map's 16-byte words
        uint4* m4 = reinterpret_cast<uint4*>(s_map);
        for (int k = tid; k < mwords; k += kThreads) m4[k] = make_uint4(~0u, ~0u, ~0u, ~0u);
    }
    if (tid < kLutEntries) s_lut[tid] = cost_lut_entry(tid);
    if (lane < kSlotStride) my_slots[lane] = 0;
    // the agent section and the tail start as padding (no slot in use)
    for (int k = kCostTokens + lane; k < kContext; k += kWave) my_row[k] = kTokPad;
    lds_barrier();
    int d_over = 0, d_row = 0, d_dup = 0, d_bad = 0;
    if (mine) {
        const uint32_t gx = st.z & 0xFFFFu, gy = st.z >> 16;
        b.active_mask[g] = (px != gx || py != gy) ? 1 : 0;
        int* tp = s_tmpl + tid * kTmplWords;
        tp[0] = (int)px;
        tp[1] = (int)py;
        tp[2] = (int)gx;
        tp[3] = (int)gy;
#pragma unroll
        for (int k = 0; k < 5; ++k) tp[4 + k] = copy_token(hist[k] & 0xFFFFu, k);
        const uint32_t inf = s_info[tid];  // refresh bits included
        d_over = (int)(inf >> kInfoOverflowShift);
        d_row = (inf & kInfoBadRow) ? 1 : 0;
        d_bad = (inf & kInfoBadGoal) ? 1 : 0;
        if (valid) {
            const uint32_t prev = map16_min(s_map, (px + kRadius) * MH + py + kRadius, (uint32_t)tid);
            if (prev != kNoAgent16) ++d_dup;  // lowest id keeps a shared cell
        } else {
            ++d_bad;  // position off the map (scatter, :336-339)
        }
        // greedy mask: from the refresh, or the mark of the agent's own cell
        // in its kept field (the cross of five cells where that cell is
        // unreachable)
        uint32_t greedy = inf & kInfoGreedy;
        if (!reset && valid)
            greedy = f_center != kUnreachable ? f_center >> 12 : kept_greedy<H, false>(b, g, (int)px, (int)py);
        tp[9] = copy_token(greedy, 5);
    }
    // wavefront sums, then one LDS add per wavefront and counter
#pragma unroll
    for (int m = 1; m < kWave; m <<= 1) {
        d_over += __shfl_xor(d_over, m, kWave);
        d_row += __shfl_xor(d_row, m, kWave);
        d_dup += __shfl_xor(d_dup, m, kWave);
        d_bad += __shfl_xor(d_bad, m, kWave);
    }
    if (lane == 0 && (d_over | d_row | d_dup | d_bad)) {
        if (d_over) atomicAdd(&s_diag[0], d_over);
        if (d_row) atomicAdd(&s_diag[1], d_row);
        if (d_dup) atomicAdd(&s_diag[2], d_dup);
        if (d_bad) atomicAdd(&s_diag[3], d_bad);
    }
    lds_barrier();
    // the launch number, needed only at the end, is taken here, where its
    // round trip overlaps the token work
    if (tid == 0 && blockIdx.x != 0) launch = single_launch_number(b);

    // ---- egos: lane constants ---------------------------------------------------
    // cost / probe cells q0 = lane and q1 = lane + 64 (lanes 57..63 repeat cell
    // 120, whose probe they leave out); LDS byte offsets per lane, so that each
    // per-ego address is one add of a wavefront-uniform base
    const bool own_q1 = lane + kWave < kCostTokens;
    const int q0 = lane, q1 = own_q1 ? lane + kWave : kCostTokens - 1;
    const int di0 = q0 / kDiam, dj0 = q0 % kDiam, di1 = q1 / kDiam, dj1 = q1 % kDiam;
    const int winb0 = (di0 * kRegionCols + dj0) * 2, winb1 = (di1 * kRegionCols + dj1) * 2;
    const int mapb0 = ((di0 - kRadius) * MH + (dj0 - kRadius)) * 2;
    const int mapb1 = ((di1 - kRadius) * MH + (dj1 - kRadius)) * 2;
    const uint32_t qd0 = (uint32_t)(abs(di0 - kRadius) + abs(dj0 - kRadius)) << kKeyDistShift;
    const uint32_t qd1 = (uint32_t)(abs(di1 - kRadius) + abs(dj1 - kRadius)) << kKeyDistShift;
    const bool not_centre = lane != kCentreCell;
    // probe lanes whose cell can hold a candidate: every q0 but the centre,
    // q1 on lanes 0..56
    constexpr uint64_t kProbe0 = ~(1ull << kCentreCell);
    constexpr uint64_t kProbe1 = (1ull << (kCostTokens - kWave)) - 1;
    // agent-section passes: token 121 + t, t = lane (pass 0), lane + 64 (pass 1),
    // lane + 128 (pass 2, lanes 0..1: slot 12's last two tokens)
    const int t_slot0 = lane / kAgentTokens, t_slot1 = (lane + kWave) / kAgentTokens;
    const int t_off0 = (lane % kAgentTokens) * 4;           // byte offset in a template
    const int t_off1 = ((lane + kWave) % kAgentTokens) * 4;
    const int t_off2 = ((lane & 1) + 8) * 4;
    constexpr uint64_t kCoord0 = coord_lanes(0, false), kCoordY0 = coord_lanes(0, true);
    constexpr uint64_t kCoord1 = coord_lanes(kWave, false), kCoordY1 = coord_lanes(kWave, true);
    const bool coord0 = (kCoord0 >> lane) & 1, coordy0 = (kCoordY0 >> lane) & 1;
    const bool coord1 = (kCoord1 >> lane) & 1, coordy1 = (kCoordY1 >> lane) & 1;
    // all ones on lanes of a y coordinate token (selects ey over ex)
    const int ysel0 = coordy0 ? -1 : 0, ysel1 = coordy1 ? -1 : 0;
    const uint8_t* map_bytes = reinterpret_cast<const uint8_t*>(s_map);
    // template words through 32-bit LDS offsets
    const uint32_t tmpl_base = (uint32_t)L.tmpl_off;

    uint16_t* const my_keys16 = reinterpret_cast<uint16_t*>(my_row);  // before the cost tokens
    uint32_t* const sink = my_slots + kSlotStride - 1;               // writes of lanes with nothing to write
    int* const row_sink = reinterpret_cast<int*>(sink);
    v4i* const env_rows = reinterpret_cast<v4i*>(b.tokens + (size_t)env * A * kContext);
    int prev_n = 0;  // slots of the row buffer's agent section written for the previous ego

    // One agent-section token from slot o's template word w: a coordinate
    // relative to the ego, clip(w - e, -20, 20) + 20 with e = ex, or ey on
    // lanes of a y field, computed as clamp(w + (20 - ex) + (ysel & (ex - ey)),
    // 0, 40); copied tokens as they are.
    auto agent_token = [&](int w, bool coord, int ysel, int x20, int dxy) {
        const int c = w + x20 + (ysel & dxy);
        const int t = c < 0 ? 0 : (c > 2 * kCostLimit ? 2 * kCostLimit : c);
        return coord ? t : w;
    };
    // Cost token of a window value through the LDS table: index clamp(d - c +
    // 21, 0, 42) (42 below -20, 43 above +20) or 43 for an unreachable cell.
    auto cost_token_lut = [&](uint32_t v, int c_minus_21) {
        const int t = (int)(v & fmask) - c_minus_21;
        const int i = t < 0 ? 0 : (t > 2 * kCostLimit + 2 ? 2 * kCostLimit + 2 : t);
        return s_lut[v == kUnreachable ? kLutUnreachable : i];
    };

    auto produce = [&](const uint4 rec, int e, const uint8_t* win_base) {
        v4i out = {kTokPad, kTokPad, kTokPad, kTokPad};
        const uint32_t pos = rec.x;
        if (pos != kNoAgent) {
            const int ex = (int)(pos & 0xFFFFu), ey = (int)(pos >> 16);
            // region row = dx + 5, column = dy + 5 + ((ey + 3) & 7) (see seg_load)
            const uint8_t* win = win_base + (rec.w >> 15);  // ((ey + 3) & 7) * 2
            const uint32_t craw = *reinterpret_cast<const uint16_t*>(win + (kRadius * kRegionCols + kRadius) * 2);
            const uint32_t center = field_distance((uint32_t)__builtin_amdgcn_readfirstlane((int)craw), fmask);
            const uint32_t v0 = *reinterpret_cast<const uint16_t*>(win + winb0);
            const uint32_t v1 = *reinterpret_cast<const uint16_t*>(win + winb1);
            const uint8_t* mrow = map_bytes + (rec.w & 0xFFFFu);
            const uint32_t id0 = *reinterpret_cast<const uint16_t*>(mrow + mapb0);
            const uint32_t id1 = *reinterpret_cast<const uint16_t*>(mrow + mapb1);
            const uint32_t centre_id = (uint32_t)__builtin_amdgcn_readlane((int)id0, kCentreCell);
            // candidates other than the centre: compacted 16-bit keys
            const uint64_t m0 = __builtin_amdgcn_ballot_w64(id0 != kNoAgent16) & kProbe0;
            const uint64_t m1 = __builtin_amdgcn_ballot_w64(id1 != kNoAgent16) & kProbe1;
            const int n0 = __popcll(m0);
            const int others = n0 + __popcll(m1);
            const uint32_t p0 = __builtin_amdgcn_mbcnt_hi((uint32_t)(m0 >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m0, 0u));
            const uint32_t p1 =
                __builtin_amdgcn_mbcnt_hi((uint32_t)(m1 >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m1, (uint32_t)n0));
            if ((id0 != kNoAgent16) & not_centre) my_keys16[p0] = (uint16_t)(qd0 | id0);
            if ((id1 != kNoAgent16) & own_q1) my_keys16[p1] = (uint16_t)(qd1 | id1);
            if (lane < 8) my_keys16[others + lane] = (uint16_t)kKeyPad16;  // pad to 8-key reads
            wave_sync();
            // rank = 1 + the number of smaller keys, 8 keys per read: the
            // sign bits of the two 16-bit differences of each word
            const uint32_t mk = my_keys16[lane];
            const v2s mine2 = __builtin_bit_cast(v2s, mk | (mk << 16));
            uint32_t r = 1;  // slot 0 is the centre's
#pragma nounroll
            for (int j = 0; j < others; j += 8) {
                const uint4 k8 = *reinterpret_cast<const uint4*>(my_keys16 + j);
                r += __builtin_popcount(__builtin_bit_cast(uint32_t, __builtin_bit_cast(v2s, k8.x) - mine2) & 0x80008000u);
                r += __builtin_popcount(__builtin_bit_cast(uint32_t, __builtin_bit_cast(v2s, k8.y) - mine2) & 0x80008000u);
                r += __builtin_popcount(__builtin_bit_cast(uint32_t, __builtin_bit_cast(v2s, k8.z) - mine2) & 0x80008000u);
                r += __builtin_popcount(__builtin_bit_cast(uint32_t, __builtin_bit_cast(v2s, k8.w) - mine2) & 0x80008000u);
            }
            if ((lane < others) & (r < (uint32_t)kVisible)) my_slots[r] = mk & ((1u << kKeyDistShift) - 1u);
            my_slots[0] = centre_id;
            const int nsel = others + 1 < kVisible ? others + 1 : kVisible;
            wave_sync();
            // cost tokens (over the keys)
            const int c21 = (int)center - (kCostLimit + 1);
            my_row[q0] = cost_token_lut(v0, c21);
            my_row[q1] = cost_token_lut(v1, c21);
            // agent section: slots in use now or for the previous ego
            const int span = (nsel > prev_n ? nsel : prev_n) * kAgentTokens;
            const int x20 = kCostLimit - ex, dxy = ex - ey;
            const int live = nsel * kAgentTokens;  // tokens of the slots in use
            {
                const uint32_t o = my_slots[t_slot0];
                const int w = *reinterpret_cast<const int*>(smem + (tmpl_base + __umul24(o, kTmplWords * 4) + t_off0));
                const int t = agent_token(w, coord0, ysel0, x20, dxy);
                my_row[kCostTokens + lane] = lane < live ? t : kTokPad;
            }
            if (span > kWave) {
                const uint32_t o = my_slots[t_slot1];
                const int w = *reinterpret_cast<const int*>(smem + (tmpl_base + __umul24(o, kTmplWords * 4) + t_off1));
                const int t = agent_token(w, coord1, ysel1, x20, dxy);
                my_row[kCostTokens + kWave + lane] = lane + kWave < live ? t : kTokPad;
                if (span > 2 * kWave) {
                    const uint32_t o2 = my_slots[kVisible - 1];
                    const int w2 =
                        *reinterpret_cast<const int*>(smem + (tmpl_base + __umul24(o2, kTmplWords * 4) + t_off2));
                    *(lane < 2 ? my_row + kCostTokens + 2 * kWave + lane : row_sink) =
                        nsel == kVisible ? w2 : kTokPad;
                }
            }
            prev_n = nsel;
            wave_sync();
            out = reinterpret_cast<const v4i*>(my_row)[lane];
            wave_sync();
        }
        // streaming store: the row is not read again by this build
        __builtin_nontemporal_store(out, env_rows + e * (kContext / 4) + lane);
    };

    if (has_pairs) {
        const uint8_t* win_a = reinterpret_cast<const uint8_t*>(my_win);
        const uint8_t* win_b = reinterpret_cast<const uint8_t*>(my_win + kSegPerEgo);
        // lanes 33..63 hold copies of segments 0..30 and store them to the
        // same words
        auto commit = [&]() {
            asm volatile("" : "+v"(ga.x), "+v"(ga.y), "+v"(ga.z), "+v"(ga.w));
            asm volatile("" : "+v"(gb.x), "+v"(gb.y), "+v"(gb.z), "+v"(gb.w));
            my_win[g_seg] = ga;
            my_win[kSegPerEgo + g_seg] = gb;
            wave_sync();
        };
        commit();
        // The hardware issues the oldest wavefront first, which lets the first
        // workgroup of a CU race ahead and leaves the last one alone at the
        // end; wavefronts further along yield instead: priority 3 for the
        // first quarter of this wavefront's pairs, 2, 1, then 0 for the last.
        const int iters = (npairs - wave + kWaves - 1) / kWaves;
        int p = wave, it = 0;
        for (int quarter = 0; quarter < 4; ++quarter) {
            switch (quarter) {
                case 0: __builtin_amdgcn_s_setprio(3); break;
                case 1: __builtin_amdgcn_s_setprio(2); break;
                case 2: __builtin_amdgcn_s_setprio(1); break;
                default: __builtin_amdgcn_s_setprio(0); break;
            }
            const int it_end = ((quarter + 1) * iters + 3) / 4;  // the first pair of the next quarter
            for (; it < it_end; ++it, p += kWaves) {
                const uint4 cur_a = rec_a, cur_b = rec_b;
                const int pn = p + kWaves;
                stage(pn < npairs ? pn : p);
                produce(cur_a, ego_a(p), win_a);
                produce(cur_b, ego_b(p), win_b);
                commit();
            }
        }
    }
    // wavefront 0 always has pairs (npairs >= 1) and reaches this point
    if (tid == 0) publish_single_diagnostics(b, s_diag, launch);
}

// History roll (mapf_gpt_append_actions_kernel, mapf_gpt_cuda.cu:155-178): one
// thread per agent, 256 agents per workgroup.  The workgroup's 2560-byte
// history segment moves between HBM and LDS as 16-byte words (element-wise
// for a partial or unaligned last segment).
constexpr int kAppendThreads = 256;
constexpr int kAppendWords = kAppendThreads * 5 * 2 / 16;

__global__ __launch_bounds__(kAppendThreads) void append_actions_kernel(
    jl_mapfgpt_t b, const uint8_t* __restrict__ actions) {
    __shared__ uint4 s_hist[kAppendWords];
    uint16_t* sh = reinterpret_cast<uint16_t*>(s_hist);
    const int N = b.n_envs * b.n_agents;
    const int base = blockIdx.x * kAppendThreads;
    const int n = (N - base) < kAppendThreads ? (N - base) : kAppendThreads;
    const int tid = threadIdx.x;
    uint16_t* seg = b.histories + (size_t)base * 5;
    const bool vec = n == kAppendThreads && (reinterpret_cast<uintptr_t>(seg) & 15u) == 0;
    if (vec) {
        if (tid < kAppendWords) s_hist[tid] = reinterpret_cast<const uint4*>(seg)[tid];
    } else {
        for (int k = tid; k < n * 5; k += kAppendThreads) sh[k] = seg[k];
    }
    __syncthreads();
    bool bad = false;
    if (tid < n) {
        const int i = base + tid;
        uint16_t a = b.active_mask[i] ? (uint16_t)actions[i] : (uint16_t)0;
        if (a >= 5) {
            bad = true;
            a = 0;
        }
        uint16_t* h = sh + tid * 5;
        const uint16_t h1 = h[1], h2 = h[2], h3 = h[3], h4 = h[4];
        h[0] = h1;
        h[1] = h2;
        h[2] = h3;
        h[3] = h4;
        h[4] = a;
    }
    __syncthreads();
    if (vec) {
        if (tid < kAppendWords) reinterpret_cast<uint4*>(seg)[tid] = s_hist[tid];
    } else {
        for (int k = tid; k < n * 5; k += kAppendThreads) seg[k] = sh[k];
    }
    const uint64_t m = __ballot(bad);
    if ((tid & (kWave - 1)) == 0 && m) atomicAdd(b.diagnostics + 1, (int)__popcll(m));
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

// cost_to_go on request: each thread turns one 16-byte strip row (8 cells)
// of a tiled field into the same 8 cells of the row-major field, greedy
// marks stripped.  Grid-stride over every field of the builder.
template <int H>
__global__ __launch_bounds__(256) void cost_to_go_kernel(jl_mapfgpt_t b) {
    const int W = b.map_w;
    const uint32_t fmask = field_mask(W, H);
    const size_t fields = (size_t)b.n_envs * b.n_agents;
    const size_t per_field = (size_t)W * (H / 8);  // 16-byte words of a row-major field
    const size_t total = fields * per_field;
    const uint32_t strip_words = strip_cells(W) / 8u;  // 16-byte rows of a strip
    const size_t tcells = tiled_cells(W, H);
    const v4i* tiles = reinterpret_cast<const v4i*>(b.cost_tiles);
    v4i* out = reinterpret_cast<v4i*>(b.cost_to_go);
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
        const size_t f = i / per_field;
        const uint32_t w = (uint32_t)(i - f * per_field);
        const uint32_t x = w / (H / 8), y8 = w - x * (H / 8);  // row, 8-cell group
        v4i v = tiles[f * (tcells / 8) + (y8 + 1) * strip_words + x + 8];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t u = (uint32_t)v[k], lo = u & 0xFFFFu, hi = u >> 16;
            v[k] = (int)(field_distance(lo, fmask) | (field_distance(hi, fmask) << 16));
        }
        __builtin_nontemporal_store(v, out + i);
    }
}

// Diagnostics of a refresh without tokens (refresh_distances): the BFS
// overflow counts and bad goals pass 1 left in agent_info, summed the way the
// token pass sums them (diagnostics[0] and [3]; the token pass's scatter
// counts, [2] and the off-map part of [3], belong to token builds only).
__global__ __launch_bounds__(256) void refresh_diag_kernel(jl_mapfgpt_t b, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    const uint32_t info = i < n ? b.agent_info[i] : 0u;
    int over = (int)(info >> kInfoOverflowShift);
    int bad = (info & kInfoBadGoal) ? 1 : 0;
#pragma unroll
    for (int m = 1; m < kWave; m <<= 1) {
        over += __shfl_xor(over, m, kWave);
        bad += __shfl_xor(bad, m, kWave);
    }
    if ((threadIdx.x & (kWave - 1)) == 0) {
        if (over) atomicAdd(b.diagnostics + 0, over);
        if (bad) atomicAdd(b.diagnostics + 3, bad);
    }
}

int check_builder(const jl_mapfgpt_t* b) {
    if (!b || b->n_envs <= 0 || b->n_agents <= 0) return JL_ERR_ARG;
    if (!profile_ok(b->map_w, b->map_h)) return JL_ERR_PROFILE;
    if ((int64_t)b->n_envs * b->n_agents > 0x7FFFFFFF) return JL_ERR_ARG;
    if (b->n_agents > 65535 || b->n_envs > 65535) return JL_ERR_ARG;
    // the token pass addresses an env's tiled fields with 32-bit byte offsets
    if ((uint64_t)b->n_agents * tiled_cells(b->map_w, b->map_h) * 2u > 0xFFFFFFFFull)
        return JL_ERR_ARG;
    if (!b->grid_bits || !b->state_packed || !b->histories || !b->labels || !b->goal_cache || !b->tokens ||
        !b->active_mask || !b->diagnostics || !b->agent_info || !b->cost_tiles)
        return JL_ERR_ARG;
    // buffers accessed 16 bytes at a time, and the build scratch's 64-bit
    // atomics on 128-byte lines
    const uintptr_t wide = reinterpret_cast<uintptr_t>(b->state_packed) |
                           reinterpret_cast<uintptr_t>(b->cost_tiles) | reinterpret_cast<uintptr_t>(b->tokens) |
                           reinterpret_cast<uintptr_t>(b->cost_to_go);
    if (wide & 15u) return JL_ERR_ARG;
    if (b->build_scratch && (reinterpret_cast<uintptr_t>(b->build_scratch) & 127u)) return JL_ERR_ARG;
    return JL_OK;
}


// Pass 1b wavefronts per workgroup: each owns a W*H uint16 LDS field; up to
// 64 KB of them per workgroup, at most 4.
inline int pass1_waves(int W, int H) {
    const size_t field = (size_t)W * H * 2;
    return field <= 16384 ? 4 : (field <= 32768 ? 2 : 1);
}

template <int H, int R, bool kRows>
int launch_pass1(const jl_mapfgpt_t* b, const int16_t* rows, const int16_t* cx, const int16_t* cy,
                 const int16_t* gx, const int16_t* gy, hipStream_t stream) {
    const int N = b->n_envs * b->n_agents;
    // maps whose tiled fields carry greedy marks (at most 4096 cells, 8 KB
    // LDS fields) run pass 1 as one launch; only that launch writes marks
    if (marked_fields(b->map_w, H)) {
        const dim3 grid((N + kWave * 4 - 1) / (kWave * 4));
        const size_t lds = (size_t)4 * marked_wave_lds(b->map_w, H);
        hipLaunchKernelGGL((unpack_bfs_kernel<H, R, kRows, 4>), grid, dim3(kWave * 4), lds, stream,
                           *b, rows, cx, cy, gx, gy);
        return launch_status();
    }
    if constexpr (R > 1) {
        // unpack and the changed goals' fields in one launch: two workgroups
        // of R wavefronts per CU (the group BFS's registers), each over a
        // whole number of passes of its threads
        const int max_groups = (N + kWave * R - 1) / (kWave * R);
        int groups = device_cus() * 2;
        if (groups > max_groups) groups = max_groups;
        constexpr int kMaxList = 3072;  // 48 KB of LDS list per workgroup
        if ((N + groups - 1) / groups > kMaxList) groups = (N + kMaxList - 1) / kMaxList;
        const int per_group = ((N + groups - 1) / groups + kWave * R - 1) / (kWave * R) * (kWave * R);
        hipLaunchKernelGGL((unpack_group_bfs_kernel<H, R, kRows>), dim3((N + per_group - 1) / per_group),
                           dim3(kWave * R), (size_t)per_group * sizeof(uint4), stream, *b, rows, cx, cy, gx, gy,
                           per_group);
        return launch_status();
    }
    hipLaunchKernelGGL((unpack_kernel<H, kRows>), dim3((N + kUnpackThreads - 1) / kUnpackThreads),
                       dim3(kUnpackThreads), 0, stream, *b, rows, cx, cy, gx, gy);
    int rc = launch_status();
    if (rc) return rc;
    const int waves = pass1_waves(b->map_w, H);
    const size_t lds = (size_t)waves * b->map_w * H * sizeof(uint16_t);
    const int per_cu = (int)(160 * 1024 / lds) < 8 ? (int)(160 * 1024 / lds) : 8;
    // whole-wavefront ranges of at least one wavefront of agents
    const int max_waves = (N + kWave - 1) / kWave;
    int total_waves = device_cus() * (per_cu > 0 ? per_cu : 1) * waves;
    if (total_waves > max_waves) total_waves = max_waves;
    const int per_wave = ((N + total_waves - 1) / total_waves + kWave - 1) / kWave * kWave;
    const int blocks = ((N + per_wave - 1) / per_wave + waves - 1) / waves;
    if (waves == 4) {
        hipLaunchKernelGGL((bfs_kernel<H, R, 4>), dim3(blocks), dim3(kWave * 4), lds, stream, *b,
                           per_wave);
    } else if (waves == 2) {
        hipLaunchKernelGGL((bfs_kernel<H, R, 2>), dim3(blocks), dim3(kWave * 2), lds, stream, *b,
                           per_wave);
    } else {
        hipLaunchKernelGGL((bfs_kernel<H, R, 1>), dim3(blocks), dim3(kWave), lds, stream, *b,
                           per_wave);
    }
    return launch_status();
}

// The whole build runs as one launch (build_kernel) on maps of at most
// kMarkedCells cells whose rows have at most 64 columns (one 64-bit word per
// row in the field refresh) when an env fits one workgroup and the builder
// has its build scratch.  Narrower maps of longer rows (at most 42 rows of
// 96-256 columns) take the two-launch build: the single launch's refresh of
// rows of several words did not fit its registers.
bool single_launch(const jl_mapfgpt_t* b) {
    if (!b->build_scratch || !marked_fields(b->map_w, b->map_h) || b->map_h > 64 || b->n_agents > 1024)
        return false;
    const int threads = build_threads(b->n_agents);
    return build_layout(b->n_agents, b->map_w, b->map_h, threads / kWave).total <= 160 * 1024;
}

template <int H, bool kRows>
int launch_single(const jl_mapfgpt_t* b, const int16_t* rows, const int16_t* cx, const int16_t* cy,
                  const int16_t* gx, const int16_t* gy, hipStream_t stream) {
    const int threads = build_threads(b->n_agents);
    const size_t lds = build_layout(b->n_agents, b->map_w, H, threads / kWave).total;
    const dim3 grid(b->n_envs);
#define JL_LAUNCH_BUILD(R, T)                                                                      \
    hipLaunchKernelGGL((build_kernel<H, kRows, R, T>), grid, dim3(T), lds, stream, *b, rows, cx, cy, \
                       gx, gy)
    if constexpr (H > 64) {
        return JL_ERR_PROFILE;  // single_launch() is false for these maps
    } else if (b->map_w <= 64) {
        if (threads == 512) JL_LAUNCH_BUILD(1, 512); else JL_LAUNCH_BUILD(1, 1024);
    } else {
        // W > 64 with W * H <= kMarkedCells: H == 32 only
        if constexpr (H == 32) {
            if (threads == 512) JL_LAUNCH_BUILD(2, 512); else JL_LAUNCH_BUILD(2, 1024);
        } else {
            return JL_ERR_PROFILE;
        }
    }
#undef JL_LAUNCH_BUILD
    return launch_status();
}

template <bool kRows>
int build(const jl_mapfgpt_t* b, const int16_t* rows, const int16_t* cx, const int16_t* cy,
          const int16_t* gx, const int16_t* gy, hipStream_t stream) {
    int rc = check_builder(b);
    if (rc) return rc;
    const int W = b->map_w;
    const TokLayout L = tok_layout(b->n_agents, W, b->map_h);
    if (L.total > 160 * 1024) return JL_ERR_AGENTS;
    if (single_launch(b)) {
        JL_DISPATCH_H(b->map_h, {
            if (b->token_events[0]) {
                rc = status(hipEventRecord((hipEvent_t)b->token_events[0], stream));
                if (rc) return rc;
            }
            rc = launch_single<H, kRows>(b, rows, cx, cy, gx, gy, stream);
            if (rc) return rc;
            if (b->token_events[1]) {
                rc = status(hipEventRecord((hipEvent_t)b->token_events[1], stream));
                if (rc) return rc;
            }
        });
        return JL_OK;
    }
    JL_DISPATCH_H(b->map_h, {
        if (W <= 64) {
            rc = launch_pass1<H, 1, kRows>(b, rows, cx, cy, gx, gy, stream);
        } else if (W <= 128) {
            rc = launch_pass1<H, 2, kRows>(b, rows, cx, cy, gx, gy, stream);
        } else {
            rc = launch_pass1<H, 4, kRows>(b, rows, cx, cy, gx, gy, stream);
        }
        if (rc) return rc;
        if (b->token_events[0]) {
            rc = status(hipEventRecord((hipEvent_t)b->token_events[0], stream));
            if (rc) return rc;
        }
        const int slice = ego_slice(b->n_agents);
        const dim3 grid2((unsigned)b->n_envs * ((b->n_agents + slice - 1) / slice));
        if (L.dense) {
            hipLaunchKernelGGL((tokens_kernel<H, true>), grid2, dim3(kTokThreads), L.total, stream, *b);
        } else {
            hipLaunchKernelGGL((tokens_kernel<H, false>), grid2, dim3(kTokThreads), L.total, stream, *b);
        }
        rc = launch_status();
        if (rc) return rc;
        if (b->token_events[1]) {
            rc = status(hipEventRecord((hipEvent_t)b->token_events[1], stream));
            if (rc) return rc;
        }
    });
    return JL_OK;
}

// ---- builds that allocate nothing ------------------------------------------
// jl_mapfgpt_build_rows_noalloc takes its build scratch from this array, one
// copy per device held until the process ends, instead of the caller's
// build_scratch.  Host code never passes the array's name to a kernel (on
// the host it is only a stand-in for the device symbol): it passes the
// device address that hipGetSymbolAddress returned for the current device.
static __device__ __align__(256) int32_t scratch[JL_BUILD_SCRATCH_WORDS];

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mutex;
int32_t* g_scratch_ptr[kMaxScratchDevices] = {};

// Device address of `scratch` on the current device, looked up once per
// device (with that device current) and kept for the life of the process
// (so a hipDeviceReset, after which the array may live elsewhere, is not
// supported between calls).
int current_scratch(int32_t** out) {
    int dev = 0;
    int rc = status(hipGetDevice(&dev));
    if (rc) return rc;
    if (dev < 0 || dev >= kMaxScratchDevices) return JL_ERR_ARG;
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (!g_scratch_ptr[dev]) {
        void* ptr = nullptr;
        rc = status(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
        if (rc) return rc;
        if (!ptr || (reinterpret_cast<uintptr_t>(ptr) & 127u)) return JL_ERR_ARG;
        g_scratch_ptr[dev] = static_cast<int32_t*>(ptr);
    }
    *out = g_scratch_ptr[dev];
    return JL_OK;
}

// Zero-fills a build scratch with vector stores (a kernel rather than a
// memset node, so the clearing also holds in captured graphs).
__global__ __launch_bounds__(256) void clear_scratch_kernel(int32_t* s) {
    for (int i = threadIdx.x; i < JL_BUILD_SCRATCH_WORDS / 4; i += 256)
        reinterpret_cast<int4*>(s)[i] = make_int4(0, 0, 0, 0);
}
static_assert(JL_BUILD_SCRATCH_WORDS % 4 == 0, "16-byte clearing");

}  // namespace

const void* append_actions_kernel_address() { return reinterpret_cast<const void*>(&append_actions_kernel); }

}  // namespace jl

using namespace jl;

extern "C" int jl_mapfgpt_build_rows_noalloc(const jl_mapfgpt_t* b, const int16_t* raw_rows,
                                             jl_stream_t stream) {
    if (!b || !raw_rows) return JL_ERR_ARG;
    jl_mapfgpt_t local = *b;
    local.build_scratch = nullptr;  // the caller's build scratch is not used
    int rc = check_builder(&local);
    if (rc) return rc;
    hipStream_t st = (hipStream_t)stream;
    if (st) {
        // the scratch address is the current device's: the stream must be its
        int dev = 0, stream_dev = 0;
        rc = status(hipGetDevice(&dev));
        if (rc) return rc;
        rc = status(hipStreamGetDevice(st, &stream_dev));
        if (rc) return rc;
        if (stream_dev != dev) return JL_ERR_ARG;
    }
    int32_t* ptr = nullptr;
    rc = current_scratch(&ptr);
    if (rc) return rc;
    local.build_scratch = ptr;
    if (single_launch(&local)) {
        // every call starts from zero counters (whatever the env count of the
        // previous call on this device), so its launch number is 1
        hipLaunchKernelGGL(clear_scratch_kernel, dim3(1), dim3(256), 0, st, ptr);
        rc = launch_status();
        if (rc) return rc;
    } else {
        local.build_scratch = nullptr;  // the two-launch build uses no scratch
    }
    return build<true>(&local, raw_rows, nullptr, nullptr, nullptr, nullptr, st);
}

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

extern "C" int jl_mapfgpt_single_launch(const jl_mapfgpt_t* b) {
    if (check_builder(b)) return 0;
    return single_launch(b) ? 1 : 0;
}

extern "C" int jl_mapfgpt_refresh_state(const jl_mapfgpt_t* b, const int16_t* cur_x,
                                        const int16_t* cur_y, const int16_t* goal_x,
                                        const int16_t* goal_y, jl_stream_t stream) {
    if (!cur_x || !cur_y || !goal_x || !goal_y) return JL_ERR_ARG;
    int rc = check_builder(b);
    if (rc) return rc;
    const int W = b->map_w;
    const int N = b->n_envs * b->n_agents;
    hipStream_t st = (hipStream_t)stream;
    JL_DISPATCH_H(b->map_h, {
        if (W <= 64) {
            rc = launch_pass1<H, 1, false>(b, nullptr, cur_x, cur_y, goal_x, goal_y, st);
        } else if (W <= 128) {
            rc = launch_pass1<H, 2, false>(b, nullptr, cur_x, cur_y, goal_x, goal_y, st);
        } else {
            rc = launch_pass1<H, 4, false>(b, nullptr, cur_x, cur_y, goal_x, goal_y, st);
        }
        if (rc) return rc;
    });
    hipLaunchKernelGGL(refresh_diag_kernel, dim3((N + 255) / 256), dim3(256), 0, st, *b, N);
    return launch_status();
}

extern "C" int jl_mapfgpt_append_actions(const jl_mapfgpt_t* b, const uint8_t* actions,
                                         jl_stream_t stream) {
    int rc = check_builder(b);
    if (rc) return rc;
    if (!actions) return JL_ERR_ARG;
    const int N = b->n_envs * b->n_agents;
    hipLaunchKernelGGL(append_actions_kernel, dim3((N + kAppendThreads - 1) / kAppendThreads),
                       dim3(kAppendThreads), 0, (hipStream_t)stream, *b, actions);
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

extern "C" int jl_mapfgpt_cost_to_go(const jl_mapfgpt_t* b, jl_stream_t stream) {
    int rc = check_builder(b);
    if (rc) return rc;
    if (!b->cost_to_go) return JL_ERR_ARG;
    const size_t words = (size_t)b->n_envs * b->n_agents * b->map_w * (b->map_h / 8);
    size_t blocks = (words + 255) / 256;
    const size_t cap = (size_t)device_cus() * 16;
    if (blocks > cap) blocks = cap;
    JL_DISPATCH_H(b->map_h, {
        hipLaunchKernelGGL((cost_to_go_kernel<H>), dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, *b);
    });
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
