// jl_magat.hip - MAGAT node features and neighbour graph for gfx950.
//
// nodes: one workgroup per (env, 64-agent slice).  The env's static and
// occupancy bitmaps and its agents' positions and goals are staged in LDS,
// the slice's 11 x 11 energy windows are requested (16-byte loads) and,
// while they are in flight, the slice's neighbour counts are taken and its
// edge total written; then one wavefront per agent assembles the 676-float
// row in LDS (lane l owning patch cells l, l + 64, l + 128) and stores it as
// 16-byte words in address order, its whole 128-byte lines non-temporally
// (the reference zero-fills
// the row and rewrites it one float per thread, 128_agents_map_stateless_
// step.cu:414-421, 438-478).  The clamped ctg value is one of 21 float
// constants k/10 (the IEEE quotients), so no division is evaluated on the
// device.
// edges: one workgroup per (env, 64-source slice) sums the node pass's slice
// totals before its own (a one-workgroup env scan runs first only beyond
// 8,192 slices); lane l of each wavefront tests source l of the slice
// against 64 ids per step (packed int16 differences, one dot2 per pair) into
// per-source neighbour bitmasks in LDS; then every thread stores one edge per
// output position, sorted by (source, destination id) (grid_world_cuda.cu:
// 17-110, stateless_step.cu:854-935).  Envs of more than 1024 agents take a
// ballot writer with an LDS ring.
#include "jl_common.h"

namespace jl {
namespace {

constexpr int kNodeThreads = 256;

typedef short jl_v2s __attribute__((ext_vector_type(2)));  // (x, y) as packed int16
typedef unsigned int jl_v4u __attribute__((ext_vector_type(4)));
typedef float jl_v4f __attribute__((ext_vector_type(4)));

// (float)k / 10.0f rounded to nearest even, k = -10..10.
__device__ __constant__ float kTenths[21] = {-1.0f, -0.9f, -0.8f, -0.7f, -0.6f, -0.5f, -0.4f,
                                            -0.3f, -0.2f, -0.1f, 0.0f,  0.1f,  0.2f,  0.3f,
                                            0.4f,  0.5f,  0.6f,  0.7f,  0.8f,  0.9f,  1.0f};

// Exact round-half-even of num / den, den > 0 (stateless_step.cu:120-138).
__device__ __forceinline__ int round_half_even(int num, int den) {
    const bool neg = num < 0;
    const unsigned mag = neg ? (unsigned)(-num) : (unsigned)num;
    unsigned q = mag / (unsigned)den;
    const unsigned r = mag - q * (unsigned)den;
    if (2 * r > (unsigned)den || (2 * r == (unsigned)den && (q & 1u))) ++q;
    return neg ? -(int)q : (int)q;
}

// Goal cell of the 13x13 patch (stateless_step.cu:480-509): the goal itself
// inside the window, else its projection onto the patch border.
__device__ __forceinline__ int goal_cell(int cx, int cy, int gx, int gy) {
    const int rx = gx - cx, ry = gy - cy;
    int fx, fy;
    const int arx = rx < 0 ? -rx : rx, ary = ry < 0 ? -ry : ry;
    if (arx <= kRadius && ary <= kRadius) {
        fx = rx + 6;
        fy = ry + 6;
    } else if (ary >= arx) {
        fy = 6 * ((ry > 0) - (ry < 0) + 1);
        fx = 6 + round_half_even(6 * rx, ary);
    } else {
        fx = 6 * ((rx > 0) - (rx < 0) + 1);
        fy = 6 + round_half_even(6 * ry, arx);
    }
    fx = fx < 0 ? 0 : (fx > 12 ? 12 : fx);
    fy = fy < 0 ? 0 : (fy > 12 ? 12 : fy);
    return fx * kPygDiam + fy;
}

__global__ __launch_bounds__(256) void occupancy_kernel(jl_magat_t m) {
    extern __shared__ __align__(16) uint32_t s_occ[];
    const int j = blockIdx.x, A = m.n_agents, E = m.n_envs;
    const int words = m.map_w * m.map_h / 32;
    const uint16_t* rows = m.states + (size_t)j * A * 8;
    const uint32_t env = rows[0];
    if (env >= (uint32_t)E) return;
    for (int k = threadIdx.x; k < words; k += blockDim.x) s_occ[k] = 0;
    __syncthreads();
    for (int i = threadIdx.x; i < A; i += blockDim.x) {
        const uint4 r = *reinterpret_cast<const uint4*>(rows + (size_t)i * 8);
        if ((r.x & 0xFFFFu) >= (uint32_t)E) continue;
        // positions off the map set no bit (the reference would write out of bounds)
        if ((r.y & 0xFFFFu) >= (uint32_t)m.map_w || (r.y >> 16) >= (uint32_t)m.map_h) continue;
        const uint32_t cell = (r.y & 0xFFFFu) * (uint32_t)m.map_h + (r.y >> 16);
        atomicOr(&s_occ[cell >> 5], 1u << (cell & 31));
    }
    __syncthreads();
    uint32_t* out = m.grid_ocp + (size_t)env * words;
    for (int k = threadIdx.x; k < words; k += blockDim.x) out[k] = s_occ[k];
}

struct NodeLayout {
    size_t st_off, oc_off, pos_off, valid_off, part_off, win_off, row_off, tenths_off,
        total;
};

__host__ __device__ inline size_t a16n(size_t v) { return (v + 15) & ~(size_t)15; }

constexpr int kNodeEgos = 64;  // agents per node workgroup: an env spans ceil(A / 64)
constexpr int kWinCells = kDiam * kDiam;
constexpr int kWinRow = 16;                  // LDS bytes per staged window row (11 used)
constexpr int kWinStride = kDiam * kWinRow;  // LDS bytes per staged window
constexpr int kWinItems = (kNodeEgos * kDiam + kNodeThreads - 1) / kNodeThreads;  // window rows per thread

__host__ __device__ inline NodeLayout node_layout(int A, int W, int H) {
    NodeLayout L;
    size_t o = 0;
    L.st_off = o;
    o = a16n(o + (size_t)W * H / 8);
    L.oc_off = o;
    o = a16n(o + (size_t)W * H / 8);
    L.pos_off = o;
    o = a16n(o + (size_t)A * 4);
    L.valid_off = o;
    o = a16n(o + (size_t)A);
    L.part_off = o;  // the slice's edge counts (accumulated by the wavefronts), then goal cells
    o = a16n(o + (size_t)kNodeEgos * 8);
    L.win_off = o;  // the slice's 11x11 energy windows, kWinStride bytes each
    o = a16n(o + (size_t)kNodeEgos * kWinStride);
    L.row_off = o;  // per wavefront: one 676-float row
    o = a16n(o + (size_t)(kNodeThreads / kWave) * kPygFeatures * 4);
    L.tenths_off = o;  // the 21 ctg values k / 10
    o = a16n(o + 21 * 4);
    L.total = o;
    return L;
}

// Workgroup = (env, slice of kNodeEgos agents).  Every slice stages the env's
// bitmaps and agents in LDS, issues the loads of its agents' energy windows,
// counts its agents' neighbours within squared radius 49 while they are in
// flight (others split over the wavefronts) and writes the slice total for
// the scan.  Then one wavefront per agent row: lane l holds patch cells l,
// l + 64, l + 128 of the 13x13 patch and writes the four channels (obstacle,
// agents, goal, ctg) of its cells into an LDS row that leaves as 16-byte
// stores.
template <int H>
__global__ __launch_bounds__(kNodeThreads) void nodes_kernel(jl_magat_t m) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int A = m.n_agents, W = m.map_w, E = m.n_envs;
    const int parts = (A + kNodeEgos - 1) / kNodeEgos;
    const int env = blockIdx.x / parts;
    const int part = blockIdx.x - env * parts;
    const int e_begin = part * kNodeEgos;
    const int e_end = (e_begin + kNodeEgos) < A ? (e_begin + kNodeEgos) : A;
    const int tid = threadIdx.x, lane = tid & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);  // uniform per wavefront
    constexpr int nwaves = kNodeThreads / kWave;
    const NodeLayout L = node_layout(A, W, H);
    uint32_t* s_st = reinterpret_cast<uint32_t*>(smem + L.st_off);
    uint32_t* s_oc = reinterpret_cast<uint32_t*>(smem + L.oc_off);
    int32_t* s_pos = reinterpret_cast<int32_t*>(smem + L.pos_off);  // (int16 x, int16 y)
    uint8_t* s_valid = smem + L.valid_off;
    int32_t* s_part = reinterpret_cast<int32_t*>(smem + L.part_off);
    const int words = W * H / 32;
    const size_t cells = (size_t)W * H;
    const size_t base = (size_t)env * A;

    for (int k = tid; k < words; k += kNodeThreads) {
        s_st[k] = m.grid_bits[(size_t)env * words + k];
        s_oc[k] = m.grid_ocp[(size_t)env * words + k];
    }
    int wide = 0;  // a position outside [-8192, 8191]: counts in 32-bit arithmetic
    for (int a = tid; a < A; a += kNodeThreads) {
        const uint4 r = *reinterpret_cast<const uint4*>(m.states + (base + a) * 8);
        s_pos[a] = (int32_t)r.y;
        const int x = (int16_t)(r.y & 0xFFFFu), y = (int16_t)(r.y >> 16);
        wide |= (x < -8192 || x > 8191 || y < -8192 || y > 8191) ? 1 : 0;
        s_valid[a] = (r.x & 0xFFFFu) < (uint32_t)E ? 1 : 0;
        if (a >= e_begin && a < e_end) {
            s_part[a - e_begin] = 0;
            s_part[kNodeEgos + a - e_begin] = goal_cell((int16_t)(r.y & 0xFFFFu), (int16_t)(r.y >> 16),
                                                        (int16_t)(r.z & 0xFFFFu), (int16_t)(r.z >> 16));
        }
    }
    wide = __syncthreads_or(wide);

    // Energy windows of the slice: item i = (agent i / 11, window row i % 11).
    // The row's 11 bytes lie in two aligned 16-byte words of the field row,
    // read with two vector loads at clamped addresses (a word off the map or
    // off the row reads as 0), then shifted into place and stored as one
    // 16-byte LDS word.  Every thread has at most kWinItems items (a slice of
    // kNodeEgos agents); an item past the slice repeats item 0 (same bytes,
    // same LDS address).  The loads are issued here and consumed after the
    // neighbour count, which runs while they are in flight.
    uint8_t* s_win = smem + L.win_off;
    float* s_tenths = reinterpret_cast<float*>(smem + L.tenths_off);
    if (tid < 21) s_tenths[tid] = kTenths[tid];
    const uint8_t* env_energy = m.energy + base * cells;
    const int nitems = (e_end - e_begin) * kDiam;
    uint4 lo[kWinItems], hi[kWinItems];
    int shift[kWinItems], dst[kWinItems];
    bool ok_lo[kWinItems], ok_hi[kWinItems];
#pragma unroll
    for (int it = 0; it < kWinItems; ++it) {
        const int i = tid + it * kNodeThreads < nitems ? tid + it * kNodeThreads : 0;
        const int el = i / kDiam, r = i - el * kDiam;
        const int a = e_begin + el;
        const int32_t pos = s_pos[a];
        const int x = (int16_t)(pos & 0xFFFF) + r - kRadius;
        const int y0 = (int16_t)(pos >> 16) - kRadius;
        const bool rok = s_valid[a] && x >= 0 && x < W;
        const int c0 = y0 >> 4;  // word of column y0 (-1 for the columns left of the map)
        ok_lo[it] = rok && c0 >= 0 && c0 < H / 16;
        ok_hi[it] = rok && c0 + 1 >= 0 && c0 + 1 < H / 16;
        const uint4* row4 =
            reinterpret_cast<const uint4*>(env_energy + (size_t)a * cells + (size_t)(rok ? x : 0) * H);
        // plain loads: the rows' whole lines are stored non-temporally (below),
        // so these lines stay cached for the next step's windows
        const jl_v4u* r4 = reinterpret_cast<const jl_v4u*>(row4);
        const jl_v4u l4 = r4[ok_lo[it] ? c0 : 0];
        const jl_v4u h4 = r4[ok_hi[it] ? c0 + 1 : 0];
        lo[it] = make_uint4(l4.x, l4.y, l4.z, l4.w);
        hi[it] = make_uint4(h4.x, h4.y, h4.z, h4.w);
        shift[it] = y0 - c0 * 16;  // 0..15: byte of column y0 in lo
        dst[it] = el * kWinStride + r * kWinRow;
    }

    // Edge counts of the slice: others within squared radius 49, all rows of
    // the env block (stateless_step.cu:513-520), lane = agent of the slice,
    // the others split over the wavefronts.  With every position in
    // [-8192, 8191] the differences fit packed int16 and the test is the sign
    // of one dot2 (the agent itself, at distance 0, is taken off after);
    // otherwise 32-bit arithmetic with the reference's wrap.  Rows that are
    // skipped keep their previous count, which the totals still include; each
    // slice writes its total, and the scan adds the env's slices.
    {
        const int a = e_begin + lane;
        if (a < e_end) {
            const int32_t me_xy = s_pos[a];
            int count = 0;
            if (!wide) {
                const jl_v2s me = __builtin_bit_cast(jl_v2s, me_xy);
#pragma unroll 8
                for (int o = wave; o < A; o += nwaves) {
                    const jl_v2s d = me - __builtin_bit_cast(jl_v2s, s_pos[o]);
                    count += (int)((uint32_t)__builtin_amdgcn_sdot2(d, d, -(kCommRadiusSq + 1), false) >> 31);
                }
                if (a % nwaves == wave) count -= 1;
            } else {
                const int cx = (int16_t)(me_xy & 0xFFFF), cy = (int16_t)(me_xy >> 16);
                for (int o = wave; o < A; o += nwaves) {
                    const int ox = (int16_t)(s_pos[o] & 0xFFFF), oy = (int16_t)(s_pos[o] >> 16);
                    count += (o != a && wrap_dist2(cx - ox, cy - oy) <= kCommRadiusSq) ? 1 : 0;
                }
            }
            if (count) atomicAdd(&s_part[lane], count);
        }
    }
#pragma unroll
    for (int it = 0; it < kWinItems; ++it) {
        // bytes shift .. shift + 11 of the 32 bytes lo:hi
        const uint4 l = ok_lo[it] ? lo[it] : make_uint4(0u, 0u, 0u, 0u);
        const uint4 h = ok_hi[it] ? hi[it] : make_uint4(0u, 0u, 0u, 0u);
        const uint32_t w = (uint32_t)shift[it] >> 2, b = (uint32_t)shift[it] & 3u;
        const uint32_t d[8] = {l.x, l.y, l.z, l.w, h.x, h.y, h.z, h.w};
        uint32_t sel[4];
#pragma unroll
        for (int q = 0; q < 4; ++q)
            sel[q] = w == 0 ? d[q] : (w == 1 ? d[q + 1] : (w == 2 ? d[q + 2] : d[q + 3]));
        uint4 v;
        v.x = __builtin_amdgcn_alignbyte(sel[1], sel[0], b);
        v.y = __builtin_amdgcn_alignbyte(sel[2], sel[1], b);
        v.z = __builtin_amdgcn_alignbyte(sel[3], sel[2], b);
        v.w = 0u;
        *reinterpret_cast<uint4*>(s_win + dst[it]) = v;
    }
    __syncthreads();
    if (wave == 0) {
        const int a = e_begin + lane;
        long long count = 0;
        if (a < e_end) {
            if (s_valid[a]) {
                count = s_part[lane];
                m.edge_counts[base + a] = (int32_t)count;
            } else {
                count = m.edge_counts[base + a];
            }
        }
        for (int off = kWave / 2; off > 0; off >>= 1) count += __shfl_xor(count, off, kWave);
        if (lane == 0) m.env_edge_base[E + 1 + (size_t)env * parts + part] = count;
    }

    // Rows: one wavefront per agent; lane l owns patch cells l, l + 64,
    // l + 128 (p < 169) of the 13x13 patch, whose rows and columns 1..11 are
    // the window, and writes their four channel values into the wavefront's
    // LDS row (a lane past the patch on the third pass repeats its second
    // cell); the row then leaves as 16-byte stores in address order, so the
    // 128-byte lines it shares with the neighbouring rows are completed in the
    // cache instead of being written twice.
    float* my_row = reinterpret_cast<float*>(smem + L.row_off) + wave * kPygFeatures;
    int prow[3], pcol[3], pwc[3];
    bool pwin[3];
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        const int p = (lane + kWave * k) < kPygArea ? lane + kWave * k : lane + kWave;
        prow[k] = p / kPygDiam;
        pcol[k] = p - prow[k] * kPygDiam;
        pwin[k] = prow[k] >= 1 && prow[k] <= kDiam && pcol[k] >= 1 && pcol[k] <= kDiam;
        pwc[k] = pwin[k] ? (prow[k] - 1) * kWinRow + (pcol[k] - 1) : 0;
    }
    for (int a = e_begin + wave; a < e_end; a += nwaves) {
        if (!s_valid[a]) continue;
        const uint8_t* win = s_win + (a - e_begin) * kWinStride;
        const int32_t pos = s_pos[a];
        const int cx = (int16_t)(pos & 0xFFFF), cy = (int16_t)(pos >> 16);
        if (lane < 2) m.pyg_pos[(base + a) * 2 + lane] = (float)(lane ? cy : cx);
        // the centre is window cell (5, 5); 0 when the agent is off the map
        const int center = win[kRadius * kWinRow + kRadius];
        const int goal_p = s_part[kNodeEgos + a - e_begin];
        float* row = m.pyg_x + (base + a) * kPygFeatures;
#pragma unroll
        for (int k = 0; k < 3; ++k) {
            // window cell: off the map by more than one ring -> ctg 1; on the
            // ring around the map or an obstacle -> obstacle 1, ctg 1; free ->
            // agents bit and ctg from the energy difference (:438-478)
            const int p = prow[k] * kPygDiam + pcol[k];
            const int tx = cx + prow[k] - 6, ty = cy + pcol[k] - 6;
            const bool inmap = (uint32_t)tx < (uint32_t)W && (uint32_t)ty < (uint32_t)H;
            const bool ring = !inmap && (uint32_t)(tx + 1) <= (uint32_t)(W + 1) &&
                              (uint32_t)(ty + 1) <= (uint32_t)(H + 1);
            const int cell = inmap ? tx * H + ty : 0;
            const bool wall = inmap && ((s_st[cell >> 5] >> (cell & 31)) & 1u);
            const bool agent = (s_oc[cell >> 5] >> (cell & 31)) & 1u;
            const bool free_cell = inmap && !wall;
            int d = center - (int)win[pwc[k]];
            d = d < -10 ? -10 : (d > 10 ? 10 : d);
            const float cv = s_tenths[d + 10];
            my_row[p] = (pwin[k] && (ring || wall)) ? 1.0f : 0.0f;
            my_row[kPygArea + p] = (pwin[k] && free_cell && agent) ? 1.0f : 0.0f;
            my_row[2 * kPygArea + p] = p == goal_p ? 1.0f : 0.0f;
            my_row[3 * kPygArea + p] = pwin[k] ? (free_cell ? cv : 1.0f) : 0.0f;
        }
        wave_sync();
        // The row's whole 128-byte lines leave non-temporally (nothing reads
        // them again in this step, and out of the caches they leave the
        // energy windows and the edge pass's data there: C4 step 134.9 ->
        // 133.1 us); the partial lines at either end, which the neighbouring
        // rows complete, go through the L2 to be merged there.
        // (The two stores are written through different types: stores of one
        // type in both branches were merged by the compiler into one plain
        // store, dropping the non-temporal hint.)
        const float4* src = reinterpret_cast<const float4*>(my_row);
        float4* dst = reinterpret_cast<float4*>(row);
        const uintptr_t row_begin = reinterpret_cast<uintptr_t>(row);
        const uintptr_t row_end = row_begin + kPygFeatures * 4;
#pragma unroll
        for (int k = 0; k < 3; ++k) {
            const int q = lane + kWave * k;
            if (q < kPygFeatures / 4) {
                const uintptr_t line = reinterpret_cast<uintptr_t>(dst + q) & ~(uintptr_t)127;
                if (line >= row_begin && line + 128 <= row_end) {
                    __builtin_nontemporal_store(*reinterpret_cast<const jl_v4f*>(src + q),
                                                reinterpret_cast<jl_v4f*>(dst + q));
                } else {
                    dst[q] = src[q];
                }
            }
        }
        wave_sync();  // the row buffer is rewritten by the next agent
    }
}

// One workgroup: env totals (the sum of each env's slice totals, stored past
// the E + 1 bases) and their exclusive scan into the bases.
__global__ __launch_bounds__(1024) void env_scan_kernel(jl_magat_t m) {
    __shared__ long long s_wave[16];
    __shared__ long long s_carry;
    const int E = m.n_envs, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int parts = (m.n_agents + kNodeEgos - 1) / kNodeEgos;
    if (tid == 0) s_carry = 0;
    __syncthreads();
    for (int b0 = 0; b0 < E; b0 += 1024) {
        const int i = b0 + tid;
        long long v = 0;
        if (i < E)
            for (int p = 0; p < parts; ++p) v += m.env_edge_base[E + 1 + (size_t)i * parts + p];
        long long incl = v;
        for (int off = 1; off < 64; off <<= 1) {
            const long long t = __shfl_up(incl, off, 64);
            if (lane >= off) incl += t;
        }
        if (lane == 63) s_wave[wave] = incl;
        __syncthreads();
        long long before = s_carry;
        for (int k = 0; k < wave; ++k) before += s_wave[k];
        if (i < E) m.env_edge_base[i] = before + incl - v;
        __syncthreads();
        if (tid == 0) {
            long long t = 0;
            for (int k = 0; k < 16; ++k) t += s_wave[k];
            s_carry += t;
        }
        __syncthreads();
    }
    if (tid == 0) {
        m.env_edge_base[E] = s_carry;
        m.num_edges[0] = s_carry;
        m.edge_prefix[(size_t)E * m.n_agents] = s_carry;
    }
}

constexpr int kEdgeThreads = 256;
constexpr int kEdgeSources = 64;  // sources per edge workgroup
static_assert(kEdgeSources == kNodeEgos, "an edge slice is a node slice: the node pass's slice totals");
// Edge launches of at most this many slices sum the node pass's slice totals
// before their own (at most 32 loads per thread) instead of reading bases
// from env_scan_kernel, one launch less.
constexpr int kSummedSlices = 8192;
constexpr int kEdgeWaves = kEdgeThreads / kWave;
constexpr int kEdgeBlock = kEdgeSources / kEdgeWaves;  // consecutive sources per wavefront
constexpr int kEdgeUnroll = 4;    // 64-candidate chunks tested per step
constexpr int kEdgeSpan = kWave * kEdgeUnroll;
constexpr int kEdgeRing = 512;    // pending edges per wavefront: >= (kWave - 1) + kEdgeSpan
static_assert(kEdgeRing >= kWave - 1 + kEdgeSpan && (kEdgeRing & (kEdgeRing - 1)) == 0, "edge ring");

// This thread's share of the node pass's edge totals of the slices before
// `slice` (slices in (env, part) order, the order of the edge list); zero
// when the bases come from env_scan_kernel.
template <bool kSummed>
__device__ __forceinline__ long long slice_totals_before(const jl_magat_t& m, int slice) {
    long long before = 0;
    if constexpr (kSummed) {
        const int64_t* totals = m.env_edge_base + m.n_envs + 1;
#pragma unroll 8
        for (int j = threadIdx.x; j < slice; j += kEdgeThreads) before += totals[j];
    }
    return before;
}

// The last slice's end is the edge count: num_edges and the closing prefix
// (what env_scan_kernel writes when it runs).
__device__ __forceinline__ void write_edge_total(const jl_magat_t& m, int slice, long long total) {
    const int parts = (m.n_agents + kEdgeSources - 1) / kEdgeSources;
    if (slice == m.n_envs * parts - 1) {
        m.env_edge_base[m.n_envs] = total;
        m.num_edges[0] = total;
        m.edge_prefix[(size_t)m.n_envs * m.n_agents] = total;
    }
}

// Edge workgroup LDS: positions padded to a multiple of kEdgeSpan with cells
// far off every map (never within the radius), one ring of pending edges per
// wavefront, then the env's counts.
__host__ __device__ inline size_t edge_lds(int A) {
    const size_t padded = (size_t)(A + kEdgeSpan - 1) / kEdgeSpan * kEdgeSpan;
    return padded * 4 + (size_t)kEdgeWaves * kEdgeRing * 8 + (size_t)A * 4;
}

// Workgroup = (env, slice of kEdgeSources sources).  The env's positions and
// counts are staged in LDS in one round trip; the slice's first edge offsets
// are the env's scanned base plus the counts before the slice plus a scan
// over the slice.  Wavefront w takes kEdgeBlock consecutive sources, so its
// edges fill one contiguous range: each source tests the others kEdgeSpan at
// a time (32-bit differences: positions are any int16) and queues its
// neighbours, in id order, in the wavefront's LDS ring as (source, id,
// output offset); whenever 64 are queued they leave with every lane storing
// one edge (the neighbour count is about 9 at C4 density, so a store per
// source would run with a seventh of the lanes).  Edges are ordered by
// (source, destination id), the reference's order (stateless_step.cu:
// 854-935); each sits at its source's first offset plus its rank.
template <bool kSummed>
__global__ __launch_bounds__(kEdgeThreads) void edges_kernel(jl_magat_t m) {
    extern __shared__ __align__(16) int32_t s_xy[];  // (int16 x, int16 y) per agent, padded
    __shared__ long long s_wave[kEdgeWaves];
    __shared__ long long s_first[kEdgeSources];
    const int A = m.n_agents;
    const int padded = (A + kEdgeSpan - 1) / kEdgeSpan * kEdgeSpan;
    int2* s_ring = reinterpret_cast<int2*>(s_xy + padded);
    int32_t* s_cnt = reinterpret_cast<int32_t*>(s_ring + kEdgeWaves * kEdgeRing);
    const int parts = (A + kEdgeSources - 1) / kEdgeSources;
    const int env = blockIdx.x / parts;
    const int part = blockIdx.x - env * parts;
    const int s_begin = part * kEdgeSources;
    const int s_end = (s_begin + kEdgeSources) < A ? (s_begin + kEdgeSources) : A;
    const int tid = threadIdx.x, lane = tid & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);  // uniform per wavefront
    const size_t base = (size_t)env * A;
    long long before = slice_totals_before<kSummed>(m, env * parts + part);
    for (int a = tid; a < padded; a += kEdgeThreads) {
        int32_t xy = 0x40004000;  // padding: (16384, 16384)
        if (a < A) {
            const float2 p = reinterpret_cast<const float2*>(m.pyg_pos)[base + a];
            const int x = (int16_t)p.x, y = (int16_t)p.y;
            xy = (x & 0xFFFF) | (y << 16);
            s_cnt[a] = m.edge_counts[base + a];
        }
        s_xy[a] = xy;
    }
    const long long env_base = kSummed ? 0 : m.env_edge_base[env];
    __syncthreads();
    // counts of the env's agents before the slice (bases from env_scan_kernel)
    if constexpr (!kSummed)
        for (int a = tid; a < s_begin; a += kEdgeThreads) before += s_cnt[a];
    for (int off = kWave / 2; off > 0; off >>= 1) before += __shfl_xor(before, off, kWave);
    if (lane == 0) s_wave[wave] = before;
    __syncthreads();
    if (wave == 0) {
        long long first = env_base;
        for (int k = 0; k < kEdgeWaves; ++k) first += s_wave[k];
        const int a = s_begin + lane;
        const long long c = a < s_end ? s_cnt[a] : 0;
        long long incl = c;
        for (int off = 1; off < kWave; off <<= 1) {
            const long long t = __shfl_up(incl, off, kWave);
            if (lane >= off) incl += t;
        }
        if (a < s_end) {
            s_first[lane] = first + incl - c;
            m.edge_prefix[base + a] = first + incl - c;
        }
        if (kSummed && lane == kWave - 1) write_edge_total(m, env * parts + part, first + incl);
    }
    __syncthreads();
    const long long cap = m.edge_capacity;
    int64_t* dst_index = m.edge_index + cap;
    const long long slice_first = s_first[0];
    int2* ring = s_ring + wave * kEdgeRing;
    // Stores `count` queued edges from ring position `from`, one per lane.
    auto flush = [&](int from, int count) {
        wave_sync();
        if (lane < count) {
            const int2 ent = ring[(from + lane) & (kEdgeRing - 1)];
            const int o = ent.x & 0xFFFF, a = s_begin + (ent.x >> 16);
            const long long e = slice_first + ent.y;
            if (e >= 0 && e < cap) {
                const int32_t sxy = s_xy[a], oxy = s_xy[o];
                const int dx = (int16_t)(sxy & 0xFFFF) - (int16_t)(oxy & 0xFFFF);
                const int dy = (sxy >> 16) - (oxy >> 16);
                m.edge_index[e] = (int64_t)(base + a);
                dst_index[e] = (int64_t)(base + o);
                float* attr = m.edge_attr + e * 3;
                attr[0] = (float)dx;
                attr[1] = (float)dy;
                attr[2] = (float)((dx < 0 ? -dx : dx) + (dy < 0 ? -dy : dy));
            }
        }
    };
    const int a_begin = s_begin + wave * kEdgeBlock;
    const int a_end = (a_begin + kEdgeBlock) < s_end ? (a_begin + kEdgeBlock) : s_end;
    int head = 0, tail = 0;  // queued / stored edges of the wavefront (uniform)
    for (int a = a_begin; a < a_end; ++a) {
        const int sl = a - s_begin;
        const int first_rel = (int)(s_first[sl] - slice_first);
        const int32_t sxy = s_xy[a];
        const int cx = (int16_t)(sxy & 0xFFFF), cy = sxy >> 16;
        int n = 0;  // neighbours of a queued so far
        for (int o0 = 0; o0 < padded; o0 += kEdgeSpan) {
            const int32_t* row = s_xy + o0 + lane;
            uint64_t bal[kEdgeUnroll];
#pragma unroll
            for (int u = 0; u < kEdgeUnroll; ++u) {
                const int32_t oxy = row[u * kWave];
                const int dx = cx - (int16_t)(oxy & 0xFFFF);
                const int dy = cy - (oxy >> 16);
                bal[u] = __ballot(wrap_dist2(dx, dy) <= kCommRadiusSq && o0 + u * kWave + lane < A);
                // the source itself
                const int self = a - (o0 + u * kWave);
                if (self >= 0 && self < kWave) bal[u] &= ~(1ull << self);
            }
#pragma unroll
            for (int u = 0; u < kEdgeUnroll; ++u) {
                if (bal[u]) {
                    if ((bal[u] >> lane) & 1ull) {
                        const int rank = (int)__builtin_amdgcn_mbcnt_hi(
                            (uint32_t)(bal[u] >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bal[u], 0u));
                        ring[(head + rank) & (kEdgeRing - 1)] =
                            make_int2((sl << 16) | (o0 + u * kWave + lane), first_rel + n + rank);
                    }
                    const int c = __popcll(bal[u]);
                    head += c;
                    n += c;
                }
            }
            while (head - tail >= kWave) {
                flush(tail, kWave);
                tail += kWave;
            }
        }
    }
    if (head > tail) flush(tail, head - tail);
}

constexpr int kMaskMaxAgents = 1024;  // mask writer: at most 16 64-id chunks per source

// Mask writer LDS: per (64-id chunk, source of the slice) neighbour bits,
// then the positions padded to whole chunks, then the env's counts.
__host__ __device__ inline size_t edge_mask_lds(int A) {
    const size_t chunks = (size_t)(A + kWave - 1) / kWave;
    return chunks * kEdgeSources * 8 + chunks * kWave * 4 + (size_t)A * 4;
}

// Edge writer for envs of at most kMaskMaxAgents agents.  Workgroup = (env,
// slice of kEdgeSources sources), as above.  The env's positions and counts
// are loaded first, then (kSummed) this thread's share of the node pass's
// slice totals before the slice, which stay in flight, in registers, until
// the masks are built: the barriers in between order LDS only.  Lane l of
// wavefront w tests source s_begin + l against the ids of chunks w, w + 4,
// ... and keeps the neighbour bits of each 64-id chunk in LDS (with
// positions in [-8192, 8191] the differences and their squares fit packed
// int16 / one dot2 per pair; other envs take 32-bit arithmetic).  Then every
// thread takes output positions i = tid, tid + 256, ... of the slice's
// contiguous edge range: source = the last one whose first offset is <= i,
// destination = the (i - first)-th set bit of its mask, so consecutive lanes
// store consecutive edges.  A position past a source's recomputed neighbours
// (a skipped row whose stored count is stale) is left as it is.
constexpr int kMaskStage = kMaskMaxAgents / kEdgeThreads;  // staged agents per thread
constexpr int kMaskTotals = 8;  // slice totals per thread held in registers (2,048 slices)

template <bool kSummed>
__global__ __launch_bounds__(kEdgeThreads) void edges_mask_kernel(jl_magat_t m) {
    extern __shared__ __align__(16) uint64_t s_mask[];  // [chunk][source of the slice]
    __shared__ long long s_wave[kEdgeWaves];
    __shared__ int s_wide[kEdgeWaves];
    __shared__ int s_rel[kEdgeSources + 1];  // first edge of each source, relative to the slice's
    const int A = m.n_agents;
    const int chunks = (A + kWave - 1) / kWave;
    const int padded = chunks * kWave;
    int32_t* s_xy = reinterpret_cast<int32_t*>(s_mask + (size_t)chunks * kEdgeSources);
    int32_t* s_cnt = s_xy + padded;
    const int parts = (A + kEdgeSources - 1) / kEdgeSources;
    const int env = blockIdx.x / parts;
    const int part = blockIdx.x - env * parts;
    const int slice = blockIdx.x;
    const int s_begin = part * kEdgeSources;
    const int s_end = (s_begin + kEdgeSources) < A ? (s_begin + kEdgeSources) : A;
    const int tid = threadIdx.x, lane = tid & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);  // uniform per wavefront
    const size_t base = (size_t)env * A;
    // the env's positions and counts, then the slice totals (in that order:
    // loads complete in issue order), each at a clamped index without a branch
    float2 pos[kMaskStage];
    int32_t cnt[kMaskStage];
#pragma unroll
    for (int k = 0; k < kMaskStage; ++k) {
        const int a = tid + k * kEdgeThreads;
        const size_t g = base + (a < A ? a : A - 1);
        pos[k] = reinterpret_cast<const float2*>(m.pyg_pos)[g];
        cnt[k] = m.edge_counts[g];
    }
    long long tot[kMaskTotals];
    if constexpr (kSummed) {
        const int64_t* totals = m.env_edge_base + m.n_envs + 1;
#pragma unroll
        for (int k = 0; k < kMaskTotals; ++k) {
            const int j = tid + k * kEdgeThreads;
            const long long t = totals[j < slice ? j : 0];
            tot[k] = j < slice ? t : 0;
        }
    }
    // every load above in flight together, received here (one round trip):
    // left to itself the compiler moves loads into the branches that use them
#pragma unroll
    for (int k = 0; k < kMaskStage; ++k) asm volatile("" : "+v"(pos[k].x), "+v"(pos[k].y), "+v"(cnt[k]));
    if constexpr (kSummed) {
#pragma unroll
        for (int k = 0; k < kMaskTotals; ++k) asm volatile("" : "+v"(tot[k]));
    }
    int wide = 0;
#pragma unroll
    for (int k = 0; k < kMaskStage; ++k) {
        const int a = tid + k * kEdgeThreads;
        if (a < padded) {
            int32_t xy = 0x40004000;  // padding: (16384, 16384), never within the radius
            if (a < A) {
                const int x = (int16_t)pos[k].x, y = (int16_t)pos[k].y;
                wide |= (x < -8192 || x > 8191 || y < -8192 || y > 8191) ? 1 : 0;
                xy = (x & 0xFFFF) | (y << 16);
                s_cnt[a] = cnt[k];
            }
            s_xy[a] = xy;
        }
    }
    const long long env_base = kSummed ? 0 : m.env_edge_base[env];
    if (lane == 0) s_wide[wave] = 0;
    wave_sync();
    if (wide) s_wide[wave] = 1;
    lds_barrier();
    wide = 0;
#pragma unroll
    for (int k = 0; k < kEdgeWaves; ++k) wide |= s_wide[k];
    if (wave == 0) {
        // offsets of the slice's sources relative to its first edge
        const int a = s_begin + lane;
        const int c = a < s_end ? s_cnt[a] : 0;
        int incl = c;
        for (int off = 1; off < kWave; off <<= 1) {
            const int t = __shfl_up(incl, off, kWave);
            if (lane >= off) incl += t;
        }
        s_rel[lane] = incl - c;
        if (lane == kWave - 1) s_rel[kWave] = incl;
    }
    {
        const int a = s_begin + lane;
        const int32_t sxy = s_xy[a < s_end ? a : 0];
        for (int c = wave; c < chunks; c += kEdgeWaves) {
            const int32_t* row = s_xy + c * kWave;
            uint64_t bits = 0;
            if (!wide) {
                // dx * dx + dy * dy - (49 + 1) is negative exactly for a neighbour:
                // its sign bit is shifted in at bit 0 (alignbit), ids in
                // descending order, so id j ends at bit j
                const jl_v2s me = __builtin_bit_cast(jl_v2s, sxy);
                uint32_t half[2] = {0u, 0u};
#pragma unroll
                for (int h = 0; h < 2; ++h) {
#pragma unroll
                    for (int j = 31; j >= 0; --j) {
                        const jl_v2s d = me - __builtin_bit_cast(jl_v2s, row[h * 32 + j]);
                        const int t = __builtin_amdgcn_sdot2(d, d, -(kCommRadiusSq + 1), false);
                        half[h] = __builtin_amdgcn_alignbit(half[h], (uint32_t)t, 31);
                    }
                }
                bits = ((uint64_t)half[1] << 32) | half[0];
            } else {
                const int cx = (int16_t)(sxy & 0xFFFF), cy = sxy >> 16;
                for (int j = 0; j < kWave; ++j) {
                    const int32_t oxy = row[j];
                    const int dx = cx - (int16_t)(oxy & 0xFFFF), dy = cy - (oxy >> 16);
                    bits |= (uint64_t)(wrap_dist2(dx, dy) <= kCommRadiusSq) << j;
                }
            }
            const int self = a - c * kWave;
            if (self >= 0 && self < kWave) bits &= ~(1ull << self);
            // padding ids (past A) are never neighbours, whatever 32-bit wrap gives
            const int real = A - c * kWave;
            if (real < kWave) bits &= (1ull << real) - 1ull;
            s_mask[c * kEdgeSources + lane] = bits;
        }
    }
    // the slice's first edge: totals of the slices before it (kSummed), or
    // the env's scanned base plus the counts of its agents before the slice
    long long before = 0;
    if constexpr (kSummed) {
#pragma unroll
        for (int k = 0; k < kMaskTotals; ++k) before += tot[k];
        const int64_t* totals = m.env_edge_base + m.n_envs + 1;
        for (int j = tid + kMaskTotals * kEdgeThreads; j < slice; j += kEdgeThreads) before += totals[j];
    } else {
        for (int a = tid; a < s_begin; a += kEdgeThreads) before += s_cnt[a];
    }
    for (int off = kWave / 2; off > 0; off >>= 1) before += __shfl_xor(before, off, kWave);
    if (lane == 0) s_wave[wave] = before;
    lds_barrier();
    long long slice_first = env_base;
#pragma unroll
    for (int k = 0; k < kEdgeWaves; ++k) slice_first += s_wave[k];
    const int nsrc = s_end - s_begin;
    const int total = s_rel[nsrc];
    if (wave == 0) {
        const int a = s_begin + lane;
        if (a < s_end) m.edge_prefix[base + a] = slice_first + s_rel[lane];
        if (kSummed && lane == 0) write_edge_total(m, slice, slice_first + total);
    }
    const long long cap = m.edge_capacity;
    int64_t* dst_index = m.edge_index + cap;
    for (int i = tid; i < total; i += kEdgeThreads) {
        int sl = 0;  // the last source whose first edge is <= i
#pragma unroll
        for (int step = kEdgeSources / 2; step > 0; step >>= 1)
            if (sl + step < nsrc && s_rel[sl + step] <= i) sl += step;
        int k = i - s_rel[sl];
        int c = 0;
        uint64_t w = 0;
        for (; c < chunks; ++c) {
            w = s_mask[c * kEdgeSources + sl];
            const int pc = __popcll(w);
            if (k < pc) break;
            k -= pc;
        }
        if (c == chunks) continue;
        // the k-th set bit of w
        uint32_t v = (uint32_t)w;
        int bit = 0;
        const int plo = __popc(v);
        if (k >= plo) {
            k -= plo;
            v = (uint32_t)(w >> 32);
            bit = 32;
        }
#pragma unroll
        for (int half = 16; half > 0; half >>= 1) {
            const int p = __popc(v & ((1u << half) - 1u));
            if (k >= p) {
                k -= p;
                v >>= half;
                bit += half;
            }
        }
        const int a = s_begin + sl, o = c * kWave + bit;
        const long long e = slice_first + i;
        if (e < cap) {
            const int32_t sxy = s_xy[a], oxy = s_xy[o];
            const int dx = (int16_t)(sxy & 0xFFFF) - (int16_t)(oxy & 0xFFFF);
            const int dy = (sxy >> 16) - (oxy >> 16);
            // index rows leave as whole lines (consecutive lanes, consecutive edges)
            __builtin_nontemporal_store((int64_t)(base + a), &m.edge_index[e]);
            __builtin_nontemporal_store((int64_t)(base + o), &dst_index[e]);
            float* attr = m.edge_attr + e * 3;
            attr[0] = (float)dx;
            attr[1] = (float)dy;
            attr[2] = (float)((dx < 0 ? -dx : dx) + (dy < 0 ? -dy : dy));
        }
    }
}

int check_magat(const jl_magat_t* m) {
    if (!m || m->n_envs <= 0 || m->n_agents <= 0) return JL_ERR_ARG;
    if (!profile_ok(m->map_w, m->map_h)) return JL_ERR_PROFILE;
    if (m->n_agents > 16384 || m->n_envs > 65535) return JL_ERR_ARG;
    if (!m->grid_bits || !m->grid_ocp || !m->states) return JL_ERR_ARG;
    return JL_OK;
}

}  // namespace
}  // namespace jl

using namespace jl;

extern "C" int jl_magat_occupancy(const jl_magat_t* m, jl_stream_t stream) {
    int rc = check_magat(m);
    if (rc) return rc;
    const size_t lds = (size_t)m->map_w * m->map_h / 8;
    hipLaunchKernelGGL(occupancy_kernel, dim3(m->n_envs), dim3(256), lds, (hipStream_t)stream, *m);
    return launch_status();
}

extern "C" int jl_magat_nodes(const jl_magat_t* m, jl_stream_t stream) {
    int rc = check_magat(m);
    if (rc) return rc;
    if (!m->energy || !m->pyg_x || !m->pyg_pos || !m->edge_counts || !m->env_edge_base)
        return JL_ERR_ARG;
    const NodeLayout L = node_layout(m->n_agents, m->map_w, m->map_h);
    const unsigned parts = (unsigned)((m->n_agents + kNodeEgos - 1) / kNodeEgos);
    JL_DISPATCH_H(m->map_h, {
        if (!lds_fits<&nodes_kernel<H>>(L.total)) return JL_ERR_AGENTS;
        hipLaunchKernelGGL((nodes_kernel<H>), dim3((unsigned)m->n_envs * parts), dim3(kNodeThreads),
                           L.total, (hipStream_t)stream, *m);
    });
    return launch_status();
}

extern "C" int jl_magat_edges(const jl_magat_t* m, jl_stream_t stream) {
    int rc = check_magat(m);
    if (rc) return rc;
    if (!m->edge_counts || !m->edge_prefix || !m->num_edges || !m->edge_index || !m->edge_attr ||
        !m->env_edge_base || !m->pyg_pos)
        return JL_ERR_ARG;
    if (m->edge_capacity < (int64_t)m->n_envs * m->n_agents * (m->n_agents - 1))
        return JL_ERR_CAPACITY;
    const unsigned eparts = (unsigned)((m->n_agents + kEdgeSources - 1) / kEdgeSources);
    const size_t slices = (size_t)m->n_envs * eparts;
    const bool summed = slices <= (size_t)kSummedSlices;
    const size_t elds = edge_lds(m->n_agents);
    if (m->n_agents > kMaskMaxAgents && !(summed ? lds_fits<&edges_kernel<true>>(elds)
                                                 : lds_fits<&edges_kernel<false>>(elds)))
        return JL_ERR_AGENTS;
    if (m->n_agents <= kMaskMaxAgents &&
        !(summed ? lds_fits<&edges_mask_kernel<true>>(edge_mask_lds(m->n_agents))
                 : lds_fits<&edges_mask_kernel<false>>(edge_mask_lds(m->n_agents))))
        return JL_ERR_AGENTS;
    if (!summed) {
        hipLaunchKernelGGL(env_scan_kernel, dim3(1), dim3(1024), 0, (hipStream_t)stream, *m);
        rc = launch_status();
        if (rc) return rc;
    }
    const dim3 grid((unsigned)slices), block(kEdgeThreads);
    if (m->n_agents <= kMaskMaxAgents) {
        if (summed) {
            hipLaunchKernelGGL(edges_mask_kernel<true>, grid, block, edge_mask_lds(m->n_agents),
                               (hipStream_t)stream, *m);
        } else {
            hipLaunchKernelGGL(edges_mask_kernel<false>, grid, block, edge_mask_lds(m->n_agents),
                               (hipStream_t)stream, *m);
        }
    } else if (summed) {
        hipLaunchKernelGGL(edges_kernel<true>, grid, block, elds, (hipStream_t)stream, *m);
    } else {
        hipLaunchKernelGGL(edges_kernel<false>, grid, block, elds, (hipStream_t)stream, *m);
    }
    return launch_status();
}
