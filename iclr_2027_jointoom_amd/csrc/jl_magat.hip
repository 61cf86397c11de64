// jl_magat.hip - MAGAT node features and neighbour graph for gfx950.
//
// nodes: one workgroup per env.  The env's static and occupancy bitmaps,
// agent positions and goals are staged in LDS; the 11x11 energy windows of a
// chunk of agents are gathered into LDS with all loads independent; then one
// wavefront writes each agent's 676-float row with 16-byte coalesced stores
// (the reference zero-fills the row and rewrites it one float per thread,
// 128_agents_map_stateless_step.cu:414-421, 438-478).  The clamped ctg
// value is one of 21 float constants k/10 (the IEEE quotients), so no
// division is evaluated on the device.
// edges: per-env edge totals -> one-workgroup scan -> per-env writer that
// scans its agents' counts in LDS and emits edges sorted by (source,
// destination id) (grid_world_cuda.cu:17-110, stateless_step.cu:854-935).
#include "jl_common.h"

namespace jl {
namespace {

constexpr int kNodeThreads = 256;

// (float)k / 10.0f rounded to nearest even, k = -10..10.
__device__ __constant__ float kTenths[21] = {-1.0f, -0.9f, -0.8f, -0.7f, -0.6f, -0.5f, -0.4f,
                                            -0.3f, -0.2f, -0.1f, 0.0f,  0.1f,  0.2f,  0.3f,
                                            0.4f,  0.5f,  0.6f,  0.7f,  0.8f,  0.9f,  1.0f};

__device__ __forceinline__ float ctg_value(int center, int cell) {
    const int d = center - cell;
    if (d >= 10) return 1.0f;
    if (d <= -10) return -1.0f;
    return kTenths[d + 10];
}

// Exact round-half-even of num / den, den > 0 (stateless_step.cu:120-138).
__device__ __forceinline__ int round_half_even(int num, int den) {
    const bool neg = num < 0;
    const unsigned mag = neg ? (unsigned)(-num) : (unsigned)num;
    unsigned q = mag / (unsigned)den;
    const unsigned r = mag - q * (unsigned)den;
    if (2 * r > (unsigned)den || (2 * r == (unsigned)den && (q & 1u))) ++q;
    return neg ? -(int)q : (int)q;
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
    int chunk;
    size_t st_off, oc_off, pos_off, goal_off, valid_off, win_off, total;
};

__host__ __device__ inline size_t a16n(size_t v) { return (v + 15) & ~(size_t)15; }

__host__ __device__ inline NodeLayout node_layout(int A, int W, int H) {
    NodeLayout L;
    L.chunk = A < 256 ? A : 256;
    size_t o = 0;
    L.st_off = o;
    o = a16n(o + (size_t)W * H / 8);
    L.oc_off = o;
    o = a16n(o + (size_t)W * H / 8);
    L.pos_off = o;
    o = a16n(o + (size_t)A * 4);
    L.goal_off = o;
    o = a16n(o + (size_t)A * 4);
    L.valid_off = o;
    o = a16n(o + (size_t)A);
    L.win_off = o;
    o = a16n(o + (size_t)L.chunk * 124);  // 121 window bytes + center, padded
    L.total = o;
    return L;
}

template <int H>
__global__ __launch_bounds__(kNodeThreads) void nodes_kernel(jl_magat_t m) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int env = blockIdx.x, A = m.n_agents, W = m.map_w, E = m.n_envs;
    const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
    constexpr int nwaves = kNodeThreads / kWave;
    const NodeLayout L = node_layout(A, W, H);
    uint32_t* s_st = reinterpret_cast<uint32_t*>(smem + L.st_off);
    uint32_t* s_oc = reinterpret_cast<uint32_t*>(smem + L.oc_off);
    int32_t* s_pos = reinterpret_cast<int32_t*>(smem + L.pos_off);  // (int16 x, int16 y)
    int32_t* s_goal = reinterpret_cast<int32_t*>(smem + L.goal_off);
    uint8_t* s_valid = smem + L.valid_off;
    uint8_t* s_win = smem + L.win_off;
    const int words = W * H / 32;
    const size_t cells = (size_t)W * H;
    const size_t base = (size_t)env * A;

    for (int k = tid; k < words; k += kNodeThreads) {
        s_st[k] = m.grid_bits[(size_t)env * words + k];
        s_oc[k] = m.grid_ocp[(size_t)env * words + k];
    }
    for (int a = tid; a < A; a += kNodeThreads) {
        const uint4 r = *reinterpret_cast<const uint4*>(m.states + (base + a) * 8);
        s_pos[a] = (int32_t)r.y;
        s_goal[a] = (int32_t)r.z;
        s_valid[a] = (r.x & 0xFFFFu) < (uint32_t)E ? 1 : 0;
    }
    __syncthreads();

    // Edge counts: others within squared radius 49, all rows of the env block
    // (stateless_step.cu:511-520).  Totals per env feed the scan; rows that
    // are skipped keep their previous count, which the scan still reads.
    int64_t env_total = 0;
    for (int a = tid; a < A; a += kNodeThreads) {
        int count;
        if (s_valid[a]) {
            const int cx = (int16_t)(s_pos[a] & 0xFFFF), cy = (int16_t)(s_pos[a] >> 16);
            count = 0;
            for (int o = 0; o < A; ++o) {
                const int ox = (int16_t)(s_pos[o] & 0xFFFF), oy = (int16_t)(s_pos[o] >> 16);
                const int dx = cx - ox, dy = cy - oy;
                count += (o != a && dx * dx + dy * dy <= kCommRadiusSq) ? 1 : 0;
            }
            m.edge_counts[base + a] = count;
            m.pyg_pos[(base + a) * 2] = (float)cx;
            m.pyg_pos[(base + a) * 2 + 1] = (float)cy;
        } else {
            count = m.edge_counts[base + a];
        }
        env_total += count;
    }
    {
        // workgroup sum of env_total
        __shared__ long long s_part[kNodeThreads / kWave];
        long long v = env_total;
        for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
        if (lane == 0) s_part[wave] = v;
        __syncthreads();
        if (tid == 0) {
            long long t = 0;
            for (int k = 0; k < nwaves; ++k) t += s_part[k];
            m.env_edge_base[env] = t;
        }
    }

    for (int c0 = 0; c0 < A; c0 += L.chunk) {
        const int nch = (A - c0) < L.chunk ? (A - c0) : L.chunk;
        // energy windows (11x11) + centre of the chunk
        const int pairs = nch * 122;
#pragma unroll 4
        for (int p = tid; p < pairs; p += kNodeThreads) {
            const int el = p / 122;
            const int c = p - el * 122;
            const int a = c0 + el;
            const int cx = (int16_t)(s_pos[a] & 0xFFFF), cy = (int16_t)(s_pos[a] >> 16);
            int x, y;
            if (c < 121) {
                x = cx + c / kDiam - kRadius;
                y = cy + c % kDiam - kRadius;
            } else {
                x = cx;
                y = cy;
            }
            uint8_t v = 0;
            if (s_valid[a] && x >= 0 && x < W && y >= 0 && y < H)
                v = m.energy[(base + a) * cells + (size_t)(x * H + y)];
            s_win[el * 124 + c] = v;
        }
        __syncthreads();
        for (int el = wave; el < nch; el += nwaves) {
            const int a = c0 + el;
            if (!s_valid[a]) continue;
            const int cx = (int16_t)(s_pos[a] & 0xFFFF), cy = (int16_t)(s_pos[a] >> 16);
            const int gx = (int16_t)(s_goal[a] & 0xFFFF), gy = (int16_t)(s_goal[a] >> 16);
            const bool center_in = cx >= 0 && cx < W && cy >= 0 && cy < H;
            const int center = center_in ? (int)s_win[el * 124 + 121] : 0;
            // goal cell of the 13x13 patch (stateless_step.cu:480-509)
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
            const int goal_p = fx * kPygDiam + fy;
            float* row = m.pyg_x + (base + a) * kPygFeatures;
            for (int q = lane; q < kPygFeatures / 4; q += kWave) {
                float v4[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int k = 4 * q + j;
                    const int ch = k / kPygArea;
                    const int p = k - ch * kPygArea;
                    float v = 0.0f;
                    if (ch == 2) {
                        v = p == goal_p ? 1.0f : 0.0f;
                    } else {
                        const int pr = p / kPygDiam, pc = p - pr * kPygDiam;
                        if (pr >= 1 && pr <= 11 && pc >= 1 && pc <= 11) {
                            const int tx = cx + pr - 6;
                            const int ty = cy + pc - 6;
                            float obs = 0.0f, occ = 0.0f, ctg = 0.0f;
                            if (tx < -1 || tx > W || ty < -1 || ty > H) {
                                ctg = 1.0f;
                            } else if (tx == -1 || tx == W || ty == -1 || ty == H) {
                                obs = 1.0f;
                                ctg = 1.0f;
                            } else {
                                const int cell = tx * H + ty;
                                if ((s_st[cell >> 5] >> (cell & 31)) & 1u) {
                                    obs = 1.0f;
                                    ctg = 1.0f;
                                } else {
                                    if ((s_oc[cell >> 5] >> (cell & 31)) & 1u) occ = 1.0f;
                                    ctg = ctg_value(center,
                                                    (int)s_win[el * 124 + (pr - 1) * kDiam + (pc - 1)]);
                                }
                            }
                            v = ch == 0 ? obs : (ch == 1 ? occ : ctg);
                        }
                    }
                    v4[j] = v;
                }
                reinterpret_cast<float4*>(row)[q] = make_float4(v4[0], v4[1], v4[2], v4[3]);
            }
        }
        __syncthreads();
    }
}

// One workgroup: exclusive scan of the E env totals (in place, E+1 entries).
__global__ __launch_bounds__(1024) void env_scan_kernel(jl_magat_t m) {
    __shared__ long long s_wave[16];
    __shared__ long long s_carry;
    const int E = m.n_envs, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (tid == 0) s_carry = 0;
    __syncthreads();
    for (int b0 = 0; b0 < E; b0 += 1024) {
        const int i = b0 + tid;
        const long long v = i < E ? m.env_edge_base[i] : 0;
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

__global__ __launch_bounds__(256) void edges_kernel(jl_magat_t m) {
    extern __shared__ __align__(16) int32_t s_xy[];  // (int16 x, int16 y) per agent
    __shared__ long long s_wave[4];
    const int env = blockIdx.x, A = m.n_agents;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const size_t base = (size_t)env * A;
    for (int a = tid; a < A; a += 256) {
        const int x = (int16_t)m.pyg_pos[(base + a) * 2];
        const int y = (int16_t)m.pyg_pos[(base + a) * 2 + 1];
        s_xy[a] = (x & 0xFFFF) | (y << 16);
    }
    long long carry = m.env_edge_base[env];
    for (int a0 = 0; a0 < A; a0 += 256) {
        const int a = a0 + tid;
        const long long c = a < A ? m.edge_counts[base + a] : 0;
        long long incl = c;
        for (int off = 1; off < 64; off <<= 1) {
            const long long t = __shfl_up(incl, off, 64);
            if (lane >= off) incl += t;
        }
        if (lane == 63) s_wave[wave] = incl;
        __syncthreads();
        long long before = carry;
        for (int k = 0; k < wave; ++k) before += s_wave[k];
        const long long first = before + incl - c;
        if (a < A) {
            m.edge_prefix[base + a] = first;
            const int cx = (int16_t)(s_xy[a] & 0xFFFF), cy = s_xy[a] >> 16;
            long long out = first;
            const long long cap = m.edge_capacity;
            for (int o = 0; o < A; ++o) {
                if (o == a) continue;
                const int dx = cx - (int16_t)(s_xy[o] & 0xFFFF);
                const int dy = cy - (s_xy[o] >> 16);
                if (dx * dx + dy * dy > kCommRadiusSq) continue;
                if (out >= 0 && out < cap) {
                    m.edge_index[out] = (int64_t)(base + a);
                    m.edge_index[cap + out] = (int64_t)(base + o);
                    m.edge_attr[out * 3] = (float)dx;
                    m.edge_attr[out * 3 + 1] = (float)dy;
                    m.edge_attr[out * 3 + 2] = (float)((dx < 0 ? -dx : dx) + (dy < 0 ? -dy : dy));
                }
                ++out;
            }
        }
        __syncthreads();
        carry += s_wave[0] + s_wave[1] + s_wave[2] + s_wave[3];
        __syncthreads();
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
    if (L.total > 160 * 1024) return JL_ERR_ARG;
    JL_DISPATCH_H(m->map_h, {
        hipLaunchKernelGGL((nodes_kernel<H>), dim3(m->n_envs), dim3(kNodeThreads), L.total,
                           (hipStream_t)stream, *m);
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
    hipLaunchKernelGGL(env_scan_kernel, dim3(1), dim3(1024), 0, (hipStream_t)stream, *m);
    rc = launch_status();
    if (rc) return rc;
    hipLaunchKernelGGL(edges_kernel, dim3(m->n_envs), dim3(256), (size_t)m->n_agents * 4,
                       (hipStream_t)stream, *m);
    return launch_status();
}
