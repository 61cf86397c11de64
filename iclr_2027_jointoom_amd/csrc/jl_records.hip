// jl_records.hip - expansion of compact expert records into stage rows.
//
// A frozen expert archive (frozen_stage_source.py:23-59) stores every stage as
// uint16 rows of 8 (MAGAT) or 13 (MAPF-GPT) columns: 16 or 26 bytes per agent
// and step.  Most of a row is implied by the producers that write it
// (mapf_gpt_online.py:215-258 with mapf_gpt_schema.py:43-66, 118-126;
// topology_async.py:90-102, 235-278):
//   env, agent          the row's place in the env-major stage
//   goal                fixed for an episode, changed only when it restarts
//   refresh flag        1 for every agent of an env at its episode start, else 0
//   history (13 cols)   the env's previous actions of the running episode,
//                       oldest first, 5 = none yet
// so the compact record carries only the position (2 x uint16) and the action
// (uint8) of each agent and step, plus one episode-start byte per env and the
// goals of the envs that start an episode.  This kernel rebuilds the full rows
// on the device, keeping the running goals and histories in HBM between
// stages: one thread per agent, rows assembled in LDS and written out as one
// contiguous, 16-byte-vectorised range per workgroup.
#include <cstring>

#include "jl_common.h"

namespace jl {
namespace {

constexpr int kRecThreads = 256;
constexpr uint64_t kEmptyHistory = 0x0505050505ull;  // 5 actions of value 5

template <int F>
__global__ __launch_bounds__(kRecThreads) void expand_records_kernel(
    const uint32_t* __restrict__ positions,     // [N] x | y << 16
    const uint8_t* __restrict__ actions,        // [N]
    const uint8_t* __restrict__ episode_start,  // [E]
    const uint32_t* __restrict__ new_goals,     // [N] x | y << 16
    uint32_t* __restrict__ goals,               // [N] running goals
    uint64_t* __restrict__ history,             // [N] bytes 0..4 = actions, oldest first
    uint16_t* __restrict__ rows,                // [N, F]
    int n, int n_agents, int vec_store) {
    __shared__ __align__(16) uint16_t s_rows[kRecThreads * F];
    const int tid = threadIdx.x;
    const int base = blockIdx.x * kRecThreads;
    const int nb = min(kRecThreads, n - base);
    if (tid < nb) {
        const int i = base + tid;
        const int env = i / n_agents;
        const int agent = i - env * n_agents;
        // every load of the common (continuing) case is issued at once; only
        // agents whose episode starts here take a second round trip
        const uint32_t pos = positions[i];
        const uint32_t act = actions[i];
        const uint32_t start = episode_start[env] != 0 ? 1u : 0u;
        uint32_t goal = goals[i];
        uint64_t h_prev = 0;
        if constexpr (F == 13) h_prev = history[i];
        if (start) {
            goal = new_goals[i];
            goals[i] = goal;
        }
        uint16_t* r = s_rows + tid * F;
        r[0] = (uint16_t)env;
        r[1] = (uint16_t)agent;
        r[2] = (uint16_t)(pos & 0xFFFFu);
        r[3] = (uint16_t)(pos >> 16);
        r[4] = (uint16_t)(goal & 0xFFFFu);
        r[5] = (uint16_t)(goal >> 16);
        r[6] = (uint16_t)act;
        r[7] = (uint16_t)start;
        if constexpr (F == 13) {
            // the row holds the history before this step's action is appended
            const uint64_t h = start ? kEmptyHistory : h_prev;
#pragma unroll
            for (int k = 0; k < 5; ++k) r[8 + k] = (uint16_t)((h >> (8 * k)) & 0xFFu);
            history[i] = ((h >> 8) & 0xFFFFFFFFull) | ((uint64_t)act << 32);
        }
    }
    __syncthreads();
    // the workgroup's rows are one contiguous range of nb * F values
    const int count = nb * F;
    uint16_t* out = rows + (int64_t)base * F;
    int k0 = 0;
    if (vec_store) {
        const int n16 = count >> 3;
        const uint4* src = reinterpret_cast<const uint4*>(s_rows);
        uint4* dst = reinterpret_cast<uint4*>(out);
        for (int k = tid; k < n16; k += kRecThreads) dst[k] = src[k];
        k0 = n16 << 3;
    }
    for (int k = k0 + tid; k < count; k += kRecThreads) out[k] = s_rows[k];
}

}  // namespace
}  // namespace jl

static int check_records(const jl_records_t* r) {
    using namespace jl;
    if (!r || r->n_envs <= 0 || r->n_agents <= 0) return JL_ERR_ARG;
    if (r->features != 8 && r->features != 13) return JL_ERR_ARG;
    const int64_t n64 = (int64_t)r->n_envs * r->n_agents;
    if (n64 > (int64_t)0x7FFFFFFF - kRecThreads || r->n_envs > 65536 || r->n_agents > 65536)
        return JL_ERR_ARG;
    if (!r->positions || !r->actions || !r->episode_start || !r->new_goals || !r->goals ||
        !r->rows)
        return JL_ERR_ARG;
    if (r->features == 13 && !r->history) return JL_ERR_ARG;
    // positions and goals are read as one 32-bit word per agent, histories as 64 bits
    if (((uintptr_t)r->positions & 3) || ((uintptr_t)r->new_goals & 3) ||
        ((uintptr_t)r->goals & 3) || ((uintptr_t)r->history & 7) || ((uintptr_t)r->rows & 1))
        return JL_ERR_ARG;
    return JL_OK;
}

static int launch_expand(const jl_records_t* r, hipStream_t s) {
    using namespace jl;
    const int n = r->n_envs * r->n_agents;
    const int grid = (n + kRecThreads - 1) / kRecThreads;
    const int vec = ((uintptr_t)r->rows & 15) == 0 ? 1 : 0;
    const uint32_t* pos = reinterpret_cast<const uint32_t*>(r->positions);
    const uint32_t* ng = reinterpret_cast<const uint32_t*>(r->new_goals);
    uint32_t* g = reinterpret_cast<uint32_t*>(r->goals);
    uint64_t* h = reinterpret_cast<uint64_t*>(r->history);
    uint16_t* rows = reinterpret_cast<uint16_t*>(r->rows);
    if (r->features == 13) {
        hipLaunchKernelGGL(expand_records_kernel<13>, dim3(grid), dim3(kRecThreads), 0, s, pos,
                           r->actions, r->episode_start, ng, g, h, rows, n, r->n_agents, vec);
    } else {
        hipLaunchKernelGGL(expand_records_kernel<8>, dim3(grid), dim3(kRecThreads), 0, s, pos,
                           r->actions, r->episode_start, ng, g, h, rows, n, r->n_agents, vec);
    }
    return launch_status();
}

extern "C" int jl_expand_records(const jl_records_t* r, jl_stream_t stream) {
    const int rc = check_records(r);
    if (rc) return rc;
    return launch_expand(r, (hipStream_t)stream);
}

// Byte layout of a compact stage slot (N agents, E envs): positions [0, 4N),
// actions [4N, 5N), episode-start flags [5N, 5N + E), goals from the next
// 16-byte boundary, 4N bytes.
static int64_t slot_goals_offset(int64_t n, int64_t e) { return (5 * n + e + 15) / 16 * 16; }

extern "C" int jl_ring_upload_compact(jl_stage_upload_t* u, jl_stream_t stream) {
    using namespace jl;
    if (!u || !u->host_slot || !u->staging || !u->device_slot || !u->staging_free) return JL_ERR_ARG;
    jl_records_t r = u->records;
    r.positions = nullptr;  // set below from the device slot
    const int64_t n = (int64_t)r.n_envs * r.n_agents, e = r.n_envs;
    if (r.n_envs <= 0 || r.n_agents <= 0) return JL_ERR_ARG;
    const int64_t head = 5 * n + e, goff = slot_goals_offset(n, e);
    if (u->slot_bytes < goff + 4 * n) return JL_ERR_ARG;
    hipStream_t s = (hipStream_t)stream;
    // the staging buffer's previous upload must have left it
    int rc = status(hipEventSynchronize((hipEvent_t)u->staging_free));
    if (rc) return rc;
    std::memcpy(u->staging, u->host_slot, (size_t)head);
    // goals of the envs that start an episode: one range from the first to the last
    const uint8_t* starts = u->host_slot + 5 * n;
    int64_t lo = -1, hi = -1;
    for (int64_t k = 0; k < e; ++k) {
        if (starts[k]) {
            if (lo < 0) lo = k;
            hi = k + 1;
        }
    }
    int64_t g0 = 0, g1 = 0;
    if (lo >= 0) {
        g0 = goff + lo * 4 * r.n_agents;
        g1 = goff + hi * 4 * r.n_agents;
        std::memcpy(u->staging + g0, u->host_slot + g0, (size_t)(g1 - g0));
    }
    rc = status(hipMemcpyAsync(u->device_slot, u->staging, (size_t)head, hipMemcpyHostToDevice, s));
    if (rc) return rc;
    if (g1 > g0) {
        rc = status(hipMemcpyAsync(u->device_slot + g0, u->staging + g0, (size_t)(g1 - g0),
                                   hipMemcpyHostToDevice, s));
        if (rc) return rc;
    }
    rc = status(hipEventRecord((hipEvent_t)u->staging_free, s));
    if (rc) return rc;
    if (u->rows_free) {
        rc = status(hipStreamWaitEvent(s, (hipEvent_t)u->rows_free, 0));
        if (rc) return rc;
    }
    r.positions = reinterpret_cast<const uint16_t*>(u->device_slot);
    r.actions = u->device_slot + 4 * n;
    r.episode_start = u->device_slot + 5 * n;
    r.new_goals = reinterpret_cast<const uint16_t*>(u->device_slot + goff);
    rc = check_records(&r);
    if (rc) return rc;
    rc = launch_expand(&r, s);
    if (rc) return rc;
    if (u->done) {
        rc = status(hipEventRecord((hipEvent_t)u->done, s));
        if (rc) return rc;
    }
    u->bytes_uploaded = head + (g1 - g0);
    return JL_OK;
}
