// jl_stream.hip - HBM streaming probe: the bandwidth a plain streaming kernel
// reaches on this device (16-byte non-temporal loads, non-temporal or plain
// stores, grid-stride or one contiguous chunk per workgroup, four accesses in
// flight per thread), the "achievable" denominator of the
// measurement beside the published peak.  Not part of the hot path: it is
// built into libjl_bench.so, which only the benchmark loads.
//
//   int jl_hbm_stream(int32_t kind, const void* src, void* dst, int64_t bytes,
//                     uint32_t* sink, int32_t workgroups, jl_stream_t stream);
//
// One launch moving `bytes` (a multiple of 16, 16-byte aligned buffers) with
// 16-byte accesses (non-temporal loads): kind 0 = read `src` only (sink: one
// word per workgroup, written only in a practically impossible case, so the
// reads are kept), 1 = write `dst` only, 2 = copy `src` to `dst`
// (non-temporal stores), 3 and 4 = write and copy with plain stores, over
// `workgroups` 256-thread workgroups striding the whole range; kinds 5-9 are
// kinds 0-4 with each workgroup streaming one contiguous chunk instead (5
// read, 6 and 7 write and copy non-temporal, 8 and 9 write and copy plain).
// Kind 10 reads one 16-byte word at the start of every 256-byte block of
// `src` (bytes a multiple of 256), for the HBM fetch granularity under the
// FETCH_SIZE counter.  Returns JL_OK or JL_ERR_ARG.
#include "jl_common.h"

namespace jl {
namespace {

constexpr int kStreamThreads = 256;
constexpr int kStreamUnroll = 4;

typedef unsigned int v4u __attribute__((ext_vector_type(4)));

template <bool kNt>
__device__ __forceinline__ void put(v4u v, v4u* p) {
    if (kNt) {
        __builtin_nontemporal_store(v, p);
    } else {
        *p = v;
    }
}

// kKind: 0 read only (the XOR of everything read lands in sink[0] per
// workgroup, so the loads are kept), 1 write only, 2 copy; kNt: non-temporal
// (streaming) stores, else plain ones.
template <int kKind, bool kNt>
__global__ __launch_bounds__(kStreamThreads) void stream_kernel(const v4u* __restrict__ src,
                                                                v4u* __restrict__ dst, size_t n,
                                                                unsigned int* __restrict__ sink) {
    const size_t stride = (size_t)gridDim.x * kStreamThreads;
    size_t i = (size_t)blockIdx.x * kStreamThreads + threadIdx.x;
    v4u acc = {0u, 0u, 0u, 0u};
    const v4u fill = {0x01010101u, 0x02020202u, 0x03030303u, (unsigned)blockIdx.x};
    for (; i + (kStreamUnroll - 1) * stride < n; i += kStreamUnroll * stride) {
        v4u v[kStreamUnroll];
        if (kKind != 1) {
#pragma unroll
            for (int u = 0; u < kStreamUnroll; ++u) v[u] = __builtin_nontemporal_load(src + i + u * stride);
        }
#pragma unroll
        for (int u = 0; u < kStreamUnroll; ++u) {
            if (kKind == 0) acc ^= v[u];
            if (kKind == 1) put<kNt>(fill, dst + i + u * stride);
            if (kKind == 2) put<kNt>(v[u], dst + i + u * stride);
        }
    }
    for (; i < n; i += stride) {
        if (kKind == 0) acc ^= __builtin_nontemporal_load(src + i);
        if (kKind == 1) put<kNt>(fill, dst + i);
        if (kKind == 2) put<kNt>(__builtin_nontemporal_load(src + i), dst + i);
    }
    if (kKind == 0) {
        const unsigned int x = acc.x ^ acc.y ^ acc.z ^ acc.w;
        if (x == 0x9E3779B9u) sink[blockIdx.x] = x;  // keeps the loads; almost never taken
    }
}

// The same with each workgroup streaming one contiguous chunk of n / grid
// 16-byte words (the threads of a workgroup on consecutive words, four
// 4 KB rounds in flight).
template <int kKind, bool kNt>
__global__ __launch_bounds__(kStreamThreads) void chunk_kernel(const v4u* __restrict__ src,
                                                               v4u* __restrict__ dst, size_t n,
                                                               unsigned int* __restrict__ sink) {
    const size_t per = (n + gridDim.x - 1) / gridDim.x;
    const size_t begin = (size_t)blockIdx.x * per;
    const size_t end = begin + per < n ? begin + per : n;
    size_t i = begin + threadIdx.x;
    v4u acc = {0u, 0u, 0u, 0u};
    const v4u fill = {0x01010101u, 0x02020202u, 0x03030303u, (unsigned)blockIdx.x};
    constexpr size_t step = kStreamThreads;
    for (; i + (kStreamUnroll - 1) * step < end; i += kStreamUnroll * step) {
        v4u v[kStreamUnroll];
        if (kKind != 1) {
#pragma unroll
            for (int u = 0; u < kStreamUnroll; ++u) v[u] = __builtin_nontemporal_load(src + i + u * step);
        }
#pragma unroll
        for (int u = 0; u < kStreamUnroll; ++u) {
            if (kKind == 0) acc ^= v[u];
            if (kKind == 1) put<kNt>(fill, dst + i + u * step);
            if (kKind == 2) put<kNt>(v[u], dst + i + u * step);
        }
    }
    for (; i < end; i += step) {
        if (kKind == 0) acc ^= __builtin_nontemporal_load(src + i);
        if (kKind == 1) put<kNt>(fill, dst + i);
        if (kKind == 2) put<kNt>(__builtin_nontemporal_load(src + i), dst + i);
    }
    if (kKind == 0) {
        const unsigned int x = acc.x ^ acc.y ^ acc.z ^ acc.w;
        if (x == 0x9E3779B9u) sink[blockIdx.x] = x;  // keeps the loads; almost never taken
    }
}

// One 16-byte load at the start of every 256-byte block of the range (the
// XOR lands in sink as in kind 0): with the FETCH_SIZE counter, the bytes the
// L2 fetches from HBM for an isolated 16-byte read.
__global__ __launch_bounds__(kStreamThreads) void sparse_read_kernel(const v4u* __restrict__ src, size_t blocks,
                                                                     unsigned int* __restrict__ sink) {
    const size_t stride = (size_t)gridDim.x * kStreamThreads;
    v4u acc = {0u, 0u, 0u, 0u};
    for (size_t i = (size_t)blockIdx.x * kStreamThreads + threadIdx.x; i < blocks; i += stride)
        acc ^= __builtin_nontemporal_load(src + i * 16);
    const unsigned int x = acc.x ^ acc.y ^ acc.z ^ acc.w;
    if (x == 0x9E3779B9u) sink[blockIdx.x] = x;  // keeps the loads; almost never taken
}

}  // namespace
}  // namespace jl

using namespace jl;

extern "C" int jl_hbm_stream(int32_t kind, const void* src, void* dst, int64_t bytes, uint32_t* sink,
                             int32_t workgroups, jl_stream_t stream) {
    if (bytes <= 0 || (bytes & 15) != 0 || workgroups <= 0) return JL_ERR_ARG;
    const bool reads = kind == 0 || kind == 2 || kind == 4 || kind == 5 || kind == 7 || kind == 9 || kind == 10;
    const bool sinks = kind == 0 || kind == 5 || kind == 10;
    if ((reads && !src) || (!sinks && !dst) || (sinks && !sink)) return JL_ERR_ARG;
    if (kind == 10 && (bytes & 255) != 0) return JL_ERR_ARG;
    if (((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) & 15u) != 0) return JL_ERR_ARG;
    const size_t n = (size_t)bytes / 16;
    const v4u* s = reinterpret_cast<const v4u*>(src);
    v4u* d = reinterpret_cast<v4u*>(dst);
    hipStream_t st = (hipStream_t)stream;
    const dim3 grid(workgroups), block(kStreamThreads);
    switch (kind) {
        case 0: hipLaunchKernelGGL((stream_kernel<0, true>), grid, block, 0, st, s, d, n, sink); break;
        case 1: hipLaunchKernelGGL((stream_kernel<1, true>), grid, block, 0, st, s, d, n, sink); break;
        case 2: hipLaunchKernelGGL((stream_kernel<2, true>), grid, block, 0, st, s, d, n, sink); break;
        case 3: hipLaunchKernelGGL((stream_kernel<1, false>), grid, block, 0, st, s, d, n, sink); break;
        case 4: hipLaunchKernelGGL((stream_kernel<2, false>), grid, block, 0, st, s, d, n, sink); break;
        case 5: hipLaunchKernelGGL((chunk_kernel<0, true>), grid, block, 0, st, s, d, n, sink); break;
        case 6: hipLaunchKernelGGL((chunk_kernel<1, true>), grid, block, 0, st, s, d, n, sink); break;
        case 7: hipLaunchKernelGGL((chunk_kernel<2, true>), grid, block, 0, st, s, d, n, sink); break;
        case 8: hipLaunchKernelGGL((chunk_kernel<1, false>), grid, block, 0, st, s, d, n, sink); break;
        case 9: hipLaunchKernelGGL((chunk_kernel<2, false>), grid, block, 0, st, s, d, n, sink); break;
        case 10: hipLaunchKernelGGL(sparse_read_kernel, grid, block, 0, st, s, n / 16, sink); break;
        default: return JL_ERR_ARG;
    }
    return launch_status();
}
