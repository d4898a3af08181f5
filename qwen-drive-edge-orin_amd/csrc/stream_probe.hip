// HBM streaming probe for gfx950: the achievable rate of the two access
// patterns of this library's HBM-bound kernels, measured with the simplest
// kernel that has them.
//   kind 0: c = a ^ b over `bytes` each: two streams read, one written (the
//           gated RMSNorm's x, z -> y)
//   kind 1: c ^= pattern in place over `bytes`: one stream read and written
//           (the decode step's state)
//   kind 2: kind 0 in one pass with no loop, the gated RMSNorm's own launch
//           shape: ceil(n / (256 P)) work-groups of 256 threads, each thread
//           moving P = `blocks` (1..4) 16-byte vectors, 256 vectors apart
// Kinds 0 and 1 move 16-byte vectors in a grid-stride loop over `blocks`
// work-groups; `nontemporal` selects non-temporal loads and stores (as the
// RMSNorm and decode kernels use).  No counterpart in the reference:
// benchmarks report it beside the kernels' rates as the chip's streaming
// ceiling.
#include "gdn_common.h"
#include "gdn_hip_diag.h"

namespace gdn {
namespace {

constexpr int kProbeThreads = 256;

template <bool NT>
__device__ inline u32x4 ld16(const u32x4* p) {
    if constexpr (NT) return __builtin_nontemporal_load(p);
    return *p;
}

template <bool NT>
__device__ inline void st16(u32x4* p, u32x4 v) {
    if constexpr (NT) __builtin_nontemporal_store(v, p);
    else *p = v;
}

template <bool NT>
__global__ __launch_bounds__(kProbeThreads) void stream_r2w1_kernel(
    const u32x4* __restrict__ a, const u32x4* __restrict__ b, u32x4* __restrict__ c, int64_t n) {
    const int64_t stride = (int64_t)gridDim.x * kProbeThreads;
    for (int64_t i = (int64_t)blockIdx.x * kProbeThreads + threadIdx.x; i < n; i += stride)
        st16<NT>(c + i, ld16<NT>(a + i) ^ ld16<NT>(b + i));
}

template <bool NT, int P>
__global__ __launch_bounds__(kProbeThreads) void stream_r2w1_once_kernel(
    const u32x4* __restrict__ a, const u32x4* __restrict__ b, u32x4* __restrict__ c, int64_t n) {
    const int64_t base = (int64_t)blockIdx.x * kProbeThreads * P + threadIdx.x;
    u32x4 va[P], vb[P];
#pragma unroll
    for (int j = 0; j < P; ++j) {
        const int64_t i = base + (int64_t)j * kProbeThreads;
        if (i < n) {
            va[j] = ld16<NT>(a + i);
            vb[j] = ld16<NT>(b + i);
        }
    }
#pragma unroll
    for (int j = 0; j < P; ++j) {
        const int64_t i = base + (int64_t)j * kProbeThreads;
        if (i < n) st16<NT>(c + i, va[j] ^ vb[j]);
    }
}

template <bool NT>
__global__ __launch_bounds__(kProbeThreads) void stream_rw_kernel(u32x4* __restrict__ c, int64_t n) {
    const int64_t stride = (int64_t)gridDim.x * kProbeThreads;
    const u32x4 pat = {0x80000000u, 0x80000000u, 0x80000000u, 0x80000000u};
    for (int64_t i = (int64_t)blockIdx.x * kProbeThreads + threadIdx.x; i < n; i += stride)
        st16<NT>(c + i, ld16<NT>(c + i) ^ pat);
}

}  // namespace
}  // namespace gdn

using namespace gdn;

extern "C" hipError_t gdn_stream_probe(int kind, int nontemporal, const void* a, const void* b,
                                       void* c, size_t bytes, int blocks, hipStream_t stream) {
    if (!c || bytes == 0 || bytes % 16 != 0 || blocks <= 0 || (kind != 1 && (!a || !b)) ||
        kind < 0 || kind > 2 || (kind == 2 && blocks > 4))
        return hipErrorInvalidValue;
    const int64_t n = (int64_t)(bytes / 16);
    const dim3 block(kProbeThreads);
    if (kind == 2) {
        const int64_t per = (int64_t)kProbeThreads * blocks;
        const int64_t g = (n + per - 1) / per;
        if (g > 0x7fffffff) return hipErrorInvalidValue;
        const dim3 grid((unsigned)g);
        auto A = static_cast<const u32x4*>(a);
        auto B = static_cast<const u32x4*>(b);
        auto C = static_cast<u32x4*>(c);
#define GDN_ONCE(P)                                                                              \
    case P:                                                                                      \
        if (nontemporal)                                                                         \
            hipLaunchKernelGGL((stream_r2w1_once_kernel<true, P>), grid, block, 0, stream, A, B, C, n); \
        else                                                                                     \
            hipLaunchKernelGGL((stream_r2w1_once_kernel<false, P>), grid, block, 0, stream, A, B, C, n); \
        break;
        switch (blocks) { GDN_ONCE(1) GDN_ONCE(2) GDN_ONCE(3) GDN_ONCE(4) }
#undef GDN_ONCE
        return hipGetLastError();
    }
    const dim3 grid((unsigned)blocks);
    if (kind == 0) {
        auto k = nontemporal ? stream_r2w1_kernel<true> : stream_r2w1_kernel<false>;
        hipLaunchKernelGGL(k, grid, block, 0, stream, static_cast<const u32x4*>(a),
                           static_cast<const u32x4*>(b), static_cast<u32x4*>(c), n);
    } else {
        auto k = nontemporal ? stream_rw_kernel<true> : stream_rw_kernel<false>;
        hipLaunchKernelGGL(k, grid, block, 0, stream, static_cast<u32x4*>(c), n);
    }
    return hipGetLastError();
}
