// HBM streaming probe for gfx950: the achievable rate of the two access
// patterns of this library's HBM-bound kernels, measured with the simplest
// kernel that has them.
//   kind 0: c = a ^ b over `bytes` each: two streams read, one written (the
//           gated RMSNorm's x, z -> y)
//   kind 1: c ^= pattern in place over `bytes`: one stream read and written
//           (the decode step's state)
// Each thread moves 16-byte vectors in a grid-stride loop; `nontemporal`
// selects non-temporal loads and stores (as the RMSNorm and decode kernels
// use).  No counterpart in the reference: benchmarks report it beside the
// kernels' rates as the chip's streaming ceiling.
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
    if (!c || bytes == 0 || bytes % 16 != 0 || blocks <= 0 || (kind == 0 && (!a || !b)) ||
        (kind != 0 && kind != 1))
        return hipErrorInvalidValue;
    const int64_t n = (int64_t)(bytes / 16);
    const dim3 grid((unsigned)blocks), block(kProbeThreads);
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
