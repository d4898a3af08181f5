// Causal depthwise conv1d over time with optional SiLU for gfx950: the step
// that produces q, k and v in transformers' Qwen3.5 gated-delta layers
// (models/qwen3_5/modeling_qwen3_5.py:199-240 for the functions, 457-476 for
// the calls).  Per channel d and token t, with K taps:
//   y[t][d] = io( act( w_dt( sum_{j<K} w[d][j] * x[t-K+1+j][d] + bias[d] ) ) )
// where x before the first token is the carried state (zero for a fresh
// sequence), the sum is accumulated in fp32 (taps oldest first as fused
// multiply-adds, then the bias: the order of torch's CPU convolution) and
// rounded to the weight dtype w_dt (F.conv1d runs in the weight dtype), act =
// SiLU evaluated in fp32 on that rounded value, and the result rounded to the
// I/O dtype -- the dtype steps of the transformers functions.
//
// Layout: x and y are [B][T][D] with channels contiguous (transformers hands
// a transposed view of exactly that), so a lane moves 16 bytes = 8 channels
// of one token.  A thread owns 8 channels and kConvTT consecutive tokens and
// keeps the K-token window in registers; neighbouring token tiles overlap by
// K-1 rows (L2 hits).  Purely HBM-bound: x read once, y written once.
#include "gdn_common.h"
#include "gdn_hip.h"

#include <math.h>

namespace gdn {
namespace {

constexpr int kConvThreads = 256;
constexpr int kConvTT = 8;          // tokens per thread
constexpr int kConvMaxState = 8;    // longest carried state of the update

// element loads / stores by dtype code (0 bf16, 1 fp16, 2 fp32)
template <int DT>
__device__ inline float ld_elem(const void* p, size_t i) {
    if constexpr (DT == 0) return bf16_bits_to_f32(static_cast<const uint16_t*>(p)[i]);
    if constexpr (DT == 1) return (float)static_cast<const _Float16*>(p)[i];
    return static_cast<const float*>(p)[i];
}

template <int IO>
__device__ inline float cv_load(uint32_t bits16) {
    if constexpr (IO == 0) return bf16_bits_to_f32(bits16);
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
}

template <int IO>
__device__ inline uint32_t cv_store(float f) {
    if constexpr (IO == 0) return f32_to_bf16_bits(f);
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)f);
}

template <int IO>
__device__ inline void unpack8(u32x4 r, float (&f)[8]) {
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        f[2 * p] = cv_load<IO>(r[p] & 0xffffu);
        f[2 * p + 1] = cv_load<IO>(r[p] >> 16);
    }
}

// act(round_w(acc)) rounded to the I/O dtype.  With fp32 weights the conv
// output is already fp32 and only the final rounding remains.
template <int IO, int WT>
__device__ inline uint32_t finish(float acc, int silu) {
    float r = (WT == 2) ? acc : cv_load<WT>(cv_store<WT>(acc));
    if (silu) r = r / (1.0f + expf(-r));
    return cv_store<IO>(r);
}

template <int IO, int WT, int K>
__global__ __launch_bounds__(kConvThreads) void causal_conv1d_fwd_kernel(
    const uint16_t* __restrict__ x, const void* __restrict__ w, const void* __restrict__ bias,
    uint16_t* __restrict__ y, int T, int D, int64_t xbs, int64_t xts, int64_t ybs, int64_t yts,
    int silu) {
    const int g8 = blockIdx.x * kConvThreads + threadIdx.x;   // 8-channel group
    if (g8 * 8 >= D) return;
    const int t0 = blockIdx.y * kConvTT;
    const int b = blockIdx.z;
    const int d0 = g8 * 8;
    const uint16_t* xb = x + (size_t)b * xbs + d0;
    uint16_t* yb = y + (size_t)b * ybs + d0;
    // all loads first: rows t0-K+1 .. t0+kConvTT-1 (rows before 0 are zero,
    // rows past T-1 re-read row T-1 and are never stored)
    u32x4 raw[kConvTT + K - 1];
#pragma unroll
    for (int i = 0; i < kConvTT + K - 1; ++i) {
        const int t = t0 - (K - 1) + i;
        const int tc = min(max(t, 0), T - 1);
        raw[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(xb + (size_t)tc * xts));
        if (t < 0) raw[i] = u32x4{0u, 0u, 0u, 0u};
    }
    float wf[8][K], bf[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
#pragma unroll
        for (int j = 0; j < K; ++j) wf[e][j] = ld_elem<WT>(w, (size_t)(d0 + e) * K + j);
        bf[e] = bias ? ld_elem<WT>(bias, d0 + e) : 0.f;
    }
#pragma unroll
    for (int i = 0; i < kConvTT; ++i) {
        const int t = t0 + i;
        float acc[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] = 0.f;
#pragma unroll
        for (int j = 0; j < K; ++j) {
            float xf[8];
            unpack8<IO>(raw[i + j], xf);
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[e] = fmaf(wf[e][j], xf[e], acc[e]);
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] += bf[e];
        u32x4 out;
#pragma unroll
        for (int p = 0; p < 4; ++p)
            out[p] = finish<IO, WT>(acc[2 * p], silu) | (finish<IO, WT>(acc[2 * p + 1], silu) << 16);
        if (t < T) __builtin_nontemporal_store(out, reinterpret_cast<u32x4*>(yb + (size_t)t * yts));
    }
}

// Decode-time update: one thread per (batch, channel).  The window is the
// carried state (state_len tokens, oldest first) followed by the T new
// tokens; the outputs are the last T positions of the valid convolution over
// the window, and the state becomes the window's last state_len tokens
// (modeling_qwen3_5.py:200-216).  The window is read into registers before
// the state is rewritten, since the two overlap whenever T < state_len.
template <int IO, int WT, int K>
__global__ __launch_bounds__(kConvThreads) void causal_conv1d_update_kernel(
    const uint16_t* __restrict__ x, uint16_t* __restrict__ state, const void* __restrict__ w,
    const void* __restrict__ bias, uint16_t* __restrict__ y, int B, int T, int D, int state_len,
    int64_t xbs, int64_t xts, int64_t xds, int64_t sbs, int64_t sds, int64_t ybs, int64_t yts,
    int64_t yds, int silu) {
    const int64_t gid = (int64_t)blockIdx.x * kConvThreads + threadIdx.x;
    if (gid >= (int64_t)B * D) return;
    const int b = (int)(gid / D), d = (int)(gid - (int64_t)b * D);
    float wf[K];
#pragma unroll
    for (int j = 0; j < K; ++j) wf[j] = ld_elem<WT>(w, (size_t)d * K + j);
    const float bv = bias ? ld_elem<WT>(bias, d) : 0.f;
    uint16_t* st = state + (size_t)b * sbs + (size_t)d * sds;
    const uint16_t* xs = x + (size_t)b * xbs + (size_t)d * xds;
    uint16_t* ys = y + (size_t)b * ybs + (size_t)d * yds;
    // the old state, then a rolling K-1 history of window values
    uint16_t old[kConvMaxState];
#pragma unroll
    for (int p = 0; p < kConvMaxState; ++p) old[p] = p < state_len ? st[p] : (uint16_t)0;
    // hist[K-1] is the newest window value; state_len >= K-1, so the K-1
    // newest state values seed the rest
    float hist[K];
#pragma unroll
    for (int j = 0; j < K - 1; ++j) {
        const int p = state_len - (K - 1) + j;
        uint16_t v = 0;
#pragma unroll
        for (int q = 0; q < kConvMaxState; ++q) v = (q == p) ? old[q] : v;
        hist[j] = cv_load<IO>(v);
    }
    for (int i = 0; i < T; ++i) {
        const uint16_t xr = xs[(size_t)i * xts];
        hist[K - 1] = cv_load<IO>(xr);
        float acc = 0.f;
#pragma unroll
        for (int j = 0; j < K; ++j) acc = fmaf(wf[j], hist[j], acc);
        acc += bv;
        ys[(size_t)i * yts] = (uint16_t)finish<IO, WT>(acc, silu);
#pragma unroll
        for (int j = 0; j < K - 1; ++j) hist[j] = hist[j + 1];
    }
    // new state: the window's last state_len tokens.  Entry p is window index
    // q = (L - state_len) + p = T + p (L = state_len + T): an old state value
    // while q < state_len, else new token q - state_len.
    for (int p = 0; p < state_len; ++p) {
        const int q = T + p;
        uint16_t v;
        if (q < state_len) {
            v = 0;
#pragma unroll
            for (int r = 0; r < kConvMaxState; ++r) v = (r == q) ? old[r] : v;
        } else {
            v = xs[(size_t)(q - state_len) * xts];
        }
        st[p] = v;
    }
}

template <int IO, int WT>
hipError_t launch_fwd(const void* x, const void* w, const void* bias, void* y, int B, int T, int D,
                      int K, int64_t xbs, int64_t xts, int64_t ybs, int64_t yts, int silu,
                      hipStream_t stream) {
    const dim3 grid((unsigned)((D / 8 + kConvThreads - 1) / kConvThreads),
                    (unsigned)((T + kConvTT - 1) / kConvTT), (unsigned)B);
    auto xp = static_cast<const uint16_t*>(x);
    auto yp = static_cast<uint16_t*>(y);
#define GDN_CONV_FWD(KK)                                                                        \
    case KK:                                                                                    \
        hipLaunchKernelGGL((causal_conv1d_fwd_kernel<IO, WT, KK>), grid, dim3(kConvThreads), 0, \
                           stream, xp, w, bias, yp, T, D, xbs, xts, ybs, yts, silu);            \
        break;
    switch (K) {
        GDN_CONV_FWD(2)
        GDN_CONV_FWD(3)
        GDN_CONV_FWD(4)
        default:
            return hipErrorInvalidValue;
    }
#undef GDN_CONV_FWD
    return hipGetLastError();
}

template <int IO, int WT>
hipError_t launch_update(const void* x, void* state, const void* w, const void* bias, void* y,
                         int B, int T, int D, int K, int state_len, int64_t xbs, int64_t xts,
                         int64_t xds, int64_t sbs, int64_t sds, int64_t ybs, int64_t yts,
                         int64_t yds, int silu, hipStream_t stream) {
    const int64_t n = (int64_t)B * D;
    const dim3 grid((unsigned)((n + kConvThreads - 1) / kConvThreads));
    auto xp = static_cast<const uint16_t*>(x);
    auto sp = static_cast<uint16_t*>(state);
    auto yp = static_cast<uint16_t*>(y);
#define GDN_CONV_UPD(KK)                                                                        \
    case KK:                                                                                    \
        hipLaunchKernelGGL((causal_conv1d_update_kernel<IO, WT, KK>), grid, dim3(kConvThreads), \
                           0, stream, xp, sp, w, bias, yp, B, T, D, state_len, xbs, xts, xds,   \
                           sbs, sds, ybs, yts, yds, silu);                                      \
        break;
    switch (K) {
        GDN_CONV_UPD(2)
        GDN_CONV_UPD(3)
        GDN_CONV_UPD(4)
        default:
            return hipErrorInvalidValue;
    }
#undef GDN_CONV_UPD
    return hipGetLastError();
}

bool conv_dtypes_ok(int io_dtype, int w_dtype) {
    if (io_dtype != GDN_DTYPE_BF16 && io_dtype != GDN_DTYPE_FP16) return false;
    return w_dtype == io_dtype || w_dtype == GDN_DTYPE_FP32;
}

}  // namespace
}  // namespace gdn

using namespace gdn;

extern "C" hipError_t gdn_causal_conv1d_fwd(const void* x, const void* w, const void* bias,
                                            void* y, int B, int T, int D, int K,
                                            int64_t x_bstride, int64_t x_tstride,
                                            int64_t y_bstride, int64_t y_tstride, int io_dtype,
                                            int w_dtype, int silu, hipStream_t stream) {
    if (B < 0 || T < 0 || D <= 0 || D % 8 != 0 || K < 2 || K > 4) return hipErrorInvalidValue;
    if (!conv_dtypes_ok(io_dtype, w_dtype) || (silu != 0 && silu != 1)) return hipErrorInvalidValue;
    if (B > 65535 || (int64_t)T > 65535LL * kConvTT) return hipErrorInvalidValue;   // grid y, z
    if (B == 0 || T == 0) return hipSuccess;
    if (!x || !w || !y) return hipErrorInvalidValue;
    // 16-byte lane accesses: every row start must stay 16-byte aligned
    if ((x_bstride | x_tstride | y_bstride | y_tstride) % 8 != 0 ||
        ((uintptr_t)x | (uintptr_t)y) % 16 != 0)
        return hipErrorInvalidValue;
    const bool bf = io_dtype == GDN_DTYPE_BF16, w32 = w_dtype == GDN_DTYPE_FP32;
#define GDN_FWD_ARGS x, w, bias, y, B, T, D, K, x_bstride, x_tstride, y_bstride, y_tstride, silu, stream
    if (bf) return w32 ? launch_fwd<0, 2>(GDN_FWD_ARGS) : launch_fwd<0, 0>(GDN_FWD_ARGS);
    return w32 ? launch_fwd<1, 2>(GDN_FWD_ARGS) : launch_fwd<1, 1>(GDN_FWD_ARGS);
#undef GDN_FWD_ARGS
}

extern "C" hipError_t gdn_causal_conv1d_update(const void* x, void* conv_state, const void* w,
                                               const void* bias, void* y, int B, int T, int D,
                                               int K, int state_len, int64_t x_bstride,
                                               int64_t x_tstride, int64_t x_dstride,
                                               int64_t s_bstride, int64_t s_dstride,
                                               int64_t y_bstride, int64_t y_tstride,
                                               int64_t y_dstride, int io_dtype, int w_dtype,
                                               int silu, hipStream_t stream) {
    if (B < 0 || T < 0 || D <= 0 || K < 2 || K > 4) return hipErrorInvalidValue;
    if (state_len < K - 1 || state_len > kConvMaxState) return hipErrorInvalidValue;
    if (!conv_dtypes_ok(io_dtype, w_dtype) || (silu != 0 && silu != 1)) return hipErrorInvalidValue;
    if ((int64_t)B * D > 65535LL * 65536LL) return hipErrorInvalidValue;   // grid x
    if (B == 0 || T == 0) return hipSuccess;
    if (!x || !conv_state || !w || !y) return hipErrorInvalidValue;
    const bool bf = io_dtype == GDN_DTYPE_BF16, w32 = w_dtype == GDN_DTYPE_FP32;
#define GDN_UPD_ARGS                                                                             \
    x, conv_state, w, bias, y, B, T, D, K, state_len, x_bstride, x_tstride, x_dstride, s_bstride, \
        s_dstride, y_bstride, y_tstride, y_dstride, silu, stream
    if (bf) return w32 ? launch_update<0, 2>(GDN_UPD_ARGS) : launch_update<0, 0>(GDN_UPD_ARGS);
    return w32 ? launch_update<1, 2>(GDN_UPD_ARGS) : launch_update<1, 1>(GDN_UPD_ARGS);
#undef GDN_UPD_ARGS
}
