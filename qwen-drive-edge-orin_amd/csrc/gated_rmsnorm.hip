// Fused gated RMSNorm for gfx950: y = rmsnorm(x) * w * silu(z).
//
// Replaces the TensorRT plugin kernel kern_gated_rmsnorm_fp16
// (export/patches/orin_text_engine/files/cpp/kernels/gatedRmsNorm/
// gatedRmsNormKernel.cu:21-64, entry gatedRmsNormForward, .h:17-18) and
// follows the dtype steps of transformers' Qwen3_5RMSNormGated.forward
// (modeling_qwen3_5.py:175-184):
//   n = round_in( x * rsqrt(mean(x^2) + eps) )      (fp32 math)
//   h = w * n       -- rounded to the input dtype when w has the input dtype,
//                      kept in fp32 when w is fp32 (torch type promotion)
//   y = round_in( h * silu(float(z)) )
//
// Layout: rows of `dv` contiguous elements.  A row is handled by
// dv / (8 kPieces) lanes, each moving kPieces 16-byte pieces of x, z and y
// (piece j of lane s at elements 8 s + j dv / kPieces, so each piece index is
// one coalesced run across the row's lanes); the row reduction is a butterfly
// over those lanes.  Purely HBM-bound: 3 * rows * dv * 2 bytes per call.
#include "gdn_common.h"
#include "gdn_hip.h"

#include <math.h>

namespace gdn {
namespace {

constexpr int kNormThreads = 256;
// 16-byte pieces per lane: 2 measured 6.46-6.58 us at 1141 x 32 rows of 128
// bf16 against 6.76-6.79 us for 1 and 8.05 us for 4 (the one-shot streaming
// probe of the same three streams: 6.05 / 6.11 / 6.89 us).
constexpr int kPieces = 2;

template <int IO>  // 0 = bf16, 1 = fp16
__device__ inline float load_elem(uint32_t bits) {
    if (IO == 0) return bf16_bits_to_f32(bits);
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits);
}

template <int IO>
__device__ inline uint32_t store_elem(float f) {
    if (IO == 0) return f32_to_bf16_bits(f);
    // the fp32 value must exist before it is rounded: fused into the
    // producing multiply(-add) (v_fma_mixlo_f16) the product is rounded to
    // fp16 once instead of to fp32 first, which differs in rare ties
    asm("" : "+v"(f));
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)f);
}

template <int IO>
__device__ inline float round_io(float f) {
    return load_elem<IO>(store_elem<IO>(f));
}

// W: 0 = same dtype as the input (bf16/fp16), 2 = fp32
template <int IO, int W, int LPR>
__global__ __launch_bounds__(kNormThreads) void gated_rmsnorm_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ z, const void* __restrict__ w,
    uint16_t* __restrict__ y, int64_t rows, float eps) {
    constexpr int P = kPieces;
    constexpr int dv = LPR * 8 * P;
    const int64_t row = ((int64_t)blockIdx.x * kNormThreads + threadIdx.x) / LPR;
    const int sub = threadIdx.x % LPR;
    const bool active = row < rows;
    // threads past the last row (last block only) read that row again and
    // store nothing, so every load is unconditional: weights first, then the
    // row of x and of z
    const int64_t off = (active ? row : rows - 1) * dv + sub * 8;

    u32x4 wr[P];
    f32x4 w0[P], w1[P];
#pragma unroll
    for (int j = 0; j < P; ++j) {
        const int e = sub * 8 + j * (LPR * 8);
        if (W == 2) {
            const f32x4* wp = reinterpret_cast<const f32x4*>(static_cast<const float*>(w) + e);
            w0[j] = wp[0];
            w1[j] = wp[1];
        } else {
            wr[j] = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(w) + e);
        }
    }
    u32x4 xr[P], zr[P];
#pragma unroll
    for (int j = 0; j < P; ++j)
        xr[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(x + off + j * (LPR * 8)));
#pragma unroll
    for (int j = 0; j < P; ++j)
        zr[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(z + off + j * (LPR * 8)));
    float xf[P][8], zf[P][8];
#pragma unroll
    for (int j = 0; j < P; ++j) {
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            xf[j][2 * p] = load_elem<IO>(xr[j][p] & 0xffffu);
            xf[j][2 * p + 1] = load_elem<IO>(xr[j][p] >> 16);
            zf[j][2 * p] = load_elem<IO>(zr[j][p] & 0xffffu);
            zf[j][2 * p + 1] = load_elem<IO>(zr[j][p] >> 16);
        }
    }
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < P; ++j) {
#pragma unroll
        for (int e = 0; e < 8; ++e) ss = fmaf(xf[j][e], xf[j][e], ss);
    }
    ss = lane_group_sum<LPR>(ss);
    const float r = 1.0f / sqrtf(ss / (float)dv + eps);

    u32x4 o4[P];
#pragma unroll
    for (int j = 0; j < P; ++j) {
        float wf[8];
        if (W == 2) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                wf[e] = w0[j][e];
                wf[4 + e] = w1[j][e];
            }
        } else {
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                wf[2 * p] = load_elem<IO>(wr[j][p] & 0xffffu);
                wf[2 * p + 1] = load_elem<IO>(wr[j][p] >> 16);
            }
        }
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            uint32_t pk = 0;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int e = 2 * p + h;
                const float n = round_io<IO>(xf[j][e] * r);
                float hv = wf[e] * n;
                if (W != 2) hv = round_io<IO>(hv);
                // silu(z) = z / (1 + e^-z) from the hardware base-2
                // exponential and reciprocal (each within about an fp32 ulp)
                const float sz = zf[j][e] * __builtin_amdgcn_rcpf(
                                                1.0f + __builtin_amdgcn_exp2f(zf[j][e] * -1.44269504088896341f));
                pk |= store_elem<IO>(hv * sz) << (16 * h);
            }
            o4[j][p] = pk;
        }
    }
    // the outputs are formed before the store's guard: otherwise the
    // compiler moves their whole computation, z and w loads included, into
    // the guarded block, behind the wait for x
#pragma unroll
    for (int j = 0; j < P; ++j) asm volatile("" ::"v"(o4[j]));
    if (active) {
#pragma unroll
        for (int j = 0; j < P; ++j)
            __builtin_nontemporal_store(o4[j], reinterpret_cast<u32x4*>(y + off + j * (LPR * 8)));
    }
}

template <int IO, int W>
hipError_t launch_norm(const void* x, const void* z, const void* w, void* y, int64_t rows, int dv,
                       float eps, hipStream_t stream) {
    const int lpr = dv / (8 * kPieces);
    const int64_t rows_per_block = kNormThreads / lpr;
    const int64_t blocks = (rows + rows_per_block - 1) / rows_per_block;
    if (blocks > 0x7fffffff) return hipErrorInvalidValue;
    const dim3 grid((unsigned)blocks), block(kNormThreads);
    auto xp = static_cast<const uint16_t*>(x);
    auto zp = static_cast<const uint16_t*>(z);
    auto yp = static_cast<uint16_t*>(y);
    switch (lpr) {
        case 4:
            if constexpr (kPieces > 1) {
                hipLaunchKernelGGL((gated_rmsnorm_kernel<IO, W, 4>), grid, block, 0, stream, xp, zp, w, yp, rows, eps);
                break;
            }
            return hipErrorInvalidValue;
        case 8:
            hipLaunchKernelGGL((gated_rmsnorm_kernel<IO, W, 8>), grid, block, 0, stream, xp, zp, w, yp, rows, eps);
            break;
        case 16:
            hipLaunchKernelGGL((gated_rmsnorm_kernel<IO, W, 16>), grid, block, 0, stream, xp, zp, w, yp, rows, eps);
            break;
        case 32:
            hipLaunchKernelGGL((gated_rmsnorm_kernel<IO, W, 32>), grid, block, 0, stream, xp, zp, w, yp, rows, eps);
            break;
        case 64:
            hipLaunchKernelGGL((gated_rmsnorm_kernel<IO, W, 64>), grid, block, 0, stream, xp, zp, w, yp, rows, eps);
            break;
        default:
            return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace
}  // namespace gdn

using namespace gdn;

extern "C" hipError_t gdn_gated_rmsnorm_forward(const void* x, const void* z, const void* w,
                                                void* y, int64_t rows, int dv, float eps,
                                                int io_dtype, int w_dtype, hipStream_t stream) {
    if (rows < 0 || !(dv == 64 || dv == 128 || dv == 256 || dv == 512)) return hipErrorInvalidValue;
    if (!(eps >= 0.f)) return hipErrorInvalidValue;
    if (io_dtype != GDN_DTYPE_BF16 && io_dtype != GDN_DTYPE_FP16) return hipErrorInvalidValue;
    if (w_dtype != io_dtype && w_dtype != GDN_DTYPE_FP32) return hipErrorInvalidValue;
    if (rows == 0) return hipSuccess;
    if (!x || !z || !w || !y) return hipErrorInvalidValue;
    if (io_dtype == GDN_DTYPE_BF16)
        return w_dtype == GDN_DTYPE_FP32
                   ? launch_norm<0, 2>(x, z, w, y, rows, dv, eps, stream)
                   : launch_norm<0, 0>(x, z, w, y, rows, dv, eps, stream);
    return w_dtype == GDN_DTYPE_FP32 ? launch_norm<1, 2>(x, z, w, y, rows, dv, eps, stream)
                                     : launch_norm<1, 0>(x, z, w, y, rows, dv, eps, stream);
}
