// Shared device helpers for the gated-delta-rule kernels (gfx950 / CDNA4).
//
// Matrix products run on v_mfma_f32_16x16x32_f16: fp16 operands, fp32
// accumulation.  bf16 inputs convert to fp16 exactly inside fp16's normal
// range (|x| in [6.1e-5, 65504]); fp16's 10-bit mantissa keeps the rounding
// of derived operands (W, V_new, M, decayed K) 8x finer than bf16 would.
//
// Operand layout of one 16x16x32 MFMA on a 64-lane wave, lane l, g = l / 16:
//   A (16 x 32): lane holds row (l % 16), 8 k-values of lane group g
//   B (32 x 16): lane holds col (l % 16), the same 8 k-values of group g
//   D (16 x 16): lane holds col (l % 16), rows 4g .. 4g+3
// Which k a (group, register) slot stands for is a free choice as long as A
// and B agree.  This library uses one fixed map for every k-block of 32:
//   k(g, j) = 16 * (j / 4) + 4 * g + (j % 4),   j = 0..7
// so registers 0..3 of a B operand are rows 4g..4g+3 of one D tile and
// registers 4..7 the same rows of the next D tile.  A D-layout accumulator
// therefore feeds the next product as its B operand without any shuffle.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gdn {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int kDK = 128;     // key head dim (only validated size)
constexpr int kDV = 128;     // value head dim
constexpr int kChunk = 64;   // chunk length
constexpr int kSlices = 8;   // value-column slices of the state per head
constexpr int kBV = kDV / kSlices;  // 16 state columns per slice

__device__ __forceinline__ f32x4 mfma16(half8 a, half8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f32x4 mfma16_bf16(bf16x8 a, bf16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// k index of (lane group g, register j) inside a 32-wide k-block
__device__ __forceinline__ constexpr int kmap(int g, int j) {
    return 16 * (j >> 2) + 4 * g + (j & 3);
}

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t bits16) {
    return __uint_as_float(bits16 << 16);
}

// fp32 -> bf16 bits, round to nearest even (hardware v_cvt_pk_bf16_f32)
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
    return __builtin_bit_cast(uint16_t, (__bf16)f);
}

__device__ __forceinline__ half4 to_half4(f32x4 v) {
    half4 h;
    h[0] = (_Float16)v[0];
    h[1] = (_Float16)v[1];
    h[2] = (_Float16)v[2];
    h[3] = (_Float16)v[3];
    return h;
}

__device__ __forceinline__ half8 cat8(half4 lo, half4 hi) {
    half8 r;
    r[0] = lo[0]; r[1] = lo[1]; r[2] = lo[2]; r[3] = lo[3];
    r[4] = hi[0]; r[5] = hi[1]; r[6] = hi[2]; r[7] = hi[3];
    return r;
}

// Two D-layout tiles a, b as an fp16 hi / lo pair of one packed operand:
// hi = fp16(x), lo = fp16(x - hi), the residual taken from the packed hi bits
// themselves.  Left alone, the compiler may form the two uses of hi
// differently when x is a product: the operand as fp16(fp32(p)) (rounded
// twice) and the residual's copy with a mixed-precision FMA, fp16(p)
// (rounded once).  Next to an fp16 rounding midpoint those differ by one ulp,
// and hi + lo is then one ulp of hi off.  x - hi is exact in fp32.
__device__ __forceinline__ void split_hilo8(f32x4 a, f32x4 b, half8& hi, half8& lo) {
    half8 h = cat8(to_half4(a), to_half4(b));
    asm volatile("" : "+v"(h));
    f32x4 ra, rb;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        ra[i] = a[i] - (float)h[i];
        rb[i] = b[i] - (float)h[4 + i];
    }
    hi = h;
    lo = cat8(to_half4(ra), to_half4(rb));
}

__device__ __forceinline__ f32x4 zero4() {
    f32x4 z = {0.f, 0.f, 0.f, 0.f};
    return z;
}

// x + (x of the lane the DPP control names), every lane's source valid
template <int kCtrl>
__device__ __forceinline__ float dpp_sum(float x) {
    const int t = __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), kCtrl, 0xf, 0xf, true);
    return x + __builtin_bit_cast(float, t);
}

// Sum over each aligned group of N lanes (N a power of two), the same value
// in every lane of the group, added in the order of an xor butterfly (lane
// i with i ^ 1, then i ^ 2, ...): within 16 lanes by DPP moves (quad
// permutes, then the half-row and row mirrors, which pair the same sums),
// across rows by LDS permutes.
template <int N>
__device__ inline float lane_group_sum(float x) {
    if constexpr (N > 1) x = dpp_sum<0xB1>(x);    // quad_perm [1,0,3,2]
    if constexpr (N > 2) x = dpp_sum<0x4E>(x);    // quad_perm [2,3,0,1]
    if constexpr (N > 4) x = dpp_sum<0x141>(x);   // row_half_mirror
    if constexpr (N > 8) x = dpp_sum<0x140>(x);   // row_mirror
#pragma unroll
    for (int m = 16; m < N; m <<= 1) x += __shfl_xor(x, m, 64);
    return x;
}

}  // namespace gdn
