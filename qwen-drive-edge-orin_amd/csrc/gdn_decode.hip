// Recurrent gated-delta-rule step (decode, T >= 1) for gfx950.
//
// The reference has no native decode; its decode path is the torch token
// recurrence transformers modeling_qwen3_5.py:331-380
// (torch_recurrent_gated_delta_rule), per token:
//   S <- e^{g} S;  kv = S^T k;  delta = beta (v - kv);  S <- S + k delta^T;
//   o = s S^T q    (o reads the updated state, s = 1/sqrt(DK))
// which this kernel fuses into one read and one write of S per call:
//   a = S^T k,  b = S^T q             (one pass over the old state)
//   delta = beta (v - e^g a)
//   o = s (e^g b + delta (k . q))     (= s S_new^T q)
//   S_new = e^g S + k delta^T         (written back in place)
//
// The state's columns evolve independently, so each (batch, v-head) is split
// over two work-groups of 256 threads, one per half of the columns: thread t
// of half h owns columns 64 h + 4 (t % 16) .. + 3 of rows (t / 16) + 16 m,
// m = 0..7, so every load/store instruction of a wave moves four 256-byte
// half rows.  Two groups of 32 state registers per thread (rather than one of
// 64) leave room for more groups per CU, whose loads overlap each other's
// arithmetic and stores.  Tokens t > 0 reuse the registers; HBM sees the
// state exactly once in each direction.
#include "gdn_common.h"
#include "gdn_hip.h"

#include <math.h>

namespace gdn {
namespace {

constexpr int kDecThreads = 256;
// Work-groups per (batch, v-head), each taking the state's columns
// [c * kDecCols, (c + 1) * kDecCols): 2 measured fastest at B=64 HV=32 (1: 50.2
// us, 2: 47.9 us, 4: 50.4 us), since two halves give 4 groups per CU at 110
// VGPRs where one group per (b, h) holds 190 VGPRs.
constexpr int kDecSplit = 2;
constexpr int kDecCols = kDV / kDecSplit;     // columns per work-group
constexpr int kColBlocks = kDecCols / 4;      // 16 column blocks of 4
constexpr int kRowGroups = kDecThreads / kColBlocks;   // 16
constexpr int kRowsPerThread = kDK / kRowGroups;       // 8
static_assert(kRowGroups * kRowsPerThread == kDK && kRowGroups % 4 == 0, "row groups");

// kNorm: q and k rows are raw and normalised here first, x rsqrt(sum x^2 +
// 1e-6) in fp32 rounded to bf16 (transformers' use_qk_l2norm_in_kernel).
template <bool kNorm>
__global__ __launch_bounds__(kDecThreads) void gdn_recurrent_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
    const uint16_t* __restrict__ v, const float* __restrict__ g,
    const float* __restrict__ beta, uint16_t* __restrict__ o, float* __restrict__ state, int T,
    int HV, int HK, float scale) {
    __shared__ float qs[kDK], ks[kDK];
    __shared__ f32x4 part[4][2][kColBlocks];  // [wave][a|b][column block]
    __shared__ float kq;

    const int tid = threadIdx.x;
    const int cb = tid & (kColBlocks - 1);   // column block: columns c0 + 4cb .. + 3
    const int rg = tid / kColBlocks;         // row group: rows rg + 16m
    const int wave = tid >> 6;
    const int bh = blockIdx.x / kDecSplit;  // b * HV + hv
    const int c0 = kDecCols * (blockIdx.x % kDecSplit);
    const int b = bh / HV, hv = bh - b * HV;
    const int hk = hv / (HV / HK);

    // A token's inputs: this thread's element of q (threads 0..127) or k
    // (128..255), its four v columns, g and beta.  Token 0's are requested
    // before the state, so forming q and k needs only them; each later
    // token's are requested during the previous token's work.
    const uint16_t* qk = tid < kDK ? q + (size_t)hk * kDK + tid : k + (size_t)hk * kDK + tid - kDK;
    float* qk_dst = tid < kDK ? qs + tid : ks + tid - kDK;
    auto load_token = [&](int t, uint16_t& qkr, uint2& vr, float& gr, float& br) {
        const size_t tk = (size_t)b * T + t;
        qkr = qk[tk * HK * kDK];
        vr = *reinterpret_cast<const uint2*>(v + (tk * HV + hv) * kDV + c0 + 4 * cb);
        gr = g[tk * HV + hv];
        br = beta[tk * HV + hv];
    };
    uint16_t qkr;
    uint2 vraw;
    float gt, bt;
    __builtin_assume(T >= 1);   // the launcher returns before T = 0
    load_token(0, qkr, vraw, gt, bt);
    __builtin_amdgcn_sched_barrier(0);   // keeps them ahead of the state loads

    float* S = state + (size_t)bh * kDK * kDV;
    f32x4 s[kRowsPerThread];
#pragma unroll
    for (int m = 0; m < kRowsPerThread; ++m)
        s[m] = __builtin_nontemporal_load(
            reinterpret_cast<const f32x4*>(S + (rg + kRowGroups * m) * kDV + c0) + cb);

    for (int t = 0; t < T; ++t) {
        const size_t tk = ((size_t)b * T + t);
        *qk_dst = bf16_bits_to_f32(qkr);
        __syncthreads();
        if (kNorm) {
            if (wave == 0) {
                const int l = tid;
                float pq = qs[l] * qs[l] + qs[l + 64] * qs[l + 64];
                float pk = ks[l] * ks[l] + ks[l + 64] * ks[l + 64];
                for (int off = 32; off > 0; off >>= 1) {
                    pq += __shfl_xor(pq, off, 64);
                    pk += __shfl_xor(pk, off, 64);
                }
                const float iq = rsqrtf(pq + 1e-6f), ik = rsqrtf(pk + 1e-6f);
                qs[l] = bf16_bits_to_f32(f32_to_bf16_bits(qs[l] * iq));
                qs[l + 64] = bf16_bits_to_f32(f32_to_bf16_bits(qs[l + 64] * iq));
                ks[l] = bf16_bits_to_f32(f32_to_bf16_bits(ks[l] * ik));
                ks[l + 64] = bf16_bits_to_f32(f32_to_bf16_bits(ks[l + 64] * ik));
            }
            __syncthreads();
        }
        if (wave == 0) {
            float p = qs[tid] * ks[tid] + qs[tid + 64] * ks[tid + 64];
            for (int off = 32; off > 0; off >>= 1) p += __shfl_xor(p, off, 64);
            if (tid == 0) kq = p;
        }
        // partial a = S^T k, b = S^T q over this thread's rows
        f32x4 pa = zero4(), pb = zero4();
#pragma unroll
        for (int m = 0; m < kRowsPerThread; ++m) {
            const int r = rg + kRowGroups * m;
            pa += s[m] * ks[r];
            pb += s[m] * qs[r];
        }
        // the lanes of a wave with one column block (lane % kColBlocks) add up
#pragma unroll
        for (int off = kColBlocks; off < 64; off <<= 1) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                pa[i] += __shfl_xor(pa[i], off, 64);
                pb[i] += __shfl_xor(pb[i], off, 64);
            }
        }
        if ((tid & 63) < kColBlocks) {
            part[wave][0][cb] = pa;
            part[wave][1][cb] = pb;
        }
        __syncthreads();
        f32x4 a = part[0][0][cb] + part[1][0][cb] + part[2][0][cb] + part[3][0][cb];
        f32x4 bq = part[0][1][cb] + part[1][1][cb] + part[2][1][cb] + part[3][1][cb];
        const float decay = expf(gt);
        f32x4 vv;
        vv[0] = bf16_bits_to_f32(vraw.x & 0xffffu);
        vv[1] = bf16_bits_to_f32(vraw.x >> 16);
        vv[2] = bf16_bits_to_f32(vraw.y & 0xffffu);
        vv[3] = bf16_bits_to_f32(vraw.y >> 16);
        const f32x4 delta = (vv - a * decay) * bt;
        if (t + 1 < T) load_token(t + 1, qkr, vraw, gt, bt);
        if (rg == 0) {
            const f32x4 ov = (bq * decay + delta * kq) * scale;
            uint2 packed;
            packed.x = (uint32_t)f32_to_bf16_bits(ov[0]) | ((uint32_t)f32_to_bf16_bits(ov[1]) << 16);
            packed.y = (uint32_t)f32_to_bf16_bits(ov[2]) | ((uint32_t)f32_to_bf16_bits(ov[3]) << 16);
            *reinterpret_cast<uint2*>(o + (tk * HV + hv) * kDV + c0 + 4 * cb) = packed;
        }
#pragma unroll
        for (int m = 0; m < kRowsPerThread; ++m) s[m] = s[m] * decay + delta * ks[rg + kRowGroups * m];
        __syncthreads();  // qs/ks/part are rewritten by the next token
    }
#pragma unroll
    for (int m = 0; m < kRowsPerThread; ++m)
        __builtin_nontemporal_store(s[m], reinterpret_cast<f32x4*>(S + (rg + kRowGroups * m) * kDV + c0) + cb);
}

}  // namespace
}  // namespace gdn

using namespace gdn;

namespace {
hipError_t recurrent_launch(const void* q, const void* k, const void* v, const float* g,
                            const float* beta, void* o, float* state, int B, int T, int HV,
                            int HQK, int DK, int DV, hipStream_t stream, bool norm) {
    if (DK != kDK || DV != kDV || B <= 0 || T < 0 || HV <= 0 || HQK <= 0 || HV % HQK != 0)
        return hipErrorInvalidValue;
    if (!state) return hipErrorInvalidValue;
    if (T > 0 && (!q || !k || !v || !g || !beta || !o)) return hipErrorInvalidValue;
    if (T == 0) return hipSuccess;
    hipLaunchKernelGGL(norm ? gdn_recurrent_kernel<true> : gdn_recurrent_kernel<false>,
                       dim3((unsigned)(kDecSplit * B * HV)), dim3(kDecThreads), 0, stream,
                       static_cast<const uint16_t*>(q), static_cast<const uint16_t*>(k),
                       static_cast<const uint16_t*>(v), g, beta, static_cast<uint16_t*>(o), state,
                       T, HV, HQK, 1.0f / sqrtf((float)kDK));
    return hipGetLastError();
}
}  // namespace

extern "C" hipError_t deltanet_recurrent_step(const void* q, const void* k, const void* v,
                                              const float* g, const float* beta, void* o,
                                              float* state, int B, int T, int HV, int HQK,
                                              int DK, int DV, hipStream_t stream) {
    return recurrent_launch(q, k, v, g, beta, o, state, B, T, HV, HQK, DK, DV, stream, false);
}

extern "C" hipError_t deltanet_recurrent_step_l2norm(const void* q, const void* k, const void* v,
                                                     const float* g, const float* beta, void* o,
                                                     float* state, int B, int T, int HV,
                                                     int HQK, int DK, int DV,
                                                     hipStream_t stream) {
    return recurrent_launch(q, k, v, g, beta, o, state, B, T, HV, HQK, DK, DV, stream, true);
}
