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
// of one token.  A thread owns 8 channels and a run of consecutive tokens and
// keeps the K-token window in registers; neighbouring runs overlap by K-1
// rows (L2 hits).  HBM-bound: x read once, y written once.
#include "gdn_common.h"
#include "gdn_hip.h"

#include <math.h>

#include <atomic>

#include <algorithm>

namespace gdn {
namespace {

constexpr int kConvThreads = 256;
// The vector decode update has one thread per 4 channels, so at decode batch
// sizes (B = 64, D = 8192: 131,072 channels) 256-thread groups would fill
// only 128 of the CUs; 128-thread groups spread it over all of them (B = 64:
// 4.78 -> 4.74 us, B = 16: 2.96 -> 2.81 us, graph-replayed)
constexpr int kUpd4Threads = 128;
constexpr int kConvMaxRun = 12;     // longest token run of the many-rounds launch
constexpr int kConvFastMax = 24;    // longest token run of the one-or-two-rounds launch
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
    // the fp32 value must exist before it is rounded: fused into the
    // producing multiply-add (v_fma_mixlo_f16) the sum is rounded to fp16
    // once instead of to fp32 first, which differs in rare ties
    asm("" : "+v"(f));
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)f);
}

// 16-bit values of a packed pair (element 0 in the low half) as fp32
template <int IO>
__device__ inline float lo16(uint32_t u) {
    if constexpr (IO == 0) return __uint_as_float(u << 16);
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(u & 0xffffu));
}

template <int IO>
__device__ inline float hi16(uint32_t u) {
    if constexpr (IO == 0) return __uint_as_float(u & 0xffff0000u);
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(u >> 16));
}

// two fp32 values rounded to nearest-even 16-bit and packed (a low)
template <int IO>
__device__ inline uint32_t pack2(float a, float b) {
    if constexpr (IO == 0) {
        // one v_cvt_pk_bf16_f32 (written out: from the vector form the
        // compiler emits a conversion per element plus masking)
        uint32_t u;
        asm("v_cvt_pk_bf16_f32 %0, %1, %2" : "=v"(u) : "v"(a), "v"(b));
        return u;
    } else {
        return cv_store<1>(a) | (cv_store<1>(b) << 16);
    }
}

// SiLU r / (1 + e^-r) in fp32 from the hardware base-2 exponential and
// reciprocal (each within about an ulp).  Far below zero (r < -87) the
// reciprocal underflows to 0 and the result is -0, where exact arithmetic
// gives |y| < 1e-36.
__device__ inline float silu_f32(float r) {
    const float e = __builtin_amdgcn_exp2f(r * -1.44269504088896341f);
    return r * __builtin_amdgcn_rcpf(1.0f + e);
}

// one output: the fp32 sum rounded to the weight dtype (unless fp32), SiLU,
// rounded to the I/O dtype (16-bit pattern)
template <int IO, int WT, bool SILU>
__device__ inline uint32_t finish1(float acc) {
    float r = (WT == 2) ? acc : cv_load<WT>(cv_store<WT>(acc));
    if constexpr (SILU) r = silu_f32(r);
    return cv_store<IO>(r);
}

// the same for one token's 8 channels, packed in pairs
template <int IO, int WT, bool SILU>
__device__ inline u32x4 finish8(const float (&acc)[8]) {
    u32x4 out;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        float a = acc[2 * p], b = acc[2 * p + 1];
        if constexpr (WT != 2) {
            const uint32_t u = pack2<WT>(a, b);
            if constexpr (!SILU && WT == IO) {
                out[p] = u;
                continue;
            }
            a = lo16<WT>(u);
            b = hi16<WT>(u);
        }
        if constexpr (SILU) {
            a = silu_f32(a);
            b = silu_f32(b);
        }
        out[p] = pack2<IO>(a, b);
    }
    return out;
}

// Work units: (batch, token run, channel tile of 2048) with the channel tile
// fastest; runs have equal lengths but the last.  Two launch regimes:
//  - one or two rounds: when runs of at most kConvFastMax tokens can cover
//    the input with at most one (else two) work-groups per CU, the run is
//    sized so they do, in the instance with the smallest slot count kMaxRun
//    (1-4, 6, 8, ..., 24) that holds it.  Each wave issues all its rows at
//    once and turns them into outputs as they arrive, with no second round
//    to wait for; the x rows are read non-temporally.
//  - many rounds: otherwise runs of at most kConvMaxRun tokens, sized for
//    about two waves per SIMD, in the 12-slot instance.
// Measured at D = 8192, K = 4, bf16 with SiLU (graph-replayed over rotated
// copies): T = 1141 takes 9.2 us in one round of 18-token runs against 10.7
// us with 9-token runs over two waves per SIMD, and 0.84-0.97x of the
// many-rounds time from T = 64 to 3000; past that (T = 4096: 31.8 us) the
// many-rounds form is as fast as any run length.  A slot past the run
// re-reads the run's last row, which a non-temporal load takes from HBM
// again: 18-token runs in the 24-slot instance took 10.4 us, hence the
// close-fitting slot counts.
// Work-groups are dealt round-robin to the 8 XCDs (each with its own L2);
// remapping the work-group id gives every XCD one contiguous range of units,
// so the K-1 halo rows a run shares with the previous run are read from the
// same L2.
__device__ inline int xcd_unit(int id, int n) {
    const int q = n / 8, r = n % 8, xcd = id % 8;
    return xcd * q + min(xcd, r) + id / 8;
}

template <int IO, int WT, int K, bool SILU, bool BIAS, int kMaxRun, bool kNT>
__global__ __launch_bounds__(kConvThreads) void causal_conv1d_fwd_kernel(
    const uint16_t* __restrict__ x, const void* __restrict__ w, const void* __restrict__ bias,
    uint16_t* __restrict__ y, int T, int D, int64_t xbs, int64_t xts, int64_t ybs, int64_t yts,
    int n_ctiles, int n_runs, int run) {
    const int unit = xcd_unit(blockIdx.x, gridDim.x);
    const int ct = unit % n_ctiles;
    const int rest = unit / n_ctiles;
    const int t0 = (rest % n_runs) * run;
    const int b = rest / n_runs;
    const int d0 = (ct * kConvThreads + threadIdx.x) * 8;
    if (d0 >= D) return;
    const int len = min(run, T - t0);   // >= 1: the launcher makes n_runs = ceil(T / run)
    __builtin_assume(len >= 1);         // the first output is unconditional
    const uint16_t* xb = x + (size_t)b * xbs + d0;
    uint16_t* yb = y + (size_t)b * ybs + d0;
    // weights (and bias) first: loads complete in issue order, so the first
    // outputs can then start as soon as their own rows arrive
    float wf[8][K], bf[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
#pragma unroll
        for (int j = 0; j < K; ++j) wf[e][j] = ld_elem<WT>(w, (size_t)(d0 + e) * K + j);
        if constexpr (BIAS) bf[e] = ld_elem<WT>(bias, d0 + e);
    }
    // then all rows t0-K+1 .. t0+len-1; rows before 0 are zero, the slots
    // past the run re-read its last row
    constexpr int kRows = kMaxRun + K - 1;
    u32x4 raw[kRows];
#pragma unroll
    for (int i = 0; i < kRows; ++i) {
        const int tc = min(max(t0 - (K - 1) + i, 0), t0 + len - 1);
        const u32x4* p = reinterpret_cast<const u32x4*>(xb + (size_t)tc * xts);
        if constexpr (kNT) raw[i] = __builtin_nontemporal_load(p);
        else raw[i] = *p;   // cached: the K-1 halo rows come from L2
    }
    // every load is issued before any is waited for: the scheduler would
    // otherwise hold back later rows behind the first rows' use
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < K - 1; ++i)
        if (t0 - (K - 1) + i < 0) raw[i] = u32x4{0u, 0u, 0u, 0u};
    // sliding window of K unpacked rows: win[j] = row i + j
    float win[K][8];
#pragma unroll
    for (int j = 0; j < K - 1; ++j) {
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            win[j][2 * p] = lo16<IO>(raw[j][p]);
            win[j][2 * p + 1] = hi16<IO>(raw[j][p]);
        }
    }
    // Rows are unpacked outside the `i < len` guards, and the first output
    // is unconditional: a row read inside one guarded block only lets the
    // compiler sink its load into that block, where it is issued late and
    // waited for at once.
#pragma unroll
    for (int i = 0; i < kMaxRun; ++i) {
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            win[K - 1][2 * p] = lo16<IO>(raw[i + K - 1][p]);
            win[K - 1][2 * p + 1] = hi16<IO>(raw[i + K - 1][p]);
        }
        if (i < len) {   // uniform over the work-group
        float acc[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            // +0 start: an all-zero window gives +0, as a sum from zero
            float a = fmaf(wf[e][0], win[0][e], 0.0f);
#pragma unroll
            for (int j = 1; j < K; ++j) a = fmaf(wf[e][j], win[j][e], a);
            if constexpr (BIAS) a += bf[e];
            acc[e] = a;
        }
        const u32x4 out = finish8<IO, WT, SILU>(acc);
        __builtin_nontemporal_store(out, reinterpret_cast<u32x4*>(yb + (size_t)(t0 + i) * yts));
        }
#pragma unroll
        for (int j = 0; j < K - 1; ++j) {
#pragma unroll
            for (int e = 0; e < 8; ++e) win[j][e] = win[j + 1][e];
        }
    }
}

// Decode-time update: one thread per (batch, channel).  The window is the
// carried state (state_len tokens, oldest first) followed by the T new
// tokens; the outputs are the last T positions of the valid convolution over
// the window, and the state becomes the window's last state_len tokens
// (modeling_qwen3_5.py:200-216).  The window is read into registers before
// the state is rewritten, since the two overlap whenever T < state_len.
template <int IO, int WT, int K, bool SILU>
__global__ __launch_bounds__(kConvThreads) void causal_conv1d_update_kernel(
    const uint16_t* __restrict__ x, uint16_t* __restrict__ state, const void* __restrict__ w,
    const void* __restrict__ bias, uint16_t* __restrict__ y, int B, int T, int D, int state_len,
    int64_t xbs, int64_t xts, int64_t xds, int64_t sbs, int64_t sds, int64_t ybs, int64_t yts,
    int64_t yds) {
    const int64_t gid = (int64_t)blockIdx.x * kConvThreads + threadIdx.x;
    if (gid >= (int64_t)B * D) return;
    const int b = (int)(gid / D), d = (int)(gid - (int64_t)b * D);
    float wf[K];
#pragma unroll
    for (int j = 0; j < K; ++j) wf[j] = ld_elem<WT>(w, (size_t)d * K + j);
    const float bv = bias ? ld_elem<WT>(bias, d) : 0.f;   // added only with a bias
    uint16_t* st = state + (size_t)b * sbs + (size_t)d * sds;
    const uint16_t* xs = x + (size_t)b * xbs + (size_t)d * xds;
    uint16_t* ys = y + (size_t)b * ybs + (size_t)d * yds;
    // the old state (one 8-byte access for the common 4-token row), then a
    // rolling K-1 history of window values
    const bool row4 = state_len == 4 && sds == 4 && (reinterpret_cast<uintptr_t>(st) & 7) == 0;
    uint16_t old[kConvMaxState];
    if (row4) {
        const uint2 u = *reinterpret_cast<const uint2*>(st);
        old[0] = (uint16_t)u.x;
        old[1] = (uint16_t)(u.x >> 16);
        old[2] = (uint16_t)u.y;
        old[3] = (uint16_t)(u.y >> 16);
#pragma unroll
        for (int p = 4; p < kConvMaxState; ++p) old[p] = 0;
    } else {
#pragma unroll
        for (int p = 0; p < kConvMaxState; ++p) old[p] = p < state_len ? st[p] : (uint16_t)0;
    }
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
        float acc = fmaf(wf[0], hist[0], 0.0f);
#pragma unroll
        for (int j = 1; j < K; ++j) acc = fmaf(wf[j], hist[j], acc);
        if (bias) acc += bv;
        ys[(size_t)i * yts] = (uint16_t)finish1<IO, WT, SILU>(acc);
#pragma unroll
        for (int j = 0; j < K - 1; ++j) hist[j] = hist[j + 1];
    }
    // new state: the window's last state_len tokens.  Entry p is window index
    // q = (L - state_len) + p = T + p (L = state_len + T): an old state value
    // while q < state_len, else new token q - state_len.
    uint16_t ns[kConvMaxState];
#pragma unroll
    for (int p = 0; p < kConvMaxState; ++p) {
        const int q = T + p;
        uint16_t v = 0;
        if (p < state_len) {
            if (q < state_len) {
#pragma unroll
                for (int r = 0; r < kConvMaxState; ++r) v = (r == q) ? old[r] : v;
            } else {
                v = xs[(size_t)(q - state_len) * xts];
            }
        }
        ns[p] = v;
    }
    if (row4) {
        uint2 u;
        u.x = (uint32_t)ns[0] | ((uint32_t)ns[1] << 16);
        u.y = (uint32_t)ns[2] | ((uint32_t)ns[3] << 16);
        *reinterpret_cast<uint2*>(st) = u;
    } else {
#pragma unroll
        for (int p = 0; p < kConvMaxState; ++p)
            if (p < state_len) st[p] = ns[p];
    }
}

// The decode update for the Qwen3.5 shape (K = 4 taps, a state of 4
// tokens): one thread per (batch, 4 consecutive channels), so the state (4
// channels x 4 tokens, 32 bytes), the weights and a token of x or y each
// move in one or two vector accesses.  Same arithmetic per channel as the
// kernel above.  Requires unit channel strides for x and y, state rows of
// exactly 4 tokens, and the alignments the launcher checks.
template <int IO, int WT, bool SILU>
__global__ __launch_bounds__(kUpd4Threads) void causal_conv1d_update4_kernel(
    const uint16_t* __restrict__ x, uint16_t* __restrict__ state, const void* __restrict__ w,
    const void* __restrict__ bias, uint16_t* __restrict__ y, int B, int T, int D, int64_t xbs,
    int64_t xts, int64_t sbs, int64_t ybs, int64_t yts) {
    const int64_t gid = (int64_t)blockIdx.x * kUpd4Threads + threadIdx.x;
    const int D4 = D / 4;
    if (gid >= (int64_t)B * D4) return;
    const int b = (int)(gid / D4), d0 = 4 * (int)(gid - (int64_t)b * D4);
    // weights [d0 .. d0+3][0..3] and bias
    float wf[4][4], bv[4] = {0.f, 0.f, 0.f, 0.f};
    if constexpr (WT == 2) {
        const f32x4* wp = reinterpret_cast<const f32x4*>(static_cast<const float*>(w) + (size_t)d0 * 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const f32x4 r = wp[e];
#pragma unroll
            for (int j = 0; j < 4; ++j) wf[e][j] = r[j];
        }
        // without a bias the same load reads the weights and is dropped: no
        // branch, so every input load is issued before the first wait
        const f32x4 r = *reinterpret_cast<const f32x4*>(static_cast<const float*>(bias ? bias : w) + d0);
#pragma unroll
        for (int e = 0; e < 4; ++e) bv[e] = bias ? r[e] : 0.f;
    } else {
        const u32x4* wp = reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(w) + (size_t)d0 * 4);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const u32x4 r = wp[h];   // channels 2h, 2h+1: taps 0..3 each
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                wf[2 * h + p / 2][2 * (p % 2)] = lo16<WT>(r[p]);
                wf[2 * h + p / 2][2 * (p % 2) + 1] = hi16<WT>(r[p]);
            }
        }
        const uint2 r = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(bias ? bias : w) + d0);
        const bool hb = bias != nullptr;
        bv[0] = hb ? lo16<WT>(r.x) : 0.f;
        bv[1] = hb ? hi16<WT>(r.x) : 0.f;
        bv[2] = hb ? lo16<WT>(r.y) : 0.f;
        bv[3] = hb ? hi16<WT>(r.y) : 0.f;
    }
    // token 0 of x before the state (the launcher returns before T = 0);
    // each later token is requested while the previous one is computed
    const uint16_t* xb = x + (size_t)b * xbs + d0;
    uint16_t* yb = y + (size_t)b * ybs + d0;
    __builtin_assume(T >= 1);
    uint2 xr = *reinterpret_cast<const uint2*>(xb);
    // state rows: channel e's 4 tokens, oldest first, 8 bytes per channel
    uint16_t* st = state + (size_t)b * sbs + (size_t)d0 * 4;
    uint16_t win[4][4];   // [channel][slot]: the last 4 window tokens, oldest first
    {
        const u32x4 r0 = reinterpret_cast<const u32x4*>(st)[0];   // channels 0, 1
        const u32x4 r1 = reinterpret_cast<const u32x4*>(st)[1];   // channels 2, 3
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const u32x4 r = e < 2 ? r0 : r1;
            const uint32_t v = r[2 * (e % 2)], u = r[2 * (e % 2) + 1];
            win[e][0] = (uint16_t)v;
            win[e][1] = (uint16_t)(v >> 16);
            win[e][2] = (uint16_t)u;
            win[e][3] = (uint16_t)(u >> 16);
        }
    }
    for (int i = 0; i < T; ++i) {
        const uint16_t xe[4] = {(uint16_t)xr.x, (uint16_t)(xr.x >> 16), (uint16_t)xr.y,
                                (uint16_t)(xr.y >> 16)};
        if (i + 1 < T) xr = *reinterpret_cast<const uint2*>(xb + (size_t)(i + 1) * xts);
        uint32_t out[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            // window slots 1..3 and the new token are the 4 taps, oldest first
#pragma unroll
            for (int j = 0; j < 3; ++j) win[e][j] = win[e][j + 1];
            win[e][3] = xe[e];
            float acc = fmaf(wf[e][0], cv_load<IO>(win[e][0]), 0.0f);
#pragma unroll
            for (int j = 1; j < 4; ++j) acc = fmaf(wf[e][j], cv_load<IO>(win[e][j]), acc);
            if (bias) acc += bv[e];
            out[e] = finish1<IO, WT, SILU>(acc);
        }
        uint2 yo;
        yo.x = out[0] | (out[1] << 16);
        yo.y = out[2] | (out[3] << 16);
        *reinterpret_cast<uint2*>(yb + (size_t)i * yts) = yo;
    }
    // new state: the window's last 4 tokens per channel
    u32x4 n0, n1;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const uint32_t v = (uint32_t)win[e][0] | ((uint32_t)win[e][1] << 16);
        const uint32_t u = (uint32_t)win[e][2] | ((uint32_t)win[e][3] << 16);
        if (e < 2) {
            n0[2 * e] = v;
            n0[2 * e + 1] = u;
        } else {
            n1[2 * (e - 2)] = v;
            n1[2 * (e - 2) + 1] = u;
        }
    }
    reinterpret_cast<u32x4*>(st)[0] = n0;
    reinterpret_cast<u32x4*>(st)[1] = n1;
}

// Compute units of the current device, queried once per device (256 when
// the query fails).
int device_cus() {
    constexpr int kDevs = 64;
    static std::atomic<int> cache[kDevs];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kDevs) return 256;
    int n = cache[dev].load(std::memory_order_relaxed);
    if (n == 0) {
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            n <= 0)
            return 256;
        cache[dev].store(n, std::memory_order_relaxed);
    }
    return n;
}

// Run length of the one-or-two-rounds launch (at most kConvFastMax tokens,
// the grid at most `rounds` work-groups per CU), or 0 where it needs more.
int fast_run(int T, int64_t per_row, int cus) {
    for (int rounds = 1; rounds <= 2; ++rounds) {
        const int64_t n_runs = (int64_t)rounds * cus / per_row;
        if (n_runs < 1) continue;
        const int64_t run = (T + n_runs - 1) / n_runs;
        if (run <= kConvFastMax) return (int)run;
    }
    return 0;
}

template <int IO, int WT, bool SILU, bool BIAS>
hipError_t launch_fwd(const void* x, const void* w, const void* bias, void* y, int B, int T, int D,
                      int K, int64_t xbs, int64_t xts, int64_t ybs, int64_t yts,
                      hipStream_t stream) {
    const int n_ctiles = (D / 8 + kConvThreads - 1) / kConvThreads;
    const int cus = device_cus();
    const int64_t per_row = (int64_t)B * n_ctiles;
    auto xp = static_cast<const uint16_t*>(x);
    auto yp = static_cast<uint16_t*>(y);
    // one or two rounds: the transformers case (K = 4, weights in the I/O
    // dtype), slot counts 1..24 with at most one slot past the run
    if constexpr (IO == WT) {
        const int run = K == 4 ? fast_run(T, per_row, cus) : 0;
        if (run > 0) {
            const int n_runs = (T + run - 1) / run;
            const dim3 grid((unsigned)(per_row * n_runs));   // <= 2 x CUs
#define GDN_CONV_FAST(R)                                                                       \
    if (run <= R) {                                                                            \
        hipLaunchKernelGGL((causal_conv1d_fwd_kernel<IO, WT, 4, SILU, BIAS, R, true>), grid,    \
                           dim3(kConvThreads), 0, stream, xp, w, bias, yp, T, D, xbs, xts, ybs, \
                           yts, n_ctiles, n_runs, run);                                        \
        return hipGetLastError();                                                              \
    }
            GDN_CONV_FAST(1) GDN_CONV_FAST(2) GDN_CONV_FAST(3) GDN_CONV_FAST(4)
            GDN_CONV_FAST(6) GDN_CONV_FAST(8) GDN_CONV_FAST(10) GDN_CONV_FAST(12)
            GDN_CONV_FAST(14) GDN_CONV_FAST(16) GDN_CONV_FAST(18) GDN_CONV_FAST(20)
            GDN_CONV_FAST(22) GDN_CONV_FAST(24)
#undef GDN_CONV_FAST
            static_assert(kConvFastMax == 24, "the slot counts above end at kConvFastMax");
        }
    }
    // many rounds: about two waves per SIMD (2 work-groups of 4 waves per
    // CU), runs of equal length up to kConvMaxRun tokens
    int64_t n_runs = (2LL * cus + per_row / 2) / per_row;
    n_runs = std::max<int64_t>(1, std::min<int64_t>(n_runs, T));
    int run = (int)((T + n_runs - 1) / n_runs);
    run = std::min(run, kConvMaxRun);
    n_runs = (T + run - 1) / run;
    const int64_t units = per_row * n_runs;
    if (units > 0x7fffffff) return hipErrorInvalidValue;
    const dim3 grid((unsigned)units);
#define GDN_CONV_FWD(KK)                                                                       \
    case KK:                                                                                   \
        hipLaunchKernelGGL((causal_conv1d_fwd_kernel<IO, WT, KK, SILU, BIAS, kConvMaxRun,      \
                                                     false>),                                  \
                           grid, dim3(kConvThreads), 0, stream, xp, w, bias, yp, T, D, xbs,    \
                           xts, ybs, yts, n_ctiles, (int)n_runs, run);                         \
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
hipError_t launch_fwd_any(const void* x, const void* w, const void* bias, void* y, int B, int T,
                          int D, int K, int64_t xbs, int64_t xts, int64_t ybs, int64_t yts,
                          int silu, hipStream_t stream) {
#define GDN_FWD_CALL(S, BI) \
    launch_fwd<IO, WT, S, BI>(x, w, bias, y, B, T, D, K, xbs, xts, ybs, yts, stream)
    if (silu) return bias ? GDN_FWD_CALL(true, true) : GDN_FWD_CALL(true, false);
    return bias ? GDN_FWD_CALL(false, true) : GDN_FWD_CALL(false, false);
#undef GDN_FWD_CALL
}

template <int IO, int WT>
hipError_t launch_update(const void* x, void* state, const void* w, const void* bias, void* y,
                         int B, int T, int D, int K, int state_len, int64_t xbs, int64_t xts,
                         int64_t xds, int64_t sbs, int64_t sds, int64_t ybs, int64_t yts,
                         int64_t yds, int silu, hipStream_t stream) {
    // the vector path: K = 4, 4-token state rows, unit channel strides, and
    // every vector access aligned (x, y: 8 bytes per 4 channels; state and
    // weights: 16; bias: 8, or 16 in fp32)
    const auto al = [](const void* p, uintptr_t a) {
        return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0;
    };
    if (K == 4 && state_len == 4 && sds == 4 && xds == 1 && yds == 1 && D % 4 == 0 &&
        (B <= 1 || (xbs % 4 == 0 && ybs % 4 == 0 && sbs % 8 == 0)) &&
        (T <= 1 || (xts % 4 == 0 && yts % 4 == 0)) && al(x, 8) && al(y, 8) && al(state, 16) &&
        al(w, 16) && (!bias || al(bias, WT == 2 ? 16 : 8))) {
        const int64_t n4 = (int64_t)B * (D / 4);
        const dim3 grid4((unsigned)((n4 + kUpd4Threads - 1) / kUpd4Threads));
        auto xp = static_cast<const uint16_t*>(x);
        auto sp = static_cast<uint16_t*>(state);
        auto yp = static_cast<uint16_t*>(y);
        const int64_t xb = B <= 1 ? 0 : xbs, yb = B <= 1 ? 0 : ybs, sb = B <= 1 ? 0 : sbs;
        if (silu)
            hipLaunchKernelGGL((causal_conv1d_update4_kernel<IO, WT, true>), grid4,
                               dim3(kUpd4Threads), 0, stream, xp, sp, w, bias, yp, B, T, D, xb,
                               xts, sb, yb, yts);
        else
            hipLaunchKernelGGL((causal_conv1d_update4_kernel<IO, WT, false>), grid4,
                               dim3(kUpd4Threads), 0, stream, xp, sp, w, bias, yp, B, T, D, xb,
                               xts, sb, yb, yts);
        return hipGetLastError();
    }
    const int64_t n = (int64_t)B * D;
    const dim3 grid((unsigned)((n + kConvThreads - 1) / kConvThreads));
    auto xp = static_cast<const uint16_t*>(x);
    auto sp = static_cast<uint16_t*>(state);
    auto yp = static_cast<uint16_t*>(y);
#define GDN_CONV_UPD(KK)                                                                        \
    case KK:                                                                                    \
        if (silu)                                                                               \
            hipLaunchKernelGGL((causal_conv1d_update_kernel<IO, WT, KK, true>), grid,          \
                               dim3(kConvThreads), 0, stream, xp, sp, w, bias, yp, B, T, D,     \
                               state_len, xbs, xts, xds, sbs, sds, ybs, yts, yds);              \
        else                                                                                    \
            hipLaunchKernelGGL((causal_conv1d_update_kernel<IO, WT, KK, false>), grid,         \
                               dim3(kConvThreads), 0, stream, xp, sp, w, bias, yp, B, T, D,     \
                               state_len, xbs, xts, xds, sbs, sds, ybs, yts, yds);              \
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
    if (B == 0 || T == 0) return hipSuccess;
    if (!x || !w || !y) return hipErrorInvalidValue;
    // 16-byte lane accesses: every row start must stay 16-byte aligned
    if ((x_bstride | x_tstride | y_bstride | y_tstride) % 8 != 0 ||
        ((uintptr_t)x | (uintptr_t)y) % 16 != 0)
        return hipErrorInvalidValue;
    const bool bf = io_dtype == GDN_DTYPE_BF16, w32 = w_dtype == GDN_DTYPE_FP32;
#define GDN_FWD_ARGS x, w, bias, y, B, T, D, K, x_bstride, x_tstride, y_bstride, y_tstride, silu, stream
    if (bf) return w32 ? launch_fwd_any<0, 2>(GDN_FWD_ARGS) : launch_fwd_any<0, 0>(GDN_FWD_ARGS);
    return w32 ? launch_fwd_any<1, 2>(GDN_FWD_ARGS) : launch_fwd_any<1, 1>(GDN_FWD_ARGS);
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
