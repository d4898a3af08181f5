// Chunked gated-delta-rule prefill for gfx950 (MI355X).
//
// Replaces the reference's four-kernel CUDA pipeline behind
// kernels/chunk_delta_cuda.h:39-55 (deltanet_prefill_workspace_size /
// deltanet_chunk_prefill).  Math per (sequence, v-head), chunk C = 64, with
// q, k rows of the v-head's k-head and s = 1/sqrt(DK):
//
//   c   = cumsum(g)            Gamma_rj = exp(c_r - c_j)  (r >= j)
//   A   = -diag(beta) (K K^T o Gamma)  strictly lower,   T = (I - A)^-1
//   M   = s (Q K^T o Gamma)    lower incl. diagonal
//   V_n = T diag(beta) V - T diag(beta e^c) K S           (= U - W S)
//   O   = diag(s e^c) Q S + M V_n
//   S  <- e^{c_63} S + K^T diag(e^{c_63 - c}) V_n
//
// (transformers modeling_qwen3_5.py:249-327, the reference's parity oracle;
// kernels/chunk_delta_cuda.cu:91-303, :312-424 and :532-674 compute the same
// terms with U, W and the decayed K kept in a workspace.)
//
// Here V_n is formed T-factored: R = beta o V - (beta e^c) o (K S), then
// V_n = R + (T - I) R.  The scan therefore needs only T - I and M per
// chunk-head from the prep (12 KB, fp16 fragments); K, Q and V come straight
// from the inputs.  The state update K^T (d o V_n) takes d o V_n as an fp16
// hi/lo pair, whose lo part goes to a second accumulator off the serial path.
//
// Two kernels:
//   prep  one work-group per (chunk, v-head): gates, K K^T and Q K^T on bf16
//         MFMA, the inverse T in fp32 (16x16 diagonal blocks by forward
//         substitution, off-diagonal blocks on fp32 MFMA), then T - I and M as
//         fp16 MFMA fragments.
//   scan  four work-groups per (sequence, v-head), each owning 32 value
//         columns of the state as two 16-column slices.  Per chunk a chain
//         wave per slice forms P = K S, V_n and S', with S in registers for the
//         whole sequence; one output wave forms O for both slices; three
//         loader waves stream K and Q (converted to fp16), V, T - I, M and the
//         gates into LDS rings.  Waves meet through LDS counters with bounded
//         waits; a wait that runs out aborts the work-group and sets the
//         workspace's status word (deltanet_prefill_status).
//
// The fused entry (deltanet_chunk_prefill_fused) and the l2norm entry run the
// same kernels on raw inputs: both kernels L2-normalise q and k rows as they
// load them, convert fp16 inputs, form g and beta from the gate inputs, and
// the scan stores o in the I/O dtype and the final state over the initial one.
#include "gdn_common.h"
#include "gdn_hip.h"
#include "gdn_hip_diag.h"
#include "gdn_seq.h"

#include <math.h>

#include <algorithm>

namespace gdn {
namespace {

constexpr int kPrepThreads = 256;
constexpr int kScanThreads = 512;
constexpr int kPairCols = 32;                      // value columns per scan work-group
constexpr int kPairsPerHead = kDV / kPairCols;     // 4
constexpr int kTri = 6;                            // nonzero (row tile, k-block) fragments of a lower-triangular 64x64
constexpr int kGateDecay = 64;
constexpr unsigned kDefaultSpin = 1u << 20;        // bounded waits: ~0.1 s of polling, then give up

// First fragment index of row tile mt among the kTri lower-triangular ones:
// (0,0) (1,0) (2,0) (2,1) (3,0) (3,1)
__host__ __device__ constexpr int tri_base(int mt) { return mt < 3 ? mt : 4; }

// Per chunk-head workspace record: (T - I) and M, kTri A-fragments each (fp16,
// 16 bytes per lane).  A 256-byte header in front holds the status word.
constexpr size_t kTriBytes = (size_t)kTri * 64 * 16;   // 6 KB
constexpr size_t kHeaderBytes = 256;

struct Workspace {
    half8* TI;          // (T - I) fragments [chunk-head][kTri][64]
    half8* M;           // M fragments, same layout
    unsigned* status;   // bit 0: a bounded wait gave up
    float* dbgT;        // optional [chunk-head][64][64]: T = (I - A)^-1
    float* dbgA;        // optional: A
    float* dbgTp;       // optional: T after the diagonal-block inversion (A below the blocks)
    float* dbgM;        // optional: M
    float* dbgC;        // optional [chunk-head][64]: in-chunk cumsum of g
    float* dbgS;        // optional [chunk-head][128][128]: state at the chunk's start
};

__host__ __device__ inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

// Byte layout of the workspace for `nch` chunk-heads.  The debug regions stay
// last: the torch binding finds them from the end.
struct WsLayout {
    size_t ti, m, dbgT, dbgA, dbgTp, dbgM, dbgC, dbgS, live, total;
    __host__ explicit WsLayout(size_t nch) {
        size_t off = kHeaderBytes;
        ti = off;    off += align256(nch * kTriBytes);
        m = off;     off += align256(nch * kTriBytes);
        live = off;
        dbgT = off;  off += align256(nch * kChunk * kChunk * 4);
        dbgA = off;  off += align256(nch * kChunk * kChunk * 4);
        dbgTp = off; off += align256(nch * kChunk * kChunk * 4);
        dbgM = off;  off += align256(nch * kChunk * kChunk * 4);
        dbgC = off;  off += align256(nch * kChunk * 4);
        dbgS = off;  off += align256(nch * (size_t)kDK * kDV * 4);
        total = off;
    }
};

// Inputs.  kRaw = 0: q, k (L2-normalised) and v are bf16, g and beta fp32.
// kRaw = 1 / 2: q and k rows are raw bf16 / fp16 (normalised while loaded), v
// has the same dtype, and the gates are g and beta (fp32) when `a` is null,
// else they come from a, b (per token and v-head, same dtype), A_log (fp32)
// and dt_bias (same dtype) per v-head.
struct PrepIn {
    const uint16_t* q;
    const uint16_t* k;
    const uint16_t* v;
    const float* g;
    const float* beta;
    const uint16_t* a;
    const uint16_t* b;
    const float* A_log;
    const uint16_t* dt_bias;
};

// ---------------------------------------------------------------------------
// element helpers
// ---------------------------------------------------------------------------
// A raw 16-bit input element as fp32 (kRaw 0/1: bf16, 2: fp16)
template <int kRaw>
__device__ inline float raw16(uint32_t bits) {
    if constexpr (kRaw == 2) return (float)__builtin_bit_cast(_Float16, (uint16_t)bits);
    return __uint_as_float(bits << 16);
}

__device__ inline uint16_t f16_bits(float x) { return __builtin_bit_cast(uint16_t, (_Float16)x); }

// The fused entry's gate math (export/patches/orin_text_engine/files/cpp/
// kernels/gdnKernels/gdnChunkPrefillSm87.cu:44-49,113-125): g = -e^{A_log}
// softplus(a + dt_bias), softplus(x) = x above 20, else log1p(e^x); and
// beta = 1 / (1 + e^-b), all in fp32.
__device__ inline void gate_from_raw(float a, float b, float A_log, float dt_bias, float& g,
                                     float& beta) {
    const float x = a + dt_bias;
    g = -expf(A_log) * (x > 20.f ? x : log1pf(expf(x)));
    beta = 1.f / (1.f + expf(-b));
}

// g and beta of one token of v-head hv (index gi = token * HV + hv).
template <int kRaw>
__device__ inline void load_gate(const PrepIn& in, size_t gi, int hv, float& g, float& beta) {
    if (kRaw != 0 && in.a != nullptr) {
        gate_from_raw(raw16<kRaw>(in.a[gi]), raw16<kRaw>(in.b[gi]), in.A_log[hv],
                      raw16<kRaw>(in.dt_bias[hv]), g, beta);
    } else {
        g = in.g[gi];
        beta = in.beta[gi];
    }
}

// Eight 16-bit row elements (one 16-byte piece) of a 128-wide row spread over
// 16 consecutive lanes: for kRaw != 0 the row is L2-normalised, x rsqrt(sum
// x^2 + 1e-6) in fp32 and rounded to bf16 (the reference adapter's
// normalisation, gdnChunkPrefillSm87.cu:52-84; transformers l2norm,
// modeling_qwen3_5.py:242-245); the result is returned as fp16, which holds
// every such bf16 value exactly in fp16's normal range.
template <int kRaw>
__device__ inline half8 row_piece_to_half8(u32x4 w) {
    float x[8];
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        x[2 * p] = raw16<kRaw>(w[p] & 0xffffu);
        x[2 * p + 1] = raw16<kRaw>(w[p] >> 16);
    }
    if constexpr (kRaw != 0) {
        float ss = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) ss = fmaf(x[e], x[e], ss);
#pragma unroll
        for (int off = 1; off < 16; off <<= 1) ss += __shfl_xor(ss, off, 64);
        const float inv = rsqrtf(ss + 1e-6f);
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = (float)(__bf16)(x[e] * inv);
    }
    half8 h;
#pragma unroll
    for (int e = 0; e < 8; ++e) h[e] = (_Float16)x[e];
    return h;
}

__device__ __forceinline__ f32x4 mfma_f32_16x16x4(float a, float b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// LDS transposing read (ds_read_b64_tr_b16).  Within each 16-lane group,
// source lane s names 4 consecutive 16-bit elements X[s][0..3]; lane i
// receives X[4 j + i / 4][i % 4] in element j.
typedef short s16x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ s16x4 lds_read_tr(const void* p) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)p);
}

__device__ __forceinline__ half4 s16x4_as_half4(s16x4 v) { return __builtin_bit_cast(half4, v); }

constexpr float kLog2e = 1.4426950408889634f;

// ---------------------------------------------------------------------------
// Block-cooperative sequence lookups (clamped cu_seqlens, gdn_seq.h)
// ---------------------------------------------------------------------------
// Prefix sums of chunk counts saturate at kSatChunks, far above any chunk
// bound a workspace can hold, so even adversarial cu_seqlens cannot wrap them.
constexpr int kSatChunks = 1 << 30;

__host__ __device__ inline int sat_add(int a, int b) {
    const long long s = (long long)a + b;
    return s > kSatChunks ? kSatChunks : (int)s;
}

// Number of chunks in sequences [0, upto) (saturating); every thread calls it.
template <int NT>
__device__ int chunks_before(const int32_t* cu, int T, int total, int upto, int* red) {
    if (!cu) return upto * ((T + kChunk - 1) / kChunk);
    int acc = 0;
    for (int s = threadIdx.x; s < upto; s += NT) acc = sat_add(acc, seq_chunks(cu, T, total, s));
    for (int off = 32; off > 0; off >>= 1) acc = sat_add(acc, __shfl_xor(acc, off, 64));
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
    __syncthreads();
    int tot = 0;
    for (int w = 0; w < NT / 64; ++w) tot = sat_add(tot, red[w]);
    __syncthreads();
    return tot;
}

// Global chunk id -> (sequence, first token, rows); false (uniformly) when cid
// is past the last chunk.  `red` holds NT ints of scratch.
template <int NT>
__device__ bool locate_chunk(const int32_t* cu, int N, int T, int total, int cid, int* red,
                             int& seq, int& tok0, int& rows) {
    if (!cu) {
        const int nc = (T + kChunk - 1) / kChunk;
        if (nc == 0 || cid >= N * nc) return false;
        seq = cid / nc;
        const int c = cid - seq * nc;
        tok0 = seq * T + c * kChunk;
        rows = min(kChunk, T - c * kChunk);
        return true;
    }
    int base = 0;
    bool found = false;
    for (int s0 = 0; s0 < N && base < kSatChunks; s0 += NT) {
        const int s = s0 + (int)threadIdx.x;
        const int cnt = (s < N) ? seq_chunks(cu, T, total, s) : 0;
        __syncthreads();
        red[threadIdx.x] = cnt;
        __syncthreads();
        for (int off = 1; off < NT; off <<= 1) {
            const int add = (threadIdx.x >= (unsigned)off) ? red[threadIdx.x - off] : 0;
            __syncthreads();
            red[threadIdx.x] = sat_add(red[threadIdx.x], add);
            __syncthreads();
        }
        const int incl = red[threadIdx.x];
        const int blk = red[NT - 1];
        const int excl = incl - cnt;   // exact wherever incl has not saturated
        __syncthreads();
        if (cnt > 0 && incl < kSatChunks && cid >= base + excl && cid < base + incl) {
            red[0] = s;
            red[1] = cid - base - excl;
        }
        __syncthreads();
        if (cid < sat_add(base, blk)) {
            seq = red[0];
            const int c = red[1];
            tok0 = seq_lo(cu, T, total, seq) + c * kChunk;
            rows = min(kChunk, seq_count(cu, T, total, seq) - c * kChunk);
            found = true;
        }
        __syncthreads();
        base = sat_add(base, blk);
        if (found) break;
    }
    return found;
}

// ---------------------------------------------------------------------------
// prep kernel: one work-group (4 waves) per (chunk, v-head)
// ---------------------------------------------------------------------------
constexpr int kKS = kDK + 8;      // bf16 K row pitch: 136 halves (272 B, 16-byte aligned)
constexpr int kMS = kChunk + 4;   // fp32 A / T row pitch: 68 floats

struct PrepSmem {
    uint16_t Kr[kChunk * kKS];   // K rows (bf16), [token][dk]
    // A (strictly lower, row-major) on entry.  The inverse overwrites it in
    // place: diagonal blocks T_ii row-major at (i, i); T_ij (i > j) stored
    // transposed at block (j, i), where A is zero and never read.  Its first
    // 1 KB is the sequence-lookup scratch before that.
    float AT[kChunk * kMS];
    float cl[kChunk];   // c * log2(e)
    float b[kChunk];    // beta
};

// T[r][c0 .. c0+3] (c0 a multiple of 4) from the in-place inverse layout.
// Row block rb and column block cb are uniform, so the branch is too.
__device__ inline f32x4 t_row4(const float* AT, int rb, int cb, int r, int c0) {
    if (cb == rb) return *reinterpret_cast<const f32x4*>(&AT[r * kMS + c0]);
    if (cb > rb) return zero4();
    f32x4 t;
#pragma unroll
    for (int e = 0; e < 4; ++e) t[e] = AT[(c0 + e) * kMS + r];
    return t;
}

// Two 4-element bf16 pieces (k-map registers 0..3 and 4..7) as one operand
__device__ inline bf16x8 bf16_frag(uint2 lo, uint2 hi) {
    const u32x4 w = {lo.x, lo.y, hi.x, hi.y};
    return __builtin_bit_cast(bf16x8, w);
}

// K K^T and K Q^T products of wave W: A column block W (row tiles W..3) and
// M^T column block W (row tiles 0..W), k-blocks outermost so the five
// accumulators' products interleave.
template <int W>
__device__ inline void am_products(const bf16x8 (&ka)[4][4], const bf16x8 (&qf)[4],
                                   f32x4 (&accA)[4], f32x4 (&accM)[4]) {
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
        accA[mt] = zero4();
        accM[mt] = zero4();
    }
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
        for (int mt = W; mt < 4; ++mt) accA[mt] = mfma16_bf16(ka[mt][kb], ka[W][kb], accA[mt]);
#pragma unroll
        for (int mt = 0; mt <= W; ++mt) accM[mt] = mfma16_bf16(ka[mt][kb], qf[kb], accM[mt]);
    }
}

// bf16 pair of a raw 16-bit pair, L2-scaled by inv (kRaw != 0)
template <int kRaw>
__device__ inline uint32_t norm_pair(uint32_t w, float inv) {
    const float lo = raw16<kRaw>(w & 0xffffu) * inv, hi = raw16<kRaw>(w >> 16) * inv;
    return (uint32_t)f32_to_bf16_bits(lo) | ((uint32_t)f32_to_bf16_bits(hi) << 16);
}

template <int kRaw>
__device__ inline float sumsq_pair(uint32_t w, float s) {
    const float lo = raw16<kRaw>(w & 0xffffu), hi = raw16<kRaw>(w >> 16);
    return fmaf(hi, hi, fmaf(lo, lo, s));
}

template <bool kDbg, int kRaw>
__global__ __launch_bounds__(kPrepThreads, 4) void gdn_prep_kernel(
    PrepIn in, const int32_t* __restrict__ cu, int N, int T, int total, int HV, int HK,
    int nch_bound, float scale, Workspace ws) {
    __shared__ PrepSmem sm;
    const uint16_t* __restrict__ q = in.q;
    const uint16_t* __restrict__ k = in.k;
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int lg = lane >> 4, lm = lane & 15;

    // this call's status word starts clear (the scan runs after this kernel)
    if (blockIdx.x == 0 && tid == 0) ws.status[0] = 0u;

    // Work-group id -> (chunk, k-head, member of its GQA group).  The rep
    // v-heads that read one k-head get ids 8 apart, i.e. the same XCD, so
    // their q / k rows come from one L2.
    const int rep = HV / HK;
    const int L = blockIdx.x;
    const int rest = L >> 3;
    const int z = (rest / rep) * 8 + (L & 7);
    const int cid = z / HK, hk = z - cid * HK;
    if (cid >= nch_bound) return;
    const int hv = hk * rep + (rest % rep);

    int seq, tok0, rows;
    if (!locate_chunk<kPrepThreads>(cu, N, T, total, cid, reinterpret_cast<int*>(sm.AT), seq,
                                    tok0, rows))
        return;
    (void)seq;
    const size_t ch = (size_t)cid * HV + hv;

    // ---- global loads, all issued before any is consumed.  Rows past the
    // chunk's end read the last valid row and are zeroed afterwards.
    float gv = 0.f, bv = 0.f;
    uint32_t ga = 0u, gb = 0u, gdt = 0u;
    float gAl = 0.f;
    const bool raw_gate = kRaw != 0 && in.a != nullptr;
    if (wave == 0) {
        const size_t gi = (size_t)(tok0 + min(lane, rows - 1)) * HV + hv;
        if (!raw_gate) {
            ga = __float_as_uint(in.g[gi]);
            gb = __float_as_uint(in.beta[gi]);
        } else {
            ga = in.a[gi];
            gb = in.b[gi];
            gAl = in.A_log[hv];
            gdt = in.dt_bias[hv];
        }
    }
    u32x4 raw[4];
    {
        const uint16_t* base = k + ((size_t)tok0 * HK + hk) * kDK + 8 * (tid & 15);
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) {
            const int r = min((tid >> 4) + 16 * ii, rows - 1);
            raw[ii] = *reinterpret_cast<const u32x4*>(base + (size_t)r * HK * kDK);
        }
    }
    uint2 qr[4][2];
    {
        const uint16_t* qs =
            q + ((size_t)(tok0 + min(wave * 16 + lm, rows - 1)) * HK + hk) * kDK + 4 * lg;
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
            qr[kb][0] = *reinterpret_cast<const uint2*>(qs + kb * 32);
            qr[kb][1] = *reinterpret_cast<const uint2*>(qs + kb * 32 + 16);
        }
    }
    // the gate arithmetic (and so the wait for its inputs) stays behind the
    // K and Q loads
    asm volatile("" : "+v"(ga), "+v"(gb), "+v"(gdt), "+v"(gAl)::"memory");
    if (wave == 0) {
        if (!raw_gate) {
            gv = __uint_as_float(ga);
            bv = __uint_as_float(gb);
        } else {
            gate_from_raw(raw16<kRaw>(ga), raw16<kRaw>(gb), gAl, raw16<kRaw>(gdt), gv, bv);
        }
    }

    if constexpr (kRaw != 0) {
        // raw inputs: K rows (16 lanes per row, 8 values each) and Q rows (4
        // lanes per row, 32 values each) L2-normalised and rounded to bf16
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) {
            float ss = 0.f;
#pragma unroll
            for (int p = 0; p < 4; ++p) ss = sumsq_pair<kRaw>(raw[ii][p], ss);
#pragma unroll
            for (int off = 1; off < 16; off <<= 1) ss += __shfl_xor(ss, off, 64);
            const float inv = rsqrtf(ss + 1e-6f);
#pragma unroll
            for (int p = 0; p < 4; ++p) raw[ii][p] = norm_pair<kRaw>(raw[ii][p], inv);
        }
        {
            float ss = 0.f;
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
                for (int h2 = 0; h2 < 2; ++h2) {
                    ss = sumsq_pair<kRaw>(qr[kb][h2].x, ss);
                    ss = sumsq_pair<kRaw>(qr[kb][h2].y, ss);
                }
            }
            ss += __shfl_xor(ss, 16, 64);
            ss += __shfl_xor(ss, 32, 64);
            const float inv = rsqrtf(ss + 1e-6f);
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
                for (int h2 = 0; h2 < 2; ++h2) {
                    qr[kb][h2].x = norm_pair<kRaw>(qr[kb][h2].x, inv);
                    qr[kb][h2].y = norm_pair<kRaw>(qr[kb][h2].y, inv);
                }
            }
        }
    }

    // ---- gates (wave 0): c = cumsum(g); padded rows have g = beta = 0
    if (wave == 0) {
        if (lane >= rows) {
            gv = 0.f;
            bv = 0.f;
        }
        float cs = gv;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const float o = __shfl_up(cs, off, 64);
            if (lane >= off) cs += o;
        }
        sm.cl[lane] = cs * kLog2e;
        sm.b[lane] = bv;
        if (kDbg) ws.dbgC[ch * kChunk + lane] = cs;
    }

    // ---- K rows -> LDS as loaded; rows past the chunk's end are zeroed
#pragma unroll
    for (int ii = 0; ii < 4; ++ii) {
        const int r = (tid >> 4) + 16 * ii;
        const uint32_t m = r < rows ? 0xffffffffu : 0u;
        *reinterpret_cast<u32x4*>(&sm.Kr[r * kKS + 8 * (tid & 15)]) = raw[ii] & m;
    }
    __syncthreads();

    // ---- A = -beta_r (k_r . k_j) Gamma_rj (r > j) and M = s (q_r . k_j) Gamma_rj (r >= j)
    // Wave w owns column block j in [16w, 16w+16) of A and query-row block
    // r in [16w, 16w+16) of M (computed as M^T = K Q^T, whose accumulators are
    // already the M fragments the scan reads).
    {
        const uint2 z2 = {0u, 0u};
        bf16x8 ka[4][4], qf[4];
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
            const uint16_t* src = &sm.Kr[(mt * 16 + lm) * kKS + 4 * lg];
#pragma unroll
            for (int kb = 0; kb < 4; ++kb)
                ka[mt][kb] = bf16_frag(*reinterpret_cast<const uint2*>(src + kb * 32),
                                       *reinterpret_cast<const uint2*>(src + kb * 32 + 16));
        }
        {
            const bool ok = wave * 16 + lm < rows;
#pragma unroll
            for (int kb = 0; kb < 4; ++kb)
                qf[kb] = bf16_frag(ok ? qr[kb][0] : z2, ok ? qr[kb][1] : z2);
        }
        f32x4 accA[4], accM[4];
        switch (wave) {
            case 0: am_products<0>(ka, qf, accA, accM); break;
            case 1: am_products<1>(ka, qf, accA, accM); break;
            case 2: am_products<2>(ka, qf, accA, accM); break;
            default: am_products<3>(ka, qf, accA, accM); break;
        }
        // A: element (r = 16mt + 4lg + i, col = 16w + lm); the upper part of
        // column block w is written as zero (every element computed, then
        // selected: the discarded exponentials may overflow harmlessly)
        const int col = wave * 16 + lm;
        const float ccol = sm.cl[col];
        f32x4 clr[4], br[4];
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
            clr[mt] = *reinterpret_cast<const f32x4*>(&sm.cl[mt * 16 + 4 * lg]);
            br[mt] = *reinterpret_cast<const f32x4*>(&sm.b[mt * 16 + 4 * lg]);
        }
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int r = mt * 16 + 4 * lg + i;
                const float av = -br[mt][i] * accA[mt][i] * __builtin_amdgcn_exp2f(clr[mt][i] - ccol);
                const float a = r > col ? av : 0.f;
                sm.AT[r * kMS + col] = a;
                if (kDbg) ws.dbgA[ch * kChunk * kChunk + r * kChunk + col] = a;
            }
        }
        // M^T tile (key tile mt, query tile w): element (key = 16mt + 4lg + i,
        // query = col); M fragment (w, kb) = key tiles 2kb, 2kb+1
        half4 mh[4];
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
            f32x4 val;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int key = mt * 16 + 4 * lg + i;
                const float mv = scale * accM[mt][i] * __builtin_amdgcn_exp2f(ccol - clr[mt][i]);
                val[i] = key <= col ? mv : 0.f;
                if (kDbg) ws.dbgM[ch * kChunk * kChunk + col * kChunk + key] = val[i];
            }
            mh[mt] = to_half4(val);
        }
        half8* mdst = ws.M + ch * (kTri * 64);
        mdst[tri_base(wave) * 64 + lane] = cat8(mh[0], mh[1]);
        if (wave >= 2) mdst[(tri_base(wave) + 1) * 64 + lane] = cat8(mh[2], mh[3]);
    }
    __syncthreads();

    // ---- T = (I - A)^-1 in fp32, in place in AT
    // (1) 16x16 diagonal blocks by forward substitution: wave 0, lane =
    //     16 * block + column; T[i][c] = sum_{j<i} A[i][j] T[j][c] for i > c,
    //     T[c][c] = 1, T[i][c] = 0 for i < c.  Each lane keeps its column in
    //     registers and writes it after every row of the block was read.
    if (wave == 0) {
        const int b0 = lg * 16, cidx = lm;
        float colv[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) colv[i] = (i == cidx) ? 1.f : 0.f;
#pragma unroll
        for (int i = 1; i < 16; ++i) {
            const float* arow = &sm.AT[(b0 + i) * kMS + b0];
            float s = 0.f;
#pragma unroll
            for (int j4 = 0; j4 < (i + 3) / 4; ++j4) {
                const f32x4 a4 = *reinterpret_cast<const f32x4*>(arow + 4 * j4);
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (4 * j4 + e < i) s = fmaf(a4[e], colv[4 * j4 + e], s);
            }
            if (i > cidx) colv[i] = s;
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) sm.AT[(b0 + i) * kMS + b0 + cidx] = colv[i];
    }
    __syncthreads();
    if (kDbg) {
        // T right after the diagonal blocks are inverted (A below them), as
        // the reference's post-leaf view (kernels/chunk_delta_cuda.cu:211-215)
        for (int e = tid; e < kChunk * kChunk; e += kPrepThreads) {
            const int r = e >> 6, c = e & 63;
            ws.dbgTp[ch * kChunk * kChunk + e] =
                ((r >> 4) == (c >> 4) || r > c) ? sm.AT[r * kMS + c] : 0.f;
        }
    }
    // (2) off-diagonal blocks level by level, block (i, j) with i - j = d:
    //     T_ij = T_ii * sum_{kk=j}^{i-1} A_{i,kk} T_{kk,j}
    //     on fp32 MFMA 16x16x4 with k = 4 * lane group + s, so the A operand
    //     is one 16-byte row read and a D-layout accumulator is directly the
    //     B operand of the next product.  Wave w takes block (w + d, w).
#pragma unroll
    for (int d = 1; d <= 3; ++d) {
        if (wave < 4 - d) {
            const int j = wave, i = wave + d;
            f32x4 Pu[3];
#pragma unroll
            for (int u = 0; u < d; ++u) {
                const int kk = j + u;
                const f32x4 a = *reinterpret_cast<const f32x4*>(&sm.AT[(16 * i + lm) * kMS + 16 * kk + 4 * lg]);
                f32x4 bt;
                if (u == 0) {
#pragma unroll
                    for (int s = 0; s < 4; ++s) bt[s] = sm.AT[(16 * j + 4 * lg + s) * kMS + 16 * j + lm];
                } else {
                    bt = *reinterpret_cast<const f32x4*>(&sm.AT[(16 * j + lm) * kMS + 16 * kk + 4 * lg]);
                }
                Pu[u] = zero4();
#pragma unroll
                for (int s = 0; s < 4; ++s) Pu[u] = mfma_f32_16x16x4(a[s], bt[s], Pu[u]);
            }
            f32x4 P = Pu[0];
#pragma unroll
            for (int u = 1; u < d; ++u) P += Pu[u];
            const f32x4 t = *reinterpret_cast<const f32x4*>(&sm.AT[(16 * i + lm) * kMS + 16 * i + 4 * lg]);
            f32x4 R0 = zero4(), R1 = zero4();
#pragma unroll
            for (int s = 0; s < 4; s += 2) {
                R0 = mfma_f32_16x16x4(t[s], P[s], R0);
                R1 = mfma_f32_16x16x4(t[s + 1], P[s + 1], R1);
            }
            const f32x4 R = R0 + R1;
            // R[s] = T_ij[4lg + s][lm] -> transposed slot (j, i)
            *reinterpret_cast<f32x4*>(&sm.AT[(16 * j + lm) * kMS + 16 * i + 4 * lg]) = R;
        }
        __syncthreads();
    }
    if (kDbg) {
        for (int e = tid; e < kChunk * kChunk; e += kPrepThreads) {
            const int r = e >> 6, c = e & 63;
            float t = 0.f;
            if ((r >> 4) == (c >> 4)) t = sm.AT[r * kMS + c];
            else if (r > c) t = sm.AT[c * kMS + r];
            ws.dbgT[ch * kChunk * kChunk + e] = t;
        }
    }

    // ---- (T - I) fragments: wave w writes row tile mt = w, k-blocks
    // kb <= mt / 2; lane (lg, lm) holds T[16mt + lm][32kb + kmap(lg, j)]
    {
        const int mt = wave;
        const int r = mt * 16 + lm;
        half8* tdst = ws.TI + ch * (kTri * 64);
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            if (kb > mt / 2) break;
            const int c0 = kb * 32 + 4 * lg;
            f32x4 t0 = t_row4(sm.AT, mt, 2 * kb, r, c0);
            f32x4 t1 = t_row4(sm.AT, mt, 2 * kb + 1, r, c0 + 16);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                if (c0 + e == r) t0[e] -= 1.f;
                if (c0 + 16 + e == r) t1[e] -= 1.f;
            }
            tdst[(tri_base(mt) + kb) * 64 + lane] = cat8(to_half4(t0), to_half4(t1));
        }
    }
}

// ---------------------------------------------------------------------------
// scan kernel: one work-group (8 waves) per (32 value columns, v-head,
// sequence).  The 32 columns form two 16-column slices, interleaved in
// groups of four: slice h holds columns 32 pr + 8 (n / 4) + 4 h + n % 4 for
// MFMA column n, so the output wave's two D tiles of one token are 8
// consecutive columns (one 16-byte store).
//
// State layout of a chain wave: accumulator tile t (0..7), lane (g, n),
// element i holds S[dk][col(n)] with dk = 32 (t/2) + 8 g + 4 (t%2) + i.  Then
// the fp16 B operand of k-block kb (tiles 2kb, 2kb+1) holds dk 32 kb + 8 g +
// 0..7 in order, matching 16-byte reads of K and Q rows, and the K^T operand
// producing tile t is two transposing LDS reads.
//
//   chains   wave h (h = 0, 1) on SIMD h: P = K S (16 MFMA), R (VALU),
//            V_n = R + (T - I) R (6), S' = e^{c63} S + K^T (d V_n)_hi (16),
//            Sc' = e^{c63} Sc + K^T (d V_n)_lo (16, off the serial path).
//   output   wave 2: O^T = (S^T Q^T) diag(s e^c) + V_n^T M^T for both slices.
//   loaders  wave 3: K rows -> fp16, gates -> ring A; wave 7: Q rows ->
//            fp16, s e^c -> ring B; wave 6: V rows and T - I -> ring A, M ->
//            ring B, as direct-to-LDS loads.  Waves 4 and 5 exit at once, so
//            each chain has its SIMD to itself.
// ---------------------------------------------------------------------------
constexpr int kRingA = 3;     // chain operand stages
constexpr int kRingB = 2;     // output operand stages
constexpr int kHand = 2;      // chain -> output hand-off slots

struct StageA {
    u32x4 K[kChunk * 16];   // fp16 K rows; piece p of row r at 16 r + (p ^ (r & 15))
    u32x4 V[kChunk * 4];    // raw 16-bit V rows of the pair's 32 columns, 4 pieces per row
    half8 TI[kTri][64];     // (T - I) fragments
    float beta[kChunk], bec[kChunk], dec[kChunk];   // beta, beta e^c, e^{c63 - c}
    float gam;                                      // e^{c63}
    float pad_[3];
};

struct StageB {
    u32x4 Q[kChunk * 16];   // fp16 Q rows, same swizzle as K
    half8 M[kTri][64];      // M fragments
    float sec[kChunk];      // s e^c
};

struct Hand {
    half8 S[2][4][64];      // S at the chunk's start, fp16 B fragments per slice
    half8 V[2][2][64];      // V_n, fp16 B fragments per slice
};

struct ScanSmem {
    StageA a[kRingA];
    StageB b[kRingB];
    Hand h[kHand];
    int fillA[2];    // chunks in ring A: 0 K loader, 1 aux loader
    int fillB[2];    // chunks in ring B: 0 Q loader, 1 aux loader
    int freeA[2];    // per chain: chunks whose ring-A stage it has finished reading
    int freeB;       // output: chunks whose ring-B stage it has finished reading
    int ready[2];    // per chain: chunks whose hand-off part is written
    int cons;        // output: chunks whose hand-off slot it has read
    int abort;       // a bounded wait ran out: every wave stops
    int seqsel;
    int red[kScanThreads / 64];
};

__device__ __forceinline__ int lds_ld(const int* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ void lds_st(int* p, int v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// Wait until every LDS operation of this wave has completed (lgkmcnt(0)).
__device__ inline void lds_wait_all() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);
    asm volatile("" ::: "memory");
}

// Wait until every vector memory operation of this wave has completed
// (vmcnt(0)), including direct-to-LDS loads.
__device__ inline void vm_wait_all() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0x0F70);
    asm volatile("" ::: "memory");
}

// Bounded wait on `ready()`.  Gives up when another wave has aborted, or
// after `limit` polls, when it aborts the work-group and sets bit 0 of the
// status word.  Returns whether the condition holds.
struct Waiter {
    int* abort;
    unsigned* status;
    unsigned limit;
    template <typename F>
    __device__ bool until(F ready) const {
        for (unsigned it = 0;; ++it) {
            if (ready()) return true;
            if (lds_ld(abort)) return false;
            if (it >= limit) {
                lds_st(abort, 1);
                if ((threadIdx.x & 63) == 0) atomicOr(status, 1u);
                return false;
            }
            __builtin_amdgcn_s_sleep(1);
        }
    }
};

struct ScanArgs {
    PrepIn in;
    Workspace ws;
    uint16_t* o;
    const float* s0;
    float* sf;
    const int32_t* cu;
    int N, T, total, HV, HK, nch_bound;
    unsigned spin;
};

// Loader of K (kQ = false, ring A, with the chains' gates) or Q (kQ = true,
// ring B, with s e^c) rows: 16 pieces of 16 bytes per lane per chunk, two
// chunks in flight; rows become fp16 (normalised first for raw inputs) and
// are written with the row swizzle.  Rows past the chunk's end are zero.
template <bool kQ, int kRaw>
__device__ void run_row_loader(ScanSmem& sm, const ScanArgs& a, const Waiter& w, int hk, int hv,
                               int tok_base, int len, int nch, float scale, int lane) {
    const uint16_t* __restrict__ src = kQ ? a.in.q : a.in.k;
    struct Buf {
        u32x4 r[16];
        float g, b;
    };
    auto load = [&](int c, Buf& f) {
        const int cc = min(c, nch - 1);
        const int t0 = tok_base + cc * kChunk, rows = min(kChunk, len - cc * kChunk);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int r = min(4 * i + (lane >> 4), rows - 1);
            f.r[i] = *reinterpret_cast<const u32x4*>(src + ((size_t)(t0 + r) * a.HK + hk) * kDK +
                                                      8 * (lane & 15));
        }
        load_gate<kRaw>(a.in, (size_t)(t0 + min(lane, rows - 1)) * a.HV + hv, hv, f.g, f.b);
    };
    auto store = [&](int c, const Buf& f) -> bool {
        const bool ok = kQ ? w.until([&] { return lds_ld(&sm.freeB) >= c - kRingB + 1; })
                           : w.until([&] {
                                 return min(lds_ld(&sm.freeA[0]), lds_ld(&sm.freeA[1])) >=
                                        c - kRingA + 1;
                             });
        if (!ok) return false;
        asm volatile("" ::: "memory");
        const int rows = min(kChunk, len - c * kChunk);
        u32x4* dst = kQ ? sm.b[c % kRingB].Q : sm.a[c % kRingA].K;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int r = 4 * i + (lane >> 4), p = lane & 15;
            half8 h = row_piece_to_half8<kRaw>(f.r[i]);
            u32x4 v = __builtin_bit_cast(u32x4, h);
            if (r >= rows) v = u32x4{0u, 0u, 0u, 0u};
            dst[16 * r + (p ^ (r & 15))] = v;
        }
        // gates: c = cumsum(g) over the chunk (padded rows g = beta = 0)
        const float gv = lane < rows ? f.g : 0.f, bv = lane < rows ? f.b : 0.f;
        float cs = gv;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const float o = __shfl_up(cs, off, 64);
            if (lane >= off) cs += o;
        }
        const float clast = __shfl(cs, 63, 64);
        const float ec = exp2f(cs * kLog2e);
        if constexpr (kQ) {
            sm.b[c % kRingB].sec[lane] = scale * ec;
        } else {
            StageA& st = sm.a[c % kRingA];
            st.beta[lane] = bv;
            st.bec[lane] = bv * ec;
            st.dec[lane] = exp2f((clast - cs) * kLog2e);
            if (lane == 0) st.gam = exp2f(clast * kLog2e);
        }
        lds_wait_all();
        if (lane == 0) lds_st(kQ ? &sm.fillB[0] : &sm.fillA[0], c + 1);
        return true;
    };
    if (nch <= 0) return;
    Buf fa, fb;
    load(0, fa);
    for (int c = 0; c < nch; c += 2) {
        load(c + 1, fb);
        if (!store(c, fa)) return;
        if (c + 1 >= nch) return;
        load(c + 2, fa);
        if (!store(c + 1, fb)) return;
    }
}

// Direct-to-LDS loader of V (the pair's 32 columns), T - I (ring A) and M
// (ring B).  A chunk's 16 loads go out as soon as its stages are free; its
// counters are set once the loads of the next chunk are issued and its own
// have landed.
__device__ void run_aux_loader(ScanSmem& sm, const ScanArgs& a, const Waiter& w, int hv, int pr,
                               int tok_base, int len, int chunk0, int nch, int lane) {
    auto issue = [&](int c) -> bool {
        const bool ok = w.until([&] {
            return min(lds_ld(&sm.freeA[0]), lds_ld(&sm.freeA[1])) >= c - kRingA + 1 &&
                   lds_ld(&sm.freeB) >= c - kRingB + 1;
        });
        if (!ok) return false;
        asm volatile("" ::: "memory");
        StageA& sa = sm.a[c % kRingA];
        StageB& sb = sm.b[c % kRingB];
        const int t0 = tok_base + c * kChunk, rows = min(kChunk, len - c * kChunk);
        // V: slot 64 i + lane = row (16 i + lane / 4), piece lane % 4
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int r = min(16 * i + (lane >> 2), rows - 1);
            const uint16_t* gp =
                a.in.v + ((size_t)(t0 + r) * a.HV + hv) * kDV + kPairCols * pr + 8 * (lane & 3);
            __builtin_amdgcn_global_load_lds(gp, (__attribute__((address_space(3))) void*)&sa.V[64 * i],
                                             16, 0, 0);
        }
        const size_t ch = (size_t)(chunk0 + c) * a.HV + hv;
        const half8* ti = a.ws.TI + ch * (kTri * 64) + lane;
        const half8* mm = a.ws.M + ch * (kTri * 64) + lane;
#pragma unroll
        for (int f = 0; f < kTri; ++f)
            __builtin_amdgcn_global_load_lds(ti + f * 64, (__attribute__((address_space(3))) void*)&sa.TI[f][0],
                                             16, 0, 0);
#pragma unroll
        for (int f = 0; f < kTri; ++f)
            __builtin_amdgcn_global_load_lds(mm + f * 64, (__attribute__((address_space(3))) void*)&sb.M[f][0],
                                             16, 0, 0);
        return true;
    };
    auto publish = [&](int c) {
        if (lane == 0) {
            lds_st(&sm.fillA[1], c + 1);
            lds_st(&sm.fillB[1], c + 1);
        }
    };
    for (int c = 0; c < nch; ++c) {
        if (!issue(c)) {
            vm_wait_all();   // no load may land in LDS after the group ends
            return;
        }
        if (c > 0) {
            // the previous chunk's 16 loads have landed (this chunk's 16 may
            // still be in flight): vmcnt(16)
            asm volatile("" ::: "memory");
            __builtin_amdgcn_s_waitcnt(0x4F70);
            asm volatile("" ::: "memory");
            publish(c - 1);
        }
    }
    if (nch > 0) {
        vm_wait_all();
        publish(nch - 1);
    }
}

template <int kRaw>
__device__ inline float v16_to_f32(uint32_t bits) {
    // fp16 V is rounded to bf16 first (the adapter's conversion)
    if constexpr (kRaw == 2) return (float)(__bf16)raw16<2>(bits);
    return __uint_as_float(bits << 16);
}

template <int kRaw, bool kDbg>
__device__ void run_chain(ScanSmem& sm, const ScanArgs& a, const Waiter& w, int h, int seq, int hv,
                          int pr, int chunk0, int nch, int lane) {
    const int lg = lane >> 4, lm = lane & 15;
    // column of MFMA column lm in this slice, and dk of (tile t, element i)
    const int col = kPairCols * pr + 8 * (lm >> 2) + 4 * h + (lm & 3);
    auto dk_of = [&](int t, int i) { return 32 * (t >> 1) + 8 * lg + 4 * (t & 1) + i; };
    const size_t sbase = ((size_t)seq * a.HV + hv) * kDK * kDV + col;

    f32x4 S[8], Sc[8];
    if (a.s0) {
#pragma unroll
        for (int t = 0; t < 8; ++t) {
#pragma unroll
            for (int i = 0; i < 4; ++i) S[t][i] = a.s0[sbase + (size_t)dk_of(t, i) * kDV];
        }
    } else {
#pragma unroll
        for (int t = 0; t < 8; ++t) S[t] = zero4();
    }
#pragma unroll
    for (int t = 0; t < 8; ++t) Sc[t] = zero4();
    half8 S16[4];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) S16[kb] = cat8(to_half4(S[2 * kb]), to_half4(S[2 * kb + 1]));

    bool ok = true;
    for (int c = 0; c < nch; ++c) {
        const int st = c % kRingA, hs = c % kHand;
        ok = w.until([&] {
            return min(lds_ld(&sm.fillA[0]), lds_ld(&sm.fillA[1])) >= c + 1 &&
                   lds_ld(&sm.cons) >= c - kHand + 1;
        });
        if (!ok) break;
        asm volatile("" ::: "memory");
        const StageA& sa = sm.a[st];
        // S at the chunk's start goes to the hand-off slot
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) sm.h[hs].S[h][kb][lane] = S16[kb];
        if (kDbg) {
            float* dst = a.ws.dbgS + ((size_t)(chunk0 + c) * a.HV + hv) * kDK * kDV + col;
#pragma unroll
            for (int t = 0; t < 8; ++t) {
#pragma unroll
                for (int i = 0; i < 4; ++i) dst[(size_t)dk_of(t, i) * kDV] = S[t][i] + Sc[t][i];
            }
        }
        // P = K S: row tile mt (tokens), k-block kb (dk)
        f32x4 P[4];
        {
            half8 kf[4][4];
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) {
                const int r = 16 * mt + lm;
#pragma unroll
                for (int kb = 0; kb < 4; ++kb)
                    kf[mt][kb] = __builtin_bit_cast(half8, sa.K[16 * r + ((4 * kb + lg) ^ (r & 15))]);
            }
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) P[mt] = zero4();
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
                for (int mt = 0; mt < 4; ++mt) P[mt] = mfma16(kf[mt][kb], S16[kb], P[mt]);
            }
        }
        // R = beta o V - (beta e^c) o P: lane (lg, lm) of tile mt holds tokens
        // 16 mt + 4 lg + i of column lm
        f32x4 R[4], dec[4];
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
            const f32x4 be = *reinterpret_cast<const f32x4*>(&sa.beta[16 * mt + 4 * lg]);
            const f32x4 bc = *reinterpret_cast<const f32x4*>(&sa.bec[16 * mt + 4 * lg]);
            dec[mt] = *reinterpret_cast<const f32x4*>(&sa.dec[16 * mt + 4 * lg]);
            // transposing read: source lane (a4 = lm / 4, b4 = lm % 4) names
            // row 16 mt + 4 lg + a4, columns 8 b4 + 4 h .. + 3
            const uint16_t* vsrc = reinterpret_cast<const uint16_t*>(sa.V) +
                                   (16 * mt + 4 * lg + (lm >> 2)) * kPairCols + 8 * (lm & 3) + 4 * h;
            const s16x4 vt = lds_read_tr(vsrc);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float vv = v16_to_f32<kRaw>((uint16_t)vt[i]);
                R[mt][i] = be[i] * vv - bc[i] * P[mt][i];
            }
        }
        const float gam = sa.gam;
        half8 Rh[2];
        Rh[0] = cat8(to_half4(R[0]), to_half4(R[1]));
        Rh[1] = cat8(to_half4(R[2]), to_half4(R[3]));
        // V_n = R + (T - I) R
        f32x4 Vn[4];
        {
            half8 ti[kTri];
#pragma unroll
            for (int f = 0; f < kTri; ++f) ti[f] = sa.TI[f][lane];
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) {
                Vn[mt] = mfma16(ti[tri_base(mt)], Rh[0], R[mt]);
                if (mt >= 2) Vn[mt] = mfma16(ti[tri_base(mt) + 1], Rh[1], Vn[mt]);
            }
        }
        half8 Vh[2];
        Vh[0] = cat8(to_half4(Vn[0]), to_half4(Vn[1]));
        Vh[1] = cat8(to_half4(Vn[2]), to_half4(Vn[3]));
        sm.h[hs].V[h][0][lane] = Vh[0];
        sm.h[hs].V[h][1][lane] = Vh[1];
        lds_wait_all();
        if (lane == 0) lds_st(&sm.ready[h], c + 1);
        // d o V_n as an fp16 hi / lo pair
        half8 hi[2], lo[2];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            f32x4 d0 = dec[2 * kb] * Vn[2 * kb], d1 = dec[2 * kb + 1] * Vn[2 * kb + 1];
            const half4 h0 = to_half4(d0), h1 = to_half4(d1);
            hi[kb] = cat8(h0, h1);
            f32x4 r0, r1;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                r0[i] = d0[i] - (float)h0[i];
                r1[i] = d1[i] - (float)h1[i];
            }
            lo[kb] = cat8(to_half4(r0), to_half4(r1));
        }
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            S[t] = S[t] * gam;
            Sc[t] = Sc[t] * gam;
        }
        // S' = e^{c63} S + K^T (d V_n): K^T fragment (tile t, k-block kb) from
        // two transposing reads; source lane (a4 = lm / 4, b4 = lm % 4) names
        // row tok0 + 4 lg + a4, dk 32 (t/2) + 8 b4 + 4 (t%2) .. + 3
        const uint16_t* kbase = reinterpret_cast<const uint16_t*>(sa.K);
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const int p = 4 * (t >> 1) + (lm & 3);
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                const int r0 = 32 * kb + 4 * lg + (lm >> 2), r1 = r0 + 16;
                const s16x4 x0 = lds_read_tr(kbase + (16 * r0 + (p ^ (r0 & 15))) * 8 + 4 * (t & 1));
                const s16x4 x1 = lds_read_tr(kbase + (16 * r1 + (p ^ (r1 & 15))) * 8 + 4 * (t & 1));
                const half8 kt = cat8(s16x4_as_half4(x0), s16x4_as_half4(x1));
                S[t] = mfma16(kt, hi[kb], S[t]);
                Sc[t] = mfma16(kt, lo[kb], Sc[t]);
            }
        }
        lds_wait_all();
        if (lane == 0) lds_st(&sm.freeA[h], c + 1);
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) S16[kb] = cat8(to_half4(S[2 * kb]), to_half4(S[2 * kb + 1]));
    }
    if (!ok) return;
#pragma unroll
    for (int t = 0; t < 8; ++t) {
#pragma unroll
        for (int i = 0; i < 4; ++i) a.sf[sbase + (size_t)dk_of(t, i) * kDV] = S[t][i] + Sc[t][i];
    }
}

template <int kRaw>
__device__ void run_output(ScanSmem& sm, const ScanArgs& a, const Waiter& w, int hv, int pr,
                           int tok_base, int len, int nch, int lane) {
    const int lg = lane >> 4, lm = lane & 15;
    for (int c = 0; c < nch; ++c) {
        const int sb = c % kRingB, hs = c % kHand;
        const bool ok = w.until([&] {
            return min(lds_ld(&sm.fillB[0]), lds_ld(&sm.fillB[1])) >= c + 1 &&
                   min(lds_ld(&sm.ready[0]), lds_ld(&sm.ready[1])) >= c + 1;
        });
        if (!ok) return;
        asm volatile("" ::: "memory");
        half8 hsf[2][4], hvf[2][2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) hsf[h][kb] = sm.h[hs].S[h][kb][lane];
            hvf[h][0] = sm.h[hs].V[h][0][lane];
            hvf[h][1] = sm.h[hs].V[h][1][lane];
        }
        lds_wait_all();
        if (lane == 0) lds_st(&sm.cons, c + 1);
        const StageB& stb = sm.b[sb];
        half8 qf[4][4], mf[kTri];
        float es[4];
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
            const int r = 16 * mt + lm;
#pragma unroll
            for (int kb = 0; kb < 4; ++kb)
                qf[mt][kb] = __builtin_bit_cast(half8, stb.Q[16 * r + ((4 * kb + lg) ^ (r & 15))]);
            es[mt] = stb.sec[r];
        }
#pragma unroll
        for (int f = 0; f < kTri; ++f) mf[f] = stb.M[f][lane];
        // O^T = (S^T Q^T) diag(s e^c) + V_n^T M^T per slice: lane (lg, lm)
        // of tile mt holds columns 4 lg .. 4 lg + 3 of the slice for token
        // 16 mt + lm
        f32x4 ov[2][4];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) ov[h][mt] = zero4();
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
                for (int mt = 0; mt < 4; ++mt) ov[h][mt] = mfma16(hsf[h][kb], qf[mt][kb], ov[h][mt]);
            }
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) {
                ov[h][mt] = ov[h][mt] * es[mt];
                ov[h][mt] = mfma16(hvf[h][0], mf[tri_base(mt)], ov[h][mt]);
                if (mt >= 2) ov[h][mt] = mfma16(hvf[h][1], mf[tri_base(mt) + 1], ov[h][mt]);
            }
        }
        lds_wait_all();
        if (lane == 0) lds_st(&sm.freeB, c + 1);
        const int rows = min(kChunk, len - c * kChunk);
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
            const int r = 16 * mt + lm;
            u32x4 pk;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
#pragma unroll
                for (int e = 0; e < 2; ++e) {
                    const float x0 = ov[h][mt][2 * e], x1 = ov[h][mt][2 * e + 1];
                    uint32_t b0 = f32_to_bf16_bits(x0), b1 = f32_to_bf16_bits(x1);
                    if constexpr (kRaw == 2) {
                        b0 = f16_bits(__uint_as_float(b0 << 16));
                        b1 = f16_bits(__uint_as_float(b1 << 16));
                    }
                    pk[2 * h + e] = b0 | (b1 << 16);
                }
            }
            if (r < rows) {
                u32x4* dst = reinterpret_cast<u32x4*>(
                    a.o + ((size_t)(tok_base + c * kChunk + r) * a.HV + hv) * kDV + kPairCols * pr + 8 * lg);
                *dst = pk;
            }
        }
    }
}

// s0 and sf may be the same buffer: a chain reads its elements of the initial
// state before its first chunk and writes the same elements after its last,
// and no other wave touches either.
template <int kRaw, bool kDbg>
__global__ __launch_bounds__(kScanThreads, 1) void gdn_scan_kernel(ScanArgs a) {
    __shared__ ScanSmem sm;
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;

    // XCD-aware id: the four groups of one (sequence, head) share id % 8
    // (one XCD, one L2), so their K, Q, T - I and M come from one L2
    const int id = blockIdx.x;
    const int xcd = id & 7, qd = id >> 3;
    const int pr = qd % kPairsPerHead;
    const int pidx = (qd / kPairsPerHead) * 8 + xcd;
    if (pidx >= a.N * a.HV) return;
    int seq = pidx / a.HV;
    const int hv = pidx - seq * a.HV;
    // Packed sequences of different lengths: groups start in id order as CUs
    // free up, so the low ids go to the longest sequences (longest first).
    if (a.cu && a.N <= kScanThreads) {
        if (tid < a.N) {
            const int my = seq_count(a.cu, a.T, a.total, tid);
            int rank = 0;
            for (int u = 0; u < a.N; ++u) {
                const int lu = seq_count(a.cu, a.T, a.total, u);
                rank += (lu > my || (lu == my && u < tid)) ? 1 : 0;
            }
            if (rank == seq) sm.seqsel = tid;
        }
        __syncthreads();
        seq = sm.seqsel;
    }
    const int hk = hv / (a.HV / a.HK);
    const int len = seq_count(a.cu, a.T, a.total, seq);
    const int tok_base = seq_lo(a.cu, a.T, a.total, seq);
    const int chunk0 = __builtin_amdgcn_readfirstlane(
        chunks_before<kScanThreads>(a.cu, a.T, a.total, seq, sm.red));
    const int nch = seq_chunks_bounded(a.cu, a.T, a.total, seq, chunk0, a.nch_bound);
    if (tid < 2) {
        lds_st(&sm.fillA[tid], 0);
        lds_st(&sm.fillB[tid], 0);
        lds_st(&sm.freeA[tid], 0);
        lds_st(&sm.ready[tid], 0);
    }
    if (tid == 0) {
        lds_st(&sm.freeB, 0);
        lds_st(&sm.cons, 0);
        lds_st(&sm.abort, 0);
    }
    __syncthreads();
    const Waiter w{&sm.abort, a.ws.status, a.spin};
    const float scale = 1.0f / sqrtf((float)kDK);
    switch (wave) {
        case 0: run_chain<kRaw, kDbg>(sm, a, w, 0, seq, hv, pr, chunk0, nch, lane); break;
        case 1: run_chain<kRaw, kDbg>(sm, a, w, 1, seq, hv, pr, chunk0, nch, lane); break;
        case 2: run_output<kRaw>(sm, a, w, hv, pr, tok_base, len, nch, lane); break;
        case 3: run_row_loader<false, kRaw>(sm, a, w, hk, hv, tok_base, len, nch, scale, lane); break;
        case 6: run_aux_loader(sm, a, w, hv, pr, tok_base, len, chunk0, nch, lane); break;
        case 7: run_row_loader<true, kRaw>(sm, a, w, hk, hv, tok_base, len, nch, scale, lane); break;
        default: break;   // waves 4, 5: each chain keeps its SIMD to itself
    }
}

// raw: 0 for prepared inputs, 1 / 2 for raw bf16 / fp16 q, k (normalised in
// the kernels; then v and o have that dtype too).
hipError_t launch_prefill(const PrepIn& in, int raw, void* o, const float* s0, float* sf,
                          const int32_t* cu, int N, int T, int total_tokens, int HV, int HK,
                          size_t nch_bound, void* workspace, size_t workspace_bytes,
                          hipStream_t stream, int dump_debug, hipEvent_t* ev = nullptr,
                          int only = -1, unsigned spin = kDefaultSpin) {
    const WsLayout L(nch_bound * (size_t)HV);
    const size_t need = dump_debug ? L.total : L.live;
    if (workspace_bytes < need) return hipErrorInvalidValue;
    char* base = static_cast<char*>(workspace);
    Workspace ws{};
    ws.TI = reinterpret_cast<half8*>(base + L.ti);
    ws.M = reinterpret_cast<half8*>(base + L.m);
    ws.status = reinterpret_cast<unsigned*>(base);
    if (dump_debug) {
        ws.dbgT = reinterpret_cast<float*>(base + L.dbgT);
        ws.dbgA = reinterpret_cast<float*>(base + L.dbgA);
        ws.dbgTp = reinterpret_cast<float*>(base + L.dbgTp);
        ws.dbgM = reinterpret_cast<float*>(base + L.dbgM);
        ws.dbgC = reinterpret_cast<float*>(base + L.dbgC);
        ws.dbgS = reinterpret_cast<float*>(base + L.dbgS);
    }
    const float scale = 1.0f / sqrtf((float)kDK);

    if (ev) (void)hipEventRecord(ev[0], stream);
    // the prep always runs (at least one group): it clears the status word
    if (only != 1) {
        const int rep = HV / HK;
        const size_t groups = (nch_bound * (size_t)HK + 7) / 8;
        const size_t grid = std::max<size_t>(groups * 8 * rep, 1);
        auto kern = raw == 1 ? gdn_prep_kernel<false, 1>
                    : raw == 2 ? gdn_prep_kernel<false, 2>
                    : dump_debug ? gdn_prep_kernel<true, 0> : gdn_prep_kernel<false, 0>;
        hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(kPrepThreads), 0, stream, in, cu, N, T,
                           total_tokens, HV, HK, (int)nch_bound, scale, ws);
        hipError_t err = hipGetLastError();
        if (err != hipSuccess) return err;
    }
    if (ev) (void)hipEventRecord(ev[1], stream);
    if (only == 0) return hipSuccess;
    ScanArgs sa{};
    sa.in = in;
    sa.ws = ws;
    sa.o = static_cast<uint16_t*>(o);
    sa.s0 = s0;
    sa.sf = sf;
    sa.cu = cu;
    sa.N = N;
    sa.T = T;
    sa.total = total_tokens;
    sa.HV = HV;
    sa.HK = HK;
    sa.nch_bound = (int)nch_bound;
    sa.spin = spin;
    const int pairs = N * HV;
    const int grp = (pairs + 7) / 8;
    auto scan = raw == 1 ? gdn_scan_kernel<1, false>
                : raw == 2 ? gdn_scan_kernel<2, false>
                : dump_debug ? gdn_scan_kernel<0, true> : gdn_scan_kernel<0, false>;
    hipLaunchKernelGGL(scan, dim3((unsigned)(grp * 8 * kPairsPerHead)), dim3(kScanThreads), 0,
                       stream, sa);
    hipError_t err = hipGetLastError();
    if (ev) (void)hipEventRecord(ev[2], stream);
    return err;
}

constexpr int kPrefillKernels = 2;
const char* const kPrefillKernelNames[kPrefillKernels] = {"gdn_prep_kernel", "gdn_scan_kernel"};

PrepIn plain_in(const void* q, const void* k, const void* v, const float* g, const float* beta) {
    PrepIn in{};
    in.q = static_cast<const uint16_t*>(q);
    in.k = static_cast<const uint16_t*>(k);
    in.v = static_cast<const uint16_t*>(v);
    in.g = g;
    in.beta = beta;
    return in;
}

bool dims_ok(int HV, int HQK, int DK, int DV, int chunk_size) {
    return DK == kDK && DV == kDV && chunk_size == kChunk && HQK > 0 && HV > 0 && HV % HQK == 0;
}

size_t ws_size(size_t nch, int HV) { return std::max<size_t>(WsLayout(nch * HV).total, 256); }

}  // namespace
}  // namespace gdn

using namespace gdn;

extern "C" size_t deltanet_prefill_workspace_size(int B, int T, int HV, int DK, int DV,
                                                  int chunk_size) {
    if (B <= 0 || T < 0 || HV <= 0 || DK != kDK || DV != kDV || chunk_size != kChunk) return 0;
    const size_t nc = (size_t)B * ((T + kChunk - 1) / kChunk);
    return ws_size(nc, HV);
}

extern "C" size_t deltanet_prefill_live_workspace_size(int B, int T, int HV, int DK, int DV,
                                                       int chunk_size) {
    if (B <= 0 || T < 0 || HV <= 0 || DK != kDK || DV != kDV || chunk_size != kChunk) return 0;
    const size_t nc = (size_t)B * ((T + kChunk - 1) / kChunk);
    return WsLayout(nc * HV).live;
}

extern "C" hipError_t deltanet_chunk_prefill(const void* q, const void* k, const void* v,
                                             const float* g, const float* beta, void* o,
                                             const float* initial_state, float* final_state,
                                             int B, int T, int HV, int HQK, int DK, int DV,
                                             int chunk_size, void* workspace,
                                             size_t workspace_bytes, hipStream_t stream,
                                             int dump_debug) {
    if (!dims_ok(HV, HQK, DK, DV, chunk_size) || B <= 0 || T < 0) return hipErrorInvalidValue;
    if (workspace == nullptr || final_state == nullptr) return hipErrorInvalidValue;
    if (T > 0 && (!q || !k || !v || !g || !beta || !o)) return hipErrorInvalidValue;
    const size_t nc = (size_t)B * ((T + kChunk - 1) / kChunk);
    return launch_prefill(plain_in(q, k, v, g, beta), 0, o, initial_state, final_state, nullptr, B,
                          T, B * T, HV, HQK, nc, workspace, workspace_bytes, stream, dump_debug);
}

extern "C" hipError_t deltanet_prefill_status(const void* workspace, size_t workspace_bytes,
                                              hipStream_t stream) {
    if (workspace == nullptr || workspace_bytes < kHeaderBytes) return hipErrorInvalidValue;
    unsigned st = 0;
    hipError_t err = hipMemcpyAsync(&st, workspace, sizeof(st), hipMemcpyDeviceToHost, stream);
    if (err == hipSuccess) err = hipStreamSynchronize(stream);
    if (err != hipSuccess) return err;
    return (st & 1u) ? hipErrorLaunchTimeOut : hipSuccess;
}

extern "C" hipError_t deltanet_chunk_prefill_spin(const void* q, const void* k, const void* v,
                                                  const float* g, const float* beta, void* o,
                                                  const float* initial_state, float* final_state,
                                                  int B, int T, int HV, int HQK, void* workspace,
                                                  size_t workspace_bytes, hipStream_t stream,
                                                  unsigned spin_limit) {
    if (!dims_ok(HV, HQK, kDK, kDV, kChunk) || B <= 0 || T < 0) return hipErrorInvalidValue;
    if (workspace == nullptr || final_state == nullptr) return hipErrorInvalidValue;
    if (T > 0 && (!q || !k || !v || !g || !beta || !o)) return hipErrorInvalidValue;
    const size_t nc = (size_t)B * ((T + kChunk - 1) / kChunk);
    return launch_prefill(plain_in(q, k, v, g, beta), 0, o, initial_state, final_state, nullptr, B,
                          T, B * T, HV, HQK, nc, workspace, workspace_bytes, stream, 0, nullptr,
                          -1, spin_limit);
}

extern "C" int deltanet_prefill_kernel_count(void) { return kPrefillKernels; }

extern "C" const char* deltanet_prefill_kernel_name(int i) {
    return (i >= 0 && i < kPrefillKernels) ? kPrefillKernelNames[i] : nullptr;
}

extern "C" hipError_t deltanet_chunk_prefill_timed(const void* q, const void* k, const void* v,
                                                   const float* g, const float* beta, void* o,
                                                   const float* initial_state,
                                                   float* final_state, int B, int T, int HV,
                                                   int HQK, int DK, int DV, int chunk_size,
                                                   void* workspace, size_t workspace_bytes,
                                                   hipStream_t stream, hipEvent_t* events,
                                                   int n_events) {
    if (!events || n_events != kPrefillKernels + 1) return hipErrorInvalidValue;
    for (int i = 0; i < n_events; ++i)
        if (!events[i]) return hipErrorInvalidValue;
    if (!dims_ok(HV, HQK, DK, DV, chunk_size) || B <= 0 || T < 0) return hipErrorInvalidValue;
    if (workspace == nullptr || final_state == nullptr) return hipErrorInvalidValue;
    if (T > 0 && (!q || !k || !v || !g || !beta || !o)) return hipErrorInvalidValue;
    const size_t nc = (size_t)B * ((T + kChunk - 1) / kChunk);
    return launch_prefill(plain_in(q, k, v, g, beta), 0, o, initial_state, final_state, nullptr, B,
                          T, B * T, HV, HQK, nc, workspace, workspace_bytes, stream, 0, events);
}

extern "C" hipError_t deltanet_chunk_prefill_kernel(const void* q, const void* k, const void* v,
                                                    const float* g, const float* beta, void* o,
                                                    const float* initial_state,
                                                    float* final_state, int B, int T, int HV,
                                                    int HQK, int DK, int DV, int chunk_size,
                                                    void* workspace, size_t workspace_bytes,
                                                    hipStream_t stream, int kernel) {
    if (kernel < 0 || kernel >= kPrefillKernels) return hipErrorInvalidValue;
    if (!dims_ok(HV, HQK, DK, DV, chunk_size) || B <= 0 || T < 0) return hipErrorInvalidValue;
    if (workspace == nullptr || final_state == nullptr) return hipErrorInvalidValue;
    if (T > 0 && (!q || !k || !v || !g || !beta || !o)) return hipErrorInvalidValue;
    const size_t nc = (size_t)B * ((T + kChunk - 1) / kChunk);
    return launch_prefill(plain_in(q, k, v, g, beta), 0, o, initial_state, final_state, nullptr, B,
                          T, B * T, HV, HQK, nc, workspace, workspace_bytes, stream, 0, nullptr,
                          kernel);
}

extern "C" size_t deltanet_prefill_varlen_workspace_size(int total_tokens, int num_seqs, int HV,
                                                         int DK, int DV, int chunk_size) {
    if (total_tokens < 0 || num_seqs <= 0 || HV <= 0 || DK != kDK || DV != kDV ||
        chunk_size != kChunk)
        return 0;
    // sum_i ceil(L_i / C) <= (sum_i L_i + (C-1) N) / C
    const size_t nc = ((size_t)total_tokens + (size_t)(kChunk - 1) * num_seqs) / kChunk;
    return ws_size(nc, HV);
}

extern "C" size_t deltanet_prefill_varlen_live_workspace_size(int total_tokens, int num_seqs,
                                                              int HV, int DK, int DV,
                                                              int chunk_size) {
    if (total_tokens < 0 || num_seqs <= 0 || HV <= 0 || DK != kDK || DV != kDV ||
        chunk_size != kChunk)
        return 0;
    const size_t nc = ((size_t)total_tokens + (size_t)(kChunk - 1) * num_seqs) / kChunk;
    return WsLayout(nc * HV).live;
}

extern "C" hipError_t deltanet_chunk_prefill_varlen(
    const void* q, const void* k, const void* v, const float* g, const float* beta, void* o,
    const float* initial_state, float* final_state, const int32_t* cu_seqlens, int num_seqs,
    int total_tokens, int HV, int HQK, int DK, int DV, int chunk_size, void* workspace,
    size_t workspace_bytes, hipStream_t stream, int dump_debug) {
    if (!dims_ok(HV, HQK, DK, DV, chunk_size) || num_seqs <= 0 || total_tokens < 0)
        return hipErrorInvalidValue;
    if (!cu_seqlens || !workspace || !final_state) return hipErrorInvalidValue;
    if (total_tokens > 0 && (!q || !k || !v || !g || !beta || !o)) return hipErrorInvalidValue;
    const size_t nc = ((size_t)total_tokens + (size_t)(kChunk - 1) * num_seqs) / kChunk;
    return launch_prefill(plain_in(q, k, v, g, beta), 0, o, initial_state, final_state, cu_seqlens,
                          num_seqs, 0, total_tokens, HV, HQK, nc, workspace, workspace_bytes,
                          stream, dump_debug);
}

extern "C" int deltanet_varlen_chunk_map(const int32_t* cu_seqlens, int num_seqs,
                                         int total_tokens, int32_t* seq_first_chunk,
                                         int32_t* seq_chunk_count, int32_t* seq_first_token,
                                         int32_t* seq_token_count) {
    if (!cu_seqlens || num_seqs <= 0 || total_tokens < 0) return -1;
    const int bound = (int)(((size_t)total_tokens + (size_t)(kChunk - 1) * num_seqs) / kChunk);
    int acc = 0;   // the scan's chunks_before, saturating like it
    for (int s = 0; s < num_seqs; ++s) {
        const int n = seq_chunks_bounded(cu_seqlens, 0, total_tokens, s, acc, bound);
        seq_first_chunk[s] = acc;
        seq_chunk_count[s] = n;
        seq_first_token[s] = seq_lo(cu_seqlens, 0, total_tokens, s);
        seq_token_count[s] = seq_count(cu_seqlens, 0, total_tokens, s);
        acc = sat_add(acc, seq_chunks(cu_seqlens, 0, total_tokens, s));
    }
    return bound;
}

// Twins of the reference's bf16-wmma o-pass variant (kernels/chunk_delta_cuda_tco.h);
// one implementation serves both names.
extern "C" size_t deltanet_tcop_prefill_workspace_size(int B, int T, int HV, int DK, int DV,
                                                       int chunk_size) {
    return deltanet_prefill_workspace_size(B, T, HV, DK, DV, chunk_size);
}

extern "C" hipError_t deltanet_tcop_chunk_prefill(const void* q, const void* k, const void* v,
                                                  const float* g, const float* beta, void* o,
                                                  const float* initial_state, float* final_state,
                                                  int B, int T, int HV, int HQK, int DK, int DV,
                                                  int chunk_size, void* workspace,
                                                  size_t workspace_bytes, hipStream_t stream,
                                                  int dump_debug) {
    return deltanet_chunk_prefill(q, k, v, g, beta, o, initial_state, final_state, B, T, HV, HQK,
                                  DK, DV, chunk_size, workspace, workspace_bytes, stream,
                                  dump_debug);
}

extern "C" hipError_t deltanet_chunk_prefill_fused(const void* q, const void* k, const void* v,
                                                   const void* a, const void* b,
                                                   const float* A_log, const void* dt_bias,
                                                   void* o, float* state, int B, int T, int HV,
                                                   int HQK, int io_dtype, void* workspace,
                                                   size_t workspace_bytes, hipStream_t stream) {
    if (!dims_ok(HV, HQK, kDK, kDV, kChunk) || B <= 0 || T < 0) return hipErrorInvalidValue;
    if (io_dtype != GDN_DTYPE_BF16 && io_dtype != GDN_DTYPE_FP16) return hipErrorInvalidValue;
    if (workspace == nullptr || state == nullptr) return hipErrorInvalidValue;
    if (T > 0 && (!q || !k || !v || !a || !b || !A_log || !dt_bias || !o))
        return hipErrorInvalidValue;
    PrepIn in{};
    in.q = static_cast<const uint16_t*>(q);
    in.k = static_cast<const uint16_t*>(k);
    in.v = static_cast<const uint16_t*>(v);
    in.a = static_cast<const uint16_t*>(a);
    in.b = static_cast<const uint16_t*>(b);
    in.A_log = A_log;
    in.dt_bias = static_cast<const uint16_t*>(dt_bias);
    const size_t nc = (size_t)B * ((T + kChunk - 1) / kChunk);
    return launch_prefill(in, io_dtype == GDN_DTYPE_FP16 ? 2 : 1, o, state, state, nullptr, B, T,
                          B * T, HV, HQK, nc, workspace, workspace_bytes, stream, 0);
}

// As deltanet_chunk_prefill / _varlen, with q and k rows L2-normalised in the
// kernels (transformers' use_qk_l2norm_in_kernel=True).  cu_seqlens NULL:
// B sequences of T tokens; else packed, num_seqs sequences of T tokens in
// total (B must be 1).
extern "C" hipError_t deltanet_chunk_prefill_l2norm(
    const void* q, const void* k, const void* v, const float* g, const float* beta, void* o,
    const float* initial_state, float* final_state, const int32_t* cu_seqlens, int num_seqs,
    int B, int T, int HV, int HQK, void* workspace, size_t workspace_bytes,
    hipStream_t stream) {
    if (!dims_ok(HV, HQK, kDK, kDV, kChunk) || B <= 0 || T < 0) return hipErrorInvalidValue;
    if (cu_seqlens && (B != 1 || num_seqs <= 0)) return hipErrorInvalidValue;
    if (workspace == nullptr || final_state == nullptr) return hipErrorInvalidValue;
    if (T > 0 && (!q || !k || !v || !g || !beta || !o)) return hipErrorInvalidValue;
    PrepIn in = plain_in(q, k, v, g, beta);
    if (cu_seqlens) {
        const size_t nc = ((size_t)T + (size_t)(kChunk - 1) * num_seqs) / kChunk;
        return launch_prefill(in, 1, o, initial_state, final_state, cu_seqlens, num_seqs, 0, T, HV,
                              HQK, nc, workspace, workspace_bytes, stream, 0);
    }
    const size_t nc = (size_t)B * ((T + kChunk - 1) / kChunk);
    return launch_prefill(in, 1, o, initial_state, final_state, nullptr, B, T, B * T, HV, HQK, nc,
                          workspace, workspace_bytes, stream, 0);
}
