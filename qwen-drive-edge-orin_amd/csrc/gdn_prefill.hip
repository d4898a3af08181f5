// Chunked gated-delta-rule prefill for gfx950 (MI355X).
//
// Replaces the reference's four-kernel CUDA pipeline behind
// kernels/chunk_delta_cuda.h:39-55 (deltanet_prefill_workspace_size /
// deltanet_chunk_prefill).  Math per (sequence, v-head), chunk C = 64:
//
//   c   = cumsum(g)            Gamma_rj = exp(c_r - c_j)  (r >= j)
//   A   = -diag(beta) (K K^T o Gamma)  strictly lower,   T = (I - A)^-1
//   U   = T diag(beta) V       W = T diag(beta e^c) K
//   M   = s (Q K^T o Gamma)    lower incl. diagonal,       s = 1/sqrt(DK)
//   V_n = U - W S              O = diag(s e^c) Q S + M V_n
//   S  <- e^{c_63} S + (diag(e^{c_63 - c}) K)^T V_n
//
// (transformers modeling_qwen3_5.py:249-327, the reference's parity oracle;
// kernels/chunk_delta_cuda.cu:91-303 and :312-424 compute the same terms.)
//
// Two kernels:
//   prep  one work-group per (chunk, v-head), up to four per CU: all
//         chunk-local work.  K K^T and K Q^T run on bf16 MFMA straight from the bf16
//         inputs; the inverse T is formed in fp32 in one LDS array (16x16
//         diagonal blocks by forward substitution, off-diagonal blocks on
//         fp32 MFMA, stored transposed in the free upper triangle).  Writes
//         W, decayed K^T and M as fp16 MFMA A-operand fragments and U as
//         fp16 accumulator fragments, so the scan moves each operand with
//         one 16-byte transfer per lane and never reshuffles.
//   scan  one work-group per (one or two state slices, v-head, sequence):
//         the state of a head is split into 8 slices of 16 value columns,
//         which evolve independently.  A chain wave per slice keeps its
//         128x16 fp32 slice in registers; three loader waves stream W, K~^T
//         and U into a 3-stage LDS ring; three output waves take every third
//         chunk and form O = (s e^c Q) S + M V_n from S and V_n handed over
//         through LDS slots guarded by counters.
//
// The fused entry (deltanet_chunk_prefill_fused) runs the same two kernels
// on raw inputs: the prep L2-normalises q and k rows, converts fp16 v to
// bf16 and forms g and beta from the gate inputs as it loads them, and the
// scan stores o in the I/O dtype and the final state over the initial one.
#include "gdn_common.h"
#include "gdn_hip.h"

#include <math.h>

#include <algorithm>

namespace gdn {
namespace {

constexpr int kPrepThreads = 256;
// scan work-group: 8 waves (chains, loaders, output waves; see the scan kernel)
constexpr int kScanThreads = 512;
constexpr int kOutWaves = 3;

// Per chunk-head record sizes (elements)
constexpr int kWfElems = kChunk * kDK;     // fp16: -W, 16 A-fragments (4 row tiles x 4 k-blocks)
constexpr int kKfElems = kDK * kChunk;     // fp16: decayed K^T, 16 A-fragments (8 dk tiles x 2 k-blocks)
constexpr int kUfElems = kChunk * kDV;     // fp16: U in accumulator order, 8 slices x 2 tile pairs
constexpr int kMfElems = kChunk * kChunk;  // fp16: M, 8 A-fragments (4 row tiles x 2 k-blocks)
constexpr int kQfElems = kChunk * kDK;     // fp16: Q, 16 fragments (4 row tiles x 4 k-blocks), per GQA group
constexpr int kGateFloats = 128;           // fp32: s e^c [64] | e^{c_63} | unused
constexpr int kGateDecay = 64;

struct Workspace {
    _Float16* Wf;
    _Float16* Kf;
    _Float16* Uf;
    _Float16* Mf;
    _Float16* Qf;   // at the chunk-head of each GQA group's first v-head
    float* gates;
    float* dbgT;   // optional: T = (I-A)^-1, [chunk-head][64][64]
    float* dbgA;   // optional: A, same layout
    float* dbgC;   // optional: in-chunk cumsum of g, [chunk-head][64]
};

// Inputs of the prep kernel.  kRaw = 0: q, k (L2-normalised) and v are bf16,
// g and beta fp32.  kRaw = 1 / 2: q and k rows are raw bf16 / fp16 (the prep
// normalises them), v has the same dtype, and the gates are g and beta (fp32)
// when `a` is null, else they come from a, b (per token and v-head, same
// dtype), A_log (fp32) and dt_bias (same dtype) per v-head.
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

__host__ __device__ inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

// Byte layout of the workspace for `nch` chunk-heads.  The three debug
// regions stay last: the torch binding finds them from the end.
struct WsLayout {
    size_t wf, kf, uf, mf, qf, gates, dbgT, dbgA, dbgC, total;
    __host__ explicit WsLayout(size_t nch) {
        size_t off = 0;
        wf = off;    off += align256(nch * kWfElems * 2);
        kf = off;    off += align256(nch * kKfElems * 2);
        uf = off;    off += align256(nch * kUfElems * 2);
        mf = off;    off += align256(nch * kMfElems * 2);
        qf = off;    off += align256(nch * kQfElems * 2);
        gates = off; off += align256(nch * kGateFloats * 4);
        dbgT = off;  off += align256(nch * kChunk * kChunk * 4);
        dbgA = off;  off += align256(nch * kChunk * kChunk * 4);
        dbgC = off;  off += align256(nch * kChunk * 4);
        total = off;
    }
};

// ---------------------------------------------------------------------------
// Sequence / chunk bookkeeping.  Fixed-length batches (cu == nullptr) are N
// sequences of length T laid out back to back, which is exactly the packed
// varlen layout with cu[i] = i * T.
// ---------------------------------------------------------------------------
__device__ inline int seq_start(const int32_t* cu, int T, int s) { return cu ? cu[s] : s * T; }
__device__ inline int seq_len(const int32_t* cu, int T, int s) { return cu ? cu[s + 1] - cu[s] : T; }

// Block-cooperative: number of chunks in sequences [0, upto).  Every thread of
// the block must call it; the result is returned to all threads.
template <int NT>
__device__ int chunks_before(const int32_t* cu, int T, int upto, int* red) {
    if (!cu) return upto * ((T + kChunk - 1) / kChunk);
    int acc = 0;
    for (int s = threadIdx.x; s < upto; s += NT) acc += (cu[s + 1] - cu[s] + kChunk - 1) / kChunk;
    for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
    __syncthreads();
    int tot = 0;
    for (int w = 0; w < NT / 64; ++w) tot += red[w];
    __syncthreads();
    return tot;
}

// Block-cooperative: map global chunk id -> (sequence, first token, rows).
// Returns false (uniformly) when cid is past the last chunk.  `red` holds NT
// ints of scratch.
template <int NT>
__device__ bool locate_chunk(const int32_t* cu, int N, int T, int cid, int* red,
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
    // running scan over sequences in blocks of NT
    int base = 0;
    bool found = false;
    for (int s0 = 0; s0 < N; s0 += NT) {
        const int s = s0 + (int)threadIdx.x;
        const int cnt = (s < N) ? (cu[s + 1] - cu[s] + kChunk - 1) / kChunk : 0;
        // inclusive block scan (Hillis-Steele through LDS)
        __syncthreads();
        red[threadIdx.x] = cnt;
        __syncthreads();
        for (int off = 1; off < NT; off <<= 1) {
            const int add = (threadIdx.x >= (unsigned)off) ? red[threadIdx.x - off] : 0;
            __syncthreads();
            red[threadIdx.x] += add;
            __syncthreads();
        }
        const int incl = red[threadIdx.x];
        const int total = red[NT - 1];
        const int excl = incl - cnt;
        __syncthreads();
        if (cnt > 0 && cid >= base + excl && cid < base + incl) {
            red[0] = s;
            red[1] = cid - base - excl;
        }
        __syncthreads();
        if (cid < base + total) {
            seq = red[0];
            const int c = red[1];
            tok0 = cu[seq] + c * kChunk;
            rows = min(kChunk, cu[seq + 1] - cu[seq] - c * kChunk);
            found = true;
        }
        __syncthreads();
        base += total;
        if (found) break;
    }
    return found;
}

__device__ inline half8 bf16x8_to_half8(uint4 raw) {
    half8 h;
    const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        h[2 * p] = (_Float16)bf16_bits_to_f32(w[p] & 0xffffu);
        h[2 * p + 1] = (_Float16)bf16_bits_to_f32(w[p] >> 16);
    }
    return h;
}

// Two 4-element bf16 pieces (k-map registers 0..3 and 4..7) as one operand
__device__ inline bf16x8 bf16_frag(uint2 lo, uint2 hi) {
    const u32x4 w = {lo.x, lo.y, hi.x, hi.y};
    return __builtin_bit_cast(bf16x8, w);
}

__device__ inline half8 bf16_frag_to_half8(uint2 lo, uint2 hi) {
    const uint4 w = {lo.x, lo.y, hi.x, hi.y};
    return bf16x8_to_half8(w);
}

__device__ __forceinline__ f32x4 mfma_f32_16x16x4(float a, float b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

constexpr float kLog2e = 1.4426950408889634f;

// ---------------------------------------------------------------------------
// prep kernel: one work-group (4 waves) per (chunk, v-head)
// ---------------------------------------------------------------------------
constexpr int kKS = kDK + 8;      // bf16 K row pitch: 136 halves (272 B, 16-byte aligned)
constexpr int kMS = kChunk + 4;   // fp32 A / T row pitch: 68 floats

struct PrepSmem {
    uint16_t Kr[kChunk * kKS];   // K rows (bf16, as loaded), [token][dk]
    // A (strictly lower, row-major) on entry.  The inverse overwrites it in
    // place: diagonal blocks T_ii row-major at (i, i); T_ij (i > j) stored
    // transposed at block (j, i), where A is zero and never read.  Its first
    // 1 KB is the sequence-lookup scratch before that.
    float AT[kChunk * kMS];
    float cl[kChunk];   // c * log2(e)
    float b[kChunk];    // beta
    float be[kChunk];   // beta e^c
    float ed[kChunk];   // e^{c_63 - c}
};

// T[r][c0 .. c0+3] (c0 a multiple of 4) from the in-place inverse layout.
// Row block rb and column block cb are compile-time, so the branch is uniform.
__device__ inline f32x4 t_row4(const float* AT, int rb, int cb, int r, int c0) {
    if (cb == rb) return *reinterpret_cast<const f32x4*>(&AT[r * kMS + c0]);
    if (cb > rb) return zero4();
    f32x4 t;
#pragma unroll
    for (int e = 0; e < 4; ++e) t[e] = AT[(c0 + e) * kMS + r];
    return t;
}

// Selector fragments: E_h is the 32 x 16 block of the identity that picks
// columns 16h .. 16h+15 of a 32-wide k-block, as an MFMA B operand
// (lane (g, l) holds rows kmap(g, j), column l).  X E_h copies a 16-column
// tile of X exactly (one product per output) into the accumulator layout,
// i.e. into the order in which a pair of such tiles is the k-mapped operand
// of the transposed product.
__device__ inline bf16x8 selector_frag(int h, int lg, int lm) {
    bf16x8 e;
#pragma unroll
    for (int j = 0; j < 8; ++j)
        e[j] = (lg == (lm >> 2) && j == 4 * h + (lm & 3)) ? (__bf16)1.0f : (__bf16)0.0f;
    return e;
}

// A raw 16-bit input element as fp32 (kRaw 1: bf16, 2: fp16)
template <int kRaw>
__device__ inline float raw16(uint32_t bits) {
    if constexpr (kRaw == 2) return (float)__builtin_bit_cast(_Float16, (uint16_t)bits);
    return __uint_as_float(bits << 16);
}

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

// n L2-normalised 16-bit values (fp32 sum of squares already reduced to
// `ss`), rounded to bf16 and packed in pairs: x rsqrt(ss + 1e-6), the
// reference adapter's normalisation (gdnChunkPrefillSm87.cu:52-84).
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

// KK^T and KQ^T products of wave W: A column block W (row tiles W..3) and
// M^T column block W (row tiles 0..W), k-blocks outermost so the five
// accumulators' products interleave instead of waiting on each other.
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

template <bool kDbg, int kRaw>
__global__ __launch_bounds__(kPrepThreads, 4) void gdn_prep_kernel(
    PrepIn in, const int32_t* __restrict__ cu, int N, int T, int HV, int HK, int nch_bound,
    float scale, Workspace ws) {
    __shared__ PrepSmem sm;
    const uint16_t* __restrict__ q = in.q;
    const uint16_t* __restrict__ k = in.k;
    const uint16_t* __restrict__ v = in.v;
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int lg = lane >> 4, lm = lane & 15;

    // Work-group id -> (chunk, k-head, member of its GQA group).  The rep
    // v-heads that read one k-head get ids 8 apart, i.e. the same XCD
    // (work-group i runs on XCD i % 8), so their q / k rows come from one L2.
    const int rep = HV / HK;
    const int L = blockIdx.x;
    const int rest = L >> 3;
    const int z = (rest / rep) * 8 + (L & 7);
    const int cid = z / HK, hk = z - cid * HK;
    if (cid >= nch_bound) return;
    const int hv = hk * rep + (rest % rep);

    int seq, tok0, rows;
    if (!locate_chunk<kPrepThreads>(cu, N, T, cid, reinterpret_cast<int*>(sm.AT), seq, tok0,
                                    rows))
        return;
    const size_t ch = (size_t)cid * HV + hv;

    // ---- global loads, all issued before any is consumed.  Rows past the
    // chunk's end read the last valid row (always in bounds) and are zeroed
    // afterwards, so no load sits behind a branch.  g and beta go first: the
    // gates need them before anything else arrives.
    // Raw gate inputs are kept as loaded and turned into g and beta only
    // after the K and Q loads are out: a use here would make wave 0 wait for
    // them before it issues its share of K.
    const bool raw_gate = kRaw != 0 && in.a != nullptr;
    uint32_t ga = 0u, gb = 0u, gdt = 0u;
    float gAl = 0.f;
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
    // K rows (16-byte pieces, row-major, bf16) go to LDS: thread t copies
    // pieces t, t + 256, ... (row piece / 16, columns 8 (piece % 16) ..).
    u32x4 raw[4];
    {
        const uint16_t* base = k + ((size_t)tok0 * HK + hk) * kDK + 8 * (tid & 15);
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) {
            const int r = min((tid >> 4) + 16 * ii, rows - 1);
            raw[ii] = *reinterpret_cast<const u32x4*>(base + (size_t)r * HK * kDK);
        }
    }
    // this wave's Q rows (k-map over dk); bf16 straight into the MFMA.
    // They are needed right after K (V, needed only at the end, is loaded
    // later)
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
    // opaque from here on: the compiler may not start the gate arithmetic
    // (and so wait for its inputs) before the K and Q loads above
    asm volatile("" : "+v"(ga), "+v"(gb), "+v"(gdt), "+v"(gAl)::"memory");
    float gv = 0.f, bv = 0.f;
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
        const float clast = __shfl(cs, 63, 64);
        const float c2 = cs * kLog2e;
        const float ec = exp2f(c2);
        sm.cl[lane] = c2;
        sm.b[lane] = bv;
        sm.be[lane] = bv * ec;
        sm.ed[lane] = exp2f((clast - cs) * kLog2e);
        float* gr = ws.gates + ch * kGateFloats;
        gr[lane] = scale * ec;
        if (lane == 0) gr[kGateDecay] = exp2f(clast * kLog2e);
        if (kDbg) ws.dbgC[ch * kChunk + lane] = cs;
    }

    // ---- K rows -> LDS as loaded; rows past the chunk's end are zeroed
    // (padding rows contribute nothing)
#pragma unroll
    for (int ii = 0; ii < 4; ++ii) {
        const int r = (tid >> 4) + 16 * ii;
        const uint32_t m = r < rows ? 0xffffffffu : 0u;
        *reinterpret_cast<u32x4*>(&sm.Kr[r * kKS + 8 * (tid & 15)]) = raw[ii] & m;
    }
    __syncthreads();

    // ---- A = -beta_r (k_r . k_j) Gamma_rj (r > j) and M = s (q_r . k_j) Gamma_rj (r >= j)
    // Wave w owns column block j in [16w, 16w+16) of A and query-row block
    // r in [16w, 16w+16) of M (computed as M^T = K Q^T so the accumulator is
    // already in A-fragment order for the scan).
    bf16x8 sel[2];
    sel[0] = selector_frag(0, lg, lm);
    sel[1] = selector_frag(1, lg, lm);
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
        // column block w is written as zero
        // (computed for every element, then selected: no per-element
        // branches; the discarded exponentials may overflow harmlessly)
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
        // M^T tile (mt, w): element (key ck = 16mt + 4lg + i, query col)
        half4 mh[4];
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
            f32x4 val;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int ck = mt * 16 + 4 * lg + i;
                const float mv = scale * accM[mt][i] * __builtin_amdgcn_exp2f(ccol - clr[mt][i]);
                val[i] = ck <= col ? mv : 0.f;
            }
            mh[mt] = to_half4(val);
        }
        half8* mdst = reinterpret_cast<half8*>(ws.Mf + ch * kMfElems);
        mdst[(wave * 2 + 0) * 64 + lane] = cat8(mh[0], mh[1]);
        mdst[(wave * 2 + 1) * 64 + lane] = cat8(mh[2], mh[3]);
        // this wave's Q rows as fp16 fragments; the v-heads of a GQA group
        // share them, so only the group's first writes them
        if (hv == hk * rep) {
            half8* qdst = reinterpret_cast<half8*>(ws.Qf + ch * kQfElems);
            const bool ok = wave * 16 + lm < rows;
#pragma unroll
            for (int kb = 0; kb < 4; ++kb)
                qdst[(wave * 4 + kb) * 64 + lane] = bf16_frag_to_half8(ok ? qr[kb][0] : z2, ok ? qr[kb][1] : z2);
        }
    }
    // ---- K^T fragments (dk tiles 2w, 2w+1; k-map over tokens): the
    // accumulator-layout K tiles of token tiles 2kb, 2kb+1 form k-block kb.
    // kt (unscaled) feeds W^T below; the decayed e^{c_63 - c_tau} k_tau[dk]
    // fragments are the scan's.
    half8 kt[2][2];
    {
        // K tiles (token tile tt, dk tile 2w + p) in accumulator layout, from
        // this wave's dk block of the K rows
        f32x4 kd[2][4];
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) {
            const uint16_t* src = &sm.Kr[(tt * 16 + lm) * kKS + 32 * wave + 4 * lg];
            const bf16x8 kw = bf16_frag(*reinterpret_cast<const uint2*>(src),
                                        *reinterpret_cast<const uint2*>(src + 16));
            kd[0][tt] = mfma16_bf16(kw, sel[0], zero4());
            kd[1][tt] = mfma16_bf16(kw, sel[1], zero4());
        }
        half8* kdst = reinterpret_cast<half8*>(ws.Kf + ch * kKfElems);
#pragma unroll
        for (int p = 0; p < 2; ++p) {
            const int mt = wave * 2 + p;
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                const int k0 = kb * 32 + 4 * lg;
                const f32x4 d0 = *reinterpret_cast<const f32x4*>(&sm.ed[k0]);
                const f32x4 d1 = *reinterpret_cast<const f32x4*>(&sm.ed[k0 + 16]);
                const f32x4 klo = kd[p][2 * kb], khi = kd[p][2 * kb + 1];
                kt[p][kb] = cat8(to_half4(klo), to_half4(khi));
                kdst[(mt * 2 + kb) * 64 + lane] = cat8(to_half4(klo * d0), to_half4(khi * d1));
            }
        }
    }
    __syncthreads();

    // this wave's V rows for value columns 32 w .. 32 w + 31 (the U slices
    // 2w, 2w+1), k-mapped like an A operand: token tile tt, row 16 tt + lm.
    // Issued here, a whole inverse ahead of their use, so they stay out of
    // the burst of K, Q and gate loads every group starts with.
    uint2 vr[4][2];
    {
        const uint16_t* vs = v + (size_t)hv * kDV + 32 * wave + 4 * lg;
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) {
            const uint16_t* vrow = vs + (size_t)(tok0 + min(16 * tt + lm, rows - 1)) * HV * kDV;
            vr[tt][0] = *reinterpret_cast<const uint2*>(vrow);
            vr[tt][1] = *reinterpret_cast<const uint2*>(vrow + 16);
        }
    }

    // ---- T = (I - A)^-1 in fp32, in place in AT
    // (1) 16x16 diagonal blocks by forward substitution: wave 0, lane =
    //     16 * block + column; T[i][c] = sum_{j<i} A[i][j] T[j][c] for i > c,
    //     T[c][c] = 1, T[i][c] = 0 for i < c.  Each lane keeps its column in
    //     registers and writes it after every row of the block was read.
    if (wave == 0) {
        const int b0 = lg * 16, cidx = lm;
        float col[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) col[i] = (i == cidx) ? 1.f : 0.f;
#pragma unroll
        for (int i = 1; i < 16; ++i) {
            const float* arow = &sm.AT[(b0 + i) * kMS + b0];
            float s = 0.f;
#pragma unroll
            for (int j4 = 0; j4 < (i + 3) / 4; ++j4) {
                const f32x4 a4 = *reinterpret_cast<const f32x4*>(arow + 4 * j4);
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (4 * j4 + e < i) s = fmaf(a4[e], col[4 * j4 + e], s);
            }
            if (i > cidx) col[i] = s;
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) sm.AT[(b0 + i) * kMS + b0 + cidx] = col[i];
    }
    __syncthreads();
    // (2) off-diagonal blocks level by level, block (i, j) with i - j = d:
    //     T_ij = T_ii * sum_{kk=j}^{i-1} A_{i,kk} T_{kk,j}
    //     on fp32 MFMA 16x16x4 with k = 4 * lane group + s, so the A operand
    //     is one 16-byte row read and a D-layout accumulator is directly the
    //     B operand of the next product.  Wave w takes block (w + d, w).
#pragma unroll
    for (int d = 1; d <= 3; ++d) {
        if (wave < 4 - d) {
            const int j = wave, i = wave + d;
            // one accumulator per term kk = j + u, so the terms' products
            // interleave; summed afterwards
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

    // ---- T fragments (rows 16mt + lm, k-map over tokens), scaled by beta
    // (U = T diag(beta) V) and by beta e^c (W = T diag(beta e^c) K).
    half8 xa[4][2], xb[4][2];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            const int r = mt * 16 + lm;
            const int k0 = kb * 32 + 4 * lg;
            const f32x4 t0 = t_row4(sm.AT, mt, 2 * kb, r, k0);
            const f32x4 t1 = t_row4(sm.AT, mt, 2 * kb + 1, r, k0 + 16);
            const f32x4 b0 = *reinterpret_cast<const f32x4*>(&sm.b[k0]);
            const f32x4 b1 = *reinterpret_cast<const f32x4*>(&sm.b[k0 + 16]);
            const f32x4 e0 = *reinterpret_cast<const f32x4*>(&sm.be[k0]);
            const f32x4 e1 = *reinterpret_cast<const f32x4*>(&sm.be[k0 + 16]);
            xa[mt][kb] = cat8(to_half4(t0 * b0), to_half4(t1 * b1));
            xb[mt][kb] = cat8(to_half4(t0 * e0), to_half4(t1 * e1));
        }
    }
    // ---- U = (T diag(beta)) V: slices nt = 2w, 2w+1, all four row tiles.
    // T is lower triangular: row tiles 0 and 1 see only tokens 0..31.
    {
        if constexpr (kRaw == 2) {
            // raw fp16 V rounded to bf16
#pragma unroll
            for (int tt = 0; tt < 4; ++tt) {
#pragma unroll
                for (int h2 = 0; h2 < 2; ++h2) {
                    vr[tt][h2].x = norm_pair<kRaw>(vr[tt][h2].x, 1.0f);
                    vr[tt][h2].y = norm_pair<kRaw>(vr[tt][h2].y, 1.0f);
                }
            }
        }
        bf16x8 vrf[4];
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) vrf[tt] = bf16_frag(vr[tt][0], vr[tt][1]);
        half8* udst = reinterpret_cast<half8*>(ws.Uf + ch * kUfElems);
#pragma unroll
        for (int p = 0; p < 2; ++p) {
            const int nt = wave * 2 + p;
            // V tiles (token tile tt, value tile nt) in accumulator layout;
            // token tiles 2kb, 2kb+1 form the k-block kb operand
            f32x4 vd[4];
#pragma unroll
            for (int tt = 0; tt < 4; ++tt) vd[tt] = mfma16_bf16(vrf[tt], sel[p], zero4());
            half8 vb[2];
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) vb[kb] = cat8(to_half4(vd[2 * kb]), to_half4(vd[2 * kb + 1]));
            half4 uh[4];
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) {
                f32x4 acc = mfma16(xa[mt][0], vb[0], zero4());
                if (mt >= 2) acc = mfma16(xa[mt][1], vb[1], acc);
                uh[mt] = to_half4(acc);
            }
            udst[(nt * 2 + 0) * 64 + lane] = cat8(uh[0], uh[1]);
            udst[(nt * 2 + 1) * 64 + lane] = cat8(uh[2], uh[3]);
        }
    }
    // ---- W^T = K^T (T diag(beta e^c))^T: dk tiles 2w, 2w+1 x token tiles nt.
    // The D layout of W^T tiles (2w, 2w+1) is W's A fragment (nt, k-block w).
    // Stored negated, so the scan's product -W S accumulates onto U and
    // yields V_n = U - W S directly.
    {
        half8* wdst = reinterpret_cast<half8*>(ws.Wf + ch * kWfElems);
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) {
            f32x4 acc0 = mfma16(kt[0][0], xb[nt][0], zero4());
            f32x4 acc1 = mfma16(kt[1][0], xb[nt][0], zero4());
            if (nt >= 2) {
                acc0 = mfma16(kt[0][1], xb[nt][1], acc0);
                acc1 = mfma16(kt[1][1], xb[nt][1], acc1);
            }
            wdst[(nt * 4 + wave) * 64 + lane] = cat8(to_half4(-acc0), to_half4(-acc1));
        }
    }
}

// ---------------------------------------------------------------------------
// scan kernel: one work-group (8 waves) per (SPW state slices, v-head,
// sequence).  The 128 value columns of a head's state form 8 slices of 16;
// columns evolve independently, so each slice has its own serial chain.
// SPW = 1 gives every slice its own CU (small grids: B = 1 fills the chip
// with 256 groups); SPW = 2 lets two chains share one copy of the chunk
// operands, twice the work per CU for grids larger than the chip.
//
//   chains      wave h < SPW keeps slice SPW*p + h's 128x16 fp32 state in
//               registers and per chunk forms V_n = U - W S and
//               S <- e^{c_63} S + K~^T V_n from a 3-stage LDS ring, reading
//               the next chunk's operands while the current products run.
//   loaders     three waves; each moves a third of a chunk's operands
//               (fragment ordered, 16 bytes per lane per fragment) from
//               global memory into the ring.  The groups of one head share
//               id % 8 (one XCD, one L2), so each operand line comes from
//               HBM once per XCD.
//   outputs     three waves; the j-th forms O (16 SPW columns) for chunks
//               c = j mod 3 from S_c and V_n handed over in LDS slot j, and
//               writes it through a private LDS tile with 16-byte stores.
//               Each issues its next chunk's loads before its stores, so it
//               never waits for its own stores to complete.
// Wave roles (waves w and w + 4 share a SIMD): SPW = 1: chain 0, loaders
// 1-3, wave 4 idle (the chain keeps its SIMD to itself), outputs 5-7;
// SPW = 2: chains 0-1, outputs 2, 3, 7, loaders 4-6.  Waves meet only
// through LDS counters with bounded waits, never through a work-group
// barrier, so no wave waits on one it does not depend on.
// ---------------------------------------------------------------------------
constexpr int kSlicesPerHead = kDV / kBV;   // 8
constexpr int kRing = 3;               // operand stages
constexpr int kHand = kOutWaves;       // hand-off slots: chunk c uses slot c % kHand (= its output wave)
constexpr int kLoaders = 3;
constexpr int kSpinLimit = 1 << 20;    // bounded waits: ~0.1 s, then the wave gives up

// Fragments of one chunk: W 0..15, K~^T 16..31, then U of each slice (2
// each); split over the loaders, fragment f sits at index f of a stage.
template <int SPW>
struct ScanCfg {
    static constexpr int kStageFrags = 32 + 2 * SPW;
    static constexpr int kLoaderBegin[kLoaders + 1] = {0, 12, 24, kStageFrags};
    static constexpr int kGroupsPerHead = kSlicesPerHead / SPW;
    static __device__ int loader_of(int wave) { return SPW == 1 ? wave - 1 : wave - 4; }   // -1 .. : not a loader
    static __device__ int output_of(int wave) { return SPW == 1 ? wave - 5 : (wave == 7 ? 2 : wave - 2); }
};

template <int SPW>
struct ScanSmem {
    half8 stage[kRing][ScanCfg<SPW>::kStageFrags][64];
    float gd[kRing];                       // e^{c_63} of the chunk in each stage
    half8 hs[kHand][SPW][4][64];           // S at the start of a chunk, per chain, B-fragments
    half8 hv[kHand][SPW][2][64];           // V_n, per chain, B-fragments
    uint16_t ot[kOutWaves][kChunk][SPW * kBV];   // output tiles (bf16), one per output wave
    int filled[4];                         // per loader: chunks whose part sits in the ring
    int freed[SPW];                        // per chain: chunks whose stage it has finished reading
    int ready[SPW];                        // per chain: chunks whose hand-off part is written
    int cons[kHand];                       // per slot: 1 + the chunk an output wave last read from it
    int red[kScanThreads / 64];
    int order[64];                         // varlen: sequences by length, longest first
};

__device__ __forceinline__ int lds_load_relaxed(const int* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

__device__ __forceinline__ void lds_store_relaxed(int* p, int v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// Wait until every LDS operation of this wave has completed.  The builtin
// (rather than inline asm) lets the compiler's own wait-count tracking see
// that the wave's LDS loads have landed, so it adds no second wait later;
// the empty asm statements keep memory operations on their side of it.
__device__ inline void lds_wait_all() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0); vmcnt 63, expcnt 7: no wait
    asm volatile("" ::: "memory");
}

// Wait (bounded) until *flag >= target; false when the bound ran out.
__device__ inline bool wait_ge(const int* flag, int target) {
    for (int it = 0; it < kSpinLimit; ++it) {
        if (lds_load_relaxed(flag) >= target) return true;
        __builtin_amdgcn_s_sleep(1);
    }
    return false;
}

// Smallest of n counters (LDS reads issued together).
template <int n>
__device__ inline int lds_min(const int* p) {
    int m = lds_load_relaxed(p);
#pragma unroll
    for (int i = 1; i < n; ++i) m = min(m, lds_load_relaxed(p + i));
    return m;
}

// Wait (bounded) until the smallest of n counters is >= target.
template <int n>
__device__ inline bool wait_min(const int* p, int target) {
    for (int it = 0; it < kSpinLimit; ++it) {
        if (lds_min<n>(p) >= target) return true;
        __builtin_amdgcn_s_sleep(1);
    }
    return false;
}

// Wait (bounded) until every loader has put chunk c in the ring and the
// hand-off slot of chunk c is free (the output wave read chunk c - kHand);
// the four LDS reads of a poll are issued together.
template <int SPW>
__device__ inline bool wait_chain(const ScanSmem<SPW>& sm, int c, int slot) {
    static_assert(kLoaders == 3, "three loader counters");
    const int cons_need = c >= kHand ? c - kHand + 1 : 0;
    for (int it = 0; it < kSpinLimit; ++it) {
        const int f0 = lds_load_relaxed(&sm.filled[0]), f1 = lds_load_relaxed(&sm.filled[1]),
                  f2 = lds_load_relaxed(&sm.filled[2]), cn = lds_load_relaxed(&sm.cons[slot]);
        if (min(f0, min(f1, f2)) >= c + 1 && cn >= cons_need) return true;
        __builtin_amdgcn_s_sleep(1);
    }
    return false;
}

// One loader wave (see the scan kernel): fragments kLoaderBegin[J] ..
// kLoaderBegin[J+1] of every chunk, with compile-time fragment indices so
// the loads and LDS writes are straight-line code; loader 2 also moves the
// decay.  Two chunks are in flight: chunk c+1's loads are issued before
// chunk c is written.  Loads past the last chunk re-read it (always in
// bounds) and are dropped.
template <int SPW, int J>
__device__ void run_loader(ScanSmem<SPW>& sm, const Workspace& ws, int chunk0, int nch, int hv,
                           int HV, int sl0, int lane) {
    constexpr int f0 = ScanCfg<SPW>::kLoaderBegin[J];
    constexpr int nf = ScanCfg<SPW>::kLoaderBegin[J + 1] - f0;
    auto load = [&](int c, u32x4 (&fr)[nf], float& dg) {
        const size_t chh = (size_t)(chunk0 + min(c, nch - 1)) * HV + hv;
        const u32x4* wsrc = reinterpret_cast<const u32x4*>(ws.Wf + chh * kWfElems) + lane;
        const u32x4* ksrc = reinterpret_cast<const u32x4*>(ws.Kf + chh * kKfElems) + lane;
        const u32x4* usrc = reinterpret_cast<const u32x4*>(ws.Uf + chh * kUfElems) + sl0 * 2 * 64 + lane;
#pragma unroll
        for (int i = 0; i < nf; ++i) {
            const int f = f0 + i;
            fr[i] = f < 16 ? wsrc[f * 64] : (f < 32 ? ksrc[(f - 16) * 64] : usrc[(f - 32) * 64]);
        }
        if (J == kLoaders - 1) dg = ws.gates[chh * kGateFloats + kGateDecay];
    };
    auto store = [&](int c, int st, const u32x4 (&fr)[nf], float dg) -> bool {
        if (c >= kRing && !wait_min<SPW>(sm.freed, c - kRing + 1)) return false;
        asm volatile("" ::: "memory");
#pragma unroll
        for (int i = 0; i < nf; ++i) *reinterpret_cast<u32x4*>(&sm.stage[st][f0 + i][lane]) = fr[i];
        if (J == kLoaders - 1 && lane == 0) sm.gd[st] = dg;
        lds_wait_all();
        if (lane == 0) lds_store_relaxed(&sm.filled[J], c + 1);
        return true;
    };
    if (nch > 0) {
        u32x4 fa[nf], fb[nf];
        float da = 0.f, db = 0.f;
        load(0, fa, da);
        int st = 0;
        for (int c = 0; c < nch; c += 2) {
            load(c + 1, fb, db);
            if (!store(c, st, fa, da)) break;
            st = (st == kRing - 1) ? 0 : st + 1;
            if (c + 1 >= nch) break;
            load(c + 2, fa, da);
            if (!store(c + 1, st, fb, db)) break;
            st = (st == kRing - 1) ? 0 : st + 1;
        }
    }
}

// kOutF16: o is stored as fp16 (the bf16-rounded value, converted exactly),
// else bf16.  s0 and sf may be the same buffer: a chain reads its slice of
// the initial state before its first chunk and writes the same elements
// after its last, and no other wave touches either.
template <int SPW, bool kOutF16>
__global__ __launch_bounds__(kScanThreads, 1) void gdn_scan_kernel(
    Workspace ws, uint16_t* __restrict__ o, const float* s0, float* sf,
    const int32_t* __restrict__ cu, int N, int T, int HV, int HK) {
    using Cfg = ScanCfg<SPW>;
    constexpr int kStageFrags = Cfg::kStageFrags;
    __shared__ ScanSmem<SPW> sm;
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int lg = lane >> 4, lm = lane & 15;

    // XCD-aware id: the groups of one (seq, head) pair share id % 8 (work-group
    // i runs on XCD i % 8), so they read the head's operands from one L2
    const int id = blockIdx.x;
    const int xcd = id & 7, qd = id >> 3;
    const int sp = qd % Cfg::kGroupsPerHead;
    const int pair = (qd / Cfg::kGroupsPerHead) * 8 + xcd;
    if (pair >= N * HV) return;
    int seq = pair / HV;
    const int hv = pair - seq * HV;
    // Packed sequences of different lengths: work-groups start in id order as
    // CUs free up, so hand the low ids to the longest sequences (longest
    // processing time first); a grid of more groups than CUs then ends close
    // to total work / CUs instead of waiting on a long sequence started last.
    if (cu && N <= 64) {
        if (tid < N) {
            const int my = cu[tid + 1] - cu[tid];
            int rank = 0;
            for (int u = 0; u < N; ++u) {
                const int lu = cu[u + 1] - cu[u];
                rank += (lu > my || (lu == my && u < tid)) ? 1 : 0;
            }
            sm.order[rank] = tid;
        }
        __syncthreads();
        seq = sm.order[seq];
    }
    const int hk = hv / (HV / HK);
    const int sl0 = SPW * sp;   // first slice of this group

    const int len = seq_len(cu, T, seq);
    const int tok0 = seq_start(cu, T, seq);
    const int nch = (len + kChunk - 1) / kChunk;
    const int chunk0 = __builtin_amdgcn_readfirstlane(chunks_before<kScanThreads>(cu, T, seq, sm.red));
    if (tid < 4) lds_store_relaxed(&sm.filled[tid], 0);
    if (tid < SPW) {
        lds_store_relaxed(&sm.freed[tid], 0);
        lds_store_relaxed(&sm.ready[tid], 0);
    }
    if (tid < kHand) lds_store_relaxed(&sm.cons[tid], 0);
    __syncthreads();

    const int li = Cfg::loader_of(wave), oi = Cfg::output_of(wave);
    if (wave < SPW) {
        // ---------------- chain wave h: slice sl0 + h
        const int h = wave;
        const size_t sbase = ((size_t)seq * HV + hv) * kDK * kDV + (sl0 + h) * kBV + lm;
        f32x4 S[8];
        if (s0) {   // one uniform branch: all 32 loads in flight together
#pragma unroll
            for (int t = 0; t < 8; ++t) {
#pragma unroll
                for (int i = 0; i < 4; ++i) S[t][i] = s0[sbase + (size_t)(t * 16 + 4 * lg + i) * kDV];
            }
        } else {
#pragma unroll
            for (int t = 0; t < 8; ++t) S[t] = zero4();
        }
        half8 sb[4];
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) sb[kb] = cat8(to_half4(S[2 * kb]), to_half4(S[2 * kb + 1]));

        // Software pipeline: chunk c + 1's W, U and decay are read from the
        // ring while chunk c's V_n is formed, its K~^T while the state update
        // runs, so the serial chain -W S + U -> V_n -> S waits on the matrix
        // cores, not on LDS.
        half8 wv[16], kv[16], u0, u1;
        float d = 0.f;
        auto read_w = [&](int st) {
            const half8(&sg)[kStageFrags][64] = sm.stage[st];
#pragma unroll
            for (int f = 0; f < 16; ++f) wv[f] = sg[f][lane];
            u0 = sg[32 + 2 * h][lane];
            u1 = sg[33 + 2 * h][lane];
            d = sm.gd[st];
        };
        auto read_k = [&](int st) {
            const half8(&sg)[kStageFrags][64] = sm.stage[st];
#pragma unroll
            for (int f = 0; f < 16; ++f) kv[f] = sg[16 + f][lane];
        };
        // counters polled during the previous chunk (monotonic, so values
        // that already satisfy a wait let the chain skip the wait)
        int pf0 = 0, pf1 = 0, pf2 = 0, pfc = 0;
        // chunk c's operands are in the ring and its hand-off slot is free
        // (its previous chunk, c - kHand, was read)
        auto ensure = [&](int c, int slot) -> bool {
            const int cons_need = c >= kHand ? c - kHand + 1 : 0;
            if (min(pf0, min(pf1, pf2)) >= c + 1 && pfc >= cons_need) return true;
            return wait_chain<SPW>(sm, c, slot);
        };
        bool ok = nch > 0 && ensure(0, 0);
        if (ok) {
            asm volatile("" ::: "memory");
            read_w(0);
            read_k(0);
        }
        int st = 0;      // stage of chunk c
        int hslot = 0;   // hand-off slot of chunk c
        for (int c = 0; c < nch && ok; ++c) {
            const int stn = (st == kRing - 1) ? 0 : st + 1;
            const int hsn = (hslot == kHand - 1) ? 0 : hslot + 1;
            const bool more = c + 1 < nch;
            // S_c goes to the hand-off slot now: it is known before the
            // chunk's products
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) sm.hs[hslot][h][kb][lane] = sb[kb];
            // V_n = U - W S (64 x 16): the stored -W accumulates onto U; k
            // over dk, the four row tiles independent and issued round-robin
            f32x4 P[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                P[0][i] = (float)u0[i];
                P[1][i] = (float)u0[4 + i];
                P[2][i] = (float)u1[i];
                P[3][i] = (float)u1[4 + i];
            }
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
                for (int mt = 0; mt < 4; ++mt) P[mt] = mfma16(wv[mt * 4 + kb], sb[kb], P[mt]);
            }
            const float dc = d;
            // chunk c + 1's W, U and decay while the products run
            if (more) {
                ok = ok && ensure(c + 1, hsn);
                asm volatile("" ::: "memory");
                read_w(stn);
            }
            // independent of P: the decayed state
#pragma unroll
            for (int t = 0; t < 8; ++t) S[t] = S[t] * dc;
            half8 vb[2];
            vb[0] = cat8(to_half4(P[0]), to_half4(P[1]));
            vb[1] = cat8(to_half4(P[2]), to_half4(P[3]));
            sm.hv[hslot][h][0][lane] = vb[0];
            sm.hv[hslot][h][1][lane] = vb[1];
            // S = d S + K~^T V_n (128 x 16), k over tokens; eight independent
            // tiles, issued round-robin
#pragma unroll
            for (int t = 0; t < 8; ++t) S[t] = mfma16(kv[t * 2 + 0], vb[0], S[t]);
#pragma unroll
            for (int t = 0; t < 8; ++t) S[t] = mfma16(kv[t * 2 + 1], vb[1], S[t]);
            // stage st is read and chunk c's hand-off written: publish both,
            // then chunk c + 1's K~^T while the update runs
            lds_wait_all();
            if (lane == 0) {
                lds_store_relaxed(&sm.freed[h], c + 1);
                lds_store_relaxed(&sm.ready[h], c + 1);
            }
            if (more) read_k(stn);
            pf0 = lds_load_relaxed(&sm.filled[0]);
            pf1 = lds_load_relaxed(&sm.filled[1]);
            pf2 = lds_load_relaxed(&sm.filled[2]);
            pfc = lds_load_relaxed(&sm.cons[(hsn == kHand - 1) ? 0 : hsn + 1]);
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) sb[kb] = cat8(to_half4(S[2 * kb]), to_half4(S[2 * kb + 1]));
            st = stn;
            hslot = hsn;
        }
#pragma unroll
        for (int t = 0; t < 8; ++t) {
#pragma unroll
            for (int i = 0; i < 4; ++i) sf[sbase + (size_t)(t * 16 + 4 * lg + i) * kDV] = S[t][i];
        }
    } else if (li >= 0 && li < kLoaders) {
        if (li == 0) run_loader<SPW, 0>(sm, ws, chunk0, nch, hv, HV, sl0, lane);
        else if (li == 1) run_loader<SPW, 1>(sm, ws, chunk0, nch, hv, HV, sl0, lane);
        else run_loader<SPW, 2>(sm, ws, chunk0, nch, hv, HV, sl0, lane);
    } else if (oi >= 0 && oi < kOutWaves) {
        // ---------------- output waves: chunks c = ow, ow + kOutWaves, ...
        const int ow = oi;
        // operands of chunk c (clamped into range, so a look-ahead past the
        // end re-reads the last chunk): Q fragments (fp16, row tile mt,
        // k-block kb, from the GQA group's first v-head), s e^c of the
        // lane's tokens and M fragments
        half8 qf[16], mf[8];
        float es[4];
        const int hq = hk * (HV / HK);
        auto load_ops = [&](int c) {
            const size_t cb = (size_t)(chunk0 + min(c, nch - 1)) * HV;
            const size_t chh = cb + hv;
            const half8* qsrc = reinterpret_cast<const half8*>(ws.Qf + (cb + hq) * kQfElems) + lane;
            const half8* msrc = reinterpret_cast<const half8*>(ws.Mf + chh * kMfElems) + lane;
#pragma unroll
            for (int f = 0; f < 16; ++f) qf[f] = qsrc[f * 64];
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) es[mt] = ws.gates[chh * kGateFloats + 16 * mt + lm];
#pragma unroll
            for (int f = 0; f < 8; ++f) mf[f] = msrc[f * 64];
        };
        if (ow < nch) load_ops(ow);
        uint16_t(&ot)[kChunk][SPW * kBV] = sm.ot[ow];
        for (int c = ow; c < nch; c += kOutWaves) {
            const int rows = min(kChunk, len - c * kChunk);
            if (!wait_min<SPW>(sm.ready, c + 1)) break;
            asm volatile("" ::: "memory");
            const int slot = ow;   // c % kHand
            half8 hsb[SPW][4], hvb[SPW][2];
#pragma unroll
            for (int s2 = 0; s2 < SPW; ++s2) {
#pragma unroll
                for (int kb = 0; kb < 4; ++kb) hsb[s2][kb] = sm.hs[slot][s2][kb][lane];
                hvb[s2][0] = sm.hv[slot][s2][0][lane];
                hvb[s2][1] = sm.hv[slot][s2][1][lane];
            }
            lds_wait_all();
            if (lane == 0) lds_store_relaxed(&sm.cons[slot], c + 1);

            // O^T = (S^T Q^T) diag(s e^c) + V_n^T M^T per slice (operands
            // swapped so each lane holds four consecutive columns of one
            // token, whose s e^c then scales them); each accumulator's
            // dependent products are issued round-robin
            f32x4 ov[SPW][4];
#pragma unroll
            for (int s2 = 0; s2 < SPW; ++s2) {
#pragma unroll
                for (int mt = 0; mt < 4; ++mt) ov[s2][mt] = mfma16(hsb[s2][0], qf[mt * 4], zero4());
#pragma unroll
                for (int kb = 1; kb < 4; ++kb) {
#pragma unroll
                    for (int mt = 0; mt < 4; ++mt) ov[s2][mt] = mfma16(hsb[s2][kb], qf[mt * 4 + kb], ov[s2][mt]);
                }
#pragma unroll
                for (int mt = 0; mt < 4; ++mt) ov[s2][mt] = ov[s2][mt] * es[mt];
#pragma unroll
                for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
                    for (int mt = 0; mt < 4; ++mt) ov[s2][mt] = mfma16(hvb[s2][kb], mf[mt * 2 + kb], ov[s2][mt]);
                }
            }
            load_ops(c + kOutWaves);   // the operand registers are free again
            // O tile (64 rows x 16 SPW columns, bf16) through LDS, then 16-byte
            // stores: lane (g, l) holds token 16 mt + l, columns 16 s2 + 4g ..
            // + 3 (one 8-byte write each); lane l then writes row l in
            // 8-column pieces
            auto out16 = [](float x) -> uint32_t {
                const uint32_t bb = f32_to_bf16_bits(x);
                if constexpr (kOutF16)
                    return __builtin_bit_cast(uint16_t, (_Float16)__uint_as_float(bb << 16));
                return bb;
            };
#pragma unroll
            for (int s2 = 0; s2 < SPW; ++s2) {
#pragma unroll
                for (int mt = 0; mt < 4; ++mt) {
                    uint2 pk;
                    pk.x = out16(ov[s2][mt][0]) | (out16(ov[s2][mt][1]) << 16);
                    pk.y = out16(ov[s2][mt][2]) | (out16(ov[s2][mt][3]) << 16);
                    *reinterpret_cast<uint2*>(&ot[mt * 16 + lm][s2 * kBV + 4 * lg]) = pk;
                }
            }
            asm volatile("" ::: "memory");   // LDS ops of one wave complete in order
            if (lane < rows) {
                const u32x4* src = reinterpret_cast<const u32x4*>(&ot[lane][0]);
                u32x4* dst = reinterpret_cast<u32x4*>(o + ((size_t)(tok0 + c * kChunk + lane) * HV + hv) * kDV + sl0 * kBV);
#pragma unroll
                for (int p4 = 0; p4 < 2 * SPW; ++p4) dst[p4] = src[p4];
            }
        }
    }
    // any other wave (SPW = 1: wave 4) is idle: waves w and w + 4 share a
    // SIMD, so the chain keeps its SIMD to itself
}

// raw: 0 for prepared inputs, 1 / 2 for raw bf16 / fp16 q, k (normalised in
// the prep; then v and o have that dtype too).
hipError_t launch_prefill(const PrepIn& in, int raw, void* o, const float* s0, float* sf,
                          const int32_t* cu, int N, int T, int total_tokens, int HV, int HK,
                          size_t nch_bound, void* workspace, size_t workspace_bytes,
                          hipStream_t stream, int dump_debug, hipEvent_t* ev = nullptr,
                          int only = -1) {
    const WsLayout L(nch_bound * (size_t)HV);
    if (workspace_bytes < L.total) return hipErrorInvalidValue;
    char* base = static_cast<char*>(workspace);
    Workspace ws;
    ws.Wf = reinterpret_cast<_Float16*>(base + L.wf);
    ws.Kf = reinterpret_cast<_Float16*>(base + L.kf);
    ws.Uf = reinterpret_cast<_Float16*>(base + L.uf);
    ws.Mf = reinterpret_cast<_Float16*>(base + L.mf);
    ws.Qf = reinterpret_cast<_Float16*>(base + L.qf);
    ws.gates = reinterpret_cast<float*>(base + L.gates);
    ws.dbgT = dump_debug ? reinterpret_cast<float*>(base + L.dbgT) : nullptr;
    ws.dbgA = dump_debug ? reinterpret_cast<float*>(base + L.dbgA) : nullptr;
    ws.dbgC = dump_debug ? reinterpret_cast<float*>(base + L.dbgC) : nullptr;
    const float scale = 1.0f / sqrtf((float)kDK);

    // ev (optional): kPrefillKernels + 1 events recorded around the launches
    if (ev) (void)hipEventRecord(ev[0], stream);
    // only (optional): launch just that kernel of the pipeline (0 prep, 1 scan)
    if (nch_bound > 0 && total_tokens > 0 && only != 1) {
        const int rep = HV / HK;
        const size_t groups = (nch_bound * (size_t)HK + 7) / 8;
        auto kern = raw == 1 ? gdn_prep_kernel<false, 1>
                    : raw == 2 ? gdn_prep_kernel<false, 2>
                    : dump_debug ? gdn_prep_kernel<true, 0> : gdn_prep_kernel<false, 0>;
        hipLaunchKernelGGL(kern, dim3((unsigned)(groups * 8 * rep)), dim3(kPrepThreads), 0, stream,
                           in, cu, N, T, HV, HK, (int)nch_bound, scale, ws);
        hipError_t err = hipGetLastError();
        if (err != hipSuccess) return err;
    }
    if (ev) (void)hipEventRecord(ev[1], stream);
    if (only == 0) return hipSuccess;
    // one slice per work-group while that still fits the chip in one pass,
    // else two (twice the work per CU)
    const int pairs = N * HV;
    const int groups = (pairs + 7) / 8;
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        cus = 0;   // unknown: two slices per group
    const bool one = (long)groups * 8 * kSlicesPerHead <= (long)cus;
    const bool f16 = raw == 2;
    auto scan = one ? (f16 ? gdn_scan_kernel<1, true> : gdn_scan_kernel<1, false>)
                    : (f16 ? gdn_scan_kernel<2, true> : gdn_scan_kernel<2, false>);
    const int gph = one ? ScanCfg<1>::kGroupsPerHead : ScanCfg<2>::kGroupsPerHead;
    hipLaunchKernelGGL(scan, dim3((unsigned)(groups * 8 * gph)), dim3(kScanThreads), 0, stream, ws,
                       static_cast<uint16_t*>(o), s0, sf, cu, N, T, HV, HK);
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

}  // namespace
}  // namespace gdn

using namespace gdn;

extern "C" size_t deltanet_prefill_workspace_size(int B, int T, int HV, int DK, int DV,
                                                  int chunk_size) {
    if (B <= 0 || T < 0 || HV <= 0 || DK != kDK || DV != kDV || chunk_size != kChunk) return 0;
    const size_t nc = (size_t)B * ((T + kChunk - 1) / kChunk);
    // at least one 256-byte block, so T = 0 (no chunks) still gets a valid
    // nonzero size and 0 keeps meaning "unsupported"
    return std::max<size_t>(WsLayout(nc * HV).total, 256);
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
    return std::max<size_t>(WsLayout(nc * HV).total, 256);
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
// prep kernel (transformers' use_qk_l2norm_in_kernel=True).  cu_seqlens NULL:
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
