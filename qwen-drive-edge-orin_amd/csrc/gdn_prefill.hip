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
//   prep  grid (chunks, HV):  all chunk-local work.  Writes W, decayed K^T,
//         scaled Q and M as fp16 MFMA A-operand fragments and U as fp32
//         accumulator fragments, so the scan issues one 16-byte load per lane
//         per fragment and never reshuffles.
//   scan  grid (8 slices x HV x sequences): the state S of one head is split
//         into 8 slices of 16 columns (columns of S evolve independently).
//         Wave 0 runs the serial chain V_n = U - W S, S <- d S + K~^T V_n
//         with the slice in registers for the whole sequence; wave 1 forms
//         O = Q~ S + M V_n from S and V_n handed over through a 2-deep LDS
//         ring.  Work-group ids are laid out so the 8 slices of a head land
//         on one XCD and share its L2.
#include "gdn_common.h"
#include "gdn_hip.h"

#include <math.h>

namespace gdn {
namespace {

constexpr int kPrepThreads = 256;
constexpr int kScanThreads = 128;

// Per chunk-head record sizes (elements)
constexpr int kWfElems = kChunk * kDK;      // fp16, 16 fragments of 64 lanes x 8
constexpr int kKfElems = kDK * kChunk;      // fp16, 16 fragments
constexpr int kQfElems = kChunk * kDK;      // fp16, 16 fragments
constexpr int kMfElems = kChunk * kChunk;   // fp16, 8 fragments
constexpr int kUfElems = kChunk * kDV;      // fp32, 8 slices x 4 tiles x 64 lanes x 4

struct Workspace {
    _Float16* Wf;
    _Float16* Kf;
    _Float16* Qf;
    _Float16* Mf;
    float* Uf;
    float* decay;
    float* dbgT;   // optional: T = (I-A)^-1, [chunk-head][64][64]
    float* dbgA;   // optional: A, same layout
    float* dbgC;   // optional: in-chunk cumsum of g, [chunk-head][64]
};

__host__ __device__ inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

// Byte layout of the workspace for `nch` chunk-heads.
struct WsLayout {
    size_t wf, kf, qf, mf, uf, decay, dbgT, dbgA, dbgC, total;
    __host__ explicit WsLayout(size_t nch) {
        size_t off = 0;
        wf = off;    off += align256(nch * kWfElems * 2);
        kf = off;    off += align256(nch * kKfElems * 2);
        qf = off;    off += align256(nch * kQfElems * 2);
        mf = off;    off += align256(nch * kMfElems * 2);
        uf = off;    off += align256(nch * kUfElems * 4);
        decay = off; off += align256(nch * 4);
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
    // wave reduce then cross-wave through LDS
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
// Returns false (uniformly) when cid is past the last chunk.
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

__device__ inline half4 bf16x4_to_half4(uint2 raw) {
    half4 h;
    h[0] = (_Float16)bf16_bits_to_f32(raw.x & 0xffffu);
    h[1] = (_Float16)bf16_bits_to_f32(raw.x >> 16);
    h[2] = (_Float16)bf16_bits_to_f32(raw.y & 0xffffu);
    h[3] = (_Float16)bf16_bits_to_f32(raw.y >> 16);
    return h;
}

// ---------------------------------------------------------------------------
// prep kernel: one work-group (4 waves) per (chunk, v-head)
// ---------------------------------------------------------------------------
constexpr int kKrStride = kDK + 8;      // fp16 row-major K  [64][136]
constexpr int kKtStride = kChunk + 8;   // fp16 K^T / V^T    [128][72]
constexpr int kMatStride = kChunk + 4;  // fp32 A / T        [64][68]

struct PrepSmem {
    _Float16 Kr[kChunk * kKrStride];
    _Float16 Kt[kDK * kKtStride];
    union {
        float A[kChunk * kMatStride];       // A, live until the inverse is done
        _Float16 Vt[kDV * kKtStride];       // V^T, written after the inverse
    } u;
    float T[kChunk * kMatStride];
    float c[kChunk];     // in-chunk cumsum of g
    float b[kChunk];     // beta
    float be[kChunk];    // beta * e^c
    float ed[kChunk];    // e^{c_63 - c}
    float es[kChunk];    // s * e^c
    int red[kPrepThreads];
};

__global__ __launch_bounds__(kPrepThreads, 2) void gdn_prep_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
    const uint16_t* __restrict__ v, const float* __restrict__ g,
    const float* __restrict__ beta, const int32_t* __restrict__ cu, int N, int T, int HV,
    int HK, float scale, Workspace ws) {
    __shared__ PrepSmem sm;
    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int lg = lane >> 4, lm = lane & 15;
    const int cid = blockIdx.x, hv = blockIdx.y;

    int seq, tok0, rows;
    if (!locate_chunk<kPrepThreads>(cu, N, T, cid, sm.red, seq, tok0, rows)) return;
    const int hk = hv / (HV / HK);
    const size_t ch = (size_t)cid * HV + hv;

    // ---- issue global loads: K (to LDS), V (kept in registers), Q fragments
    uint4 vraw[4];
#pragma unroll
    for (int it = 0; it < 4; ++it) {
        const int e = tid + it * kPrepThreads;  // 16-byte piece of the 64x128 tile
        const int r = e >> 4, c8 = (e & 15) * 8;
        uint4 kr = {0u, 0u, 0u, 0u}, vr = {0u, 0u, 0u, 0u};
        if (r < rows) {
            kr = *reinterpret_cast<const uint4*>(k + ((size_t)(tok0 + r) * HK + hk) * kDK + c8);
            vr = *reinterpret_cast<const uint4*>(v + ((size_t)(tok0 + r) * HV + hv) * kDV + c8);
        }
        vraw[it] = vr;
        const half8 kh = bf16x8_to_half8(kr);
        *reinterpret_cast<half8*>(&sm.Kr[r * kKrStride + c8]) = kh;
#pragma unroll
        for (int j = 0; j < 8; ++j) sm.Kt[(c8 + j) * kKtStride + r] = kh[j];
    }
    // Q rows of this wave's 16-row block, as B/A fragments for the 4 k-blocks
    half8 qf[4];
    {
        const int r = wave * 16 + lm;
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
            uint2 lo = {0u, 0u}, hi = {0u, 0u};
            if (r < rows) {
                const uint16_t* src = q + ((size_t)(tok0 + r) * HK + hk) * kDK + kb * 32 + 4 * lg;
                lo = *reinterpret_cast<const uint2*>(src);
                hi = *reinterpret_cast<const uint2*>(src + 16);
            }
            qf[kb] = cat8(bf16x4_to_half4(lo), bf16x4_to_half4(hi));
        }
    }
    // gates: wave 0 scans g over the 64 rows
    if (wave == 0) {
        const bool valid = lane < rows;
        const float gv = valid ? g[(size_t)(tok0 + lane) * HV + hv] : 0.f;
        const float bv = valid ? beta[(size_t)(tok0 + lane) * HV + hv] : 0.f;
        float cs = gv;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const float o = __shfl_up(cs, off, 64);
            if (lane >= off) cs += o;
        }
        const float clast = __shfl(cs, 63, 64);
        const float ec = expf(cs);
        sm.c[lane] = cs;
        sm.b[lane] = bv;
        sm.be[lane] = bv * ec;
        sm.ed[lane] = expf(clast - cs);
        sm.es[lane] = scale * ec;
        if (lane == 0) ws.decay[ch] = expf(clast);
        if (ws.dbgC) ws.dbgC[ch * kChunk + lane] = cs;
    }
    __syncthreads();

    // ---- A = -beta_r (k_r . k_j) Gamma_rj (r > j) and M = s (q_r . k_j) Gamma_rj (r >= j)
    // wave w owns column block j in [16w, 16w+16) of A and query-row block
    // r in [16w, 16w+16) of M (computed as M^T = K Q^T so the accumulator is
    // already in A-fragment order for the scan).
    {
        half8 kb_w[4];  // K rows of block w as B operand (B[k][n] = K[16w+n][k])
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
            const _Float16* src = &sm.Kr[(wave * 16 + lm) * kKrStride + kb * 32 + 4 * lg];
            kb_w[kb] = cat8(*reinterpret_cast<const half4*>(src),
                            *reinterpret_cast<const half4*>(src + 16));
        }
        f32x4 accA[4], accM[4];
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
            accA[mt] = zero4();
            accM[mt] = zero4();
            if (mt >= wave || mt <= wave) {
#pragma unroll
                for (int kb = 0; kb < 4; ++kb) {
                    const _Float16* src = &sm.Kr[(mt * 16 + lm) * kKrStride + kb * 32 + 4 * lg];
                    const half8 a = cat8(*reinterpret_cast<const half4*>(src),
                                         *reinterpret_cast<const half4*>(src + 16));
                    if (mt >= wave) accA[mt] = mfma16(a, kb_w[kb], accA[mt]);
                    if (mt <= wave) accM[mt] = mfma16(a, qf[kb], accM[mt]);
                }
            }
        }
        // A: element (r = 16mt + 4lg + i, col = 16w + lm)
        const int col = wave * 16 + lm;
        const float ccol = sm.c[col];
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int r = mt * 16 + 4 * lg + i;
                float a = 0.f;
                if (r > col) a = -sm.b[r] * accA[mt][i] * expf(sm.c[r] - ccol);
                sm.u.A[r * kMatStride + col] = a;
                if (ws.dbgA) ws.dbgA[ch * kChunk * kChunk + r * kChunk + col] = a;
            }
        }
        // M^T tile (mt, w): element (key c = 16mt + 4lg + i, query r = 16w + lm)
        const int rq = wave * 16 + lm;
        const float crq = sm.c[rq];
        half4 mh[4];
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
            f32x4 val;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int ck = mt * 16 + 4 * lg + i;
                val[i] = (ck <= rq) ? scale * accM[mt][i] * expf(crq - sm.c[ck]) : 0.f;
            }
            mh[mt] = to_half4(val);
        }
        // Mf fragment (row block w, k-block kbm) = tiles 2kbm, 2kbm+1
        half8* mdst = reinterpret_cast<half8*>(ws.Mf + ch * kMfElems);
        mdst[(wave * 2 + 0) * 64 + lane] = cat8(mh[0], mh[1]);
        mdst[(wave * 2 + 1) * 64 + lane] = cat8(mh[2], mh[3]);
        // Qf fragments: s e^{c_r} q_r, row block w
        const float es = sm.es[rq];
        half8* qdst = reinterpret_cast<half8*>(ws.Qf + ch * kQfElems);
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
            half8 o;
#pragma unroll
            for (int j = 0; j < 8; ++j) o[j] = (_Float16)((float)qf[kb][j] * es);
            qdst[(wave * 4 + kb) * 64 + lane] = o;
        }
    }
    __syncthreads();

    // ---- T = (I - A)^-1 in fp32: 16x16 diagonal blocks by forward
    // substitution (wave w owns block w, lanes 0..15 own its columns), then
    // the off-diagonal blocks level by level:
    //   T_ij = T_ii * sum_{k=j}^{i-1} A_ik T_kj
    if (lm == lane) {  // lanes 0..15 of every wave
        const int b0 = wave * 16;
        const int cidx = lm;
        float col[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) col[i] = (i == cidx) ? 1.f : 0.f;
#pragma unroll
        for (int i = 1; i < 16; ++i) {
            const float* arow = &sm.u.A[(b0 + i) * kMatStride + b0];
            float s = 0.f;
#pragma unroll
            for (int j = 0; j < i; ++j) s = fmaf(arow[j], col[j], s);
            if (i > cidx) col[i] = s;
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) sm.T[(b0 + i) * kMatStride + b0 + cidx] = col[i];
    }
    // zero the strictly upper blocks of T
    for (int e = tid; e < 6 * 256; e += kPrepThreads) {
        const int blk = e >> 8, w = e & 255;
        // upper block pairs (i < j): (0,1)(0,2)(0,3)(1,2)(1,3)(2,3)
        const int bi = (blk < 3) ? 0 : (blk < 5 ? 1 : 2);
        const int bj = (blk < 3) ? blk + 1 : (blk < 5 ? blk - 1 : 3);
        sm.T[(bi * 16 + (w >> 4)) * kMatStride + bj * 16 + (w & 15)] = 0.f;
    }
    __syncthreads();
    // levels d = 1..3: blocks (j + d, j) for j = 0 .. 3-d
#pragma unroll
    for (int d = 1; d <= 3; ++d) {
        const int nblk = 4 - d;
        // P_ij = sum_{k=j}^{i-1} A_ik T_kj  -> registers
        float pv[3];
#pragma unroll
        for (int it = 0; it < 3; ++it) {
            const int e = tid + it * kPrepThreads;
            pv[it] = 0.f;
            if (e < nblk * 256) {
                const int j = e >> 8, i = j + d;
                const int r = (e >> 4) & 15, cc = e & 15;
                float s = 0.f;
                for (int kk = j * 16; kk < i * 16; ++kk)
                    s = fmaf(sm.u.A[(i * 16 + r) * kMatStride + kk], sm.T[kk * kMatStride + j * 16 + cc], s);
                pv[it] = s;
            }
        }
        __syncthreads();
        // stash P in the (still zero) target block of T
#pragma unroll
        for (int it = 0; it < 3; ++it) {
            const int e = tid + it * kPrepThreads;
            if (e < nblk * 256) {
                const int j = e >> 8, i = j + d;
                const int r = (e >> 4) & 15, cc = e & 15;
                sm.T[(i * 16 + r) * kMatStride + j * 16 + cc] = pv[it];
            }
        }
        __syncthreads();
        // T_ij = T_ii P_ij
#pragma unroll
        for (int it = 0; it < 3; ++it) {
            const int e = tid + it * kPrepThreads;
            pv[it] = 0.f;
            if (e < nblk * 256) {
                const int j = e >> 8, i = j + d;
                const int r = (e >> 4) & 15, cc = e & 15;
                float s = 0.f;
#pragma unroll
                for (int kk = 0; kk < 16; ++kk)
                    s = fmaf(sm.T[(i * 16 + r) * kMatStride + i * 16 + kk],
                             sm.T[(i * 16 + kk) * kMatStride + j * 16 + cc], s);
                pv[it] = s;
            }
        }
        __syncthreads();
#pragma unroll
        for (int it = 0; it < 3; ++it) {
            const int e = tid + it * kPrepThreads;
            if (e < nblk * 256) {
                const int j = e >> 8, i = j + d;
                const int r = (e >> 4) & 15, cc = e & 15;
                sm.T[(i * 16 + r) * kMatStride + j * 16 + cc] = pv[it];
            }
        }
        __syncthreads();
    }
    if (ws.dbgT) {
        for (int e = tid; e < kChunk * kChunk; e += kPrepThreads)
            ws.dbgT[ch * kChunk * kChunk + e] = sm.T[(e >> 6) * kMatStride + (e & 63)];
    }
    // ---- V^T into LDS (A is dead now)
#pragma unroll
    for (int it = 0; it < 4; ++it) {
        const int e = tid + it * kPrepThreads;
        const int r = e >> 4, c8 = (e & 15) * 8;
        const half8 vh = bf16x8_to_half8(vraw[it]);
#pragma unroll
        for (int j = 0; j < 8; ++j) sm.u.Vt[(c8 + j) * kKtStride + r] = vh[j];
    }
    __syncthreads();

    // ---- U = (T diag(beta)) V : tiles (mt 0..3) x (nt = 2w, 2w+1)
    {
        half8 xa[4][2];  // A fragments of T diag(beta)
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                const int r = mt * 16 + lm;
                const int k0 = kb * 32 + 4 * lg;
                const f32x4 t0 = *reinterpret_cast<const f32x4*>(&sm.T[r * kMatStride + k0]);
                const f32x4 t1 = *reinterpret_cast<const f32x4*>(&sm.T[r * kMatStride + k0 + 16]);
                const f32x4 b0 = *reinterpret_cast<const f32x4*>(&sm.b[k0]);
                const f32x4 b1 = *reinterpret_cast<const f32x4*>(&sm.b[k0 + 16]);
                xa[mt][kb] = cat8(to_half4(t0 * b0), to_half4(t1 * b1));
            }
        }
        f32x4* udst = reinterpret_cast<f32x4*>(ws.Uf + ch * kUfElems);
#pragma unroll
        for (int p = 0; p < 2; ++p) {
            const int nt = wave * 2 + p;
            half8 vb[2];
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                const _Float16* src = &sm.u.Vt[(nt * 16 + lm) * kKtStride + kb * 32 + 4 * lg];
                vb[kb] = cat8(*reinterpret_cast<const half4*>(src),
                              *reinterpret_cast<const half4*>(src + 16));
            }
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) {
                f32x4 acc = zero4();
                acc = mfma16(xa[mt][0], vb[0], acc);
                acc = mfma16(xa[mt][1], vb[1], acc);
                udst[(nt * 4 + mt) * 64 + lane] = acc;  // slice nt, row tile mt
            }
        }
    }
    // ---- W^T = K^T (T diag(beta e^c))^T : tiles (dk mt = 2w, 2w+1) x (token nt 0..3)
    {
        half8 ka[2][2];
#pragma unroll
        for (int p = 0; p < 2; ++p) {
            const int mt = wave * 2 + p;
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                const _Float16* src = &sm.Kt[(mt * 16 + lm) * kKtStride + kb * 32 + 4 * lg];
                ka[p][kb] = cat8(*reinterpret_cast<const half4*>(src),
                                 *reinterpret_cast<const half4*>(src + 16));
            }
        }
        half8* wdst = reinterpret_cast<half8*>(ws.Wf + ch * kWfElems);
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) {
            half8 xb[2];
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                const int r = nt * 16 + lm;
                const int k0 = kb * 32 + 4 * lg;
                const f32x4 t0 = *reinterpret_cast<const f32x4*>(&sm.T[r * kMatStride + k0]);
                const f32x4 t1 = *reinterpret_cast<const f32x4*>(&sm.T[r * kMatStride + k0 + 16]);
                const f32x4 b0 = *reinterpret_cast<const f32x4*>(&sm.be[k0]);
                const f32x4 b1 = *reinterpret_cast<const f32x4*>(&sm.be[k0 + 16]);
                xb[kb] = cat8(to_half4(t0 * b0), to_half4(t1 * b1));
            }
            f32x4 acc0 = zero4(), acc1 = zero4();
            acc0 = mfma16(ka[0][0], xb[0], acc0);
            acc0 = mfma16(ka[0][1], xb[1], acc0);
            acc1 = mfma16(ka[1][0], xb[0], acc1);
            acc1 = mfma16(ka[1][1], xb[1], acc1);
            // W fragment (row tile nt, k-block w): regs 0..3 = dk tile 2w, 4..7 = 2w+1
            wdst[(nt * 4 + wave) * 64 + lane] = cat8(to_half4(acc0), to_half4(acc1));
        }
    }
    // ---- K~^T fragments: e^{c_63 - c_tau} k_tau[dk], dk tiles 2w, 2w+1
    {
        half8* kdst = reinterpret_cast<half8*>(ws.Kf + ch * kKfElems);
#pragma unroll
        for (int p = 0; p < 2; ++p) {
            const int mt = wave * 2 + p;
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                const int k0 = kb * 32 + 4 * lg;
                const _Float16* src = &sm.Kt[(mt * 16 + lm) * kKtStride + k0];
                const half4 lo = *reinterpret_cast<const half4*>(src);
                const half4 hi = *reinterpret_cast<const half4*>(src + 16);
                const f32x4 d0 = *reinterpret_cast<const f32x4*>(&sm.ed[k0]);
                const f32x4 d1 = *reinterpret_cast<const f32x4*>(&sm.ed[k0 + 16]);
                f32x4 l, h;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    l[j] = (float)lo[j] * d0[j];
                    h[j] = (float)hi[j] * d1[j];
                }
                kdst[(mt * 2 + kb) * 64 + lane] = cat8(to_half4(l), to_half4(h));
            }
        }
    }
}

// ---------------------------------------------------------------------------
// scan kernel: one work-group (2 waves) per (state slice, v-head, sequence)
// ---------------------------------------------------------------------------
struct ScanSmem {
    half8 ringS[2][4][64];   // S as B-operand fragments (4 k-blocks over dk)
    half8 ringV[2][2][64];   // V_new as B-operand fragments (2 k-blocks over tokens)
    int red[kScanThreads / 64];
};

struct ChainOps {
    half8 w[16];
    half8 k[16];
    f32x4 u[4];
    float d;
};

__device__ inline void load_chain(const Workspace& ws, size_t ch, int sl, int lane, ChainOps& op) {
    const half8* wsrc = reinterpret_cast<const half8*>(ws.Wf + ch * kWfElems);
    const half8* ksrc = reinterpret_cast<const half8*>(ws.Kf + ch * kKfElems);
    const f32x4* usrc = reinterpret_cast<const f32x4*>(ws.Uf + ch * kUfElems);
#pragma unroll
    for (int f = 0; f < 16; ++f) op.w[f] = wsrc[f * 64 + lane];
#pragma unroll
    for (int f = 0; f < 16; ++f) op.k[f] = ksrc[f * 64 + lane];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) op.u[mt] = usrc[(sl * 4 + mt) * 64 + lane];
    op.d = ws.decay[ch];
}

struct OutOps {
    half8 q[16];
    half8 m[8];
};

__device__ inline void load_out(const Workspace& ws, size_t ch, int lane, OutOps& op) {
    const half8* qsrc = reinterpret_cast<const half8*>(ws.Qf + ch * kQfElems);
    const half8* msrc = reinterpret_cast<const half8*>(ws.Mf + ch * kMfElems);
#pragma unroll
    for (int f = 0; f < 16; ++f) op.q[f] = qsrc[f * 64 + lane];
#pragma unroll
    for (int f = 0; f < 8; ++f) op.m[f] = msrc[f * 64 + lane];
}

__device__ inline void chain_step(const ChainOps& op, f32x4 (&S)[8], half8 (&sb)[4], half8 (&vb)[2]) {
    // P = W S  (64 x 16), k over dk
    f32x4 P[4];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
        P[mt] = zero4();
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) P[mt] = mfma16(op.w[mt * 4 + kb], sb[kb], P[mt]);
    }
    // V_new = U - P
    f32x4 vn[4];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) vn[mt] = op.u[mt] - P[mt];
    vb[0] = cat8(to_half4(vn[0]), to_half4(vn[1]));
    vb[1] = cat8(to_half4(vn[2]), to_half4(vn[3]));
    // S = d S + K~^T V_new   (128 x 16), k over tokens
#pragma unroll
    for (int t = 0; t < 8; ++t) {
        f32x4 acc = S[t] * op.d;
        acc = mfma16(op.k[t * 2 + 0], vb[0], acc);
        acc = mfma16(op.k[t * 2 + 1], vb[1], acc);
        S[t] = acc;
    }
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) sb[kb] = cat8(to_half4(S[2 * kb]), to_half4(S[2 * kb + 1]));
}

__global__ __launch_bounds__(kScanThreads, 1) void gdn_scan_kernel(
    Workspace ws, uint16_t* __restrict__ o, const float* __restrict__ s0,
    float* __restrict__ sf, const int32_t* __restrict__ cu, int N, int T, int HV) {
    __shared__ ScanSmem sm;
    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int lg = lane >> 4, lm = lane & 15;

    // XCD-aware id: the 8 slices of one (seq, head) pair share id % 8
    const int id = blockIdx.x;
    const int xcd = id & 7, qd = id >> 3;
    const int sl = qd & 7;
    const int pair = (qd >> 3) * 8 + xcd;
    if (pair >= N * HV) return;
    const int seq = pair / HV, hv = pair - seq * HV;

    const int len = seq_len(cu, T, seq);
    const int tok0 = seq_start(cu, T, seq);
    const int nch = (len + kChunk - 1) / kChunk;
    const int chunk0 = chunks_before<kScanThreads>(cu, T, seq, sm.red);
    const size_t sbase = ((size_t)seq * HV + hv) * kDK * kDV + sl * kBV + lm;

    if (wave == 0) {
        // ---- chain wave
        f32x4 S[8];
#pragma unroll
        for (int t = 0; t < 8; ++t) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
                S[t][i] = s0 ? s0[sbase + (size_t)(t * 16 + 4 * lg + i) * kDV] : 0.f;
        }
        half8 sb[4], vb[2];
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) sb[kb] = cat8(to_half4(S[2 * kb]), to_half4(S[2 * kb + 1]));
        ChainOps cur, nxt;
        if (nch > 0) load_chain(ws, (size_t)chunk0 * HV + hv, sl, lane, cur);
        for (int c = 0; c < nch; ++c) {
            if (c + 1 < nch) load_chain(ws, (size_t)(chunk0 + c + 1) * HV + hv, sl, lane, nxt);
            half8* rs = &sm.ringS[c & 1][0][0];
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) rs[kb * 64 + lane] = sb[kb];
            chain_step(cur, S, sb, vb);
            half8* rv = &sm.ringV[c & 1][0][0];
            rv[0 * 64 + lane] = vb[0];
            rv[1 * 64 + lane] = vb[1];
            __syncthreads();
            cur = nxt;
        }
#pragma unroll
        for (int t = 0; t < 8; ++t) {
#pragma unroll
            for (int i = 0; i < 4; ++i) sf[sbase + (size_t)(t * 16 + 4 * lg + i) * kDV] = S[t][i];
        }
    } else {
        // ---- output wave
        OutOps cur, nxt;
        if (nch > 0) load_out(ws, (size_t)chunk0 * HV + hv, lane, cur);
        for (int c = 0; c < nch; ++c) {
            if (c + 1 < nch) load_out(ws, (size_t)(chunk0 + c + 1) * HV + hv, lane, nxt);
            __syncthreads();
            half8 sb[4], vb[2];
            const half8* rs = &sm.ringS[c & 1][0][0];
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) sb[kb] = rs[kb * 64 + lane];
            const half8* rv = &sm.ringV[c & 1][0][0];
            vb[0] = rv[lane];
            vb[1] = rv[64 + lane];
            const int rows = min(kChunk, len - c * kChunk);
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) {
                f32x4 acc = zero4();
#pragma unroll
                for (int kb = 0; kb < 4; ++kb) acc = mfma16(cur.q[mt * 4 + kb], sb[kb], acc);
                acc = mfma16(cur.m[mt * 2 + 0], vb[0], acc);
                acc = mfma16(cur.m[mt * 2 + 1], vb[1], acc);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int r = mt * 16 + 4 * lg + i;
                    if (r < rows)
                        o[((size_t)(tok0 + c * kChunk + r) * HV + hv) * kDV + sl * kBV + lm] =
                            f32_to_bf16_bits(acc[i]);
                }
            }
            cur = nxt;
        }
    }
}

hipError_t launch_prefill(const void* q, const void* k, const void* v, const float* g,
                          const float* beta, void* o, const float* s0, float* sf,
                          const int32_t* cu, int N, int T, int total_tokens, int HV, int HK,
                          size_t nch_bound, void* workspace, size_t workspace_bytes,
                          hipStream_t stream, int dump_debug, hipEvent_t* ev = nullptr) {
    const WsLayout L(nch_bound * (size_t)HV);
    if (workspace_bytes < L.total) return hipErrorInvalidValue;
    char* base = static_cast<char*>(workspace);
    Workspace ws;
    ws.Wf = reinterpret_cast<_Float16*>(base + L.wf);
    ws.Kf = reinterpret_cast<_Float16*>(base + L.kf);
    ws.Qf = reinterpret_cast<_Float16*>(base + L.qf);
    ws.Mf = reinterpret_cast<_Float16*>(base + L.mf);
    ws.Uf = reinterpret_cast<float*>(base + L.uf);
    ws.decay = reinterpret_cast<float*>(base + L.decay);
    ws.dbgT = dump_debug ? reinterpret_cast<float*>(base + L.dbgT) : nullptr;
    ws.dbgA = dump_debug ? reinterpret_cast<float*>(base + L.dbgA) : nullptr;
    ws.dbgC = dump_debug ? reinterpret_cast<float*>(base + L.dbgC) : nullptr;
    const float scale = 1.0f / sqrtf((float)kDK);

    // ev (optional): kPrefillKernels + 1 events recorded around the launches
    if (ev) hipEventRecord(ev[0], stream);
    if (nch_bound > 0 && total_tokens > 0) {
        hipLaunchKernelGGL(gdn_prep_kernel, dim3((unsigned)nch_bound, HV), dim3(kPrepThreads), 0,
                           stream, static_cast<const uint16_t*>(q), static_cast<const uint16_t*>(k),
                           static_cast<const uint16_t*>(v), g, beta, cu, N, T, HV, HK, scale, ws);
        hipError_t err = hipGetLastError();
        if (err != hipSuccess) return err;
    }
    if (ev) hipEventRecord(ev[1], stream);
    const int pairs = N * HV;
    const int groups = (pairs + 7) / 8;
    hipLaunchKernelGGL(gdn_scan_kernel, dim3((unsigned)(groups * 64)), dim3(kScanThreads), 0, stream,
                       ws, static_cast<uint16_t*>(o), s0, sf, cu, N, T, HV);
    hipError_t err = hipGetLastError();
    if (ev) hipEventRecord(ev[2], stream);
    return err;
}

constexpr int kPrefillKernels = 2;
const char* const kPrefillKernelNames[kPrefillKernels] = {"gdn_prep_kernel", "gdn_scan_kernel"};

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
    return WsLayout(nc * HV).total;
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
    return launch_prefill(q, k, v, g, beta, o, initial_state, final_state, nullptr, B, T, B * T,
                          HV, HQK, nc, workspace, workspace_bytes, stream, dump_debug);
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
    return launch_prefill(q, k, v, g, beta, o, initial_state, final_state, nullptr, B, T, B * T,
                          HV, HQK, nc, workspace, workspace_bytes, stream, 0, events);
}

extern "C" size_t deltanet_prefill_varlen_workspace_size(int total_tokens, int num_seqs, int HV,
                                                         int DK, int DV, int chunk_size) {
    if (total_tokens < 0 || num_seqs <= 0 || HV <= 0 || DK != kDK || DV != kDV ||
        chunk_size != kChunk)
        return 0;
    // sum_i ceil(L_i / C) <= (sum_i L_i + (C-1) N) / C
    const size_t nc = ((size_t)total_tokens + (size_t)(kChunk - 1) * num_seqs) / kChunk;
    return WsLayout(nc * HV).total;
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
    return launch_prefill(q, k, v, g, beta, o, initial_state, final_state, cu_seqlens, num_seqs,
                          0, total_tokens, HV, HQK, nc, workspace, workspace_bytes, stream,
                          dump_debug);
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
