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
//   U   = T diag(beta) V,      W = T diag(beta e^c) K
//   V_n = U - W S
//   O   = diag(s e^c) Q S + M V_n
//   S  <- e^{c_63} S + K^T diag(e^{c_63 - c}) V_n
//
// (transformers modeling_qwen3_5.py:249-327, the reference's parity oracle;
// kernels/chunk_delta_cuda.cu:91-303, :312-424 and :532-674 compute the same
// terms.)
//
// Two kernels:
//   prep  one work-group per (chunk, v-head): gates, K K^T and Q K^T on fp16
//         MFMA, the inverse T in fp32 (16x16 diagonal blocks by forward
//         substitution, off-diagonal blocks on fp32 MFMA), then -W (fp16,
//         from W^T = K^T (T diag(beta e^c))^T on fp16 MFMA), T - I as an
//         fp16 hi / lo pair, M, a gates record, and Q as fp16 fragments.
//   scan  one work-group per (16 value columns, v-head, sequence), eight
//         specialised waves: a chain wave keeps the 128 x 16 state slice in
//         registers and per chunk forms V_n = U - W S (fp16 MFMA, U the
//         accumulator's fp32 initial value) and S <- e^{c63} S + K^T (d V_n)
//         (bf16 MFMA on the input K, d V_n as a bf16 hi / lo pair); a lo
//         helper wave adds the lo part into a second accumulator off the
//         serial path; a producer wave forms U = beta V + (T - I)(beta V)
//         from hi / lo fp16 products; two output waves form O; two loader
//         waves move K^T, -W, V and the gates into LDS rings with
//         direct-to-LDS loads; a norm wave serves the gated-RMSNorm epilogue.
//         Waves meet through LDS counters with bounded waits; a wait that runs
//         out aborts the work-group and sets the workspace's status word
//         (deltanet_prefill_status).  Once a call's 16-column groups would
//         outnumber the CUs, a paired instance gives each work-group 32
//         columns as two 16-column halves sharing the chunk operands
//         (gdn_scan2_kernel; bitwise the same results).
//
// Rounding budget (checked against an fp64 emulation of each operand class):
// W and S rounded to fp16 for V_n change the final state by < 1e-4 relative;
// U, and d V_n in the state update, are kept to ~16 bits or more, since a
// single fp16 rounding of either gives 1.4 - 2.7e-3.
//
// The fused entry (deltanet_chunk_prefill_fused) and the l2norm entry run the
// same kernels on raw inputs: the prep L2-normalises q and k rows as it loads
// them, converts fp16 inputs, forms g and beta from the gate inputs and
// writes the normalised k rows for the scan; the scan stores o in the I/O
// dtype and the final state over the initial one.
#include "gdn_common.h"
#include "gdn_hip.h"
#include "gdn_hip_diag.h"
#include "gdn_seq.h"

#include <math.h>

#include <algorithm>
#include <mutex>
#include <vector>

namespace gdn {
namespace {

constexpr int kPrepThreads = 256;
constexpr int kSliceCols = 16;                     // value columns per scan work-group
constexpr int kSlicesPerHead = kDV / kSliceCols;   // 8
constexpr int kTri = 6;                            // nonzero (row tile, k-block) fragments of a lower-triangular 64x64
constexpr unsigned kDefaultSpin = 1u << 20;        // bounded waits: ~0.1 s of polling, then give up

// First fragment index of row tile mt among the kTri lower-triangular ones:
// (0,0) (1,0) (2,0) (2,1) (3,0) (3,1)
__host__ __device__ constexpr int tri_base(int mt) { return mt < 3 ? mt : 4; }

// Per chunk-head workspace records (fp16 fragments, 16 bytes per lane):
//   TI, TIlo  (T - I) as hi / lo pair       kTri fragments each     6 KB each
//   M                                        kTri fragments          6 KB
//   W         -W, row tile mt, k-block kb   16 fragments            16 KB
//   gates     beta, d = e^{c63 - c}, s e^c, c63                      1 KB
//   Q         Q rows as fp16 fragments, per (chunk, k-head)          16 KB
//   KT        K^T as bf16 A-operand fragments of the state update, per
//             (chunk, k-head): tile t = dk block, k-block kb = tokens        16 KB
//   SSQ       gated-RMSNorm epilogue: per (slice, token) the slice's sum of
//             squares of o, fp32 bits with the sign bit clear once written
//             (the prep fills the slots with all-ones)                        2 KB
// A 256-byte header in front holds the status word.
constexpr size_t kFrag = 64 * 16;                      // one fragment: 1 KB
constexpr size_t kTriBytes = (size_t)kTri * kFrag;     // 6 KB
constexpr size_t kWBytes = 16 * kFrag;                 // 16 KB
constexpr size_t kGateBytes = 1024;
constexpr size_t kQBytes = 16 * kFrag;                 // 16 KB
constexpr size_t kKTBytes = 16 * kFrag;                // 16 KB
constexpr size_t kNormCntBytes = 16;   // one arrival counter per chunk-head (16-byte store)
constexpr size_t kHeaderBytes = 256;

// gates record: float offsets
constexpr int kGBeta = 0, kGDec = 64, kGSec = 128, kGC63 = 192;

struct Workspace {
    half8* TI;          // (T - I) hi fragments [chunk-head][kTri][64]
    half8* TIlo;        // (T - I) lo fragments, same layout
    half8* M;           // M fragments, same layout
    half8* W;           // -W fragments [chunk-head][mt * 4 + kb][64]
    float* gates;       // [chunk-head][256]
    half8* Q;           // Q fragments [chunk * HK + hk][mt * 4 + kb][64]
    u32x4* KT;          // K^T bf16 fragments [chunk * HK + hk][t * 2 + kb][64]
    uint32_t* ncnt;     // [chunk-head][4]: word 0 counts the slice groups whose o is written (norm epilogue only, else null)
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
    size_t ti, tilo, m, w, gates, q, kt, ncnt, dbgT, dbgA, dbgTp, dbgM, dbgC, dbgS, live, total;
    __host__ explicit WsLayout(size_t nch) {
        size_t off = kHeaderBytes;
        ti = off;    off += align256(nch * kTriBytes);
        tilo = off;  off += align256(nch * kTriBytes);
        m = off;     off += align256(nch * kTriBytes);
        w = off;     off += align256(nch * kWBytes);
        gates = off; off += align256(nch * kGateBytes);
        q = off;     off += align256(nch * kQBytes);
        kt = off;    off += align256(nch * kKTBytes);
        ncnt = off;  off += align256(nch * kNormCntBytes);
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
    const float* s0;   // the scan's initial state (the prep only touches it)
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

// Eight 16-bit elements of a 128-wide row (one 16-byte piece) as fp32, the
// row spread over `kLanes` lanes of consecutive lane ids xor-masks (16 lanes
// for one piece per lane, or lanes 16 apart for four pieces per lane).  For
// kRaw != 0 the row is L2-normalised, x rsqrt(sum x^2 + 1e-6) in fp32, and
// rounded to bf16 (the reference adapter's normalisation,
// gdnChunkPrefillSm87.cu:52-84; transformers l2norm, modeling_qwen3_5.py:
// 242-245).
template <int kRaw>
__device__ inline void unpack8(u32x4 w, float (&x)[8]) {
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        x[2 * p] = raw16<kRaw>(w[p] & 0xffffu);
        x[2 * p + 1] = raw16<kRaw>(w[p] >> 16);
    }
}

__device__ inline half8 f32x8_to_half8(const float (&x)[8]) {
    half8 h;
#pragma unroll
    for (int e = 0; e < 8; ++e) h[e] = (_Float16)x[e];
    return h;
}

__device__ inline u32x4 f32x8_to_bf16x8(const float (&x)[8]) {
    u32x4 w;
#pragma unroll
    for (int p = 0; p < 4; ++p)
        w[p] = (uint32_t)f32_to_bf16_bits(x[2 * p]) | ((uint32_t)f32_to_bf16_bits(x[2 * p + 1]) << 16);
    return w;
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

__device__ __forceinline__ half8 tr_pair_half8(s16x4 lo, s16x4 hi) {
    return cat8(__builtin_bit_cast(half4, lo), __builtin_bit_cast(half4, hi));
}

__device__ __forceinline__ bf16x8 tr_pair_bf16x8(s16x4 lo, s16x4 hi) {
    typedef short s16x8 __attribute__((ext_vector_type(8)));
    s16x8 r;
    r[0] = lo[0]; r[1] = lo[1]; r[2] = lo[2]; r[3] = lo[3];
    r[4] = hi[0]; r[5] = hi[1]; r[6] = hi[2]; r[7] = hi[3];
    return __builtin_bit_cast(bf16x8, r);
}

// Row pieces of a 64 x 128 16-bit tile in LDS: piece p (8 elements) of row r
// sits at slot 16 r + (p ^ sw(r)), sw(r) = the two 2-bit halves of r % 16
// swapped.  sw is a bijection on r % 16, so 16 consecutive rows' piece p and
// one row's 16 pieces each fill 16 distinct slots; and for 4 consecutive rows
// (r % 4 = 0..3) x 4 consecutive pieces (p % 4 = 0..3) -- a 16-lane group of
// the transposing reads below -- the high bits of p ^ sw(r) follow the row
// and the low bits the piece, so those 16 reads hit 16 distinct slots too:
// all three patterns are free of bank conflicts.
__device__ __forceinline__ int row_swz(int r) { return ((r & 3) << 2) | ((r >> 2) & 3); }
__device__ __forceinline__ int row_slot(int r, int p) { return 16 * r + (p ^ row_swz(r)); }

// Transposed operand of rows tile t (0..7) and token k-block kb (0..1) of a
// 64-token tile stored as above: lane (g, m) receives rows
// dk(t, m) = 32 (t / 2) + 8 (m / 4) + 4 (t % 2) + m % 4 for the 8 tokens
// 32 kb + kmap(g, j).  A product with this as its A operand yields D tiles
// whose lane (g, n), element i is dk 32 (t / 2) + 8 g + 4 (t % 2) + i: two
// tiles 2p, 2p+1 hold dk 32 p + 8 g + 0..7 in order.
__device__ __forceinline__ void kt_reads(const uint16_t* base, int t, int kb, int lane, s16x4& x0,
                                         s16x4& x1) {
    const int lg = lane >> 4, lm = lane & 15;
    const int p = 4 * (t >> 1) + (lm & 3);
    const int r0 = 32 * kb + 4 * lg + (lm >> 2), r1 = r0 + 16;
    x0 = lds_read_tr(base + row_slot(r0, p) * 8 + 4 * (t & 1));
    x1 = lds_read_tr(base + row_slot(r1, p) * 8 + 4 * (t & 1));
}

constexpr float kLog2e = 1.4426950408889634f;

// ---------------------------------------------------------------------------
// Block-cooperative sequence lookups (clamped cu_seqlens, gdn_seq.h).  Their
// host twins (deltanet_varlen_chunks_before / deltanet_varlen_locate_chunk)
// run the same phases thread by thread, for tests on the CPU.
// ---------------------------------------------------------------------------
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
// is past the last chunk.  `red` holds NT ints of scratch.  Sequences are
// taken NT at a time: an inclusive scan of their chunk counts, the one
// sequence whose range holds cid (at most one: the ranges are disjoint)
// posts itself, and seq_chunk_rows validates what was posted, so a result is
// in bounds even where no sequence posted (a saturated prefix).
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
    const int tid = (int)threadIdx.x;
    int base = 0;
    bool found = false;
    for (int s0 = 0; s0 < N && base < kSatChunks; s0 += NT) {
        const int s = s0 + tid;
        const int cnt = (s < N) ? seq_chunks(cu, T, total, s) : 0;
        __syncthreads();
        red[tid] = cnt;
        __syncthreads();
        for (int off = 1; off < NT; off <<= 1) {
            const int v = scan_step(red, tid, off);
            __syncthreads();
            red[tid] = v;
            __syncthreads();
        }
        const int incl = red[tid];
        const int blk = red[NT - 1];
        __syncthreads();
        if (tid == 0) {   // no sequence has posted yet
            red[0] = -1;
            red[1] = -1;
        }
        __syncthreads();
        if (owns_chunk(cnt, incl, base, cid)) {
            red[0] = s;
            red[1] = cid - base - (incl - cnt);
        }
        __syncthreads();
        const bool here = cid < sat_add(base, blk);
        if (here) {
            seq = red[0];
            found = seq_chunk_rows(cu, N, T, total, seq, red[1], tok0, rows);
        }
        __syncthreads();
        base = sat_add(base, blk);
        if (here) break;
    }
    return found;
}

// Store of a workspace record for the scan, at device scope (sc1): the line
// is written through this XCD's L2 while the prep runs.  A plain store leaves
// it dirty in L2, and the kernel's end must then write back every dirty line
// before the next kernel may start (the eight XCDs' L2s are not coherent with
// each other): after the prep's 30 MB of workspace that write-back held the
// scan back ~5 us, with these stores ~1.3 us.  Non-temporal stores (kNt)
// avoid the write-back too, but the lines then come back from HBM: slower
// while a call's records fit the 256 MB memory-side cache (T1141 HV32
// 37.2 -> 40.8 us; up to 233 MB of workspace 3-10 % slower), faster once
// they do not, when the scan reads them from HBM either way and the written
// lines only push older ones out (276 to 686 MB of workspace: 3.3-5.5 %
// faster); the launcher picks them above kNtWorkspaceBytes.  The prep never
// waits for these stores.  The scan's o and state
// stores stay plain: a wave's later loads complete only after its earlier
// stores, and waiting behind write-through stores slowed the output waves by
// more than the write-back they save.  A store of more than 8 bytes reads its data
// registers after issue: a VALU write to them needs two wait states first,
// which the compiler inserts after its own stores but cannot see inside an
// asm statement, so the 16-byte form carries its own s_nop.
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
constexpr size_t kNtWorkspaceBytes = size_t(256) << 20;
template <bool kNt = false, typename V>
__device__ __forceinline__ void st_through(V* p, const V& v) {
    static_assert(sizeof(V) == 4 || sizeof(V) == 8 || sizeof(V) == 16, "4, 8 or 16 bytes");
    if constexpr (sizeof(V) == 16) {
        if constexpr (kNt)
            asm volatile("global_store_dwordx4 %0, %1, off nt\n\ts_nop 1" ::"v"(p),
                         "v"(__builtin_bit_cast(u32x4, v))
                         : "memory");
        else
            asm volatile("global_store_dwordx4 %0, %1, off sc1\n\ts_nop 1" ::"v"(p),
                         "v"(__builtin_bit_cast(u32x4, v))
                         : "memory");
    } else if constexpr (sizeof(V) == 8) {
        if constexpr (kNt)
            asm volatile("global_store_dwordx2 %0, %1, off nt" ::"v"(p),
                         "v"(__builtin_bit_cast(u32x2, v))
                         : "memory");
        else
            asm volatile("global_store_dwordx2 %0, %1, off sc1" ::"v"(p),
                         "v"(__builtin_bit_cast(u32x2, v))
                         : "memory");
    } else {
        if constexpr (kNt)
            asm volatile("global_store_dword %0, %1, off nt" ::"v"(p),
                         "v"(__builtin_bit_cast(uint32_t, v))
                         : "memory");
        else
            asm volatile("global_store_dword %0, %1, off sc1" ::"v"(p),
                         "v"(__builtin_bit_cast(uint32_t, v))
                         : "memory");
    }
}

// x + (x moved by one DPP control), sources outside the row and rows outside
// the row mask contributing 0
template <int kCtrl, int kRowMask>
__device__ __forceinline__ float dpp_add(float x) {
    const int t = __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), kCtrl, kRowMask, 0xf,
                                              true);
    return x + __builtin_bit_cast(float, t);
}

// Inclusive prefix sum over the 64 lanes of a wave with DPP moves (no LDS
// round trip): row shifts by 1, 2, 4 and 8 within each row of 16 lanes, then
// lane 15 of rows 0 and 2 into rows 1 and 3 (row_bcast:15) and lane 31 into
// rows 2 and 3 (row_bcast:31).
__device__ inline float wave_prefix_sum(float x) {
    x = dpp_add<0x111, 0xf>(x);   // row_shr:1
    x = dpp_add<0x112, 0xf>(x);   // row_shr:2
    x = dpp_add<0x114, 0xf>(x);   // row_shr:4
    x = dpp_add<0x118, 0xf>(x);   // row_shr:8
    x = dpp_add<0x142, 0xa>(x);   // row_bcast:15
    x = dpp_add<0x143, 0xc>(x);   // row_bcast:31
    return x;
}

// ---------------------------------------------------------------------------
// prep kernel: one work-group (4 waves) per (chunk, v-head)
// ---------------------------------------------------------------------------
constexpr int kMS = kChunk + 4;   // fp32 A / T row pitch: 68 floats

struct PrepSmem {
    u32x4 K[kChunk * 16];   // fp16 K rows, row_slot layout
    // A (strictly lower, row-major) on entry.  The inverse overwrites it in
    // place: diagonal blocks T_ii row-major at (i, i); T_ij (i > j) stored
    // transposed at block (j, i), where A is zero and never read.  Its first
    // 1 KB is the sequence-lookup scratch before that.
    float AT[kChunk * kMS];
    float cl[kChunk];   // c * log2(e)
    float b[kChunk];    // beta
    float bec[kChunk];  // beta e^c
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

// K K^T and K Q^T products of wave W: A column block W (row tiles W..3) and
// M^T column block W (row tiles 0..W), k-blocks outermost so the five
// accumulators' products interleave.  Every operand holds 8 consecutive dk.
template <int W>
__device__ inline void am_products(const half8 (&ka)[4][4], const half8 (&qf)[4],
                                   f32x4 (&accA)[4], f32x4 (&accM)[4]) {
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
        accA[mt] = zero4();
        accM[mt] = zero4();
    }
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
        for (int mt = W; mt < 4; ++mt) accA[mt] = mfma16(ka[mt][kb], ka[W][kb], accA[mt]);
#pragma unroll
        for (int mt = 0; mt <= W; ++mt) accM[mt] = mfma16(ka[mt][kb], qf[kb], accM[mt]);
    }
}

template <bool kDbg, int kRaw, bool kNt = false>
__global__ __launch_bounds__(kPrepThreads, 4) void gdn_prep_kernel(
    PrepIn in, const int32_t* __restrict__ cu, int N, int T, int total, int HV, int HK,
    int nch_bound, float scale, Workspace ws) {
    __shared__ PrepSmem sm;
    // The kernel arguments (240 bytes) span four 64-byte lines, which the
    // scalar cache would otherwise fetch in three dependent round trips (each
    // use waits before the branch that leads to the next): fields at most 32
    // bytes apart, all requested together, cost one.
    asm volatile("" ::"s"(in.q), "s"(in.A_log), "s"(cu), "s"(nch_bound), "s"(ws.TIlo),
                 "s"(ws.gates), "s"(ws.ncnt), "s"(ws.dbgT), "s"(ws.dbgM), "s"(ws.dbgS));
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
    const int member = rest % rep;
    const int hv = hk * rep + member;

    int seq, tok0, rows;
    if (!locate_chunk<kPrepThreads>(cu, N, T, total, cid, reinterpret_cast<int*>(sm.AT), seq,
                                    tok0, rows))
        return;
    const size_t ch = (size_t)cid * HV + hv;
    // this call's gated-RMSNorm arrival counter of the chunk-head starts at
    // zero (only when the scan runs the norm epilogue)
    if (ws.ncnt && tid == 0)
        st_through(reinterpret_cast<u32x4*>(ws.ncnt + ch * (kNormCntBytes / 4)),
                   u32x4{0u, 0u, 0u, 0u});

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
    // K: thread tid holds piece tid % 16 of rows tid / 16 + 16 ii
    u32x4 raw[4];
    {
        const uint16_t* base = k + ((size_t)tok0 * HK + hk) * kDK + 8 * (tid & 15);
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) {
            const int r = min((tid >> 4) + 16 * ii, rows - 1);
            raw[ii] = *reinterpret_cast<const u32x4*>(base + (size_t)r * HK * kDK);
        }
    }
    // Q: wave w, lane (lg, lm) holds row 16 w + lm, dk 32 kb + 8 lg .. + 7
    u32x4 qr[4];
    {
        const uint16_t* qs =
            q + ((size_t)(tok0 + min(wave * 16 + lm, rows - 1)) * HK + hk) * kDK + 8 * lg;
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) qr[kb] = *reinterpret_cast<const u32x4*>(qs + kb * 32);
    }
    // The scan's first step waits on the initial state; read cold from HBM
    // that costs it ~2 us.  Each group here reads a 4 KB share of its
    // (sequence, v-head) state (chunk cs of the sequence: bytes [4 cs, 4 cs
    // + 4) KB, so 16 chunks cover the 64 KB), which leaves it in the
    // memory-side cache for the scan; the values are discarded.
    u32x4 ts0 = u32x4{0u, 0u, 0u, 0u};
    if (in.s0) {
        const int cs = (tok0 - seq_lo(cu, T, total, seq)) / kChunk;
        const size_t off = (size_t)cs * (kPrepThreads * 4) + 4 * tid;
        if (off < (size_t)kDK * kDV)
            ts0 = *reinterpret_cast<const u32x4*>(in.s0 + ((size_t)seq * HV + hv) * kDK * kDV + off);
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

    // ---- K rows -> fp16 into LDS (normalised first for raw inputs); rows
    // past the chunk's end are zeroed.
    const bool writer = member == 0;
#pragma unroll
    for (int ii = 0; ii < 4; ++ii) {
        const int r = (tid >> 4) + 16 * ii, p = tid & 15;
        float x[8];
        unpack8<kRaw>(raw[ii], x);
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
        u32x4 v = __builtin_bit_cast(u32x4, f32x8_to_half8(x));
        if (r >= rows) v = u32x4{0u, 0u, 0u, 0u};
        sm.K[row_slot(r, p)] = v;
    }
    // ---- Q row pieces -> fp16 (normalised first for raw inputs: a row's 128
    // values are spread over the 4 lanes lm, lm + 16, lm + 32, lm + 48)
    half8 qf[4];
    {
        float x[4][8];
        float ss = 0.f;
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
            unpack8<kRaw>(qr[kb], x[kb]);
#pragma unroll
            for (int e = 0; e < 8; ++e) ss = fmaf(x[kb][e], x[kb][e], ss);
        }
        if constexpr (kRaw != 0) {
            ss += __shfl_xor(ss, 16, 64);
            ss += __shfl_xor(ss, 32, 64);
            const float inv = rsqrtf(ss + 1e-6f);
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
                for (int e = 0; e < 8; ++e) x[kb][e] = (float)(__bf16)(x[kb][e] * inv);
            }
        }
        const bool ok = wave * 16 + lm < rows;
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
            qf[kb] = f32x8_to_half8(x[kb]);
            if (!ok) qf[kb] = half8{};
        }
        // Q fragments for the scan's output wave: fragment (mt = wave, kb)
        if (writer) {
            half8* qdst = ws.Q + ((size_t)cid * HK + hk) * 16 * 64;
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) st_through<kNt>(&qdst[(wave * 4 + kb) * 64 + lane], qf[kb]);
        }
    }

    // ---- gates (wave 0): c = cumsum(g); padded rows have g = beta = 0.  The
    // gates record holds beta, d = e^{c63 - c} (0 on padded rows), s e^c and
    // c63.
    if (wave == 0) {
        if (lane >= rows) {
            gv = 0.f;
            bv = 0.f;
        }
        const float cs = wave_prefix_sum(gv);
        const float c63 = __builtin_bit_cast(
            float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, cs), 63));
        const float clog = cs * kLog2e;
        const float ec = __builtin_amdgcn_exp2f(clog);
        sm.cl[lane] = clog;
        sm.b[lane] = bv;
        sm.bec[lane] = bv * ec;
        float* gr = ws.gates + ch * (kGateBytes / 4);
        st_through<kNt>(&gr[kGBeta + lane], bv);
        st_through<kNt>(&gr[kGDec + lane], lane < rows ? __builtin_amdgcn_exp2f((c63 - cs) * kLog2e) : 0.f);
        st_through<kNt>(&gr[kGSec + lane], scale * ec);
        st_through<kNt>(&gr[kGC63 + lane], lane == 0 ? c63 : 0.f);
        if (kDbg) ws.dbgC[ch * kChunk + lane] = cs;
    }
    asm volatile("" ::"v"(ts0));   // the share is read (and waited for) before the products
    __syncthreads();

    // ---- A = -beta_r (k_r . k_j) Gamma_rj (r > j) and M = s (q_r . k_j) Gamma_rj (r >= j)
    // Wave w owns column block j in [16w, 16w+16) of A and query-row block
    // r in [16w, 16w+16) of M (computed as M^T = K Q^T, whose accumulators are
    // already the M fragments the scan reads).
    {
        half8 ka[4][4];
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
            const int r = mt * 16 + lm;
#pragma unroll
            for (int kb = 0; kb < 4; ++kb)
                ka[mt][kb] = __builtin_bit_cast(half8, sm.K[row_slot(r, 4 * kb + lg)]);
        }
        f32x4 accA[4], accM[4];
        switch (wave) {
            case 0: am_products<0>(ka, qf, accA, accM); break;
            case 1: am_products<1>(ka, qf, accA, accM); break;
            case 2: am_products<2>(ka, qf, accA, accM); break;
            default: am_products<3>(ka, qf, accA, accM); break;
        }
        // Element (r = 16mt + 4lg + i, col = 16w + lm) of A (r > col) and
        // of M^T (key r <= col: M fragment (w, kb) = key tiles 2kb, 2kb+1):
        // exactly one of the two is nonzero, so one exponential serves both,
        // e^{c_r - c_col} for A, e^{c_col - c_r} for M; the upper part of A's
        // column block w and the lower part of M's are written as zero
        const int col = wave * 16 + lm;
        const float ccol = sm.cl[col];
        f32x4 clr[4], br[4];
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
            clr[mt] = *reinterpret_cast<const f32x4*>(&sm.cl[mt * 16 + 4 * lg]);
            br[mt] = *reinterpret_cast<const f32x4*>(&sm.b[mt * 16 + 4 * lg]);
        }
        half4 mh[4];
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
            f32x4 val;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int r = mt * 16 + 4 * lg + i;
                const bool lower = r > col;
                const float e = __builtin_amdgcn_exp2f(lower ? clr[mt][i] - ccol : ccol - clr[mt][i]);
                // both products, then selects: no branch per element
                float av = -br[mt][i] * accA[mt][i] * e, mv = scale * accM[mt][i] * e;
                asm volatile("" : "+v"(av), "+v"(mv));
                const float a = lower ? av : 0.f;
                sm.AT[r * kMS + col] = a;
                if (kDbg) ws.dbgA[ch * kChunk * kChunk + r * kChunk + col] = a;
                val[i] = lower ? 0.f : mv;
                if (kDbg) ws.dbgM[ch * kChunk * kChunk + col * kChunk + r] = val[i];
            }
            mh[mt] = to_half4(val);
        }
        half8* mdst = ws.M + ch * (kTri * 64);
        st_through<kNt>(&mdst[tri_base(wave) * 64 + lane], cat8(mh[0], mh[1]));
        if (wave >= 2) st_through<kNt>(&mdst[(tri_base(wave) + 1) * 64 + lane], cat8(mh[2], mh[3]));
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

    // ---- (T - I) fragments as an fp16 hi / lo pair: wave w writes row tile
    // mt = w, k-blocks kb <= mt / 2; lane (lg, lm) holds T[16mt + lm][32kb +
    // kmap(lg, j)]
    {
        const int mt = wave;
        const int r = mt * 16 + lm;
        half8* tdst = ws.TI + ch * (kTri * 64);
        half8* ldst = ws.TIlo + ch * (kTri * 64);
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
            half8 hi, lo;
            split_hilo8(t0, t1, hi, lo);
            st_through<kNt>(&tdst[(tri_base(mt) + kb) * 64 + lane], hi);
            st_through<kNt>(&ldst[(tri_base(mt) + kb) * 64 + lane], lo);
        }
    }

    // ---- -W = -T diag(beta e^c) K as W^T = K^T (T diag(beta e^c))^T: wave w
    // forms dk tiles t = 2w, 2w+1 (dk 32 w .. 32 w + 31) for every token tile
    // mt.  The A operand is K^T from the transposing reads; the B operand of
    // (k-block kb, token tile mt) holds T[16 mt + n][32 kb + kmap(g, j)]
    // beta_j e^{c_j}, rounded once to fp16.  Lane (g, n) then holds -W[16 mt
    // + n][32 w + 8 g + 0..7]: fragment (mt, kb = w) of the scan's A operand.
    {
        const uint16_t* kbase = reinterpret_cast<const uint16_t*>(sm.K);
        half8 kt[2][2];
        u32x4* ktdst = ws.KT + ((size_t)cid * HK + hk) * (16 * 64);
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                s16x4 x0, x1;
                kt_reads(kbase, 2 * wave + tt, kb, lane, x0, x1);
                kt[tt][kb] = tr_pair_half8(x0, x1);
                // the scan's K^T operand of tile 2 w + tt, k-block kb (bf16:
                // the fp16 values convert back exactly, they were bf16)
                if (writer) {
                    bf16x8 kb16;
#pragma unroll
                    for (int e = 0; e < 8; ++e) kb16[e] = (__bf16)(float)kt[tt][kb][e];
                    st_through<kNt>(&ktdst[((2 * wave + tt) * 2 + kb) * 64 + lane],
                               __builtin_bit_cast(u32x4, kb16));
                }
            }
        }
        f32x4 bec[2][2];   // beta e^c at columns 32 kb + 4 g (+16) .. + 3
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
            for (int hh = 0; hh < 2; ++hh)
                bec[kb][hh] = *reinterpret_cast<const f32x4*>(&sm.bec[32 * kb + 16 * hh + 4 * lg]);
        }
        half8* wdst = ws.W + ch * (16 * 64);
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
            const int r = 16 * mt + lm;
            f32x4 acc0 = zero4(), acc1 = zero4();
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                if (kb > mt / 2) break;
                f32x4 t0 = t_row4(sm.AT, mt, 2 * kb, r, 32 * kb + 4 * lg);
                f32x4 t1 = t_row4(sm.AT, mt, 2 * kb + 1, r, 32 * kb + 16 + 4 * lg);
                const half8 bt = cat8(to_half4(t0 * bec[kb][0]), to_half4(t1 * bec[kb][1]));
                acc0 = mfma16(kt[0][kb], bt, acc0);
                acc1 = mfma16(kt[1][kb], bt, acc1);
            }
            st_through<kNt>(&wdst[(mt * 4 + wave) * 64 + lane], cat8(to_half4(-acc0), to_half4(-acc1)));
        }
    }
}

// ---------------------------------------------------------------------------
// scan kernel: one work-group (8 waves) per (16 value columns, v-head,
// sequence).
//
// State layout of the chain: accumulator tile t (0..7), lane (g, n), element
// i holds S[dk][16 sl + n] with dk = 32 (t/2) + 8 g + 4 (t%2) + i, so the
// fp16 B operand of k-block kb (tiles 2kb, 2kb+1) holds dk 32 kb + 8 g + 0..7
// in order, matching the -W row-piece fragments, and the K^T operand that
// produces tile t is the prep's K^T fragment pair (t * 2 + kb) of the chunk.
//
//   chain     wave 0: V_n = U + (-W) S16 (16 fp16 MFMA), d V_n -> bf16 hi,
//             S' = e^{c63} S + K^T hi (16 bf16 MFMA), d V_n handed to the lo
//             helper (the debug build does the helper's products here).
//   producer  wave 1: U = beta V + (T - I)(beta V) with the product as
//             hi/hi + hi/lo + lo/hi fp16 MFMAs (18), into ring P.
//   output    waves 2 and 3, chunks of even and odd index:
//             O^T = (S^T Q^T) diag(s e^c) + V_n^T M^T, with Q, M and s e^c
//             loaded to registers as soon as the wave's previous chunk has
//             read them, two chain steps before they are needed.
//   norm      wave 4: the gated-RMSNorm epilogue's row sums across the 8
//             slice groups (norm epilogue only; otherwise it exits at once).
//   lo helper wave 7: Sc <- e^{c63} Sc + K^T lo, the lo part of the state
//             update, off the chain's serial path.
//   loaders   waves 6 and 5, chunks of even and odd index: direct-to-LDS
//             loads of chunk c's K^T fragments and -W into ring C (3 stages, 32 KB
//             each) and of chunk c + 1's V and gates record into ring P (4
//             stages, 7 KB each).  Each loader has one chunk in flight and
//             publishes it as soon as it lands, so the two keep two chunks in
//             flight without one's wait for a free stage holding back the
//             other's publication.
// ---------------------------------------------------------------------------
constexpr int kRingC = 3;     // chain operand stages (K rows, -W)
constexpr int kRingP = 4;     // producer stages (V, gates, U)
constexpr int kLeadP = 1;     // ring P is filled this many chunks ahead of ring C
constexpr int kHand = 4;      // chain -> output hand-off slots
constexpr int kLoSlots = 2;   // chain -> lo-helper hand-off slots
constexpr int kScanWaves = 8;
constexpr int kScanThreads = 64 * kScanWaves;
static_assert(kRingP >= kRingC + kLeadP, "ring P must hold the chunks ring C and the lead span");
static_assert(kHand % 2 == 0, "a hand-off slot is reused by a chunk of the same parity");

struct StageC {
    u32x4 KT[16][64];       // K^T bf16 fragments (t * 2 + kb)
    half8 W[16][64];        // -W fragments (mt * 4 + kb)
};

struct StageP {
    u32x4 V[kChunk * 2];    // V rows of the slice's 16 columns, 2 pieces per row
    float gates[256];       // gates record
    f32x4 U[4][64];         // U, D layout per row tile (producer)
};

struct Hand {
    half8 S[4][64];         // S at the chunk's start, fp16 B fragments
    half8 V[2][64];         // V_n, fp16 B fragments
};

struct LoHand {
    f32x4 d[4][64];         // d o V_n (fp32, D layout per row tile)
    float gam;              // e^{c63} of the chunk
    float pad_[63];
};

struct ScanSmem {
    StageC c[kRingC];
    StageP p[kRingP];
    Hand h[kHand];
    LoHand lo[kLoSlots];   // after the last chunk: the helper's Sc (8 KB)
    int fill[2];     // per loader: chunks of its parity whose ring-C loads have landed
    int pfill[2];    // per loader: chunks c of its parity whose next chunk's ring-P loads
                     // (V, gates of c + 1) have landed
    int uready;      // chunks whose U is in ring P (producer)
    int freeC;       // chunks whose ring-C and ring-P stages the chain has finished reading
    int kfree;       // chunks whose ring-C K^T the lo helper has finished reading
    int ready;       // chunks whose hand-off slot the chain has written
    int cons[2];     // per output wave: chunks of its parity whose hand-off slot it has read
    int dvready;     // chunks whose d o V_n the chain has handed to the helper
    int lodone;      // chunks whose lo slot the helper has read
    int scdone;      // the helper's Sc is in the lo slots
    int abort;       // a bounded wait ran out: every wave stops
    int seqsel;
    int red[kScanWaves];
    // norm epilogue, per output wave: chunks of its parity whose o is written
    // (stores complete at the device-coherent level)
    int npub[2];
};

__device__ __forceinline__ int lds_ld(const int* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ void lds_st(int* p, int v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// LDS store of a counter, invisible to the compiler's wait placement: use
// only where an explicit s_waitcnt has already ordered what it publishes, or
// where what it publishes are this wave's earlier LDS writes (a wave's LDS
// operations are performed in issue order) and reads whose values this wave
// has already consumed.
__device__ __forceinline__ void lds_st_asm(int* p, int v) {
    const uint32_t addr = (uint32_t)(size_t)(__attribute__((address_space(3))) int*)p;
    asm volatile("ds_write_b32 %0, %1" ::"v"(addr), "v"(v) : "memory");
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
    uint16_t* o;              // o, or y = gated_rmsnorm(o, z) for the norm epilogue
    const uint16_t* z;        // norm epilogue: gate input z, [token][HV][128] bf16
    const uint16_t* nw;       // norm epilogue: weight [128] bf16
    float eps;
    const float* s0;
    float* sf;
    const int32_t* cu;
    int N, T, total, HV, HK, nch_bound;
    unsigned spin;
};

struct ScanCtx {
    int seq, hv, hk, sl, tok_base, len, chunk0, nch;
};

__device__ __forceinline__ void lds_dma16(const void* g, void* lds) {
    __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void*)lds, 16, 0, 0);
}

// s_waitcnt immediates: vmcnt(n) with expcnt and lgkmcnt left at their
// maxima; vmcnt's 6 bits are split over bits 3:0 and 15:14
constexpr unsigned vmcnt_imm(unsigned n) { return 0x0F70u | (n & 15u) | ((n >> 4) << 14); }
static_assert(vmcnt_imm(16) == 0x4F70 && vmcnt_imm(0) == 0x0F70, "s_waitcnt encoding");

constexpr int kPLoads = 3;   // direct-to-LDS loads of one ring-P stage (V: 2, gates: 1)

// Loader j (0 or 1) takes the chunks c of parity j: it issues one group of
// direct-to-LDS loads, ring C for chunk c (K^T: 16, -W: 16) and then ring P
// for chunk c + kLeadP (V: 2, gates: 1), and publishes each part as it lands
// (loads complete in order, so ring C is in while ring P's three may still be
// in flight): V comes from the caller's input, possibly from HBM, and the
// chain's next step needs only ring C.  Past the sequence's end the ring-P
// index is clamped, so every group holds the same number of loads.  Loader 0
// also loads ring P's lead chunk first, in with its first ring-C stage.
__device__ void run_loader(ScanSmem& sm, const ScanArgs& a, const Waiter& w, const ScanCtx& x,
                           int j, int lane) {
    auto rows_of = [&](int c) { return min(kChunk, x.len - c * kChunk); };
    auto ch_of = [&](int c) { return (size_t)(x.chunk0 + c) * a.HV + x.hv; };
    auto issue_p = [&](int cp) {
        const int c = min(cp, x.nch - 1);
        StageP& st = sm.p[cp % kRingP];
        const int t0 = x.tok_base + c * kChunk, rows = rows_of(c);
        // V: slot 64 i + lane -> row (64 i + lane) / 2, piece lane % 2
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int s = 64 * i + lane, r = min(s >> 1, rows - 1);
            lds_dma16(a.in.v + ((size_t)(t0 + r) * a.HV + x.hv) * kDV + kSliceCols * x.sl + 8 * (s & 1),
                      &st.V[64 * i]);
        }
        lds_dma16(a.ws.gates + ch_of(c) * (kGateBytes / 4) + 4 * lane, &st.gates[0]);
    };
    auto issue_c = [&](int c) {
        StageC& st = sm.c[c % kRingC];
        const u32x4* ksrc = a.ws.KT + ((size_t)(x.chunk0 + c) * a.HK + x.hk) * (16 * 64) + lane;
#pragma unroll
        for (int f = 0; f < 16; ++f) lds_dma16(ksrc + f * 64, &st.KT[f][0]);
        const half8* wsrc = a.ws.W + ch_of(c) * (16 * 64) + lane;
#pragma unroll
        for (int f = 0; f < 16; ++f) lds_dma16(wsrc + f * 64, &st.W[f][0]);
    };
    // an empty sequence has no chunk to load (issue_p would form chunk -1)
    if (x.nch <= 0) return;
    if (j == 0) {
        for (int c = 0; c < kLeadP; ++c) issue_p(c);
    } else if (!w.until([&] { return lds_ld(&sm.fill[0]) >= 1; })) {
        // chunk 1 goes out once chunk 0 is in (see run_producer)
        return;
    }
    for (int c = j; c < x.nch; c += 2) {
        // ring-C stage c % kRingC held chunk c - kRingC (read by the chain
        // and the lo helper); ring-P stage (c + kLeadP) % kRingP held chunk
        // c + kLeadP - kRingP <= c - kRingC
        if (!w.until([&] {
                const bool fc = lds_ld(&sm.freeC) >= c - kRingC + 1;
                const bool fk = lds_ld(&sm.kfree) >= c - kRingC + 1;
                return fc & fk;
            }))
            break;
        asm volatile("" ::: "memory");
        issue_c(c);
        asm volatile("" ::: "memory");   // ring P's loads are issued after ring C's
        issue_p(c + kLeadP);
        static_assert(kPLoads == 3, "ring P's loads may stay in flight");
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(kPLoads));   // ring C's 32 loads (and older) are in
        // The store goes through asm: the compiler places a wait for every
        // direct-to-LDS load before any LDS access it cannot tell apart from
        // their destinations, which would hold it back for ring P's loads too.
        if (lane == 0) lds_st_asm(&sm.fill[j], (c >> 1) + 1);
        vm_wait_all();
        if (lane == 0) lds_st(&sm.pfill[j], (c >> 1) + 1);
    }
    vm_wait_all();   // no load may land in LDS after the group ends
}

template <int kRaw>
__device__ inline float v16_to_f32(uint32_t bits) {
    // fp16 V is rounded to bf16 first (the adapter's conversion)
    if constexpr (kRaw == 2) return (float)(__bf16)raw16<2>(bits);
    return __uint_as_float(bits << 16);
}

// Producer: U = beta V + (T - I)(beta V) per chunk into ring P.  With X =
// beta V (fp32, D layout), the product is (T-I)_hi X_hi + (T-I)_hi X_lo +
// (T-I)_lo X_hi on fp16 MFMA, accumulated onto X.  The (T - I) fragments come
// straight from global memory three chunks ahead, in three register sets
// used in turn (a set is refilled right after its chunk's products have read
// it, so no copy ever waits for a load in flight).

template <int kRaw>
__device__ void run_producer(ScanSmem& sm, const ScanArgs& a, const Waiter& w, const ScanCtx& x,
                             int lane) {
    const int lg = lane >> 4, lm = lane & 15;
    auto load_t = [&](int c, half8 (&h)[kTri], half8 (&l)[kTri]) {
        const int cc = min(c, x.nch - 1);
        const size_t ch = (size_t)(x.chunk0 + cc) * a.HV + x.hv;
        const half8* ph = a.ws.TI + ch * (kTri * 64) + lane;
        const half8* pl = a.ws.TIlo + ch * (kTri * 64) + lane;
#pragma unroll
        for (int f = 0; f < kTri; ++f) {
            h[f] = ph[f * 64];
            l[f] = pl[f * 64];
        }
    };
    auto step = [&](int c, half8 (&th)[kTri], half8 (&tl)[kTri], bool refill = true) -> bool {
        // ring P of chunk c landed with loader group c - kLeadP (pfill); chunk
        // 0's, issued before loader 0's first ring-C stage, with that (fill)
        const int lc = c - kLeadP;
        if (!w.until([&] {
                return lc < 0 ? lds_ld(&sm.fill[0]) >= 1
                              : lds_ld(&sm.pfill[lc & 1]) >= (lc >> 1) + 1;
            }))
            return false;
        asm volatile("" ::: "memory");
        StageP& st = sm.p[c % kRingP];
        // X = beta V: lane (g, n) of tile mt holds tokens 16 mt + 4 g + i of
        // column n (transposing read: source lane (a4 = lm / 4, b4 = lm % 4)
        // names row 16 mt + 4 lg + a4, columns 4 b4 .. + 3)
        f32x4 X[4];
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
            const f32x4 be = *reinterpret_cast<const f32x4*>(&st.gates[kGBeta + 16 * mt + 4 * lg]);
            const uint16_t* vsrc = reinterpret_cast<const uint16_t*>(st.V) +
                                   (16 * mt + 4 * lg + (lm >> 2)) * kSliceCols + 4 * (lm & 3);
            const s16x4 vt = lds_read_tr(vsrc);
#pragma unroll
            for (int i = 0; i < 4; ++i) X[mt][i] = be[i] * v16_to_f32<kRaw>((uint16_t)vt[i]);
        }
        half8 xh[2], xl[2];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) split_hilo8(X[2 * kb], X[2 * kb + 1], xh[kb], xl[kb]);
        f32x4 U[4];
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
            U[mt] = X[mt];
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                if (kb > mt / 2) break;
                const int f = tri_base(mt) + kb;
                U[mt] = mfma16(th[f], xh[kb], U[mt]);
                U[mt] = mfma16(th[f], xl[kb], U[mt]);
                U[mt] = mfma16(tl[f], xh[kb], U[mt]);
            }
        }
        // the products have read this set: chunk c + 3's fragments go in
        if (refill) load_t(c + 3, th, tl);
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) st.U[mt][lane] = U[mt];
        // published behind the U writes (LDS operations are performed in
        // issue order)
        asm volatile("" ::: "memory");
        if (lane == 0) lds_st_asm(&sm.uready, c + 1);
        return true;
    };
    if (x.nch <= 0) return;
    half8 t0h[kTri], t0l[kTri], t1h[kTri], t1l[kTri], t2h[kTri], t2l[kTri];
    load_t(0, t0h, t0l);
    load_t(1, t1h, t1l);
    // Start-up order: every group asks for its first records at once, so
    // what the first chain steps need (ring C and P of chunk 0, T - I of
    // chunks 0 and 1, the initial state) goes out first; loader 1's chunk 1
    // and the output waves' Q and M wait until chunk 0 has landed (-0.3 us
    // on the cold T=1141 HV=32 call).
    if (!w.until([&] { return lds_ld(&sm.fill[0]) >= 1; })) return;
    asm volatile("" ::: "memory");
    // U(0) is formed here, before any later T - I set goes out. Inside the
    // loop below, the wait the compiler places in front of a step's products
    // also covers loads issued after that step's own set. A U(0) formed
    // there would wait for sets issued after chunk 0 landed (cold T=1141
    // HV=32 call -0.14 to -0.30 us, bitwise unchanged).
    // step() is false only when a bounded wait gave up
    if (!step(0, t0h, t0l, false)) return;
    load_t(2, t2h, t2l);
    load_t(3, t0h, t0l);
    for (int c = 1; c < x.nch; c += 3) {
        if (!step(c, t1h, t1l)) return;
        if (c + 1 < x.nch && !step(c + 1, t2h, t2l)) return;
        if (c + 2 < x.nch && !step(c + 2, t0h, t0l)) return;
    }
}

// Two floats as a packed bf16 pair (round to nearest even), one
// v_cvt_pk_bf16_f32
__device__ inline uint32_t pack_bf16x2(float lo, float hi) {
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    const f32x2 v = {lo, hi};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}

// Hand-off slot c % kHand is free once the chunk that used it before,
// c - kHand (same parity), has been read by its output wave.  Loads without
// a branch, so it can share one LDS round trip with other counter loads.
__device__ inline bool slot_free(const ScanSmem& sm, int c) {
    const int need = c >= kHand ? ((c - kHand) >> 1) + 1 : 0;
    return lds_ld(&sm.cons[c & 1]) >= need;
}

template <bool kDbg>
__device__ void run_chain(ScanSmem& sm, const ScanArgs& a, const Waiter& w, const ScanCtx& x,
                          int lane) {
    const int lg = lane >> 4, lm = lane & 15;
    const int col = kSliceCols * x.sl + lm;
    auto dk_of = [&](int t, int i) { return 32 * (t >> 1) + 8 * lg + 4 * (t & 1) + i; };
    const size_t sbase = ((size_t)x.seq * a.HV + x.hv) * kDK * kDV + col;

    // S: the state's bf16-hi accumulation; Sc: the lo part, decayed every
    // chunk, so S + Sc is the state at each chunk's start
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
    for (int c = 0; c < x.nch; ++c) {
        const int hs = c % kHand;
        StageC& sc = sm.c[c % kRingC];
        StageP& sp = sm.p[c % kRingP];
        auto ready = [&] {   // every counter loaded, no short-circuit: one round trip
            const bool f = lds_ld(&sm.fill[c & 1]) >= (c >> 1) + 1;
            const bool u = lds_ld(&sm.uready) >= c + 1;
            const bool h = slot_free(sm, c);
            const bool l = kDbg || lds_ld(&sm.lodone) >= c - kLoSlots + 1;
            return f & u & h & l;
        };
        // (1) reads for V_n: U (accumulator init), -W, the gates.  They go
        // out together with the counter reads, before the counters are
        // known: a wave's LDS operations complete in order, so when the
        // counters say the chunk is there, these reads saw it; otherwise
        // the wave waits and reads again.  The usual case costs one LDS
        // round trip instead of two.
        f32x4 Vn[4], dec[4];
        half8 wf[16];
        float c63;
        auto read_operands = [&] {
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) Vn[mt] = sp.U[mt][lane];
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
                for (int mt = 0; mt < 4; ++mt) wf[mt * 4 + kb] = sc.W[mt * 4 + kb][lane];
            }
            c63 = sp.gates[kGC63];
#pragma unroll
            for (int mt = 0; mt < 4; ++mt)
                dec[mt] = *reinterpret_cast<const f32x4*>(&sp.gates[kGDec + 16 * mt + 4 * lg]);
        };
        const bool early = ready();
        asm volatile("" ::: "memory");
        read_operands();
        if (!early) {
            ok = w.until(ready);
            if (!ok) break;
            asm volatile("" ::: "memory");
            read_operands();
        }
        asm volatile("" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);   // the reads stay ahead of the products
        if (kDbg) {
            float* dst = a.ws.dbgS + ((size_t)(x.chunk0 + c) * a.HV + x.hv) * kDK * kDV + col;
#pragma unroll
            for (int t = 0; t < 8; ++t) {
#pragma unroll
                for (int i = 0; i < 4; ++i) dst[(size_t)dk_of(t, i) * kDV] = S[t][i] + Sc[t][i];
            }
        }
        // (2) V_n = U + (-W) S16: row tile mt (tokens), k-block kb (dk)
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) Vn[mt] = mfma16(wf[mt * 4 + kb], S16[kb], Vn[mt]);
        }
        // (3) K^T operands of the state update (16 fragment reads)
        bf16x8 kt[8][2];
#pragma unroll
        for (int t = 0; t < 8; ++t) {
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) kt[t][kb] = __builtin_bit_cast(bf16x8, sc.KT[t * 2 + kb][lane]);
        }
        // (4) decay of the state while the V_n products run; S at the
        // chunk's start goes to the hand-off slot
        const float gam = __builtin_amdgcn_exp2f(c63 * kLog2e);
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) sm.h[hs].S[kb][lane] = S16[kb];
#pragma unroll
        for (int t = 0; t < 8; ++t) S[t] = S[t] * gam;
        // A wave issues in order: each product is followed by independent
        // VALU work and reads, so they run while the product is in the
        // matrix pipe instead of after all products.
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
            __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);   // VALU
            __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);   // LDS read
        }
        asm volatile("" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
        // (5) d o V_n, hi part (bf16): B operand of token k-block kb (tiles
        // 2kb, 2kb+1)
        f32x4 dv[4];
        u32x4 hw[2];
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
            dv[mt] = dec[mt] * Vn[mt];
            // rounded here, as the helper sees it: no later use may fuse
            // the product into an FMA
            asm volatile("" : "+v"(dv[mt]));
        }
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
#pragma unroll
                for (int p = 0; p < 2; ++p)
                    hw[kb][2 * h + p] = pack_bf16x2(dv[2 * kb + h][2 * p], dv[2 * kb + h][2 * p + 1]);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        // (6) d o V_n and the decay to the lo helper (SIMD 3), which adds K^T
        // lo to its decayed Sc off the serial path; published with the
        // chunk's other counters.  The debug build does that work here.
        if constexpr (!kDbg) {
            LoHand& lh = sm.lo[c % kLoSlots];
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) lh.d[mt][lane] = dv[mt];
            if (lane == 0) lh.gam = gam;
        }
        // (7) S' = e^{c63} S + K^T hi.  Issue order is fixed piece by piece
        // (the wave issues in order): the S16 and V_n conversions (and, in
        // the debug build, the lo residuals) are spread between the products.
        u32x4 lw[2];
        auto lo_pair = [&](int kb, int q) {   // q = 2 h + p: one packed pair
            const int h = q >> 1, p = q & 1;
            const f32x4& d = dv[2 * kb + h];
            const uint32_t hp = hw[kb][q];
            const float r0 = d[2 * p] - __uint_as_float(hp << 16);
            const float r1 = d[2 * p + 1] - __uint_as_float(hp & 0xffff0000u);
            lw[kb][q] = pack_bf16x2(r0, r1);
        };
        half8 vh[2];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            const bf16x8 hi = __builtin_bit_cast(bf16x8, hw[kb]);
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                S[t] = mfma16_bf16(kt[t][kb], hi, S[t]);
                if (kDbg && (t & 1)) lo_pair(kb, t >> 1);
                if (kb == 0 && t < 2) vh[t] = cat8(to_half4(Vn[2 * t]), to_half4(Vn[2 * t + 1]));
                if (kb == 1 && (t & 1))
                    S16[t >> 1] = cat8(to_half4(S[t - 1]), to_half4(S[t]));
                if (kDbg && kb == 1) Sc[t] = Sc[t] * gam;
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        if constexpr (kDbg) {
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
                for (int t = 0; t < 8; ++t)
                    Sc[t] = mfma16_bf16(kt[t][kb], __builtin_bit_cast(bf16x8, lw[kb]), Sc[t]);
            }
        }
        // (8) hand-off of V_n (fp16) for the output
        sm.h[hs].V[0][lane] = vh[0];
        sm.h[hs].V[1][lane] = vh[1];
        __builtin_amdgcn_sched_barrier(0);
        // The counters go out behind this step's hand-off writes without
        // waiting for them: a wave's LDS operations are performed in issue
        // order, so a wave that sees a counter also sees what it publishes.
        // The chain's reads of ring C and ring P have completed (the products
        // consumed them), so freeC may release those stages.
        asm volatile("" ::: "memory");
        if (lane == 0) {
            lds_st_asm(&sm.ready, c + 1);
            lds_st_asm(&sm.freeC, c + 1);
            if (!kDbg) lds_st_asm(&sm.dvready, c + 1);
            else lds_st_asm(&sm.kfree, c + 1);   // no helper: the chain read K^T
        }
    }
    if (!ok) return;
    if (!kDbg && x.nch > 0) {
        // the helper's Sc, left in the lo slots after its last chunk
        if (!w.until([&] { return lds_ld(&sm.scdone) != 0; })) return;
        asm volatile("" ::: "memory");
        const f32x4* src = &sm.lo[0].d[0][0];
#pragma unroll
        for (int t = 0; t < 8; ++t) Sc[t] = src[t * 64 + lane];
    }
#pragma unroll
    for (int t = 0; t < 8; ++t) {
#pragma unroll
        for (int i = 0; i < 4; ++i) a.sf[sbase + (size_t)dk_of(t, i) * kDV] = S[t][i] + Sc[t][i];
    }
}

// Lo helper (SIMD 3): Sc <- e^{c63} Sc + K^T lo per chunk, with d o V_n from
// the chain split again into its bf16 hi part and the residual lo =
// bf16(d o V_n - hi), the same values the chain's hi part leaves out.  The K^T
// fragments are read from the chunk's ring-C stage, which the loaders refill
// only after this wave has read it (kfree): each chunk's K^T crosses from L2
// to the CU once.  After the last chunk Sc goes to the lo slots for the chain.
__device__ void run_lo_helper(ScanSmem& sm, const ScanArgs& a, const Waiter& w, const ScanCtx& x,
                              int lane) {
    if (x.nch <= 0) return;
    f32x4 Sc[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) Sc[t] = zero4();
    for (int c = 0; c < x.nch; ++c) {
        if (!w.until([&] { return lds_ld(&sm.dvready) >= c + 1; })) return;
        asm volatile("" ::: "memory");
        const LoHand& lh = sm.lo[c % kLoSlots];
        const StageC& sc = sm.c[c % kRingC];
        f32x4 d[4];
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) d[mt] = lh.d[mt][lane];
        const float gam = lh.gam;
        u32x4 kc[16];
#pragma unroll
        for (int f = 0; f < 16; ++f) kc[f] = sc.KT[f][lane];
        lds_wait_all();
        if (lane == 0) {
            lds_st(&sm.lodone, c + 1);
            lds_st(&sm.kfree, c + 1);
        }
        bf16x8 lo[2];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            u32x4 lw;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
#pragma unroll
                for (int p = 0; p < 2; ++p) {
                    const f32x4& dd = d[2 * kb + h];
                    const uint32_t hp = pack_bf16x2(dd[2 * p], dd[2 * p + 1]);
                    const float r0 = dd[2 * p] - __uint_as_float(hp << 16);
                    const float r1 = dd[2 * p + 1] - __uint_as_float(hp & 0xffff0000u);
                    lw[2 * h + p] = pack_bf16x2(r0, r1);
                }
            }
            lo[kb] = __builtin_bit_cast(bf16x8, lw);
        }
#pragma unroll
        for (int t = 0; t < 8; ++t) Sc[t] = Sc[t] * gam;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
            for (int t = 0; t < 8; ++t)
                Sc[t] = mfma16_bf16(__builtin_bit_cast(bf16x8, kc[t * 2 + kb]), lo[kb], Sc[t]);
        }
    }
    // every chunk's slot has been read: Sc goes to the lo slots
    f32x4* dst = &sm.lo[0].d[0][0];
#pragma unroll
    for (int t = 0; t < 8; ++t) dst[t * 64 + lane] = Sc[t];
    lds_wait_all();
    if (lane == 0) lds_st(&sm.scdone, 1);
}

// Gated-RMSNorm epilogue (kNorm; bf16 o, z and weight), y = gated_rmsnorm(o, z)
// in place over o, with the arithmetic of gated_rmsnorm_kernel (bf16, 8
// lanes per row of 128, two 16-byte pieces a lane: the same sums in the same
// order, so the same bits as the prefill followed by that kernel).  A row's
// 128 columns come from the 8 slice groups of its head.  Each output wave
// writes its chunk's o through to the device-coherent level and waits for
// those stores; the norm wave (wave 4) then adds 1 to the chunk-head's
// arrival counter (device-scope atomic; the prep zeroes it).  The group that
// brings it to 8 normalises the whole chunk-head, reading the other groups'
// o with device-scope loads.  No group waits on another.
__device__ inline uint32_t* norm_counter(const ScanArgs& a, const ScanCtx& x, int c) {
    return a.ws.ncnt + ((size_t)(x.chunk0 + c) * a.HV + x.hv) * (kNormCntBytes / 4);
}

// 16 bytes of o written by any group of the call: two device-scope 8-byte loads
__device__ __forceinline__ u32x4 ld_o_agent(const uint16_t* p) {
    const uint64_t* q = reinterpret_cast<const uint64_t*>(p);
    const uint64_t a = __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint64_t b = __hip_atomic_load(q + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return u32x4{(uint32_t)a, (uint32_t)(a >> 32), (uint32_t)b, (uint32_t)(b >> 32)};
}

// y for chunk c of this (sequence, v-head), all 128 columns: lane = 8 rr +
// sub takes rows rr, rr + 8, ... and columns 8 sub .. + 7 and 64 + 8 sub .. + 7
__device__ void norm_chunk(const ScanArgs& a, const ScanCtx& x, int c, const u32x4 (&wr)[2],
                           int lane) {
    constexpr int kPasses = kChunk / 8;
    const int sub = lane & 7, rr = lane >> 3;
    const int rows = min(kChunk, x.len - c * kChunk);
    u32x4 xr[kPasses][2], zr[kPasses][2];
#pragma unroll
    for (int ps = 0; ps < kPasses; ++ps) {
        const int r = min(8 * ps + rr, rows - 1);
        const size_t off = ((size_t)(x.tok_base + c * kChunk + r) * a.HV + x.hv) * kDV + 8 * sub;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            xr[ps][j] = ld_o_agent(a.o + off + 64 * j);
            zr[ps][j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(a.z + off + 64 * j));
        }
    }
    float wf[2][8];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            wf[j][2 * q] = bf16_bits_to_f32(wr[j][q] & 0xffffu);
            wf[j][2 * q + 1] = bf16_bits_to_f32(wr[j][q] >> 16);
        }
#pragma unroll
    for (int ps = 0; ps < kPasses; ++ps) {
        float xf[2][8], zf[2][8];
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                xf[j][2 * q] = bf16_bits_to_f32(xr[ps][j][q] & 0xffffu);
                xf[j][2 * q + 1] = bf16_bits_to_f32(xr[ps][j][q] >> 16);
                zf[j][2 * q] = bf16_bits_to_f32(zr[ps][j][q] & 0xffffu);
                zf[j][2 * q + 1] = bf16_bits_to_f32(zr[ps][j][q] >> 16);
            }
        float ss = 0.f;
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int e = 0; e < 8; ++e) ss = fmaf(xf[j][e], xf[j][e], ss);
        ss = lane_group_sum<8>(ss);
        const float rs = 1.0f / sqrtf(ss / (float)kDV + a.eps);
        u32x4 y4[2];
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                uint32_t pk = 0;
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const int e = 2 * q + h;
                    const float n = bf16_bits_to_f32(f32_to_bf16_bits(xf[j][e] * rs));
                    const float hv = bf16_bits_to_f32(f32_to_bf16_bits(wf[j][e] * n));
                    const float sz = zf[j][e] * __builtin_amdgcn_rcpf(
                                                    1.0f + __builtin_amdgcn_exp2f(zf[j][e] * -1.44269504088896341f));
                    pk |= (uint32_t)f32_to_bf16_bits(hv * sz) << (16 * h);
                }
                y4[j][q] = pk;
            }
        if (8 * ps + rr < rows) {
            const size_t off =
                ((size_t)(x.tok_base + c * kChunk + 8 * ps + rr) * a.HV + x.hv) * kDV + 8 * sub;
#pragma unroll
            for (int j = 0; j < 2; ++j)
                __builtin_nontemporal_store(y4[j], reinterpret_cast<u32x4*>(a.o + off + 64 * j));
        }
    }
}

// Norm wave (wave 4, norm epilogue only): per chunk, once this group's o for
// it is written, count the group in; the eighth group normalises the chunk.
__device__ void run_norm(ScanSmem& sm, const ScanArgs& a, const Waiter& w, const ScanCtx& x,
                         int lane) {
    u32x4 wr[2];
#pragma unroll
    for (int j = 0; j < 2; ++j)
        wr[j] = *reinterpret_cast<const u32x4*>(a.nw + 8 * (lane & 7) + 64 * j);
    for (int c = 0; c < x.nch; ++c) {
        const int jc = c & 1, kc = c >> 1;
        if (!w.until([&] { return lds_ld(&sm.npub[jc]) >= kc + 1; })) return;
        asm volatile("" ::: "memory");
        unsigned old = 0;
        if (lane == 0)
            old = __hip_atomic_fetch_add(norm_counter(a, x, c), 1u, __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
        old = __shfl(old, 0, 64);
        if (old == kSlices - 1) norm_chunk(a, x, c, wr, lane);
    }
}

// Output wave j (0 or 1): chunks j, j + 2, ...
template <int kRaw, bool kNorm>
__device__ void run_output(ScanSmem& sm, const ScanArgs& a, const Waiter& w, const ScanCtx& x,
                           int j, int lane) {
    const int lg = lane >> 4, lm = lane & 15;
    // Q and M fragments and s e^c go straight to registers; the next chunk's
    // loads are issued as soon as the current chunk's products have read them
    half8 qf[16], mf[kTri];
    float es[4];
    auto load = [&](int c) {
        const int cc = min(c, x.nch - 1);
        const size_t ch = (size_t)(x.chunk0 + cc) * a.HV + x.hv;
        const half8* qq = a.ws.Q + ((size_t)(x.chunk0 + cc) * a.HK + x.hk) * (16 * 64) + lane;
#pragma unroll
        for (int f = 0; f < 16; ++f) qf[f] = qq[f * 64];
        const half8* mm = a.ws.M + ch * (kTri * 64) + lane;
#pragma unroll
        for (int f = 0; f < kTri; ++f) mf[f] = mm[f * 64];
        const float* gr = a.ws.gates + ch * (kGateBytes / 4) + kGSec + lm;
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) es[mt] = gr[16 * mt];
    };
    if (j >= x.nch) return;
    // the first Q and M go out once chunk 0's chain operands are in (see
    // run_producer)
    if (!w.until([&] { return lds_ld(&sm.fill[0]) >= 1; })) return;
    asm volatile("" ::: "memory");
    load(j);
    for (int c = j; c < x.nch; c += 2) {
        const int hs = c % kHand;
        if (!w.until([&] { return lds_ld(&sm.ready) >= c + 1; })) return;
        asm volatile("" ::: "memory");
        half8 hsf[4], hvf[2];
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) hsf[kb] = sm.h[hs].S[kb][lane];
        hvf[0] = sm.h[hs].V[0][lane];
        hvf[1] = sm.h[hs].V[1][lane];
        lds_wait_all();
        if (lane == 0) lds_st(&sm.cons[j], (c >> 1) + 1);
        // O^T = (S^T Q^T) diag(s e^c) + V_n^T M^T: lane (lg, lm) of tile mt
        // holds columns 4 lg .. 4 lg + 3 of the slice for token 16 mt + lm
        f32x4 ov[4];
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) ov[mt] = zero4();
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) ov[mt] = mfma16(hsf[kb], qf[mt * 4 + kb], ov[mt]);
        }
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
            ov[mt] = ov[mt] * es[mt];
            ov[mt] = mfma16(hvf[0], mf[tri_base(mt)], ov[mt]);
            if (mt >= 2) ov[mt] = mfma16(hvf[1], mf[tri_base(mt) + 1], ov[mt]);
        }
        // the products have read Q, M and s e^c: the next chunk's go out now
        // (norm epilogue: after this chunk's o stores, which are waited for)
        asm volatile("" : "+v"(ov[0]), "+v"(ov[1]), "+v"(ov[2]), "+v"(ov[3]));
        if constexpr (!kNorm) load(c + 2);
        const int rows = min(kChunk, x.len - c * kChunk);
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
            const int r = 16 * mt + lm;
            uint2 pk;
            uint32_t b[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                b[e] = f32_to_bf16_bits(ov[mt][e]);
                if constexpr (kRaw == 2) b[e] = f16_bits(__uint_as_float(b[e] << 16));
            }
            pk.x = b[0] | (b[1] << 16);
            pk.y = b[2] | (b[3] << 16);
            if (r < rows) {
                uint2* dst = reinterpret_cast<uint2*>(
                    a.o + ((size_t)(x.tok_base + c * kChunk + r) * a.HV + x.hv) * kDV +
                    kSliceCols * x.sl + 4 * lg);
                if constexpr (kNorm) st_through(dst, pk);   // read back by another group
                else *dst = pk;
            }
        }
        if constexpr (kNorm) {
            // the stores have reached the device-coherent level: the norm
            // wave may count this group in for the chunk
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            if (lane == 0) lds_st(&sm.npub[j], (c >> 1) + 1);
            load(c + 2);
        }
    }
}

// The (sequence, v-head, k-head) of scan work-group pair index pidx (< N HV,
// uniform over the group) and its sequence's token and chunk ranges.  Packed
// sequences of different lengths: groups start in id order as CUs free up,
// so the low pair indices go to the longest sequences (longest first).
// seqsel and red are LDS scratch; every thread of the group calls this.
__device__ inline void scan_context(const ScanArgs& a, int pidx, int* seqsel, int* red,
                                    ScanCtx& x) {
    const int tid = threadIdx.x;
    x.seq = pidx / a.HV;
    x.hv = pidx - x.seq * a.HV;
    // pidx % 8 is the XCD: give the v-heads of one k-head the same XCD (one
    // L2 then holds that k-head's K^T and Q records for all of them) when
    // the heads tile the 8 XCDs evenly
    const int rep = a.HV / a.HK;
    if (rep > 1 && a.HV % 8 == 0 && a.HK % 8 == 0) {
        const int r = x.hv >> 3, xcd = x.hv & 7;
        x.hv = (xcd + 8 * (r / rep)) * rep + r % rep;
    }
    if (a.cu && a.N <= kScanThreads) {
        if (tid < a.N) {
            const int my = seq_count(a.cu, a.T, a.total, tid);
            int rank = 0;
            for (int u = 0; u < a.N; ++u) {
                const int lu = seq_count(a.cu, a.T, a.total, u);
                rank += (lu > my || (lu == my && u < tid)) ? 1 : 0;
            }
            if (rank == x.seq) *seqsel = tid;
        }
        __syncthreads();
        x.seq = *seqsel;
    }
    x.hk = x.hv / (a.HV / a.HK);
    x.len = seq_count(a.cu, a.T, a.total, x.seq);
    x.tok_base = seq_lo(a.cu, a.T, a.total, x.seq);
    x.chunk0 = __builtin_amdgcn_readfirstlane(
        chunks_before<kScanThreads>(a.cu, a.T, a.total, x.seq, red));
    x.nch = seq_chunks_bounded(a.cu, a.T, a.total, x.seq, x.chunk0, a.nch_bound);
}

// s0 and sf may be the same buffer: the chain reads its elements of the
// initial state before its first chunk and writes the same elements after its
// last, and no other wave touches either.
template <int kRaw, bool kDbg, bool kNorm = false>
__global__ __launch_bounds__(kScanThreads, 1) void gdn_scan_kernel(ScanArgs a) {
    __shared__ ScanSmem sm;
    // The kernel arguments (288 bytes) span five 64-byte lines, which the
    // scalar cache would otherwise fetch in three dependent round trips:
    // fields at most 32 bytes apart, all requested together, cost one.
    asm volatile("" ::"s"(a.in.q), "s"(a.in.beta), "s"(a.in.dt_bias), "s"(a.ws.M), "s"(a.ws.KT),
                 "s"(a.ws.dbgT), "s"(a.ws.dbgC), "s"(a.z), "s"(a.s0), "s"(a.N), "s"(a.HK),
                 "s"(a.spin));
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;

    // XCD-aware id: the eight groups of one (sequence, head) share id % 8
    // (one XCD, one L2), so their K, -W, Q and M come from one L2, and so
    // do the heads of one k-head where scan_context can arrange it
    const int id = blockIdx.x;
    const int xcd = id & 7, qd = id >> 3;
    ScanCtx x;
    x.sl = qd % kSlicesPerHead;
    const int pidx = (qd / kSlicesPerHead) * 8 + xcd;
    if (pidx >= a.N * a.HV) return;
    scan_context(a, pidx, &sm.seqsel, sm.red, x);
    if (tid == 0) {
        lds_st(&sm.fill[0], 0);
        lds_st(&sm.fill[1], 0);
        lds_st(&sm.pfill[0], 0);
        lds_st(&sm.pfill[1], 0);
        lds_st(&sm.uready, 0);
        lds_st(&sm.freeC, 0);
        lds_st(&sm.kfree, 0);
        lds_st(&sm.ready, 0);
        lds_st(&sm.cons[0], 0);
        lds_st(&sm.cons[1], 0);
        lds_st(&sm.dvready, 0);
        lds_st(&sm.lodone, 0);
        lds_st(&sm.scdone, 0);
        lds_st(&sm.npub[0], 0);
        lds_st(&sm.npub[1], 0);
        lds_st(&sm.abort, 0);
    }
    __syncthreads();
    const Waiter w{&sm.abort, a.ws.status, a.spin};
    // Waves go to SIMDs round-robin (wave w on SIMD w % 4): the chain has
    // SIMD 0 to itself but for the norm wave (norm epilogue only; otherwise
    // wave 4 exits at once), which issues a few memory operations per chunk;
    // the loaders share SIMDs 1 and 2
    // with the producer and an output wave, the lo helper SIMD 3 with the
    // other output wave.
    switch (wave) {
        case 0: run_chain<kDbg>(sm, a, w, x, lane); break;
        case 1: run_producer<kRaw>(sm, a, w, x, lane); break;
        case 2: run_output<kRaw, kNorm>(sm, a, w, x, 0, lane); break;
        case 3: run_output<kRaw, kNorm>(sm, a, w, x, 1, lane); break;
        case 4:
            if constexpr (kNorm) run_norm(sm, a, w, x, lane);
            break;
        case 5: run_loader(sm, a, w, x, 1, lane); break;
        case 6: run_loader(sm, a, w, x, 0, lane); break;
        default:
            // the debug build does the lo helper's work in the chain
            if constexpr (!kDbg) run_lo_helper(sm, a, w, x, lane);
            break;
    }
}

// ---------------------------------------------------------------------------
// paired scan kernel: one work-group (8 waves) per (32 value columns, v-head,
// sequence), for calls whose 16-column work-groups outnumber the CUs (packed
// or batched sequences).  The two 16-column halves of a group share its
// ring-C stages (K^T, -W), the gates, the (T - I) fragments, Q and M, so a
// chunk's operands cross from L2 to a CU once per 32 columns instead of once
// per 16, and the call takes half the group-steps.  Each half's arithmetic is
// the 16-column kernel's, operation for operation, so o and the final state
// are bitwise the same.
//
//   chains    waves 0 and 1 (SIMDs 0 and 1): one 128 x 16 state slice each,
//             the 16-column chain step; each also forms its half's bf16 lo
//             residual of d o V_n for the helper (the 16-column helper's own
//             arithmetic, moved so that two chunks fit the lo slots).
//   producer  wave 2: U of both halves.
//   lo helper wave 3: Sc of both halves; K^T read once per chunk.
//   loaders   waves 4 and 5 (beside the chains), chunks of even and odd
//             index: K^T, -W, V of both halves and the gates record of chunk
//             c into ring-C and ring-P stage c % 3 together.
//   outputs   waves 6 and 7, chunks of even and odd index: O of both halves.
//
// LDS, 162,920 of 163,840 bytes: ring C 3 x 32 KB, ring P 3 x 5 KB, a U ring
// 2 x 8 KB, 2 hand-off slots x 12 KB and 2 lo slots x 4 KB.  The helper's
// final Sc (16 KB) goes to ring-C stage nch % 3, which no chunk uses by then.
// ---------------------------------------------------------------------------
constexpr int kPairCols = 2 * kSliceCols;            // 32
constexpr int kPairsPerHead = kDV / kPairCols;       // 4
constexpr int kRingP2 = kRingC;   // V of both halves and gates, with ring C's stage
constexpr int kRingU2 = 2;        // U of both halves
constexpr int kHand2 = 2;         // chain -> output hand-off slots
static_assert(kHand2 % 2 == 0, "a hand-off slot is reused by a chunk of the same parity");

struct StageP2 {
    u32x4 V[2][kChunk * 2];   // per half: V rows of its 16 columns, 2 pieces per row
    float gates[256];         // gates record
};

struct StageU2 {
    f32x4 U[2][4][64];        // per half: U, D layout per row tile
};

struct Hand2 {
    half8 S[2][4][64];        // per half: S at the chunk's start, fp16 B fragments
    half8 V[2][2][64];        // per half: V_n, fp16 B fragments
};

struct LoHand2 {
    u32x4 lw[2][2][64];       // per half, k-block: bf16 lo residual of d o V_n (B operand)
};
constexpr int kLoSlots2 = 2;  // chain -> lo-helper hand-off slots

struct ScanSmem2 {
    StageC c[kRingC];
    StageP2 p[kRingP2];
    StageU2 u[kRingU2];
    Hand2 h[kHand2];
    LoHand2 lo[kLoSlots2];
    float gam[kLoSlots2];    // e^{c63} of the chunk in each lo slot
    int fill[2];      // per loader: chunks of its parity whose ring-C and ring-P loads have landed
    int uready;       // chunks whose U (both halves) is in the U ring
    int freeC[2];     // per chain: chunks whose ring-C, ring-P and U stages it has finished reading
    int kfree;        // chunks whose ring-C K^T the lo helper has finished reading
    int ready[2];     // per chain: chunks whose hand-off half it has written
    int cons[2];      // per output wave: chunks of its parity whose hand-off slot it has read
    int dvready[2];   // per chain: chunks whose lo residual half is in its lo slot
    int lodone;       // chunks whose lo slot the helper has read
    int scdone;       // the helper's Sc is in ring-C stage nch % 3
    int abort;        // a bounded wait ran out: every wave stops
    int seqsel;
    int red[kScanWaves];
};
static_assert(sizeof(ScanSmem2) <= 160 * 1024, "paired scan LDS");
static_assert(sizeof(StageC) >= 2 * 8 * 64 * sizeof(f32x4), "a ring-C stage holds both halves' Sc");

// Loader j (0 or 1) takes the chunks c of parity j: once stage c % 3 is free
// (chunk c - 3 read by both chains, the lo helper and the producer), one group
// of direct-to-LDS loads for chunk c: K^T (16), -W (16), V of both halves (4)
// and the gates record (1), published when all have landed.
__device__ void run_loader2(ScanSmem2& sm, const ScanArgs& a, const Waiter& w, const ScanCtx& x,
                            int j, int lane) {
    if (x.nch <= 0) return;
    for (int c = j; c < x.nch; c += 2) {
        const int need = c - kRingC + 1;
        if (!w.until([&] {
                const bool f0 = lds_ld(&sm.freeC[0]) >= need;
                const bool f1 = lds_ld(&sm.freeC[1]) >= need;
                const bool fk = lds_ld(&sm.kfree) >= need;
                const bool fu = lds_ld(&sm.uready) >= need;
                return f0 & f1 & fk & fu;
            }))
            break;
        asm volatile("" ::: "memory");
        const size_t ch = (size_t)(x.chunk0 + c) * a.HV + x.hv;
        StageC& st = sm.c[c % kRingC];
        const u32x4* ksrc = a.ws.KT + ((size_t)(x.chunk0 + c) * a.HK + x.hk) * (16 * 64) + lane;
#pragma unroll
        for (int f = 0; f < 16; ++f) lds_dma16(ksrc + f * 64, &st.KT[f][0]);
        const half8* wsrc = a.ws.W + ch * (16 * 64) + lane;
#pragma unroll
        for (int f = 0; f < 16; ++f) lds_dma16(wsrc + f * 64, &st.W[f][0]);
        StageP2& sp = sm.p[c % kRingP2];
        const int t0 = x.tok_base + c * kChunk, rows = min(kChunk, x.len - c * kChunk);
        // V: slot 64 i + lane of half h -> row (64 i + lane) / 2, piece lane % 2
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int s = 64 * i + lane, r = min(s >> 1, rows - 1);
                lds_dma16(a.in.v + ((size_t)(t0 + r) * a.HV + x.hv) * kDV + kPairCols * x.sl +
                              kSliceCols * h + 8 * (s & 1),
                          &sp.V[h][64 * i]);
            }
        }
        lds_dma16(a.ws.gates + ch * (kGateBytes / 4) + 4 * lane, &sp.gates[0]);
        vm_wait_all();
        if (lane == 0) lds_st(&sm.fill[j], (c >> 1) + 1);
    }
    vm_wait_all();   // no load may land in LDS after the group ends
}

// Producer: U = beta V + (T - I)(beta V) for both halves, the 16-column
// producer's products per half; (T - I) fragments two chunks ahead in two
// register sets used in turn.  U stage c % 2 is written once both chains have
// finished chunk c - 2.
template <int kRaw>
__device__ void run_producer2(ScanSmem2& sm, const ScanArgs& a, const Waiter& w,
                              const ScanCtx& x, int lane) {
    const int lg = lane >> 4, lm = lane & 15;
    auto load_t = [&](int c, half8 (&h)[kTri], half8 (&l)[kTri]) {
        const int cc = min(c, x.nch - 1);
        const size_t ch = (size_t)(x.chunk0 + cc) * a.HV + x.hv;
        const half8* ph = a.ws.TI + ch * (kTri * 64) + lane;
        const half8* pl = a.ws.TIlo + ch * (kTri * 64) + lane;
#pragma unroll
        for (int f = 0; f < kTri; ++f) {
            h[f] = ph[f * 64];
            l[f] = pl[f * 64];
        }
    };
    auto step = [&](int c, half8 (&th)[kTri], half8 (&tl)[kTri]) -> bool {
        if (!w.until([&] {
                const bool f = lds_ld(&sm.fill[c & 1]) >= (c >> 1) + 1;
                const bool u0 = lds_ld(&sm.freeC[0]) >= c - kRingU2 + 1;
                const bool u1 = lds_ld(&sm.freeC[1]) >= c - kRingU2 + 1;
                return f & u0 & u1;
            }))
            return false;
        asm volatile("" ::: "memory");
        const StageP2& st = sm.p[c % kRingP2];
        StageU2& su = sm.u[c % kRingU2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            // X = beta V, as the 16-column producer forms it
            f32x4 X[4];
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) {
                const f32x4 be = *reinterpret_cast<const f32x4*>(&st.gates[kGBeta + 16 * mt + 4 * lg]);
                const uint16_t* vsrc = reinterpret_cast<const uint16_t*>(st.V[h]) +
                                       (16 * mt + 4 * lg + (lm >> 2)) * kSliceCols + 4 * (lm & 3);
                const s16x4 vt = lds_read_tr(vsrc);
#pragma unroll
                for (int i = 0; i < 4; ++i) X[mt][i] = be[i] * v16_to_f32<kRaw>((uint16_t)vt[i]);
            }
            half8 xh[2], xl[2];
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) split_hilo8(X[2 * kb], X[2 * kb + 1], xh[kb], xl[kb]);
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) {
                f32x4 U = X[mt];
#pragma unroll
                for (int kb = 0; kb < 2; ++kb) {
                    if (kb > mt / 2) break;
                    const int f = tri_base(mt) + kb;
                    U = mfma16(th[f], xh[kb], U);
                    U = mfma16(th[f], xl[kb], U);
                    U = mfma16(tl[f], xh[kb], U);
                }
                su.U[h][mt][lane] = U;
            }
        }
        // the products have read this set: chunk c + 2's fragments go in
        load_t(c + 2, th, tl);
        asm volatile("" ::: "memory");
        if (lane == 0) lds_st_asm(&sm.uready, c + 1);
        return true;
    };
    if (x.nch <= 0) return;
    half8 t0h[kTri], t0l[kTri], t1h[kTri], t1l[kTri];
    load_t(0, t0h, t0l);
    load_t(1, t1h, t1l);
    // step() is false only when a bounded wait gave up
    for (int c = 0; c < x.nch; c += 2) {
        if (!step(c, t0h, t0l)) return;
        if (c + 1 < x.nch && !step(c + 1, t1h, t1l)) return;
    }
}

// Chain of half hh: the 16-column chain step on columns 32 sl + 16 hh ..
// + 15, with the paired kernel's stages and per-half counters.
__device__ void run_chain2(ScanSmem2& sm, const ScanArgs& a, const Waiter& w, const ScanCtx& x,
                           int hh, int lane) {
    const int lg = lane >> 4, lm = lane & 15;
    const int col = kPairCols * x.sl + kSliceCols * hh + lm;
    auto dk_of = [&](int t, int i) { return 32 * (t >> 1) + 8 * lg + 4 * (t & 1) + i; };
    const size_t sbase = ((size_t)x.seq * a.HV + x.hv) * kDK * kDV + col;

    f32x4 S[8];
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
    half8 S16[4];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) S16[kb] = cat8(to_half4(S[2 * kb]), to_half4(S[2 * kb + 1]));

    bool ok = true;
    for (int c = 0; c < x.nch; ++c) {
        const int hs = c % kHand2;
        StageC& sc = sm.c[c % kRingC];
        StageP2& sp = sm.p[c % kRingP2];
        StageU2& su = sm.u[c % kRingU2];
        auto ready = [&] {   // every counter loaded, no short-circuit: one round trip
            const bool f = lds_ld(&sm.fill[c & 1]) >= (c >> 1) + 1;
            const bool u = lds_ld(&sm.uready) >= c + 1;
            const bool h = lds_ld(&sm.cons[c & 1]) >= (c >= kHand2 ? ((c - kHand2) >> 1) + 1 : 0);
            const bool l = lds_ld(&sm.lodone) >= c - kLoSlots2 + 1;
            return f & u & h & l;
        };
        // (1) U, -W and the gates, read together with the counters (as in the
        // 16-column chain)
        f32x4 Vn[4], dec[4];
        half8 wf[16];
        float c63;
        auto read_operands = [&] {
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) Vn[mt] = su.U[hh][mt][lane];
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
                for (int mt = 0; mt < 4; ++mt) wf[mt * 4 + kb] = sc.W[mt * 4 + kb][lane];
            }
            c63 = sp.gates[kGC63];
#pragma unroll
            for (int mt = 0; mt < 4; ++mt)
                dec[mt] = *reinterpret_cast<const f32x4*>(&sp.gates[kGDec + 16 * mt + 4 * lg]);
        };
        const bool early = ready();
        asm volatile("" ::: "memory");
        read_operands();
        if (!early) {
            ok = w.until(ready);
            if (!ok) break;
            asm volatile("" ::: "memory");
            read_operands();
        }
        asm volatile("" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
        // (2) V_n = U + (-W) S16
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) Vn[mt] = mfma16(wf[mt * 4 + kb], S16[kb], Vn[mt]);
        }
        // (3) K^T operands of the state update
        bf16x8 kt[8][2];
#pragma unroll
        for (int t = 0; t < 8; ++t) {
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) kt[t][kb] = __builtin_bit_cast(bf16x8, sc.KT[t * 2 + kb][lane]);
        }
        // (4) decay; S at the chunk's start to the hand-off slot
        const float gam = __builtin_amdgcn_exp2f(c63 * kLog2e);
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) sm.h[hs].S[hh][kb][lane] = S16[kb];
#pragma unroll
        for (int t = 0; t < 8; ++t) S[t] = S[t] * gam;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
            __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);   // VALU
            __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);   // LDS read
        }
        asm volatile("" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
        // (5) d o V_n, hi part (bf16)
        f32x4 dv[4];
        u32x4 hw[2];
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
            dv[mt] = dec[mt] * Vn[mt];
            asm volatile("" : "+v"(dv[mt]));
        }
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
#pragma unroll
                for (int p = 0; p < 2; ++p)
                    hw[kb][2 * h + p] = pack_bf16x2(dv[2 * kb + h][2 * p], dv[2 * kb + h][2 * p + 1]);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        // (6) the bf16 lo residual of d o V_n and the decay to the lo helper
        {
            LoHand2& lh = sm.lo[c % kLoSlots2];
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                u32x4 lw;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int h = q >> 1, p = q & 1;
                    const f32x4& d = dv[2 * kb + h];
                    const uint32_t hp = hw[kb][q];
                    const float r0 = d[2 * p] - __uint_as_float(hp << 16);
                    const float r1 = d[2 * p + 1] - __uint_as_float(hp & 0xffff0000u);
                    lw[q] = pack_bf16x2(r0, r1);
                }
                lh.lw[hh][kb][lane] = lw;
            }
            if (hh == 0 && lane == 0) sm.gam[c % kLoSlots2] = gam;
        }
        // (7) S' = e^{c63} S + K^T hi
        half8 vh[2];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            const bf16x8 hi = __builtin_bit_cast(bf16x8, hw[kb]);
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                S[t] = mfma16_bf16(kt[t][kb], hi, S[t]);
                if (kb == 0 && t < 2) vh[t] = cat8(to_half4(Vn[2 * t]), to_half4(Vn[2 * t + 1]));
                if (kb == 1 && (t & 1))
                    S16[t >> 1] = cat8(to_half4(S[t - 1]), to_half4(S[t]));
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        // (8) hand-off of V_n (fp16) for the output
        sm.h[hs].V[hh][0][lane] = vh[0];
        sm.h[hs].V[hh][1][lane] = vh[1];
        __builtin_amdgcn_sched_barrier(0);
        // published behind this step's LDS writes, as in the 16-column chain
        asm volatile("" ::: "memory");
        if (lane == 0) {
            lds_st_asm(&sm.ready[hh], c + 1);
            lds_st_asm(&sm.freeC[hh], c + 1);
            lds_st_asm(&sm.dvready[hh], c + 1);
        }
    }
    if (!ok) return;
    f32x4 Sc[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) Sc[t] = zero4();
    if (x.nch > 0) {
        // the helper's Sc, left in ring-C stage nch % 3 after its last chunk
        if (!w.until([&] { return lds_ld(&sm.scdone) != 0; })) return;
        asm volatile("" ::: "memory");
        const f32x4* src = reinterpret_cast<const f32x4*>(&sm.c[x.nch % kRingC]) + hh * 8 * 64;
#pragma unroll
        for (int t = 0; t < 8; ++t) Sc[t] = src[t * 64 + lane];
    }
#pragma unroll
    for (int t = 0; t < 8; ++t) {
#pragma unroll
        for (int i = 0; i < 4; ++i) a.sf[sbase + (size_t)dk_of(t, i) * kDV] = S[t][i] + Sc[t][i];
    }
}

// Lo helper: Sc <- e^{c63} Sc + K^T lo for both halves, with the lo residuals
// the chains formed and K^T read once per chunk from its ring-C stage.
__device__ void run_lo_helper2(ScanSmem2& sm, const ScanArgs& a, const Waiter& w,
                               const ScanCtx& x, int lane) {
    if (x.nch <= 0) return;
    f32x4 Sc[2][8];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
        for (int t = 0; t < 8; ++t) Sc[h][t] = zero4();
    }
    for (int c = 0; c < x.nch; ++c) {
        if (!w.until([&] {
                const bool d0 = lds_ld(&sm.dvready[0]) >= c + 1;
                const bool d1 = lds_ld(&sm.dvready[1]) >= c + 1;
                return d0 & d1;
            }))
            return;
        asm volatile("" ::: "memory");
        const StageC& sc = sm.c[c % kRingC];
        const LoHand2& lh = sm.lo[c % kLoSlots2];
        u32x4 lwv[2][2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) lwv[h][kb] = lh.lw[h][kb][lane];
        }
        const float gam = sm.gam[c % kLoSlots2];
        u32x4 kc[16];
#pragma unroll
        for (int f = 0; f < 16; ++f) kc[f] = sc.KT[f][lane];
        lds_wait_all();
        if (lane == 0) {
            lds_st(&sm.lodone, c + 1);
            lds_st(&sm.kfree, c + 1);
        }
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            bf16x8 lo[2];
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) lo[kb] = __builtin_bit_cast(bf16x8, lwv[h][kb]);
#pragma unroll
            for (int t = 0; t < 8; ++t) Sc[h][t] = Sc[h][t] * gam;
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
                for (int t = 0; t < 8; ++t)
                    Sc[h][t] = mfma16_bf16(__builtin_bit_cast(bf16x8, kc[t * 2 + kb]), lo[kb], Sc[h][t]);
            }
        }
    }
    // every chunk is done: no wave reads ring-C stage nch % 3 (it last held
    // chunk nch - 3, which both chains and this wave have finished) and no
    // loader fills it again
    f32x4* dst = reinterpret_cast<f32x4*>(&sm.c[x.nch % kRingC]);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
        for (int t = 0; t < 8; ++t) dst[(h * 8 + t) * 64 + lane] = Sc[h][t];
    }
    lds_wait_all();
    if (lane == 0) lds_st(&sm.scdone, 1);
}

// Output wave j: O of both halves for the chunks of parity j, the 16-column
// output's products per half; Q, M and s e^c are shared by the halves.
template <int kRaw>
__device__ void run_output2(ScanSmem2& sm, const ScanArgs& a, const Waiter& w, const ScanCtx& x,
                            int j, int lane) {
    const int lg = lane >> 4, lm = lane & 15;
    half8 qf[16], mf[kTri];
    float es[4];
    auto load = [&](int c) {
        const int cc = min(c, x.nch - 1);
        const size_t ch = (size_t)(x.chunk0 + cc) * a.HV + x.hv;
        const half8* qq = a.ws.Q + ((size_t)(x.chunk0 + cc) * a.HK + x.hk) * (16 * 64) + lane;
#pragma unroll
        for (int f = 0; f < 16; ++f) qf[f] = qq[f * 64];
        const half8* mm = a.ws.M + ch * (kTri * 64) + lane;
#pragma unroll
        for (int f = 0; f < kTri; ++f) mf[f] = mm[f * 64];
        const float* gr = a.ws.gates + ch * (kGateBytes / 4) + kGSec + lm;
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) es[mt] = gr[16 * mt];
    };
    if (j >= x.nch) return;
    load(j);
    for (int c = j; c < x.nch; c += 2) {
        const int hs = c % kHand2;
        if (!w.until([&] {
                const bool r0 = lds_ld(&sm.ready[0]) >= c + 1;
                const bool r1 = lds_ld(&sm.ready[1]) >= c + 1;
                return r0 & r1;
            }))
            return;
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
        if (lane == 0) lds_st(&sm.cons[j], (c >> 1) + 1);
        f32x4 ov[2][4];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) ov[h][mt] = zero4();
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
                for (int mt = 0; mt < 4; ++mt) ov[h][mt] = mfma16(hsf[h][kb], qf[mt * 4 + kb], ov[h][mt]);
            }
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) {
                ov[h][mt] = ov[h][mt] * es[mt];
                ov[h][mt] = mfma16(hvf[h][0], mf[tri_base(mt)], ov[h][mt]);
                if (mt >= 2) ov[h][mt] = mfma16(hvf[h][1], mf[tri_base(mt) + 1], ov[h][mt]);
            }
        }
        // the products have read Q, M and s e^c: the next chunk's go out now
        asm volatile("" : "+v"(ov[0][0]), "+v"(ov[0][1]), "+v"(ov[0][2]), "+v"(ov[0][3]),
                     "+v"(ov[1][0]), "+v"(ov[1][1]), "+v"(ov[1][2]), "+v"(ov[1][3]));
        load(c + 2);
        const int rows = min(kChunk, x.len - c * kChunk);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) {
                const int r = 16 * mt + lm;
                uint32_t b[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    b[e] = f32_to_bf16_bits(ov[h][mt][e]);
                    if constexpr (kRaw == 2) b[e] = f16_bits(__uint_as_float(b[e] << 16));
                }
                if (r < rows) {
                    uint2* dst = reinterpret_cast<uint2*>(
                        a.o + ((size_t)(x.tok_base + c * kChunk + r) * a.HV + x.hv) * kDV +
                        kPairCols * x.sl + kSliceCols * h + 4 * lg);
                    *dst = make_uint2(b[0] | (b[1] << 16), b[2] | (b[3] << 16));
                }
            }
        }
    }
}

template <int kRaw>
__global__ __launch_bounds__(kScanThreads, 1) void gdn_scan2_kernel(ScanArgs a) {
    __shared__ ScanSmem2 sm;
    // kernel-argument lines requested together (as in gdn_scan_kernel)
    asm volatile("" ::"s"(a.in.q), "s"(a.in.beta), "s"(a.in.dt_bias), "s"(a.ws.M), "s"(a.ws.KT),
                 "s"(a.ws.dbgT), "s"(a.ws.dbgC), "s"(a.z), "s"(a.s0), "s"(a.N), "s"(a.HK),
                 "s"(a.spin));
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    // XCD-aware id: the four groups of one (sequence, head) share id % 8
    const int id = blockIdx.x;
    const int xcd = id & 7, qd = id >> 3;
    ScanCtx x;
    x.sl = qd % kPairsPerHead;
    const int pidx = (qd / kPairsPerHead) * 8 + xcd;
    if (pidx >= a.N * a.HV) return;
    scan_context(a, pidx, &sm.seqsel, sm.red, x);
    if (tid == 0) {
        lds_st(&sm.fill[0], 0);
        lds_st(&sm.fill[1], 0);
        lds_st(&sm.uready, 0);
        lds_st(&sm.freeC[0], 0);
        lds_st(&sm.freeC[1], 0);
        lds_st(&sm.kfree, 0);
        lds_st(&sm.ready[0], 0);
        lds_st(&sm.ready[1], 0);
        lds_st(&sm.cons[0], 0);
        lds_st(&sm.cons[1], 0);
        lds_st(&sm.dvready[0], 0);
        lds_st(&sm.dvready[1], 0);
        lds_st(&sm.lodone, 0);
        lds_st(&sm.scdone, 0);
        lds_st(&sm.abort, 0);
    }
    __syncthreads();
    const Waiter w{&sm.abort, a.ws.status, a.spin};
    // wave w runs on SIMD w % 4: each chain shares its SIMD with a loader
    switch (wave) {
        case 0: run_chain2(sm, a, w, x, 0, lane); break;
        case 1: run_chain2(sm, a, w, x, 1, lane); break;
        case 2: run_producer2<kRaw>(sm, a, w, x, lane); break;
        case 3: run_lo_helper2(sm, a, w, x, lane); break;
        case 4: run_loader2(sm, a, w, x, 0, lane); break;
        case 5: run_loader2(sm, a, w, x, 1, lane); break;
        case 6: run_output2<kRaw>(sm, a, w, x, 0, lane); break;
        default: run_output2<kRaw>(sm, a, w, x, 1, lane); break;
    }
}

// raw: 0 for prepared inputs, 1 / 2 for raw bf16 / fp16 q, k (normalised in
// the prep; then v and o have that dtype too).
// The gated-RMSNorm epilogue's inputs (bf16 z [token][HV][128], bf16 weight
// [128], eps); o then receives y.
struct NormIn {
    const uint16_t* z;
    const uint16_t* w;
    float eps;
};

// Scan work-groups of a call over N sequences of HV heads.
inline long long scan_groups(int N, int HV) {
    return (long long)((N * HV + 7) / 8) * 8 * kSlicesPerHead;
}

// ... and of the paired instance (32 columns per group).
inline long long scan2_groups(int N, int HV) {
    return (long long)((N * HV + 7) / 8) * 8 * kPairsPerHead;
}

// CUs of the current device (cached per device; 256 if the query fails).
int device_cus() {
    constexpr int kDevs = 64;
    static int cached[kDevs] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kDevs) return 256;
    int n = __atomic_load_n(&cached[dev], __ATOMIC_RELAXED);
    if (n <= 0) {
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            n <= 0)
            n = 256;
        __atomic_store_n(&cached[dev], n, __ATOMIC_RELAXED);
    }
    return n;
}

// Scan instance: 16-column groups while they fit on the CUs at once (one
// group per CU), the paired 32-column groups once they would run in rounds
// (then the halves' shared operands halve the rounds).  cols forces 16 or 32
// (diagnostics); the debug dump and the norm epilogue exist in the 16-column
// instance only.
bool use_pair_scan(int cols, int N, int HV, int dump_debug, bool norm) {
    if (cols == 32) return true;
    if (cols == 16 || dump_debug || norm) return false;
    return (long long)N * HV * kSlicesPerHead > device_cus();
}

hipError_t launch_prefill(const PrepIn& in, int raw, void* o, const float* s0, float* sf,
                          const int32_t* cu, int N, int T, int total_tokens, int HV, int HK,
                          size_t nch_bound, void* workspace, size_t workspace_bytes,
                          hipStream_t stream, int dump_debug, hipEvent_t* ev = nullptr,
                          int only = -1, unsigned spin = kDefaultSpin,
                          const NormIn* norm = nullptr, int cols = 0) {
    const bool pair = use_pair_scan(cols, N, HV, dump_debug, norm != nullptr);
    if (pair && (dump_debug || norm)) return hipErrorInvalidValue;
    const WsLayout L(nch_bound * (size_t)HV);
    const size_t need = dump_debug ? L.total : L.live;
    if (workspace_bytes < need) return hipErrorInvalidValue;
    char* base = static_cast<char*>(workspace);
    Workspace ws{};
    ws.TI = reinterpret_cast<half8*>(base + L.ti);
    ws.TIlo = reinterpret_cast<half8*>(base + L.tilo);
    ws.M = reinterpret_cast<half8*>(base + L.m);
    ws.W = reinterpret_cast<half8*>(base + L.w);
    ws.gates = reinterpret_cast<float*>(base + L.gates);
    ws.Q = reinterpret_cast<half8*>(base + L.q);
    ws.KT = reinterpret_cast<u32x4*>(base + L.kt);
    ws.ncnt = norm ? reinterpret_cast<uint32_t*>(base + L.ncnt) : nullptr;   // norm epilogue only
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
        // records that cannot stay in the memory-side cache go out
        // non-temporally (see st_through)
        const bool nt = !dump_debug && need > kNtWorkspaceBytes;
        auto kern = raw == 1 ? (nt ? gdn_prep_kernel<false, 1, true> : gdn_prep_kernel<false, 1>)
                    : raw == 2 ? (nt ? gdn_prep_kernel<false, 2, true> : gdn_prep_kernel<false, 2>)
                    : dump_debug ? gdn_prep_kernel<true, 0>
                    : nt ? gdn_prep_kernel<false, 0, true> : gdn_prep_kernel<false, 0>;
        PrepIn pin = in;
        pin.s0 = s0;
        hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(kPrepThreads), 0, stream, pin, cu, N, T,
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
    if (norm) {
        sa.z = norm->z;
        sa.nw = norm->w;
        sa.eps = norm->eps;
    }
    const unsigned grid = (unsigned)(pair ? scan2_groups(N, HV) : scan_groups(N, HV));
    hipError_t err;
    if (pair) {
        auto scan = raw == 1 ? gdn_scan2_kernel<1> : raw == 2 ? gdn_scan2_kernel<2> : gdn_scan2_kernel<0>;
        hipLaunchKernelGGL(scan, dim3(grid), dim3(kScanThreads), 0, stream, sa);
        err = hipGetLastError();
    } else if (norm) {
        hipLaunchKernelGGL((gdn_scan_kernel<0, false, true>), dim3(grid), dim3(kScanThreads), 0,
                           stream, sa);
        err = hipGetLastError();
    } else {
        auto scan = raw == 1 ? gdn_scan_kernel<1, false>
                    : raw == 2 ? gdn_scan_kernel<2, false>
                    : dump_debug ? gdn_scan_kernel<0, true> : gdn_scan_kernel<0, false>;
        hipLaunchKernelGGL(scan, dim3(grid), dim3(kScanThreads), 0, stream, sa);
        err = hipGetLastError();
    }
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

namespace {
bool norm_args_ok(const void* q, const void* k, const void* v, const float* g, const float* beta,
                  const void* z, const void* norm_weight, float eps, void* y, float* final_state,
                  int B, int T, int HV, int HQK, int DK, int DV, int chunk_size,
                  void* workspace) {
    if (!dims_ok(HV, HQK, DK, DV, chunk_size) || B <= 0 || T < 0) return false;
    if (workspace == nullptr || final_state == nullptr) return false;
    if (T > 0 && (!q || !k || !v || !g || !beta || !z || !norm_weight || !y)) return false;
    return eps >= 0.f;
}

// The prefill writes o into y, then the gated RMSNorm kernel rewrites it in
// place: two kernels that never wait on each other.
hipError_t prefill_then_norm(const void* q, const void* k, const void* v, const float* g,
                             const float* beta, const void* z, const void* norm_weight, float eps,
                             void* y, const float* initial_state, float* final_state, int B,
                             int T, int HV, int HQK, void* workspace, size_t workspace_bytes,
                             hipStream_t stream) {
    const size_t nc = (size_t)B * ((T + kChunk - 1) / kChunk);
    hipError_t e = launch_prefill(plain_in(q, k, v, g, beta), 0, y, initial_state, final_state,
                                  nullptr, B, T, B * T, HV, HQK, nc, workspace, workspace_bytes,
                                  stream, 0);
    if (e != hipSuccess || T == 0) return e;
    return gdn_gated_rmsnorm_forward(y, z, norm_weight, y, (int64_t)B * T * HV, kDV, eps,
                                     GDN_DTYPE_BF16, GDN_DTYPE_BF16, stream);
}
}  // namespace

extern "C" hipError_t deltanet_chunk_prefill_norm(const void* q, const void* k, const void* v,
                                                  const float* g, const float* beta, const void* z,
                                                  const void* norm_weight, float eps, void* y,
                                                  const float* initial_state, float* final_state,
                                                  int B, int T, int HV, int HQK, int DK, int DV,
                                                  int chunk_size, void* workspace,
                                                  size_t workspace_bytes, hipStream_t stream) {
    if (!norm_args_ok(q, k, v, g, beta, z, norm_weight, eps, y, final_state, B, T, HV, HQK, DK,
                      DV, chunk_size, workspace))
        return hipErrorInvalidValue;
    return prefill_then_norm(q, k, v, g, beta, z, norm_weight, eps, y, initial_state, final_state,
                             B, T, HV, HQK, workspace, workspace_bytes, stream);
}

extern "C" hipError_t deltanet_chunk_prefill_norm_fused(
    const void* q, const void* k, const void* v, const float* g, const float* beta, const void* z,
    const void* norm_weight, float eps, void* y, const float* initial_state, float* final_state,
    int B, int T, int HV, int HQK, int DK, int DV, int chunk_size, void* workspace,
    size_t workspace_bytes, hipStream_t stream) {
    if (!norm_args_ok(q, k, v, g, beta, z, norm_weight, eps, y, final_state, B, T, HV, HQK, DK,
                      DV, chunk_size, workspace))
        return hipErrorInvalidValue;
    // The epilogue lives in the 16-column scan; where the plain prefill would
    // take the paired 32-column instance (more slice groups than CUs) the
    // two-kernel path runs instead.
    if (use_pair_scan(0, B, HV, 0, false))
        return prefill_then_norm(q, k, v, g, beta, z, norm_weight, eps, y, initial_state,
                                 final_state, B, T, HV, HQK, workspace, workspace_bytes, stream);
    const size_t nc = (size_t)B * ((T + kChunk - 1) / kChunk);
    const NormIn n{static_cast<const uint16_t*>(z), static_cast<const uint16_t*>(norm_weight), eps};
    return launch_prefill(plain_in(q, k, v, g, beta), 0, y, initial_state, final_state, nullptr,
                          B, T, B * T, HV, HQK, nc, workspace, workspace_bytes, stream, 0, nullptr,
                          -1, kDefaultSpin, &n);
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

extern "C" hipError_t deltanet_chunk_prefill_cols(const void* q, const void* k, const void* v,
                                                  const float* g, const float* beta, void* o,
                                                  const float* initial_state, float* final_state,
                                                  const int32_t* cu_seqlens, int num_seqs, int T,
                                                  int HV, int HQK, void* workspace,
                                                  size_t workspace_bytes, hipStream_t stream,
                                                  int slice_cols, unsigned spin_limit) {
    if (slice_cols != 0 && slice_cols != kSliceCols && slice_cols != kPairCols)
        return hipErrorInvalidValue;
    if (!dims_ok(HV, HQK, kDK, kDV, kChunk) || num_seqs <= 0 || T < 0) return hipErrorInvalidValue;
    if (workspace == nullptr || final_state == nullptr) return hipErrorInvalidValue;
    if (T > 0 && (!q || !k || !v || !g || !beta || !o)) return hipErrorInvalidValue;
    const unsigned spin = spin_limit ? spin_limit : kDefaultSpin;
    if (cu_seqlens) {
        const size_t nc = ((size_t)T + (size_t)(kChunk - 1) * num_seqs) / kChunk;
        return launch_prefill(plain_in(q, k, v, g, beta), 0, o, initial_state, final_state,
                              cu_seqlens, num_seqs, 0, T, HV, HQK, nc, workspace, workspace_bytes,
                              stream, 0, nullptr, -1, spin, nullptr, slice_cols);
    }
    if ((long long)num_seqs * T > 0x7fffffffLL) return hipErrorInvalidValue;
    const size_t nc = (size_t)num_seqs * ((T + kChunk - 1) / kChunk);
    return launch_prefill(plain_in(q, k, v, g, beta), 0, o, initial_state, final_state, nullptr,
                          num_seqs, T, num_seqs * T, HV, HQK, nc, workspace, workspace_bytes,
                          stream, 0, nullptr, -1, spin, nullptr, slice_cols);
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

// Host twins of the kernels' block-cooperative lookups: the same phases, run
// for every simulated thread between the points where the kernel has a
// barrier, on the shared gdn_seq.h arithmetic.
extern "C" int deltanet_varlen_chunks_before(const int32_t* cu_seqlens, int num_seqs,
                                             int total_tokens, int upto, int nt) {
    if (!cu_seqlens || num_seqs <= 0 || total_tokens < 0 || upto < 0 || upto > num_seqs ||
        nt < 64 || nt > 1024 || nt % 64 != 0)
        return -1;
    std::vector<int> acc(nt, 0), nxt(nt);
    for (int t = 0; t < nt; ++t)
        for (int s = t; s < upto; s += nt)
            acc[t] = sat_add(acc[t], seq_chunks(cu_seqlens, 0, total_tokens, s));
    for (int off = 32; off > 0; off >>= 1) {   // butterfly within each wave of 64
        for (int t = 0; t < nt; ++t) nxt[t] = sat_add(acc[t], acc[t ^ off]);
        acc.swap(nxt);
    }
    int tot = 0;
    for (int w = 0; w < nt / 64; ++w) tot = sat_add(tot, acc[w * 64]);
    return tot;
}

extern "C" int deltanet_varlen_locate_chunk(const int32_t* cu_seqlens, int num_seqs,
                                            int total_tokens, int cid, int nt,
                                            int32_t* seq_tok_rows) {
    if (!cu_seqlens || !seq_tok_rows || num_seqs <= 0 || total_tokens < 0 || nt < 2 ||
        nt > 1024 || (nt & (nt - 1)) != 0)
        return -1;
    const int N = num_seqs;
    std::vector<int> red(nt), cnt(nt), incl(nt), v(nt);
    int base = 0;
    bool found = false;
    for (int s0 = 0; s0 < N && base < kSatChunks; s0 += nt) {
        for (int t = 0; t < nt; ++t) {
            const int s = s0 + t;
            cnt[t] = (s < N) ? seq_chunks(cu_seqlens, 0, total_tokens, s) : 0;
            red[t] = cnt[t];
        }
        for (int off = 1; off < nt; off <<= 1) {
            for (int t = 0; t < nt; ++t) v[t] = scan_step(red.data(), t, off);
            red.swap(v);
        }
        for (int t = 0; t < nt; ++t) incl[t] = red[t];
        const int blk = red[nt - 1];
        red[0] = -1;
        red[1] = -1;
        for (int t = 0; t < nt; ++t) {
            if (owns_chunk(cnt[t], incl[t], base, cid)) {
                red[0] = s0 + t;
                red[1] = cid - base - (incl[t] - cnt[t]);
            }
        }
        const bool here = cid < sat_add(base, blk);
        if (here) {
            int tok0 = 0, rows = 0;
            found = seq_chunk_rows(cu_seqlens, N, 0, total_tokens, red[0], red[1], tok0, rows);
            if (found) {
                seq_tok_rows[0] = red[0];
                seq_tok_rows[1] = tok0;
                seq_tok_rows[2] = rows;
            }
        }
        base = sat_add(base, blk);
        if (here) break;
    }
    return found ? 1 : 0;
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

// ---------------------------------------------------------------------------
// Allocation-free prefill: the workspace is a file-scope device array.
// ---------------------------------------------------------------------------
// 48 MiB per GPU that loads the library, held until the process ends: the
// live workspace of up to (48 MiB - 256 B) / 69 KB = 712 chunk-heads, e.g.
// T <= 1408 at HV = 32 (22 chunks).
constexpr size_t kNoAllocScratchBytes = size_t(48) << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The array's device address on the current device, looked up once per
// device: in host code `scratch` names a host-side stand-in, never the
// device memory.
hipError_t noalloc_scratch(void** out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        if (!p) return hipErrorInvalidSymbol;
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return hipSuccess;
}
}  // namespace

extern "C" hipError_t deltanet_chunk_prefill_noalloc(const void* q, const void* k, const void* v,
                                                     const float* g, const float* beta, void* o,
                                                     const float* initial_state,
                                                     float* final_state, int B, int T, int HV,
                                                     int HQK, int DK, int DV, int chunk_size,
                                                     hipStream_t stream) {
    if (!dims_ok(HV, HQK, DK, DV, chunk_size) || B <= 0 || T < 0) return hipErrorInvalidValue;
    if (final_state == nullptr) return hipErrorInvalidValue;
    if (T > 0 && (!q || !k || !v || !g || !beta || !o)) return hipErrorInvalidValue;
    const size_t nc = (size_t)B * ((T + kChunk - 1) / kChunk);
    if (WsLayout(nc * HV).live > kNoAllocScratchBytes) return hipErrorInvalidValue;   // too large
    void* ws = nullptr;
    const hipError_t e = noalloc_scratch(&ws);
    if (e != hipSuccess) return e;
    return launch_prefill(plain_in(q, k, v, g, beta), 0, o, initial_state, final_state, nullptr, B,
                          T, B * T, HV, HQK, nc, ws, kNoAllocScratchBytes, stream, 0);
}

extern "C" hipError_t deltanet_prefill_noalloc_status(hipStream_t stream) {
    void* ws = nullptr;
    const hipError_t e = noalloc_scratch(&ws);
    if (e != hipSuccess) return e;
    return deltanet_prefill_status(ws, kNoAllocScratchBytes, stream);
}

// ---------------------------------------------------------------------------
// Two-level chunk-group scan (diagnostic): each sequence's chunks are cut
// into `segments` chunk-aligned segments, which the kernels above treat as
// sequences of their own (same global chunk ids, so one prep serves every
// pass).  A chunk maps the state affinely, S -> A_n S + B_n, so a segment's
// end state is Phi_j S_entry + B_j:
//   pass 1a  scan from a zero state (the first segment of a sequence from its
//            initial state): B_j, and the first segment's final outputs;
//   pass 1b  scan of v = 0 from S = I: Phi_j = A_last ... A_first;
//   combine  E_1 = (pass 1a end state of segment 0),
//            E_j = Phi_{j-1} E_{j-1} + B_{j-1}, in fp32, serial over j;
//   replay   scan from the entry states E_j: o and the final state.
// The serial depth is max segment length (pass 1), segments - 2 (combine) and
// max segment length (replay) instead of the sequence's chunk count, at
// about three times the chain work.
// ---------------------------------------------------------------------------
namespace {

constexpr int kSt = kDK * kDV;   // floats per (sequence, head) state

// s0a[seg] = the sequence's initial state for its first segment, else 0;
// s0i[seg] = I; zero v rows.
__global__ __launch_bounds__(256) void twolevel_init_kernel(const float* __restrict__ s0,
                                                            const int32_t* __restrict__ seg_seq,
                                                            const int32_t* __restrict__ seg_first,
                                                            int nseg, int HV, float* s0a,
                                                            float* s0i, uint32_t* zv,
                                                            size_t zv_words) {
    const size_t n = (size_t)nseg * HV * kSt;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) {
        const size_t sh = i / kSt;
        const int seg = (int)(sh / HV), h = (int)(sh % HV);
        const int e = (int)(i % kSt), r = e / kDV, c = e % kDV;
        const bool first = seg_first[seg] != 0;
        s0a[i] = (first && s0) ? s0[((size_t)seg_seq[seg] * HV + h) * kSt + e] : 0.f;
        s0i[i] = r == c ? 1.f : 0.f;
    }
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < zv_words;
         i += (size_t)gridDim.x * 256)
        zv[i] = 0u;
}

// One work-group per (sequence, head, 16-column slice): the entry states of
// the sequence's segments 1.. in order, E_j[:, slice] = Phi_{j-1} E_{j-1} +
// B_{j-1} (fp32; E_1 = B_0, which already started from the initial state).
__global__ __launch_bounds__(256) void twolevel_combine_kernel(
    const float* __restrict__ phi, const float* __restrict__ bst,
    const int32_t* __restrict__ seq_seg0, const int32_t* __restrict__ seq_nseg, int HV,
    float* __restrict__ E) {
    __shared__ float prev[kDK][16];
    const int sl = blockIdx.x % 8, h = (blockIdx.x / 8) % HV, s = blockIdx.x / (8 * HV);
    const int seg0 = seq_seg0[s], ns = seq_nseg[s];
    const int t = threadIdx.x, r = t >> 1, c0 = (t & 1) * 8;
    const int col = sl * 16 + c0;
    if (ns < 2) return;
    // E_1 = B_0
    {
        const float* b = bst + ((size_t)seg0 * HV + h) * kSt + (size_t)r * kDV + col;
        float* e = E + ((size_t)(seg0 + 1) * HV + h) * kSt + (size_t)r * kDV + col;
        for (int i = 0; i < 8; ++i) {
            e[i] = b[i];
            prev[r][c0 + i] = b[i];
        }
    }
    __syncthreads();
    for (int j = 2; j < ns; ++j) {
        const float* p = phi + ((size_t)(seg0 + j - 1) * HV + h) * kSt + (size_t)r * kDV;
        const float* b = bst + ((size_t)(seg0 + j - 1) * HV + h) * kSt + (size_t)r * kDV + col;
        float acc[8];
        for (int i = 0; i < 8; ++i) acc[i] = b[i];
        for (int kk = 0; kk < kDK; ++kk) {
            const float pv = p[kk];
            for (int i = 0; i < 8; ++i) acc[i] = fmaf(pv, prev[kk][c0 + i], acc[i]);
        }
        __syncthreads();
        float* e = E + ((size_t)(seg0 + j) * HV + h) * kSt + (size_t)r * kDV + col;
        for (int i = 0; i < 8; ++i) {
            e[i] = acc[i];
            prev[r][c0 + i] = acc[i];
        }
        __syncthreads();
    }
}

// final_state[s] = the replay's end state of sequence s's last segment
__global__ __launch_bounds__(256) void twolevel_gather_kernel(const float* __restrict__ sfr,
                                                              const int32_t* __restrict__ seq_last,
                                                              int nseq, int HV,
                                                              float* __restrict__ sf) {
    const size_t n = (size_t)nseq * HV * kSt;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) {
        const size_t sh = i / kSt;
        const int s = (int)(sh / HV), h = (int)(sh % HV);
        sf[i] = sfr[((size_t)seq_last[s] * HV + h) * kSt + i % kSt];
    }
}

struct TwoLevelPlan {
    std::vector<int32_t> seg_cu, seg_seq, seg_first, seq_seg0, seq_nseg, seq_last;
    int nseg = 0, nseq = 0, total = 0, chunks = 0;
};

// Chunk-aligned segments of every sequence: sequence s of n_s chunks gets
// min(segments, n_s) segments (one when it is empty) of near-equal chunk
// counts.  cu_host NULL: B sequences of T tokens.
bool twolevel_plan(const int32_t* cu_host, int nseq, int T, int segments, TwoLevelPlan& p) {
    if (nseq <= 0 || segments <= 0 || segments > 1024) return false;
    p.nseq = nseq;
    p.seg_cu.assign(1, 0);
    int pos = 0;
    for (int s = 0; s < nseq; ++s) {
        const int lo = cu_host ? cu_host[s] : s * T, hi = cu_host ? cu_host[s + 1] : (s + 1) * T;
        if (lo != pos || hi < lo) return false;   // well-formed, starting at 0
        const int len = hi - lo, nc = (len + kChunk - 1) / kChunk;
        const int g = nc > 0 ? std::min(segments, nc) : 1;
        p.seq_seg0.push_back(p.nseg);
        p.seq_nseg.push_back(g);
        for (int j = 0; j < g; ++j) {
            const int c1 = (int)((long long)nc * (j + 1) / g);
            p.seg_cu.push_back(j + 1 == g ? hi : lo + c1 * kChunk);
            p.seg_seq.push_back(s);
            p.seg_first.push_back(j == 0);
        }
        p.nseg += g;
        p.seq_last.push_back(p.nseg - 1);
        p.chunks += nc;
        pos = hi;
    }
    p.total = pos;
    return true;
}

size_t twolevel_ws_bytes(const TwoLevelPlan& p, int HV, size_t* off) {
    size_t o = 0;
    auto put = [&](int i, size_t bytes) {
        off[i] = o;
        o += align256(bytes);
    };
    const size_t st = (size_t)p.nseg * HV * kSt * 4;
    put(0, WsLayout((size_t)std::max(p.chunks, 1) * HV).live);   // prefill workspace
    put(1, (p.nseg + 1) * 4);                                      // seg cu
    put(2, p.nseg * 4);                                            // seg -> sequence
    put(3, p.nseg * 4);                                            // first-segment flags
    put(4, p.nseq * 4 * 3);                                        // seq: first seg, count, last
    for (int i = 5; i < 11; ++i) put(i, st);   // s0a, s0i, B, Phi, E, replay end states
    put(11, (size_t)p.total * HV * kDV * 2);   // zero v
    put(12, (size_t)p.total * HV * kDV * 2);   // pass 1b o (discarded)
    return o;
}

}  // namespace

extern "C" size_t deltanet_prefill_twolevel_workspace_size(const int32_t* cu_seqlens_host,
                                                           int num_seqs, int T, int HV,
                                                           int segments) {
    TwoLevelPlan p;
    if (HV <= 0 || T < 0 || !twolevel_plan(cu_seqlens_host, num_seqs, T, segments, p)) return 0;
    size_t off[13];
    return twolevel_ws_bytes(p, HV, off);
}

extern "C" hipError_t deltanet_chunk_prefill_twolevel(
    const void* q, const void* k, const void* v, const float* g, const float* beta, void* o,
    const float* initial_state, float* final_state, const int32_t* cu_seqlens_host, int num_seqs,
    int T, int HV, int HQK, int segments, void* workspace, size_t workspace_bytes,
    hipStream_t stream, hipEvent_t* events, int n_events) {
    if (!dims_ok(HV, HQK, kDK, kDV, kChunk) || T < 0 || !final_state || !workspace)
        return hipErrorInvalidValue;
    if (events && n_events != 6) return hipErrorInvalidValue;
    TwoLevelPlan p;
    if (!twolevel_plan(cu_seqlens_host, num_seqs, T, segments, p)) return hipErrorInvalidValue;
    if (p.total > 0 && (!q || !k || !v || !g || !beta || !o)) return hipErrorInvalidValue;
    size_t off[13];
    if (workspace_bytes < twolevel_ws_bytes(p, HV, off)) return hipErrorInvalidValue;
    char* base = static_cast<char*>(workspace);
    auto at = [&](int i) { return base + off[i]; };
    // the segment table, copied in (host memory: wait for the copy)
    std::vector<int32_t> seqtab(p.seq_seg0);
    seqtab.insert(seqtab.end(), p.seq_nseg.begin(), p.seq_nseg.end());
    seqtab.insert(seqtab.end(), p.seq_last.begin(), p.seq_last.end());
    hipError_t e = hipSuccess;
    auto copy = [&](int i, const std::vector<int32_t>& h) {
        if (e == hipSuccess && !h.empty())
            e = hipMemcpyAsync(at(i), h.data(), h.size() * 4, hipMemcpyHostToDevice, stream);
    };
    copy(1, p.seg_cu);
    copy(2, p.seg_seq);
    copy(3, p.seg_first);
    copy(4, seqtab);
    if (e == hipSuccess) e = hipStreamSynchronize(stream);
    if (e != hipSuccess) return e;
    const int32_t* seg_cu = reinterpret_cast<const int32_t*>(at(1));
    const int32_t* seq_seg0 = reinterpret_cast<const int32_t*>(at(4));
    float* s0a = reinterpret_cast<float*>(at(5));
    float* s0i = reinterpret_cast<float*>(at(6));
    float* bst = reinterpret_cast<float*>(at(7));
    float* phi = reinterpret_cast<float*>(at(8));
    float* E = reinterpret_cast<float*>(at(9));
    float* sfr = reinterpret_cast<float*>(at(10));
    void* zv = at(11);
    void* o_junk = at(12);
    void* ws = at(0);
    const size_t wsb = off[1] - off[0];
    const size_t nch = (size_t)std::max(p.chunks, 1);
    auto rec = [&](int i) {
        if (events) (void)hipEventRecord(events[i], stream);
    };
    rec(0);
    const size_t zv_words = (size_t)p.total * HV * kDV / 2;
    hipLaunchKernelGGL(twolevel_init_kernel, dim3(1024), dim3(256), 0, stream, initial_state,
                       reinterpret_cast<const int32_t*>(at(2)),
                       reinterpret_cast<const int32_t*>(at(3)), p.nseg, HV, s0a, s0i,
                       static_cast<uint32_t*>(zv), zv_words);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    const PrepIn in = plain_in(q, k, v, g, beta);
    // prep over the segment chunking (same global chunk ids as the plain call)
    e = launch_prefill(in, 0, o, s0a, bst, seg_cu, p.nseg, 0, p.total, HV, HQK, nch, ws, wsb,
                       stream, 0, nullptr, 0);
    if (e != hipSuccess) return e;
    rec(1);
    // pass 1a: B_j (and the first segments' final outputs)
    e = launch_prefill(in, 0, o, s0a, bst, seg_cu, p.nseg, 0, p.total, HV, HQK, nch, ws, wsb,
                       stream, 0, nullptr, 1);
    if (e != hipSuccess) return e;
    rec(2);
    // pass 1b: Phi_j from v = 0 and S = I
    const PrepIn in0 = plain_in(q, k, zv, g, beta);
    e = launch_prefill(in0, 0, o_junk, s0i, phi, seg_cu, p.nseg, 0, p.total, HV, HQK, nch, ws,
                       wsb, stream, 0, nullptr, 1);
    if (e != hipSuccess) return e;
    rec(3);
    hipLaunchKernelGGL(twolevel_combine_kernel, dim3(p.nseq * HV * 8), dim3(256), 0, stream, phi,
                       bst, seq_seg0, seq_seg0 + p.nseq, HV, E);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    rec(4);
    // replay from the entry states, the first segments again from their
    // initial state (s0a)
    for (int s = 0; s < p.nseq; ++s) {
        const size_t bytes = (size_t)HV * kSt * 4;
        const size_t seg = (size_t)p.seq_seg0[s];
        e = hipMemcpyAsync(E + seg * HV * kSt, s0a + seg * HV * kSt, bytes,
                           hipMemcpyDeviceToDevice, stream);
        if (e != hipSuccess) return e;
    }
    e = launch_prefill(in, 0, o, E, sfr, seg_cu, p.nseg, 0, p.total, HV, HQK, nch, ws, wsb,
                       stream, 0, nullptr, 1);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(twolevel_gather_kernel, dim3(256), dim3(256), 0, stream, sfr,
                       seq_seg0 + 2 * p.nseq, p.nseq, HV, final_state);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    rec(5);
    return hipSuccess;
}
