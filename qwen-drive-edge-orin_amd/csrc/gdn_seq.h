// Sequence and chunk bookkeeping of the chunked prefill, shared by the
// kernels (device) and deltanet_varlen_chunk_map (host, for tests).
//
// Packed variable-length batches give cu_seqlens [N + 1].  Every value is
// clamped into [0, total_tokens] and a sequence's end is clamped to be no
// earlier than its start, so any cu_seqlens -- including a non-monotone or
// out-of-range one -- gives token ranges inside [0, total_tokens).  Chunk ids
// at or past the workspace's chunk bound are never formed: the prep skips
// them and the scan truncates a sequence that would reach them.  Malformed
// input thus gives wrong results, never an access out of bounds.  Fixed-length
// batches (cu == nullptr) are N sequences of T tokens, cu[i] = i * T.
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define GDN_HD __host__ __device__
#else
#define GDN_HD
#endif

namespace gdn {

constexpr int kChunkRows = 64;

GDN_HD inline int clamp_tok(int32_t x, int total) { return x < 0 ? 0 : (x > total ? total : (int)x); }

// First token of sequence s.
GDN_HD inline int seq_lo(const int32_t* cu, int T, int total, int s) {
    return cu ? clamp_tok(cu[s], total) : s * T;
}

// Token count of sequence s (>= 0).
GDN_HD inline int seq_count(const int32_t* cu, int T, int total, int s) {
    if (!cu) return T;
    const int lo = clamp_tok(cu[s], total), hi = clamp_tok(cu[s + 1], total);
    return hi > lo ? hi - lo : 0;
}

GDN_HD inline int seq_chunks(const int32_t* cu, int T, int total, int s) {
    const int n = seq_count(cu, T, total, s);
    return n / kChunkRows + (n % kChunkRows != 0);   // no n + 63 overflow near INT_MAX
}

// Chunks a sequence may use when its first chunk id is chunk0 and the
// workspace holds nch_bound chunks per head.
GDN_HD inline int seq_chunks_bounded(const int32_t* cu, int T, int total, int s, int chunk0,
                                     int nch_bound) {
    const int n = seq_chunks(cu, T, total, s);
    const int room = nch_bound - chunk0;
    return room <= 0 ? 0 : (n < room ? n : room);
}

// Prefix sums of chunk counts saturate at kSatChunks, far above any chunk
// bound a workspace can hold, so even adversarial cu_seqlens cannot wrap
// them.  For a, b >= 0, sat_add(a, b) = min(a + b, kSatChunks), which is
// associative and commutative: every reduction order gives the same sum.
constexpr int kSatChunks = 1 << 30;

GDN_HD inline int sat_add(int a, int b) {
    const long long s = (long long)a + b;
    return s > kSatChunks ? kSatChunks : (int)s;
}

// Step `off` of the block-cooperative inclusive scan (Hillis-Steele) over
// red[0, NT): thread tid's new value.
GDN_HD inline int scan_step(const int* red, int tid, int off) {
    return tid >= off ? sat_add(red[tid], red[tid - off]) : red[tid];
}

// Whether the sequence holding `cnt` chunks, whose inclusive prefix within a
// block of sequences is `incl` and whose block starts at chunk id `base`,
// holds chunk id cid (exact while the prefix has not saturated).
GDN_HD inline bool owns_chunk(int cnt, int incl, int base, int cid) {
    const int excl = incl - cnt;
    return cnt > 0 && incl < kSatChunks && cid >= base + excl && cid < base + incl;
}

// Chunk c of sequence seq (0 <= seq < N): its first token and row count, or
// false when no such chunk exists.  Whatever seq and c a lookup produced,
// a true result names rows [tok0, tok0 + rows) inside [0, total), 1 <= rows
// <= 64.
GDN_HD inline bool seq_chunk_rows(const int32_t* cu, int N, int T, int total, int seq, int c,
                                  int& tok0, int& rows) {
    if (seq < 0 || seq >= N || c < 0) return false;
    const int n = seq_count(cu, T, total, seq);
    if (c >= n / kChunkRows + (n % kChunkRows != 0)) return false;
    tok0 = seq_lo(cu, T, total, seq) + c * kChunkRows;
    const int left = n - c * kChunkRows;
    rows = left < kChunkRows ? left : kChunkRows;
    return true;
}

}  // namespace gdn
