// Split key ranges of the forward (float32 and bf16 kernels): when the grid of query tiles fills at
// most half of the workgroups that fit on the device at once (few heads, long rows), each query
// tile's key tiles run as near-equal pieces, each writing its normalized partial output and lse
// to the forward's workspace, and fwd_split_merge_kernel combines them.
#pragma once

#include "common.hpp"
#include "params.hpp"

namespace dc {
namespace {

// Key tiles (of BN keys) query tile qt (of kBM queries) reads, and the pieces of at most `chunk`
// tiles it runs as when key ranges are split (1 without a split).  Piece p of n covers tiles
// [p * tiles / n, (p + 1) * tiles / n).
__host__ __device__ inline int fwd_tiles(const AttnShape &s, int kBM, int BN, int qt) {
    const int kv_end = s.causal ? min((qt + 1) * kBM, s.S) : s.S;
    return (kv_end + BN - 1) / BN;
}
__host__ __device__ inline int fwd_pieces(const AttnShape &s, int kBM, int BN, int qt, int chunk) {
    if (chunk <= 0) return 1;
    const int n = (fwd_tiles(s, kBM, BN, qt) + chunk - 1) / chunk;
    return n > 1 ? n : 1;
}

struct FwdSplitPlan {
    int chunk = 0, max_pieces = 1;  // chunk 0: no split
    int64_t blocks = 0;             // pieces over all query tiles and heads
    size_t bytes = 0;               // workspace: float32 partial rows, then their lse
};

// Workgroups of `kernel` (threads per workgroup) that fit on the current device at once; 0 when
// unknown or when a grid of `blocks` workgroups certainly fills more than half of them (no CU
// holds more than 8 workgroups of these kernels).
inline int64_t split_slots(const void *kernel, int threads, int64_t blocks) {
    const int cus = device_cus();
    if (cus <= 0 || 2 * blocks > 8 * (int64_t)cus) return 0;
    return (int64_t)cus * device_occupancy(kernel, threads);
}

// The split for a grid of query tiles of kBM queries over key tiles of BN keys, `slots`
// workgroups resident at once.  Pieces hold at least 4 key tiles (a piece's fixed costs, its
// queries, the first tile's latency, the partial row and its merge, are then spread over 128+
// keys), and there are no more pieces than slots: a second, partial wave of pieces doubles the
// time.
inline FwdSplitPlan plan_split(const AttnShape &s, int kBM, int BN, int64_t slots) {
    FwdSplitPlan p;
    if (s.mask != nullptr || s.L == 0 || s.S == 0) return p;
    const int nqt = (s.L + kBM - 1) / kBM;
    const int64_t BH = (int64_t)s.B * s.H;
    if (slots <= 0 || 2 * nqt * BH > slots) return p;
    int64_t tiles = 0;
    int most = 0;
    for (int qt = 0; qt < nqt; ++qt) {
        const int n = fwd_tiles(s, kBM, BN, qt);
        tiles += n;
        most = n > most ? n : most;
    }
    tiles *= BH;
    int64_t chunk = (tiles + slots - 1) / slots;
    for (chunk = chunk < 4 ? 4 : chunk; chunk < most; ++chunk) {
        p.blocks = 0;
        for (int qt = 0; qt < nqt; ++qt) p.blocks += BH * fwd_pieces(s, kBM, BN, qt, (int)chunk);
        if (p.blocks <= slots) break;
    }
    if (chunk >= most) return FwdSplitPlan{};
    p.chunk = (int)chunk;
    for (int qt = 0; qt < nqt; ++qt) {
        const int np = fwd_pieces(s, kBM, BN, qt, p.chunk);
        p.max_pieces = np > p.max_pieces ? np : p.max_pieces;
    }
    const size_t rows = (size_t)BH * s.L * p.max_pieces;
    p.bytes = rows * s.E * sizeof(float) + rows * sizeof(float);
    return p;
}

// Block `bid` of a split grid as (query tile, head, piece, pieces): query tiles longest first,
// the pieces of one head contiguous.  Returns false past the grid (not reached).
DEVI bool split_block(const AttnShape &s, int kBM, int BN, int chunk, int bid, int *qt, int *bh,
                      int *piece, int *npieces) {
    const int nqt = (s.L + kBM - 1) / kBM;
    int per_head = 0;
    for (int t = 0; t < nqt; ++t) per_head += fwd_pieces(s, kBM, BN, t, chunk);
    *bh = bid / per_head;
    int r = bid % per_head;
    for (int t = nqt - 1; t >= 0; --t) {
        const int np = fwd_pieces(s, kBM, BN, t, chunk);
        if (r < np) {
            *qt = t, *piece = r, *npieces = np;
            return *bh < s.B * s.H;
        }
        r -= np;
    }
    return false;
}

DEVI void store_out(float *p, float x) { *p = x; }
DEVI void store_out(__bf16 *p, float x) { *p = static_cast<__bf16>(x); }

// Combines the pieces of split query tiles, 16 lanes per query row: with the pieces' lse values
// l_p and normalized outputs o_p, lse = log sum exp(l_p) and out = sum exp(l_p - lse) o_p.  A row
// no piece sees any key of keeps the reference's out = 0, lse = 0.  Rows of query tiles that ran
// whole were written by the forward and are skipped.  Each lane carries 4 consecutive dims of
// each 64 (16-byte loads when the partial rows' width is a multiple of 4), so a wave merges 4
// rows with independent loads.
template <typename OutT>
__global__ __launch_bounds__(256) void fwd_split_merge_kernel(FwdArgs a, int kBM, int BN) {
    const AttnShape &s = a.s;
    const int64_t row = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);
    const int sub = threadIdx.x & 15;
    if (row >= (int64_t)s.B * s.H * s.L) return;
    const int np = fwd_pieces(s, kBM, BN, (int)(row % s.L) / kBM, a.split_chunk);
    if (np <= 1) return;
    const float *pl = a.split_lse + row * a.split_max;
    const float *po = a.split_o + row * a.split_max * s.E;
    OutT *orow = static_cast<OutT *>(a.out) + row * s.E;
    float mx = -INFINITY;
    for (int p = 0; p < np; ++p) mx = fmaxf(mx, pl[p]);
    if (mx == -INFINITY) {
        for (int d = sub; d < s.E; d += 16) store_out(orow + d, 0.f);
        if (sub == 0) a.lse[row] = 0.f;
        return;
    }
    float wsum = 0.f;
    if ((s.E & 3) == 0) {
        f32x4 acc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};  // dims 4 sub + 64 j, E <= 128
#pragma unroll 4
        for (int p = 0; p < np; ++p) {
            const float w = expf(pl[p] - mx);
            wsum += w;
            const float *src = po + (int64_t)p * s.E;
#pragma unroll
            for (int j = 0; j < 2; ++j)
                if (4 * sub + 64 * j < s.E) acc[j] += w * *reinterpret_cast<const f32x4 *>(src + 4 * sub + 64 * j);
        }
        const float inv = 1.f / wsum;
#pragma unroll
        for (int j = 0; j < 2; ++j)
            if (4 * sub + 64 * j < s.E)
#pragma unroll
                for (int e = 0; e < 4; ++e) store_out(orow + 4 * sub + 64 * j + e, acc[j][e] * inv);
    } else {
        for (int p = 0; p < np; ++p) wsum += expf(pl[p] - mx);
        const float inv = 1.f / wsum;
        for (int d = sub; d < s.E; d += 16) {
            float acc = 0.f;
            for (int p = 0; p < np; ++p) acc = fmaf(expf(pl[p] - mx), po[(int64_t)p * s.E + d], acc);
            store_out(orow + d, acc * inv);
        }
    }
    if (sub == 0) a.lse[row] = mx + logf(wsum);
}

}  // namespace
}  // namespace dc
