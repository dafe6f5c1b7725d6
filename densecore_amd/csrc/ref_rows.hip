// Rows whose reference result is fixed by the reference's blocking, not by the attention math:
// causal attention with a scale that is not positive, and a NaN scale.
//
// The reference writes -inf into causally masked scores before it scales them
// (src/torch_attention.rs:202-207, then mul_reduce_max :216 / :48-87, or scale_add_mask :212,
// :130-141), over the whole kvb-wide key block (:182) of the last block a query block visits
// (`num_keys - n <= kvs`, :202).  With scale < 0 a filled score becomes +inf, the row max +inf and
// exp(+inf - +inf) NaN; with scale 0 (or -0) it becomes NaN.  Either way every row with at least
// one filled score in its last block gets NaN out and lse.  That set follows from the reference's
// own tile policy (q_split :26-35, KV_SPLIT :14): row i of the query block [m, m + qb) visits keys
// up to num_keys = min(m + qb, S); its last block starts at n = the largest multiple of
// kvs = min(512, S) below num_keys and ends at min(n + kvs, S); the row has a filled score there
// iff i + 1 < that end.  A NaN scale makes every score NaN: every row with a key is NaN, except
// that without a mask a block narrower than 4 keys has only the scalar tail of mul_reduce_max,
// whose std_max (:42-45, :73-76) skips NaN, so its max stays -inf and the row is taken as fully
// masked (:219-222): out 0, lse 0.
//
// The flash kernels compute those rows as PyTorch's own kernels would (masked keys at
// probability 0); the forward pass here then overwrites them with the reference's values.
//
// The backward, given such rows (NaN lse, or NaN dsum = rowsum(dO * out)), spreads NaN as the
// reference does (:336-452): P = exp(score - lse) is NaN at every visited key of a NaN-lse row
// and the causal fill zeroes P only after the exponential (:363-367); dS = P (dP - dsum) is NaN
// at every visited key, zeroed ones included, of a NaN-dsum row.  So dQ of such a row is NaN; dK
// is NaN at every key a NaN-dS entry reaches (causal: [0, end of the row's last block) for a NaN
// dsum, [0, i] for a NaN lse; otherwise all S keys); dV at every key a NaN P reaches (causal
// [0, i], otherwise all).  The kernels reach a subset of those keys (they skip key tiles past the
// diagonal and fully masked ones); the backward pass here completes the set.
#include <cmath>

#include "common.hpp"
#include "params.hpp"

namespace dc {
namespace {

// src/torch_attention.rs:26-35 (q_split) and :14 (KV_SPLIT): the end of the last key block the
// reference visits for query row i under causal masking (0: it visits none).
DEVI int ref_causal_block_end(int i, int L, int S) {
    int qs = L >= 768 ? 256 : (L >= 192 ? 64 : 32);
    qs = min(qs, L);
    const int kvs = min(512, S);
    const int m = i / qs * qs, qb = min(qs, L - m);
    const int num_keys = min(m + qb, S);
    if (num_keys <= 0) return 0;
    return min((num_keys - 1) / kvs * kvs + kvs, S);
}

constexpr uint16_t kBf16NaN = 0x7fc0;

// Row value v (NaN or 0) over E elements, by the 64 lanes of one wave.
DEVI void fill_row(void *base, int64_t row, int E, bool bf16, float v, int lane) {
    if (bf16) {
        uint16_t *p = static_cast<uint16_t *>(base) + row * E;
        const uint16_t x = v != v ? kBf16NaN : 0;
        for (int c = lane; c < E; c += 64) p[c] = x;
    } else {
        float *p = static_cast<float *>(base) + row * E;
        for (int c = lane; c < E; c += 64) p[c] = v;
    }
}

// One wave per query row.  mode 0: causal, scale <= 0 (the rows with a filled score in their last
// block); mode 1: NaN scale, every row; mode 2: NaN scale, no mask, S < 4: every row 0, lse 0.
__global__ __launch_bounds__(256) void fwd_ref_rows_kernel(AttnShape s, void *out, float *lse, bool bf16,
                                                          int mode) {
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= (int64_t)s.B * s.H * s.L) return;
    const int i = (int)(row % s.L);
    if (mode == 0 && i + 1 >= ref_causal_block_end(i, s.L, s.S)) return;
    const float v = mode == 2 ? 0.f : NAN;
    fill_row(out, row, s.E, bf16, v, lane);
    if (lane == 0) lse[row] = v;
}

// One workgroup per (batch, kv head): the reference's NaN reach of the rows of its query heads
// whose lse (or, with a NaN scale, every row's P) or dsum is NaN.
__global__ __launch_bounds__(256) void bwd_ref_nan_kernel(AttnShape s, const float *lse, const float *dsum,
                                                         void *dq, void *dk, void *dv, bool bf16,
                                                         bool nan_scale) {
    __shared__ int bound_k, bound_v;
    const int bk = blockIdx.x, b = bk / s.Hkv, hk = bk % s.Hkv;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (threadIdx.x == 0) bound_k = 0, bound_v = 0;
    __syncthreads();
    int wk = 0, wv = 0;
    const int rows = s.repeat * s.L;
    for (int r = wave; r < rows; r += 4) {
        const int h = hk * s.repeat + r / s.L, i = r % s.L;
        const int64_t at = ((int64_t)b * s.H + h) * s.L + i;
        const bool dn = dsum[at] != dsum[at];
        const bool ln = nan_scale || lse[at] != lse[at];
        if (!(dn || ln) || s.S == 0) continue;
        fill_row(dq, at, s.E, bf16, NAN, lane);
        if (s.causal) {
            const int seen = min(i + 1, s.S);
            // A NaN scale is the alpha of the dK product (:442-454): NaN over whole visited blocks.
            if (dn || nan_scale) wk = max(wk, ref_causal_block_end(i, s.L, s.S));
            if (ln) wk = max(wk, seen), wv = max(wv, seen);
        } else {
            wk = s.S;
            if (ln) wv = s.S;
        }
    }
    if (lane == 0) {
        atomicMax(&bound_k, wk);
        atomicMax(&bound_v, wv);
    }
    __syncthreads();
    const int64_t kv0 = (int64_t)bk * s.S;
    for (int j = wave; j < bound_k; j += 4) fill_row(dk, kv0 + j, s.E, bf16, NAN, lane);
    for (int j = wave; j < bound_v; j += 4) fill_row(dv, kv0 + j, s.E, bf16, NAN, lane);
    if (nan_scale) {
        // Every score is NaN, also those of the kernels' padding rows past L, whose probability
        // is otherwise exp(score - inf) = 0: the keys past the reach get the reference's 0 (no
        // visited block holds them for dK; only zeroed probabilities reach them for dV).
        for (int j = bound_k + wave; j < s.S; j += 4) fill_row(dk, kv0 + j, s.E, bf16, 0.f, lane);
        for (int j = bound_v + wave; j < s.S; j += 4) fill_row(dv, kv0 + j, s.E, bf16, 0.f, lane);
    }
}

}  // namespace

bool ref_rows_needed(const AttnShape &s) { return s.S > 0 && ((s.causal && !(s.scale > 0.f)) || std::isnan(s.scale)); }

hipError_t launch_fwd_ref_rows(const FwdArgs &a, bool bf16, hipStream_t st) {
    const AttnShape &s = a.s;
    if (!ref_rows_needed(s)) return hipSuccess;
    const int64_t rows = (int64_t)s.B * s.H * s.L;
    if (rows == 0) return hipSuccess;
    const int mode = !std::isnan(s.scale) ? 0 : (s.mask == nullptr && s.S < 4 ? 2 : 1);
    const int64_t blocks = (rows + 3) / 4;
    if (blocks > INT32_MAX) return hipErrorInvalidConfiguration;
    return launch(fwd_ref_rows_kernel, dim3((unsigned)blocks), dim3(256), st, s, a.out, a.lse, bf16, mode);
}

hipError_t launch_bwd_ref_nan(const BwdArgs &a, bool bf16, hipStream_t st) {
    const AttnShape &s = a.s;
    if (!ref_rows_needed(s) || (int64_t)s.B * s.Hkv == 0 || s.L == 0) return hipSuccess;
    const bool nan_scale = std::isnan(s.scale);
    return launch(bwd_ref_nan_kernel, dim3(s.B * s.Hkv), dim3(256), st, s, a.lse,
                  static_cast<const float *>(a.dsum), a.dq, a.dk, a.dv, bf16, nan_scale);
}

}  // namespace dc
