// Attention for head dims above 128: the flash kernels instantiate head dims up to 128, while
// DenseCore's forward and backward take any head dim (src/torch_attention.rs:150-171, 300-320
// size their buffers by q_split * E with no cap).  Wider heads run here, materialized over blocks
// of query rows, with the batched products on dc_bmm's MFMA kernel (bmm.hip):
//
//   forward, per row block:  S = Q K^T;  P = softmax(scale * S + mask, causal) row by row, with
//                            lse = max + ln(sum) (fully masked rows: P = 0, lse = 0,
//                            :223-226, :258-264);  O = P V
//   backward, per row block: S = Q K^T;  P = exp(scale * S + mask - lse);  dV += P^T dO;
//                            dP = dO V^T;  dS = scale * P * (dP - dsum);  dQ = dS K;
//                            dK += dS^T Q
//
// Each (batch, kv head) item owns the rows of its query heads, which lie contiguously in q, out,
// lse, dq and dO: row j of item (b, hk) is query l = j % L of head h = hk * repeat + j / L, so
// grouped heads need no widening and dK / dV sum over the group's query heads in the products.
// Row blocks run in order and dK / dV accumulate in that order: results are identical from run to
// run.  bf16 inputs are copied to float32 first (the arithmetic is float32 throughout, as the
// reference's), and bf16 outputs are rounded once at the end.  All buffers are in the caller's
// workspace; a smaller workspace only shortens the row blocks (down to one row).
#include "bwd_common.hpp"
#include "common.hpp"
#include "params.hpp"

namespace dc {
namespace {

constexpr size_t kRowBlockBytes = (size_t)512 << 20;  // one score buffer at the full workspace
constexpr int kRowsPerBlock = 4;                       // rows (one wave each) per workgroup

size_t align256(size_t n) { return (n + 255) / 256 * 256; }

struct WideRows {
    AttnShape s;
    float *x;            // (items, rows, S) scores in, P (forward / backward) out
    float *y;            // backward: (items, rows, S) dP in, dS out
    const float *lse_in; // backward: the forward's lse (B, H, L)
    const float *dsum;   // backward: rowsum(dO * O) (B, H, L)
    float *lse_out;      // forward: lse (B, H, L)
    int row0, rows;      // this block's rows of every item
};

// Row r of the block: its item, (b, h, l), and the (B, H, L) index of its lse / dsum.
struct RowId {
    int64_t item, b, h, l, bhl;
};
DEVI RowId row_id(const WideRows &w, int64_t g) {
    const AttnShape &s = w.s;
    RowId r;
    r.item = g / w.rows;
    const int64_t j = w.row0 + g % w.rows;
    r.b = r.item / s.Hkv;
    r.h = (r.item % s.Hkv) * s.repeat + j / s.L;
    r.l = j % s.L;
    r.bhl = (r.b * s.H + r.h) * s.L + r.l;
    return r;
}

// scale * S + mask with causal (top-left) keys past the query at -inf.
DEVI float score(const WideRows &w, const RowId &r, const float *mrow, int key, float raw) {
    if (w.s.causal && key > r.l) return -INFINITY;
    const float x = raw * w.s.scale;
    return mrow ? x + mrow[key] : x;
}

DEVI float wave_max(float x) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) x = fmaxf(x, __shfl_xor(x, o, 64));
    return x;
}
DEVI float wave_sum(float x) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) x += __shfl_xor(x, o, 64);
    return x;
}

DEVI const float *mask_row(const WideRows &w, const RowId &r) {
    const AttnShape &s = w.s;
    return s.mask ? s.mask + r.b * s.msb + r.h * s.msh + r.l * s.msl : nullptr;
}

// Forward: P = exp(x - lse) for x = scale * S + mask (causal), lse = max + ln(sum exp(x - max));
// a row with no visible key gives P = 0 and lse = 0.  One wave per row.
__global__ __launch_bounds__(64 * kRowsPerBlock) void wide_softmax_kernel(WideRows w) {
    const int64_t g = (int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
    if (g >= (int64_t)w.s.B * w.s.Hkv * w.rows) return;  // whole waves exit together
    const int lane = threadIdx.x & 63, S = w.s.S;
    const RowId r = row_id(w, g);
    const float *mrow = mask_row(w, r);
    float *x = w.x + g * S;
    float mx = -INFINITY;
    for (int key = lane; key < S; key += 64) {
        const float v = score(w, r, mrow, key, x[key]);
        x[key] = v;
        mx = fmaxf(mx, v);
    }
    mx = wave_max(mx);
    float lse = 0.f;
    if (mx != -INFINITY) {
        float sum = 0.f;
        for (int key = lane; key < S; key += 64) sum += expf(x[key] - mx);
        lse = mx + logf(wave_sum(sum));
    }
    for (int key = lane; key < S; key += 64) x[key] = mx == -INFINITY ? 0.f : expf(x[key] - lse);
    if (lane == 0) w.lse_out[r.bhl] = lse;
}

// The same with the row in registers (NV values per lane, rows of at most 64 NV keys): one read
// and one write of the row instead of three reads and two writes.
template <int NV>
__global__ __launch_bounds__(64 * kRowsPerBlock) void wide_softmax_reg_kernel(WideRows w) {
    const int64_t g = (int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
    if (g >= (int64_t)w.s.B * w.s.Hkv * w.rows) return;  // whole waves exit together
    const int lane = threadIdx.x & 63, S = w.s.S;
    const RowId r = row_id(w, g);
    const float *mrow = mask_row(w, r);
    float *x = w.x + g * S;
    float v[NV];
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int key = 64 * i + lane;
        v[i] = key < S ? score(w, r, mrow, key, x[key]) : -INFINITY;
        mx = fmaxf(mx, v[i]);
    }
    mx = wave_max(mx);
    float lse = 0.f;
    if (mx != -INFINITY) {
        float sum = 0.f;
#pragma unroll
        for (int i = 0; i < NV; ++i) sum += expf(v[i] - mx);
        lse = mx + logf(wave_sum(sum));
    }
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int key = 64 * i + lane;
        if (key < S) x[key] = mx == -INFINITY ? 0.f : expf(v[i] - lse);
    }
    if (lane == 0) w.lse_out[r.bhl] = lse;
}

// Backward: P = exp(scale * S + mask - lse) (causal keys past the query: 0).
__global__ __launch_bounds__(64 * kRowsPerBlock) void wide_p_kernel(WideRows w) {
    const int64_t g = (int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
    if (g >= (int64_t)w.s.B * w.s.Hkv * w.rows) return;
    const int lane = threadIdx.x & 63, S = w.s.S;
    const RowId r = row_id(w, g);
    const float *mrow = mask_row(w, r);
    const float lse = w.lse_in[r.bhl];
    float *x = w.x + g * S;
    // Causal keys past the query get 0 after the exponential, as in the reference (:363-367), so
    // that a NaN lse leaves them 0.
    for (int key = lane; key < S; key += 64)
        x[key] = w.s.causal && key > r.l ? 0.f : expf(score(w, r, mrow, key, x[key]) - lse);
}

// Backward: dS = scale * P * (dP - dsum), over the dP buffer.
__global__ __launch_bounds__(64 * kRowsPerBlock) void wide_ds_kernel(WideRows w) {
    const int64_t g = (int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
    if (g >= (int64_t)w.s.B * w.s.Hkv * w.rows) return;
    const int lane = threadIdx.x & 63, S = w.s.S;
    const RowId r = row_id(w, g);
    const float dsum = w.dsum[r.bhl];
    const float *p = w.x + g * S;
    float *y = w.y + g * S;
    // Keys past the query (causal) get 0 without reading dP: its tiles past the diagonal are
    // not computed (the score products skip them).
    for (int key = lane; key < S; key += 64)
        y[key] = w.s.causal && key > r.l ? 0.f : w.s.scale * (p[key] * (y[key] - dsum));
}

template <typename Src, typename Dst>
__global__ __launch_bounds__(256) void cast_kernel(const Src *src, Dst *dst, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
        dst[i] = from_f32<Dst>(to_f32<Src>(src[i]));
}

__global__ __launch_bounds__(256) void fill_zero_kernel(float *p, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) p[i] = 0.f;
}

dim3 grid_for(int64_t n) {
    const int64_t b = (n + 255) / 256;
    return dim3((unsigned)(b < 65536 ? (b > 0 ? b : 1) : 65536));
}

template <typename Src, typename Dst>
hipError_t cast(const void *src, void *dst, int64_t n, hipStream_t st) {
    if (n == 0) return hipSuccess;
    return launch(cast_kernel<Src, Dst>, grid_for(n), dim3(256), st, static_cast<const Src *>(src),
                  static_cast<Dst *>(dst), n);
}

hipError_t zero(float *p, int64_t n, hipStream_t st) {
    if (n == 0) return hipSuccess;
    return launch(fill_zero_kernel, grid_for(n), dim3(256), st, p, n);
}

// One batched product over the items of a row block: C (+)= A B, m x k times k x n.
// causal: 0, or the mode of BmmArgs::causal_mode for a product over the block's rows (row0 + m,
// or row0 + k in mode 3, of each item); taken only for causal attention.
hipError_t product(int items, int m, int n, int k, const float *a, int64_t sab, int64_t sam, int64_t sak,
                   const float *b, int64_t sbb, int64_t sbk, int64_t sbn, float *c, int64_t scb, int64_t scm,
                   bool acc, hipStream_t st, int causal = 0, const AttnShape *s = nullptr, int64_t row0 = 0) {
    BmmArgs g{};
    g.a = a, g.b = b, g.c = c;
    g.batch = items, g.m = m, g.n = n, g.k = k;
    g.sab = sab, g.sam = sam, g.sak = sak, g.sbb = sbb, g.sbk = sbk, g.sbn = sbn;
    g.scb = scb, g.scm = scm, g.acc = acc;
    if (causal && s && s->causal && s->L > 0) g.causal_mode = causal, g.causal_L = s->L, g.causal_row0 = (int)row0;
    return launch_bmm(g, st);
}

// Sizes shared by the workspace queries and the launchers.
struct Geometry {
    int64_t items, M;                    // (batch, kv head) items, rows per item (repeat * L)
    size_t nq, nk;                       // elements of q (and out, dO, dq) and of k (v, dk, dv)
    size_t fixed;                        // bytes before the score buffers
    size_t row_bytes;                    // bytes of one row of every score buffer
};
Geometry geometry(const AttnShape &s, bool bf16, bool backward) {
    Geometry g;
    g.items = (int64_t)s.B * s.Hkv;
    g.M = (int64_t)s.repeat * s.L;
    g.nq = (size_t)s.B * s.H * s.L * s.E;
    g.nk = (size_t)s.B * s.Hkv * s.S * s.E;
    size_t f = 0;
    if (bf16) {  // float32 copies of the inputs and float32 outputs (rounded to bf16 at the end)
        f += align256(g.nq * 4) + 2 * align256(g.nk * 4);                        // q, k, v
        f += backward ? align256(g.nq * 4) + align256(g.nq * 4) + 2 * align256(g.nk * 4)  // dO, dq, dk, dv
                      : align256(g.nq * 4);                                        // out
    }
    g.fixed = f;
    g.row_bytes = (backward ? 2 : 1) * (size_t)g.items * s.S * 4;
    return g;
}

}  // namespace

size_t wide_ws_bytes(const AttnShape &s, bool bf16, bool backward) {
    const Geometry g = geometry(s, bf16, backward);
    int64_t rows = g.row_bytes ? (int64_t)(kRowBlockBytes * (backward ? 2 : 1) / g.row_bytes) : g.M;
    rows = rows < 1 ? 1 : (rows > g.M ? g.M : rows);
    return g.fixed + align256((size_t)rows * g.row_bytes) + 256;
}

int64_t wide_rows(const AttnShape &s, bool bf16, bool backward, size_t bytes) {
    const Geometry g = geometry(s, bf16, backward);
    if (bytes < g.fixed + 256 + g.row_bytes) return 0;
    if (g.row_bytes == 0) return g.M > 0 ? g.M : 1;  // no keys: nothing is buffered
    int64_t rows = (int64_t)((bytes - g.fixed - 256) / g.row_bytes);
    return rows > g.M ? g.M : rows;
}

hipError_t launch_wide_fwd(const FwdArgs &a, bool bf16, void *ws, size_t bytes, hipStream_t st) {
    const AttnShape &s = a.s;
    const Geometry g = geometry(s, bf16, false);
    const int64_t R = wide_rows(s, bf16, false, bytes);
    record_schedule(materialized_rows, (int)R);
    if (R <= 0) return hipErrorInvalidValue;  // the ABI checked the workspace
    char *p = static_cast<char *>(ws);
    const float *q = static_cast<const float *>(a.q), *k = static_cast<const float *>(a.k),
                *v = static_cast<const float *>(a.v);
    float *out = static_cast<float *>(a.out);
    if (bf16) {
        float *qf = reinterpret_cast<float *>(p);
        float *kf = reinterpret_cast<float *>(p + align256(g.nq * 4));
        float *vf = reinterpret_cast<float *>(p + align256(g.nq * 4) + align256(g.nk * 4));
        out = reinterpret_cast<float *>(p + align256(g.nq * 4) + 2 * align256(g.nk * 4));
        return_if((cast<__bf16, float>(a.q, qf, g.nq, st)));
        return_if((cast<__bf16, float>(a.k, kf, g.nk, st)));
        return_if((cast<__bf16, float>(a.v, vf, g.nk, st)));
        q = qf, k = kf, v = vf;
    }
    float *sbuf = reinterpret_cast<float *>(p + g.fixed);
    const int E = s.E, S = s.S;
    const int64_t ME = g.M * E, SE = (int64_t)S * E;
    for (int64_t row0 = 0; row0 < g.M; row0 += R) {
        const int rows = (int)(g.M - row0 < R ? g.M - row0 : R);
        // S = Q K^T (K^T: the transposed view of k)
        // (causal: tiles whose keys all lie past their queries are skipped; the softmax never
        // reads those scores)
        return_if(product((int)g.items, rows, S, E, q + row0 * E, ME, E, 1, k, SE, 1, E, sbuf, (int64_t)rows * S, S,
                          false, st, 1, &s, row0));
        WideRows w{};
        w.s = s, w.x = sbuf, w.lse_out = a.lse, w.row0 = (int)row0, w.rows = rows;
        const int64_t nrows = g.items * rows;
        const dim3 rgrid((unsigned)((nrows + kRowsPerBlock - 1) / kRowsPerBlock)), rblock(64 * kRowsPerBlock);
        if (S <= 512) return_if(launch(wide_softmax_reg_kernel<8>, rgrid, rblock, st, w));
        else if (S <= 1024) return_if(launch(wide_softmax_reg_kernel<16>, rgrid, rblock, st, w));
        else if (S <= 2048) return_if(launch(wide_softmax_reg_kernel<32>, rgrid, rblock, st, w));
        else if (S <= 4096) return_if(launch(wide_softmax_reg_kernel<64>, rgrid, rblock, st, w));
        else return_if(launch(wide_softmax_kernel, rgrid, rblock, st, w));
        // O = P V (causal: keys up to each row tile's last query)
        return_if(product((int)g.items, rows, E, S, sbuf, (int64_t)rows * S, S, 1, v, SE, E, 1, out + row0 * E, ME,
                          E, false, st, 2, &s, row0));
    }
    if (bf16) return_if((cast<float, __bf16>(out, a.out, g.nq, st)));
    return hipSuccess;
}

hipError_t launch_wide_bwd(const BwdArgs &a, bool bf16, void *ws, size_t bytes, hipStream_t st) {
    const AttnShape &s = a.s;
    const Geometry g = geometry(s, bf16, true);
    const int64_t R = wide_rows(s, bf16, true, bytes);
    record_schedule(materialized_rows, (int)R);
    if (R <= 0) return hipErrorInvalidValue;
    char *p = static_cast<char *>(ws);
    const float *q = static_cast<const float *>(a.q), *k = static_cast<const float *>(a.k),
                *v = static_cast<const float *>(a.v), *dout = static_cast<const float *>(a.dout);
    float *dq = static_cast<float *>(a.dq), *dk = static_cast<float *>(a.dk), *dv = static_cast<float *>(a.dv);
    const int64_t nrows = (int64_t)s.B * s.H * s.L;  // dsum = rowsum(dO * O), in the input dtype
    if (nrows > 0) {
        if (bf16) return_if(launch(bwd_pre_kernel<__bf16, false>, dim3((unsigned)((nrows + 15) / 16)), dim3(256), st, a));
        else return_if(launch(bwd_pre_kernel<float, false>, dim3((unsigned)((nrows + 15) / 16)), dim3(256), st, a));
    }
    if (bf16) {
        size_t at = 0;
        auto take = [&](size_t n) {
            float *r = reinterpret_cast<float *>(p + at);
            at += align256(n * 4);
            return r;
        };
        float *qf = take(g.nq), *kf = take(g.nk), *vf = take(g.nk), *dof = take(g.nq);
        dq = take(g.nq), dk = take(g.nk), dv = take(g.nk);
        return_if((cast<__bf16, float>(a.q, qf, g.nq, st)));
        return_if((cast<__bf16, float>(a.k, kf, g.nk, st)));
        return_if((cast<__bf16, float>(a.v, vf, g.nk, st)));
        return_if((cast<__bf16, float>(a.dout, dof, g.nq, st)));
        q = qf, k = kf, v = vf, dout = dof;
    }
    return_if(zero(dk, (int64_t)g.nk, st));
    return_if(zero(dv, (int64_t)g.nk, st));
    float *sbuf = reinterpret_cast<float *>(p + g.fixed);
    float *pbuf = sbuf + (size_t)g.items * R * s.S;
    const int E = s.E, S = s.S;
    const int64_t ME = g.M * E, SE = (int64_t)S * E;
    for (int64_t row0 = 0; row0 < g.M; row0 += R) {
        const int rows = (int)(g.M - row0 < R ? g.M - row0 : R);
        const int64_t RS = (int64_t)rows * S;
        const float *qb = q + row0 * E, *ob = dout + row0 * E;
        WideRows w{};
        w.s = s, w.x = sbuf, w.y = pbuf, w.lse_in = a.lse, w.dsum = a.dsum, w.row0 = (int)row0, w.rows = rows;
        const dim3 rgrid((unsigned)((g.items * rows + kRowsPerBlock - 1) / kRowsPerBlock)), rblock(64 * kRowsPerBlock);
        // S = Q K^T, then P in place
        return_if(product((int)g.items, rows, S, E, qb, ME, E, 1, k, SE, 1, E, sbuf, RS, S, false, st, 1, &s, row0));
        return_if(launch(wide_p_kernel, rgrid, rblock, st, w));
        // dV += P^T dO (P^T: the transposed view of the block's P)
        return_if(product((int)g.items, S, E, rows, sbuf, RS, 1, S, ob, ME, E, 1, dv, SE, E, true, st, 3, &s, row0));
        // dP = dO V^T, then dS = scale P (dP - dsum) in place
        return_if(product((int)g.items, rows, S, E, ob, ME, E, 1, v, SE, 1, E, pbuf, RS, S, false, st, 1, &s, row0));
        return_if(launch(wide_ds_kernel, rgrid, rblock, st, w));
        // dQ = dS K (the block's rows), dK += dS^T Q
        return_if(product((int)g.items, rows, E, S, pbuf, RS, S, 1, k, SE, E, 1, dq + row0 * E, ME, E, false, st, 2,
                          &s, row0));
        return_if(product((int)g.items, S, E, rows, pbuf, RS, 1, S, qb, ME, E, 1, dk, SE, E, true, st, 3, &s, row0));
    }
    if (bf16) {
        return_if((cast<float, __bf16>(dq, a.dq, g.nq, st)));
        return_if((cast<float, __bf16>(dk, a.dk, g.nk, st)));
        return_if((cast<float, __bf16>(dv, a.dv, g.nk, st)));
    }
    return hipSuccess;
}

}  // namespace dc
