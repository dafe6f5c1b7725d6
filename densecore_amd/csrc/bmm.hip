// Float32 batched matrix product on CDNA4 MFMA (v_mfma_f32_32x32x2_f32): C[b] = A[b] B[b].
//
// The reference registers one bmm kernel, (Cpu, Float32) (src/batched_matmul.rs:28-49), which runs
// PyTorch's bmm on the operands' strided storage (src/torch_blas.rs:404-449): A is (batch, m, k),
// B is (batch, k, n), each read through its own element strides (a transposed view is just other
// strides), and C is a fresh row-major (batch, m, n).  This is the device entry of that table: the
// math attention path's two products (q k^T, a transposed view of k, and weights v) and MHA's.
//
// Blocking (this kernel's own): a workgroup of 4 waves computes a BM x BN tile of one batch item
// (waves 2 x 2, each (BM/2) x (BN/2) as 32 x 32 MFMA tiles), over k in steps of BK.  A and B
// tiles are staged in LDS k-major ([k][m], [k][n]), so an MFMA operand is 32 consecutive floats
// per half-wave (lane l takes A[m = l % 32][k = l / 32] and B[k = l / 32][n = l % 32]).  Global
// loads follow the operand's contiguous dimension: 16-byte loads along m or n are stored as they
// are; 16-byte loads along k are stored transposed (lanes along m or n, conflict-free); other
// layouts load one element per lane.  The next k tile is loaded into registers while the current
// one is multiplied (one barrier per k tile).  Where every tile has the same k extent (no causal
// trimming of k) BK = 16: half the LDS of BK = 32, so four workgroups run per CU and four waves per
// SIMD hide the loads' latency (on one MI355X, 32 items of 2048 x 256 x 2048: 705 -> 598 us; 256
// items of 512 x 64 x 512: 148 -> 134 us).  Products whose tiles stop k at the diagonal (causal
// modes 2 and 3) keep BK = 32 and two workgroups per CU: their longest tiles set the time, and
// sharing a SIMD four ways slowed them (D = 256 causal P V 529 -> 610 us).  Accumulation is
// float32 (the reference sums the products in k order; here the MFMA's order, within the float32
// tolerance).  The launcher also serves the attention path of head dims above 128 (wide.hip),
// which writes C through strides and can add A B into C.
#include "common.hpp"
#include "params.hpp"

namespace dc {
namespace {

constexpr int kThreads = 256;
constexpr int kPad = 4;  // LDS row padding (floats): keeps 16-byte stores aligned

template <int BM, int BN, int BK>
struct alignas(16) BmmSmem {
    float a[2][BK][BM + kPad];
    float b[2][BK][BN + kPad];
};

// How an operand's tile is loaded: CONTIG_K: 16-byte loads along k (stored transposed);
// CONTIG_MN: 16-byte loads along m (A) or n (B); SCALAR: one element per lane, any strides.
enum Layout { CONTIG_K = 0, CONTIG_MN = 1, SCALAR = 2 };

// The register stage of one operand tile: R rows (m or n) by BK, from `p` (the batch item's base)
// with strides (s_r along the rows, s_k along k); rows past `rows` and k past `kk` read zero.
template <int R, int L, int BK>
struct Stage {
    static constexpr int N = R * BK / (L == SCALAR ? 1 : 4) / kThreads;
    static_assert(N >= 1, "tile too small for the workgroup");
    f32x4 v[L == SCALAR ? 1 : N];
    float s[L == SCALAR ? N : 1];

    DEVI void load(const float *p, int64_t s_r, int64_t s_k, int r0, int rows, int k0, int kk, int tid) {
        if constexpr (L == CONTIG_K) {
#pragma unroll
            for (int j = 0; j < N; ++j) {
                const int i = tid + kThreads * j, r = i % R, c = (i / R) * 4;  // lanes along rows
                const int rr = r0 + r, k = k0 + c;
                v[j] = (rr < rows && k < kk) ? *reinterpret_cast<const f32x4 *>(p + rr * s_r + k)
                                             : f32x4{0.f, 0.f, 0.f, 0.f};
            }
        } else if constexpr (L == CONTIG_MN) {
#pragma unroll
            for (int j = 0; j < N; ++j) {
                const int i = tid + kThreads * j, c = (i % (R / 4)) * 4, k = i / (R / 4);
                const int rr = r0 + c, kg = k0 + k;
                v[j] = (rr < rows && kg < kk) ? *reinterpret_cast<const f32x4 *>(p + kg * s_k + rr)
                                              : f32x4{0.f, 0.f, 0.f, 0.f};
            }
        } else {
#pragma unroll
            for (int j = 0; j < N; ++j) {
                const int i = tid + kThreads * j, r = i % R, k = i / R;
                const int rr = r0 + r, kg = k0 + k;
                s[j] = (rr < rows && kg < kk) ? p[rr * s_r + kg * s_k] : 0.f;
            }
        }
    }
    DEVI void store(float (*t)[R + kPad], int tid) const {
        if constexpr (L == CONTIG_K) {
#pragma unroll
            for (int j = 0; j < N; ++j) {
                const int i = tid + kThreads * j, r = i % R, c = (i / R) * 4;
#pragma unroll
                for (int u = 0; u < 4; ++u) t[c + u][r] = v[j][u];
            }
        } else if constexpr (L == CONTIG_MN) {
#pragma unroll
            for (int j = 0; j < N; ++j) {
                const int i = tid + kThreads * j, c = (i % (R / 4)) * 4, k = i / (R / 4);
                *reinterpret_cast<f32x4 *>(&t[k][c]) = v[j];
            }
        } else {
#pragma unroll
            for (int j = 0; j < N; ++j) {
                const int i = tid + kThreads * j, r = i % R, k = i / R;
                t[k][r] = s[j];
            }
        }
    }
};

template <int BM, int BN, int LA, int LB, int BK>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(BK == 16 ? 4 : 2, BK == 16 ? 4 : 2))) void bmm_f32_kernel(BmmArgs g) {
    constexpr int TM = BM / 64, TN = BN / 64;  // 32 x 32 MFMA tiles per wave along m, n
    static_assert(TM >= 1 && TN >= 1, "a wave covers at least 32 x 32");
    __shared__ BmmSmem<BM, BN, BK> sm;
    const int tid = threadIdx.x, lane = tid & 63, lr = lane & 31, gh = lane >> 5;
    const int wave = tid >> 6, wm = wave >> 1, wn = wave & 1;
    const int mt = (g.m + BM - 1) / BM, nt = (g.n + BN - 1) / BN, per = mt * nt;
    // The tiles of one batch item run on one XCD (workgroup w goes to XCD w % 8), so its A and B
    // panels are read from one L2.
    const int n = gridDim.x, bid = blockIdx.x;
    const int w = (n & 7) == 0 ? (bid & 7) * (n >> 3) + (bid >> 3) : bid;
    const int bt = w / per, r = w % per, m0 = (r / nt) * BM, n0 = (r % nt) * BN;
    const float *ap = g.a + (int64_t)bt * g.sab;
    const float *bp = g.b + (int64_t)bt * g.sbb;
    // Causal products: the largest query index among rows [r0, r1] of the block (rows across a
    // head boundary: L - 1).
    auto max_query = [&](int r0, int r1) {
        const int64_t j0 = (int64_t)g.causal_row0 + r0, j1 = (int64_t)g.causal_row0 + r1;
        return j0 / g.causal_L != j1 / g.causal_L ? g.causal_L - 1 : (int)(j1 % g.causal_L);
    };
    int kk = g.k;
    if (g.causal_mode == 1 && n0 > max_query(m0, min(m0 + BM, g.m) - 1)) return;  // no key visible
    if (g.causal_mode == 2) kk = min(kk, max_query(m0, min(m0 + BM, g.m) - 1) + 1);
    const int nk = (kk + BK - 1) / BK;
    // The first k tile at or after kt that contributes (mode 3: some row of it sees key m0).
    auto next_live = [&](int kt) {
        if (g.causal_mode == 3)
            while (kt < nk && max_query(kt * BK, min((kt + 1) * BK, g.k) - 1) < m0) ++kt;
        return kt;
    };

    Stage<BM, LA, BK> sa;
    Stage<BN, LB, BK> sb;
    int kt = next_live(0);
    // B's "rows" are its n columns: its row stride is the n stride, its k stride the k stride.
    sa.load(ap, g.sam, g.sak, m0, g.m, kt * BK, kk, tid);
    sb.load(bp, g.sbn, g.sbk, n0, g.n, kt * BK, kk, tid);
    sa.store(sm.a[0], tid);
    sb.store(sm.b[0], tid);
    __syncthreads();

    f32x16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

    for (int buf = 0; kt < nk; buf ^= 1) {
        const int next = next_live(kt + 1);
        if (next < nk) {
            sa.load(ap, g.sam, g.sak, m0, g.m, next * BK, kk, tid);
            sb.load(bp, g.sbn, g.sbk, n0, g.n, next * BK, kk, tid);
        }
        const float(*ta)[BM + kPad] = sm.a[buf];
        const float(*tb)[BN + kPad] = sm.b[buf];
#pragma unroll
        for (int k = 0; k < BK; k += 2) {
            float fa[TM], fb[TN];
#pragma unroll
            for (int i = 0; i < TM; ++i) fa[i] = ta[k + gh][wm * (BM / 2) + 32 * i + lr];
#pragma unroll
            for (int j = 0; j < TN; ++j) fb[j] = tb[k + gh][wn * (BN / 2) + 32 * j + lr];
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j) acc[i][j] = mfma_f32(fa[i], fb[j], acc[i][j]);
        }
        if (next < nk) {
            sa.store(sm.a[buf ^ 1], tid);
            sb.store(sm.b[buf ^ 1], tid);
        }
        __syncthreads();
        kt = next;
    }

    float *cp = g.c + (int64_t)bt * g.scb;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int col = n0 + wn * (BN / 2) + 32 * j + lr;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int row = m0 + wm * (BM / 2) + 32 * i + acc_row(e, gh);
                if (row < g.m && col < g.n) {
                    float *dst = cp + (int64_t)row * g.scm + col;
                    *dst = g.acc ? *dst + acc[i][j][e] : acc[i][j][e];
                }
            }
        }
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// The load layout of an operand: contig (the stride that is 1), its extent along that dimension,
// and the other strides must all keep 16-byte chunks aligned.
int layout_a(const BmmArgs &g) {
    if (!aligned16(g.a) || g.sab % 4) return SCALAR;
    if (g.sak == 1 && g.k % 4 == 0 && g.sam % 4 == 0) return CONTIG_K;
    if (g.sam == 1 && g.m % 4 == 0 && g.sak % 4 == 0) return CONTIG_MN;
    return SCALAR;
}
int layout_b(const BmmArgs &g) {
    if (!aligned16(g.b) || g.sbb % 4) return SCALAR;
    if (g.sbk == 1 && g.k % 4 == 0 && g.sbn % 4 == 0) return CONTIG_K;
    if (g.sbn == 1 && g.n % 4 == 0 && g.sbk % 4 == 0) return CONTIG_MN;
    return SCALAR;
}

template <int BM, int BN, int LA, int BK>
hipError_t launch_b(const BmmArgs &g, int lb, dim3 grid, hipStream_t st) {
    if (lb == CONTIG_K) return launch(bmm_f32_kernel<BM, BN, LA, CONTIG_K, BK>, grid, dim3(kThreads), st, g);
    if (lb == CONTIG_MN) return launch(bmm_f32_kernel<BM, BN, LA, CONTIG_MN, BK>, grid, dim3(kThreads), st, g);
    return launch(bmm_f32_kernel<BM, BN, LA, SCALAR, BK>, grid, dim3(kThreads), st, g);
}

template <int BM, int BN, int BK>
hipError_t launch_k(const BmmArgs &g, hipStream_t st) {
    const int64_t tiles = (int64_t)((g.m + BM - 1) / BM) * ((g.n + BN - 1) / BN) * g.batch;
    const dim3 grid((unsigned)tiles);
    const int la = layout_a(g), lb = layout_b(g);
    if (la == CONTIG_K) return launch_b<BM, BN, CONTIG_K, BK>(g, lb, grid, st);
    if (la == CONTIG_MN) return launch_b<BM, BN, CONTIG_MN, BK>(g, lb, grid, st);
    return launch_b<BM, BN, SCALAR, BK>(g, lb, grid, st);
}

// BK = 16 (four workgroups per CU) unless the causal mode trims k per tile.
template <int BM, int BN>
hipError_t launch_t(const BmmArgs &g, hipStream_t st) {
    return g.causal_mode >= 2 ? launch_k<BM, BN, 32>(g, st) : launch_k<BM, BN, 16>(g, st);
}

// Zeroes C when k == 0 (the reference returns zeros); C is (batch, m, n) through its strides.
__global__ __launch_bounds__(256) void bmm_zero_kernel(BmmArgs g) {
    const int64_t count = (int64_t)g.batch * g.m * g.n;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < count; i += (int64_t)gridDim.x * 256) {
        const int64_t bt = i / ((int64_t)g.m * g.n), r = i % ((int64_t)g.m * g.n);
        g.c[bt * g.scb + (r / g.n) * g.scm + r % g.n] = 0.f;
    }
}

}  // namespace

hipError_t launch_bmm(const BmmArgs &g, hipStream_t st) {
    if (g.batch == 0 || g.m == 0 || g.n == 0) return hipSuccess;
    if (g.k == 0) {
        if (g.acc) return hipSuccess;
        const int64_t count = (int64_t)g.batch * g.m * g.n;
        const int64_t blocks = (count + 255) / 256 < 65536 ? (count + 255) / 256 : 65536;
        return launch(bmm_zero_kernel, dim3((unsigned)blocks), dim3(256), st, g);
    }
    // 128 x 64 tiles when n is narrow (the weights-times-v product of attention, n = head dim).
    if (g.n <= 64) return launch_t<128, 64>(g, st);
    return launch_t<128, 128>(g, st);
}

}  // namespace dc
