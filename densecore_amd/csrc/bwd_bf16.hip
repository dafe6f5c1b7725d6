// bfloat16 attention backward (fp32 accumulation) on CDNA4 MFMA (v_mfma_f32_32x32x16_bf16).
//
// Same mathematics as the float32 backward and DenseCore's torch_attention::backward
// (src/torch_attention.rs:286-468) on bf16 inputs; everything accumulates in float32 and P
// and dS enter their products as two bf16 terms each (hi = bf16(x), lo = bf16(x - hi)), so
// they are carried to about 2^-17.  dK and dV are written as bf16; dQ is accumulated in a
// float32 workspace with atomics and converted at the end.
//
// Blocking (per workgroup: 128 keys of one (batch, kv head), 4 waves x 32 keys):
//   * K and V rows of the wave's keys stay in VGPRs as bf16x8 B operands;
//   * each step stages 32 queries of Q and dO in LDS twice: as rows ([query][d], A operands of
//     S = Q K^T and dP = dO V^T) and transposed ([d][query], A operands of dV^T = dO^T P and
//     dK^T = Q^T dS).  The transpose is done in registers on 4x8 blocks, as in the forward;
//   * the next step's Q and dO blocks are loaded into registers while a step computes;
//   * dQ = dS K: the four waves write dS (hi and lo) into one shared 32 x 128 LDS tile, and after
//     the next barrier each wave multiplies its share of it by the workgroup's K tile (kept
//     transposed in LDS, [d][key]) into disjoint 16 x 16 blocks of dQ, one global atomic per
//     element per workgroup step.
#include "bwd_common.hpp"
#include "common.hpp"
#include "params.hpp"

namespace dc {
namespace {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kBN = 32 * kWaves;
constexpr int kBM = 32;

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

DEVI uint32_t pack_lo(uint32_t a, uint32_t b) { return __builtin_amdgcn_perm(b, a, 0x05040100u); }
DEVI uint32_t pack_hi(uint32_t a, uint32_t b) { return __builtin_amdgcn_perm(b, a, 0x07060302u); }

template <int D>
struct alignas(16) BwdSmemBf16 {
    __bf16 qn[kBM][D + 8];
    __bf16 don[kBM][D + 8];
    __bf16 qt[D][kBM + 4];
    __bf16 dot[D][kBM + 4];
    __bf16 kt[D][kBN + 8];
    __bf16 ds[2][kBM][kBN + 8];  // dS of the step as hi and lo bf16 parts, all four waves' keys
    float lse[kBM];
    float dsum[kBM];
};

// 16 bytes (8 bf16) of row `row` at column c of a (rows, E) bf16 matrix, zero outside.
DEVI u32x4 load8(const __bf16 *base, int row, int rows, int c, int E, bool vec, int D) {
    if (vec && row < rows) return *reinterpret_cast<const u32x4 *>(base + (int64_t)row * D + c);
    u32x4 x = {0u, 0u, 0u, 0u};
    if (row < rows) {
        uint16_t h[8];
#pragma unroll
        for (int e = 0; e < 8; ++e)
            h[e] = c + e < E ? __builtin_bit_cast(uint16_t, base[(int64_t)row * E + c + e]) : (uint16_t)0;
#pragma unroll
        for (int w = 0; w < 4; ++w) x[w] = (uint32_t)h[2 * w] | ((uint32_t)h[2 * w + 1] << 16);
    }
    return x;
}

// Writes a 4-row x 8-column block (rows r0..r0+3, columns c..c+7) both as rows of `nat`
// and as columns of `tr` (tr[c + e][r0 .. r0 + 3]).
template <int NS, int TS>
DEVI void store_block(__bf16 (*nat)[NS], __bf16 (*tr)[TS], const u32x4 (&v)[4], int r0, int c) {
#pragma unroll
    for (int u = 0; u < 4; ++u) *reinterpret_cast<u32x4 *>(&nat[r0 + u][c]) = v[u];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        const u32x2 even = {pack_lo(v[0][w], v[1][w]), pack_lo(v[2][w], v[3][w])};
        const u32x2 odd = {pack_hi(v[0][w], v[1][w]), pack_hi(v[2][w], v[3][w])};
        *reinterpret_cast<u32x2 *>(&tr[c + 2 * w][r0]) = even;
        *reinterpret_cast<u32x2 *>(&tr[c + 2 * w + 1][r0]) = odd;
    }
}

// One step's Q and dO as 4x8 blocks in registers (loaded during the previous step).
template <int D>
struct QStageBf16 {
    static constexpr int QBLK = (kBM / 4) * (D / 8);  // blocks per tensor
    static constexpr int N = (2 * QBLK + kThreads - 1) / kThreads;
    u32x4 v[N][4];
    float lse, dsum;

    DEVI void load(const __bf16 *qb, const __bf16 *gb, const float *lseb, const float *dsumb,
                   int m0, int L, int E, bool vec, int tid) {
#pragma unroll
        for (int j = 0; j < N; ++j) {
            const int blk = tid + kThreads * j;
            const bool isq = blk < QBLK;
            const int bi = isq ? blk : blk - QBLK;
            const int r0 = (bi / (D / 8)) * 4, c = (bi % (D / 8)) * 8;
#pragma unroll
            for (int u = 0; u < 4; ++u)
                v[j][u] = blk < 2 * QBLK ? load8(isq ? qb : gb, m0 + r0 + u, L, c, E, vec, D)
                                         : u32x4{0u, 0u, 0u, 0u};
        }
        if (tid < kBM) {
            const int qq = m0 + tid;
            lse = qq < L ? lseb[qq] : INFINITY;
            dsum = qq < L ? dsumb[qq] : 0.f;
        }
    }
    DEVI void store(BwdSmemBf16<D> &sm, int tid) const {
#pragma unroll
        for (int j = 0; j < N; ++j) {
            const int blk = tid + kThreads * j;
            if (blk >= 2 * QBLK) continue;
            const bool isq = blk < QBLK;
            const int bi = isq ? blk : blk - QBLK;
            const int r0 = (bi / (D / 8)) * 4, c = (bi % (D / 8)) * 8;
            if (isq)
                store_block(sm.qn, sm.qt, v[j], r0, c);
            else
                store_block(sm.don, sm.dot, v[j], r0, c);
        }
        if (tid < kBM) sm.lse[tid] = lse, sm.dsum[tid] = dsum;
    }
};

// dQ[m0 .. m0+31][:] += scale * dS K for the step whose dS (hi, lo) is in sm.ds: the 32 x D
// tile is split into 16 x 16 blocks, D/32 per wave, each reduced over `nkeys` keys with
// v_mfma_f32_16x16x32_bf16 (lane l supplies A[l%16][8(l/16)..+7], B[8(l/16)..+7][l%16] and
// holds C[4(l/16) + v][l%16]); one global atomic per element per workgroup step.
template <int D>
DEVI void dq_product(const BwdSmemBf16<D> &sm, float *dqb, int m0, int nkeys, int L, int E,
                     float scale, int wave, int lane) {
    constexpr int TPW = D / 32;
    const int r16 = lane & 15, c4 = lane >> 4;
    const int qh = wave >> 1, dbase = (wave & 1) * (D / 2);
    f32x4 acc[TPW];
#pragma unroll
    for (int j = 0; j < TPW; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
    const int steps = (nkeys + 31) / 32;
    for (int st = 0; st < steps; ++st) {
        const int kc = 32 * st + 8 * c4;
        const bf16x8 ah = *reinterpret_cast<const bf16x8 *>(&sm.ds[0][qh * 16 + r16][kc]);
        const bf16x8 al = *reinterpret_cast<const bf16x8 *>(&sm.ds[1][qh * 16 + r16][kc]);
#pragma unroll
        for (int j = 0; j < TPW; ++j) {
            const bf16x8 kk = *reinterpret_cast<const bf16x8 *>(&sm.kt[dbase + 16 * j + r16][kc]);
            acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, kk, acc[j], 0, 0, 0);
            acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, kk, acc[j], 0, 0, 0);
        }
    }
#pragma unroll
    for (int j = 0; j < TPW; ++j) {
        const int d = dbase + 16 * j + r16;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int qq = m0 + qh * 16 + 4 * c4 + v;
            if (qq < L && d < E) unsafeAtomicAdd(dqb + (int64_t)qq * E + d, acc[j][v] * scale);
        }
    }
}

template <int D, bool CAUSAL, bool MASK>
__global__ __launch_bounds__(kThreads) void bwd_bf16_kernel(BwdArgs a) {
    constexpr int KS = D / 16;
    constexpr int NDT = D / 32;
    __shared__ BwdSmemBf16<D> sm;

    const AttnShape &s = a.s;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, lr = lane & 31, g = lane >> 5;
    const int BHk = s.B * s.Hkv;
    const int bid = blockIdx.x;
    const int ktile = bid / BHk;
    const int bhk = bid % BHk, b = bhk / s.Hkv, hk = bhk % s.Hkv;
    const int n0 = ktile * kBN;
    const int kw0 = n0 + wave * 32;
    const int key = kw0 + lr;
    const int D_ = D;

    const __bf16 *kb = static_cast<const __bf16 *>(a.k) + (int64_t)bhk * s.S * s.E;
    const __bf16 *vb = static_cast<const __bf16 *>(a.v) + (int64_t)bhk * s.S * s.E;

    bf16x8 kreg[KS], vreg[KS];
#pragma unroll
    for (int t = 0; t < KS; ++t) {
        const u32x4 x = load8(kb, key, s.S, 16 * t + 8 * g, s.E, s.vec, D_);
        const u32x4 y = load8(vb, key, s.S, 16 * t + 8 * g, s.E, s.vec, D_);
        kreg[t] = __builtin_bit_cast(bf16x8, x);
        vreg[t] = __builtin_bit_cast(bf16x8, y);
    }
    // The workgroup's K tile, transposed: kt[d][key - n0].
    for (int blk = tid; blk < (kBN / 4) * (D / 8); blk += kThreads) {
        const int r0 = (blk / (D / 8)) * 4, c = (blk % (D / 8)) * 8;
        u32x4 v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) v[u] = load8(kb, n0 + r0 + u, s.S, c, s.E, s.vec, D_);
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const u32x2 even = {pack_lo(v[0][w], v[1][w]), pack_lo(v[2][w], v[3][w])};
            const u32x2 odd = {pack_hi(v[0][w], v[1][w]), pack_hi(v[2][w], v[3][w])};
            *reinterpret_cast<u32x2 *>(&sm.kt[c + 2 * w][r0]) = even;
            *reinterpret_cast<u32x2 *>(&sm.kt[c + 2 * w + 1][r0]) = odd;
        }
    }

    f32x16 dk[NDT], dv[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) dk[dt][r] = 0.f, dv[dt][r] = 0.f;

    const int m_begin = CAUSAL ? (n0 / kBM) * kBM : 0;
    const int per_head = s.L > m_begin ? (s.L - m_begin + kBM - 1) / kBM : 0;
    const int nsteps = per_head * s.repeat;
    const int key_end = min(kBN, s.S - n0);
    auto step_head = [&](int i) { return b * s.H + hk * s.repeat + i / per_head; };
    auto step_m0 = [&](int i) { return m_begin + (i % per_head) * kBM; };
    auto step_keys = [&](int m0) { return CAUSAL ? max(0, min(key_end, m0 + kBM - n0)) : key_end; };
    auto qptr = [&](int bh) { return static_cast<const __bf16 *>(a.q) + (int64_t)bh * s.L * s.E; };
    auto gptr = [&](int bh) { return static_cast<const __bf16 *>(a.dout) + (int64_t)bh * s.L * s.E; };

    QStageBf16<D> stage;
    if (nsteps > 0) {
        const int bh = step_head(0);
        stage.load(qptr(bh), gptr(bh), a.lse + (int64_t)bh * s.L, a.dsum + (int64_t)bh * s.L,
                   step_m0(0), s.L, s.E, s.vec, tid);
    }
    int prev_bh = -1, prev_m0 = 0;
    for (int i = 0; i < nsteps; ++i) {
        const int bh = step_head(i), h = bh - b * s.H, m0 = step_m0(i);
        __syncthreads();  // the previous step's readers of Q/dO and writers of dS are done
        if (prev_bh >= 0)
            dq_product<D>(sm, a.dq_acc + (int64_t)prev_bh * s.L * s.E, prev_m0, step_keys(prev_m0),
                          s.L, s.E, s.scale, wave, lane);
        stage.store(sm, tid);
        __syncthreads();  // staged, and the previous dQ product has read sm.ds
        if (i + 1 < nsteps) {
            const int nbh = step_head(i + 1);
            stage.load(qptr(nbh), gptr(nbh), a.lse + (int64_t)nbh * s.L, a.dsum + (int64_t)nbh * s.L,
                       step_m0(i + 1), s.L, s.E, s.vec, tid);
        }
        prev_bh = bh, prev_m0 = m0;

        const bool live = kw0 < s.S && (!CAUSAL || m0 + kBM - 1 >= kw0);
        if (!live) continue;
        const float *mbase = MASK ? s.mask + (int64_t)b * s.msb + (int64_t)h * s.msh : nullptr;

        f32x16 sacc, pacc;
#pragma unroll
        for (int r = 0; r < 16; ++r) sacc[r] = 0.f, pacc[r] = 0.f;
#pragma unroll
        for (int t = 0; t < KS; ++t) {
            const bf16x8 qa = *reinterpret_cast<const bf16x8 *>(&sm.qn[lr][16 * t + 8 * g]);
            const bf16x8 oa = *reinterpret_cast<const bf16x8 *>(&sm.don[lr][16 * t + 8 * g]);
            sacc = mfma_bf16(qa, kreg[t], sacc);
            pacc = mfma_bf16(oa, vreg[t], pacc);
        }

        const bool edge = kw0 + 31 >= s.S || (CAUSAL && kw0 + 31 > m0);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int qrow = acc_row(r, g), qq = m0 + qrow;
            // scale * q.k (+ mask) - lse in natural-log units, as the reference forms it,
            // then one conversion to base 2 for v_exp_f32.
            float x = sacc[r] * s.scale;
            if (MASK) x += (qq < s.L && key < s.S) ? mbase[(int64_t)qq * s.msl + key] : 0.f;
            float p = exp2_fast((x - sm.lse[qrow]) * kLog2e);
            if (edge && (key >= s.S || (CAUSAL && key > qq))) p = 0.f;
            sacc[r] = p;
            pacc[r] = p * (pacc[r] - sm.dsum[qrow]);
            const __bf16 hv = static_cast<__bf16>(pacc[r]);
            sm.ds[0][qrow][wave * 32 + lr] = hv;
            sm.ds[1][qrow][wave * 32 + lr] = static_cast<__bf16>(pacc[r] - static_cast<float>(hv));
        }

        // dV^T += dO^T P and dK^T += Q^T dS: 16 queries per MFMA, registers 8u..8u+7 hold
        // queries 16u + {4g..4g+3, 8+4g..8+4g+3}.
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            bf16x8 ph, pl, sh, sl;
            split_bf16(sacc, 8 * u, ph, pl);
            split_bf16(pacc, 8 * u, sh, sl);
            const int qc = 16 * u + 4 * g;
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt) {
                const bf16x4 olo = *reinterpret_cast<const bf16x4 *>(&sm.dot[dt * 32 + lr][qc]);
                const bf16x4 ohi = *reinterpret_cast<const bf16x4 *>(&sm.dot[dt * 32 + lr][qc + 8]);
                const bf16x4 qlo = *reinterpret_cast<const bf16x4 *>(&sm.qt[dt * 32 + lr][qc]);
                const bf16x4 qhi = *reinterpret_cast<const bf16x4 *>(&sm.qt[dt * 32 + lr][qc + 8]);
                const bf16x8 oa = {olo[0], olo[1], olo[2], olo[3], ohi[0], ohi[1], ohi[2], ohi[3]};
                const bf16x8 qa = {qlo[0], qlo[1], qlo[2], qlo[3], qhi[0], qhi[1], qhi[2], qhi[3]};
                dv[dt] = mfma_bf16(oa, ph, dv[dt]);
                dv[dt] = mfma_bf16(oa, pl, dv[dt]);
                dk[dt] = mfma_bf16(qa, sh, dk[dt]);
                dk[dt] = mfma_bf16(qa, sl, dk[dt]);
            }
        }
    }
    __syncthreads();
    if (prev_bh >= 0)
        dq_product<D>(sm, a.dq_acc + (int64_t)prev_bh * s.L * s.E, prev_m0, step_keys(prev_m0), s.L,
                      s.E, s.scale, wave, lane);

    if (key < s.S) {
        __bf16 *dkr = static_cast<__bf16 *>(a.dk) + ((int64_t)bhk * s.S + key) * s.E;
        __bf16 *dvr = static_cast<__bf16 *>(a.dv) + ((int64_t)bhk * s.S + key) * s.E;
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
            for (int r = 0; r < 16; r += 4) {
                const int d = dt * 32 + acc_row(r, g);
                if (s.vec) {
                    const bf16x4 kx = {static_cast<__bf16>(dk[dt][r] * s.scale),
                                       static_cast<__bf16>(dk[dt][r + 1] * s.scale),
                                       static_cast<__bf16>(dk[dt][r + 2] * s.scale),
                                       static_cast<__bf16>(dk[dt][r + 3] * s.scale)};
                    const bf16x4 vx = {static_cast<__bf16>(dv[dt][r]), static_cast<__bf16>(dv[dt][r + 1]),
                                       static_cast<__bf16>(dv[dt][r + 2]), static_cast<__bf16>(dv[dt][r + 3])};
                    *reinterpret_cast<bf16x4 *>(dkr + d) = kx;
                    *reinterpret_cast<bf16x4 *>(dvr + d) = vx;
                } else {
#pragma unroll
                    for (int u = 0; u < 4; ++u)
                        if (d + u < s.E) {
                            dkr[d + u] = static_cast<__bf16>(dk[dt][r + u] * s.scale);
                            dvr[d + u] = static_cast<__bf16>(dv[dt][r + u]);
                        }
                }
            }
    }
}

template <int D>
hipError_t launch_d(const BwdArgs &args, hipStream_t st) {
    BwdArgs a = args;
    a.s.vec = args.s.vec && args.s.E == D;
    const int nkt = (a.s.S + kBN - 1) / kBN;
    const dim3 grid(nkt * a.s.B * a.s.Hkv), block(kThreads);
    const bool mask = a.s.mask != nullptr;
    if (a.s.causal && mask)
        return_if(launch(bwd_bf16_kernel<D, true, true>, grid, block, st, a));
    else if (a.s.causal)
        return_if(launch(bwd_bf16_kernel<D, true, false>, grid, block, st, a));
    else if (mask)
        return_if(launch(bwd_bf16_kernel<D, false, true>, grid, block, st, a));
    else
        return_if(launch(bwd_bf16_kernel<D, false, false>, grid, block, st, a));
    return hipSuccess;
}

}  // namespace

hipError_t launch_bwd_bf16(const BwdArgs &a, hipStream_t st) {
    const int64_t rows = (int64_t)a.s.B * a.s.H * a.s.L;
    if (rows > 0) {
        return_if(launch(bwd_pre_kernel<__bf16>, dim3((rows + 15) / 16), dim3(256), st, a));
    }
    if (a.s.B * a.s.Hkv > 0 && a.s.S > 0) {
        hipError_t e;
        if (a.s.E <= 32)
            e = launch_d<32>(a, st);
        else if (a.s.E <= 64)
            e = launch_d<64>(a, st);
        else
            e = launch_d<128>(a, st);
        if (e != hipSuccess) return e;
    }
    const int64_t n = rows * a.s.E;
    if (n > 0) {
        return_if(launch(bwd_dq_convert_kernel<__bf16>, dim3((n + 255) / 256), dim3(256), st, a, n));
        return hipSuccess;
    }
    return hipSuccess;
}

}  // namespace dc
