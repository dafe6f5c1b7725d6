// Float32 attention backward on CDNA4 MFMA (v_mfma_f32_32x32x2_f32).
//
// Computes what DenseCore's torch_attention::backward computes (src/torch_attention.rs:286-468):
//   dsum = rowsum(dO * O);  P = exp(scale * q k^T + mask - lse) (0 where causal-masked);
//   dV += P^T dO;  dP = dO V^T;  dS = P * (dP - dsum);  dQ += scale dS K;  dK += scale dS^T Q,
// accumulating over the query heads that share a kv head (:321-324).  The blocking is its own:
//
//   * a workgroup owns 128 keys of one (batch, kv head); each of its 4 waves owns 32 keys and
//     keeps them in VGPRs (K and V as MFMA B operands) together with its dK^T and dV^T
//     accumulators, for the whole sweep over query tiles;
//   * each step stages a 32-query tile of Q and dO (plus lse and dsum) in LDS;
//   * S and dP are computed with queries as rows and this wave's keys as columns, so P and dS
//     feed dV^T += dO^T P and dK^T += Q^T dS directly from the accumulators;
//   * dQ needs dS with queries on lanes: each wave bounces its 32x32 dS tile through a private
//     LDS tile, multiplies by its K rows (also kept in LDS) and adds the 32 x D partial into a
//     float32 dQ accumulator with coalesced global atomics.
// A small pre-kernel computes dsum and clears the dQ accumulator.
#include "bwd_common.hpp"
#include "common.hpp"
#include "params.hpp"

namespace dc {
namespace {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kBN = 32 * kWaves;  // keys per workgroup
constexpr int kBM = 32;           // queries per step

template <int D>
struct BwdSmem {
    float k[kBN][D + 4];
    float q[kBM][D + 4];
    float dout[kBM][D + 4];
    float lse[kBM];
    float dsum[kBM];
    float ds[kWaves][32][36];
};

template <int D, bool CAUSAL, bool MASK>
__global__ __launch_bounds__(kThreads) void bwd_f32_kernel(BwdArgs a) {
    constexpr int DH = D / 2;
    constexpr int NDT = D / 32;
    __shared__ BwdSmem<D> sm;

    const AttnShape &s = a.s;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, lr = lane & 31, g = lane >> 5;
    const int BHk = s.B * s.Hkv;
    const int bid = blockIdx.x;
    const int kt = bid / BHk;  // kv tile; tile 0 has the most causal work, so it goes first
    const int bhk = bid % BHk, b = bhk / s.Hkv, hk = bhk % s.Hkv;
    const int n0 = kt * kBN;
    const int kw0 = n0 + wave * 32;  // this wave's first key
    const int key = kw0 + lr;        // this lane's key column

    const float *kb = static_cast<const float *>(a.k) + (int64_t)bhk * s.S * s.E;
    const float *vb = static_cast<const float *>(a.v) + (int64_t)bhk * s.S * s.E;

    // K and V rows of this lane's key: K[key][g*DH + t], V[key][g*DH + t].
    float kreg[DH], vreg[DH];
    {
        const float *kr = kb + (int64_t)key * s.E, *vr = vb + (int64_t)key * s.E;
        if (s.vec && key < s.S) {
#pragma unroll
            for (int t = 0; t < DH; t += 4) {
                const f32x4 x = *reinterpret_cast<const f32x4 *>(kr + g * DH + t);
                const f32x4 y = *reinterpret_cast<const f32x4 *>(vr + g * DH + t);
#pragma unroll
                for (int u = 0; u < 4; ++u) kreg[t + u] = x[u], vreg[t + u] = y[u];
            }
        } else {
#pragma unroll
            for (int t = 0; t < DH; ++t) {
                const int d = g * DH + t;
                const bool ok = key < s.S && d < s.E;
                kreg[t] = ok ? kr[d] : 0.f;
                vreg[t] = ok ? vr[d] : 0.f;
            }
        }
    }
    // The workgroup's K tile in LDS, read with lanes along the head dim by the dQ product.
    for (int i = tid; i < kBN * D; i += kThreads) {
        const int r = i / D, c = i % D, kk = n0 + r;
        sm.k[r][c] = (kk < s.S && c < s.E) ? kb[(int64_t)kk * s.E + c] : 0.f;
    }

    f32x16 dk[NDT], dv[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) dk[dt][r] = 0.f, dv[dt][r] = 0.f;

    const int m_begin = CAUSAL ? (n0 / kBM) * kBM : 0;
    for (int rep = 0; rep < s.repeat; ++rep) {
        const int h = hk * s.repeat + rep;
        const int bh = b * s.H + h;
        const float *qb = static_cast<const float *>(a.q) + (int64_t)bh * s.L * s.E;
        const float *gb = static_cast<const float *>(a.dout) + (int64_t)bh * s.L * s.E;
        const float *mbase = MASK ? s.mask + (int64_t)b * s.msb + (int64_t)h * s.msh : nullptr;
        float *dqb = a.dq_acc + (int64_t)bh * s.L * s.E;

        for (int m0 = m_begin; m0 < s.L; m0 += kBM) {
            __syncthreads();  // previous step's readers are done
            for (int i = tid; i < kBM * D; i += kThreads) {
                const int r = i / D, c = i % D, qq = m0 + r;
                const bool ok = qq < s.L && c < s.E;
                sm.q[r][c] = ok ? qb[(int64_t)qq * s.E + c] : 0.f;
                sm.dout[r][c] = ok ? gb[(int64_t)qq * s.E + c] : 0.f;
            }
            if (tid < kBM) {
                const int qq = m0 + tid;
                sm.lse[tid] = qq < s.L ? a.lse[(int64_t)bh * s.L + qq] : INFINITY;
                sm.dsum[tid] = qq < s.L ? a.dsum[(int64_t)bh * s.L + qq] : 0.f;
            }
            __syncthreads();

            // A wave has work if some query of the tile sees one of its keys.
            const bool live = kw0 < s.S && (!CAUSAL || m0 + kBM - 1 >= kw0);
            if (!live) continue;

            // S = Q K^T and dP = dO V^T: rows are queries, columns are this wave's keys.
            f32x16 sacc, pacc;
#pragma unroll
            for (int r = 0; r < 16; ++r) sacc[r] = 0.f, pacc[r] = 0.f;
#pragma unroll
            for (int t4 = 0; t4 < DH; t4 += 4) {
                const f32x4 qq = *reinterpret_cast<const f32x4 *>(&sm.q[lr][g * DH + t4]);
                const f32x4 oo = *reinterpret_cast<const f32x4 *>(&sm.dout[lr][g * DH + t4]);
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    sacc = mfma_f32(qq[u], kreg[t4 + u], sacc);
                    pacc = mfma_f32(oo[u], vreg[t4 + u], pacc);
                }
            }

            // P and dS, elementwise in the accumulator layout.
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int qrow = acc_row(r, g), qq = m0 + qrow;
                // scale * q.k (+ mask) - lse in natural-log units, as the reference forms it,
                // then one conversion to base 2 for v_exp_f32.
                float x = sacc[r] * s.scale;
                if (MASK) x += (qq < s.L && key < s.S) ? mbase[(int64_t)qq * s.msl + key] : 0.f;
                float p = exp2_fast((x - sm.lse[qrow]) * kLog2e);
                if (key >= s.S || (CAUSAL && key > qq)) p = 0.f;
                sacc[r] = p;
                pacc[r] = p * (pacc[r] - sm.dsum[qrow]);
            }

            // dV^T += dO^T P and dK^T += Q^T dS (reduction over this tile's queries).
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int qrow = acc_row(r, g);
                    dv[dt] = mfma_f32(sm.dout[qrow][dt * 32 + lr], sacc[r], dv[dt]);
                    dk[dt] = mfma_f32(sm.q[qrow][dt * 32 + lr], pacc[r], dk[dt]);
                }

            // dQ (queries x D) += dS K over this wave's 32 keys, via a private LDS transpose.
            float(*ds)[36] = sm.ds[wave];
#pragma unroll
            for (int r = 0; r < 16; ++r) ds[acc_row(r, g)][lr] = pacc[r];
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the tile is in LDS
            __builtin_amdgcn_wave_barrier();
            f32x16 dq[NDT];
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
                for (int r = 0; r < 16; ++r) dq[dt][r] = 0.f;
#pragma unroll
            for (int s4 = 0; s4 < 4; ++s4) {
                const f32x4 dsv = *reinterpret_cast<const f32x4 *>(&ds[lr][8 * s4 + 4 * g]);
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const int kk = wave * 32 + 8 * s4 + 4 * g + u;
#pragma unroll
                    for (int dt = 0; dt < NDT; ++dt)
                        dq[dt] = mfma_f32(dsv[u], sm.k[kk][dt * 32 + lr], dq[dt]);
                }
            }
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt) {
                const int d = dt * 32 + lr;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int qq = m0 + acc_row(r, g);
                    if (qq < s.L && d < s.E)
                        unsafeAtomicAdd(dqb + (int64_t)qq * s.E + d, dq[dt][r] * s.scale);
                }
            }
        }
    }

    // dK = scale * dK^T^T, dV = dV^T^T for this lane's key.
    if (key < s.S) {
        float *dkr = static_cast<float *>(a.dk) + ((int64_t)bhk * s.S + key) * s.E;
        float *dvr = static_cast<float *>(a.dv) + ((int64_t)bhk * s.S + key) * s.E;
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
            for (int r = 0; r < 16; r += 4) {
                const int d = dt * 32 + acc_row(r, g);
                if (s.vec) {
                    *reinterpret_cast<f32x4 *>(dkr + d) =
                        f32x4{dk[dt][r] * s.scale, dk[dt][r + 1] * s.scale,
                              dk[dt][r + 2] * s.scale, dk[dt][r + 3] * s.scale};
                    *reinterpret_cast<f32x4 *>(dvr + d) =
                        f32x4{dv[dt][r], dv[dt][r + 1], dv[dt][r + 2], dv[dt][r + 3]};
                } else {
#pragma unroll
                    for (int u = 0; u < 4; ++u)
                        if (d + u < s.E) {
                            dkr[d + u] = dk[dt][r + u] * s.scale;
                            dvr[d + u] = dv[dt][r + u];
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
        return_if(launch(bwd_f32_kernel<D, true, true>, grid, block, st, a));
    else if (a.s.causal)
        return_if(launch(bwd_f32_kernel<D, true, false>, grid, block, st, a));
    else if (mask)
        return_if(launch(bwd_f32_kernel<D, false, true>, grid, block, st, a));
    else
        return_if(launch(bwd_f32_kernel<D, false, false>, grid, block, st, a));
    return hipSuccess;
}

}  // namespace

hipError_t launch_bwd_f32(const BwdArgs &a, hipStream_t st) {
    const int64_t rows = (int64_t)a.s.B * a.s.H * a.s.L;
    if (rows > 0) {
        return_if(launch(bwd_pre_kernel<float>, dim3((rows + 15) / 16), dim3(256), st, a));
    }
    if (a.s.B * a.s.Hkv == 0 || a.s.S == 0) return hipSuccess;
    if (a.s.E <= 32) return launch_d<32>(a, st);
    if (a.s.E <= 64) return launch_d<64>(a, st);
    return launch_d<128>(a, st);
}

}  // namespace dc
