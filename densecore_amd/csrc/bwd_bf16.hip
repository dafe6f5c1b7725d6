// bfloat16 attention backward (fp32 accumulation) on CDNA4 MFMA (v_mfma_f32_32x32x16_bf16).
//
// Same mathematics as the float32 backward and DenseCore's torch_attention::backward
// (src/torch_attention.rs:286-468) on bf16 inputs:
//   dsum = rowsum(dO * O);  P = exp(scale * q k^T + mask - lse) (0 where causal-masked);
//   dV = P^T dO;  dP = dO V^T;  dS = P * (dP - dsum);  dQ = scale dS K;  dK = scale dS^T Q,
// accumulating over the query heads that share a kv head (:321-324).  Everything accumulates
// in float32.  The products run in one of two forms:
//   * with the workspace's fp16 copies (the default): q, k, v and dO are copied to fp16, each
//     (batch, kv head) slab scaled by a power of two (exact for its bf16 values, f16_stage.hip);
//     P and dS are rounded once to fp16 (2^-12), and an MFMA block in which some P exceeds kLoP
//     also takes the rounding error of its P and dS as a second fp16 term (about 2^-22);
//   * without them (a workspace of dsum alone): the bf16 inputs themselves, with P and dS as two
//     bf16 terms each (hi = bf16(x), lo = bf16(x - hi)), carried to about 2^-17.
// Either way the only bf16 roundings of the results are those of the outputs.
//
// Two kernels, neither with atomics (dQ is deterministic):
//   * bwd_dkdv_bf16_kernel (keys stationary): a workgroup of 8 waves owns 128 keys of one
//     (batch, kv head); waves w and w + 4 own the same 32 keys and split each 64-query step.
//     K and V tiles stay in LDS; per step, Q and dO tiles stream in by global_load_lds while
//     the previous step computes.  S = Q K^T and dP = dO V^T have queries as rows, so P and
//     dS feed dV^T += dO^T P and dK^T += Q^T dS straight from the accumulators, with dO^T and
//     Q^T read from the [query][d] tiles by ds_read_b64_tr_b16.  The two waves' partial dK,
//     dV are summed through LDS at the end.
//   * bwd_dq_bf16_kernel (queries stationary, the forward's structure): a workgroup of 4
//     waves owns 128 queries, keeps Q and dO in VGPRs and streams 64-key K/V tiles;
//     S^T = K Q^T and dP^T = V dO^T have keys as rows, so dS^T feeds dQ^T += K^T dS^T
//     from the accumulator, with K^T read from the [key][d] tile by ds_read_b64_tr_b16.
//     S and dP are computed twice overall (here and in the dK/dV kernel).
// A pre-kernel forms dsum.
//
// LDS tiles are chunk-major: 16-byte chunk c of row r sits at slot c * (R + 4) + r (R rows).
// A row read (lanes = 32 consecutive rows, one chunk) is 512 contiguous bytes, and a
// transposed read (8 rows x 4 chunks x 8 bytes) hits every bank exactly twice; all inner-loop
// addresses are a per-lane base plus a constant.
#include <algorithm>
#include <type_traits>

#include "bwd_common.hpp"
#include "common.hpp"
#include "fwd_split.hpp"
#include "params.hpp"
#include "tile_bf16.hpp"

namespace dc {
namespace {

// ---------------------------------------------------------------------------------------
// dK / dV (keys stationary)
// ---------------------------------------------------------------------------------------
constexpr int kKW = 8;             // waves (head dims up to 128)
constexpr int kKThreads = 64 * kKW;
constexpr int kKN = 128;           // keys per workgroup (head dims up to 128; split grids)
constexpr int kKM = 64;            // queries per step

// The dK/dV workgroup: up to head dim 128, 8 waves over 128 keys with each step's Q and dO tiles
// double-buffered; at 256, where a 64-row tile takes 34 KB, 4 waves over 64 keys with one Q / dO
// buffer: 136 KB of LDS, one workgroup per CU and one wave per SIMD, whose 512 registers hold the
// 2 x 256-dim dK / dV accumulators of its 32 keys.
template <int D>
struct KLayout {
    static constexpr int W = D > 128 ? 4 : kKW;          // waves
    static constexpr int N = 16 * W;                     // keys (32 per pair of waves)
    static constexpr int QB = D > 128 ? 1 : 2;           // Q / dO buffers
    static constexpr int THREADS = 64 * W;
};

template <int D>
struct alignas(16) DkdvSmem {
    using TK = CMTile<KLayout<D>::N, D>;
    using TQ = CMTile<kKM, D>;
    static constexpr int QB = KLayout<D>::QB;
    struct Main {
        u32x4 k[TK::SLOTS];
        u32x4 v[TK::SLOTS];
        u32x4 q[QB][TQ::SLOTS];
        u32x4 o[QB][TQ::SLOTS];
        float lse[QB][kKM];
        float dsum[QB][kKM];
    };
    // End of the sweep: the second wave of each pair hands its partial dK^T, dV^T over.
    struct Red {
        float acc[KLayout<D>::W / 2][2 * (D / 32)][16][64];
    };
    union {
        Main m;
        Red r;
    };
};

// The fp16 mode of both kernels (F16): q, k, v, dout are the fp16 copies, scaled by 2^e_q,
// 2^e_k, 2^e_v, 2^e_do per (b, kv head), and P and dS are rounded once to fp16, so each of the
// P / dS products is one fp16 MFMA instead of the bf16 hi + lo pair.  The scores' scale takes
// 2^-(e_q + e_k), dsum is stored times 2^(e_do + e_v) so that dP - dsum comes out scaled by
// that too, and dS is formed as P (dP - dsum) 2^(e_do + e_v - 24): |dP - dsum| is below
// 2 E max|dO| max|V| (dsum = dO . out with |out| <= max|V|), so this is below 2^14 for E <= 128.
// The outputs take the inverse powers: dV 2^-e_do, dK 2^-(e_q + e_do + e_v - 24), dQ
// 2^-(e_k + e_do + e_v - 24).
struct F16Scales {
    float sc_log2 = 0.f, sc = 0.f;  // scale (base 2 and natural), times 2^-(e_q + e_k)
    int e_pv = 0;                   // e_do + e_v
    int e_q = 0, e_k = 0, e_do = 0;
};

DEVI F16Scales f16_scales(const BwdArgs &a, int bhk) {
    const int n = a.s.B * a.s.Hkv;
    F16Scales f;
    f.e_q = a.exps[bhk], f.e_k = a.exps[n + bhk], f.e_do = a.exps[3 * n + bhk];
    f.e_pv = f.e_do + a.exps[2 * n + bhk];
    f.sc_log2 = ldexpf(a.s.scale_log2, -(f.e_q + f.e_k));
    f.sc = ldexpf(a.s.scale, -(f.e_q + f.e_k));
    return f;
}

// The fp16 products round P and dS once, to 2^-12 of each term.  Where large terms cancel
// (early keys of a long causal row get P ~ 1 / (query + 1) from the nearby queries while their
// dV sums thousands of terms to something small) that rounding alone reaches 1% of rms(dV) at
// L = 8192.  So an MFMA block (16 queries x 32 keys, or 16 keys x 32 queries) in which some P
// exceeds kLoP also multiplies the rounding error of its P and dS (cvt_f16x8_lo) in a second
// product: those terms are then carried to about 2^-22.  On N(0, 1) inputs at C5's shape about
// 1% of the blocks take it (the early queries); the largest dV error falls from 0.97 of the bf16
// bar to 0.16 (float64 simulation of head 7 of C5).
constexpr float kLoP = 0x1p-4f;
// The dK/dV kernel forms P times 2^kPShift (folded into the exponent) so that the low parts of
// P >= kLoP are normal fp16 numbers (>= 2^-2); dV is scaled back at the end (P <= 1, so P times
// 2^14 stays below fp16's largest value even for an lse a few units off).
constexpr int kPShift = 14;
// dS = P (dP - dsum) 2^(e_do + e_v - 24) of the fp16 mode is formed from P 2^kPShift times
// 2^-kDsShift: the kernel computes p 2^(kPShift - kDsShift) = p 2^-24 directly (the exponent
// carries it), and P 2^kPShift from that by 2^kDsShift (exact).
constexpr int kDsShift = kPShift + 24;

template <bool F16>
DEVI f32x16 mfma16(bf16x8 x, bf16x8 y, f32x16 c) {
    if constexpr (F16) return mfma_f16(x, y, c);
    else return mfma_bf16(x, y, c);
}

// Query steps (of kKM queries, over the query heads sharing the kv head) of key tile kt, and the
// pieces of at most `chunk` steps it runs as when split (1 without a split).
__host__ __device__ inline int dkdv_steps(const AttnShape &s, int kt) {
    const int m_begin = s.causal ? kt * kKN : 0;  // a multiple of kKM
    const int per_head = s.L > m_begin ? (s.L - m_begin + kKM - 1) / kKM : 0;
    return per_head * s.repeat;
}
__host__ __device__ inline int dkdv_pieces(const AttnShape &s, int kt, int chunk) {
    if (chunk <= 0) return 1;
    const int n = (dkdv_steps(s, kt) + chunk - 1) / chunk;
    return n > 1 ? n : 1;
}

template <int D, bool CAUSAL, bool MASK, bool VEC, bool F16, bool SPLIT = false>
__global__ __launch_bounds__(KLayout<D>::THREADS) void bwd_dkdv_bf16_kernel(BwdArgs a) {
    constexpr int KSTEP = D / 16, NDT = D / 32;
    constexpr int KW = KLayout<D>::W, KN = KLayout<D>::N, QB = KLayout<D>::QB;
    static_assert(!SPLIT || KN == kKN, "split grids are planned over 128-key tiles");
    __shared__ DkdvSmem<D> sm;

    const AttnShape &s = a.s;
    const int tid = threadIdx.x, lane = tid & 63, lr = lane & 31, g = lane >> 5;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int kw = wave % (KW / 2), qh = wave / (KW / 2);
    const int nkt = (s.S + KN - 1) / KN;
    const int w = logical_block();
    int bhk = w / nkt, kt_ = w % nkt;  // causal: small n0 (most queries) first
    // Split: blocks run over (kv head, key tile, piece), the pieces of a key tile adjacent.
    int piece = 0, npieces = 1;
    if constexpr (SPLIT) {
        int per = 0;
        for (int t = 0; t < nkt; ++t) per += dkdv_pieces(s, t, a.chunk_k);
        bhk = w / per;
        int r = w % per;
        for (kt_ = 0; kt_ < nkt; ++kt_) {
            const int np = dkdv_pieces(s, kt_, a.chunk_k);
            if (r < np) break;
            r -= np;
        }
        if (bhk >= s.B * s.Hkv || kt_ >= nkt) return;  // not reached: the grid holds the pieces
        piece = r, npieces = dkdv_pieces(s, kt_, a.chunk_k);
    }
    const int n0 = kt_ * KN;
    const int b = bhk / s.Hkv, hk = bhk % s.Hkv;
    const int kw0 = n0 + 32 * kw;
    const int key = kw0 + lr;  // this lane's key column

    const __bf16 *kb = static_cast<const __bf16 *>(a.k) + (int64_t)bhk * s.S * s.E;
    const __bf16 *vb = static_cast<const __bf16 *>(a.v) + (int64_t)bhk * s.S * s.E;
    F16Scales fs;
    if constexpr (F16) fs = f16_scales(a, bhk);
    const float sc_log2 = F16 ? fs.sc_log2 : s.scale_log2, sc = F16 ? fs.sc : s.scale;
    const int nkeys = min(KN, s.S - n0);
    fill_cm<KN, D, VEC, KW>(sm.m.k, kb + (int64_t)n0 * s.E, nkeys, s.E, wave, lane);
    fill_cm<KN, D, VEC, KW>(sm.m.v, vb + (int64_t)n0 * s.E, nkeys, s.E, wave, lane);

    const int m_begin = CAUSAL ? n0 : 0;  // n0 is a multiple of kKM
    const int per_head = s.L > m_begin ? (s.L - m_begin + kKM - 1) / kKM : 0;
    const int all_steps = per_head * s.repeat;
    // This block's steps [i_begin, nsteps): all of them, or its piece's.
    const int i_begin = SPLIT ? piece * all_steps / npieces : 0;
    const int nsteps = SPLIT ? (piece + 1) * all_steps / npieces : all_steps;
    auto step_bh = [&](int i) { return b * s.H + hk * s.repeat + i / per_head; };
    auto step_m0 = [&](int i) { return m_begin + (i % per_head) * kKM; };
    auto fill_step = [&](int i) {
        const int bh = step_bh(i), m0 = step_m0(i), buf = i % QB;
        const int rows = min(kKM, s.L - m0);
        const int64_t off = ((int64_t)bh * s.L + m0) * s.E;
        fill_cm<kKM, D, VEC, KW>(sm.m.q[buf], static_cast<const __bf16 *>(a.q) + off, rows, s.E, wave, lane);
        fill_cm<kKM, D, VEC, KW>(sm.m.o[buf], static_cast<const __bf16 *>(a.dout) + off, rows, s.E, wave, lane);
    };
    // -lse log2 e (-inf past L: P = 0 there) and -dsum of a step, one value per lane of waves
    // 0 and 1.  (The float32 kernels subtract lse in natural-log units first, which saves one
    // rounding of size |lse| 2^-24 in the exponent; at bf16 precision it is noise.)  The global
    // load (load_row_raw) and the arithmetic on it (row_stat) are apart so that the next step's
    // load is issued at the top of a step and waited for at its end: computed at once, the value
    // would make waves 0 and 1 wait out the load's latency before their step's work.
    struct RowRaw {
        float x;
        bool in;  // the row is below L
    };
    auto load_row_raw = [&](int i) -> RowRaw {
        const int bh = step_bh(i), qq = step_m0(i) + lane;
        if (qq >= s.L) return {0.f, false};
        return {wave == 0 ? a.lse[(int64_t)bh * s.L + qq] : a.dsum[(int64_t)bh * s.L + qq], true};
    };
    auto row_stat = [&](RowRaw r) -> float {
        if (wave == 0) return r.in ? -r.x * kLog2e + (F16 ? (float)(kPShift - kDsShift) : 0.f) : -INFINITY;
        const float ds = r.in ? -r.x : 0.f;
        return F16 ? ldexpf(ds, fs.e_pv) : ds;
    };
    auto store_row_stat = [&](int i, float x) {
        if (wave == 0) sm.m.lse[i % QB][lane] = x;
        else sm.m.dsum[i % QB][lane] = x;
    };
    if (QB == 2 && i_begin < nsteps) {
        fill_step(i_begin);
        if (wave < 2) store_row_stat(i_begin, row_stat(load_row_raw(i_begin)));
    }

    const uint32_t rowb = row_lanebase<kKM, D>(lane);
    const uint32_t rowbk = row_lanebase<KN, D>(lane);
    const uint32_t trb = tr_lanebase<kKM, D>(lane);

    f32x16 dk[NDT], dv[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) dk[dt][r] = 0.f, dv[dt][r] = 0.f;

    for (int i = i_begin; i < nsteps; ++i) {
        const int bh = step_bh(i), h = bh - b * s.H, m0 = step_m0(i), buf = i % QB;
        RowRaw stat = {0.f, false};
        if constexpr (QB == 2) {
            if (VEC) wait_vmem();
            __syncthreads();  // step i's tiles landed (and K/V at i = 0); step i - 1 is done
            if (i + 1 < nsteps) {
                if (wave < 2) stat = load_row_raw(i + 1);
                fill_step(i + 1);
            }
        } else {
            // One buffer: step i's tiles are loaded once step i - 1 is done with the buffer.
            if (i > i_begin) __syncthreads();
            fill_step(i);
            if (wave < 2) store_row_stat(i, row_stat(load_row_raw(i)));
            if (VEC) wait_vmem();
            __syncthreads();  // step i's tiles landed (and K/V at the first step)
        }

        const int mq = m0 + 32 * qh;  // this wave's 32 queries
        const u32x4 *qt = sm.m.q[buf], *ot = sm.m.o[buf];
        const float *mbase = MASK ? s.mask + (int64_t)b * s.msb + (int64_t)h * s.msh : nullptr;
        const bool live = kw0 < s.S && mq < s.L && (!CAUSAL || mq + 31 >= kw0);
        if (live) {
            // dP accumulates onto -dsum, so the MFMAs leave dP - dsum.  The rows' -lse log2 e are
            // read here too: LDS reads complete in order, and read after the first product
            // group's operands they would make the elementwise work wait for those.
            f32x16 sacc, pacc;
            f32x4 nl[4];
#pragma unroll
            for (int r4 = 0; r4 < 4; ++r4) {
                const int row0 = 32 * qh + 8 * r4 + 4 * g;  // rows of registers 4 r4 .. 4 r4 + 3
                const f32x4 nd = *reinterpret_cast<const f32x4 *>(&sm.m.dsum[buf][row0]);
                nl[r4] = *reinterpret_cast<const f32x4 *>(&sm.m.lse[buf][row0]);
#pragma unroll
                for (int j = 0; j < 4; ++j) sacc[4 * r4 + j] = 0.f, pacc[4 * r4 + j] = nd[j];
            }
            __builtin_amdgcn_sched_barrier(0);  // keep these reads out of the MFMA schedule below
#pragma unroll
            for (int st = 0; st < KSTEP; ++st) {
                sacc = mfma16<F16>(row_frag<kKM, D>(qt, rowb, 32 * qh, st),
                                   row_frag<KN, D>(sm.m.k, rowbk, 32 * kw, st), sacc);
                pacc = mfma16<F16>(row_frag<kKM, D>(ot, rowb, 32 * qh, st),
                                   row_frag<KN, D>(sm.m.v, rowbk, 32 * kw, st), pacc);
            }
            // Keep the operand reads (two per MFMA) four MFMAs ahead of their use.
            sched_reads_ahead<2 * KSTEP, 2, 4>();
            __builtin_amdgcn_sched_barrier(0);

            // dV^T += dO^T P and dK^T += Q^T dS, 16 queries per MFMA, in four groups: (16-query
            // half u = 0, P), (0, dS), (1, P), (1, dS).  A group's transposed operand (dO^T or
            // Q^T) is read while the previous group's MFMAs run; the first one's while P and dS
            // are formed.
            bf16x8 fa[2][NDT];
            auto load_group = [&](int grp, bf16x8 *dst) {
                const u32x4 *t = (grp & 1) ? qt : ot;
#pragma unroll
                for (int dt = 0; dt < NDT; ++dt) dst[dt] = tr_frag<kKM, D>(t, trb, 32 * qh + 16 * (grp >> 1), dt);
            };
            load_group(0, fa[0]);

            // P and dS.  F16: sacc becomes p 2^-24 (the exponent carries kPShift - kDsShift), so
            // that dS = sacc (dP - dsum) needs one multiply, and P 2^kPShift = sacc 2^kDsShift;
            // both are rounded to fp16 in the product groups.  Otherwise sacc = p and pacc = dS.
            // EDGE (keys past S or crossing the diagonal) is a separate instantiation so that the
            // common path carries no per-element masking.
            auto elementwise = [&](auto edge_c) {
                constexpr bool EDGE = decltype(edge_c)::value;
#pragma unroll
                for (int r4 = 0; r4 < 4; ++r4) {
                    const int row0 = 32 * qh + 8 * r4 + 4 * g;
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const int r = 4 * r4 + j, qq = m0 + row0 + j;
                        // exponent in base 2: scale q.k (+ mask) - lse, times log2 e
                        float x;
                        if (MASK) {
                            const float mk = (qq < s.L && key < s.S) ? mbase[(int64_t)qq * s.msl + key] : 0.f;
                            x = fmaf(fmaf(sacc[r], sc, mk), kLog2e, nl[r4][j]);
                        } else {
                            x = fmaf(sacc[r], sc_log2, nl[r4][j]);
                        }
                        if (EDGE && (key >= s.S || (CAUSAL && key > qq))) x = -INFINITY;
                        const float p = exp2_fast(x);
                        sacc[r] = p;
                        if constexpr (!F16) pacc[r] = p * pacc[r];
                    }
                }
            };
            if (kw0 + 31 >= s.S || (CAUSAL && kw0 + 31 > mq)) elementwise(std::true_type{});
            else elementwise(std::false_type{});

            bool lo = false;  // F16: this half's P and dS also enter as their rounding errors
#pragma unroll
            for (int grp = 0; grp < 4; ++grp) {
                const int u = grp >> 1;
                if (grp + 1 < 4) load_group(grp + 1, fa[(grp + 1) & 1]);
                const bf16x8 *f = fa[grp & 1];
                f32x16 *acc = (grp & 1) ? dk : dv;
                bf16x8 ph, pl;
                if constexpr (F16) {
                    if (grp & 1) {
                        ph = cvt_f16x8_prod(sacc, pacc, 8 * u);
                    } else {
                        ph = cvt_f16x8_mul(sacc, 8 * u, 0x1p+38f);
                        lo = any_above_nonneg(sacc, 8 * u, kLoP * 0x1p-24f);
                    }
                } else {
                    split_bf16((grp & 1) ? pacc : sacc, 8 * u, ph, pl);
                }
#pragma unroll
                for (int dt = 0; dt < NDT; ++dt) acc[dt] = mfma16<F16>(f[dt], ph, acc[dt]);
                if (!F16 || lo) {
                    if constexpr (F16) {
                        pl = (grp & 1) ? cvt_f16x8_prod_lo(sacc, pacc, 8 * u, ph)
                                       : cvt_f16x8_mul_lo(sacc, 8 * u, 0x1p+38f, ph);
                    }
#pragma unroll
                    for (int dt = 0; dt < NDT; ++dt) acc[dt] = mfma16<F16>(f[dt], pl, acc[dt]);
                }
            }
        }
        if (QB == 2 && i + 1 < nsteps && wave < 2) store_row_stat(i + 1, row_stat(stat));
    }

    // Sum the two partials of each key group (waves kw and kw + 4) and write dK, dV.  The
    // reduction buffer overlays the tiles: no transfer may still be in flight (with no steps
    // the K/V transfers were never waited for).
    if (VEC) wait_vmem();
    __syncthreads();
    if (qh == 1) {
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                sm.r.acc[kw][dt][r][lane] = dk[dt][r];
                sm.r.acc[kw][NDT + dt][r][lane] = dv[dt][r];
            }
    }
    __syncthreads();
    if (qh == 1 || key >= s.S) return;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            dk[dt][r] += sm.r.acc[kw][dt][r][lane];
            dv[dt][r] += sm.r.acc[kw][NDT + dt][r][lane];
            if constexpr (F16) {  // undo the copies' scales (exact powers of two)
                dk[dt][r] = ldexpf(dk[dt][r], -(fs.e_q + fs.e_pv - 24));
                dv[dt][r] = ldexpf(dv[dt][r], -(fs.e_do + kPShift));
            }
        }
    if (SPLIT && npieces > 1) {
        // A piece: its float32 partials go to slot `piece` of the key's rows
        // (bwd_split_reduce_kernel sums them).
        const size_t nrows = (size_t)s.B * s.Hkv * s.S;
        const int64_t row = (int64_t)bhk * s.S + key;
        float *pk = a.split + ((size_t)piece * nrows + row) * s.E;
        float *pv = a.split + ((size_t)(a.max_k + piece) * nrows + row) * s.E;
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
            for (int r = 0; r < 16; r += 4) {
                const int d = dt * 32 + acc_row(r, g);
#pragma unroll
                for (int u = 0; u < 4; ++u)
                    if (d + u < s.E) {
                        pk[d + u] = dk[dt][r + u] * s.scale;
                        pv[d + u] = dv[dt][r + u];
                    }
            }
        return;
    }
    __bf16 *dkr = static_cast<__bf16 *>(a.dk) + ((int64_t)bhk * s.S + key) * s.E;
    __bf16 *dvr = static_cast<__bf16 *>(a.dv) + ((int64_t)bhk * s.S + key) * s.E;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int r = 0; r < 16; r += 4) {
            const int d = dt * 32 + acc_row(r, g);
            if (VEC) {
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

// ---------------------------------------------------------------------------------------
// dQ (queries stationary)
// ---------------------------------------------------------------------------------------
constexpr int kQW = 4;
constexpr int kQThreads = 64 * kQW;
constexpr int kQM = 32 * kQW;  // queries per workgroup
constexpr int kQN = 64;        // keys per tile

template <int D>
struct alignas(16) DqSmem {
    using T = CMTile<kQN, D>;
    u32x4 k[2][T::SLOTS];
    u32x4 v[2][T::SLOTS];
};

// Waves per SIMD of the dQ kernel: two workgroups per CU up to head dim 128; at 256 its K/V tiles
// take 136 KB of LDS and its Q, dO and dQ registers 256 per lane: one workgroup, one wave per SIMD.
constexpr int dq_waves_per_eu(int D) { return D > 128 ? 1 : 2; }

template <int D, bool CAUSAL, bool MASK, bool VEC, bool F16, bool SPLIT = false>
__global__ __launch_bounds__(kQThreads) __attribute__((amdgpu_waves_per_eu(dq_waves_per_eu(D), dq_waves_per_eu(D)))) void bwd_dq_bf16_kernel(BwdArgs a) {
    constexpr int KSTEP = D / 16, NDT = D / 32, NT = kQN / 32;
    __shared__ DqSmem<D> sm;

    const AttnShape &s = a.s;
    const int tid = threadIdx.x, lane = tid & 63, lr = lane & 31, g = lane >> 5;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nqt = (s.L + kQM - 1) / kQM;
    const int w = logical_block();
    int bh = w / nqt, qt = CAUSAL ? nqt - 1 - w % nqt : w % nqt;
    // Split: blocks run over (head, query tile longest first, piece) (fwd_split.hpp).
    int piece = 0, npieces = 1;
    if constexpr (SPLIT) {
        if (!split_block(s, kQM, kQN, a.chunk_q, w, &qt, &bh, &piece, &npieces)) return;
    }
    const int b = bh / s.H, h = bh % s.H, hk = h / s.repeat;
    const int q0 = qt * kQM;
    const int qi = q0 + wave * 32 + lr;
    const int wave_q0 = q0 + wave * 32, wave_last_q = wave_q0 + 31;

    const __bf16 *kb = static_cast<const __bf16 *>(a.k) + (int64_t)(b * s.Hkv + hk) * s.S * s.E;
    const __bf16 *vb = static_cast<const __bf16 *>(a.v) + (int64_t)(b * s.Hkv + hk) * s.S * s.E;
    F16Scales fs;
    if constexpr (F16) fs = f16_scales(a, b * s.Hkv + hk);
    const float sc_log2 = F16 ? fs.sc_log2 : s.scale_log2, sc = F16 ? fs.sc : s.scale;

    // Q and dO rows of this lane's query as B operands (step t, half g: dims 16t + 8g + 0..7).
    bf16x8 qreg[KSTEP], oreg[KSTEP];
    {
        const int64_t ro = ((int64_t)bh * s.L + qi) * s.E;
        const __bf16 *qrow = static_cast<const __bf16 *>(a.q) + ro;
        const __bf16 *orow = static_cast<const __bf16 *>(a.dout) + ro;
#pragma unroll
        for (int t = 0; t < KSTEP; ++t) {
            const int d0 = 16 * t + 8 * g;
            if (VEC && qi < s.L) {
                qreg[t] = *reinterpret_cast<const bf16x8 *>(qrow + d0);
                oreg[t] = *reinterpret_cast<const bf16x8 *>(orow + d0);
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const bool ok = qi < s.L && d0 + e < s.E;
                    qreg[t][e] = ok ? qrow[d0 + e] : static_cast<__bf16>(0.f);
                    oreg[t][e] = ok ? orow[d0 + e] : static_cast<__bf16>(0.f);
                }
            }
        }
    }
    const float lse_q = qi < s.L ? a.lse[(int64_t)bh * s.L + qi] : 0.f;
    // -lse in base 2.  (The float32 kernels subtract lse in natural-log units first, which
    // saves one rounding of size |lse| 2^-24 in the exponent; at bf16 precision it is noise.)
    // F16: the exponent also carries the 2^-24 of dS = P (dP - dsum) 2^(e_do + e_v - 24), so
    // sacc = 2^x (dP - dsum) needs no further scaling.
    const float nlse2 = -lse_q * kLog2e - (F16 ? 24.f : 0.f);
    float dsum_q = qi < s.L ? a.dsum[(int64_t)bh * s.L + qi] : 0.f;
    if constexpr (F16) dsum_q = ldexpf(dsum_q, fs.e_pv);
    const float *mrow = nullptr;
    if (MASK) mrow = s.mask + (int64_t)b * s.msb + (int64_t)h * s.msh + (int64_t)qi * s.msl;

    f32x16 dq[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) dq[dt][r] = 0.f;

    const int kv_end = CAUSAL ? min(q0 + kQM, s.S) : s.S;
    const int all_tiles = (kv_end + kQN - 1) / kQN;
    // This block's key tiles [t_begin, ntiles): all of them, or its piece's.
    const int t_begin = SPLIT ? piece * all_tiles / npieces : 0;
    const int ntiles = SPLIT ? (piece + 1) * all_tiles / npieces : all_tiles;
    auto fill = [&](int t) {
        const int n0 = t * kQN, rows = min(kQN, s.S - n0);
        fill_cm<kQN, D, VEC, kQW>(sm.k[t & 1], kb + (int64_t)n0 * s.E, rows, s.E, wave, lane);
        fill_cm<kQN, D, VEC, kQW>(sm.v[t & 1], vb + (int64_t)n0 * s.E, rows, s.E, wave, lane);
    };
    if (t_begin < ntiles) fill(t_begin);
    const uint32_t rowb = row_lanebase<kQN, D>(lane);
    const uint32_t trb = tr_lanebase<kQN, D>(lane);

    for (int t = t_begin; t < ntiles; ++t) {
        const int n0 = t * kQN;
        if (VEC) wait_vmem();
        __syncthreads();
        if (t + 1 < ntiles) fill(t + 1);
        const u32x4 *kt_ = sm.k[t & 1], *vt_ = sm.v[t & 1];

        bool live[NT];
#pragma unroll
        for (int kt = 0; kt < NT; ++kt)
            live[kt] = (n0 + kt * 32 < s.S) && (!CAUSAL || n0 + kt * 32 <= wave_last_q);
        float mv[MASK ? NT : 1][16];
        if constexpr (MASK) {
#pragma unroll
            for (int kt = 0; kt < NT; ++kt) {
                bool any_open = false;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int key = n0 + kt * 32 + acc_row(r, g);
                    mv[kt][r] = (live[kt] && key < s.S && qi < s.L) ? mrow[key] : -INFINITY;
                    any_open |= mv[kt][r] != -INFINITY;
                }
                live[kt] = live[kt] && __any(any_open);
            }
        }
        const bool edge = n0 + kQN > s.S || (CAUSAL && n0 + kQN - 1 > wave_q0);

#pragma unroll
        for (int kt = 0; kt < NT; ++kt) {
            if (!live[kt]) continue;
            // Issue priority: a wave raises it for its MFMA stretches and drops it for the
            // elementwise work, so that of the waves sharing a SIMD (two workgroups per CU) the
            // one with MFMAs to issue goes first and the other's VALU work fills in around them
            // (C5: 1646 -> 1530 us with the K^T reads ahead; the dK/dV kernel, whose two waves
            // per SIMD pass the same barriers, measured no difference).
            __builtin_amdgcn_s_setprio(1);
            f32x16 sacc, pacc;
#pragma unroll
            for (int r = 0; r < 16; ++r) sacc[r] = 0.f, pacc[r] = 0.f;
#pragma unroll
            for (int st = 0; st < KSTEP; ++st) {
                sacc = mfma16<F16>(row_frag<kQN, D>(kt_, rowb, 32 * kt, st), qreg[st], sacc);
                pacc = mfma16<F16>(row_frag<kQN, D>(vt_, rowb, 32 * kt, st), oreg[st], pacc);
            }
            // Keep the operand reads (one per MFMA) four MFMAs ahead of their use.
            sched_reads_ahead<2 * KSTEP, 1, 4>();
            __builtin_amdgcn_sched_barrier(0);
            __builtin_amdgcn_s_setprio(0);
            // K^T for dQ^T += K^T dS^T, one 16-key half u at a time.  Without a mask both halves
            // are read here, while dS^T is formed; the masked kernels (whose mask values take 32
            // more registers) read each just before its products.
            bf16x8 fa[2][NDT];
            auto load_fa = [&](int u) {
#pragma unroll
                for (int dt = 0; dt < NDT; ++dt) fa[u][dt] = tr_frag<kQN, D>(kt_, trb, 32 * kt + 16 * u, dt);
            };
            if constexpr (!MASK) load_fa(0), load_fa(1);
            // dS^T; EDGE (keys past S or past the diagonal) is a separate instantiation so
            // that the common path carries no per-element masking.  pm[u]: the largest P 2^-24
            // of the 16-key half u, as bits (P >= 0 orders as an unsigned integer); where some P
            // exceeds kLoP, dS also enters as its rounding error.
            uint32_t pm[2] = {0u, 0u};
            auto elementwise = [&](auto edge_c) {
                constexpr bool EDGE = decltype(edge_c)::value;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    // exponent in base 2: scale q.k (+ mask) - lse, times log2 e
                    float x;
                    if (MASK) x = fmaf(fmaf(sacc[r], sc, mv[kt][r]), kLog2e, nlse2);
                    else x = fmaf(sacc[r], sc_log2, nlse2);
                    if (EDGE) {
                        const int key = n0 + kt * 32 + acc_row(r, g);
                        if (key >= s.S || (CAUSAL && key > qi)) x = -INFINITY;
                    }
                    const float p = exp2_fast(x);
                    if (F16) pm[r >> 3] = max(pm[r >> 3], __float_as_uint(p));
                    sacc[r] = p * (pacc[r] - dsum_q);
                }
            };
            if (edge) elementwise(std::true_type{});
            else elementwise(std::false_type{});
            // dQ^T += K^T dS^T, 16 keys per MFMA.
            __builtin_amdgcn_s_setprio(1);
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                bf16x8 sh, sl;
                bool lo = false;  // F16: this block's dS also enters as its rounding error
                if constexpr (F16) {
                    sh = cvt_f16x8(sacc, 8 * u);
                    lo = __builtin_amdgcn_ballot_w64(pm[u] > __float_as_uint(kLoP * 0x1p-24f)) != 0;
                } else {
                    split_bf16(sacc, 8 * u, sh, sl);
                }
                if constexpr (MASK) load_fa(u);
#pragma unroll
                for (int dt = 0; dt < NDT; ++dt) dq[dt] = mfma16<F16>(fa[u][dt], sh, dq[dt]);
                if (!F16 || lo) {
                    if constexpr (F16) sl = cvt_f16x8_lo(sacc, 8 * u, sh);
#pragma unroll
                    for (int dt = 0; dt < NDT; ++dt) dq[dt] = mfma16<F16>(fa[u][dt], sl, dq[dt]);
                }
            }
        }
    }

    if constexpr (F16) {  // undo the copies' scales (exact powers of two)
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
            for (int r = 0; r < 16; ++r) dq[dt][r] = ldexpf(dq[dt][r], -(fs.e_k + fs.e_pv - 24));
    }
    if (SPLIT && npieces > 1) {
        // A piece: its float32 partial goes to slot `piece` of the query's row
        // (bwd_split_reduce_kernel sums them).
        if (qi < s.L) {
            const size_t nrows = (size_t)s.B * s.H * s.L;
            float *pq = a.split + ((size_t)2 * a.max_k * s.B * s.Hkv * s.S * s.E) +
                        ((size_t)piece * nrows + (int64_t)bh * s.L + qi) * s.E;
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
                for (int r = 0; r < 16; r += 4) {
                    const int d = dt * 32 + acc_row(r, g);
#pragma unroll
                    for (int u = 0; u < 4; ++u)
                        if (d + u < s.E) pq[d + u] = dq[dt][r + u] * s.scale;
                }
        }
        return;
    }
    if (qi < s.L) {
        __bf16 *dqr = static_cast<__bf16 *>(a.dq) + ((int64_t)bh * s.L + qi) * s.E;
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
            for (int r = 0; r < 16; r += 4) {
                const int d = dt * 32 + acc_row(r, g);
                if (VEC) {
                    const bf16x4 o = {static_cast<__bf16>(dq[dt][r] * s.scale),
                                      static_cast<__bf16>(dq[dt][r + 1] * s.scale),
                                      static_cast<__bf16>(dq[dt][r + 2] * s.scale),
                                      static_cast<__bf16>(dq[dt][r + 3] * s.scale)};
                    *reinterpret_cast<bf16x4 *>(dqr + d) = o;
                } else {
#pragma unroll
                    for (int u = 0; u < 4; ++u)
                        if (d + u < s.E) dqr[d + u] = static_cast<__bf16>(dq[dt][r + u] * s.scale);
                }
            }
    }
}

// Sums the float32 partials of split rows in piece order into a bf16 output, one thread per 4
// consecutive dims of a row: rows of dK and dV (`which` 0: key rows, key tile = row % S / kKN) or
// of dQ (`which` 1: query rows, query tile = row % L / kQM).  Rows of tiles that ran whole were
// written by their kernel and are skipped.
__global__ __launch_bounds__(256) void bwd_split_reduce_kernel(BwdArgs a, int which) {
    const AttnShape &s = a.s;
    const int cpr = (s.E + 3) / 4;  // 4-dim groups per row
    const int64_t nrows = which == 0 ? (int64_t)s.B * s.Hkv * s.S : (int64_t)s.B * s.H * s.L;
    const int64_t id = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (id >= nrows * cpr) return;
    const int64_t row = id / cpr;
    const int d0 = (int)(id % cpr) * 4;
    const int np = which == 0 ? dkdv_pieces(s, (int)(row % s.S) / kKN, a.chunk_k)
                              : fwd_pieces(s, kQM, kQN, (int)(row % s.L) / kQM, a.chunk_q);
    if (np <= 1) return;
    const int nout = which == 0 ? 2 : 1;
    const float *base = a.split + (which == 0 ? 0 : (size_t)2 * a.max_k * s.B * s.Hkv * s.S * s.E);
    const bool vec = (s.E & 3) == 0;  // partial rows 16-byte aligned (the workspace is)
    for (int o = 0; o < nout; ++o) {
        const float *src = base + ((size_t)o * a.max_k * nrows + row) * s.E + d0;
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        if (vec) {
#pragma unroll 4
            for (int p = 0; p < np; ++p) acc += *reinterpret_cast<const f32x4 *>(src + (size_t)p * nrows * s.E);
        } else {
            for (int p = 0; p < np; ++p)
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (d0 + e < s.E) acc[e] += src[(size_t)p * nrows * s.E + e];
        }
        __bf16 *dst = static_cast<__bf16 *>(which == 1 ? a.dq : o == 0 ? a.dk : a.dv) + row * s.E + d0;
#pragma unroll
        for (int e = 0; e < 4; ++e)
            if (d0 + e < s.E) dst[e] = static_cast<__bf16>(acc[e]);
    }
}

// The split of both backward grids on the current device (the fp16-copy path without a mask):
// pieces of at least 4 steps (dK/dV) or 4 key tiles (dQ), no more pieces than resident
// workgroups, only for grids that fill at most half of them.
struct BwdSplitPlan {
    int chunk_k = 0, max_k = 1, chunk_q = 0, max_q = 1;
    int64_t blocks_k = 0, blocks_q = 0;
    size_t bytes = 0;
};

template <int D>
BwdSplitPlan plan_bwd(const AttnShape &s) {
    static_assert(D <= 128, "head dims above 128 run whole grids");
    BwdSplitPlan p;
    if (s.mask != nullptr || s.L == 0 || s.S == 0) return p;
    const int nkt = (s.S + kKN - 1) / kKN;
    const int64_t BHk = (int64_t)s.B * s.Hkv;
    const int64_t slots_k = split_slots(
        reinterpret_cast<const void *>(&bwd_dkdv_bf16_kernel<D, true, false, true, true, true>), kKThreads, nkt * BHk);
    if (slots_k > 0 && 2 * nkt * BHk <= slots_k) {
        int64_t steps = 0;
        int most = 0;
        for (int kt = 0; kt < nkt; ++kt) {
            const int n = dkdv_steps(s, kt);
            steps += n;
            most = n > most ? n : most;
        }
        int64_t chunk = (steps * BHk + slots_k - 1) / slots_k;
        for (chunk = chunk < 4 ? 4 : chunk; chunk < most; ++chunk) {
            p.blocks_k = 0;
            for (int kt = 0; kt < nkt; ++kt) p.blocks_k += BHk * dkdv_pieces(s, kt, (int)chunk);
            if (p.blocks_k <= slots_k) break;
        }
        if (chunk < most) {
            p.chunk_k = (int)chunk;
            for (int kt = 0; kt < nkt; ++kt) p.max_k = std::max(p.max_k, dkdv_pieces(s, kt, p.chunk_k));
        }
    }
    const int64_t nqt = (s.L + kQM - 1) / kQM;
    const int64_t slots_q = split_slots(
        reinterpret_cast<const void *>(&bwd_dq_bf16_kernel<D, true, false, true, true, true>), kQThreads,
        nqt * s.B * s.H);
    const FwdSplitPlan q = plan_split(s, kQM, kQN, slots_q);
    p.chunk_q = q.chunk, p.max_q = q.max_pieces, p.blocks_q = q.blocks;
    const size_t kv_rows = p.chunk_k > 0 ? (size_t)2 * p.max_k * BHk * s.S : (size_t)2 * BHk * s.S;
    const size_t q_rows = p.chunk_q > 0 ? (size_t)p.max_q * s.B * s.H * s.L : 0;
    if (p.chunk_k > 0 || p.chunk_q > 0) p.bytes = (kv_rows + q_rows) * s.E * sizeof(float);
    return p;
}

// The split grids and their reductions (the fp16-copy path without a mask).
template <int D, bool VEC>
hipError_t launch_split(const BwdArgs &args, const BwdSplitPlan &p, hipStream_t st) {
    BwdArgs a = args;
    a.chunk_k = p.chunk_k, a.max_k = p.max_k, a.chunk_q = p.chunk_q, a.max_q = p.max_q;
    const bool causal = a.s.causal;
    const dim3 bk(kKThreads), bq(kQThreads), br(256);
    if (p.chunk_k > 0) {
        const dim3 gk((unsigned)p.blocks_k);
        if (causal) return_if(launch(bwd_dkdv_bf16_kernel<D, true, false, VEC, true, true>, gk, bk, st, a));
        else return_if(launch(bwd_dkdv_bf16_kernel<D, false, false, VEC, true, true>, gk, bk, st, a));
        const int64_t n = (int64_t)a.s.B * a.s.Hkv * a.s.S * ((a.s.E + 3) / 4);
        return_if(launch(bwd_split_reduce_kernel, dim3((unsigned)((n + 255) / 256)), br, st, a, 0));
    } else {
        const dim3 gk(((a.s.S + kKN - 1) / kKN) * a.s.B * a.s.Hkv);
        if (causal) return_if(launch(bwd_dkdv_bf16_kernel<D, true, false, VEC, true>, gk, bk, st, a));
        else return_if(launch(bwd_dkdv_bf16_kernel<D, false, false, VEC, true>, gk, bk, st, a));
    }
    if (p.chunk_q > 0) {
        const dim3 gq((unsigned)p.blocks_q);
        if (causal) return_if(launch(bwd_dq_bf16_kernel<D, true, false, VEC, true, true>, gq, bq, st, a));
        else return_if(launch(bwd_dq_bf16_kernel<D, false, false, VEC, true, true>, gq, bq, st, a));
        const int64_t n = (int64_t)a.s.B * a.s.H * a.s.L * ((a.s.E + 3) / 4);
        return launch(bwd_split_reduce_kernel, dim3((unsigned)((n + 255) / 256)), br, st, a, 1);
    }
    const dim3 gq(((a.s.L + kQM - 1) / kQM) * a.s.B * a.s.H);
    if (causal) return launch(bwd_dq_bf16_kernel<D, true, false, VEC, true>, gq, bq, st, a);
    return launch(bwd_dq_bf16_kernel<D, false, false, VEC, true>, gq, bq, st, a);
}

template <int D, bool VEC, bool F16>
hipError_t launch_dvf(const BwdArgs &a, hipStream_t st) {
    const bool mask = a.s.mask != nullptr, causal = a.s.causal;
    constexpr int KN = KLayout<D>::N;
    const dim3 gk(((a.s.S + KN - 1) / KN) * a.s.B * a.s.Hkv), bk(KLayout<D>::THREADS);
    const dim3 gq(((a.s.L + kQM - 1) / kQM) * a.s.B * a.s.H), bq(kQThreads);
    if (a.s.S > 0) {
        if (causal && mask) return_if(launch(bwd_dkdv_bf16_kernel<D, true, true, VEC, F16>, gk, bk, st, a));
        else if (causal) return_if(launch(bwd_dkdv_bf16_kernel<D, true, false, VEC, F16>, gk, bk, st, a));
        else if (mask) return_if(launch(bwd_dkdv_bf16_kernel<D, false, true, VEC, F16>, gk, bk, st, a));
        else return_if(launch(bwd_dkdv_bf16_kernel<D, false, false, VEC, F16>, gk, bk, st, a));
    }
    if (a.s.L > 0) {
        if (causal && mask) return_if(launch(bwd_dq_bf16_kernel<D, true, true, VEC, F16>, gq, bq, st, a));
        else if (causal) return_if(launch(bwd_dq_bf16_kernel<D, true, false, VEC, F16>, gq, bq, st, a));
        else if (mask) return_if(launch(bwd_dq_bf16_kernel<D, false, true, VEC, F16>, gq, bq, st, a));
        else return_if(launch(bwd_dq_bf16_kernel<D, false, false, VEC, F16>, gq, bq, st, a));
    }
    return hipSuccess;
}

// With the fp16 copies: convert (q and dout per group of query heads sharing a kv head, k and
// v per kv head), then run the kernels on the copies.
template <int D, bool VEC>
hipError_t launch_dv(const BwdArgs &a, hipStream_t st) {
    if (!a.q16) return launch_dvf<D, VEC, false>(a, st);
    record_schedule(f16_products, 1);
    const int64_t n = (int64_t)a.s.B * a.s.Hkv;
    const int64_t qslab = (int64_t)a.s.repeat * a.s.L * a.s.E, kslab = (int64_t)a.s.S * a.s.E;
    const F16Copy copies[4] = {{a.q, a.q16, qslab, a.exps},
                               {a.k, a.k16, kslab, a.exps + n},
                               {a.v, a.v16, kslab, a.exps + 2 * n},
                               {a.dout, a.do16, qslab, a.exps + 3 * n}};
    return_if(launch_to_f16(copies, 4, n, a.f16_partial, st));
    BwdArgs f = a;
    f.q = a.q16, f.k = a.k16, f.v = a.v16, f.dout = a.do16;
    if constexpr (D <= 128) {
        if (a.split) {
            const BwdSplitPlan p = plan_bwd<D>(a.s);
            if ((p.chunk_k > 0 || p.chunk_q > 0) && p.bytes <= a.split_bytes) {
                record_schedule(split_chunk_k, p.chunk_k);
                record_schedule(split_chunk_q, p.chunk_q);
                return launch_split<D, VEC>(f, p, st);
            }
        }
    }
    return launch_dvf<D, VEC, true>(f, st);
}

template <int D>
hipError_t launch_d(const BwdArgs &args, hipStream_t st) {
    BwdArgs a = args;
    a.s.vec = args.s.vec && args.s.E == D;
    return a.s.vec ? launch_dv<D, true>(a, st) : launch_dv<D, false>(a, st);
}

}  // namespace

size_t bwd_bf16_split_bytes(const AttnShape &s) {
    if (s.B * s.Hkv == 0 || s.L == 0 || s.S == 0) return 0;
    if (s.E <= 32) return plan_bwd<32>(s).bytes;
    if (s.E <= 64) return plan_bwd<64>(s).bytes;
    if (s.E <= 128) return plan_bwd<128>(s).bytes;
    return 0;  // head dims above 128: no split
}

hipError_t launch_bwd_bf16(const BwdArgs &a, hipStream_t st) {
    const int64_t rows = (int64_t)a.s.B * a.s.H * a.s.L;
    if (rows > 0) {
        return_if(launch(bwd_pre_kernel<__bf16, false>, dim3((rows + 15) / 16), dim3(256), st, a));
    }
    if (a.s.B * a.s.Hkv == 0) return hipSuccess;
    if (a.s.E <= 32) return launch_d<32>(a, st);
    if (a.s.E <= 64) return launch_d<64>(a, st);
    if (a.s.E <= 128) return launch_d<128>(a, st);
    return launch_d<256>(a, st);
}

}  // namespace dc
