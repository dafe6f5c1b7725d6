// bfloat16 attention forward (fp32 accumulation) on CDNA4 MFMA (v_mfma_f32_32x32x16_bf16).
//
// Same mathematics as the float32 kernel and as DenseCore's torch_attention::forward
// (src/torch_attention.rs:143-284) evaluated on the bf16 inputs: scores, softmax state and
// the output accumulator are float32.  P enters the P V product as two bf16 terms
// (hi = bf16(P), lo = bf16(P - hi)), so it is carried to about 2^-17 rather than bf16's 2^-9;
// the only bf16 rounding left is the output's own.  Output is bf16, lse float32.
//
//   * 4 waves x 32 queries per workgroup; queries stay in VGPRs as bf16x8 B operands of
//     S^T = K Q^T (keys x queries), so the softmax state is per lane;
//   * K and V tiles of 64 keys are double-buffered in LDS, chunk-major (16-byte chunk c of
//     key r at slot c * 68 + r), and filled by global_load_lds_dwordx4 while the previous tile
//     is computed: no VGPR staging, and every transfer of a full tile has the same per-lane
//     offset, so the fill costs no VALU work;
//   * S^T reads 32 consecutive keys of one chunk per half-wave (512 contiguous bytes), and
//     O^T += V^T P^T takes V^T straight from the same layout with ds_read_b64_tr_b16 (each
//     16-lane group reads a 4-key x 16-dim block and gets it transposed), and P straight from
//     the S^T accumulator (the MFMA reduction index is permuted to the accumulator's row
//     order: registers 8u..8u+7 of a lane in half g hold keys 16u + {4g..4g+3,
//     8+4g..8+4g+3}); every address in the inner loop is a per-lane base plus a constant;
//   * the running max moves only when a tile's max exceeds it by more than 8 (base 2), so the
//     output accumulator is rarely rescaled;
//   * workgroups are ordered (batch*head)-major, longest causal tile first, and spread so that
//     the blocks of one (batch, head) run on the same XCD (blocks are dealt to the 8 XCDs
//     round-robin), which keeps its K/V in that XCD's L2.
#include "common.hpp"
#include "fwd_split.hpp"
#include "params.hpp"
#include "tile_bf16.hpp"

namespace dc {
namespace {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kBM = 32 * kWaves;  // queries per workgroup
constexpr int kBN = 64;           // keys per tile

// One K/V tile pair (chunk-major, 64 keys).
template <int D>
struct alignas(16) KVTileBf16 {
    u32x4 k[CMTile<kBN, D>::SLOTS];
    u32x4 v[CMTile<kBN, D>::SLOTS];
};

// Fill `t` with keys [n0, n0 + kBN); keys past S are zero.
template <int D, bool VEC>
DEVI void fill_tile(KVTileBf16<D> &t, const __bf16 *kb, const __bf16 *vb, int n0, int S, int E,
                    int wave, int lane) {
    fill_cm<kBN, D, VEC, kWaves>(t.k, kb + (int64_t)n0 * E, S - n0, E, wave, lane);
    fill_cm<kBN, D, VEC, kWaves>(t.v, vb + (int64_t)n0 * E, S - n0, E, wave, lane);
}

// Waves per SIMD of the 4-wave kernel: two workgroups per CU up to head dim 128; at 256 its K/V
// tiles take 136 KB of LDS and its queries and output 192 registers per lane, so one workgroup
// per CU and one wave per SIMD (512 registers).
constexpr int fwd_waves_per_eu(int D) { return D > 128 ? 1 : 2; }

template <int D, bool CAUSAL, bool MASK, bool VEC>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(fwd_waves_per_eu(D), fwd_waves_per_eu(D)))) void fwd_bf16_kernel(FwdArgs a) {
    constexpr int NT = kBN / 32;  // 32-key sub-tiles per tile
    constexpr int KSTEP = D / 16; // MFMA k-steps over the head dim
    constexpr int NDT = D / 32;   // 32-dim output tiles
    __shared__ KVTileBf16<D> sm[2];

    const AttnShape &s = a.s;
    const int tid = threadIdx.x, lane = tid & 63, lr = lane & 31, g = lane >> 5;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: branches stay scalar
    const int nqt = (s.L + kBM - 1) / kBM;
    const int nblk = gridDim.x;
    int w = blockIdx.x;
    if ((nblk & 7) == 0) w = (w & 7) * (nblk >> 3) + (w >> 3);
    const int bh = w / nqt, qt = CAUSAL ? nqt - 1 - w % nqt : w % nqt;
    const int b = bh / s.H, h = bh % s.H, hk = h / s.repeat;
    const int q0 = qt * kBM;
    const int qi = q0 + wave * 32 + lr;  // this lane's query
    const int wave_q0 = q0 + wave * 32, wave_last_q = wave_q0 + 31;

    const __bf16 *kb = static_cast<const __bf16 *>(a.k) + (int64_t)(b * s.Hkv + hk) * s.S * s.E;
    const __bf16 *vb = static_cast<const __bf16 *>(a.v) + (int64_t)(b * s.Hkv + hk) * s.S * s.E;

    // Scores are formed as fma(q.k, c, -m) in base-2 units; a negative scale is folded into
    // the queries (a sign flip, exact) so that the max of the raw products is the max score.  A
    // zero scale enters as the smallest normal float: every visible key then gets P = 1, as with
    // 0, and a masked (-inf) score stays -inf instead of becoming -inf * 0 = NaN.
    const bool neg = s.scale_log2 < 0.f;
    const float c = MASK ? 1.f : fmaxf(fabsf(s.scale_log2), 0x1p-126f);

    // Queries: step t, half g supplies Q[qi][16t + 8g + 0..7].
    bf16x8 qreg[KSTEP];
    {
        const __bf16 *qrow = static_cast<const __bf16 *>(a.q) + ((int64_t)bh * s.L + qi) * s.E;
#pragma unroll
        for (int t = 0; t < KSTEP; ++t) {
            const int d0 = 16 * t + 8 * g;
            if (VEC && qi < s.L) {
                qreg[t] = *reinterpret_cast<const bf16x8 *>(qrow + d0);
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    qreg[t][e] = (qi < s.L && d0 + e < s.E) ? qrow[d0 + e] : static_cast<__bf16>(0.f);
            }
            if (!MASK && neg) {
                u32x4 x = __builtin_bit_cast(u32x4, qreg[t]);
                x ^= 0x80008000u;
                qreg[t] = __builtin_bit_cast(bf16x8, x);
            }
        }
    }
    const float *mrow = nullptr;
    if (MASK) mrow = s.mask + (int64_t)b * s.msb + (int64_t)h * s.msh + (int64_t)qi * s.msl;

    f32x16 oacc[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) oacc[dt][r] = 0.f;
    float m_run = -INFINITY, l_part = 0.f;  // l_part: this half-wave's keys only

    const int kv_end = CAUSAL ? min(q0 + kBM, s.S) : s.S;
    const int ntiles = (kv_end + kBN - 1) / kBN;
    if (ntiles > 0) fill_tile<D, VEC>(sm[0], kb, vb, 0, s.S, s.E, wave, lane);

    const uint32_t rowb = row_lanebase<kBN, D>(lane);
    const uint32_t trb = tr_lanebase<kBN, D>(lane);

    auto tile = [&](int t) {
        const int n0 = t * kBN;
        KVTileBf16<D> &cur = sm[t & 1];
        if (VEC) wait_vmem();  // this wave's transfers of tile t landed
        __syncthreads();       // everyone's landed; everyone is done with tile t - 1
        if (t + 1 < ntiles) fill_tile<D, VEC>(sm[(t + 1) & 1], kb, vb, n0 + kBN, s.S, s.E, wave, lane);

        // K rows kt * 32 + (l % 32) for S^T; V^T (dims on lanes) for keys 16u + {4g..4g+3,
        // 8+4g..8+4g+3} of sub-tile kt, the rows P's accumulator registers 8u..8u+7 hold.
        auto kfrag = [&](int kt, int st) { return row_frag<kBN, D>(cur.k, rowb, kt * 32, st); };
        auto vfrag = [&](int kt, int u, int dt) { return tr_frag<kBN, D>(cur.v, trb, kt * 32 + 16 * u, dt); };

        bool live[NT];
#pragma unroll
        for (int kt = 0; kt < NT; ++kt)
            live[kt] = (n0 + kt * 32 < s.S) && (!CAUSAL || n0 + kt * 32 <= wave_last_q);
        // With a mask its values are read first; a sub-tile whose mask is -inf for every
        // (query, key) of the wave is skipped (its probabilities are exactly 0).
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
        bool any_live = false;
#pragma unroll
        for (int kt = 0; kt < NT; ++kt) any_live |= live[kt];
        if (!any_live) return;
        const bool edge = n0 + kBN > s.S || (CAUSAL && n0 + kBN - 1 > wave_q0);

        f32x16 sacc[NT];
#pragma unroll
        for (int kt = 0; kt < NT; ++kt)
#pragma unroll
            for (int r = 0; r < 16; ++r) sacc[kt][r] = 0.f;
        if (live[NT - 1]) {
            // Every sub-tile live: their independent MFMA chains are interleaved, with the K
            // fragment reads kept four MFMAs ahead (the compiler would otherwise issue each
            // read just before its MFMA and expose the LDS latency every time).
#pragma unroll
            for (int st = 0; st < KSTEP; ++st)
#pragma unroll
                for (int kt = 0; kt < NT; ++kt) sacc[kt] = mfma_bf16(kfrag(kt, st), qreg[st], sacc[kt]);
            sched_reads_ahead<KSTEP * NT, 1, 4>();
        } else {
            // One uniform test per sub-tile, outside its chain.
#pragma unroll
            for (int kt = 0; kt < NT; ++kt) {
                if (!live[kt]) continue;
#pragma unroll
                for (int st = 0; st < KSTEP; ++st) sacc[kt] = mfma_bf16(kfrag(kt, st), qreg[st], sacc[kt]);
            }
        }

        if constexpr (MASK) {
#pragma unroll
            for (int kt = 0; kt < NT; ++kt)
#pragma unroll
                for (int r = 0; r < 16; ++r) sacc[kt][r] = (sacc[kt][r] * s.scale + mv[kt][r]) * kLog2e;
        }
        if (edge) {
#pragma unroll
            for (int kt = 0; kt < NT; ++kt)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int key = n0 + kt * 32 + acc_row(r, g);
                    if (key >= s.S || (CAUSAL && key > qi) || !live[kt]) sacc[kt][r] = -INFINITY;
                }
        }
        float mx = -INFINITY;
#pragma unroll
        for (int kt = 0; kt < NT; ++kt)
#pragma unroll
            for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sacc[kt][r]);
        mx = xor32_max(mx) * c;
        // Lazy rescaling: the exponent reference m_run moves (and O, l are rescaled) only when
        // some lane's tile max exceeds it by more than 8, so P <= 2^8 and most tiles skip the
        // rescale of the accumulator; out = O / l and lse = m_run + log2(l) are unchanged.
        if (__any(mx > m_run + 8.f)) {
            const float m_new = fmaxf(m_run, mx);
            const float alpha = exp2_fast(m_run - (m_new == -INFINITY ? 0.f : m_new));
            l_part *= alpha;
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
                for (int r = 0; r < 16; ++r) oacc[dt][r] *= alpha;
            m_run = m_new;
        }
        const float neg_m = m_run == -INFINITY ? 0.f : -m_run;
#pragma unroll
        for (int kt = 0; kt < NT; ++kt)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float p = exp2_fast(fmaf(sacc[kt][r], c, neg_m));
                sacc[kt][r] = p;
                l_part += p;
            }

        // O^T += V^T P^T, 16 keys per MFMA, P as hi + lo.
#pragma unroll
        for (int kt = 0; kt < NT; ++kt) {
            if (!live[kt]) continue;
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                bf16x8 ph, pl;
                split_bf16(sacc[kt], 8 * u, ph, pl);
                bf16x8 va[NDT];
#pragma unroll
                for (int dt = 0; dt < NDT; ++dt) va[dt] = vfrag(kt, u, dt);
#pragma unroll
                for (int dt = 0; dt < NDT; ++dt) oacc[dt] = mfma_bf16(va[dt], ph, oacc[dt]);
#pragma unroll
                for (int dt = 0; dt < NDT; ++dt) oacc[dt] = mfma_bf16(va[dt], pl, oacc[dt]);
            }
        }
    };
    for (int t = 0; t < ntiles; ++t) tile(t);

    const float l_run = xor32_add(l_part);
    if (qi < s.L) {
        const bool empty = l_run == 0.f;
        const float inv = empty ? 0.f : 1.f / l_run;
        __bf16 *orow = static_cast<__bf16 *>(a.out) + ((int64_t)bh * s.L + qi) * s.E;
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
            for (int r = 0; r < 16; r += 4) {
                const int d = dt * 32 + acc_row(r, g);
                if (VEC) {
                    const bf16x4 o = {static_cast<__bf16>(oacc[dt][r] * inv),
                                      static_cast<__bf16>(oacc[dt][r + 1] * inv),
                                      static_cast<__bf16>(oacc[dt][r + 2] * inv),
                                      static_cast<__bf16>(oacc[dt][r + 3] * inv)};
                    *reinterpret_cast<bf16x4 *>(orow + d) = o;
                } else {
#pragma unroll
                    for (int u = 0; u < 4; ++u)
                        if (d + u < s.E) orow[d + u] = static_cast<__bf16>(oacc[dt][r + u] * inv);
                }
            }
        if (g == 0)
            a.lse[(int64_t)bh * s.L + qi] = empty ? 0.f : (m_run + log2_fast(l_run)) * kLn2;
    }
}

// Unmasked variants: two groups of four waves ping-pong.  Waves w and w + 4 of a workgroup
// share a SIMD; a SIMD overlaps one wave's MFMA work with another wave's VALU work, but not
// the two within one wave.  So the workgroup runs in phases separated by barriers, and in
// each phase one group runs its GEMM step while the other runs its softmax step:
//   GEMM(t):     S(t) = K(t) Q^T (16 MFMAs) and O^T += V(t-1)^T P(t-1)^T (32 MFMAs);
//   SOFTMAX(t):  edge masking, tile max, lazy rescale, P(t) = exp2(S(t) c - m), l += P, and
//                P(t) split into its bf16 hi and lo halves for the next GEMM step.
// Group 0 runs GEMM(0), SOFTMAX(0), GEMM(1), ... and group 1 the same one phase later.  Each
// group owns 128 queries (the workgroup 256) and both read the same K/V tiles: K(t) is read in
// phases 2t and 2t + 1, V(t) in phases 2t + 2 and 2t + 3; at every even phase 2s the waves
// issue K(s + 1) and V(s) into the double buffers, and wait for them at the end of phase
// 2s + 1.  A wave skips the steps (not the barriers or its share of the transfers) of tiles
// whose keys all follow its last query.
constexpr int kPPWaves = 8;
constexpr int kPPThreads = 64 * kPPWaves;
constexpr int kPPM = 32 * kPPWaves;  // queries per workgroup

// F16V: V is the fp16 copy (scaled by 2^vexp[b, kv head]) and P is rounded once to fp16, so the
// P V product is one fp16 MFMA per fragment instead of the bf16 hi + lo pair.
template <int D, bool CAUSAL, bool VEC, bool F16V, bool SPLIT = false>
__global__ __launch_bounds__(kPPThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void fwd_bf16_pp_kernel(FwdArgs a) {
    constexpr int NT = kBN / 32, KSTEP = D / 16, NDT = D / 32;
    __shared__ KVTileBf16<D> sm[2];

    const AttnShape &s = a.s;
    const int tid = threadIdx.x, lane = tid & 63, lr = lane & 31, g = lane >> 5;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int grp = wave >> 2;
    const int nqt = (s.L + kPPM - 1) / kPPM;
    const int w = logical_block();
    int bh = w / nqt, qt = CAUSAL ? nqt - 1 - w % nqt : w % nqt;
    // Split key ranges: blocks run over (head, query tile longest first, piece) (fwd_split.hpp).
    int piece = 0, npieces = 1;
    if constexpr (SPLIT) {
        if (!split_block(s, kPPM, kBN, a.split_chunk, w, &qt, &bh, &piece, &npieces)) return;
    }
    const int b = bh / s.H, h = bh % s.H, hk = h / s.repeat;
    const int q0 = qt * kPPM;
    const int wave_q0 = q0 + grp * 128 + (wave & 3) * 32, wave_last_q = wave_q0 + 31;
    const int qi = wave_q0 + lr;

    const __bf16 *kb = static_cast<const __bf16 *>(a.k) + (int64_t)(b * s.Hkv + hk) * s.S * s.E;
    const __bf16 *vb = static_cast<const __bf16 *>(a.v) + (int64_t)(b * s.Hkv + hk) * s.S * s.E;

    const bool neg = s.scale_log2 < 0.f;  // folded as in fwd_bf16_kernel, zero scale included
    const float c = fmaxf(fabsf(s.scale_log2), 0x1p-126f);
    bf16x8 qreg[KSTEP];
    {
        const __bf16 *qrow = static_cast<const __bf16 *>(a.q) + ((int64_t)bh * s.L + qi) * s.E;
#pragma unroll
        for (int t = 0; t < KSTEP; ++t) {
            const int d0 = 16 * t + 8 * g;
            if (VEC && qi < s.L) {
                qreg[t] = *reinterpret_cast<const bf16x8 *>(qrow + d0);
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    qreg[t][e] = (qi < s.L && d0 + e < s.E) ? qrow[d0 + e] : static_cast<__bf16>(0.f);
            }
            if (neg) {
                u32x4 x = __builtin_bit_cast(u32x4, qreg[t]);
                x ^= 0x80008000u;
                qreg[t] = __builtin_bit_cast(bf16x8, x);
            }
        }
    }

    f32x16 oacc[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) oacc[dt][r] = 0.f;
    float m_run = -INFINITY, l_part = 0.f;
    f32x16 sc[NT];                // S(t), raw
    bf16x8 ph[NT][2], pl[NT][2];  // P(t) as hi + lo, sub-tile kt, 16-key half u

    const int kv_end = CAUSAL ? min(q0 + kPPM, s.S) : s.S;
    const int ntiles = (kv_end + kBN - 1) / kBN;
    // This block's key tiles [t_begin, t_end): all of them, or its piece's.
    const int t_begin = SPLIT ? piece * ntiles / npieces : 0;
    const int t_end = SPLIT ? (piece + 1) * ntiles / npieces : ntiles;
    const uint32_t rowb = row_lanebase<kBN, D>(lane);
    const uint32_t trb = tr_lanebase<kBN, D>(lane);

    auto fill_k = [&](int t) {
        fill_cm<kBN, D, VEC, kPPWaves>(sm[t & 1].k, kb + (int64_t)t * kBN * s.E, s.S - t * kBN, s.E, wave, lane);
    };
    auto fill_v = [&](int t) {
        fill_cm<kBN, D, VEC, kPPWaves>(sm[t & 1].v, vb + (int64_t)t * kBN * s.E, s.S - t * kBN, s.E, wave, lane);
    };
    // Sub-tile kt of tile t holds a key this wave's queries see.
    auto sub_live = [&](int t, int kt) {
        const int k0 = t * kBN + kt * 32;
        return k0 < s.S && (!CAUSAL || k0 <= wave_last_q);
    };

    // PV(t-1) first, then S(t): P's registers are dead before S is written, so the two share
    // registers.  PV runs in groups of 16 keys (sub-tile kt = grp / 2, half u = grp % 2); a
    // group's V^T fragments are read while the previous group's MFMAs run (only this group's
    // wave issues MFMAs on its SIMD in this phase, so a read waited for right before its MFMA
    // stalls the SIMD).  A sub-tile with no key this wave's queries see (past the diagonal or
    // past S) enters too, as straight-line code: its P is exactly 0 (scores at -inf) and its V
    // rows are finite (rows past S are zero-filled), so it adds nothing.
    auto gemm = [&](int t) {
        if (t > t_begin && sub_live(t - 1, 0)) {
            const u32x4 *vt_ = sm[(t - 1) & 1].v;
            constexpr int NG = 2 * NT;
            constexpr int MF = F16V ? NDT : 2 * NDT;  // MFMAs per group
            constexpr int RPM = 2 * NDT / MF;         // V^T reads per MFMA
            bf16x8 va[2][NDT];
            auto load_v = [&](int grp) {
#pragma unroll
                for (int dt = 0; dt < NDT; ++dt) va[grp & 1][dt] = tr_frag<kBN, D>(vt_, trb, 16 * grp, dt);
            };
            load_v(0);
#pragma unroll
            for (int grp = 0; grp < NG; ++grp) {
                if (grp + 1 < NG) load_v(grp + 1);
                const int kt = grp >> 1, u = grp & 1;
                if constexpr (F16V) {
#pragma unroll
                    for (int dt = 0; dt < NDT; ++dt) oacc[dt] = mfma_f16(va[grp & 1][dt], ph[kt][u], oacc[dt]);
                } else {
#pragma unroll
                    for (int dt = 0; dt < NDT; ++dt) oacc[dt] = mfma_bf16(va[grp & 1][dt], ph[kt][u], oacc[dt]);
#pragma unroll
                    for (int dt = 0; dt < NDT; ++dt) oacc[dt] = mfma_bf16(va[grp & 1][dt], pl[kt][u], oacc[dt]);
                }
            }
            __builtin_amdgcn_sched_group_barrier(0x100, 2 * NDT, 0);  // group 0's reads
#pragma unroll
            for (int grp = 0; grp + 1 < NG; ++grp)
#pragma unroll
                for (int i = 0; i < MF; ++i) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);    // an MFMA of this group
                    __builtin_amdgcn_sched_group_barrier(0x100, RPM, 0);  // reads of the next
                }
            __builtin_amdgcn_sched_group_barrier(0x008, MF, 0);
            __builtin_amdgcn_sched_barrier(0);
        }
        if (t < t_end && sub_live(t, 0)) {
            const u32x4 *kt_ = sm[t & 1].k;
#pragma unroll
            for (int kt = 0; kt < NT; ++kt)
#pragma unroll
                for (int r = 0; r < 16; ++r) sc[kt][r] = 0.f;
#pragma unroll
            for (int st = 0; st < KSTEP; ++st)
#pragma unroll
                for (int kt = 0; kt < NT; ++kt)
                    sc[kt] = mfma_bf16(row_frag<kBN, D>(kt_, rowb, kt * 32, st), qreg[st], sc[kt]);
            // K reads six MFMAs ahead (C5 forward 1163 -> 1155 us against four; eight: 1157).
            sched_reads_ahead<KSTEP * NT, 1, 6>();
        }
    };
    // Keys past S or (causal) past the query get -inf; the exponent reference m_run moves (and O,
    // l are rescaled) only when some lane's tile max exceeds it by more than 8, so P <= 2^8;
    // out = O / l and lse = m_run + log2(l) are exact either way.
    auto softmax = [&](int t) {
        if (t >= t_end || !sub_live(t, 0)) return;
        const int n0 = t * kBN;
        if (n0 + kBN > s.S || (CAUSAL && n0 + kBN - 1 > wave_q0)) {
            // Register r of sub-tile kt holds key n0 + 32 kt + 4g + (8 (r/4) + r%4).
#pragma unroll
            for (int kt = 0; kt < NT; ++kt) {
                const int base = n0 + kt * 32 + 4 * g;
                const int lim = min(s.S - base, CAUSAL ? qi - base + 1 : s.S - base);
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    if (8 * (r >> 2) + (r & 3) >= lim) sc[kt][r] = -INFINITY;
            }
        }
        float mx = -INFINITY;
#pragma unroll
        for (int kt = 0; kt < NT; ++kt)
#pragma unroll
            for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sc[kt][r]);
        mx = xor32_max(mx) * c;
        if (__any(mx > m_run + 8.f)) {
            const float m_new = fmaxf(m_run, mx);
            const float alpha = exp2_fast(m_run - (m_new == -INFINITY ? 0.f : m_new));
            l_part *= alpha;
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
                for (int r = 0; r < 16; ++r) oacc[dt][r] *= alpha;
            m_run = m_new;
        }
        const float neg_m = m_run == -INFINITY ? 0.f : -m_run;
#pragma unroll
        for (int kt = 0; kt < NT; ++kt) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float p = exp2_fast(fmaf(sc[kt][r], c, neg_m));
                sc[kt][r] = p;
                l_part += p;
            }
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                if constexpr (F16V)
                    ph[kt][u] = cvt_f16x8(sc[kt], 8 * u);
                else
                    split_bf16(sc[kt], 8 * u, ph[kt][u], pl[kt][u]);
            }
        }
    };

    // fill(t) at phase 2t: K(t + 1) into K(t - 1)'s buffer, V(t) into V(t - 2)'s buffer.
    auto fill = [&](int t) {
        if (t + 1 < t_end) fill_k(t + 1);
        if (t < t_end) fill_v(t);
    };
    if (t_begin < t_end) fill_k(t_begin);
    if (VEC) wait_vmem();
    __syncthreads();
    // Phases 0 .. 2 ntiles + 1, one barrier each; the transfers issued at an even phase are
    // waited for at the end of the next (odd) one.  Each group has its own loop, so that only
    // the registers of S (group 1) or of P (group 0) are carried from one iteration to the next.
    if (grp == 0) {
        for (int t = t_begin; t <= t_end; ++t) {
            fill(t);
            gemm(t);
            __syncthreads();
            softmax(t);
            if (VEC) wait_vmem();
            __syncthreads();
        }
    } else {
        for (int t = t_begin; t <= t_end; ++t) {
            fill(t);
            if (t > t_begin) softmax(t - 1);
            __syncthreads();
            gemm(t);
            if (VEC) wait_vmem();
            __syncthreads();
        }
    }

    const float l_run = xor32_add(l_part);
    if (SPLIT && npieces > 1) {
        // A piece of a split range: its normalized partial (float32) and lse (-inf: no visible
        // key) go to the row's slot `piece`; fwd_split_merge_kernel combines them.
        if (qi < s.L) {
            const bool empty = l_run == 0.f;
            float inv = empty ? 0.f : 1.f / l_run;
            if constexpr (F16V) inv = ldexpf(inv, -a.vexp[b * s.Hkv + hk]);
            const int64_t row = (int64_t)bh * s.L + qi;
            float *prow = a.split_o + (row * a.split_max + piece) * s.E;
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
                for (int r = 0; r < 16; r += 4) {
                    const int d = dt * 32 + acc_row(r, g);
                    if (VEC) {
                        *reinterpret_cast<f32x4 *>(prow + d) = f32x4{oacc[dt][r] * inv, oacc[dt][r + 1] * inv,
                                                                     oacc[dt][r + 2] * inv, oacc[dt][r + 3] * inv};
                    } else {
#pragma unroll
                        for (int u = 0; u < 4; ++u)
                            if (d + u < s.E) prow[d + u] = oacc[dt][r + u] * inv;
                    }
                }
            if (g == 0)
                a.split_lse[row * a.split_max + piece] = empty ? -INFINITY : (m_run + log2_fast(l_run)) * kLn2;
        }
        return;
    }
    if (qi < s.L) {
        const bool empty = l_run == 0.f;
        float inv = empty ? 0.f : 1.f / l_run;
        if constexpr (F16V) inv = ldexpf(inv, -a.vexp[b * s.Hkv + hk]);  // undo V's 2^vexp
        __bf16 *orow = static_cast<__bf16 *>(a.out) + ((int64_t)bh * s.L + qi) * s.E;
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
            for (int r = 0; r < 16; r += 4) {
                const int d = dt * 32 + acc_row(r, g);
                if (VEC) {
                    const bf16x4 o = {static_cast<__bf16>(oacc[dt][r] * inv),
                                      static_cast<__bf16>(oacc[dt][r + 1] * inv),
                                      static_cast<__bf16>(oacc[dt][r + 2] * inv),
                                      static_cast<__bf16>(oacc[dt][r + 3] * inv)};
                    *reinterpret_cast<bf16x4 *>(orow + d) = o;
                } else {
#pragma unroll
                    for (int u = 0; u < 4; ++u)
                        if (d + u < s.E) orow[d + u] = static_cast<__bf16>(oacc[dt][r + u] * inv);
                }
            }
        if (g == 0)
            a.lse[(int64_t)bh * s.L + qi] = empty ? 0.f : (m_run + log2_fast(l_run)) * kLn2;
    }
}

// The split of the unmasked (ping-pong, fp16 P V) forward's grid on the current device.
template <int D>
FwdSplitPlan plan(const AttnShape &s) {
    const int64_t blocks = (int64_t)(s.L + kPPM - 1) / kPPM * s.B * s.H;
    const int64_t slots = split_slots(reinterpret_cast<const void *>(&fwd_bf16_pp_kernel<D, true, true, true, true>),
                                      kPPThreads, blocks);
    return plan_split(s, kPPM, kBN, slots);
}

template <int D, bool VEC>
hipError_t launch_dv(const FwdArgs &a, hipStream_t st) {
    const bool mask = a.s.mask != nullptr;
    if constexpr (D > 128) {
        // Head dims 129-256: the 4-wave kernel, with or without a mask (the ping-pong kernel's
        // 8 waves would need more than 256 registers each); P enters P V as bf16 hi + lo.
        const int nqt = (a.s.L + kBM - 1) / kBM;
        const dim3 grid(nqt * a.s.B * a.s.H), block(kThreads);
        if (a.s.causal && mask) return launch(fwd_bf16_kernel<D, true, true, VEC>, grid, block, st, a);
        if (a.s.causal) return launch(fwd_bf16_kernel<D, true, false, VEC>, grid, block, st, a);
        if (mask) return launch(fwd_bf16_kernel<D, false, true, VEC>, grid, block, st, a);
        return launch(fwd_bf16_kernel<D, false, false, VEC>, grid, block, st, a);
    } else {  // head dims up to 128 (the ping-pong kernel exists only there)
        if (!mask) {
            const int nqt = (a.s.L + kPPM - 1) / kPPM;
            const dim3 grid(nqt * a.s.B * a.s.H), block(kPPThreads);
            if (a.v16) {
                record_schedule(f16_products, 1);
                FwdArgs f = a;
                const F16Copy vcopy{a.v, a.v16, (int64_t)a.s.S * a.s.E, a.vexp};
                return_if(launch_to_f16(&vcopy, 1, (int64_t)a.s.B * a.s.Hkv, a.f16_partial, st));
                f.v = a.v16;
                if (a.split_o) {
                    const FwdSplitPlan p = plan<D>(a.s);
                    if (p.chunk > 0 && p.bytes <= a.split_bytes) {
                        record_schedule(split_chunk, p.chunk);
                        record_schedule(split_pieces, p.max_pieces);
                        f.split_chunk = p.chunk, f.split_max = p.max_pieces;
                        f.split_lse = f.split_o + (size_t)a.s.B * a.s.H * a.s.L * p.max_pieces * a.s.E;
                        const dim3 sgrid((unsigned)p.blocks);
                        if (a.s.causal)
                            return_if(launch(fwd_bf16_pp_kernel<D, true, VEC, true, true>, sgrid, block, st, f));
                        else
                            return_if(launch(fwd_bf16_pp_kernel<D, false, VEC, true, true>, sgrid, block, st, f));
                        const int64_t rows = (int64_t)a.s.B * a.s.H * a.s.L;
                        return launch(fwd_split_merge_kernel<__bf16>, dim3((unsigned)((rows + 15) / 16)), dim3(256), st, f,
                                      kPPM, kBN);
                    }
                }
                if (a.s.causal) return launch(fwd_bf16_pp_kernel<D, true, VEC, true>, grid, block, st, f);
                return launch(fwd_bf16_pp_kernel<D, false, VEC, true>, grid, block, st, f);
            }
            if (a.s.causal) return launch(fwd_bf16_pp_kernel<D, true, VEC, false>, grid, block, st, a);
            return launch(fwd_bf16_pp_kernel<D, false, VEC, false>, grid, block, st, a);
        }
        const int nqt = (a.s.L + kBM - 1) / kBM;
        const dim3 grid(nqt * a.s.B * a.s.H), block(kThreads);
        if (a.s.causal) return launch(fwd_bf16_kernel<D, true, true, VEC>, grid, block, st, a);
        return launch(fwd_bf16_kernel<D, false, true, VEC>, grid, block, st, a);
    }
}

template <int D>
hipError_t launch_d(const FwdArgs &args, hipStream_t st) {
    FwdArgs a = args;
    a.s.vec = args.s.vec && args.s.E == D;  // the ABI checked 16-byte alignment; E must fill D
    return a.s.vec ? launch_dv<D, true>(a, st) : launch_dv<D, false>(a, st);
}

}  // namespace

size_t fwd_bf16_split_bytes(const AttnShape &s) {
    if (s.B == 0 || s.H == 0 || s.L == 0) return 0;
    if (s.E <= 32) return plan<32>(s).bytes;
    if (s.E <= 64) return plan<64>(s).bytes;
    if (s.E <= 128) return plan<128>(s).bytes;
    return 0;  // head dims above 128: no split
}

hipError_t launch_fwd_bf16(const FwdArgs &a, hipStream_t st) {
    if (a.s.B == 0 || a.s.H == 0 || a.s.L == 0) return hipSuccess;
    if (a.s.E <= 32) return launch_d<32>(a, st);
    if (a.s.E <= 64) return launch_d<64>(a, st);
    if (a.s.E <= 128) return launch_d<128>(a, st);
    return launch_d<256>(a, st);
}

}  // namespace dc
