// Float32 attention forward on CDNA4 MFMA (v_mfma_f32_32x32x2_f32).
//
// Computes what DenseCore's torch_attention::forward computes (src/torch_attention.rs:143-284):
// out = softmax(scale * q k^T + mask, causal) v and lse = max + ln(sum), with fully masked
// rows giving out = 0 and lse = 0 (:223-226, :258-264).  The blocking is this kernel's own:
//
//   * one workgroup = 4 waves = 128 queries of one (batch, head); each wave owns 32 queries;
//   * the wave's queries stay in VGPRs as the B operand of S^T = K Q^T (keys x queries), so
//     every lane owns one query column and the online-softmax state (max, sum) is a scalar per
//     lane, combined with the other half-wave by one cross-lane exchange;
//   * K and V tiles of BN keys are staged through LDS with the next tile's loads in flight
//     during compute: on the fast path (E == D, aligned rows) by global_load_lds into
//     a second LDS buffer, otherwise through registers into rows padded to D + 4 floats (which
//     keeps ds_read_b128 conflict-free);
//   * P = exp2(S * scale * log2 e - m) never leaves registers: the S^T accumulator is fed back
//     as the B operand of O^T += V^T P^T with the reduction index permuted to match.
//
// Head dims below the instantiated D are zero-padded on load; keys past S and (causal) keys
// past the query are -inf before the softmax.
#include <type_traits>

#include "common.hpp"
#include "fwd_split.hpp"
#include "params.hpp"

namespace dc {
namespace {

// W waves per workgroup, 32 queries per wave (4; 2 or 1 for short causal problems).

template <int D, int BN>
struct alignas(16) FwdSmem {
    float k[BN][D + 4];
    float v[BN][D + 4];
};

// Global -> register staging of one K/V tile (fast path: E == D, 16-byte aligned rows).
template <int D, int BN, int W>
struct KVStage {
    static constexpr int kThreads = 64 * W;
    static constexpr int C4 = D / 4;
    static constexpr int N = BN * C4 / kThreads;
    static_assert(BN * C4 % kThreads == 0, "tile must split evenly over the workgroup");
    f32x4 k[N], v[N];

    DEVI void load(const float *kb, const float *vb, int n0, int S, int tid) {
#pragma unroll
        for (int j = 0; j < N; ++j) {
            const int i = tid + kThreads * j, r = i / C4, c = (i % C4) * 4, key = n0 + r;
            if (key < S) {
                k[j] = *reinterpret_cast<const f32x4 *>(kb + (int64_t)key * D + c);
                v[j] = *reinterpret_cast<const f32x4 *>(vb + (int64_t)key * D + c);
            } else {
                k[j] = f32x4{0.f, 0.f, 0.f, 0.f};
                v[j] = f32x4{0.f, 0.f, 0.f, 0.f};
            }
        }
    }
    DEVI void store(FwdSmem<D, BN> &sm, int tid) const {
#pragma unroll
        for (int j = 0; j < N; ++j) {
            const int i = tid + kThreads * j, r = i / C4, c = (i % C4) * 4;
            *reinterpret_cast<f32x4 *>(&sm.k[r][c]) = k[j];
            *reinterpret_cast<f32x4 *>(&sm.v[r][c]) = v[j];
        }
    }
};

// Generic path: any E <= D, any alignment; loads straight into LDS.
template <int D, int BN, int W>
DEVI void load_kv_generic(FwdSmem<D, BN> &sm, const float *kb, const float *vb, int n0, int S,
                          int E, int tid) {
    for (int i = tid; i < BN * D; i += 64 * W) {
        const int r = i / D, c = i % D, key = n0 + r;
        const bool ok = key < S && c < E;
        sm.k[r][c] = ok ? kb[(int64_t)key * E + c] : 0.f;
        sm.v[r][c] = ok ? vb[(int64_t)key * E + c] : 0.f;
    }
}

// Asynchronous path (E == D, 16-byte aligned rows): K and V tiles are double-buffered in LDS
// and filled with global_load_lds_dwordx4 (lane i of a wave lands at the wave's LDS base +
// 16 i), so no VGPRs stage them and the next tile streams in while this one is computed.  Rows
// are unpadded and their 16-byte chunks are stored XOR-swizzled, chunk c of row r at c ^ swz(r),
// which keeps both read patterns conflict-free: ds_read_b128 of one chunk by 16 consecutive
// rows, and ds_read_b32 of 32 consecutive floats by rows R and R + 4 (the two half-waves).
template <int D, int BN>
struct alignas(16) FwdSmemAsync {  // one buffer of the pair
    float k[BN][D];
    float v[BN][D];
};

struct NoSmem {};

template <int D>
DEVI int swz(int row) {
    return (row ^ ((row & 4) << 1)) & (D / 4 - 1);
}

// Global loads per wave for one K (or V) tile: each wave-wide load fills 64 / (D / 4) rows.
template <int D, int BN, int W>
constexpr int kTileLoads = BN / W / (64 / (D / 4));

// Issue this wave's share of tile [n0, n0 + BN) into buffer `buf`: K and V, or only one of
// them (keys past the end read a valid row, S - 1; their scores are -inf, so they contribute
// nothing).
template <int D, int BN, int W, bool DO_K = true, bool DO_V = true>
DEVI void issue_tile(FwdSmemAsync<D, BN> &sm, const float *kb, const float *vb, int n0, int S,
                     int wave, int lane) {
    constexpr int C = D / 4;             // 16-byte chunks per row
    constexpr int RPL = 64 / C;          // rows per wave-wide load
    constexpr int ROWS = BN / W;         // rows per wave
    static_assert(ROWS % RPL == 0, "a wave loads whole rows");
    if (n0 + BN <= S) {
        // No row to clamp: the tile's base in SGPRs and a lane offset that is the same for
        // every tile (hoisted out of the tile loop), so the transfers cost no VALU instructions
        // (float32 MFMAs and VALU instructions do not overlap; the clamped addresses took ~6
        // per transfer).
        const float *kt = kb + (int64_t)n0 * D, *vt = vb + (int64_t)n0 * D;
        constexpr int NJ = ROWS / RPL;
        auto lane_off = [&](int j) {
            const int row = wave * ROWS + j * RPL + lane / C;
            return (uint32_t)(row * D + (((lane % C) ^ swz<D>(row)) << 2)) * 4u;
        };
        if constexpr (W == 1 && (DO_K != DO_V)) {
            // One-wave workgroups (K or V alone): transfers in pairs, one m0 save per pair and the
            // LDS address cast once (B64 H6 L256 causal 41.4 -> 40.5 us; the 4-wave kernels, whose
            // wave index the LDS addresses carry, measured ~1% slower this way).
            const uint64_t gb = sgpr_addr(DO_K ? kt : vt);
            const uint32_t lb = lds_addr(DO_K ? &sm.k[0][0] : &sm.v[0][0]);
#pragma unroll
            for (int j = 0; j + 1 < NJ; j += 2)
                lds_dma16_pair(gb, lane_off(j), lb + (uint32_t)(j * RPL * D * 4), gb, lane_off(j + 1),
                               lb + (uint32_t)((j + 1) * RPL * D * 4));
            if constexpr (NJ % 2 == 1)
                lds_dma16_off(DO_K ? kt : vt, lane_off(NJ - 1),
                              DO_K ? &sm.k[(NJ - 1) * RPL][0] : &sm.v[(NJ - 1) * RPL][0]);
            return;
        }
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const int r0 = wave * ROWS + j * RPL;
            const uint32_t off = lane_off(j);
            if constexpr (DO_K) lds_dma16_off(kt, off, &sm.k[r0][0]);
            if constexpr (DO_V) lds_dma16_off(vt, off, &sm.v[r0][0]);
        }
        return;
    }
#pragma unroll
    for (int j = 0; j < ROWS / RPL; ++j) {
        const int r0 = wave * ROWS + j * RPL;
        const int row = r0 + lane / C;
        const int chunk = (lane % C) ^ swz<D>(row);  // logical chunk stored at this slot
        const int64_t off = (int64_t)min(n0 + row, S - 1) * D + chunk * 4;
        if constexpr (DO_K) lds_dma16(kb + off, &sm.k[r0][0]);
        if constexpr (DO_V) lds_dma16(vb + off, &sm.v[r0][0]);
    }
}

template <int D, int BN, int W, bool CAUSAL, bool MASK, bool ASYNC, bool ROWMASK = false, bool SPLIT = false>
__global__ __launch_bounds__(64 * W) __attribute__((amdgpu_waves_per_eu(D <= 64 || !ASYNC ? 2 : 1, D <= 64 || !ASYNC ? 2 : 1))) void fwd_f32_kernel(FwdArgs a) {
    [[maybe_unused]] constexpr int kThreads = 64 * W;
    constexpr int kBM = 32 * W;
    constexpr int NT = BN / 32;  // key sub-tiles of 32 per kv tile
    constexpr int DH = D / 2;    // head-dim values each half-wave supplies per query
    // One-wave workgroups (short causal rows without a mask) stage K and V in ONE buffer,
    // loaded out of phase: K(t + 1) streams in while the wave computes softmax(t) and P V(t),
    // V(t + 1) while it computes Q K(t + 1).  16 KB of LDS per wave at D = 64 and no barriers:
    // ten independent waves per CU, dispatched longest first.  (Two-wave workgroups couple
    // their SIMDs through each tile's barrier, which left the long query tiles of such problems
    // sharing their SIMDs for most of the kernel: B64 H6 L256 D64 47.0 -> 43.1 us.)
    constexpr bool ONEBUF = ASYNC && W == 1 && !MASK && !SPLIT;
    constexpr int NLD = kTileLoads<D, BN, W>;
    using Smem = typename std::conditional<ASYNC, FwdSmemAsync<D, BN>, FwdSmem<D, BN>>::type;
    using Smem2 = typename std::conditional<ASYNC && !ONEBUF, FwdSmemAsync<D, BN>, NoSmem>::type;
    __shared__ Smem sm;
    __shared__ Smem2 sm2;  // the second buffer of the asynchronous path

    const AttnShape &s = a.s;
    const int tid = threadIdx.x, lane = tid & 63, lr = lane & 31, g = lane >> 5;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: branches stay scalar
    const int BH = s.B * s.H;
    const int nqt = (s.L + kBM - 1) / kBM;
    const int bid = blockIdx.x;
    int qt = CAUSAL ? nqt - 1 - bid / BH : bid / BH;  // longest causal tiles first
    int bh = bid % BH;
    // Split key ranges: blocks run over (head, query tile longest first, piece), the pieces of a
    // head dealt to one XCD (blocks go to XCD bid % 8) so that its K/V stays in one L2.
    int piece = 0, npieces = 1;
    if constexpr (SPLIT) {
        const int n = gridDim.x, w = (n & 7) == 0 ? (bid & 7) * (n >> 3) + (bid >> 3) : bid;
        if (!split_block(s, kBM, BN, a.split_chunk, w, &qt, &bh, &piece, &npieces)) return;
    }
    if (ROWMASK && a.order) {
        // Heads in descending order of live key tiles, dealt to the 8 XCDs round-robin (blocks
        // go to XCD bid % 8), the query tiles of one head on one XCD: its K/V stays in one L2.
        const int x = bid & 7, slot = bid >> 3;
        const int r = 8 * (slot / nqt) + x;
        if (r >= BH) return;
        bh = a.order[r];
        qt = slot % nqt;
    }
    const int b = bh / s.H, h = bh % s.H, hk = h / s.repeat;
    const int q0 = qt * kBM;
    const int qi = q0 + wave * 32 + lr;  // this lane's query
    const int wave_last_q = q0 + wave * 32 + 31;

    const float *qp = static_cast<const float *>(a.q);
    const float *kb = static_cast<const float *>(a.k) + (int64_t)(b * s.Hkv + hk) * s.S * s.E;
    const float *vb = static_cast<const float *>(a.v) + (int64_t)(b * s.Hkv + hk) * s.S * s.E;

    // Queries: lane supplies Q[qi][g*DH + t] for t = 0..DH-1.
    float qreg[DH];
    {
        const float *qrow = qp + ((int64_t)bh * s.L + qi) * s.E;
        if (s.vec && qi < s.L) {
#pragma unroll
            for (int t = 0; t < DH; t += 4) {
                f32x4 x = *reinterpret_cast<const f32x4 *>(qrow + g * DH + t);
                qreg[t] = x[0], qreg[t + 1] = x[1], qreg[t + 2] = x[2], qreg[t + 3] = x[3];
            }
        } else {
#pragma unroll
            for (int t = 0; t < DH; ++t) {
                const int d = g * DH + t;
                qreg[t] = (qi < s.L && d < s.E) ? qrow[d] : 0.f;
            }
        }
    }
    // Without a mask the scale is applied after the tile max and inside each exponent's FMA
    // (float32 MFMAs and VALU instructions do not overlap, and this saves a multiply per score):
    // for a positive scale the max of the rounded products equals the rounded product of the
    // max, so the running max is unchanged, and the exponent is rounded once instead of twice.
    // A negative scale enters as its magnitude with the queries negated; a zero scale as the
    // smallest normal float (every visible score then gives exp2 of a value below 2^-100, which
    // is 1, as it is with 0).
    const float csc = MASK ? 0.f : fmaxf(fabsf(s.scale_log2), 0x1p-126f);
    if (!MASK && s.scale_log2 < 0.f) {
#pragma unroll
        for (int t = 0; t < DH; ++t) qreg[t] = -qreg[t];
    }
    const float *mrow = nullptr;
    if (MASK) mrow = s.mask + (int64_t)b * s.msb + (int64_t)h * s.msh + (int64_t)qi * s.msl;
    // ROWMASK: the mask does not depend on the query (stride 0 along L, e.g. key padding).  Each
    // wave then reads a tile's mask with one coalesced load (lane l: key n0 + l), a tile ahead,
    // takes the sub-tiles' liveness from a ballot, and hands the values to the accumulator
    // layout through its own 64-float LDS slot.
    static_assert(!ROWMASK || (MASK && BN <= 64), "row masks: one value per lane and tile");
    __shared__ float mslot[ROWMASK ? W : 1][64];
    auto row_mask = [&](int t) -> float {
        const int key = t * BN + lane;
        return (ROWMASK && lane < BN && key < s.S) ? mrow[key] : -INFINITY;
    };
    float mask_next = 0.f;

    f32x16 oacc[D / 32];
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) oacc[dt][r] = 0.f;
    float m_run = -INFINITY, l_run = 0.f;

    const int kv_end = CAUSAL ? min(q0 + kBM, s.S) : s.S;
    const int ntiles = (kv_end + BN - 1) / BN;
    // This block's key tiles [t_begin, t_end): all of them, or its piece's (the query tile's
    // tiles cut into npieces near-equal ranges).
    const int t_begin = SPLIT ? piece * ntiles / npieces : 0;
    const int t_end = SPLIT ? (piece + 1) * ntiles / npieces : ntiles;

    KVStage<D, BN, W> stage;
    if constexpr (ONEBUF) {
        if (t_begin < t_end) {
            issue_tile<D, BN, W, true, false>(sm, kb, vb, t_begin * BN, s.S, wave, lane);
            issue_tile<D, BN, W, false, true>(sm, kb, vb, t_begin * BN, s.S, wave, lane);
        }
    } else if constexpr (ASYNC) {
        if (t_begin < t_end) issue_tile<D, BN, W>(sm, kb, vb, t_begin * BN, s.S, wave, lane);
    } else if (s.vec && t_begin < t_end) {
        stage.load(kb, vb, t_begin * BN, s.S, tid);
    }
    if constexpr (ROWMASK) mask_next = row_mask(t_begin);

    // One tile per call; the asynchronous path alternates two distinct LDS objects so that
    // the compiler can see the in-flight loads never alias the tile being read.
    // tn: the tile to stream in next (t + 1; -1: none).
    auto tile = [&](int t, auto &cur, auto &nxt, int tn) {
        const int n0 = t * BN;
        if constexpr (ONEBUF) {
            // In flight: K(t), then V(t).  (Every tile of a one-buffer wave has visible keys:
            // causal tiles end at the wave's last query, so no tile takes the early return.)
            wait_vmem_but<NLD>();
        } else if constexpr (ASYNC) {
            __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): this wave's loads of tile t landed
            __syncthreads();  // everyone's loads landed; everyone is done with the previous tile
            if (tn >= 0) issue_tile<D, BN, W>(nxt, kb, vb, tn * BN, s.S, wave, lane);
        } else {
            __syncthreads();  // everyone is done reading the previous tile
            if (s.vec) {
                stage.store(cur, tid);
            } else {
                load_kv_generic<D, BN, W>(cur, kb, vb, n0, s.S, s.E, tid);
            }
            __syncthreads();
            if (s.vec && t + 1 < t_end) stage.load(kb, vb, n0 + BN, s.S, tid);
        }
        // K row kr, dims d..d+3 (d a multiple of 4), and V row vr, dim d, of the current tile.
        auto kread = [&](int kr, int d) -> f32x4 {
            if constexpr (ASYNC)
                return *reinterpret_cast<const f32x4 *>(&cur.k[kr][((d >> 2) ^ swz<D>(kr)) << 2]);
            else
                return *reinterpret_cast<const f32x4 *>(&cur.k[kr][d]);
        };
        auto vread = [&](int vr, int d) -> float {
            if constexpr (ASYNC)
                return cur.v[vr][(((d >> 2) ^ swz<D>(vr)) << 2) | (d & 3)];
            else
                return cur.v[vr][d];
        };

        // Which 32-key sub-tiles have any key visible to this wave's queries (a prefix of
        // them), and whether any key of the tile needs masking for this wave (causal diagonal,
        // end of the sequence).  Both are wave-uniform.
        bool live[NT];
#pragma unroll
        for (int kt = 0; kt < NT; ++kt)
            live[kt] = (n0 + kt * 32 < s.S) && (!CAUSAL || n0 + kt * 32 <= wave_last_q);
        // With a mask, its values are read first, and a sub-tile whose mask is -inf for every
        // (query, key) of the wave is skipped like an invisible one (key padding): its
        // probabilities are exactly 0.  Queries past L count as fully masked.
        float mv[MASK ? NT : 1][16];
        if constexpr (ROWMASK) {
            const float mcur = mask_next;
            if (tn >= 0) mask_next = row_mask(tn);
            // Liveness from a ballot; the values reach the accumulator layout through the wave's
            // LDS slot.
            const uint64_t open = __ballot(mcur != -INFINITY);
            float *slot = mslot[wave];
            slot[lane] = mcur * kLog2e;  // in log2 units: one multiply per key, not per score
#pragma unroll
            for (int kt = 0; kt < NT; ++kt) {
                live[kt] = live[kt] && ((open >> (32 * kt)) & 0xffffffffull) != 0;
                // registers r = 4j .. 4j + 3 hold keys 32 kt + 8j + 4g + 0..3
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const f32x4 x = *reinterpret_cast<const f32x4 *>(&slot[32 * kt + 8 * j + 4 * g]);
#pragma unroll
                    for (int e = 0; e < 4; ++e) mv[kt][4 * j + e] = x[e];
                }
            }
        } else if constexpr (MASK) {
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
        if (!any_live) return;  // nothing visible: the next barrier is at the loop top
        const bool edge = n0 + BN > s.S || (CAUSAL && n0 + BN - 1 > wave_last_q - 31);

        // S^T = K Q^T: rows are keys, columns are this wave's 32 queries.
        f32x16 sacc[NT];
#pragma unroll
        for (int kt = 0; kt < NT; ++kt)
#pragma unroll
            for (int r = 0; r < 16; ++r) sacc[kt][r] = 0.f;
        // The sub-tiles' independent MFMA chains are interleaved (measured faster here than
        // testing liveness once per sub-tile outside its chain).
#pragma unroll
        for (int t4 = 0; t4 < DH; t4 += 4) {
#pragma unroll
            for (int kt = 0; kt < NT; ++kt) {
                if (!live[kt]) continue;
                const f32x4 kk = kread(kt * 32 + lr, g * DH + t4);
                sacc[kt] = mfma_f32(kk[0], qreg[t4 + 0], sacc[kt]);
                sacc[kt] = mfma_f32(kk[1], qreg[t4 + 1], sacc[kt]);
                sacc[kt] = mfma_f32(kk[2], qreg[t4 + 2], sacc[kt]);
                sacc[kt] = mfma_f32(kk[3], qreg[t4 + 3], sacc[kt]);
            }
        }

        if constexpr (ONEBUF) {
            wait_lds();  // K(t)'s reads have returned: the buffer takes K(t + 1)
            if (tn >= 0) issue_tile<D, BN, W, true, false>(sm, kb, vb, tn * BN, s.S, wave, lane);
            // In flight: V(t), then K(t + 1).
            if (tn >= 0) wait_vmem_but<NLD>();
            else wait_vmem();
        }
        // With two or more waves the V operands are read ahead here (their LDS latency hides
        // under the softmax) and each P column feeds its products as soon as it is formed:
        // B8 H12 L1024 causal 131.4 -> 129.8 us, B1 H8 L2048 62.0 -> 60.1 us.  (One-wave
        // workgroups measured faster without: 43.1 against 43.9 us.)
        constexpr bool VAHEAD = D <= 64 && !ONEBUF;
        float vv[VAHEAD ? NT : 1][VAHEAD ? D / 32 : 1][16];
        if constexpr (VAHEAD) {
#pragma unroll
            for (int kt = 0; kt < NT; ++kt)
#pragma unroll
                for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
                    for (int r = 0; r < 16; ++r) vv[kt][dt][r] = vread(kt * 32 + acc_row(r, g), dt * 32 + lr);
        }
        // Scores in log2 units (with a mask; without one the raw products, see csc), masked on
        // edge tiles; tile max per query.
        // A row mask arrives times log2 e, so its score is one FMA with scale log2 e (bit-identical
        // to the two-step form when the scale is a power of two, as at head dims 16, 64 and 256;
        // B16 H16 L512 key padding 101.7 -> 99.9 us).
        if constexpr (ROWMASK) {
#pragma unroll
            for (int kt = 0; kt < NT; ++kt)
#pragma unroll
                for (int r = 0; r < 16; ++r) sacc[kt][r] = fmaf(sacc[kt][r], s.scale_log2, mv[kt][r]);
        } else if constexpr (MASK) {
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
        mx = xor32_max(mx);
        if constexpr (!MASK) mx *= csc;
        // p = 2^(score in log2 units - m)
        auto expo = [&](float x, float m) { return exp2_fast(MASK ? x - m : fmaf(x, csc, -m)); };
        // Lazy rescaling: the exponent reference m_run moves (and O, l are rescaled) only when
        // some lane's tile max exceeds it by more than 8, so P <= 2^8 and most tiles skip the
        // rescale of the accumulator; out = O / l and lse = m_run + log2(l) are unchanged.
        if (__any(mx > m_run + 8.f)) {
            const float m_new = fmaxf(m_run, mx);
            const float alpha = exp2_fast(m_run - (m_new == -INFINITY ? 0.f : m_new));
            l_run *= alpha;
#pragma unroll
            for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
                for (int r = 0; r < 16; ++r) oacc[dt][r] *= alpha;
            m_run = m_new;
        }
        const float m_use = m_run == -INFINITY ? 0.f : m_run;
        float ls = 0.f;
        if constexpr (VAHEAD) {
#pragma unroll
            for (int kt = 0; kt < NT; ++kt)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const float p = expo(sacc[kt][r], m_use);
                    ls += p;
                    if (live[kt]) {
#pragma unroll
                        for (int dt = 0; dt < D / 32; ++dt) oacc[dt] = mfma_f32(vv[kt][dt][r], p, oacc[dt]);
                    }
                }
            l_run += xor32_add(ls);
            return;
        }
#pragma unroll
        for (int kt = 0; kt < NT; ++kt)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float p = expo(sacc[kt][r], m_use);
                sacc[kt][r] = p;
                ls += p;
            }
        l_run += xor32_add(ls);

        // O^T += V^T P^T: A = V[key][d] from LDS, B = P straight from the S^T accumulator.
#pragma unroll
        for (int kt = 0; kt < NT; ++kt) {
            if (!live[kt]) continue;
#pragma unroll
            for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    oacc[dt] = mfma_f32(vread(kt * 32 + acc_row(r, g), dt * 32 + lr), sacc[kt][r],
                                        oacc[dt]);
        }
    };
    if constexpr (ONEBUF) {
        wait_vmem();  // the queries (and tile t_begin): no load of the loop waits for them again
        for (int t = t_begin; t < t_end; ++t) {
            const int tn = t + 1 < t_end ? t + 1 : -1;
            tile(t, sm, sm, tn);
            wait_lds();  // V(t)'s reads have returned: the buffer takes V(t + 1)
            if (tn >= 0) issue_tile<D, BN, W, false, true>(sm, kb, vb, tn * BN, s.S, wave, lane);
        }
    } else if constexpr (ASYNC) {
        for (int t = t_begin; t < t_end; t += 2) {
            tile(t, sm, sm2, t + 1 < t_end ? t + 1 : -1);
            if (t + 1 < t_end) tile(t + 1, sm2, sm, t + 2 < t_end ? t + 2 : -1);
        }
    } else {
        for (int t = t_begin; t < t_end; ++t) tile(t, sm, sm, -1);
    }

    if (qi < s.L) {
        const bool empty = l_run == 0.f;
        const float inv = empty ? 0.f : 1.f / l_run;
        const int64_t row = (int64_t)bh * s.L + qi;
        // A piece of a split range writes its normalized partial and lse (-inf: no visible key)
        // to the row's slot `piece`; fwd_split_merge_kernel combines them.
        const bool partial = SPLIT && npieces > 1;
        float *orow = partial ? a.split_o + (row * a.split_max + piece) * s.E
                              : static_cast<float *>(a.out) + row * s.E;
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
            for (int r = 0; r < 16; r += 4) {
                const int d = dt * 32 + acc_row(r, g);
                if (s.vec) {
                    f32x4 o = {oacc[dt][r] * inv, oacc[dt][r + 1] * inv, oacc[dt][r + 2] * inv,
                               oacc[dt][r + 3] * inv};
                    *reinterpret_cast<f32x4 *>(orow + d) = o;
                } else {
#pragma unroll
                    for (int u = 0; u < 4; ++u)
                        if (d + u < s.E) orow[d + u] = oacc[dt][r + u] * inv;
                }
            }
        if (g == 0) {
            if (partial)
                a.split_lse[row * a.split_max + piece] = empty ? -INFINITY : (m_run + log2_fast(l_run)) * kLn2;
            else
                a.lse[row] = empty ? 0.f : (m_run + log2_fast(l_run)) * kLn2;
        }
    }
}

// The BN-key tiles of one mask row (S keys) that hold any key whose mask is not -inf, counted by
// one wave.  The loads of 8 x 64 keys are all issued before any is tested, so a row costs one
// memory latency per 512 keys instead of one per 64 (C3's step, order pass plus forward: 90.7 ->
// 90.4 us; the rest of the pass is its launch).
template <int BN>
DEVI int live_tiles(const float *row, int S, int lane) {
    constexpr int U = 8;
    int c = 0;
    for (int k0 = 0; k0 < S; k0 += 64 * U) {
        float x[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int key = k0 + 64 * u + lane;
            x[u] = key < S ? row[key] : -INFINITY;
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint64_t live = __ballot(x[u] != -INFINITY);
            if (BN == 64) c += live != 0;
            else c += ((live & 0xffffffffull) != 0) + ((live >> 32) != 0);
        }
    }
    return c;
}

// One wave per (b, h) of a query-independent mask: the number of BN-key tiles that hold any key
// whose mask is not -inf (the tiles the forward computes; the others it skips).
template <int BN>
__global__ __launch_bounds__(64) void rowmask_tiles_kernel(FwdArgs a) {
    static_assert(BN == 32 || BN == 64, "one or two tiles per wave-wide pass");
    const AttnShape &s = a.s;
    const int bh = blockIdx.x, lane = threadIdx.x;
    const float *row = s.mask + (int64_t)(bh / s.H) * s.msb + (int64_t)(bh % s.H) * s.msh;
    const int count = live_tiles<BN>(row, s.S, lane);
    if (lane == 0) a.tiles[bh] = count;
}

// One workgroup: a counting sort of the heads by live tiles, descending (ties in any order; the
// results do not depend on the order).
__global__ __launch_bounds__(1024) void rowmask_order_kernel(FwdArgs a, int ntiles) {
    __shared__ int start[kOrderMaxTiles + 1];
    const int BH = a.s.B * a.s.H, tid = threadIdx.x;
    for (int v = tid; v <= ntiles; v += 1024) start[v] = 0;
    __syncthreads();
    for (int i = tid; i < BH; i += 1024) atomicAdd(&start[a.tiles[i]], 1);
    __syncthreads();
    if (tid == 0) {  // start[v] = number of heads with more live tiles than v
        int run = 0;
        for (int v = ntiles; v >= 0; --v) {
            const int c = start[v];
            start[v] = run;
            run += c;
        }
    }
    __syncthreads();
    for (int i = tid; i < BH; i += 1024) a.order[atomicAdd(&start[a.tiles[i]], 1)] = i;
}

// Masks that depend on the batch and the key only (head and query strides 0: key padding, C3):
// one launch instead of the two above.  One workgroup counts the live tiles of each batch's mask
// row, a wave per row, and sorts the heads by their batch's count, descending.
template <int BN>
__global__ __launch_bounds__(1024) void rowmask_batch_order_kernel(FwdArgs a, int ntiles) {
    static_assert(BN == 32 || BN == 64, "one or two tiles per wave-wide pass");
    __shared__ int count[kOrderMaxBatch];
    __shared__ int start[kOrderMaxTiles + 1];
    const AttnShape &s = a.s;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    for (int v = tid; v <= ntiles; v += 1024) start[v] = 0;
    for (int b = wave; b < s.B; b += 16) {
        const int c = live_tiles<BN>(s.mask + (int64_t)b * s.msb, s.S, lane);
        if (lane == 0) count[b] = c;
    }
    __syncthreads();
    const int BH = s.B * s.H;
    for (int i = tid; i < BH; i += 1024) atomicAdd(&start[count[i / s.H]], 1);
    __syncthreads();
    if (tid == 0) {  // start[v] = number of heads with more live tiles than v
        int run = 0;
        for (int v = ntiles; v >= 0; --v) {
            const int c = start[v];
            start[v] = run;
            run += c;
        }
    }
    __syncthreads();
    for (int i = tid; i < BH; i += 1024) a.order[atomicAdd(&start[count[i / s.H]], 1)] = i;
}

// The split of this instantiation's grid on the current device (fwd_split.hpp).
// Split pieces at D = 128 take the register-staged kernel: it fits two waves per SIMD (the
// asynchronous one needs ~330 registers for its swizzled LDS addresses and runs one), and few
// long rows gain from that (B1 H8 L2048 D128 causal: 111.8 -> 109.5 us in bench.py's schedule
// timings, 125 -> 104 us over 200 back-to-back calls after 1000 warm-up calls) while full grids
// lose (B2 H16 L2048 D128 causal 347 -> 396 us, same back-to-back timing): those keep the
// asynchronous kernel.
template <int D>
constexpr bool kSplitAsync = D != 128;

template <int D, int BN, int W>
FwdSplitPlan plan(const AttnShape &s) {
    const int64_t blocks = (int64_t)(s.L + 32 * W - 1) / (32 * W) * s.B * s.H;
    const int64_t slots = split_slots(
        reinterpret_cast<const void *>(&fwd_f32_kernel<D, BN, W, true, false, kSplitAsync<D>, false, true>), 64 * W,
        blocks);
    return plan_split(s, 32 * W, BN, slots);
}

template <int D, int BN, int W>
hipError_t launch_d(const FwdArgs &args, hipStream_t st) {
    FwdArgs a = args;
    a.s.vec = args.s.vec && args.s.E == D;  // the ABI checked alignment; E must fill D
    const int nqt = (a.s.L + 32 * W - 1) / (32 * W);
    const dim3 grid(nqt * a.s.B * a.s.H), block(64 * W);
    const bool mask = a.s.mask != nullptr;
    if (a.split_o) {
        const FwdSplitPlan p = plan<D, BN, W>(a.s);
        if (p.chunk > 0 && p.bytes <= a.split_bytes) {
            record_schedule(split_chunk, p.chunk);
            record_schedule(split_pieces, p.max_pieces);
            a.split_chunk = p.chunk, a.split_max = p.max_pieces;
            a.split_lse = a.split_o + (size_t)a.s.B * a.s.H * a.s.L * p.max_pieces * a.s.E;
            const dim3 sgrid((unsigned)p.blocks);
            if (a.s.vec && kSplitAsync<D>) {
                if (a.s.causal)
                    return_if(launch(fwd_f32_kernel<D, BN, W, true, false, true, false, true>, sgrid, block, st, a));
                else
                    return_if(launch(fwd_f32_kernel<D, BN, W, false, false, true, false, true>, sgrid, block, st, a));
            } else if (a.s.causal) {
                return_if(launch(fwd_f32_kernel<D, BN, W, true, false, false, false, true>, sgrid, block, st, a));
            } else {
                return_if(launch(fwd_f32_kernel<D, BN, W, false, false, false, false, true>, sgrid, block, st, a));
            }
            const int64_t rows = (int64_t)a.s.B * a.s.H * a.s.L;
            return launch(fwd_split_merge_kernel<float>, dim3((unsigned)((rows + 15) / 16)), dim3(256), st, a,
                          32 * W, BN);
        }
    }
    if constexpr (W == 1) {  // short causal rows without a mask (with_config)
        if (a.s.vec)
            return launch(fwd_f32_kernel<D, BN, W, true, false, true>, grid, block, st, a);
        return launch(fwd_f32_kernel<D, BN, W, true, false, false>, grid, block, st, a);
    } else if (a.s.vec && !(mask && a.s.causal)) {  // (causal + mask: register staging, fewer VGPRs)
        if (a.s.causal)
            return_if(launch(fwd_f32_kernel<D, BN, W, true, false, true>, grid, block, st, a));
        else if (mask && a.s.msl == 0 && BN <= 64) {
            const int ntiles = (a.s.S + BN - 1) / BN;
            if (a.order && a.s.B * a.s.H <= kOrderMaxHeads && ntiles <= kOrderMaxTiles) {
                if (a.s.msh == 0 && a.s.B <= kOrderMaxBatch) {
                    return_if(launch(rowmask_batch_order_kernel<BN>, dim3(1), dim3(1024), st, a, ntiles));
                } else {
                    return_if(launch(rowmask_tiles_kernel<BN>, dim3(a.s.B * a.s.H), dim3(64), st, a));
                    return_if(launch(rowmask_order_kernel, dim3(1), dim3(1024), st, a, ntiles));
                }
                const dim3 ogrid(nqt * 8 * ((a.s.B * a.s.H + 7) / 8));
                return_if(launch(fwd_f32_kernel<D, BN, W, false, true, true, true>, ogrid, block, st, a));
            } else {
                a.order = nullptr;
                return_if(launch(fwd_f32_kernel<D, BN, W, false, true, true, true>, grid, block, st, a));
            }
        }
        else if (mask)
            return_if(launch(fwd_f32_kernel<D, BN, W, false, true, true>, grid, block, st, a));
        else
            return_if(launch(fwd_f32_kernel<D, BN, W, false, false, true>, grid, block, st, a));
    } else if (a.s.causal && mask) {
        return_if(launch(fwd_f32_kernel<D, BN, W, true, true, false>, grid, block, st, a));
    } else if (a.s.causal) {
        return_if(launch(fwd_f32_kernel<D, BN, W, true, false, false>, grid, block, st, a));
    } else if (mask) {
        return_if(launch(fwd_f32_kernel<D, BN, W, false, true, false>, grid, block, st, a));
    } else {
        return_if(launch(fwd_f32_kernel<D, BN, W, false, false, false>, grid, block, st, a));
    }
    return hipSuccess;
}

// The instantiation the forward runs for a shape: head dim D, key tile BN, waves W.  Short causal
// problems take smaller workgroups over 32-key tiles: their causal work units are finer, which
// balances the CUs better (measured on one MI355X: B64 H6 L256 D64 causal 54.0 -> 49.5 us with
// 2 waves; B8 H12 L1024 unchanged; non-causal B16 H16 L512 slower, 161 -> 171 us), and one wave
// each when no mask is given (49.5 -> 43.1 us, the one-buffer path of fwd_f32_kernel).  At D = 64
// the 4-wave workgroups take 32-key tiles: half the LDS of 64-key tiles (32 KB), so four
// workgroups fit a CU instead of two (B8 H12 L1024 causal 148.7 -> 145.7 us, B2 H12 L4096 causal
// 480 -> 457 us).
template <typename F>
auto with_config(const AttnShape &s, F f) {
    const bool small = s.causal && s.L <= 256;
    const bool one = small && s.mask == nullptr;
    if (s.E <= 32) {
        if (one) return f.template operator()<32, 32, 1>();
        return small ? f.template operator()<32, 32, 2>() : f.template operator()<32, 64, 4>();
    }
    if (s.E <= 64) {
        if (one) return f.template operator()<64, 32, 1>();
        return small ? f.template operator()<64, 32, 2>() : f.template operator()<64, 32, 4>();
    }
    return f.template operator()<128, 32, 4>();
}

struct SplitBytes {
    const AttnShape &s;
    template <int D, int BN, int W>
    size_t operator()() const { return plan<D, BN, W>(s).bytes; }
};

struct Launch {
    const FwdArgs &a;
    hipStream_t st;
    template <int D, int BN, int W>
    hipError_t operator()() const { return launch_d<D, BN, W>(a, st); }
};

}  // namespace

size_t fwd_f32_split_bytes(const AttnShape &s) {
    if (s.B == 0 || s.H == 0 || s.L == 0) return 0;
    return with_config(s, SplitBytes{s});
}

hipError_t launch_fwd_f32(const FwdArgs &a, hipStream_t st) {
    if (a.s.B == 0 || a.s.H == 0 || a.s.L == 0) return hipSuccess;
    return with_config(a.s, Launch{a, st});
}

}  // namespace dc
