// bfloat16 attention forward (fp32 accumulation) on CDNA4 MFMA (v_mfma_f32_32x32x16_bf16).
//
// Same mathematics as the float32 kernel and as DenseCore's torch_attention::forward
// (src/torch_attention.rs:143-284) evaluated on the bf16 inputs: scores, softmax state and
// the output accumulator are float32.  P enters the P V product as two bf16 terms
// (hi = bf16(P), lo = bf16(P - hi)), so it is carried to about 2^-17 rather than bf16's 2^-9;
// the only bf16 rounding left is the output's own.  Output is bf16, lse float32.
//
//   * 4 waves x 32 queries per workgroup; queries stay in VGPRs as bf16x8 B operands of
//     S^T = K Q^T (keys x queries), so the softmax state is per lane as in the fp32 kernel;
//   * K tiles are staged naturally in LDS ([key][d], ds_read_b128 along d);
//   * V tiles are transposed on their way into LDS ([d][key]): each thread loads a 4-key x
//     8-dim block (four 16-byte rows), transposes it in registers with byte permutes and
//     writes eight 8-byte columns, so that O^T += V^T P^T reads 4 consecutive keys per lane;
//   * P goes from the S^T accumulator straight into the bf16 B operand (the reduction index of
//     the MFMA is permuted to match the accumulator's row order);
//   * the running max moves only when a tile's max exceeds it by more than 8 (base 2), so the
//     output accumulator is rarely rescaled.
#include "common.hpp"
#include "params.hpp"

namespace dc {
namespace {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kBM = 32 * kWaves;
constexpr int kBN = 64;

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <int D>
struct alignas(16) FwdSmemBf16 {
    __bf16 k[kBN][D + 8];   // row stride = D/2 + 4 words: ds_read_b128 conflict-free
    // [d][key] with the two middle 4-key groups of every 16 swapped (see vt_col), so a lane's
    // 8 keys of one MFMA step are contiguous; row stride 36 words: ds_read_b128 conflict-free.
    __bf16 vt[D][kBN + 8];
};

// Column of 4-key group kb4 in vt: inside each 16 keys the groups are stored 0, 2, 1, 3, so that
// the keys {4g..4g+3, 8+4g..8+4g+3} a half-wave g feeds one bf16 MFMA step sit at 8g..8g+7.
DEVI int vt_col(int kb4) {
    const int grp = kb4 & 3;
    return (kb4 & ~3) * 4 + (grp == 1 ? 2 : grp == 2 ? 1 : grp) * 4;
}

// Low / high 16 bits of two dwords packed into one: (a.lo, b.lo) and (a.hi, b.hi).
DEVI uint32_t pack_lo(uint32_t a, uint32_t b) { return __builtin_amdgcn_perm(b, a, 0x05040100u); }
DEVI uint32_t pack_hi(uint32_t a, uint32_t b) { return __builtin_amdgcn_perm(b, a, 0x07060302u); }

// One thread's share of a K/V tile: K chunks of 8 dims, and one 4-key x 8-dim V block.
template <int D>
struct StageBf16 {
    static constexpr int KCH = kBN * D / 8;          // 16-byte K chunks per tile
    static constexpr int KN = (KCH + kThreads - 1) / kThreads;
    static constexpr int VBLK = (kBN / 4) * (D / 8); // 4x8 V blocks per tile
    static constexpr int VN = (VBLK + kThreads - 1) / kThreads;
    u32x4 k[KN];
    u32x4 v[VN][4];

    // vec: E == D and 16-byte aligned rows.  Otherwise element loads with bounds.
    DEVI void load(const __bf16 *kb, const __bf16 *vb, int n0, int S, int E, bool vec, int tid) {
#pragma unroll
        for (int j = 0; j < KN; ++j) {
            const int i = tid + kThreads * j;
            const int r = i / (D / 8), c = (i % (D / 8)) * 8, key = n0 + r;
            k[j] = load8(kb, key, c, S, E, vec && i < KCH, i < KCH);
        }
#pragma unroll
        for (int j = 0; j < VN; ++j) {
            const int blk = tid + kThreads * j;
            const int kb4 = blk / (D / 8), c = (blk % (D / 8)) * 8;
#pragma unroll
            for (int u = 0; u < 4; ++u)
                v[j][u] = load8(vb, n0 + kb4 * 4 + u, c, S, E, vec && blk < VBLK, blk < VBLK);
        }
    }
    static DEVI u32x4 load8(const __bf16 *base, int key, int c, int S, int E, bool vec, bool valid) {
        if (vec && key < S) return *reinterpret_cast<const u32x4 *>(base + (int64_t)key * D + c);
        u32x4 x = {0u, 0u, 0u, 0u};
        if (valid && key < S) {
            uint16_t h[8];
#pragma unroll
            for (int e = 0; e < 8; ++e)
                h[e] = c + e < E ? __builtin_bit_cast(uint16_t, base[(int64_t)key * E + c + e])
                                 : (uint16_t)0;
#pragma unroll
            for (int w = 0; w < 4; ++w) x[w] = (uint32_t)h[2 * w] | ((uint32_t)h[2 * w + 1] << 16);
        }
        return x;
    }
    DEVI void store(FwdSmemBf16<D> &sm, int tid) const {
#pragma unroll
        for (int j = 0; j < KN; ++j) {
            const int i = tid + kThreads * j;
            if (i < KCH) {
                const int r = i / (D / 8), c = (i % (D / 8)) * 8;
                *reinterpret_cast<u32x4 *>(&sm.k[r][c]) = k[j];
            }
        }
#pragma unroll
        for (int j = 0; j < VN; ++j) {
            const int blk = tid + kThreads * j;
            if (blk >= VBLK) continue;
            const int kb4 = blk / (D / 8), c = (blk % (D / 8)) * 8;
            // Column e of the 4x8 block = (row0[e], row1[e], row2[e], row3[e]).
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                const u32x2 even = {pack_lo(v[j][0][w], v[j][1][w]), pack_lo(v[j][2][w], v[j][3][w])};
                const u32x2 odd = {pack_hi(v[j][0][w], v[j][1][w]), pack_hi(v[j][2][w], v[j][3][w])};
                *reinterpret_cast<u32x2 *>(&sm.vt[c + 2 * w][vt_col(kb4)]) = even;
                *reinterpret_cast<u32x2 *>(&sm.vt[c + 2 * w + 1][vt_col(kb4)]) = odd;
            }
        }
    }
};

template <int D, bool CAUSAL, bool MASK>
__global__ __launch_bounds__(kThreads) void fwd_bf16_kernel(FwdArgs a) {
    constexpr int NT = kBN / 32;
    constexpr int KS = D / 16;  // MFMA k-steps over the head dim
    __shared__ FwdSmemBf16<D> sm;

    const AttnShape &s = a.s;
    const int tid = threadIdx.x, lane = tid & 63, lr = lane & 31, g = lane >> 5;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: branches stay scalar
    const int BH = s.B * s.H;
    const int nqt = (s.L + kBM - 1) / kBM;
    const int bid = blockIdx.x;
    const int qt = CAUSAL ? nqt - 1 - bid / BH : bid / BH;
    const int bh = bid % BH, b = bh / s.H, h = bh % s.H, hk = h / s.repeat;
    const int q0 = qt * kBM;
    const int qi = q0 + wave * 32 + lr;
    const int wave_last_q = q0 + wave * 32 + 31;

    const __bf16 *kb = static_cast<const __bf16 *>(a.k) + (int64_t)(b * s.Hkv + hk) * s.S * s.E;
    const __bf16 *vb = static_cast<const __bf16 *>(a.v) + (int64_t)(b * s.Hkv + hk) * s.S * s.E;

    // Queries: step t, half g supplies Q[qi][16t + 8g + 0..7].
    bf16x8 qreg[KS];
    {
        const __bf16 *qrow = static_cast<const __bf16 *>(a.q) + ((int64_t)bh * s.L + qi) * s.E;
#pragma unroll
        for (int t = 0; t < KS; ++t) {
            const int d0 = 16 * t + 8 * g;
            if (s.vec && qi < s.L) {
                qreg[t] = *reinterpret_cast<const bf16x8 *>(qrow + d0);
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    qreg[t][e] = (qi < s.L && d0 + e < s.E) ? qrow[d0 + e] : static_cast<__bf16>(0.f);
            }
        }
    }
    const float *mrow = nullptr;
    if (MASK) mrow = s.mask + (int64_t)b * s.msb + (int64_t)h * s.msh + (int64_t)qi * s.msl;

    f32x16 oacc[D / 32];
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) oacc[dt][r] = 0.f;
    float m_run = -INFINITY, l_run = 0.f;

    const int kv_end = CAUSAL ? min(q0 + kBM, s.S) : s.S;
    const int ntiles = (kv_end + kBN - 1) / kBN;

    StageBf16<D> stage;
    if (ntiles > 0) stage.load(kb, vb, 0, s.S, s.E, s.vec, tid);

    for (int t = 0; t < ntiles; ++t) {
        const int n0 = t * kBN;
        __syncthreads();
        stage.store(sm, tid);
        __syncthreads();
        if (t + 1 < ntiles) stage.load(kb, vb, n0 + kBN, s.S, s.E, s.vec, tid);

        bool live[NT];
#pragma unroll
        for (int kt = 0; kt < NT; ++kt)
            live[kt] = (n0 + kt * 32 < s.S) && (!CAUSAL || n0 + kt * 32 <= wave_last_q);

        f32x16 sacc[NT];
#pragma unroll
        for (int kt = 0; kt < NT; ++kt)
#pragma unroll
            for (int r = 0; r < 16; ++r) sacc[kt][r] = 0.f;
        // All sub-tiles live (every tile but the causal diagonal): the sub-tiles' independent
        // MFMA chains are interleaved.  Otherwise one uniform test per sub-tile, outside its
        // chain (a test inside the chain makes the compiler copy the accumulator around).
        auto s_step = [&](int kt, int st) {
            const bf16x8 kk = *reinterpret_cast<const bf16x8 *>(&sm.k[kt * 32 + lr][16 * st + 8 * g]);
            sacc[kt] = mfma_bf16(kk, qreg[st], sacc[kt]);
        };
        if (live[NT - 1]) {
#pragma unroll
            for (int st = 0; st < KS; ++st)
#pragma unroll
                for (int kt = 0; kt < NT; ++kt) s_step(kt, st);
        } else {
#pragma unroll
            for (int kt = 0; kt < NT; ++kt) {
                if (!live[kt]) continue;
#pragma unroll
                for (int st = 0; st < KS; ++st) s_step(kt, st);
            }
        }

        float mx = -INFINITY;
#pragma unroll
        for (int kt = 0; kt < NT; ++kt)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int key = n0 + kt * 32 + acc_row(r, g);
                float x;
                if (MASK) {
                    const float mv = (key < s.S && qi < s.L) ? mrow[key] : 0.f;
                    x = (sacc[kt][r] * s.scale + mv) * kLog2e;
                } else {
                    x = sacc[kt][r] * s.scale_log2;
                }
                if (key >= s.S || (CAUSAL && key > qi) || !live[kt]) x = -INFINITY;
                sacc[kt][r] = x;
                mx = fmaxf(mx, x);
            }
        mx = xor32_max(mx);
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
#pragma unroll
        for (int kt = 0; kt < NT; ++kt)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float p = exp2_fast(sacc[kt][r] - m_use);
                sacc[kt][r] = p;
                ls += p;
            }
        l_run += xor32_add(ls);

        // O^T += V^T P^T, 16 keys per MFMA: registers 8u..8u+7 of the S^T accumulator hold
        // keys 16u + {4g..4g+3, 8+4g..8+4g+3} of the 32-key sub-tile, stored contiguously in vt.
#pragma unroll
        for (int kt = 0; kt < NT; ++kt) {
            if (!live[kt]) continue;
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                bf16x8 ph, pl;
                split_bf16(sacc[kt], 8 * u, ph, pl);
                const int kc = kt * 32 + 16 * u + 8 * g;
#pragma unroll
                for (int dt = 0; dt < D / 32; ++dt) {
                    const bf16x8 va = *reinterpret_cast<const bf16x8 *>(&sm.vt[dt * 32 + lr][kc]);
                    oacc[dt] = mfma_bf16(va, ph, oacc[dt]);
                    oacc[dt] = mfma_bf16(va, pl, oacc[dt]);
                }
            }
        }
    }

    if (qi < s.L) {
        const bool empty = l_run == 0.f;
        const float inv = empty ? 0.f : 1.f / l_run;
        __bf16 *orow = static_cast<__bf16 *>(a.out) + ((int64_t)bh * s.L + qi) * s.E;
#pragma unroll
        for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
            for (int r = 0; r < 16; r += 4) {
                const int d = dt * 32 + acc_row(r, g);
                if (s.vec) {
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

template <int D>
hipError_t launch_d(const FwdArgs &args, hipStream_t st) {
    FwdArgs a = args;
    a.s.vec = args.s.vec && args.s.E == D;
    const int nqt = (a.s.L + kBM - 1) / kBM;
    const dim3 grid(nqt * a.s.B * a.s.H), block(kThreads);
    const bool mask = a.s.mask != nullptr;
    if (a.s.causal && mask)
        return_if(launch(fwd_bf16_kernel<D, true, true>, grid, block, st, a));
    else if (a.s.causal)
        return_if(launch(fwd_bf16_kernel<D, true, false>, grid, block, st, a));
    else if (mask)
        return_if(launch(fwd_bf16_kernel<D, false, true>, grid, block, st, a));
    else
        return_if(launch(fwd_bf16_kernel<D, false, false>, grid, block, st, a));
    return hipSuccess;
}

}  // namespace

hipError_t launch_fwd_bf16(const FwdArgs &a, hipStream_t st) {
    if (a.s.B == 0 || a.s.H == 0 || a.s.L == 0) return hipSuccess;
    if (a.s.E <= 32) return launch_d<32>(a, st);
    if (a.s.E <= 64) return launch_d<64>(a, st);
    return launch_d<128>(a, st);
}

}  // namespace dc
