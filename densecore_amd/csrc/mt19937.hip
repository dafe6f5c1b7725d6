// The reference's CPU generator stream (src/torch_random.rs:9-98, PyTorch's mt19937) drawn on
// the GPU, for dropout masks that are bit-identical to Generator::bernoulli
// (src/torch_random.rs:241-254): element e keeps iff the double built from outputs 2e and
// 2e + 1, (hi << 32 | lo) & (2^53 - 1) times 2^-53, is below p.
//
// The engine's untempered words satisfy x[t + 624] = x[t + 397] ^ twist(x[t], x[t + 1]) for every
// t >= 0 (the in-place update of next_state, src/torch_random.rs:66-77), so the stream is one
// linear recurrence over GF(2).  A window of 624 consecutive words that follows at least one
// update lies in the 19937-dimensional subspace on which that recurrence has the primitive
// characteristic polynomial phi (degree 19937), so the window d words later is
//     W(t + d) = sum_i g_i W(t + i),   g = z^d mod phi,
// a XOR of shifted copies of the sequence (the standard jump-ahead of F2-linear generators).
//
// Layout of one draw of n elements (positions relative to the start of the engine's current
// block of 624 words, r = position of the next output):
//   head      elements [0, Eh), Eh = 64: generated from the current block by one workgroup
//             (mt_base_kernel), which also writes the window at A0 = r + 2 Eh (A0 >= 1, so that
//             window follows an update even when the block is a freshly seeded one);
//   chunks    chunk c covers elements [Eh + c J/2, Eh + (c + 1) J/2), J = 2^17 words; its window
//             is W(A0 + c J), reached from W(A0) through a radix-64 tree of jumps (c = 64 c1 + c0:
//             a jump by c1 2^23, then one by c0 2^17; mt_jump_kernel), and one wave generates its
//             words from that window (mt_chunk_kernel).
// Keep bits: element e is bit e % 32 of word e / 32 (heads and chunks write whole words).  The
// engine block that holds the last output drawn is written back to the state (by the base
// workgroup or by the chunk whose range holds the block's first word), and the host moves
// (left, next) the way next_state/random do.
//
// The jump polynomials (128 of them) are computed once on the host: phi by Berlekamp-Massey on
// 2 * 19937 bits of the stream, then z^(digit * 2^(17 + 6 level)) mod phi by squaring and
// multiplying; the caller uploads them into its own device buffer (dc_mt19937_table_init).
#include <cstring>
#include <mutex>
#include <vector>

#include "common.hpp"
#include "params.hpp"

namespace dc {
namespace mt {

namespace {

// ---------------------------------------------------------------- host: GF(2) polynomials

constexpr int kPW = kTableWords / 2;  // 312 uint64 words: 19968 bits, degree < 19937 fits

inline uint32_t twist(uint32_t u, uint32_t v) {
    return (((u & 0x80000000u) | (v & 0x7fffffffu)) >> 1) ^ ((v & 1u) ? 0x9908b0dfu : 0u);
}

typedef std::vector<uint64_t> Bits;  // bit i of a polynomial = coefficient of z^i

inline bool bit(const Bits &a, int i) { return (a[i >> 6] >> (i & 63)) & 1u; }
inline void flip(Bits &a, int i) { a[i >> 6] ^= 1ull << (i & 63); }

// a ^= b << s (b has nb words; a is large enough).
void xor_shifted(Bits &a, const Bits &b, int nb, int s) {
    const int ws = s >> 6, bs = s & 63;
    for (int i = 0; i < nb; ++i) {
        if (!b[i]) continue;
        a[i + ws] ^= b[i] << bs;
        if (bs) a[i + ws + 1] ^= b[i] >> (64 - bs);
    }
}

// Characteristic polynomial of the engine: Berlekamp-Massey on bit 0 of the untempered words
// x[624 .. 624 + 2 * 19937) of the engine seeded with 5489.
Bits char_poly() {
    const int n = 2 * kDegree;
    std::vector<uint32_t> x(kState + n + 1);
    x[0] = 5489u;
    for (int j = 1; j < kState; ++j) x[j] = 1812433253u * (x[j - 1] ^ (x[j - 1] >> 30)) + (uint32_t)j;
    for (int t = 0; t + kState < (int)x.size(); ++t)
        x[t + kState] = x[t + kM] ^ twist(x[t], x[t + 1]);
    const int W = kPW + 1;
    Bits C(W + 1, 0), B(W + 1, 0), R(W + 1, 0), T;
    C[0] = B[0] = 1;
    int L = 0, m = 1;
    for (int k = 0; k < n; ++k) {
        // R bit j = s[k - j]: shift in s[k].
        for (int w = W; w > 0; --w) R[w] = (R[w] << 1) | (R[w - 1] >> 63);
        R[0] = (R[0] << 1) | (x[kState + k] & 1u);
        int d = 0;
        for (int w = 0; w <= W; ++w) d ^= __builtin_popcountll(C[w] & R[w]) & 1;
        if (!d) {
            ++m;
        } else if (2 * L <= k) {
            T = C;
            xor_shifted(C, B, W + 1 - (m >> 6) - 1, m);
            L = k + 1 - L;
            B = T;
            m = 1;
        } else {
            xor_shifted(C, B, W + 1 - (m >> 6) - 1, m);
            ++m;
        }
    }
    // phi(z) = z^L C(1/z).
    Bits phi(kPW, 0);
    if (L != kDegree) return Bits();
    for (int i = 0; i <= L; ++i)
        if (bit(C, i)) flip(phi, L - i);
    return phi;
}

struct Field {
    Bits phi;

    // a * b mod phi, both of degree < 19937.
    Bits mul(const Bits &a, const Bits &b) const {
        Bits tab[16];
        for (int w = 0; w < 16; ++w) {
            tab[w].assign(kPW + 1, 0);
            for (int s = 0; s < 4; ++s)
                if (w >> s & 1) xor_shifted(tab[w], b, kPW, s);
        }
        Bits r(2 * kPW + 2, 0);
        for (int p = 0; p < kPW * 16; ++p) {
            const int nib = (int)(a[p >> 4] >> (4 * (p & 15))) & 15;
            if (nib) xor_shifted(r, tab[nib], kPW + 1, 4 * p);
        }
        return reduce(r);
    }

    // r mod phi for any length of r (top-down: each step clears bit i and touches no bit above).
    Bits reduce(Bits r) const {
        const int top = (int)r.size() * 64 - 1;
        r.resize(r.size() + kPW + 2, 0);
        for (int i = top; i >= kDegree; --i)
            if (bit(r, i)) xor_shifted(r, phi, kPW, i - kDegree);
        r.resize(kPW);
        return r;
    }

    // z^e mod phi (square and multiply from the top set bit of e).
    Bits pow_z(uint64_t e) const {
        Bits r(kPW, 0);
        r[0] = 1;
        for (int b = 63 - (e ? __builtin_clzll(e) : 63); b >= 0; --b) {
            r = mul(r, r);
            if (e >> b & 1) {
                Bits s(kPW + 1, 0);
                xor_shifted(s, r, kPW, 1);
                r = reduce(s);
            }
        }
        return r;
    }
};

struct Tables {
    bool ok = false;
    Field f;
    std::vector<uint32_t> words;  // kTablePolys polynomials of kTableWords uint32 words
};

const Tables &tables() {
    static Tables t;
    static std::once_flag once;
    std::call_once(once, [] {
        t.f.phi = char_poly();
        if (t.f.phi.empty()) return;
        t.words.assign((size_t)kTablePolys * kTableWords, 0);
        Bits base = t.f.pow_z(1ull << kChunkLog2);  // z^(2^17)
        for (int level = 0; level < kJumpLevels; ++level) {
            Bits p(kPW, 0);
            p[0] = 1;
            for (int digit = 0; digit < kRadix; ++digit) {
                uint32_t *dst = &t.words[((size_t)level * kRadix + digit) * kTableWords];
                std::memcpy(dst, p.data(), kTableWords * sizeof(uint32_t));
                p = t.f.mul(p, base);
            }
            base = p;  // base^16
        }
        t.ok = true;
    });
    return t;
}

// The window d words after `win` (which must follow at least one engine update).
void jump_host(const Field &f, const uint32_t *win, uint64_t d, uint32_t *out) {
    const Bits g = f.pow_z(d);
    std::vector<uint32_t> seq(kState + kDegree + 1);
    std::memcpy(seq.data(), win, kState * sizeof(uint32_t));
    for (int t = 0; t + kState < (int)seq.size(); ++t)
        seq[t + kState] = seq[t + kM] ^ twist(seq[t], seq[t + 1]);
    std::vector<uint32_t> acc(kState, 0);
    for (int i = 0; i < kDegree; ++i)
        if (bit(g, i))
            for (int j = 0; j < kState; ++j) acc[j] ^= seq[i + j];
    std::memcpy(out, acc.data(), kState * sizeof(uint32_t));
}

// ---------------------------------------------------------------- device

DEVI uint32_t twist_d(uint32_t u, uint32_t v) {
    return (((u & 0x80000000u) | (v & 0x7fffffffu)) >> 1) ^ ((v & 1u) ? 0x9908b0dfu : 0u);
}

// src/torch_random.rs:86-89.
DEVI uint32_t temper(uint32_t y) {
    y ^= y >> 11;
    y ^= (y << 7) & 0x9d2c5680u;
    y ^= (y << 15) & 0xefc60000u;
    y ^= y >> 18;
    return y;
}

// uniform_f64 (src/torch_random.rs:106-110) of the pair (hi, lo) compared with p: with
// r = (hi << 32 | lo) & (2^53 - 1), r * 2^-53 < p exactly when r < ceil(p * 2^53) (both sides
// scaled by a power of two, r an integer), the threshold the host computes.
DEVI bool keep(uint32_t hi, uint32_t lo, uint64_t thr) {
    const uint64_t r = (((uint64_t)hi << 32) | lo) & ((1ull << 53) - 1);
    return r < thr;
}

// Orders this wave's LDS accesses around it (the LDS executes one wave's instructions in order,
// so the compiler is the only thing that could move a read above another lane's write): the
// wave-scope release / wave barrier / acquire sequence, no wait on global stores.
DEVI void wave_lds_order() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// One workgroup: the current block `state` (positions 0..623), the words after it up to
// A0 + 623, the head's keep bits, the window at A0, and (when the last drawn output lies before
// A0) the engine block that holds it.
constexpr int kBaseWords = 2048;

__global__ __launch_bounds__(256) void mt_base_kernel(MtArgs a) {
    __shared__ uint32_t x[kBaseWords];
    const int tid = threadIdx.x;
    for (int i = tid; i < kState; i += 256) x[i] = a.state[i];
    __syncthreads();
    const int total = a.a0 + kState;  // positions [0, total) are needed
    for (int base = kState; base < total; base += 128) {
        const int u = base + tid;
        if (tid < 128 && u < total) x[u] = x[u - 227] ^ twist_d(x[u - 624], x[u - 623]);
        __syncthreads();
    }
    // Head elements [0, min(Eh, n)): outputs r + 2e, r + 2e + 1, 64 elements per wave pass.
    const int lane = tid & 63, wave = tid >> 6;
    const int64_t head = a.n < a.eh ? a.n : a.eh;
    for (int e0 = wave * 64; e0 < a.eh; e0 += 256) {
        const int e = e0 + lane;
        bool k = false;
        if (e < head) k = keep(temper(x[a.r + 2 * e]), temper(x[a.r + 2 * e + 1]), a.thr);
        const uint64_t m = __ballot(k);
        if (e0 < head) {
            if (lane == 0) a.bits[e0 >> 5] = (uint32_t)m;
            if (lane == 1 && e0 + 32 < head) a.bits[(e0 >> 5) + 1] = (uint32_t)(m >> 32);
        }
    }
    for (int i = tid; i < kState; i += 256) a.win[i] = x[a.a0 + i];
    if (a.state_block >= 0 && a.state_block * kState < a.a0)
        for (int i = tid; i < kState; i += 256) a.state[i] = x[a.state_block * kState + i];
}

// One workgroup per destination window: dst[w] = W(src[w / 64] + digit * step), digit = w % 64,
// with g = table[level][digit].  The sequence seq[i] = x[src + i], i < 20576, is generated into
// LDS once; wave v sums the g-terms of i in its eighth of [0, 19937): lanes < 52 own 12
// consecutive output words each and read a 20-word window of seq per group of 8 terms; the
// eight partial windows are then XORed together.
constexpr int kSeqWords = 20576;                        // >= 19937 + 624 + 15, a multiple of 8
constexpr int kJumpWaves = 8;
constexpr int kGroups = (kDegree + 7) / 8;              // groups of 8 terms
constexpr int kGroupsPerWave = (kGroups + kJumpWaves - 1) / kJumpWaves;
constexpr int kOwn = 12, kOwners = kState / kOwn;       // 52 owner lanes per wave

__global__ __launch_bounds__(512) void mt_jump_kernel(const uint32_t *src, uint32_t *dst,
                                                      const uint32_t *table, int level, int count) {
    __shared__ __align__(16) uint32_t seq[kSeqWords];
    const int w = blockIdx.x;
    if (w >= count) return;
    const int digit = w % kRadix;
    const uint32_t *in = src + (size_t)(w / kRadix) * kState;
    uint32_t *out = dst + (size_t)w * kState;
    const int tid = threadIdx.x;
    if (digit == 0) {
        for (int i = tid; i < kState; i += 512) out[i] = in[i];
        return;
    }
    const uint32_t *g = table + ((size_t)level * kRadix + digit) * kTableWords;
    for (int i = tid; i < kState; i += 512) seq[i] = in[i];
    __syncthreads();
    for (int base = kState; base < kSeqWords; base += 227) {  // x[u] needs x[u - 227]: 227 at a time
        const int u = base + tid;
        if (tid < 227 && u < kSeqWords) seq[u] = seq[u - 227] ^ twist_d(seq[u - 624], seq[u - 623]);
        __syncthreads();
    }
    // Every lane runs the sum (lanes past the owners repeat the last owner's words and store
    // nothing), so the group index and the polynomial bits are wave-uniform: the bits come from
    // two VGPRs loaded up front (word w of this wave's 78 at lane w % 64 of gw[w / 64]) through
    // readlane, and the term tests are scalar branches.
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int j0 = kOwn * (lane < kOwners ? lane : kOwners - 1);
    const int g_begin = wave * kGroupsPerWave;
    const int g_end = g_begin + kGroupsPerWave < kGroups ? g_begin + kGroupsPerWave : kGroups;
    static_assert(kGroupsPerWave % 4 == 0 && kGroupsPerWave / 4 <= 128, "g words per wave");
    const int w0 = g_begin / 4;  // first g word of this wave (4 groups of 8 bits per word)
    const uint32_t gw0 = w0 + lane < kTableWords ? g[w0 + lane] : 0u;
    const uint32_t gw1 = w0 + 64 + lane < kTableWords ? g[w0 + 64 + lane] : 0u;
    uint32_t acc[kOwn];
#pragma unroll
    for (int u = 0; u < kOwn; ++u) acc[u] = 0;
    for (int gi = g_begin; gi < g_end; ++gi) {
        const int wi = (gi >> 2) - w0;
        const uint32_t word = wi < 64 ? __builtin_amdgcn_readlane(gw0, wi)
                                      : __builtin_amdgcn_readlane(gw1, wi - 64);
        const uint32_t gb = (word >> (8 * (gi & 3))) & 0xffu;  // g bits 8 gi .. 8 gi + 7
        if (gb == 0) continue;
        uint32_t win[kOwn + 8];  // seq[8 gi + j0 + 0 .. 19]: five 16-byte reads
#pragma unroll
        for (int u = 0; u < kOwn + 8; u += 4) {
            const u32x4 x = *reinterpret_cast<const u32x4 *>(&seq[8 * gi + j0 + u]);
            win[u] = x[0], win[u + 1] = x[1], win[u + 2] = x[2], win[u + 3] = x[3];
        }
#pragma unroll
        for (int d = 0; d < 8; ++d)
            if (gb >> d & 1u)
#pragma unroll
                for (int u = 0; u < kOwn; ++u) acc[u] ^= win[d + u];
    }
    __syncthreads();  // every wave is done with seq: reuse it for the partial windows
    if (lane < kOwners)
#pragma unroll
        for (int u = 0; u < kOwn; ++u) seq[wave * kState + j0 + u] = acc[u];
    __syncthreads();
    for (int j = tid; j < kState; j += 512) {
        uint32_t x = 0;
#pragma unroll
        for (int v = 0; v < kJumpWaves; ++v) x ^= seq[v * kState + j];
        out[j] = x;
    }
}

// One wave per pair of chunks, one chunk per half-wave (chunks 2 b and 2 b + 1): each half
// makes 64 words (32 elements, one word of keep bits) per step from its chunk's window in its own
// LDS ring.  A word depends on the word 227 before it, so a step's words depend only on steps
// three or more back: one LDS ordering point every three steps is enough, and the three steps
// between them overlap their LDS latency.
struct Half {
    int64_t e_begin;  // first element of the chunk
    int n;            // elements of the chunk
    int words;        // words to make: 2 n, or up to the end of the engine block it writes back
    int sb;           // that block's first word (relative), or -1
};

DEVI Half half_of(const MtArgs &a, int c, int chunks) {
    Half h{0, 0, 0, -1};
    if (c >= chunks) return h;
    h.e_begin = a.eh + (int64_t)c * (kChunkWords / 2);
    const int64_t n = a.n - h.e_begin;
    h.n = n < kChunkWords / 2 ? (int)n : kChunkWords / 2;
    h.words = 2 * h.n;
    const int64_t chunk_pos = a.a0 + (int64_t)c * kChunkWords;  // relative position of word 0
    if (a.state_block >= 0 && a.state_block * (int64_t)kState >= a.a0) {
        const int64_t sb = a.state_block * (int64_t)kState - chunk_pos;
        if (sb >= 0 && sb < kChunkWords) {
            h.sb = (int)sb;
            if (h.sb + kState > h.words) h.words = h.sb + kState;
        }
    }
    return h;
}

__global__ __launch_bounds__(64) void mt_chunk_kernel(MtArgs a, const uint32_t *wins, int chunks) {
    __shared__ __align__(16) uint32_t rings[2][1024];
    const int lane = threadIdx.x, half = lane >> 5, hl = lane & 31;
    const int c = 2 * blockIdx.x + half;
    const Half hh = half_of(a, c, chunks);
    const int words_max = max(half_of(a, 2 * blockIdx.x, chunks).words,
                              half_of(a, 2 * blockIdx.x + 1, chunks).words);
    uint32_t *ring = rings[half];
    if (c < chunks) {
        const uint32_t *win = wins + (size_t)c * kState;
        for (int i = hl; i < kState; i += 32) ring[i] = win[i];
    }
    wave_lds_order();
    uint32_t *bits = a.bits + (hh.e_begin >> 5);  // e_begin is a multiple of 64
    const uint64_t thr = a.thr;
    // Keep bits of the pair (w0, w1) at words u0, u0 + 1 of this half's step starting at base.
    auto emit = [&](int base, uint32_t w0, uint32_t w1) {
        const int e = base / 2 + hl;
        const uint64_t r = (((uint64_t)temper(w0) << 32) | temper(w1)) & ((1ull << 53) - 1);
        const uint64_t m = __ballot(e < hh.n && r < thr);
        if (hl == 0 && base / 2 < hh.n) bits[base / 64] = (uint32_t)(m >> (32 * half));
    };
    auto make = [&](int u0, uint32_t &w0, uint32_t &w1) {
        const uint32_t x0 = ring[(u0 - 624) & 1023], x1 = ring[(u0 - 623) & 1023];
        const uint32_t x2 = ring[(u0 - 622) & 1023];
        w0 = ring[(u0 - 227) & 1023] ^ twist_d(x0, x1);
        w1 = ring[(u0 - 226) & 1023] ^ twist_d(x1, x2);
        *reinterpret_cast<uint2 *>(&ring[u0 & 1023]) = make_uint2(w0, w1);
    };
    // Words 0 .. 639: the window, then the first generated words (which read only the window).
    for (int base = 0; base < 640; base += 64) {
        const int u0 = base + 2 * hl;
        uint32_t w0, w1;
        if (u0 < kState) {
            w0 = ring[u0];
            w1 = ring[u0 + 1];
        } else {
            make(u0, w0, w1);
        }
        emit(base, w0, w1);
    }
    wave_lds_order();
    bool captured = false;
    for (int base = 640; base < words_max; base += 192) {
        // All reads of the three steps first (none of them reads a word the three steps
        // write), then the words, the ring writes and the keep bits.
        uint32_t x[3][5];
#pragma unroll
        for (int k = 0; k < 3; ++k) {
            const int u0 = base + 64 * k + 2 * hl;
            x[k][0] = ring[(u0 - 624) & 1023];
            x[k][1] = ring[(u0 - 623) & 1023];
            x[k][2] = ring[(u0 - 622) & 1023];
            x[k][3] = ring[(u0 - 227) & 1023];
            x[k][4] = ring[(u0 - 226) & 1023];
        }
        // Three independent chains, straight-line: words, ring writes, keep ballots; then the
        // (branching) stores of the three keep words.
        uint32_t w[3][2];
#pragma unroll
        for (int k = 0; k < 3; ++k) {
            w[k][0] = x[k][3] ^ twist_d(x[k][0], x[k][1]);
            w[k][1] = x[k][4] ^ twist_d(x[k][1], x[k][2]);
        }
#pragma unroll
        for (int k = 0; k < 3; ++k)
            *reinterpret_cast<uint2 *>(&ring[(base + 64 * k + 2 * hl) & 1023]) = make_uint2(w[k][0], w[k][1]);
        uint64_t m[3];
#pragma unroll
        for (int k = 0; k < 3; ++k) {
            const int e = (base + 64 * k) / 2 + hl;
            const uint64_t r = (((uint64_t)temper(w[k][0]) << 32) | temper(w[k][1])) & ((1ull << 53) - 1);
            m[k] = __ballot(e < hh.n && r < thr);
        }
        if (hl == 0) {
#pragma unroll
            for (int k = 0; k < 3; ++k)
                if ((base + 64 * k) / 2 < hh.n) bits[(base + 64 * k) / 64] = (uint32_t)(m[k] >> (32 * half));
        }
        wave_lds_order();
        // The engine block this chunk writes back: copied once its last word is made (the ring
        // still holds it: at most 624 + 191 words were made since its first).
        if (hh.sb >= 0 && !captured && base + 192 >= hh.sb + kState) {
            for (int i = hl; i < kState; i += 32) a.state[i] = ring[(hh.sb + i) & 1023];
            captured = true;
        }
    }
    if (hh.sb >= 0 && !captured)  // the block lies within words 0 .. 639
        for (int i = hl; i < kState; i += 32) a.state[i] = ring[(hh.sb + i) & 1023];
}

// y = x * (keep ? scale : 0): the reference's input * noise, noise = bernoulli / float32(1 - p)
// (python/densecore/functional.py:244, 638-641).  Four elements per thread (one 16-byte load
// and store, four bits of one word) when the tensors allow it.
__global__ __launch_bounds__(256) void dropout_apply_kernel(const uint32_t *bits, int64_t n, float scale,
                                                            const float *x, float *y) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    const bool k = (bits[i >> 5] >> (i & 31)) & 1u;
    y[i] = x[i] * (k ? scale : 0.0f);
}

__global__ __launch_bounds__(256) void dropout_apply4_kernel(const uint32_t *bits, int64_t n4, float scale,
                                                             const f32x4 *x, f32x4 *y) {
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (t >= n4) return;
    const uint32_t b = bits[t >> 3] >> (4 * (t & 7));
    f32x4 v = load_nt(x + t);  // x and y stream through once
#pragma unroll
    for (int c = 0; c < 4; ++c) v[c] = v[c] * ((b >> c & 1u) ? scale : 0.0f);
    __builtin_nontemporal_store(v, y + t);
}

}  // namespace

size_t window_words(int chunks) {
    if (chunks == 0) return kState;
    const int n1 = (chunks + kRadix - 1) / kRadix;
    return (size_t)(1 + n1 + chunks) * kState;
}

bool tables_ready() { return tables().ok; }

const uint32_t *table_words() { return tables().ok ? tables().words.data() : nullptr; }

bool jump_window_host(const uint32_t *win, uint64_t d, uint32_t *out) {
    const Tables &t = tables();
    if (!t.ok) return false;
    jump_host(t.f, win, d, out);
    return true;
}

void twist_block_host(const uint32_t *in, uint32_t *out) {
    uint32_t x[2 * kState];
    std::memcpy(x, in, kState * sizeof(uint32_t));
    for (int t = 0; t < kState; ++t) x[t + kState] = x[t + kM] ^ twist(x[t], x[t + 1]);
    std::memcpy(out, x + kState, kState * sizeof(uint32_t));
}

hipError_t launch_bernoulli(const MtArgs &a, const uint32_t *table, int chunks, uint32_t *wins,
                            hipStream_t st) {
    return_if(launch(mt_base_kernel, dim3(1), dim3(256), st, a));
    if (chunks == 0) return hipSuccess;
    // Radix-64 tree: level 1 (c1), then level 0 (c0).  Window arrays are carved from `wins`
    // (window_words(chunks) words): [W(A0)] [n1 level-1 windows] [chunk windows].
    const int n1 = (chunks + kRadix - 1) / kRadix;
    uint32_t *l1 = wins + kState, *l0 = l1 + (size_t)n1 * kState;
    return_if(launch(mt_jump_kernel, dim3(n1), dim3(512), st, (const uint32_t *)wins, l1, table, 1, n1));
    return_if(launch(mt_jump_kernel, dim3(chunks), dim3(512), st, (const uint32_t *)l1, l0, table, 0, chunks));
    return launch(mt_chunk_kernel, dim3((chunks + 1) / 2), dim3(64), st, a, (const uint32_t *)l0, chunks);
}

hipError_t launch_dropout_apply(const uint32_t *bits, int64_t n, float scale, const float *x, float *y,
                                hipStream_t st) {
    if (n % 4 == 0 && ((uintptr_t)x & 15) == 0 && ((uintptr_t)y & 15) == 0) {
        const int64_t n4 = n / 4;
        return launch(dropout_apply4_kernel, dim3((unsigned)((n4 + 255) / 256)), dim3(256), st, bits, n4,
                      scale, reinterpret_cast<const f32x4 *>(x), reinterpret_cast<f32x4 *>(y));
    }
    return launch(dropout_apply_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), st, bits, n, scale, x, y);
}

}  // namespace mt
}  // namespace dc
