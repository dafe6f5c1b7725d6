// Single-query (decode) attention over a contiguous KV cache: split-KV partials + merge.
//
// The reference has no decode kernel: a decode step is torch_attention::forward with L = 1,
// non-causal (src/torch_attention.rs:157, 176-180), i.e. for each (batch, head)
//     out = softmax(scale * q k^T) v,  lse = max + ln(sum).
// That is a streaming read of K and V with a few flops per byte, so this path is bound by HBM
// bandwidth, not by the matrix cores.  Layout and work split:
//
//   * grid = B*H*splits workgroups: each owns split_len consecutive keys of one head;
//   * a lane loads 16 bytes per row (4 floats or 8 bf16), D/VEC lanes cover one key row, so
//     every global load instruction of a wave reads whole, contiguous 64-byte-aligned rows;
//   * pass 1 streams the split's K rows, reduces q.k across the row's lanes with butterflies
//     and keeps the split's scores (log2 units) in LDS; pass 2 streams V rows and accumulates
//     p * v per lane, reduced across row groups and waves through LDS;
//   * each split writes (acc[E], max, sum) to the workspace; a merge kernel rescales and sums
//     the splits per head and writes out and lse.
#include <mutex>

#include "common.hpp"
#include "params.hpp"

namespace dc {
namespace {

// Scratch of the allocation-free entry point (dc_sdpa_decode_noalloc): the split partials live
// in this file-scope array instead of a caller's workspace.  Each GPU the library runs on holds
// its own copy, at its own address, until the process ends.  Host code never passes the array's
// name to a kernel (on the host it is only a stand-in): it passes the device address that
// hipGetSymbolAddress returns for the current device, looked up once per device.
static __device__ __align__(256) float scratch[kDecodeScratchBytes / sizeof(float)];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
float *g_scratch[kMaxDevices];

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kMaxSplitLen = 2048;
constexpr int kUnroll = 8;

template <typename T> struct Vec16;
template <> struct Vec16<float> {
    static constexpr int N = 4;
    typedef f32x4 type;
};
template <> struct Vec16<__bf16> {
    static constexpr int N = 8;
    typedef bf16x8 type;
};

// Part of a key or value row (read once: nontemporal loads, B32 H32 S4096 D128 6.1 -> 6.9 TB/s).
template <typename T, int N>
DEVI void load_row_part(float (&x)[N], const T *row, int d0, int E, bool vec) {
    if (vec) {
        const auto v = load_nt(reinterpret_cast<const typename Vec16<T>::type *>(row + d0));
#pragma unroll
        for (int i = 0; i < N; ++i) x[i] = to_f32<T>(v[i]);
    } else {
#pragma unroll
        for (int i = 0; i < N; ++i) x[i] = d0 + i < E ? to_f32<T>(row[d0 + i]) : 0.f;
    }
}

template <typename T, int D>
__global__ __launch_bounds__(kThreads) void decode_split_kernel(DecodeArgs a) {
    constexpr int VEC = Vec16<T>::N;
    constexpr int LPR = D / VEC;          // lanes per key row
    constexpr int RPW = 64 / LPR;         // rows per wave per step
    constexpr int RPS = RPW * kWaves;     // rows per workgroup per step
    __shared__ float sc[kMaxSplitLen];
    __shared__ float red[kWaves][RPW][D];
    __shared__ float wred[kWaves];

    const AttnShape &s = a.s;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int sub = lane / LPR, part = lane % LPR, d0 = part * VEC;
    const int split = blockIdx.x % a.splits, bh = blockIdx.x / a.splits;
    const int b = bh / s.H, h = bh % s.H, hk = h / s.repeat;
    const int k0 = split * a.split_len, k1 = min(s.S, k0 + a.split_len);
    const int n = max(0, k1 - k0);
    const T *kb = static_cast<const T *>(a.k) + ((int64_t)(b * s.Hkv + hk) * s.S) * s.E;
    const T *vb = static_cast<const T *>(a.v) + ((int64_t)(b * s.Hkv + hk) * s.S) * s.E;

    float qv[VEC];
    load_row_part<T, VEC>(qv, static_cast<const T *>(a.q) + (int64_t)bh * s.E, d0, s.E, s.vec);
#pragma unroll
    for (int i = 0; i < VEC; ++i) qv[i] *= s.scale_log2;

    // Pass 1: scores for rows k0 + step*RPS + wave*RPW + sub.
    const int my_row0 = wave * RPW + sub;
    for (int base = 0; base < n; base += RPS * kUnroll) {
        float kx[kUnroll][VEC];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const int r = base + u * RPS + my_row0;
            if (r < n)
                load_row_part<T, VEC>(kx[u], kb + (int64_t)(k0 + r) * s.E, d0, s.E, s.vec);
            else
#pragma unroll
                for (int i = 0; i < VEC; ++i) kx[u][i] = 0.f;
        }
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            float dot = 0.f;
#pragma unroll
            for (int i = 0; i < VEC; ++i) dot = fmaf(qv[i], kx[u][i], dot);
#pragma unroll
            for (int off = 1; off < LPR; off <<= 1) dot += __shfl_xor(dot, off, 64);
            const int r = base + u * RPS + my_row0;
            if (part == 0 && r < n) sc[r] = dot;
        }
    }
    __syncthreads();

    // Split max and sum of exp2(score - max).
    float mx = -INFINITY;
    for (int r = tid; r < n; r += kThreads) mx = fmaxf(mx, sc[r]);
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
    if (lane == 0) wred[wave] = mx;
    __syncthreads();
    mx = wred[0];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) mx = fmaxf(mx, wred[w]);
    const float m_use = mx == -INFINITY ? 0.f : mx;
    float sum = 0.f;
    for (int r = tid; r < n; r += kThreads) {
        const float p = exp2_fast(sc[r] - m_use);
        sc[r] = p;
        sum += p;
    }
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) sum += __shfl_xor(sum, off, 64);
    __syncthreads();  // everyone read wred (max) and wrote sc (p)
    if (lane == 0) wred[wave] = sum;
    __syncthreads();
    sum = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) sum += wred[w];

    // Pass 2: acc[d] = sum_r p[r] * V[r][d].
    float acc[VEC];
#pragma unroll
    for (int i = 0; i < VEC; ++i) acc[i] = 0.f;
    for (int base = 0; base < n; base += RPS * kUnroll) {
        float vx[kUnroll][VEC];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const int r = base + u * RPS + my_row0;
            if (r < n)
                load_row_part<T, VEC>(vx[u], vb + (int64_t)(k0 + r) * s.E, d0, s.E, s.vec);
            else
#pragma unroll
                for (int i = 0; i < VEC; ++i) vx[u][i] = 0.f;
        }
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const int r = base + u * RPS + my_row0;
            const float p = r < n ? sc[r] : 0.f;
#pragma unroll
            for (int i = 0; i < VEC; ++i) acc[i] = fmaf(p, vx[u][i], acc[i]);
        }
    }
#pragma unroll
    for (int i = 0; i < VEC; ++i) red[wave][sub][d0 + i] = acc[i];
    __syncthreads();
    float *out = a.part + ((int64_t)bh * a.splits + split) * (s.E + 2);
    for (int d = tid; d < s.E; d += kThreads) {
        float t = 0.f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w)
#pragma unroll
            for (int r = 0; r < RPW; ++r) t += red[w][r][d];
        out[d] = t;
    }
    if (tid == 0) {
        out[s.E] = mx;
        out[s.E + 1] = sum;
    }
}

// One wave per (batch, head): rescale the splits to the global max and sum them.
template <typename T>
__global__ __launch_bounds__(64) void decode_merge_kernel(DecodeArgs a) {
    const AttnShape &s = a.s;
    const int bh = blockIdx.x, lane = threadIdx.x;
    const float *p = a.part + (int64_t)bh * a.splits * (s.E + 2);
    float m = -INFINITY;
    for (int i = 0; i < a.splits; ++i) m = fmaxf(m, p[i * (s.E + 2) + s.E]);
    const float m_use = m == -INFINITY ? 0.f : m;
    float l = 0.f;
    for (int i = 0; i < a.splits; ++i)
        l += p[i * (s.E + 2) + s.E + 1] * exp2_fast(p[i * (s.E + 2) + s.E] - m_use);
    const bool empty = l == 0.f;
    const float inv = empty ? 0.f : 1.f / l;
    T *o = static_cast<T *>(a.out) + (int64_t)bh * s.E;
    for (int d = lane; d < s.E; d += 64) {
        float t = 0.f;
        for (int i = 0; i < a.splits; ++i)
            t += p[i * (s.E + 2) + d] * exp2_fast(p[i * (s.E + 2) + s.E] - m_use);
        o[d] = from_f32<T>(t * inv);
    }
    if (lane == 0) a.lse[bh] = empty ? 0.f : (m_use + log2_fast(l)) * kLn2;
}

template <typename T, int D>
hipError_t launch_t(const DecodeArgs &args, hipStream_t st) {
    DecodeArgs a = args;
    a.s.vec = args.s.vec && args.s.E == D;
    const int BH = a.s.B * a.s.H;
    return_if(launch(decode_split_kernel<T, D>, dim3((int64_t)a.splits * BH), dim3(kThreads), st, a));
    return_if(launch(decode_merge_kernel<T>, dim3(BH), dim3(64), st, a));
    return hipSuccess;
}

template <typename T>
hipError_t launch_dtype(const DecodeArgs &a, hipStream_t st) {
    if (a.s.E <= 32) return launch_t<T, 32>(a, st);
    if (a.s.E <= 64) return launch_t<T, 64>(a, st);
    if (a.s.E <= 128) return launch_t<T, 128>(a, st);
    return launch_t<T, 256>(a, st);
}

}  // namespace

// Enough splits for ~4K workgroups (16 per CU on 256 CUs), at most kMaxSplitLen keys each.
// Measured on C4 (B32 H32 S4096 D128 fp32, per call): 2K workgroups 6087 GB/s, 4K 6117-6121,
// 6K 6085, 8K 6051-6063, 16K 5820.
int decode_splits(const AttnShape &s, int *split_len) {
    const int64_t BH = (int64_t)s.B * s.H;
    int64_t splits = BH > 0 ? (4096 + BH - 1) / BH : 1;
    const int64_t max_splits = (s.S + 63) / 64;
    if (splits > max_splits) splits = max_splits;
    if (splits < 1) splits = 1;
    int64_t len = (s.S + splits - 1) / splits;
    if (len > kMaxSplitLen) {
        len = kMaxSplitLen;
        splits = (s.S + len - 1) / len;
    }
    *split_len = (int)(len < 1 ? 1 : len);
    return (int)splits;
}

hipError_t launch_decode(const DecodeArgs &a, bool bf16, hipStream_t st) {
    return bf16 ? launch_dtype<__bf16>(a, st) : launch_dtype<float>(a, st);
}

hipError_t decode_scratch(float **ptr) {
    int dev = -1;
    return_if(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (g_scratch[dev] == nullptr) {
        void *p = nullptr;
        return_if(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        g_scratch[dev] = static_cast<float *>(p);
    }
    *ptr = g_scratch[dev];
    return hipSuccess;
}

}  // namespace dc
