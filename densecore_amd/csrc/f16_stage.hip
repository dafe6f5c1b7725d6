// bfloat16 -> float16 copies of the attention operands, scaled by a power of two per
// (batch, head) slab, for the bf16 kernels' fp16 products.
//
// The bf16 kernels round P (and, in the backward, dS) once to a 16-bit float before their
// products.  Rounded to bf16 (8 bits) that breaks the elementwise bf16 bar by 1.5-4.5x at
// L = 512-2048; rounded to fp16 (11 bits) it stays at 0.35-0.46 of it.  fp16 MFMA needs both
// operands in fp16, so V (forward) and Q, K, V, dO (backward) are copied to fp16 first.  A bf16
// value needs 8 significant bits, which fp16 holds exactly between 2^-14 and 65504; each slab
// is therefore scaled by 2^e, e chosen so that its largest finite magnitude m lands in
// [2^14, 2^15): no value can overflow, and every value down to m * 2^-28 converts exactly (the
// rest, at most m * 2^-39 in absolute error each, are below anything the bar can see).  Infinite
// and NaN values convert to themselves and do not set the scale.  The kernels fold 2^-e back
// into the scalars they already multiply by.
//
// Two passes: slab_max_kernel reduces each of `parts` segments (of `per` elements) of a slab to
// its largest finite magnitude; slab_convert_kernel reads a slab's partial maxima, derives e
// (written once per slab) and converts its segment.
#include <cmath>

#include "common.hpp"
#include "params.hpp"

namespace dc {
namespace {

typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));

constexpr int kThreads = 256;

DEVI float finite_abs(uint16_t bits) {
    const float x = __uint_as_float((uint32_t)bits << 16);
    return (bits & 0x7f80u) == 0x7f80u ? 0.f : fabsf(x);  // inf / NaN: no say in the scale
}

DEVI void segment(int64_t slab, int64_t per, int p, int64_t *begin, int64_t *end) {
    *begin = per * p < slab ? per * p : slab;
    *end = *begin + per < slab ? *begin + per : slab;
}

__global__ __launch_bounds__(kThreads) void slab_max_kernel(const uint16_t *src, int64_t slab, int parts,
                                                            int64_t per, bool vec, float *partial) {
    const int s = blockIdx.x / parts, p = blockIdx.x % parts;
    int64_t i0, i1;
    segment(slab, per, p, &i0, &i1);
    const uint16_t *x = src + (int64_t)s * slab;
    float m = 0.f;
    if (vec) {  // segments start at multiples of 8 elements (slab % 8 == 0, per % 8 == 0)
#pragma unroll 4
        for (int64_t i = i0 + 8 * threadIdx.x; i < i1; i += 8 * kThreads) {
            const u16x8 v = *reinterpret_cast<const u16x8 *>(x + i);
#pragma unroll
            for (int e = 0; e < 8; ++e) m = fmaxf(m, finite_abs(v[e]));
        }
    } else {
        for (int64_t i = i0 + threadIdx.x; i < i1; i += kThreads) m = fmaxf(m, finite_abs(x[i]));
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    __shared__ float wm[kThreads / 64];
    if ((threadIdx.x & 63) == 0) wm[threadIdx.x >> 6] = m;
    __syncthreads();
    if (threadIdx.x == 0) {
        float r = wm[0];
#pragma unroll
        for (int w = 1; w < kThreads / 64; ++w) r = fmaxf(r, wm[w]);
        partial[blockIdx.x] = r;
    }
}

// 2^e with m * 2^e in [2^14, 2^15) for m > 0 (m = f 2^k, f in [0.5, 1): e = 15 - k); 0 for m = 0.
DEVI int slab_exp(float m) {
    if (!(m > 0.f)) return 0;
    int k;
    frexpf(m, &k);
    return 15 - k;
}

__global__ __launch_bounds__(kThreads) void slab_convert_kernel(const uint16_t *src, _Float16 *dst, int64_t slab,
                                                                int parts, int64_t per, bool vec,
                                                                const float *partial, int *exps) {
    const int s = blockIdx.x / parts, p = blockIdx.x % parts;
    // The slab's largest finite magnitude: its `parts` partial maxima, reduced by the block.
    float m = 0.f;
    for (int j = threadIdx.x; j < parts; j += kThreads) m = fmaxf(m, partial[(int64_t)s * parts + j]);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    __shared__ float wm[kThreads / 64];
    if ((threadIdx.x & 63) == 0) wm[threadIdx.x >> 6] = m;
    __syncthreads();
#pragma unroll
    for (int w = 0; w < kThreads / 64; ++w) m = fmaxf(m, wm[w]);
    const int e = slab_exp(m);
    if (p == 0 && threadIdx.x == 0) exps[s] = e;
    int64_t i0, i1;
    segment(slab, per, p, &i0, &i1);
    const uint16_t *x = src + (int64_t)s * slab;
    _Float16 *y = dst + (int64_t)s * slab;
    auto cvt = [&](uint16_t bits) {
        return static_cast<_Float16>(ldexpf(__uint_as_float((uint32_t)bits << 16), e));
    };
    if (vec) {
#pragma unroll 4
        for (int64_t i = i0 + 8 * threadIdx.x; i < i1; i += 8 * kThreads) {
            const u16x8 v = *reinterpret_cast<const u16x8 *>(x + i);
            f16x8 o;
#pragma unroll
            for (int c = 0; c < 8; ++c) o[c] = cvt(v[c]);
            *reinterpret_cast<f16x8 *>(y + i) = o;
        }
    } else {
        for (int64_t i = i0 + threadIdx.x; i < i1; i += kThreads) y[i] = cvt(x[i]);
    }
}

}  // namespace

// Segment length for `nslabs` slabs of `slab` elements: a multiple of 2048 (8 elements per
// thread, so 16-byte accesses stay aligned), at most 64K elements, and short enough that the
// grid has about 1024 workgroups when the slabs are few (4 slabs of 512K elements: 32
// workgroups of 64K took 10-12 us per pass; the copies are HBM-bound only with a full grid).
int64_t f16_segment(int64_t nslabs, int64_t slab) {
    const int64_t want = nslabs > 0 ? (1024 + nslabs - 1) / nslabs : 1;  // segments per slab
    int64_t per = (slab + want - 1) / want;
    per = (per + 2047) / 2048 * 2048;
    if (per > 65536) per = 65536;
    if ((slab + per - 1) / per > 1024) per = ((slab + 1023) / 1024 + 7) / 8 * 8;  // at most 1024 segments
    return per > 0 ? per : 1;
}

int f16_parts(int64_t nslabs, int64_t slab) {
    const int64_t per = f16_segment(nslabs, slab);
    const int64_t parts = (slab + per - 1) / per;
    return (int)(parts < 1 ? 1 : parts);
}

hipError_t launch_to_f16(const void *src, void *dst, int64_t nslabs, int64_t slab, float *partial, int *exps,
                         hipStream_t st) {
    if (nslabs == 0 || slab == 0) return hipSuccess;
    const int64_t per = f16_segment(nslabs, slab);
    const int parts = f16_parts(nslabs, slab);
    const bool vec = slab % 8 == 0 && per % 8 == 0 && ((uintptr_t)src & 15) == 0 && ((uintptr_t)dst & 15) == 0;
    const dim3 grid((unsigned)(nslabs * parts)), block(kThreads);
    return_if(launch(slab_max_kernel, grid, block, st, static_cast<const uint16_t *>(src), slab, parts, per, vec,
                     partial));
    return launch(slab_convert_kernel, grid, block, st, static_cast<const uint16_t *>(src),
                  static_cast<_Float16 *>(dst), slab, parts, per, vec, static_cast<const float *>(partial), exps);
}

}  // namespace dc
