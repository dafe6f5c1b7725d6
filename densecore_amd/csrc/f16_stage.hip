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
// (written once per slab) and converts its segment.  Each pass is one launch for all the
// tensors a call copies (the backward's four): its blocks are dealt to the tensors in order.
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

// The tensors of one launch: copy j has nslabs slabs of slab[j] elements, cut into parts[j]
// segments of per[j]; its blocks are [first[j], first[j + 1]).
struct SlabJobs {
    const uint16_t *src[kMaxF16Copies];
    _Float16 *dst[kMaxF16Copies];
    float *partial[kMaxF16Copies];
    int *exps[kMaxF16Copies];
    int64_t slab[kMaxF16Copies], per[kMaxF16Copies];
    int parts[kMaxF16Copies];
    bool vec[kMaxF16Copies];
    int first[kMaxF16Copies + 1];
    int n;
};

// The copy j of launch-wide block `idx` and its block index within that copy (wave-uniform).
DEVI int job_of(const SlabJobs &J, int idx, int *local) {
    int j = 0;
    while (j + 1 < J.n && idx >= J.first[j + 1]) ++j;
    *local = idx - J.first[j];
    return j;
}

__global__ __launch_bounds__(kThreads) void slab_max_kernel(SlabJobs J) {
    int b;
    const int j = job_of(J, (int)blockIdx.x, &b);
    const int64_t slab = J.slab[j], per = J.per[j];
    const int parts = J.parts[j];
    const bool vec = J.vec[j];
    const int s = b / parts, p = b % parts;
    int64_t i0, i1;
    segment(slab, per, p, &i0, &i1);
    const uint16_t *x = J.src[j] + (int64_t)s * slab;
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
        J.partial[j][b] = r;
    }
}

// 2^e with m * 2^e in [2^14, 2^15) for m > 0 (m = f 2^k, f in [0.5, 1): e = 15 - k); 0 for m = 0.
DEVI int slab_exp(float m) {
    if (!(m > 0.f)) return 0;
    int k;
    frexpf(m, &k);
    return 15 - k;
}

// Blocks run in reverse order of the max pass's: the data that pass read last is the most likely
// to be still in the caches (four tensors exceed the 256 MB last-level cache).
__global__ __launch_bounds__(kThreads) void slab_convert_kernel(SlabJobs J) {
    int b;
    const int j = job_of(J, (int)(gridDim.x - 1 - blockIdx.x), &b);
    const int64_t slab = J.slab[j], per = J.per[j];
    const int parts = J.parts[j];
    const bool vec = J.vec[j];
    const float *partial = J.partial[j];
    const int s = b / parts, p = b % parts;
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
    if (p == 0 && threadIdx.x == 0) J.exps[j][s] = e;
    int64_t i0, i1;
    segment(slab, per, p, &i0, &i1);
    const uint16_t *x = J.src[j] + (int64_t)s * slab;
    _Float16 *y = J.dst[j] + (int64_t)s * slab;
    auto cvt = [&](uint16_t bits) {
        return static_cast<_Float16>(ldexpf(__uint_as_float((uint32_t)bits << 16), e));
    };
    if (vec) {
#pragma unroll 4
        for (int64_t i = i0 + 8 * threadIdx.x; i < i1; i += 8 * kThreads) {
            const u16x8 v = load_nt(reinterpret_cast<const u16x8 *>(x + i));  // its last read
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

size_t f16_partial_floats(int64_t nslabs, const F16Copy *copies, int n) {
    size_t total = 0;
    for (int j = 0; j < n; ++j) total += (size_t)nslabs * f16_parts(nslabs, copies[j].slab);
    return total;
}

hipError_t launch_to_f16(const F16Copy *copies, int n, int64_t nslabs, float *partial, hipStream_t st) {
    SlabJobs J{};
    J.first[0] = 0;
    float *at = partial;
    for (int j = 0; j < n; ++j) {
        const F16Copy &c = copies[j];
        const int64_t slab = nslabs > 0 ? c.slab : 0;
        const int parts = slab > 0 ? f16_parts(nslabs, slab) : 0;
        J.src[J.n] = static_cast<const uint16_t *>(c.src);
        J.dst[J.n] = static_cast<_Float16 *>(c.dst);
        J.exps[J.n] = c.exps;
        J.slab[J.n] = slab;
        J.per[J.n] = slab > 0 ? f16_segment(nslabs, slab) : 1;
        J.parts[J.n] = parts;
        J.vec[J.n] = slab % 8 == 0 && J.per[J.n] % 8 == 0 && ((uintptr_t)c.src & 15) == 0 &&
                     ((uintptr_t)c.dst & 15) == 0;
        J.partial[J.n] = at;
        if (slab == 0) continue;  // nothing to copy: the copy takes no blocks
        at += nslabs * parts;
        J.first[J.n + 1] = J.first[J.n] + (int)(nslabs * parts);
        ++J.n;
    }
    if (J.n == 0) return hipSuccess;
    const dim3 grid((unsigned)J.first[J.n]), block(kThreads);
    return_if(launch(slab_max_kernel, grid, block, st, J));
    return launch(slab_convert_kernel, grid, block, st, J);
}

}  // namespace dc
