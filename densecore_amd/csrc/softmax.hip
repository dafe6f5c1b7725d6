// Row softmax over the last axis for the composed attention path (include/dc_math.h).
//
// Forward (src/torch_softmax.rs:57-67): m = max(row), e = exp(row - m), y = e * (1 / sum(e)),
// here fused with the additive mask the math path adds first (python/densecore/functional.py:
// 330-333) and its safe softmax (:334-337: a row that is all -inf gives 0).  Backward
// (src/torch_softmax.rs:90-97): grad_x = (grad_y - sum(grad_y * y)) * y.
//
// HBM-bound (one read and one write per element forward, two reads and one write backward):
// one wave per row, four rows per workgroup.  Rows of up to 4096 elements stay in registers
// (NV float4 per lane, 16-byte loads when rows, mask rows and pointers allow it, else 4-byte
// loads of a lane-strided layout); longer rows are streamed twice (an online max/sum pass, then
// the write pass).  exp is the accurate expf (the reference uses SLEEF's 1-ulp expf); sums are
// wave trees, so the low bits differ from the reference's 4-lane order.
#include "common.hpp"
#include "params.hpp"

namespace dc {

namespace {

constexpr float kNegInf = -__builtin_inff();

// NaN if either operand is NaN (the reference's NEON FMAX, src/torch_softmax.rs:43-54).
DEVI float nan_max(float x, float y) { return (x != x || y != y) ? x + y : fmaxf(x, y); }

DEVI float wave_max(float x) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) x = nan_max(x, __shfl_xor(x, o));
    return x;
}
DEVI float wave_sum(float x) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o);
    return x;
}

DEVI const float *mask_row(const SoftmaxArgs &a, int64_t row) {
    const int64_t l = row % a.q_len, bh = row / a.q_len;
    return a.mask + (bh / a.heads) * a.msb + (bh % a.heads) * a.msh + l * a.msl;
}

// Element k of this lane's register row: column 4*lane + 256*(k/4) + k%4 (VEC) or
// lane + 64*k (scalar layout).
template <bool VEC> DEVI int col_of(int lane, int k) {
    return VEC ? 4 * lane + 256 * (k >> 2) + (k & 3) : lane + 64 * k;
}

template <int NV, bool VEC, bool MASK>
DEVI void load_row(const float *src, const float *msk, int W, int lane, float (&v)[NV * 4],
                   float pad) {
    if (VEC) {
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int j = 4 * lane + 256 * i;
            f32x4 t = {pad, pad, pad, pad};
            if (j < W) {
                t = load_nt(reinterpret_cast<const f32x4 *>(src + j));  // read once
                if (MASK) t += *reinterpret_cast<const f32x4 *>(msk + j);  // shared by rows
            }
#pragma unroll
            for (int c = 0; c < 4; ++c) v[4 * i + c] = t[c];
        }
    } else {
#pragma unroll
        for (int k = 0; k < NV * 4; ++k) {
            const int j = lane + 64 * k;
            v[k] = pad;
            if (j < W) v[k] = MASK ? src[j] + msk[j] : src[j];
        }
    }
}

template <int NV, bool VEC>
DEVI void store_row(float *dst, int W, int lane, const float (&v)[NV * 4]) {
    if (VEC) {
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int j = 4 * lane + 256 * i;
            if (j < W)
                __builtin_nontemporal_store(f32x4{v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]},
                                            reinterpret_cast<f32x4 *>(dst + j));
        }
    } else {
#pragma unroll
        for (int k = 0; k < NV * 4; ++k) {
            const int j = lane + 64 * k;
            if (j < W) dst[j] = v[k];
        }
    }
}

template <int NV, bool VEC, bool MASK>
__global__ __launch_bounds__(256) void softmax_fwd_kernel(SoftmaxArgs a) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= a.rows) return;
    const int W = a.width;
    const float *msk = MASK ? mask_row(a, row) : nullptr;
    float v[NV * 4];
    load_row<NV, VEC, MASK>(a.a + row * W, msk, W, lane, v, kNegInf);
    float m = v[0];
#pragma unroll
    for (int k = 1; k < NV * 4; ++k) m = nan_max(m, v[k]);
    m = wave_max(m);
    if (a.safe && m == kNegInf) {
#pragma unroll
        for (int k = 0; k < NV * 4; ++k) v[k] = 0.f;
        store_row<NV, VEC>(a.out + row * W, W, lane, v);
        return;
    }
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < NV * 4; ++k) {
        // Padding columns hold -inf: exp gives 0 (or NaN when m is -inf, a row the reference
        // also turns into NaN).
        v[k] = expf(v[k] - m);
        if (col_of<VEC>(lane, k) < W) s += v[k];
    }
    const float inv = 1.0f / wave_sum(s);
#pragma unroll
    for (int k = 0; k < NV * 4; ++k) v[k] *= inv;
    store_row<NV, VEC>(a.out + row * W, W, lane, v);
}

// Rows longer than the register path: an online (max, sum) pass, then the write pass.
template <bool MASK>
__global__ __launch_bounds__(256) void softmax_fwd_stream_kernel(SoftmaxArgs a) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= a.rows) return;
    const int W = a.width;
    const float *x = a.a + row * W;
    const float *msk = MASK ? mask_row(a, row) : nullptr;
    float m = kNegInf, s = 0.f;
    for (int j = lane; j < W; j += 64) {
        const float t = MASK ? x[j] + msk[j] : x[j];
        const float mn = nan_max(m, t);
        if (mn != kNegInf) s = s * expf(m - mn) + expf(t - mn);
        m = mn;
    }
    const float M = wave_max(m);
    float *y = a.out + row * W;
    if (a.safe && M == kNegInf) {
        for (int j = lane; j < W; j += 64) y[j] = 0.f;
        return;
    }
    const float S = wave_sum(m == kNegInf ? 0.f : s * expf(m - M));
    const float inv = M == kNegInf ? __builtin_nanf("") : 1.0f / S;
    for (int j = lane; j < W; j += 64) {
        const float t = MASK ? x[j] + msk[j] : x[j];
        y[j] = expf(t - M) * inv;
    }
}

template <int NV, bool VEC>
__global__ __launch_bounds__(256) void softmax_bwd_kernel(SoftmaxArgs a) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= a.rows) return;
    const int W = a.width;
    float g[NV * 4], y[NV * 4];
    load_row<NV, VEC, false>(a.a + row * W, nullptr, W, lane, g, 0.f);
    load_row<NV, VEC, false>(a.b + row * W, nullptr, W, lane, y, 0.f);
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < NV * 4; ++k) s += g[k] * y[k];
    s = wave_sum(s);
#pragma unroll
    for (int k = 0; k < NV * 4; ++k) g[k] = (g[k] - s) * y[k];
    store_row<NV, VEC>(a.out + row * W, W, lane, g);
}

__global__ __launch_bounds__(256) void softmax_bwd_stream_kernel(SoftmaxArgs a) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= a.rows) return;
    const int W = a.width;
    const float *g = a.a + row * W, *y = a.b + row * W;
    float s = 0.f;
    for (int j = lane; j < W; j += 64) s += g[j] * y[j];
    s = wave_sum(s);
    float *dx = a.out + row * W;
    for (int j = lane; j < W; j += 64) dx[j] = (g[j] - s) * y[j];
}

// Smallest register layout that holds a row of W (0: stream).
int nv_for(int W) {
    for (int nv = 1; nv <= 16; nv *= 2)
        if (W <= 256 * nv) return nv;
    return 0;
}

template <bool VEC, bool MASK>
hipError_t fwd_dispatch(const SoftmaxArgs &a, dim3 grid, hipStream_t st) {
    switch (nv_for(a.width)) {
    case 1: return launch(softmax_fwd_kernel<1, VEC, MASK>, grid, dim3(256), st, a);
    case 2: return launch(softmax_fwd_kernel<2, VEC, MASK>, grid, dim3(256), st, a);
    case 4: return launch(softmax_fwd_kernel<4, VEC, MASK>, grid, dim3(256), st, a);
    case 8: return launch(softmax_fwd_kernel<8, VEC, MASK>, grid, dim3(256), st, a);
    case 16: return launch(softmax_fwd_kernel<16, VEC, MASK>, grid, dim3(256), st, a);
    default: return launch(softmax_fwd_stream_kernel<MASK>, grid, dim3(256), st, a);
    }
}

template <bool VEC>
hipError_t bwd_dispatch(const SoftmaxArgs &a, dim3 grid, hipStream_t st) {
    switch (nv_for(a.width)) {
    case 1: return launch(softmax_bwd_kernel<1, VEC>, grid, dim3(256), st, a);
    case 2: return launch(softmax_bwd_kernel<2, VEC>, grid, dim3(256), st, a);
    case 4: return launch(softmax_bwd_kernel<4, VEC>, grid, dim3(256), st, a);
    case 8: return launch(softmax_bwd_kernel<8, VEC>, grid, dim3(256), st, a);
    case 16: return launch(softmax_bwd_kernel<16, VEC>, grid, dim3(256), st, a);
    default: return launch(softmax_bwd_stream_kernel, grid, dim3(256), st, a);
    }
}

}  // namespace

// `vec`: every row (and mask row) starts 16-byte aligned and the width is a multiple of 4.
hipError_t launch_softmax_fwd(const SoftmaxArgs &a, bool vec, hipStream_t st) {
    const dim3 grid((unsigned)((a.rows + 3) / 4));
    if (a.mask) return vec ? fwd_dispatch<true, true>(a, grid, st) : fwd_dispatch<false, true>(a, grid, st);
    return vec ? fwd_dispatch<true, false>(a, grid, st) : fwd_dispatch<false, false>(a, grid, st);
}

hipError_t launch_softmax_bwd(const SoftmaxArgs &a, bool vec, hipStream_t st) {
    const dim3 grid((unsigned)((a.rows + 3) / 4));
    return vec ? bwd_dispatch<true>(a, grid, st) : bwd_dispatch<false>(a, grid, st);
}

}  // namespace dc
