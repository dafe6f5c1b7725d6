// Helpers shared by the float32 and bfloat16 backward launchers.
#pragma once

#include "common.hpp"
#include "params.hpp"

namespace dc {

// dsum[row] = sum_d dO[row][d] * O[row][d]; also clears the float32 dQ accumulator row.
template <typename T>
__global__ __launch_bounds__(256) void bwd_pre_kernel(BwdArgs a) {
    const AttnShape &s = a.s;
    const int64_t rows = (int64_t)s.B * s.H * s.L;
    const int64_t row = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);
    const int part = threadIdx.x & 15;
    if (row >= rows) return;  // whole 16-lane groups exit together
    const T *go = static_cast<const T *>(a.dout) + row * s.E;
    const T *o = static_cast<const T *>(a.out) + row * s.E;
    float acc = 0.f;
    for (int d = part; d < s.E; d += 16) acc = fmaf(to_f32<T>(go[d]), to_f32<T>(o[d]), acc);
#pragma unroll
    for (int off = 1; off < 16; off <<= 1) acc += __shfl_xor(acc, off, 64);
    if (part == 0) a.dsum[row] = acc;
    float *dq = a.dq_acc + row * s.E;
    for (int d = part; d < s.E; d += 16) dq[d] = 0.f;
}

// dq[i] = T(dq_acc[i]): the bfloat16 path accumulates dQ in a float32 workspace.
template <typename T>
__global__ __launch_bounds__(256) void bwd_dq_convert_kernel(BwdArgs a, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) static_cast<T *>(a.dq)[i] = from_f32<T>(a.dq_acc[i]);
}

}  // namespace dc
