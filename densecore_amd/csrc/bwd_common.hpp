// Helpers shared by the float32 and bfloat16 backward launchers.
#pragma once

#include "common.hpp"
#include "params.hpp"

namespace dc {

// dsum[row] = sum_d dO[row][d] * O[row][d]; with CLEAR also zeroes the float32 dQ accumulator
// row (the float32 backward accumulates dQ into its output with atomics).
// One 256-thread block handles rows 16 * block .. 16 * block + 15.
template <typename T, bool CLEAR>
DEVI void bwd_pre_block(const BwdArgs &a, int64_t block) {
    const AttnShape &s = a.s;
    const int64_t rows = (int64_t)s.B * s.H * s.L;
    const int64_t row = block * 16 + (threadIdx.x >> 4);
    const int part = threadIdx.x & 15;
    if (row >= rows) return;  // whole 16-lane groups exit together
    const T *go = static_cast<const T *>(a.dout) + row * s.E;
    const T *o = static_cast<const T *>(a.out) + row * s.E;
    float acc = 0.f;
    // 16-byte chunks per lane when rows are whole chunks on 16-byte boundaries.
    constexpr int VW = 16 / sizeof(T);
    typedef T tvec __attribute__((ext_vector_type(VW)));
    if (s.E % VW == 0 && ((reinterpret_cast<uintptr_t>(a.dout) | reinterpret_cast<uintptr_t>(a.out)) & 15) == 0) {
        for (int c = part; c < s.E / VW; c += 16) {
            const tvec x = *reinterpret_cast<const tvec *>(go + c * VW);
            const tvec y = *reinterpret_cast<const tvec *>(o + c * VW);
#pragma unroll
            for (int e = 0; e < VW; ++e) acc = fmaf(to_f32<T>(x[e]), to_f32<T>(y[e]), acc);
        }
    } else {
        for (int d = part; d < s.E; d += 16) acc = fmaf(to_f32<T>(go[d]), to_f32<T>(o[d]), acc);
    }
#pragma unroll
    for (int off = 1; off < 16; off <<= 1) acc += __shfl_xor(acc, off, 64);
    if (part == 0) a.dsum[row] = acc;
    if (CLEAR) {
        float *dq = a.dq_acc + row * s.E;
        for (int d = part; d < s.E; d += 16) dq[d] = 0.f;
    }
}

template <typename T, bool CLEAR>
__global__ __launch_bounds__(256) void bwd_pre_kernel(BwdArgs a) {
    bwd_pre_block<T, CLEAR>(a, blockIdx.x);
}

}  // namespace dc
