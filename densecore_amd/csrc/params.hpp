// Kernel parameter blocks and launcher declarations shared by the C ABI (abi.hip) and the
// kernel translation units.  Sizes are validated by the ABI before any launch.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dc {

struct AttnShape {
    int B, H, Hkv, L, S, E;
    int repeat;        // H / Hkv
    float scale;       // natural-log units, as the reference computes it
    float scale_log2;  // scale * log2(e)
    bool causal;
    const float *mask; // additive, or nullptr
    int64_t msb, msh, msl;
    bool vec;          // E equals the kernel's padded head dim and pointers are 16-byte aligned
};

struct FwdArgs {
    AttnShape s;
    const void *q, *k, *v;
    void *out;
    float *lse;
};

struct BwdArgs {
    AttnShape s;
    const void *dout, *q, *k, *v, *out;
    const float *lse;
    void *dq, *dk, *dv;
    float *dsum;    // (B, H, L) workspace: rowsum(dout * out)
    float *dq_acc;  // (B, H, L, E) float32 accumulator (== dq for float32)
};

struct DecodeArgs {
    AttnShape s;
    const void *q, *k, *v;
    void *out;
    float *lse;
    float *part;    // (B*H, splits, E + 2) workspace: acc[E], max, sum
    int splits, split_len;
};

// Row softmax (softmax.hip).
struct SoftmaxArgs {
    const float *a;    // forward: scores; backward: grad_y
    const float *b;    // backward: y
    float *out;        // forward: y; backward: grad_x
    const float *mask;
    int64_t rows;
    int width, heads, q_len;
    int64_t msb, msh, msl;
    bool safe;
};

// Each launcher returns hipSuccess or the launch error; it never synchronizes.
hipError_t launch_fwd_f32(const FwdArgs &a, hipStream_t st);
hipError_t launch_fwd_bf16(const FwdArgs &a, hipStream_t st);
hipError_t launch_bwd_f32(const BwdArgs &a, hipStream_t st);
hipError_t launch_bwd_bf16(const BwdArgs &a, hipStream_t st);
hipError_t launch_decode(const DecodeArgs &a, bool bf16, hipStream_t st);
int decode_splits(const AttnShape &s, int *split_len);
// `vec`: rows (and mask rows) start 16-byte aligned and the width is a multiple of 4.
hipError_t launch_softmax_fwd(const SoftmaxArgs &a, bool vec, hipStream_t st);
hipError_t launch_softmax_bwd(const SoftmaxArgs &a, bool vec, hipStream_t st);

// Largest head dim each kernel family instantiates.
constexpr int kMaxHeadDim = 256;

}  // namespace dc
