/*
 * dc_math.h — C ABI of the device-side pieces of DenseCore's composed ("math") attention path,
 * in the same library as dc_attn.h (libdcattn.so).
 *
 * The reference's math path (python/densecore/functional.py:318-340, used for dropout, masks
 * the flash path rejects, Ev != E and masks that require a gradient) and its
 * multi_head_attention_forward (functional.py:400-461) are composed from bmm, an additive
 * mask, softmax over the last axis and dropout.  This header covers each of them:
 *
 *   dc_bmm           replaces  the (Cpu, Float32) entry of the bmm registry
 *                              src/batched_matmul.rs:28-49 -> torch_blas::bmm src/torch_blas.rs:404-449
 *                    (a device entry of that table: strided (batch, m, k) x (batch, k, n))
 *   dc_softmax_fwd   replaces  Tensor.softmax(-1) on the scores   src/lib.rs:269-270
 *                              -> activation_dispatch::softmax     src/activation_dispatch.rs:61
 *                              -> torch_softmax::softmax_lastdim   src/torch_softmax.rs:57-67
 *                    fused with the additive mask (functional.py:330-333) and the math path's
 *                    safe softmax (functional.py:334-337: rows that are all -inf give 0)
 *   dc_softmax_bwd   replaces  torch_softmax::softmax_backward_lastdim src/torch_softmax.rs:90-97
 *   dc_bernoulli     replaces  Generator::bernoulli(n, p)       src/torch_random.rs:241-254
 *                    as the math path's dropout draws it (functional.py:244, 638-641 via
 *                    _random.py:86-87, random_api.rs:127-134): the same mt19937 stream
 *                    (src/torch_random.rs:29-98), drawn on the GPU, as packed keep bits
 *   dc_dropout_apply replaces  input * Tensor(noise)            python/densecore/functional.py:244
 *   dc_mt19937_seed, dc_mt19937_advance: host-side Generator::manual_seed
 *                    (src/torch_random.rs:43-56) and a skip-ahead of the same engine
 *
 * Conventions: scores x, probabilities y and their gradients are contiguous float32 rows of
 * `width` elements, `rows` rows.  Row r is (b, h, l) with l = r % q_len, h = (r / q_len) % heads,
 * b = r / (q_len * heads); the optional additive float32 mask element of (row r, column s) is
 * mask[b*mask_stride_b + h*mask_stride_h + l*mask_stride_l + s] (a stride of 0 broadcasts).
 * Device pointers; calls are asynchronous on `stream` (a hipStream_t).
 */
#ifndef DC_MATH_H
#define DC_MATH_H

#include <stddef.h>
#include <stdint.h>

#include "dc_attn.h"

#ifdef __cplusplus
extern "C" {
#endif

/* C[b] = A[b] B[b] in float32.  A is (batch, m, k), B is (batch, k, n), each read through its
 * element strides (a transposed view is other strides; any layout is accepted, the fastest have
 * a stride of 1 along m, n or k with 16-byte aligned rows); C is contiguous (batch, m, n).  k == 0
 * gives zeros (src/batched_matmul.rs:63-65).  Sizes above 2^31 - 1 are DC_UNSUPPORTED. */
typedef struct {
    int64_t batch, m, n, k;
    int64_t a_stride_batch, a_stride_m, a_stride_k;
    int64_t b_stride_batch, b_stride_k, b_stride_n;
} dc_bmm_desc;

dc_status dc_bmm(const dc_bmm_desc *d, const float *a, const float *b, float *c, void *stream);

typedef struct {
    int64_t rows, width;
    int64_t heads, q_len;                                 /* row decomposition for the mask */
    int64_t mask_stride_b, mask_stride_h, mask_stride_l;  /* elements; used when mask != NULL */
    int32_t safe;     /* 1: a row whose masked scores are all -inf gives y = 0 (and zero grads) */
    int32_t reserved;
} dc_softmax_desc;

/* y = softmax(x + mask) over each row.  src/torch_softmax.rs:57-67 (max, exp(x - max), sum,
 * multiply by 1 / sum), python/densecore/functional.py:330-337 (mask, safe rows). */
dc_status dc_softmax_fwd(const dc_softmax_desc *d, const float *x, const float *mask, float *y,
                         void *stream);

/* grad_x = (grad_y - sum(grad_y * y)) * y over each row.  src/torch_softmax.rs:90-97. */
dc_status dc_softmax_bwd(const dc_softmax_desc *d, const float *grad_y, const float *y,
                         float *grad_x, void *stream);

/* ---- the reference's CPU generator (PyTorch's mt19937), drawn on the GPU ----
 *
 * Engine state as the reference keeps it (src/torch_random.rs:19-26): 624 words plus the
 * position pair (left, next); the next output is state[next] when left > 1, and the first word
 * of the next block (after a twist) when left == 1.  Valid pairs: left == 1 (any next), or
 * 2 <= left <= 624 with left + next == 625. */
#define DC_MT19937_WORDS 624

/* Generator::manual_seed (src/torch_random.rs:43-56): words = the seeded engine; the position
 * of a freshly seeded engine is left = 1, next = 0.  Host memory. */
void dc_mt19937_seed(uint64_t seed, uint32_t *words);

/* Skip `count` outputs: the engine state after `count` calls of random() (host memory; the
 * jump-ahead polynomials are computed on first use, about a second). */
dc_status dc_mt19937_advance(uint32_t *words, int64_t *left, int64_t *next, uint64_t count);

/* Device buffer of jump-ahead polynomials that dc_bernoulli reads: size it with
 * dc_mt19937_table_bytes and fill it once per device with dc_mt19937_table_init (which copies
 * from host memory and returns when the copy has been queued on `stream`). */
size_t dc_mt19937_table_bytes(void);
dc_status dc_mt19937_table_init(void *table, void *stream);

/* n Bernoulli(p) draws exactly as Generator::bernoulli(n, p) makes them: element e is kept iff
 * the double (random64 & (2^53 - 1)) * 2^-53 of outputs 2e, 2e + 1 is below p.  `state` is the
 * engine's 624 words in device memory (read and written on `stream`); *left / *next are the
 * host-side position, advanced by 2n outputs on return.  keep_bits (device, ceil(n / 32)
 * words): element e is bit e % 32 of word e / 32.  n <= dc_bernoulli_max_draws() per call. */
int64_t dc_bernoulli_max_draws(void);
size_t dc_bernoulli_workspace_size(int64_t n);
dc_status dc_bernoulli(const void *table, uint32_t *state, int64_t *left, int64_t *next,
                       int64_t n, double p, uint32_t *keep_bits, void *workspace,
                       size_t workspace_bytes, void *stream);

/* y[i] = x[i] * (kept(i) ? scale : 0.0f), scale = 1.0f / (float)(1 - p) as the reference
 * rounds it (float32 division).  Also the gradient of dropout (the same product). */
dc_status dc_dropout_apply(const uint32_t *keep_bits, int64_t n, float scale, const float *x,
                           float *y, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* DC_MATH_H */
