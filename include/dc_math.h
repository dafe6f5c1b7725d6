/*
 * dc_math.h — C ABI of the device-side pieces of DenseCore's composed ("math") attention path,
 * in the same library as dc_attn.h (libdcattn.so).
 *
 * The reference's math path (python/densecore/functional.py:318-340, used for dropout, masks
 * the flash path rejects, Ev != E and masks that require a gradient) and its
 * multi_head_attention_forward (functional.py:400-461) are composed from bmm, an additive
 * mask, softmax over the last axis and dropout.  The two products are plain batched GEMMs (the
 * caller's BLAS); this header covers the rest:
 *
 *   dc_softmax_fwd   replaces  Tensor.softmax(-1) on the scores   src/lib.rs:269-270
 *                              -> activation_dispatch::softmax     src/activation_dispatch.rs:61
 *                              -> torch_softmax::softmax_lastdim   src/torch_softmax.rs:57-67
 *                    fused with the additive mask (functional.py:330-333) and the math path's
 *                    safe softmax (functional.py:334-337: rows that are all -inf give 0)
 *   dc_softmax_bwd   replaces  torch_softmax::softmax_backward_lastdim src/torch_softmax.rs:90-97
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

#ifdef __cplusplus
}
#endif

#endif /* DC_MATH_H */
