/*
 * dc_attn.h — C ABI of the MI355X (gfx950) scaled-dot-product-attention library
 * (libdcattn.so, built from densecore_amd/csrc).
 *
 * This is the drop-in boundary for DenseCore's flash-attention path.  It replaces the two
 * pyo3 entry points of the reference and the CPU kernels behind them:
 *
 *   dc_sdpa_fwd     replaces  _flash_attention           src/lib.rs:609-638
 *                             -> torch_attention::forward  src/torch_attention.rs:143-284
 *   dc_sdpa_bwd     replaces  _flash_attention_backward  src/lib.rs:640-683
 *                             -> torch_attention::backward src/torch_attention.rs:286-468
 *   dc_sdpa_decode  single-query attention; in the reference this is forward() with L = 1,
 *                   non-causal (src/torch_attention.rs:157, 176-180); here it is a split-KV
 *                   kernel pair
 *   dc_last_error   the message the reference would raise (src/lib.rs:561-571, 601-605,
 *                   633, 658-662, 677)
 *
 * Conventions (the reference's, src/torch_attention.rs:7 and src/lib.rs:555-607):
 *   q, out, grad_out, dq : contiguous row-major (B, H, L, E)
 *   k, v, dk, dv         : contiguous row-major (B, Hkv, S, E), H % Hkv == 0 (grouped heads)
 *   lse                  : contiguous (B, H, L), float32, natural log
 *   mask                 : optional additive float32 mask indexed (b, h, l, s) at
 *                          b*mask_stride_b + h*mask_stride_h + l*mask_stride_l + s; the
 *                          reference's (B, H, L, S) contiguous mask has strides
 *                          (H*L*S, L*S, S); a stride of 0 broadcasts that dimension
 *   causal               : top-left aligned, key s visible to query l iff s <= l
 *   scale                : has_scale ? (float)scale : (float)(1 / sqrt((double)E))
 *   fully masked row     : out = 0, lse = 0, and zero gradients
 *
 * All pointers are device pointers (hipMalloc'd or equivalent).  Calls are asynchronous and
 * ordered on `stream` (a hipStream_t; NULL is the null stream).  The caller owns every buffer;
 * workspaces are sized by the matching *_workspace_size call and must be 256-byte aligned.
 * The library's global state: the thread-local last error, per-device caches of facts the
 * launchers size grids by (compute-unit count, kernel occupancy; looked up once, read-only
 * after), and, once the generator of dc_math.h is first used, its jump-ahead polynomials (built
 * once, read-only after).
 */
#ifndef DC_ATTN_H
#define DC_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
    DC_OK = 0,
    DC_INVALID_ARGUMENT = 1, /* shape / argument errors: the reference raises ValueError */
    DC_UNSUPPORTED = 2,      /* outside what the kernels implement (e.g. dims >= 2^31) */
    DC_EXECUTION_FAILED = 3  /* a HIP launch or runtime error: the reference's RuntimeError */
} dc_status;

typedef enum { DC_F32 = 0, DC_BF16 = 1 } dc_dtype;

typedef struct {
    int64_t batch, heads, kv_heads, q_len, kv_len, head_dim;
    int32_t causal;    /* 0 / 1 */
    int32_t has_scale; /* 0: scale = 1/sqrt(head_dim), computed in double then rounded */
    double scale;
    int32_t dtype;     /* dc_dtype of q, k, v, out, grad_out, dq, dk, dv (lse is float32) */
    int32_t flags;     /* DC_FLAG_* bits; 0 for the defaults */
    int64_t mask_stride_b, mask_stride_h, mask_stride_l; /* elements; used when mask != NULL */
} dc_attn_desc;

/* dc_attn_desc.flags.  DC_FLAG_CONSISTENT_SCORES (float32 backward, head dims 65-128): form the
 * scores q.k in the forward's order of products (v_mfma_f32_32x32x2_f32 with the forward's pairing
 * of dims, 32 keys per wave), so that exp(score - lse) normalizes exactly as the forward's did.
 * Without it these head dims take an 8-wave tile of 16 keys on 16x16x4 products (about 20% faster
 * on few-heads shapes), whose scores round in another order: at ordinary scores the results are the
 * same to the float32 bar, at scores near 100 the gradients' error against exact arithmetic grows
 * to a few times the reference's.  No effect elsewhere (head dims up to 64 always use the
 * forward's order).  Other bits are reserved and must be 0. */
#define DC_FLAG_CONSISTENT_SCORES 1

/* Version of this ABI (bumped on any incompatible change). */
int dc_abi_version(void);

/* Forward (out, lse).  src/lib.rs:609-638, src/torch_attention.rs:143-284.  Any head_dim: up to
 * 128 the flash kernels, above 128 the same mathematics materialized over blocks of query rows in
 * the workspace (required then; a smaller one than the size returned only shortens the blocks).
 * Up to 128 the workspace is optional: it holds the longest-first workgroup order of a query-independent mask
 * (mask_stride_l == 0, e.g. key padding); for float32 without a mask, when the query tiles fill
 * at most half of the current device, the partial outputs of split key ranges (so the size
 * depends on the device current at the call); for bf16 without a mask, the power-of-two-scaled
 * fp16 copy of v that the P V product uses.  With less (or none) the forward runs in the natural
 * order, whole key ranges per query tile, and for bf16 takes P as a bf16 hi + lo pair. */
size_t dc_sdpa_fwd_workspace_size(const dc_attn_desc *d);
dc_status dc_sdpa_fwd(const dc_attn_desc *d, const void *q, const void *k, const void *v,
                      const float *mask, void *out, float *lse, void *workspace,
                      size_t workspace_bytes, void *stream);

/* Backward (dq, dk, dv) from the saved out and lse.  src/lib.rs:640-683,
 * src/torch_attention.rs:286-468.  The workspace must hold dsum (batch * heads * q_len floats);
 * the size returned also covers, for float32, the partials that make the result identical from
 * run to run (each key tile's dQ share, and on few-tile grids the dK / dV shares of key tiles
 * split between workgroups, summed in a fixed order; with less, these shares are added with
 * float atomics and the last bits of dq, dk, dv can vary between runs), for bf16, scaled fp16
 * copies of q, k, v and grad_out (with less, P and dS enter their products as bf16 hi + lo
 * pairs) and, for bf16 without a mask on grids that fill at most half of the current device,
 * the float32 partials of its split grids.  The size depends on the device current at the call
 * (its compute-unit count sets the few-tile schedules). */
size_t dc_sdpa_bwd_workspace_size(const dc_attn_desc *d);
dc_status dc_sdpa_bwd(const dc_attn_desc *d, const void *grad_out, const void *q, const void *k,
                      const void *v, const void *out, const float *lse, const float *mask,
                      void *dq, void *dk, void *dv, void *workspace, size_t workspace_bytes,
                      void *stream);

/* Single-query (q_len == 1), non-causal attention over a contiguous KV cache, split over the
 * keys and merged (head_dim up to 256; above, the forward's materialized path at L = 1).  Same
 * results as dc_sdpa_fwd at q_len == 1 (the reference's decode). */
size_t dc_sdpa_decode_workspace_size(const dc_attn_desc *d);
dc_status dc_sdpa_decode(const dc_attn_desc *d, const void *q, const void *k, const void *v,
                         void *out, float *lse, void *workspace, size_t workspace_bytes,
                         void *stream);

/* dc_sdpa_decode without a workspace, for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).  No counterpart
 * in the reference.  It allocates nothing: the split partials go to a static device array of
 * 16 MiB (16 << 20 bytes) that each GPU the library runs on holds until the process ends, so
 * batch * heads * splits * (head_dim + 2) * 4 bytes (dc_sdpa_decode_workspace_size) must fit in
 * it, else DC_UNSUPPORTED.  Every call on one GPU shares that array: calls that overlap on one GPU
 * (other streams, other threads) race and must not be issued.  Results are identical to
 * dc_sdpa_decode's. */
dc_status dc_sdpa_decode_noalloc(const dc_attn_desc *d, const void *q, const void *k, const void *v,
                                 void *out, float *lse, void *stream);

/* Message of the last non-DC_OK status on the calling thread ("" if none). */
const char *dc_last_error(void);

/* The schedule dc_sdpa_fwd / dc_sdpa_bwd would run for a descriptor on the current device, given
 * whether a mask is passed and the workspace size.  No counterpart in the reference (whose
 * schedule is fixed, src/torch_attention.rs:14-35, 107-128): it lets a caller (and the tests)
 * see which grid a call takes.  The query runs the launchers' own decision code without launching
 * anything and touches no device memory. */
typedef struct {
    int32_t split_chunk;    /* forward: key tiles per piece of a split query tile; 0: no split */
    int32_t split_pieces;   /* forward: most pieces of one query tile (1 without a split) */
    int32_t streamk_ranges; /* float32 backward: stream-K ranges; 0: one workgroup per key tile */
    int32_t split_chunk_k;  /* bf16 backward: query steps per dK/dV piece; 0: whole key tiles */
    int32_t split_chunk_q;  /* bf16 backward: key tiles per dQ piece; 0: whole query tiles */
    int32_t f16_products;   /* bf16: 1 when the products run on the scaled fp16 copies */
    int32_t deterministic;  /* backward: 1 when dq, dk, dv are identical from run to run */
    int32_t materialized_rows; /* head_dim > 128: query rows per materialized block; 0: flash */
    int64_t workgroups;     /* workgroups of all the call's launches */
    int32_t chunks;         /* float32 backward: pieces (whole batches, or kv heads of one batch)
                               run one after another so that a smaller workspace still holds the
                               deterministic partials of each; 1: the whole problem at once */
    int32_t reserved;
} dc_sdpa_schedule;

dc_status dc_sdpa_fwd_schedule(const dc_attn_desc *d, int has_mask, size_t workspace_bytes,
                               dc_sdpa_schedule *out);
dc_status dc_sdpa_bwd_schedule(const dc_attn_desc *d, int has_mask, size_t workspace_bytes,
                               dc_sdpa_schedule *out);

#ifdef __cplusplus
}
#endif

#endif /* DC_ATTN_H */
