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
    bool consistent;   // DC_FLAG_CONSISTENT_SCORES: float32 backward scores in the forward's order
};

struct FwdArgs {
    AttnShape s;
    const void *q, *k, *v;
    void *out;
    float *lse;
    // Workspace of a query-independent mask (key padding): each (b, h)'s count of live key tiles
    // and the (b, h) in descending order of it, which sets the workgroup order (longest first).
    // nullptr: natural order.
    int *tiles, *order;
    // bf16 inputs: V copied to fp16, scaled by 2^vexp per (b, kv head) (f16_stage.hip), with the
    // copy's scratch; nullptr: P enters the P V product as bf16 hi + lo.
    void *v16;
    float *f16_partial;
    int *vexp;
    // Split key ranges (no mask, grids that fill under half the device): query tiles
    // of more than split_chunk key tiles run as pieces of split_chunk tiles, each writing its
    // normalized partial output and lse, split_max slots per query row, merged afterwards.
    // nullptr: no split.
    float *split_o, *split_lse;
    size_t split_bytes;  // bytes at split_o (split_lse included)
    int split_chunk, split_max;
};

// Longest-first ordering of a key-padding mask's heads: used when the workspace holds it and
// the grid is small enough for one workgroup to sort.
constexpr int kOrderMaxHeads = 65536;
constexpr int kOrderMaxTiles = 1024;
constexpr int kOrderMaxBatch = 1024;  // batch rows of the one-launch order (key-padding masks)

struct BwdArgs {
    AttnShape s;
    const void *dout, *q, *k, *v, *out;
    const float *lse;
    void *dq, *dk, *dv;
    float *dsum;    // (B, H, L) workspace: rowsum(dout * out)
    float *dq_acc;  // (B, H, L, E) float32 accumulator (== dq for float32)
    // float32, deterministic (when the workspace holds them): each key tile's dQ share goes to a
    // slot of its own (the rows its steps cover), summed in tile order by a reduction; tiles the
    // stream-K schedule cuts between ranges leave each range's dK / dV share in that range's
    // slot, summed in range order.  nullptr: float atomics into dq (and dk / dv of cut tiles).
    float *dq_part, *kv_part;
    size_t part_bytes;  // workspace bytes at dq_part
    // bf16: q, k, v, dout copied to fp16 (f16_stage.hip), each scaled by 2^e per (b, kv head)
    // (q and dout per group of query heads sharing a kv head); exps holds e_q, e_k, e_v, e_do,
    // B*Hkv each.  nullptr: P and dS enter their products as bf16 hi + lo.
    void *q16, *k16, *v16, *do16;
    float *f16_partial;
    int *exps;
    // bf16 with the fp16 copies, no mask, grids that fill under half the device: the dK/dV
    // kernel's key tiles run as pieces of at most chunk_k query steps and the dQ kernel's query
    // tiles as pieces of at most chunk_q key tiles, each writing float32 partials (max_k / max_q
    // slots per row) that a reduction sums in piece order into the bf16 outputs.  nullptr: no
    // split.
    float *split;
    size_t split_bytes;
    int chunk_k, max_k, chunk_q, max_q;
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

// Batched float32 matrix product (bmm.hip): C[b] = A[b] B[b], A (batch, m, k) and B (batch, k, n)
// through element strides, C contiguous (batch, m, n).
struct BmmArgs {
    const float *a, *b;
    float *c;
    int batch, m, n, k;
    int64_t sab, sam, sak;  // A's strides: batch, m, k
    int64_t sbb, sbk, sbn;  // B's strides: batch, k, n
    int64_t scb, scm;       // C's strides: batch, m (unit stride along n)
    bool acc;               // C += A B (else C = A B)
    // Causal attention products of the materialized path (wide.hip); 0 for a plain product.  The
    // m index is row causal_row0 + m of an item whose rows are queries j % causal_L (heads of L
    // rows each), keys are visible up to the query index.  1: n is the key index (scores):
    // tiles whose keys all lie past every query of the tile are skipped, C left unwritten there.
    // 2: k is the key index (P V, dS K): the k loop stops after the tile's last visible key.
    // 3: m is the key index and k the block's rows (P^T dO, dS^T Q): k tiles whose rows all see
    // none of the tile's keys are skipped.
    int causal_mode, causal_L, causal_row0;
};
hipError_t launch_bmm(const BmmArgs &g, hipStream_t st);

// Attention for head dims above 128 (wide.hip), materialized over blocks of query rows in the
// workspace: its full size, the rows per block a given workspace allows (0: too small), and the
// launchers (the backward's workspace starts after dsum).
size_t wide_ws_bytes(const AttnShape &s, bool bf16, bool backward);
int64_t wide_rows(const AttnShape &s, bool bf16, bool backward, size_t bytes);
hipError_t launch_wide_fwd(const FwdArgs &a, bool bf16, void *ws, size_t bytes, hipStream_t st);
hipError_t launch_wide_bwd(const BwdArgs &a, bool bf16, void *ws, size_t bytes, hipStream_t st);
constexpr int kFlashMaxHeadDim = 128;      // the float32 flash kernels' widest instantiation
constexpr int kFlashMaxHeadDimBf16 = 256;  // the bf16 flash kernels' widest instantiation
inline int flash_max_head_dim(bool bf16) { return bf16 ? kFlashMaxHeadDimBf16 : kFlashMaxHeadDim; }

// Rows the reference's blocking fixes (ref_rows.hip): causal attention with a scale that is not
// positive, or a NaN scale.  The forward pass overwrites the rows the reference makes NaN (or 0);
// the backward pass extends NaN rows of lse / dsum to every gradient element the reference's NaN
// reaches.  Both launch nothing unless ref_rows_needed.
bool ref_rows_needed(const AttnShape &s);
hipError_t launch_fwd_ref_rows(const FwdArgs &a, bool bf16, hipStream_t st);
hipError_t launch_bwd_ref_nan(const BwdArgs &a, bool bf16, hipStream_t st);

// Compute units of the current device, and workgroups of `kernel` (`threads` per workgroup) that
// fit on one of them; both looked up once per device (and kernel) and cached.  0 if unknown.
int device_cus();
int device_occupancy(const void *kernel, int threads);

// bf16 -> fp16 copies scaled per slab (f16_stage.hip): segments per slab, and the two passes.
int f16_parts(int64_t nslabs, int64_t slab);
// One tensor to copy: nslabs slabs of `slab` elements (the count is shared by the launch),
// exponents to exps[0 .. nslabs).
constexpr int kMaxF16Copies = 4;
struct F16Copy {
    const void *src;
    void *dst;
    int64_t slab;
    int *exps;
};
// Floats of per-segment maxima that launch_to_f16 needs for these copies.
size_t f16_partial_floats(int64_t nslabs, const F16Copy *copies, int n);
// Up to kMaxF16Copies tensors in two launches (all maxima, then all conversions).
hipError_t launch_to_f16(const F16Copy *copies, int n, int64_t nslabs, float *partial, hipStream_t st);

// Each launcher returns hipSuccess or the launch error; it never synchronizes.
hipError_t launch_fwd_f32(const FwdArgs &a, hipStream_t st);
// Workspace bytes the float32 forward uses to split key ranges on the current device (0: it
// does not split this shape).
size_t fwd_f32_split_bytes(const AttnShape &s);
hipError_t launch_fwd_bf16(const FwdArgs &a, hipStream_t st);
// The same for the bf16 forward (its unmasked path with the fp16 copy of V).
size_t fwd_bf16_split_bytes(const AttnShape &s);
hipError_t launch_bwd_f32(const BwdArgs &a, hipStream_t st);
// Workspace bytes of the float32 backward's deterministic partials on the current device (dQ
// slots, then the stream-K cut tiles' dK / dV slots), with or without a mask.
size_t bwd_f32_part_bytes(const AttnShape &s);
hipError_t launch_bwd_bf16(const BwdArgs &a, hipStream_t st);
// Workspace bytes the bf16 backward uses to split its grids on the current device (0: it does not
// split this shape).
size_t bwd_bf16_split_bytes(const AttnShape &s);
hipError_t launch_decode(const DecodeArgs &a, bool bf16, hipStream_t st);
int decode_splits(const AttnShape &s, int *split_len);
// The allocation-free decode's scratch (a static device array in decode.hip): its size, and its
// address on the current device (looked up with hipGetSymbolAddress once per device).
constexpr size_t kDecodeScratchBytes = (size_t)16 << 20;
constexpr int kDecodeMaxHeadDim = 256;  // the split kernel's widest instantiation
hipError_t decode_scratch(float **ptr);
// `vec`: rows (and mask rows) start 16-byte aligned and the width is a multiple of 4.
hipError_t launch_softmax_fwd(const SoftmaxArgs &a, bool vec, hipStream_t st);
hipError_t launch_softmax_bwd(const SoftmaxArgs &a, bool vec, hipStream_t st);

// The reference's generator stream on the GPU (mt19937.hip).
namespace mt {
constexpr int kState = 624, kM = 397, kDegree = 19937;
constexpr int kTableWords = 624;  // uint32 words per jump polynomial (19968 bits)
constexpr int kRadix = 64, kJumpLevels = 2, kTablePolys = kRadix * kJumpLevels;
constexpr int kChunkLog2 = 17, kChunkWords = 1 << kChunkLog2;  // words per chunk (one wave)
constexpr int kHead = 64;                                       // elements of the base workgroup
constexpr int kMaxChunks = kRadix * kRadix;

struct MtArgs {
    uint32_t *state;      // the engine block (624 words), in/out
    uint32_t *bits;       // keep bits, element e = bit e % 32 of word e / 32
    uint32_t *win;        // out: the window at A0
    int64_t n;            // elements
    uint64_t thr;         // keep iff the 53-bit integer r < thr = ceil(p * 2^53) (r * 2^-53 < p)
    int r, a0, eh;        // first output, first chunk word (relative to the block), head elements
    int64_t state_block;  // block (relative) holding the last output, or -1 when n == 0
};

size_t window_words(int chunks);
bool tables_ready();
const uint32_t *table_words();
bool jump_window_host(const uint32_t *win, uint64_t d, uint32_t *out);
void twist_block_host(const uint32_t *in, uint32_t *out);
hipError_t launch_bernoulli(const MtArgs &a, const uint32_t *table, int chunks, uint32_t *wins,
                            hipStream_t st);
hipError_t launch_dropout_apply(const uint32_t *bits, int64_t n, float scale, const float *x,
                                float *y, hipStream_t st);
}  // namespace mt


}  // namespace dc
