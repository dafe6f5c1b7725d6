// The C ABI declared in include/dc_attn.h and include/dc_math.h: argument checks with the reference's messages,
// scale computation, workspace carving, and dispatch to the kernel launchers.
//
// Checks follow the reference boundary (src/lib.rs:555-580 attention_dims, :594-607
// attention_mask, :658-663 backward shapes); violations return DC_INVALID_ARGUMENT with the
// reference's ValueError text.  Launch failures return DC_EXECUTION_FAILED (the reference's
// RuntimeError, src/lib.rs:633, 677).
#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdint>
#include <map>
#include <mutex>
#include <string>
#include <tuple>

#include "common.hpp"
#include "dc_attn.h"
#include "dc_math.h"
#include "params.hpp"

namespace dc {
namespace {
// Per-device facts the launchers consult on every call (grid sizing), looked up once.
constexpr int kMaxDevices = 64;
std::atomic<int> g_cus[kMaxDevices];
std::mutex g_occupancy_mutex;
std::map<std::tuple<int, const void *, int>, int> g_occupancy;
}  // namespace

int device_cus() {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 0;
    if (dev < kMaxDevices) {
        const int c = g_cus[dev].load(std::memory_order_relaxed);
        if (c > 0) return c;
    }
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    if (dev < kMaxDevices && cus > 0) g_cus[dev].store(cus, std::memory_order_relaxed);
    return cus;
}

int device_occupancy(const void *kernel, int threads) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 0;
    const auto key = std::make_tuple(dev, kernel, threads);
    {
        std::lock_guard<std::mutex> lock(g_occupancy_mutex);
        const auto it = g_occupancy.find(key);
        if (it != g_occupancy.end()) return it->second;
    }
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, threads, 0) != hipSuccess) return 0;
    std::lock_guard<std::mutex> lock(g_occupancy_mutex);
    g_occupancy[key] = per_cu;
    return per_cu;
}

}  // namespace dc

namespace {

thread_local std::string g_error;

dc_status fail(dc_status st, const std::string &msg) {
    g_error = msg;
    return st;
}

dc_status ok() { return DC_OK; }

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// A tensor pointer may be null only when the tensor has no elements.
bool present(const void *p, int64_t count) { return count == 0 || p != nullptr; }
const char *kNullMsg = "flash attention got a null pointer for a non-empty tensor";

constexpr size_t kAlign = 256;
size_t round_up(size_t n) { return (n + kAlign - 1) / kAlign * kAlign; }

// src/lib.rs:555-580 plus this library's own limits (int32 indexing, head dim).
dc_status check_dims(const dc_attn_desc *d, dc::AttnShape *s) {
    if (d == nullptr) return fail(DC_INVALID_ARGUMENT, "flash attention descriptor is null");
    const int64_t dims[6] = {d->batch, d->heads, d->kv_heads, d->q_len, d->kv_len, d->head_dim};
    for (int64_t x : dims)
        if (x < 0) return fail(DC_INVALID_ARGUMENT, "flash attention takes (B, H, L, E) tensors");
    if (d->kv_heads <= 0 || d->heads % d->kv_heads != 0)
        return fail(DC_INVALID_ARGUMENT, "flash attention q/k/v shapes do not match");
    if (d->dtype != DC_F32 && d->dtype != DC_BF16)
        return fail(DC_INVALID_ARGUMENT, "flash attention dtype must be float32 or bfloat16");
    if ((d->flags & ~DC_FLAG_CONSISTENT_SCORES) != 0)
        return fail(DC_INVALID_ARGUMENT, "flash attention flags has unknown bits");
    for (int64_t x : dims)
        if (x > INT32_MAX)
            return fail(DC_UNSUPPORTED, "flash attention dimension exceeds 2^31 - 1");
    if (d->batch * d->heads > INT32_MAX / 2 || d->batch * d->kv_heads > INT32_MAX / 2)
        return fail(DC_UNSUPPORTED, "flash attention batch * heads exceeds 2^30");
    s->B = (int)d->batch;
    s->H = (int)d->heads;
    s->Hkv = (int)d->kv_heads;
    s->L = (int)d->q_len;
    s->S = (int)d->kv_len;
    s->E = (int)d->head_dim;
    s->repeat = s->H / s->Hkv;
    // sdp::calculate_scale, src/torch_attention.rs:37-40: double, stored as float.
    s->scale = d->has_scale ? (float)d->scale : (float)(1.0 / std::sqrt((double)d->head_dim));
    s->scale_log2 = s->scale * 1.4426950408889634f;
    s->causal = d->causal != 0;
    s->mask = nullptr;
    s->msb = s->msh = s->msl = 0;
    s->vec = true;
    s->consistent = (d->flags & DC_FLAG_CONSISTENT_SCORES) != 0;
    return ok();
}

// src/lib.rs:594-607: the reference takes exactly a (B, H, L, S) mask; strides generalise it.
dc_status check_mask(const dc_attn_desc *d, const float *mask, dc::AttnShape *s) {
    if (mask == nullptr) return ok();
    if (d->mask_stride_b < 0 || d->mask_stride_h < 0 || d->mask_stride_l < 0)
        return fail(DC_INVALID_ARGUMENT, "flash attention mask must be (B, H, L, S)");
    s->mask = mask;
    s->msb = d->mask_stride_b;
    s->msh = d->mask_stride_h;
    s->msl = d->mask_stride_l;
    return ok();
}

dc_status launched(hipError_t e) {
    if (e != hipSuccess) return fail(DC_EXECUTION_FAILED, std::string("HIP launch failed: ") +
                                                             hipGetErrorString(e));
    return ok();
}

// The forward's workspace: two int arrays of B*H (live key tiles per head, and the heads in
// descending order of them), used by masks that do not depend on the query; for bf16, then the
// scaled fp16 copy of V with its per-slab scratch (partial maxima, exponents).
size_t fwd_order_ws(const dc::AttnShape &s) { return round_up((size_t)2 * s.B * s.H * sizeof(int)); }
size_t fwd_v16_ws(const dc::AttnShape &s) { return round_up((size_t)s.B * s.Hkv * s.S * s.E * 2); }
size_t fwd_partial_ws(const dc::AttnShape &s) {
    const dc::F16Copy v{nullptr, nullptr, (int64_t)s.S * s.E, nullptr};
    return round_up(dc::f16_partial_floats((int64_t)s.B * s.Hkv, &v, 1) * sizeof(float));
}
size_t fwd_exp_ws(const dc::AttnShape &s) { return round_up((size_t)s.B * s.Hkv * sizeof(int)); }
size_t fwd_ws(const dc::AttnShape &s, bool bf16) {
    if (s.E > dc::flash_max_head_dim(bf16)) return dc::wide_ws_bytes(s, bf16, false);  // required, not optional
    size_t n = fwd_order_ws(s);
    // bf16 up to head dim 128: the fp16 copy of V for the P V product (above, P enters as bf16 hi + lo).
    if (bf16 && s.E <= dc::kFlashMaxHeadDim)
        n += fwd_v16_ws(s) + fwd_partial_ws(s) + fwd_exp_ws(s) + round_up(dc::fwd_bf16_split_bytes(s));
    else n += round_up(dc::fwd_f32_split_bytes(s));
    return n;
}

// The backward's workspace: dsum (B*H*L floats), then for float32 the deterministic partials
// (each key tile's dQ slot and the stream-K cut tiles' dK / dV slots; without them dQ is
// accumulated in its output with atomics), for bf16 the scaled fp16 copies of q, k, v, dout with
// their per-slab scratch, then the float32 partials of split grids (small grids on the current
// device; none otherwise).
struct BwdLayout {
    size_t dsum, part, q16, k16, v16, do16, partial, exps, copies_end, split, total;
};
BwdLayout bwd_layout(const dc::AttnShape &s, bool bf16) {
    BwdLayout l{};
    size_t at = 0;
    auto take = [&](size_t n) {
        const size_t off = at;
        at += round_up(n);
        return off;
    };
    l.dsum = take((size_t)s.B * s.H * s.L * sizeof(float));
    l.part = at;
    if (s.E > dc::flash_max_head_dim(bf16)) {  // beyond the flash kernels: the materialized path's buffers
        take(dc::wide_ws_bytes(s, bf16, true));
        l.total = at;
        return l;
    }
    if (!bf16) take(dc::bwd_f32_part_bytes(s));
    if (bf16) {
        const size_t nq = (size_t)s.B * s.H * s.L * s.E, nk = (size_t)s.B * s.Hkv * s.S * s.E;
        const int64_t qslab = (int64_t)s.repeat * s.L * s.E, kslab = (int64_t)s.S * s.E;
        const int64_t nslabs = (int64_t)s.B * s.Hkv;
        const dc::F16Copy sizes[4] = {{nullptr, nullptr, qslab, nullptr}, {nullptr, nullptr, kslab, nullptr},
                                      {nullptr, nullptr, kslab, nullptr}, {nullptr, nullptr, qslab, nullptr}};
        l.q16 = take(nq * 2);
        l.do16 = take(nq * 2);
        l.k16 = take(nk * 2);
        l.v16 = take(nk * 2);
        l.partial = take(dc::f16_partial_floats(nslabs, sizes, 4) * sizeof(float));  // all four copies' maxima
        l.exps = take((size_t)4 * s.B * s.Hkv * sizeof(int));
        l.copies_end = at;
        l.split = take(dc::bwd_bf16_split_bytes(s));
    }
    l.total = at;
    return l;
}
size_t bwd_ws(const dc::AttnShape &s, bool bf16) { return bwd_layout(s, bf16).total; }
// The least the backward needs (dsum): the float32 deterministic partials and the bf16 fp16
// copies are used only when they fit.
size_t bwd_ws_min(const dc::AttnShape &s) { return bwd_layout(s, false).part; }

// The float32 backward over a piece of the problem: nb whole batches from b0, or (nb == 0) nh kv
// heads of batch b0 from kv head hk0.  Each is contiguous in every tensor, so the piece is the
// same backward over offset pointers; dsum and lse keep the whole problem's layout.
dc::BwdArgs bwd_piece(const dc::BwdArgs &a, int b0, int nb, int hk0, int nh) {
    const dc::AttnShape &s = a.s;
    dc::BwdArgs c = a;
    const int h0 = hk0 * s.repeat;
    if (nb > 0) {
        c.s.B = nb;
    } else {
        c.s.B = 1, c.s.Hkv = nh, c.s.H = nh * s.repeat;
    }
    const int64_t qrow = (int64_t)b0 * s.H + h0, krow = (int64_t)b0 * s.Hkv + hk0;
    const int64_t qoff = qrow * s.L * s.E, koff = krow * s.S * s.E;
    auto off = [](const void *p, int64_t n) -> const void * {
        return p ? static_cast<const float *>(p) + n : nullptr;
    };
    auto offw = [](void *p, int64_t n) -> void * { return p ? static_cast<float *>(p) + n : nullptr; };
    c.dout = off(a.dout, qoff), c.q = off(a.q, qoff), c.out = off(a.out, qoff);
    c.k = off(a.k, koff), c.v = off(a.v, koff);
    c.dq = offw(a.dq, qoff), c.dk = offw(a.dk, koff), c.dv = offw(a.dv, koff);
    c.dq_acc = static_cast<float *>(c.dq);
    c.lse = a.lse + qrow * s.L;
    c.dsum = a.dsum + qrow * s.L;
    if (s.mask) c.s.mask = s.mask + (int64_t)b0 * s.msb + (int64_t)h0 * s.msh;
    c.s.vec = s.vec && aligned16(c.dout) && aligned16(c.q) && aligned16(c.out) && aligned16(c.k) &&
              aligned16(c.v) && aligned16(c.dq) && aligned16(c.dk) && aligned16(c.dv);
    return c;
}

// The float32 backward when `avail` bytes of partials (after dsum) are less than the whole
// problem needs for a result identical from run to run: pieces of whole batches, or of one
// batch's kv heads, each small enough for its partials to fit, run one after another on the
// same stream (each piece is a full backward, so the sums keep their fixed order); if not even
// one kv head fits, the whole problem runs once with float atomics.
dc_status bwd_f32_chunked(const dc::BwdArgs &a, size_t avail, hipStream_t st) {
    const dc::AttnShape &s = a.s;
    auto fits = [&](int nb, int nh) { return dc::bwd_f32_part_bytes(bwd_piece(a, 0, nb, 0, nh).s) <= avail; };
    // The largest piece that fits, stepping down from an estimate (the dQ slots grow linearly with
    // the piece; the stream-K slots of small grids add a bounded amount).
    auto largest = [&](int n, auto fit) {
        int k = n - 1;
        while (k >= 1 && !fit(k)) k -= std::max(1, k / 16);
        return k;
    };
    const int nb = avail > 0 && s.B > 1 ? largest(s.B, [&](int k) { return fits(k, 0); }) : 0;
    const int nh = avail == 0 || nb >= 1 ? 0 : largest(s.Hkv, [&](int k) { return fits(0, k); });
    dc::BwdArgs whole = a;
    if (nb < 1 && nh < 1) {  // float atomics over the whole problem
        whole.dq_part = nullptr, whole.part_bytes = 0;
        return launched(dc::launch_bwd_f32(whole, st));
    }
    int pieces = 0;
    if (nb >= 1) {
        for (int b0 = 0; b0 < s.B; b0 += nb, ++pieces) {
            dc_status r = launched(dc::launch_bwd_f32(bwd_piece(a, b0, std::min(nb, s.B - b0), 0, 0), st));
            if (r != DC_OK) return r;
        }
    } else {
        for (int b0 = 0; b0 < s.B; ++b0)
            for (int hk0 = 0; hk0 < s.Hkv; hk0 += nh, ++pieces) {
                dc_status r = launched(dc::launch_bwd_f32(bwd_piece(a, b0, 0, hk0, std::min(nh, s.Hkv - hk0)), st));
                if (r != DC_OK) return r;
            }
    }
    record_schedule(chunks, pieces);
    return ok();
}

size_t decode_ws(const dc::AttnShape &s, bool bf16) {
    if (s.E > dc::kDecodeMaxHeadDim) return dc::wide_ws_bytes(s, bf16, false);
    int split_len = 0;
    const int splits = dc::decode_splits(s, &split_len);
    return round_up((size_t)s.B * s.H * splits * (s.E + 2) * sizeof(float));
}


// src/activation_dispatch.rs:7-16 (the reference's softmax shape errors) plus the mask's row
// decomposition and this library's int32 column indexing.
dc_status check_softmax(const dc_softmax_desc *d, const float *mask, dc::SoftmaxArgs *a) {
    if (d == nullptr) return fail(DC_INVALID_ARGUMENT, "softmax descriptor is null");
    if (d->rows < 0 || d->width < 0) return fail(DC_INVALID_ARGUMENT, "softmax shape is negative");
    if (d->width == 0)
        return fail(DC_INVALID_ARGUMENT, "softmax requires a nonempty reduction axis");
    if (d->width > INT32_MAX) return fail(DC_UNSUPPORTED, "softmax row length exceeds 2^31 - 1");
    if (d->rows > (int64_t)4 * ((int64_t)UINT32_MAX >> 1))
        return fail(DC_UNSUPPORTED, "softmax row count exceeds 2^33");
    *a = dc::SoftmaxArgs{};
    a->rows = d->rows;
    a->width = (int)d->width;
    a->heads = 1;
    a->q_len = 1;
    a->safe = d->safe != 0;
    if (mask != nullptr) {
        if (d->heads <= 0 || d->q_len <= 0 || d->heads > INT32_MAX || d->q_len > INT32_MAX ||
            d->rows % (d->heads * d->q_len) != 0)
            return fail(DC_INVALID_ARGUMENT, "softmax mask rows must be (B, H, L) with rows == B*H*L");
        if (d->mask_stride_b < 0 || d->mask_stride_h < 0 || d->mask_stride_l < 0)
            return fail(DC_INVALID_ARGUMENT, "softmax mask strides must be non-negative");
        a->mask = mask;
        a->heads = (int)d->heads;
        a->q_len = (int)d->q_len;
        a->msb = d->mask_stride_b;
        a->msh = d->mask_stride_h;
        a->msl = d->mask_stride_l;
    }
    return ok();
}

// A decode launch, then the rows a NaN scale fixes (the decode path is non-causal).
dc_status decode_then_ref_rows(const dc::DecodeArgs &a, bool bf16, hipStream_t st) {
    dc_status r = launched(dc::launch_decode(a, bf16, st));
    if (r != DC_OK) return r;
    const dc::FwdArgs f{a.s, a.q, a.k, a.v, a.out, a.lse, nullptr, nullptr, nullptr, nullptr, nullptr};
    return launched(dc::launch_fwd_ref_rows(f, bf16, st));
}

bool softmax_vec(const dc::SoftmaxArgs &a, const void *p0, const void *p1, const void *p2) {
    bool v = a.width % 4 == 0 && aligned16(p0) && aligned16(p1) && (p2 == nullptr || aligned16(p2));
    if (a.mask) v = v && aligned16(a.mask) && a.msb % 4 == 0 && a.msh % 4 == 0 && a.msl % 4 == 0;
    return v;
}

// The reference's engine position (src/torch_random.rs:79-91, from_words :290-296): the next
// output's index relative to the current block, r in [0, 624].
dc_status mt_position(const void *words, const int64_t *left, const int64_t *next, int64_t *r) {
    if (words == nullptr || left == nullptr || next == nullptr)
        return fail(DC_INVALID_ARGUMENT, "invalid generator state");
    const int64_t l = *left, n = *next;
    if (l < 1 || l > dc::mt::kState || n < 0 || n > dc::mt::kState)
        return fail(DC_INVALID_ARGUMENT, "invalid generator state");
    if (l == 1) {
        *r = dc::mt::kState;
        return ok();
    }
    if (l + n != dc::mt::kState + 1) return fail(DC_INVALID_ARGUMENT, "invalid generator state");
    *r = n;
    return ok();
}

int bernoulli_chunks(int64_t n) {
    if (n <= dc::mt::kHead) return 0;
    return (int)((n - dc::mt::kHead + dc::mt::kChunkWords / 2 - 1) / (dc::mt::kChunkWords / 2));
}

}  // namespace

extern "C" {

int dc_abi_version(void) { return 1; }

const char *dc_last_error(void) { return g_error.c_str(); }

size_t dc_sdpa_fwd_workspace_size(const dc_attn_desc *d) {
    dc::AttnShape s;
    if (check_dims(d, &s) != DC_OK) return 0;
    return fwd_ws(s, d->dtype == DC_BF16);
}

dc_status dc_sdpa_fwd(const dc_attn_desc *d, const void *q, const void *k, const void *v,
                      const float *mask, void *out, float *lse, void *workspace,
                      size_t workspace_bytes, void *stream) {
    dc::AttnShape s;
    dc_status st = check_dims(d, &s);
    if (st != DC_OK) return st;
    if ((st = check_mask(d, mask, &s)) != DC_OK) return st;
    const int64_t nq = (int64_t)s.B * s.H * s.L, nkv = (int64_t)s.B * s.Hkv * s.S * s.E;
    if (nq == 0) return ok();
    if (!present(q, nq * s.E) || !present(k, nkv) || !present(v, nkv) ||
        !present(out, nq * s.E) || !present(lse, nq))
        return fail(DC_INVALID_ARGUMENT, kNullMsg);
    s.vec = aligned16(q) && aligned16(k) && aligned16(v) && aligned16(out);
    dc::FwdArgs a{s, q, k, v, out, lse, nullptr, nullptr, nullptr, nullptr, nullptr};
    if (s.E > dc::flash_max_head_dim(d->dtype == DC_BF16)) {  // materialized over row blocks (wide.hip)
        const bool bf16 = d->dtype == DC_BF16;
        if (workspace == nullptr || dc::wide_rows(s, bf16, false, workspace_bytes) <= 0)
            return fail(DC_INVALID_ARGUMENT,
                        "flash attention forward with head_dim above the flash kernels' (128 for float32, "
                        "256 for bfloat16) needs a workspace of "
                        "dc_sdpa_fwd_workspace_size bytes (at least one row of scores per kv head)");
        hipStream_t strm = static_cast<hipStream_t>(stream);
        dc_status st2 = launched(dc::launch_wide_fwd(a, bf16, workspace, workspace_bytes, strm));
        if (st2 != DC_OK) return st2;
        return launched(dc::launch_fwd_ref_rows(a, bf16, strm));
    }
    // A workspace too small (or none) only gives up the longest-first order of key-padding masks,
    // the split key ranges of small grids, and for bf16 the fp16 P V product (the bf16 hi + lo
    // pair is used instead).
    char *ws = static_cast<char *>(workspace);
    if (mask && ws && workspace_bytes >= fwd_order_ws(s)) {
        a.tiles = reinterpret_cast<int *>(ws);
        a.order = a.tiles + (size_t)s.B * s.H;
    }
    if (d->dtype == DC_F32 && !mask && ws && workspace_bytes > fwd_order_ws(s)) {
        a.split_o = reinterpret_cast<float *>(ws + fwd_order_ws(s));
        a.split_bytes = workspace_bytes - fwd_order_ws(s);
    }
    const size_t bf16_copy = fwd_order_ws(s) + fwd_v16_ws(s) + fwd_partial_ws(s) + fwd_exp_ws(s);
    if (d->dtype == DC_BF16 && !mask && ws && workspace_bytes >= bf16_copy) {
        char *p = ws + fwd_order_ws(s);
        a.v16 = p;
        a.f16_partial = reinterpret_cast<float *>(p + fwd_v16_ws(s));
        a.vexp = reinterpret_cast<int *>(p + fwd_v16_ws(s) + fwd_partial_ws(s));
        if (workspace_bytes > bf16_copy) {
            a.split_o = reinterpret_cast<float *>(ws + bf16_copy);
            a.split_bytes = workspace_bytes - bf16_copy;
        }
    }
    hipStream_t strm = static_cast<hipStream_t>(stream);
    st = launched(d->dtype == DC_F32 ? dc::launch_fwd_f32(a, strm) : dc::launch_fwd_bf16(a, strm));
    if (st != DC_OK) return st;
    return launched(dc::launch_fwd_ref_rows(a, d->dtype == DC_BF16, strm));
}

size_t dc_sdpa_bwd_workspace_size(const dc_attn_desc *d) {
    dc::AttnShape s;
    if (check_dims(d, &s) != DC_OK) return 0;
    return bwd_ws(s, d->dtype == DC_BF16);
}

dc_status dc_sdpa_bwd(const dc_attn_desc *d, const void *grad_out, const void *q, const void *k,
                      const void *v, const void *out, const float *lse, const float *mask,
                      void *dq, void *dk, void *dv, void *workspace, size_t workspace_bytes,
                      void *stream) {
    dc::AttnShape s;
    dc_status st = check_dims(d, &s);
    if (st != DC_OK) return st;
    if ((st = check_mask(d, mask, &s)) != DC_OK) return st;
    const bool bf16 = d->dtype == DC_BF16;
    if (workspace_bytes < bwd_ws_min(s))
        return fail(DC_INVALID_ARGUMENT, "flash attention backward workspace is too small");
    const int64_t nq = (int64_t)s.B * s.H * s.L, nkv = (int64_t)s.B * s.Hkv * s.S * s.E;
    if (!present(grad_out, nq * s.E) || !present(q, nq * s.E) || !present(k, nkv) ||
        !present(v, nkv) || !present(out, nq * s.E) || !present(lse, nq) ||
        !present(dq, nq * s.E) || !present(dk, nkv) || !present(dv, nkv) ||
        !present(workspace, (int64_t)bwd_ws_min(s)))
        return fail(DC_INVALID_ARGUMENT, kNullMsg);
    if (nq == 0 && nkv == 0) return ok();
    s.vec = aligned16(grad_out) && aligned16(q) && aligned16(k) && aligned16(v) &&
            aligned16(out) && aligned16(dq) && aligned16(dk) && aligned16(dv);
    char *ws = static_cast<char *>(workspace);
    dc::BwdArgs a{};
    a.s = s;
    a.dout = grad_out, a.q = q, a.k = k, a.v = v, a.out = out, a.lse = lse;
    a.dq = dq, a.dk = dk, a.dv = dv;
    a.dsum = reinterpret_cast<float *>(ws);
    a.dq_acc = bf16 ? nullptr : static_cast<float *>(dq);
    const BwdLayout l = bwd_layout(s, bf16);
    if (!bf16 && s.E <= dc::kFlashMaxHeadDim && workspace_bytes > l.part) {
        a.dq_part = reinterpret_cast<float *>(ws + l.part);
        a.part_bytes = workspace_bytes - l.part;
    }
    // bf16: the fp16 products when the workspace holds the copies (else the bf16 hi + lo pairs).
    if (bf16 && workspace_bytes >= l.copies_end) {
        a.q16 = ws + l.q16, a.k16 = ws + l.k16, a.v16 = ws + l.v16, a.do16 = ws + l.do16;
        a.f16_partial = reinterpret_cast<float *>(ws + l.partial);
        a.exps = reinterpret_cast<int *>(ws + l.exps);
        if (l.total > l.split && workspace_bytes >= l.total) {
            a.split = reinterpret_cast<float *>(ws + l.split);
            a.split_bytes = l.total - l.split;
        }
    }
    hipStream_t strm = static_cast<hipStream_t>(stream);
    if (!bf16 && s.E <= dc::kFlashMaxHeadDim && workspace_bytes < l.total) {
        // The whole problem's deterministic partials do not fit: run it in pieces whose do.
        st = bwd_f32_chunked(a, workspace_bytes - l.part, strm);
        if (st != DC_OK) return st;
        return launched(dc::launch_bwd_ref_nan(a, bf16, strm));
    }
    if (s.E > dc::flash_max_head_dim(bf16)) {  // materialized over row blocks after dsum (wide.hip)
        if (dc::wide_rows(s, bf16, true, workspace_bytes - l.part) <= 0)
            return fail(DC_INVALID_ARGUMENT,
                        "flash attention backward with head_dim above the flash kernels' (128 for float32, "
                        "256 for bfloat16) needs a workspace of "
                        "dc_sdpa_bwd_workspace_size bytes (at least one row of scores per kv head)");
        st = launched(dc::launch_wide_bwd(a, bf16, ws + l.part, workspace_bytes - l.part, strm));
    } else {
        st = launched(bf16 ? dc::launch_bwd_bf16(a, strm) : dc::launch_bwd_f32(a, strm));
    }
    if (st != DC_OK) return st;
    return launched(dc::launch_bwd_ref_nan(a, bf16, strm));
}

}  // extern "C"

namespace {

// Runs `call` (a dc_sdpa_* entry point over stand-in addresses) as a dry run and reports the
// schedule its launchers chose.  Nothing is launched, so the addresses are never dereferenced.
template <typename F>
dc_status dry_run(dc_sdpa_schedule *out, F call) {
    if (out == nullptr) return fail(DC_INVALID_ARGUMENT, "flash attention schedule output is null");
    dc::Schedule sch;
    dc::g_schedule = &sch;
    const dc_status st = call(reinterpret_cast<void *>(uintptr_t{1} << 12));
    dc::g_schedule = nullptr;
    if (st != DC_OK) return st;
    *out = dc_sdpa_schedule{};
    out->split_chunk = sch.split_chunk;
    out->split_pieces = sch.split_pieces;
    out->streamk_ranges = sch.streamk_ranges;
    out->split_chunk_k = sch.split_chunk_k;
    out->split_chunk_q = sch.split_chunk_q;
    out->f16_products = sch.f16_products;
    out->deterministic = sch.deterministic;
    out->materialized_rows = sch.materialized_rows;
    out->workgroups = sch.workgroups;
    out->chunks = sch.chunks;
    return ok();
}

}  // namespace

extern "C" {

dc_status dc_sdpa_fwd_schedule(const dc_attn_desc *d, int has_mask, size_t workspace_bytes,
                               dc_sdpa_schedule *out) {
    return dry_run(out, [&](void *p) {
        return dc_sdpa_fwd(d, p, p, p, has_mask ? static_cast<const float *>(p) : nullptr, p,
                           static_cast<float *>(p), workspace_bytes ? p : nullptr, workspace_bytes,
                           nullptr);
    });
}

dc_status dc_sdpa_bwd_schedule(const dc_attn_desc *d, int has_mask, size_t workspace_bytes,
                               dc_sdpa_schedule *out) {
    return dry_run(out, [&](void *p) {
        return dc_sdpa_bwd(d, p, p, p, p, p, static_cast<const float *>(p),
                           has_mask ? static_cast<const float *>(p) : nullptr, p, p, p,
                           workspace_bytes ? p : nullptr, workspace_bytes, nullptr);
    });
}

size_t dc_sdpa_decode_workspace_size(const dc_attn_desc *d) {
    dc::AttnShape s;
    if (check_dims(d, &s) != DC_OK) return 0;
    return decode_ws(s, d->dtype == DC_BF16);
}

dc_status dc_sdpa_decode(const dc_attn_desc *d, const void *q, const void *k, const void *v,
                         void *out, float *lse, void *workspace, size_t workspace_bytes,
                         void *stream) {
    dc::AttnShape s;
    dc_status st = check_dims(d, &s);
    if (st != DC_OK) return st;
    if (s.L != 1) return fail(DC_INVALID_ARGUMENT, "flash attention decode takes q_len == 1");
    if (s.causal)
        return fail(DC_INVALID_ARGUMENT,
                    "flash attention decode is non-causal (top-left causal at L = 1 sees one key)");
    if (workspace_bytes < decode_ws(s, d->dtype == DC_BF16))
        return fail(DC_INVALID_ARGUMENT, "flash attention decode workspace is too small");
    const int64_t nq = (int64_t)s.B * s.H, nkv = (int64_t)s.B * s.Hkv * s.S * s.E;
    if (nq == 0) return ok();
    if (!present(q, nq * s.E) || !present(k, nkv) || !present(v, nkv) ||
        !present(out, nq * s.E) || !present(lse, nq) || !present(workspace, 1))
        return fail(DC_INVALID_ARGUMENT, kNullMsg);
    s.vec = aligned16(q) && aligned16(k) && aligned16(v) && aligned16(out);
    if (s.E > dc::kDecodeMaxHeadDim) {  // the forward's materialized path at L = 1 (wide.hip)
        dc::FwdArgs f{s, q, k, v, out, lse, nullptr, nullptr, nullptr, nullptr, nullptr};
        st = launched(dc::launch_wide_fwd(f, d->dtype == DC_BF16, workspace, workspace_bytes,
                                          static_cast<hipStream_t>(stream)));
        if (st != DC_OK) return st;
        return launched(dc::launch_fwd_ref_rows(f, d->dtype == DC_BF16, static_cast<hipStream_t>(stream)));
    }
    dc::DecodeArgs a{};
    a.s = s;
    a.q = q, a.k = k, a.v = v, a.out = out, a.lse = lse;
    a.part = static_cast<float *>(workspace);
    a.splits = dc::decode_splits(s, &a.split_len);
    return decode_then_ref_rows(a, d->dtype == DC_BF16, static_cast<hipStream_t>(stream));
}

dc_status dc_sdpa_decode_noalloc(const dc_attn_desc *d, const void *q, const void *k, const void *v,
                                 void *out, float *lse, void *stream) {
    dc::AttnShape s;
    dc_status st = check_dims(d, &s);
    if (st != DC_OK) return st;
    if (s.L != 1) return fail(DC_INVALID_ARGUMENT, "flash attention decode takes q_len == 1");
    if (s.causal)
        return fail(DC_INVALID_ARGUMENT,
                    "flash attention decode is non-causal (top-left causal at L = 1 sees one key)");
    if (s.E > dc::kDecodeMaxHeadDim)
        return fail(DC_UNSUPPORTED, "flash attention decode without a workspace takes head_dim up to 256; "
                                    "use dc_sdpa_decode with a workspace");
    const size_t need = decode_ws(s, d->dtype == DC_BF16);
    if (need > dc::kDecodeScratchBytes)
        return fail(DC_UNSUPPORTED, "flash attention decode needs " + std::to_string(need) +
                                        " bytes of split partials, more than the " +
                                        std::to_string(dc::kDecodeScratchBytes) +
                                        " bytes of scratch the allocation-free entry point holds "
                                        "(batch * heads too large); use dc_sdpa_decode with a workspace");
    const int64_t nq = (int64_t)s.B * s.H, nkv = (int64_t)s.B * s.Hkv * s.S * s.E;
    if (nq == 0) return ok();
    if (!present(q, nq * s.E) || !present(k, nkv) || !present(v, nkv) ||
        !present(out, nq * s.E) || !present(lse, nq))
        return fail(DC_INVALID_ARGUMENT, kNullMsg);
    s.vec = aligned16(q) && aligned16(k) && aligned16(v) && aligned16(out);
    dc::DecodeArgs a{};
    a.s = s;
    a.q = q, a.k = k, a.v = v, a.out = out, a.lse = lse;
    st = launched(dc::decode_scratch(&a.part));  // the device address, never the array's name
    if (st != DC_OK) return st;
    a.splits = dc::decode_splits(s, &a.split_len);
    return decode_then_ref_rows(a, d->dtype == DC_BF16, static_cast<hipStream_t>(stream));
}

dc_status dc_bmm(const dc_bmm_desc *d, const float *a, const float *b, float *c, void *stream) {
    if (d == nullptr) return fail(DC_INVALID_ARGUMENT, "bmm descriptor is null");
    const int64_t dims[4] = {d->batch, d->m, d->n, d->k};
    for (int64_t x : dims)
        if (x < 0) return fail(DC_INVALID_ARGUMENT, "bmm requires rank-3 operands");
    for (int64_t x : dims)
        if (x > INT32_MAX) return fail(DC_UNSUPPORTED, "bmm dimension exceeds 2^31 - 1");
    const int64_t tiles = ((d->m + 127) / 128) * ((d->n + 63) / 64) * d->batch;
    if (tiles > INT32_MAX) return fail(DC_UNSUPPORTED, "bmm has more than 2^31 - 1 output tiles");
    if (d->batch == 0 || d->m == 0 || d->n == 0) return ok();
    if (c == nullptr || (d->k > 0 && (a == nullptr || b == nullptr)))
        return fail(DC_INVALID_ARGUMENT, "bmm got a null pointer for a non-empty tensor");
    dc::BmmArgs g{};
    g.a = a, g.b = b, g.c = c;
    g.batch = (int)d->batch, g.m = (int)d->m, g.n = (int)d->n, g.k = (int)d->k;
    g.sab = d->a_stride_batch, g.sam = d->a_stride_m, g.sak = d->a_stride_k;
    g.sbb = d->b_stride_batch, g.sbk = d->b_stride_k, g.sbn = d->b_stride_n;
    g.scb = d->m * d->n, g.scm = d->n, g.acc = false;
    return launched(dc::launch_bmm(g, static_cast<hipStream_t>(stream)));
}

dc_status dc_softmax_fwd(const dc_softmax_desc *d, const float *x, const float *mask, float *y,
                         void *stream) {
    dc::SoftmaxArgs a;
    dc_status st = check_softmax(d, mask, &a);
    if (st != DC_OK) return st;
    if (a.rows == 0) return ok();
    if (x == nullptr || y == nullptr) return fail(DC_INVALID_ARGUMENT, "softmax got a null pointer");
    a.a = x;
    a.out = y;
    return launched(dc::launch_softmax_fwd(a, softmax_vec(a, x, y, nullptr),
                                           static_cast<hipStream_t>(stream)));
}

dc_status dc_softmax_bwd(const dc_softmax_desc *d, const float *grad_y, const float *y,
                         float *grad_x, void *stream) {
    dc::SoftmaxArgs a;
    dc_status st = check_softmax(d, nullptr, &a);
    if (st != DC_OK) return st;
    if (a.rows == 0) return ok();
    if (grad_y == nullptr || y == nullptr || grad_x == nullptr)
        return fail(DC_INVALID_ARGUMENT, "softmax got a null pointer");
    a.a = grad_y;
    a.b = y;
    a.out = grad_x;
    return launched(dc::launch_softmax_bwd(a, softmax_vec(a, grad_y, y, grad_x),
                                           static_cast<hipStream_t>(stream)));
}

void dc_mt19937_seed(uint64_t seed, uint32_t *words) {
    if (words == nullptr) return;
    words[0] = (uint32_t)seed;
    for (int j = 1; j < dc::mt::kState; ++j)
        words[j] = 1812433253u * (words[j - 1] ^ (words[j - 1] >> 30)) + (uint32_t)j;
}

dc_status dc_mt19937_advance(uint32_t *words, int64_t *left, int64_t *next, uint64_t count) {
    int64_t r;
    dc_status st = mt_position(words, left, next, &r);
    if (st != DC_OK) return st;
    if (count == 0) return ok();
    if (!dc::mt::tables_ready())
        return fail(DC_EXECUTION_FAILED, "mt19937 jump-ahead tables could not be built");
    const uint64_t last = (uint64_t)r + count - 1;
    const uint64_t block = last / dc::mt::kState;
    if (block > 0) {
        uint32_t w1[dc::mt::kState];
        dc::mt::twist_block_host(words, w1);
        dc::mt::jump_window_host(w1, (block - 1) * dc::mt::kState, words);
    }
    *next = (int64_t)(last - block * dc::mt::kState) + 1;
    *left = dc::mt::kState + 1 - *next;
    return ok();
}

size_t dc_mt19937_table_bytes(void) {
    return (size_t)dc::mt::kTablePolys * dc::mt::kTableWords * sizeof(uint32_t);
}

dc_status dc_mt19937_table_init(void *table, void *stream) {
    if (table == nullptr) return fail(DC_INVALID_ARGUMENT, "mt19937 table pointer is null");
    const uint32_t *w = dc::mt::table_words();
    if (w == nullptr) return fail(DC_EXECUTION_FAILED, "mt19937 jump-ahead tables could not be built");
    const hipError_t e = hipMemcpyAsync(table, w, dc_mt19937_table_bytes(), hipMemcpyHostToDevice,
                                        static_cast<hipStream_t>(stream));
    if (e != hipSuccess)
        return fail(DC_EXECUTION_FAILED, std::string("HIP copy failed: ") + hipGetErrorString(e));
    return ok();
}

int64_t dc_bernoulli_max_draws(void) {
    return dc::mt::kHead + (int64_t)dc::mt::kMaxChunks * (dc::mt::kChunkWords / 2);
}

size_t dc_bernoulli_workspace_size(int64_t n) {
    if (n < 0 || n > dc_bernoulli_max_draws()) return 0;
    return round_up(dc::mt::window_words(bernoulli_chunks(n)) * sizeof(uint32_t));
}

dc_status dc_bernoulli(const void *table, uint32_t *state, int64_t *left, int64_t *next,
                       int64_t n, double p, uint32_t *keep_bits, void *workspace,
                       size_t workspace_bytes, void *stream) {
    int64_t r;
    dc_status st = mt_position(state, left, next, &r);
    if (st != DC_OK) return st;
    if (n < 0) return fail(DC_INVALID_ARGUMENT, "bernoulli count is negative");
    if (!(p >= 0.0 && p <= 1.0)) return fail(DC_INVALID_ARGUMENT, "bernoulli expects 0 <= p <= 1");
    if (n > dc_bernoulli_max_draws())
        return fail(DC_UNSUPPORTED, "bernoulli draws more than dc_bernoulli_max_draws() in one call");
    if (n == 0) return ok();
    if (table == nullptr || keep_bits == nullptr || workspace == nullptr)
        return fail(DC_INVALID_ARGUMENT, "bernoulli got a null pointer");
    if (workspace_bytes < dc_bernoulli_workspace_size(n))
        return fail(DC_INVALID_ARGUMENT, "bernoulli workspace is too small");
    dc::mt::MtArgs a{};
    a.state = state;
    a.bits = keep_bits;
    a.win = static_cast<uint32_t *>(workspace);
    a.n = n;
    a.thr = (uint64_t)std::ceil(p * 0x1p53);  // exact: p in [0, 1], scaled by a power of two
    a.r = (int)r;
    a.eh = dc::mt::kHead;
    a.a0 = a.r + 2 * a.eh;
    const int64_t last = r + 2 * n - 1;
    a.state_block = last / dc::mt::kState;
    st = launched(dc::mt::launch_bernoulli(a, static_cast<const uint32_t *>(table), bernoulli_chunks(n),
                                           a.win, static_cast<hipStream_t>(stream)));
    if (st != DC_OK) return st;
    *next = last - a.state_block * dc::mt::kState + 1;
    *left = dc::mt::kState + 1 - *next;
    return ok();
}

dc_status dc_dropout_apply(const uint32_t *keep_bits, int64_t n, float scale, const float *x,
                           float *y, void *stream) {
    if (n < 0) return fail(DC_INVALID_ARGUMENT, "dropout count is negative");
    if (n == 0) return ok();
    if (keep_bits == nullptr || x == nullptr || y == nullptr)
        return fail(DC_INVALID_ARGUMENT, "dropout got a null pointer");
    if (n > (int64_t)256 * INT32_MAX) return fail(DC_UNSUPPORTED, "dropout count exceeds 2^39");
    return launched(dc::mt::launch_dropout_apply(keep_bits, n, scale, x, y, static_cast<hipStream_t>(stream)));
}

}  // extern "C"
