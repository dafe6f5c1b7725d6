/*
 * TEST INFRASTRUCTURE ONLY: the CPU oracle for DenseCore's scaled-dot-product attention.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load this library,
 * and only as the checker (or the timed CPU baseline).  The product path (densecore_amd)
 * never links, loads or calls it.
 *
 * What it is: a plain-C restatement of DenseCore's Linux float32 flash-attention path, read
 * from the Rust sources as text (the reference needs rustc/cargo, which this image lacks, so
 * it cannot be compiled here).  Every function names the reference file:line it follows:
 *
 *   src/torch_attention.rs:14-284   forward (q/kv split policy, online softmax, repack)
 *   src/torch_attention.rs:286-468  backward (P recomputed from the saved logsumexp)
 *   src/torch_softmax.rs:9-54       reduce_all / add / NEON maximum
 *   src/torch_blas.rs:59-79,95-134,583-642  normalize_last_dims, naive sgemm_, gemm_raw
 *   src/sleef.rs:497-514            SLEEF xexpf (1.0 ULP), lane-wise
 *   src/sleef.rs:1184-1196          glibc expf / logf
 *   src/sleef.rs:1213-1255          exp_u20 (Arm Optimized Routines expf via PyTorch NEON),
 *                                   including its per-4-lane-group fallback to SLEEF expf
 *   src/torch_sum.rs:17-68          thread count (splits work only; never changes bits)
 *   src/torch_softmax.rs:57-67,90-97  softmax_lastdim / softmax_backward_lastdim (the math
 *                                   path's Tensor.softmax(-1) and its gradient)
 *   src/torch_random.rs:9-110,241-254 the generator (PyTorch's mt19937: manual_seed, twist,
 *                                   random, random64, uniform_f64) and bernoulli, sequential
 *
 * Build flags matter: -O2 -ffp-contract=off -fno-fast-math.  Rust never contracts a*b+c,
 * so every explicit Rust `mul_add` is an explicit fmaf here and nothing else is fused.
 *
 * Attribution (the reference's own notices for the code it ported): PyTorch (BSD-3-Clause),
 * SLEEF (Boost Software License 1.0), Arm Optimized Routines (MIT OR Apache-2.0 WITH
 * LLVM-exception).
 *
 * Pinning (see tests/test_oracle.py): closed forms, float64 brute force, torch's CPU SDPA,
 * and per-function checks of the exp kernels, gemm_raw and reduce_all.
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#define EXPORT __attribute__((visibility("default")))

enum { ORACLE_OK = 0, ORACLE_GEMM_LAYOUT = 1, ORACLE_NOMEM = 2, ORACLE_BAD_DIMS = 3 };

static inline float bits_f(uint32_t b) { float f; memcpy(&f, &b, 4); return f; }
static inline uint32_t f_bits(float f) { uint32_t b; memcpy(&b, &f, 4); return b; }

/* Rust `f32 as i32`: truncate toward zero, saturate, NaN -> 0 (NEON vcvtq_s32_f32 too). */
static inline int32_t sat_i32(float x) {
    if (isnan(x)) return 0;
    if (x >= 2147483648.0f) return INT32_MAX;
    if (x < -2147483648.0f) return INT32_MIN;
    return (int32_t)x;
}

/* ---- torch_softmax.rs:43-54 `maximum` (NEON FMAX) and torch_attention.rs:42-45 `std_max` ---- */
static inline float nmax(float a, float b) {
    if (isnan(a) || isnan(b)) return NAN;
    if (a == b) return signbit(a) ? b : a;
    return a > b ? a : b;
}
static inline float std_max(float a, float b) { return a < b ? b : a; }

/* ---- sleef.rs:480-514 SLEEF xexpf, one lane (every step of it is lane-wise) ---- */
#define R_LN2F 1.442695040888963407359924681001892137426645954152985934135449406931f
#define L2UF 0.693145751953125f
#define L2LF 1.428606765330187045e-06f

static inline float pow2i(int32_t q) { return bits_f(((uint32_t)q + 0x7fu) << 23); }
/* vldexp2_vf_vf_vi2: d * 2^(e>>1) * 2^(e - (e>>1)), left to right. */
static inline float ldexp2(float d, int32_t e) {
    int32_t h = e >> 1; /* arithmetic shift, as Rust's i32 >> */
    return d * pow2i(h) * pow2i((int32_t)((uint32_t)e - (uint32_t)h));
}

static float sleef_expf(float d) {
    int32_t q = sat_i32(rintf(d * R_LN2F)); /* round half to even, then saturating cast */
    float qf = (float)q;
    float s = fmaf(qf, -L2UF, d);
    s = fmaf(qf, -L2LF, s);
    float u = (float)0.000198527617612853646278381;
    u = fmaf(u, s, (float)0.00139304355252534151077271);
    u = fmaf(u, s, (float)0.00833336077630519866943359);
    u = fmaf(u, s, (float)0.0416664853692054748535156);
    u = fmaf(u, s, (float)0.166666671633720397949219);
    u = fmaf(u, s, (float)0.5);
    u = 1.0f + fmaf(s * s, u, s);
    u = ldexp2(u, q);
    if (d < -104.0f) u = 0.0f;
    if (100.0f < d) u = INFINITY;
    return u;
}

/* ---- sleef.rs:1213-1255 exp_u20 on one 4-lane group ---- */
static void exp_u20_4(const float x[4], float y[4]) {
    const float bound = bits_f(0x42AEAF15u), inv_ln2 = bits_f(0x3FB8AA3Bu);
    const float ln2_hi = bits_f(0x3F317200u), ln2_lo = bits_f(0x35BFBE8Eu);
    const float c0 = bits_f(0x3C072010u), c1 = bits_f(0x3D2B9F17u), c2 = bits_f(0x3E2AAF33u);
    const float c3 = bits_f(0x3EFFFEDBu), c4 = bits_f(0x3F7FFFF6u);
    int any_big = 0;
    for (int l = 0; l < 4; ++l) any_big |= fabsf(x[l]) > bound;
    if (any_big) { /* the whole group takes SLEEF's expf */
        for (int l = 0; l < 4; ++l) y[l] = sleef_expf(x[l]);
        return;
    }
    for (int l = 0; l < 4; ++l) {
        float n = roundf(x[l] * inv_ln2); /* vrndaq: halves away from zero */
        float r = fmaf(-n, ln2_hi, x[l]);
        r = fmaf(-n, ln2_lo, r);
        float scale = bits_f(((uint32_t)sat_i32(n) << 23) + 0x3f800000u);
        float r2 = r * r;
        float p = fmaf(r, c0, c1);
        float q = fmaf(r, c2, c3);
        q = fmaf(p, r2, q);
        p = c4 * r;
        float poly = fmaf(q, r2, p);
        y[l] = fmaf(poly, scale, scale);
    }
}

/* ---- torch_softmax.rs:14-37 reduce_all, for the two reductions the path uses ---- */
static float reduce_all_max(const float *v, size_t size) {
    if (size < 4) {
        float acc = v[0];
        for (size_t i = 1; i < size; ++i) acc = nmax(acc, v[i]);
        return acc;
    }
    float acc[4] = {v[0], v[1], v[2], v[3]};
    size_t whole = size - size % 4, d = 4;
    for (; d < whole; d += 4)
        for (int l = 0; l < 4; ++l) acc[l] = nmax(acc[l], v[d + l]);
    for (size_t l = 0; l < size - d; ++l) acc[l] = nmax(acc[l], v[d + l]);
    return nmax(nmax(acc[0], acc[2]), nmax(acc[1], acc[3]));
}

/* values(i) = a[i] * b[i] (one rounding), op = add (torch_attention.rs:327-330). */
static float reduce_all_dot(const float *a, const float *b, size_t size) {
    if (size < 4) {
        float acc = a[0] * b[0];
        for (size_t i = 1; i < size; ++i) acc = acc + a[i] * b[i];
        return acc;
    }
    float acc[4];
    for (int l = 0; l < 4; ++l) acc[l] = a[l] * b[l];
    size_t whole = size - size % 4, d = 4;
    for (; d < whole; d += 4)
        for (int l = 0; l < 4; ++l) acc[l] = acc[l] + a[d + l] * b[d + l];
    for (size_t l = 0; l < size - d; ++l) acc[l] = acc[l] + a[d + l] * b[d + l];
    return (acc[0] + acc[2]) + (acc[1] + acc[3]);
}

/* ---- torch_attention.rs:47-87 mul_reduce_max ---- */
static float mul_reduce_max(float *row, size_t size, float scale) {
    size_t end_n = size / 8 * 8, end = size / 4 * 4, i = 0;
    float acc[2][4], tail[4];
    for (int l = 0; l < 4; ++l) acc[0][l] = acc[1][l] = tail[l] = -INFINITY;
    for (; i < end_n; i += 8)
        for (int h = 0; h < 2; ++h)
            for (int l = 0; l < 4; ++l) {
                float x = row[i + 4 * h + l] * scale;
                row[i + 4 * h + l] = x;
                acc[h][l] = nmax(acc[h][l], x);
            }
    for (; i < end; i += 4)
        for (int l = 0; l < 4; ++l) {
            float x = row[i + l] * scale;
            row[i + l] = x;
            tail[l] = nmax(tail[l], x);
        }
    for (int l = 0; l < 4; ++l) acc[0][l] = nmax(acc[0][l], tail[l]);
    float tmp_max = -INFINITY;
    for (; i < size; ++i) {
        row[i] *= scale;
        tmp_max = std_max(tmp_max, row[i]);
    }
    float v[4];
    for (int l = 0; l < 4; ++l) v[l] = nmax(acc[0][l], acc[1][l]);
    float reduced = nmax(nmax(v[0], v[2]), nmax(v[1], v[3]));
    return isnan(reduced) ? NAN : std_max(tmp_max, reduced);
}

/* ---- torch_attention.rs:89-105 exp_reduce_sum ---- */
static float exp_reduce_sum(float *row, size_t size, float max) {
    size_t end = size / 4 * 4;
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (size_t i = 0; i < end; i += 4) {
        float x[4], e[4];
        for (int l = 0; l < 4; ++l) x[l] = row[i + l] - max;
        exp_u20_4(x, e);
        for (int l = 0; l < 4; ++l) {
            acc[l] = acc[l] + e[l];
            row[i + l] = e[l];
        }
    }
    float sum = (acc[0] + acc[2]) + (acc[1] + acc[3]);
    for (size_t i = end; i < size; ++i) {
        float e = expf(row[i] - max); /* glibc, sleef.rs:1184-1187 */
        sum += e;
        row[i] = e;
    }
    return sum;
}

/* ---- torch_attention.rs:130-141 scale_add_mask ---- */
static void scale_add_mask(float *row, const float *mask, size_t size, float scale) {
    size_t whole = size / 4 * 4;
    for (size_t i = 0; i < size; ++i)
        row[i] = i < whole ? row[i] * scale + mask[i] : fmaf(row[i], scale, mask[i]);
}

/* ---- torch_blas.rs:59-79 normalize_last_dims, :95-134 portable sgemm_, :583-642 gemm_raw ---- */
static int gemm_raw(int ta, int tb, size_t m, size_t n, size_t k, float alpha, const float *a,
                    size_t lda, const float *b, size_t ldb, float beta, float *c, size_t ldc) {
    if (n == 1) ldc = m;
    if (ta) {
        if (m == 1) lda = k;
    } else if (k == 1) {
        lda = m;
    }
    if (tb) {
        if (k == 1) ldb = n;
    } else if (n == 1) {
        ldb = k;
    }
    size_t dims[6] = {m, n, k, lda, ldb, ldc};
    for (int i = 0; i < 6; ++i)
        if (dims[i] > (size_t)INT32_MAX) return ORACLE_GEMM_LAYOUT;
    size_t need_a = ta ? k : m, need_b = tb ? n : k;
    if (lda < (need_a ? need_a : 1) || ldb < (need_b ? need_b : 1) || ldc < (m ? m : 1))
        return ORACLE_GEMM_LAYOUT;
    if (m == 0 || n == 0) return ORACLE_OK;
    for (size_t j = 0; j < n; ++j)
        for (size_t i = 0; i < m; ++i) {
            float sum = 0.0f;
            for (size_t p = 0; p < k; ++p) {
                float av = a[ta ? p + i * lda : i + p * lda];
                float bv = b[tb ? j + p * ldb : p + j * ldb];
                sum += av * bv;
            }
            float *out = c + i + j * ldc;
            *out = beta == 0.0f ? alpha * sum : alpha * sum + beta * *out;
        }
    return ORACLE_OK;
}

/* ---- torch_attention.rs:16-40 dims, q_split, scale ---- */
typedef struct {
    size_t batch, heads, kv_heads, q_len, kv_len, head_dim;
} dims_t;

#define KV_SPLIT 512
static size_t q_split(size_t q_len) { return q_len >= 768 ? 256 : q_len >= 192 ? 64 : 32; }
static float scale_factor(size_t e, int has_scale, double scale) {
    return has_scale ? (float)scale : (float)(1.0 / sqrt((double)e));
}
static size_t min_sz(size_t a, size_t b) { return a < b ? a : b; }
static size_t at_least1(size_t a) { return a ? a : 1; }

/* ---- torch_attention.rs:107-128 par_chunks: task i runs on thread i*threads/parts ---- */
typedef struct {
    void (*fn)(void *ctx, size_t task);
    void *ctx;
    size_t parts, threads, me;
} worker_t;

static void *worker_main(void *arg) {
    worker_t *w = (worker_t *)arg;
    for (size_t i = 0; i < w->parts; ++i)
        if (i * w->threads / w->parts == w->me) w->fn(w->ctx, i);
    return NULL;
}

static size_t g_threads = 0; /* torch_sum.rs:17-68: 0 means "ask the OS" */
static size_t num_threads(void) {
    if (g_threads) return g_threads;
    long n = sysconf(_SC_NPROCESSORS_ONLN);
    return n > 0 ? (size_t)n : 1;
}

static void par_tasks(size_t parts, void (*fn)(void *, size_t), void *ctx) {
    if (parts == 0) return;
    size_t threads = min_sz(num_threads(), parts);
    if (threads < 1) threads = 1;
    worker_t *ws = (worker_t *)calloc(threads, sizeof(worker_t));
    pthread_t *ts = (pthread_t *)calloc(threads, sizeof(pthread_t));
    for (size_t t = 0; t < threads; ++t) {
        ws[t] = (worker_t){fn, ctx, parts, threads, t};
        if (t + 1 < threads) pthread_create(&ts[t], NULL, worker_main, &ws[t]);
    }
    worker_main(&ws[threads - 1]);
    for (size_t t = 0; t + 1 < threads; ++t) pthread_join(ts[t], NULL);
    free(ws);
    free(ts);
}

/* ---- torch_attention.rs:143-284 forward ---- */
typedef struct {
    const float *q, *k, *v, *mask;
    dims_t d;
    int causal;
    float scale;
    size_t qs, kvs;
    float *out, *lse;
    volatile int failed;
} fwd_ctx;

static void fwd_task(void *p, size_t t) {
    fwd_ctx *c = (fwd_ctx *)p;
    const dims_t d = c->d;
    const size_t e = d.head_dim, qs = c->qs, kvs = c->kvs, repeat = d.heads / d.kv_heads;
    const size_t b = t / d.heads, h = t % d.heads;
    const size_t qb_base = t * d.q_len * e;
    const size_t kv_base = (b * d.kv_heads + h / repeat) * d.kv_len * e;
    float *out = c->out + t * d.q_len * e, *lse = c->lse + t * d.q_len;
    float *qk = (float *)calloc(at_least1(qs * kvs), sizeof(float));
    float *dst = (float *)calloc(at_least1(qs * e), sizeof(float));
    float *qk_max = (float *)calloc(at_least1(qs), sizeof(float));
    float *qk_sum = (float *)calloc(at_least1(qs), sizeof(float));
    if (!qk || !dst || !qk_max || !qk_sum) {
        c->failed = ORACLE_NOMEM;
        goto done;
    }
    for (size_t m = 0; m < d.q_len; m += (qs ? qs : 1)) {
        size_t qb = min_sz(qs, d.q_len - m);
        for (size_t r = 0; r < qb; ++r) qk_max[r] = -INFINITY, qk_sum[r] = 0.0f;
        size_t num_keys = c->causal ? min_sz(m + qb, d.kv_len) : d.kv_len;
        for (size_t n = 0; n < num_keys; n += (kvs ? kvs : 1)) {
            size_t kvb = min_sz(kvs, d.kv_len - n);
            int r = gemm_raw(1, 0, kvb, qb, e, 1.0f, c->k + kv_base + n * e, e,
                             c->q + qb_base + m * e, e, 0.0f, qk, kvb);
            if (r) {
                c->failed = r;
                goto done;
            }
            if (c->causal && num_keys - n <= kvs)
                for (size_t row = 0; row < qb; ++row) {
                    size_t from = m + row + 1 > n ? m + row + 1 - n : 0;
                    from = min_sz(from, kvb);
                    for (size_t i = from; i < kvb; ++i) qk[row * kvb + i] = -INFINITY;
                }
            for (size_t row = 0; row < qb; ++row) {
                float *rr = qk + row * kvb;
                float tmp_max;
                if (c->mask) {
                    size_t at = (t * d.q_len + m + row) * d.kv_len + n;
                    scale_add_mask(rr, c->mask + at, kvb, c->scale);
                    tmp_max = reduce_all_max(rr, kvb);
                } else {
                    tmp_max = mul_reduce_max(rr, kvb, c->scale);
                }
                tmp_max = qk_max[row] > tmp_max ? qk_max[row] : tmp_max;
                if (tmp_max == -INFINITY) {
                    for (size_t i = 0; i < kvb; ++i) rr[i] = 0.0f;
                    continue;
                }
                float tmp_sum = exp_reduce_sum(rr, kvb, tmp_max);
                float exp_tmp = expf(qk_max[row] - tmp_max);
                qk_sum[row] = fmaf(exp_tmp, qk_sum[row], tmp_sum);
                qk_max[row] = tmp_max;
                if (n > 0)
                    for (size_t i = 0; i < e; ++i) dst[row * e + i] *= exp_tmp;
            }
            float beta = n == 0 ? 0.0f : 1.0f;
            r = gemm_raw(0, 0, e, qb, kvb, 1.0f, c->v + kv_base + n * e, e, qk, kvb, beta, dst, e);
            if (r) {
                c->failed = r;
                goto done;
            }
        }
        for (size_t row = 0; row < qb; ++row) {
            if (qk_max[row] == -INFINITY) qk_max[row] = 0.0f;
            if (qk_sum[row] == 0.0f) qk_sum[row] = 1.0f;
            float recip = 1.0f / qk_sum[row];
            for (size_t i = 0; i < e; ++i) out[(m + row) * e + i] = dst[row * e + i] * recip;
            lse[m + row] = qk_max[row] + logf(qk_sum[row]);
        }
    }
done:
    free(qk);
    free(dst);
    free(qk_max);
    free(qk_sum);
}

static int check_dims(dims_t d) {
    if (d.kv_heads == 0 || d.heads % d.kv_heads) return ORACLE_BAD_DIMS;
    return ORACLE_OK;
}

EXPORT int oracle_forward(const float *q, const float *k, const float *v, const float *mask,
                          size_t batch, size_t heads, size_t kv_heads, size_t q_len, size_t kv_len,
                          size_t head_dim, int causal, int has_scale, double scale, float *out,
                          float *lse) {
    dims_t d = {batch, heads, kv_heads, q_len, kv_len, head_dim};
    if (check_dims(d)) return ORACLE_BAD_DIMS;
    fwd_ctx c = {q, k, v, mask, d, causal, scale_factor(head_dim, has_scale, scale),
                 min_sz(q_split(q_len), q_len), min_sz(KV_SPLIT, kv_len), out, lse, 0};
    /* The reference returns zero-initialised rows for tasks it never touches. */
    memset(out, 0, batch * heads * q_len * head_dim * sizeof(float));
    memset(lse, 0, batch * heads * q_len * sizeof(float));
    par_tasks(batch * heads, fwd_task, &c);
    return c.failed;
}

/* ---- torch_attention.rs:286-468 backward ---- */
typedef struct {
    const float *g, *q, *k, *v, *o, *lse, *mask;
    dims_t d;
    int causal;
    float scale;
    size_t qs, kvs;
    float *gq, *gk, *gv;
    volatile int failed;
} bwd_ctx;

static void bwd_task(void *p, size_t t) {
    bwd_ctx *c = (bwd_ctx *)p;
    const dims_t d = c->d;
    const size_t e = d.head_dim, qs = c->qs, kvs = c->kvs, repeat = d.heads / d.kv_heads;
    const size_t kv_base = t * d.kv_len * e;
    float *gk = c->gk + kv_base, *gv = c->gv + kv_base;
    float *attn = (float *)calloc(at_least1(qs * kvs), sizeof(float));
    float *grad_attn = (float *)calloc(at_least1(qs * kvs), sizeof(float));
    float *dsum = (float *)calloc(at_least1(qs), sizeof(float));
    int r = ORACLE_OK;
    if (!attn || !grad_attn || !dsum) {
        r = ORACLE_NOMEM;
        goto done;
    }
    for (size_t rep = 0; rep < repeat; ++rep) {
        size_t j = t * repeat + rep; /* (batch, head) index of this query head */
        size_t q_base = j * d.q_len * e;
        float *gq = c->gq + q_base;
        for (size_t m = 0; m < d.q_len; m += (qs ? qs : 1)) {
            size_t qb = min_sz(qs, d.q_len - m);
            for (size_t row = 0; row < qb; ++row) {
                size_t at = q_base + (m + row) * e;
                dsum[row] = reduce_all_dot(c->g + at, c->o + at, e);
            }
            size_t num_keys = c->causal ? min_sz(m + qb, d.kv_len) : d.kv_len;
            for (size_t n = 0; n < num_keys; n += (kvs ? kvs : 1)) {
                size_t kvb = min_sz(kvs, d.kv_len - n);
                if ((r = gemm_raw(1, 0, kvb, qb, e, c->scale, c->k + kv_base + n * e, e,
                                  c->q + q_base + m * e, e, 0.0f, attn, kvb)))
                    goto done;
                if (c->mask)
                    for (size_t row = 0; row < qb; ++row) {
                        size_t at = (j * d.q_len + m + row) * d.kv_len + n;
                        for (size_t i = 0; i < kvb; ++i) attn[row * kvb + i] += c->mask[at + i];
                    }
                for (size_t row = 0; row < qb; ++row) {
                    float norm = c->lse[j * d.q_len + m + row];
                    for (size_t i = 0; i < kvb; ++i)
                        attn[row * kvb + i] = sleef_expf(attn[row * kvb + i] - norm);
                }
                if (c->causal && num_keys - n <= kvs)
                    for (size_t row = 0; row < qb; ++row) {
                        size_t from = m + row + 1 > n ? m + row + 1 - n : 0;
                        from = min_sz(from, kvb);
                        for (size_t i = from; i < kvb; ++i) attn[row * kvb + i] = 0.0f;
                    }
                if ((r = gemm_raw(0, 1, e, kvb, qb, 1.0f, c->g + q_base + m * e, e, attn, kvb,
                                  1.0f, gv + n * e, e)))
                    goto done;
                if ((r = gemm_raw(1, 0, kvb, qb, e, 1.0f, c->v + kv_base + n * e, e,
                                  c->g + q_base + m * e, e, 0.0f, grad_attn, kvb)))
                    goto done;
                for (size_t row = 0; row < qb; ++row)
                    for (size_t i = 0; i < kvb; ++i) {
                        float a = attn[row * kvb + i];
                        grad_attn[row * kvb + i] = a * (grad_attn[row * kvb + i] - dsum[row]);
                    }
                if ((r = gemm_raw(0, 0, e, qb, kvb, c->scale, c->k + kv_base + n * e, e, grad_attn,
                                  kvb, 1.0f, gq + m * e, e)))
                    goto done;
                if ((r = gemm_raw(0, 1, e, kvb, qb, c->scale, c->q + q_base + m * e, e, grad_attn,
                                  kvb, 1.0f, gk + n * e, e)))
                    goto done;
            }
        }
    }
done:
    if (r) c->failed = r;
    free(attn);
    free(grad_attn);
    free(dsum);
}

EXPORT int oracle_backward(const float *grad_out, const float *q, const float *k, const float *v,
                           const float *out, const float *lse, const float *mask, size_t batch,
                           size_t heads, size_t kv_heads, size_t q_len, size_t kv_len,
                           size_t head_dim, int causal, int has_scale, double scale, float *gq,
                           float *gk, float *gv) {
    dims_t d = {batch, heads, kv_heads, q_len, kv_len, head_dim};
    if (check_dims(d)) return ORACLE_BAD_DIMS;
    bwd_ctx c = {grad_out, q, k, v, out, lse, mask, d, causal,
                 scale_factor(head_dim, has_scale, scale), min_sz(q_split(q_len), q_len),
                 min_sz(KV_SPLIT, kv_len), gq, gk, gv, 0};
    memset(gq, 0, batch * heads * q_len * head_dim * sizeof(float));
    memset(gk, 0, batch * kv_heads * kv_len * head_dim * sizeof(float));
    memset(gv, 0, batch * kv_heads * kv_len * head_dim * sizeof(float));
    par_tasks(batch * kv_heads, bwd_task, &c);
    return c.failed;
}

/* ---- torch_softmax.rs:14-37 reduce_all with op = add over plain values ---- */
static float reduce_all_sum(const float *v, size_t size) {
    if (size < 4) {
        float acc = v[0];
        for (size_t i = 1; i < size; ++i) acc = acc + v[i];
        return acc;
    }
    float acc[4] = {v[0], v[1], v[2], v[3]};
    size_t whole = size - size % 4, d = 4;
    for (; d < whole; d += 4)
        for (int l = 0; l < 4; ++l) acc[l] = acc[l] + v[d + l];
    for (size_t l = 0; l < size - d; ++l) acc[l] = acc[l] + v[d + l];
    return (acc[0] + acc[2]) + (acc[1] + acc[3]);
}

/* ---- torch_softmax.rs:57-67 softmax_lastdim: max, exp_array (SLEEF expf lane by lane,
 * sleef.rs:1292-1298, 1502-1503), sum, then e * (1 / sum) ---- */
EXPORT void oracle_softmax(const float *x, size_t rows, size_t width, float *y) {
    for (size_t r = 0; r < rows; ++r) {
        const float *row = x + r * width;
        float *out = y + r * width;
        const float max = reduce_all_max(row, width);
        for (size_t i = 0; i < width; ++i) out[i] = sleef_expf(row[i] - max);
        const float inv = 1.0f / reduce_all_sum(out, width);
        for (size_t i = 0; i < width; ++i) out[i] = out[i] * inv;
    }
}

/* ---- torch_softmax.rs:90-97 softmax_backward_lastdim: (g - sum(g * y)) * y ---- */
EXPORT void oracle_softmax_backward(const float *g, const float *y, size_t rows, size_t width,
                                    float *dx) {
    for (size_t r = 0; r < rows; ++r) {
        const float *gr = g + r * width, *yr = y + r * width;
        const float sum = reduce_all_dot(gr, yr, width);
        for (size_t i = 0; i < width; ++i) dx[r * width + i] = (gr[i] - sum) * yr[i];
    }
}

/* ---- torch_random.rs:9-110, 241-254: the reference's generator, one output at a time ---- */
typedef struct {
    uint32_t state[624];
    int64_t left, next;
} mt_t;

static uint32_t mt_twist(uint32_t u, uint32_t v) {
    return (((u & 0x80000000u) | (v & 0x7fffffffu)) >> 1) ^ ((v & 1u) ? 0x9908b0dfu : 0u);
}

/* manual_seed, torch_random.rs:43-56 */
EXPORT void oracle_mt_seed(mt_t *g, uint64_t seed) {
    g->state[0] = (uint32_t)seed;
    for (int j = 1; j < 624; ++j)
        g->state[j] = 1812433253u * (g->state[j - 1] ^ (g->state[j - 1] >> 30)) + (uint32_t)j;
    g->left = 1;
    g->next = 0;
}

/* next_state, torch_random.rs:66-77 (in place, three loops) */
static void mt_next_state(mt_t *g) {
    uint32_t *s = g->state;
    g->left = 624;
    g->next = 0;
    for (int j = 0; j < 624 - 397; ++j) s[j] = s[j + 397] ^ mt_twist(s[j], s[j + 1]);
    for (int j = 624 - 397; j < 623; ++j) s[j] = s[j + 397 - 624] ^ mt_twist(s[j], s[j + 1]);
    s[623] = s[396] ^ mt_twist(s[623], s[0]);
}

/* random, torch_random.rs:79-91 */
static uint32_t mt_random(mt_t *g) {
    if (--g->left == 0) mt_next_state(g);
    uint32_t y = g->state[g->next++];
    y ^= y >> 11;
    y ^= (y << 7) & 0x9d2c5680u;
    y ^= (y << 15) & 0xefc60000u;
    y ^= y >> 18;
    return y;
}

/* uniform_f64(0, 1), torch_random.rs:93-110: random64 = hi << 32 | lo, 53 bits, then
 * mul_add(1 - 0, 0) which leaves the product unchanged. */
static double mt_uniform_f64(mt_t *g) {
    const uint64_t hi = mt_random(g), lo = mt_random(g);
    const uint64_t r = ((hi << 32) | lo) & ((1ull << 53) - 1);
    return fma((double)r * (1.0 / (double)(1ull << 53)), 1.0, 0.0);
}

EXPORT void oracle_mt_random(mt_t *g, uint32_t *out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = mt_random(g);
}

EXPORT void oracle_mt_uniform_f64(mt_t *g, double *out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = mt_uniform_f64(g);
}

/* bernoulli, torch_random.rs:241-254: 1.0 where the double uniform is below p. */
EXPORT void oracle_mt_bernoulli(mt_t *g, double p, float *out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = mt_uniform_f64(g) < p ? 1.0f : 0.0f;
}

/* ---- thread count, torch_sum.rs:51-68 ---- */
EXPORT void oracle_set_num_threads(size_t n) { g_threads = n; }
EXPORT size_t oracle_get_num_threads(void) { return num_threads(); }

/* ---- single functions, exported so tests can pin each against the mathematics ---- */
EXPORT void oracle_exp_u20(const float *x, float *y, size_t n) {
    for (size_t i = 0; i + 4 <= n; i += 4) exp_u20_4(x + i, y + i);
}
EXPORT void oracle_sleef_expf(const float *x, float *y, size_t n) {
    for (size_t i = 0; i < n; ++i) y[i] = sleef_expf(x[i]);
}
EXPORT float oracle_reduce_max(const float *x, size_t n) { return reduce_all_max(x, n); }
EXPORT float oracle_reduce_dot(const float *a, const float *b, size_t n) {
    return reduce_all_dot(a, b, n);
}
EXPORT float oracle_mul_reduce_max(float *row, size_t n, float scale) {
    return mul_reduce_max(row, n, scale);
}
EXPORT float oracle_exp_reduce_sum(float *row, size_t n, float max) {
    return exp_reduce_sum(row, n, max);
}
EXPORT int oracle_gemm_raw(int ta, int tb, size_t m, size_t n, size_t k, float alpha,
                           const float *a, size_t lda, const float *b, size_t ldb, float beta,
                           float *c, size_t ldc) {
    return gemm_raw(ta, tb, m, n, k, alpha, a, lda, b, ldb, beta, c, ldc);
}
EXPORT float oracle_scale_factor(size_t e, int has_scale, double scale) {
    return scale_factor(e, has_scale, scale);
}
EXPORT size_t oracle_q_split(size_t q_len) { return q_split(q_len); }
