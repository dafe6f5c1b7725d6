// Shared device helpers for the gfx950 attention kernels.
//
// MFMA layouts used throughout (CDNA3/CDNA4 ISA, wave64):
//   v_mfma_f32_32x32x2_f32 (a, b, c):  A is 32x2, B is 2x32, C is 32x32.
//     lane l supplies a = A[l % 32][l / 32] and b = B[l / 32][l % 32];
//     lane l holds C[i][l % 32] in c[r] for i = 8*(r/4) + 4*(l/32) + r%4, r = 0..15.
//   v_mfma_f32_32x32x16_bf16 (a, b, c): A is 32x16, B is 16x32, same C layout;
//     lane l supplies A[l % 32][8*(l/32) + 0..7] and B[8*(l/32) + 0..7][l % 32].
// Because the reduction index of an MFMA may be permuted freely (as long as A and B agree),
// an accumulator C[i][j] (lane <-> column j) can feed the next MFMA directly as its B operand
// with "row i of C" as the reduction index: step s of a 32x32x2 chain takes register s, which
// is row perm2(s, l/32) = 8*(s/4) + 4*(l/32) + s%4.  The kernels use this to keep P in
// registers between the two products of attention.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));

#define DEVI __device__ __forceinline__

namespace dc {

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

DEVI f32x16 mfma_f32(float a, float b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}
DEVI f32x16 mfma_bf16(bf16x8 a, bf16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
// fp16 operands carried in bf16x8 registers (16-bit patterns; the tiles hold either type).
DEVI f32x16 mfma_f16(bf16x8 a, bf16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b),
                                                   c, 0, 0, 0);
}
// x[at + j] (j = 0..7) rounded to nearest fp16, as 16-bit patterns in a bf16x8 register.
DEVI bf16x8 cvt_f16x8(const f32x16 &x, int at) {
    f16x8 h;
#pragma unroll
    for (int j = 0; j < 8; ++j) h[j] = static_cast<_Float16>(x[at + j]);
    return __builtin_bit_cast(bf16x8, h);
}

// The rounding error that cvt_f16x8(x, at) leaves, x[at + j] - hi[j], itself rounded to fp16:
// hi + lo carries x to about 2^-22 of its magnitude.
DEVI bf16x8 cvt_f16x8_lo(const f32x16 &x, int at, bf16x8 hi) {
    const f16x8 h = __builtin_bit_cast(f16x8, hi);
    f16x8 l;
#pragma unroll
    for (int j = 0; j < 8; ++j) l[j] = static_cast<_Float16>(x[at + j] - static_cast<float>(h[j]));
    return __builtin_bit_cast(bf16x8, l);
}
// True in every lane when any lane's x[at .. at + 7] exceeds `t` (one wave-wide vote).
DEVI bool any_above(const f32x16 &x, int at, float t) {
    float m = x[at];
#pragma unroll
    for (int j = 1; j < 8; ++j) m = fmaxf(m, x[at + j]);
    return __builtin_amdgcn_ballot_w64(m > t) != 0;
}
// The same for values known to be +0 or positive (t too): their bit patterns order as unsigned
// integers, so the maximum takes integer max3 operations and no NaN canonicalization.  (The
// elements are read as values: __builtin_bit_cast of an ext-vector element reads element 0 with
// this compiler.)
DEVI bool any_above_nonneg(const f32x16 &x, int at, float t) {
    uint32_t m = __float_as_uint(x[at]);
#pragma unroll
    for (int j = 1; j < 8; ++j) m = max(m, __float_as_uint(x[at + j]));
    return __builtin_amdgcn_ballot_w64(m > __float_as_uint(t)) != 0;
}

// fp16 of x[at + j] * m and of x[at + j] * y[at + j]: one mixed-precision multiply with an
// fp16 result (v_fma_mix) per element, rounded once.
DEVI bf16x8 cvt_f16x8_mul(const f32x16 &x, int at, float m) {
    f16x8 h;
#pragma unroll
    for (int j = 0; j < 8; ++j) h[j] = static_cast<_Float16>(x[at + j] * m);
    return __builtin_bit_cast(bf16x8, h);
}
DEVI bf16x8 cvt_f16x8_prod(const f32x16 &x, const f32x16 &y, int at) {
    f16x8 h;
#pragma unroll
    for (int j = 0; j < 8; ++j) h[j] = static_cast<_Float16>(x[at + j] * y[at + j]);
    return __builtin_bit_cast(bf16x8, h);
}
// Their rounding errors, x m - hi and x y - hi (the products in float32), rounded to fp16.
DEVI bf16x8 cvt_f16x8_mul_lo(const f32x16 &x, int at, float m, bf16x8 hi) {
    const f16x8 h = __builtin_bit_cast(f16x8, hi);
    f16x8 l;
#pragma unroll
    for (int j = 0; j < 8; ++j) l[j] = static_cast<_Float16>(x[at + j] * m - static_cast<float>(h[j]));
    return __builtin_bit_cast(bf16x8, l);
}
DEVI bf16x8 cvt_f16x8_prod_lo(const f32x16 &x, const f32x16 &y, int at, bf16x8 hi) {
    const f16x8 h = __builtin_bit_cast(f16x8, hi);
    f16x8 l;
#pragma unroll
    for (int j = 0; j < 8; ++j) l[j] = static_cast<_Float16>(x[at + j] * y[at + j] - static_cast<float>(h[j]));
    return __builtin_bit_cast(bf16x8, l);
}

// Row index (within a 32-row MFMA tile) that accumulator register r of this lane holds.
DEVI int acc_row(int r, int g) { return 8 * (r >> 2) + 4 * g + (r & 3); }

// v_exp_f32 / v_log_f32: base-2, about 1 ulp.
DEVI float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }
DEVI float log2_fast(float x) { return __builtin_amdgcn_logf(x); }

// Combine a value with the one held by lane l ^ 32 (the other half of the wave) through
// v_permlane32_swap (no LDS): the pair it returns holds, in every lane, the values of lanes
// l % 32 and l % 32 + 32, in the same order in both halves, so both halves get bit-identical
// results.
DEVI float xor32_max(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
DEVI float xor32_add(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

DEVI float bf16_to_f32(__bf16 x) { return static_cast<float>(x); }
DEVI __bf16 f32_to_bf16(float x) { return static_cast<__bf16>(x); }  // round to nearest even

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Two float32 values rounded to nearest bf16, packed low/high (one v_cvt_pk_bf16_f32).
DEVI uint32_t cvt_pk_bf16(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){a, b}, bf16x2));
}

// x[at + j] (j = 0..7) as hi + lo with hi = bf16(x) and lo = bf16(x - hi), converted in pairs:
// 6 VALU operations per pair (two packed conversions, two unpacks, two subtractions).
DEVI void split_bf16(const f32x16 &x, int at, bf16x8 &hi, bf16x8 &lo) {
    u32x4 h, l;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        const float x0 = x[at + 2 * w], x1 = x[at + 2 * w + 1];
        h[w] = cvt_pk_bf16(x0, x1);
        l[w] = cvt_pk_bf16(x0 - __uint_as_float(h[w] << 16), x1 - __uint_as_float(h[w] & 0xffff0000u));
    }
    hi = __builtin_bit_cast(bf16x8, h);
    lo = __builtin_bit_cast(bf16x8, l);
}

template <typename T> DEVI float to_f32(T x);
template <> DEVI float to_f32<float>(float x) { return x; }
template <> DEVI float to_f32<__bf16>(__bf16 x) { return static_cast<float>(x); }
template <typename T> DEVI T from_f32(float x);
template <> DEVI float from_f32<float>(float x) { return x; }
template <> DEVI __bf16 from_f32<__bf16>(float x) { return static_cast<__bf16>(x); }

// One global_load_lds_dwordx4: lane i's 16 bytes at `src` land at LDS `dst` + 16 i (`dst` is
// wave-uniform; lanes switched off by EXEC write nothing).  Written as inline assembly so that
// the compiler's wait-count pass does not treat the transfer as aliasing every later LDS read,
// which would make each tile wait for the next tile's loads; the caller waits (vmcnt(0) +
// barrier) before reading a filled buffer.
//
// The instruction takes its LDS address from m0, a register the compiler reserves (and may hold
// live values in).  So the assembly saves m0 into an SGPR of its own, sets it, and restores it
// after the load has issued (m0 is read at issue): the compiler's view of m0 is never changed,
// and m0 need not be declared clobbered.  GFX9 parts need one wait state between an SALU write
// of m0 and an LDS-DMA instruction that reads it (the s_nop).
DEVI void lds_dma16(const void *src, void *dst) {
    const uint32_t base = __builtin_amdgcn_readfirstlane(
        (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void *)dst);
    uint32_t saved;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\ts_nop 0\n\t"
                 "global_load_lds_dwordx4 %2, off\n\ts_mov_b32 m0, %0"
                 : "=&s"(saved)
                 : "s"(base), "v"(src)
                 : "memory");
}

// The same transfer addressed as a wave-uniform 64-bit base (held in SGPRs) plus a per-lane
// 32-bit byte offset (the saddr form of the instruction), so a caller whose lane offsets do not
// change between transfers spends no VALU on addresses.
DEVI void lds_dma16_off(const void *base, uint32_t off, void *dst) {
    // readfirstlane returns int: each half goes back to uint32_t before widening, or a low
    // half with bit 31 set would sign-extend over the high half.
    const uint64_t p = (uint64_t)(uintptr_t)base;
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)p);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(p >> 32));
    const uint64_t sbase = ((uint64_t)hi << 32) | lo;
    const uint32_t m = __builtin_amdgcn_readfirstlane(
        (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void *)dst);
    uint32_t saved;  // m0 saved and restored as in lds_dma16
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\ts_nop 0\n\t"
                 "global_load_lds_dwordx4 %2, %3\n\ts_mov_b32 m0, %0"
                 : "=&s"(saved)
                 : "s"(m), "v"(off), "s"(sbase)
                 : "memory");
}

// A wave-uniform global address as an SGPR pair (each half read from the first lane).
DEVI uint64_t sgpr_addr(const void *p) {
    const uint64_t x = (uint64_t)(uintptr_t)p;
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)x);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(x >> 32));
    return ((uint64_t)hi << 32) | lo;
}

// The LDS byte address of a pointer into LDS: cast once and reused, it spares each transfer the
// null test of a generic-to-LDS conversion.
DEVI uint32_t lds_addr(const void *p) {
    return __builtin_amdgcn_readfirstlane(
        (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const void *)p);
}

// Two saddr-form transfers (global base g + lane offset off, into LDS address l) in one statement,
// m0 saved before the first and restored after the second: three SALU instructions per transfer
// instead of lds_dma16_off's seven.
DEVI void lds_dma16_pair(uint64_t g0, uint32_t off0, uint32_t l0, uint64_t g1, uint32_t off1, uint32_t l1) {
    l0 = __builtin_amdgcn_readfirstlane(l0), l1 = __builtin_amdgcn_readfirstlane(l1);
    uint32_t saved;
    asm volatile("s_mov_b32 %0, m0\n\t"
                 "s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %2, %3\n\t"
                 "s_mov_b32 m0, %4\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %5, %6\n\t"
                 "s_mov_b32 m0, %0"
                 : "=&s"(saved)
                 : "s"(l0), "v"(off0), "s"(g0), "s"(l1), "v"(off1), "s"(g1)
                 : "memory");
}

// A global load marked nontemporal (global_load ... nt): for data a kernel streams once.  On one
// MI355X a read of 4 GiB in 16-byte loads ran at 7.1 TB/s this way against 6.3 TB/s without.
template <typename V>
DEVI V load_nt(const V *p) { return __builtin_nontemporal_load(p); }

// s_waitcnt vmcnt(0): every global load of this wave (including lds_dma16 transfers) is done.
DEVI void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0f70); }

// s_waitcnt vmcnt(N): all but the N most recently issued global loads of this wave are done
// (they complete in issue order).  N < 64: its low four bits go in [3:0], the rest in [15:14].
template <int N>
DEVI void wait_vmem_but() {
    static_assert(N >= 0 && N < 64, "vmcnt holds 6 bits");
    __builtin_amdgcn_s_waitcnt(0x0f70 | (N & 15) | ((N >> 4) << 14));
}

// s_waitcnt lgkmcnt(0): every LDS read of this wave has returned its data.
DEVI void wait_lds() { __builtin_amdgcn_s_waitcnt(0xc07f); }

// Scheduling hint for a straight run of NMFMA MFMAs, each consuming R LDS reads issued in the
// same block: the reads are kept AHEAD MFMAs in front of their use (the compiler otherwise
// issues each read just before its MFMA and exposes the LDS latency on every one).
template <int NMFMA, int R, int AHEAD>
DEVI void sched_reads_ahead() {
    __builtin_amdgcn_sched_group_barrier(0x100, R * AHEAD, 0);  // DS reads
#pragma unroll
    for (int i = 0; i < NMFMA - AHEAD; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);      // MFMA
        __builtin_amdgcn_sched_group_barrier(0x100, R, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, AHEAD, 0);
}

// The schedule a launcher chose (dc_sdpa_schedule of dc_attn.h).  While g_schedule is set on a
// thread, launchers record their choices there and launch() starts nothing (a dry run: the
// schedule query runs the very code that decides a launch).
struct Schedule {
    int split_chunk = 0, split_pieces = 1;  // forward split key ranges
    int streamk_ranges = 0;                 // float32 backward
    int split_chunk_k = 0, split_chunk_q = 0;  // bf16 backward split grids
    int f16_products = 0;                   // bf16 products on the fp16 copies
    int deterministic = 1;                  // backward results identical from run to run
    int materialized_rows = 0;              // head dims above 128: rows per block (wide.hip)
    int64_t workgroups = 0;                 // workgroups of the launches, summed
    int chunks = 1;                         // float32 backward: launch sequences (abi.hip)
};
inline thread_local Schedule *g_schedule = nullptr;

// Launches `kernel` and returns the status of this launch alone (hipGetLastError would also
// report errors left behind by unrelated earlier calls in the process).
template <typename... Params, typename... Args>
inline hipError_t launch(void (*kernel)(Params...), dim3 grid, dim3 block, hipStream_t stream,
                         Args... args) {
    static_assert(sizeof...(Params) == sizeof...(Args), "argument count");
    if (g_schedule) {
        g_schedule->workgroups += (int64_t)grid.x * grid.y * grid.z;
        return hipSuccess;
    }
    void *ptrs[] = {static_cast<void *>(&args)...};
    return hipLaunchKernel(reinterpret_cast<const void *>(kernel), grid, block, ptrs, 0, stream);
}
// Records a choice of the launcher when a dry run asks for it.
#define record_schedule(field, value)                  \
    do {                                               \
        if (::dc::g_schedule) ::dc::g_schedule->field = (value); \
    } while (0)

#define return_if(expr)                      \
    do {                                     \
        const hipError_t err_ = (expr);      \
        if (err_ != hipSuccess) return err_; \
    } while (0)

}  // namespace dc
