// Chunk-major bf16 LDS tiles shared by the bfloat16 forward and backward kernels.
//
// A tile of R rows x D bf16 is stored as D/8 chunk columns of 16 bytes: chunk c of row r sits
// at slot c * (R + 4) + r (4 pad slots per column).  A row read (lanes = 32 consecutive rows,
// one chunk) is 512 contiguous bytes, and a transposed read (8 rows x 4 chunks x 8 bytes) hits
// every bank exactly twice; all inner-loop addresses are a per-lane base plus a constant.
#pragma once

#include "common.hpp"

namespace dc {
namespace {

typedef short s16x4 __attribute__((ext_vector_type(4)));

template <int R, int D>
struct CMTile {
    static_assert(R % 64 == 0, "tiles are filled 64 rows at a time");
    static constexpr int C = D / 8;        // 16-byte chunks per row
    static constexpr int P = R + 4;        // slots per chunk column (4 pad slots)
    static constexpr int SLOTS = C * P;
    static constexpr int RB = R / 64;      // 64-row blocks
    static constexpr int NT = C * RB;      // wave-wide transfers per tile
    static constexpr int CS = P * 16;      // chunk column stride, bytes
};

// Fills a chunk-major tile with rows [0, nrows) of `src` (row stride E elements); rows past
// nrows and dims past E are zero, pad slots are not written.  Transfer i of the tile (dealt to
// the W waves round-robin) moves chunk i / RB of rows 64 (i % RB) + l, l = lane; so with VEC
// (E == D, 16-byte aligned rows) each transfer of a full tile is one global_load_lds_dwordx4
// with a wave-uniform base and the same per-lane offset (l * D * 2 bytes) every time: no
// per-tile address arithmetic in VGPRs and no per-lane bounds tests.
template <int R, int D, bool VEC, int W>
DEVI void fill_cm(u32x4 *dst, const __bf16 *src, int nrows, int E, int wave, int lane) {
    using T = CMTile<R, D>;
    constexpr int count = (T::NT + W - 1) / W;
    const uint32_t loff = (uint32_t)lane * (D * 2);
    if (VEC && nrows >= R) {
#pragma unroll
        for (int j = 0; j < count; ++j) {
            const int inst = wave + W * j;
            if (T::NT % W != 0 && inst >= T::NT) break;  // wave-uniform
            const int c = inst / T::RB, rb = inst % T::RB;
            lds_dma16_off(src + (int64_t)(64 * rb) * D + 8 * c, loff, dst + c * T::P + 64 * rb);
        }
        return;
    }
#pragma unroll
    for (int j = 0; j < count; ++j) {
        const int inst = wave + W * j;
        if (T::NT % W != 0 && inst >= T::NT) break;
        const int c = inst / T::RB, rb = inst % T::RB, row = 64 * rb + lane;
        u32x4 *d = dst + c * T::P + 64 * rb;
        if (VEC) {
            if (row < nrows)
                lds_dma16_off(src + (int64_t)(64 * rb) * D + 8 * c, loff, d);
            else
                d[lane] = u32x4{0u, 0u, 0u, 0u};
        } else {
            uint16_t h[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int dd = 8 * c + e;
                h[e] = (row < nrows && dd < E) ? __builtin_bit_cast(uint16_t, src[(int64_t)row * E + dd])
                                               : (uint16_t)0;
            }
            u32x4 x;
#pragma unroll
            for (int w = 0; w < 4; ++w) x[w] = (uint32_t)h[2 * w] | ((uint32_t)h[2 * w + 1] << 16);
            d[lane] = x;
        }
    }
}

// Row fragment (MFMA operand with rows on lanes): rows row0 + (l % 32), dims 16 st + 8 (l / 32)
// + 0..7.  `lanebase` = (l % 32) * 16 + (l / 32) * CS.
template <int R, int D>
DEVI bf16x8 row_frag(const u32x4 *tile, uint32_t lanebase, int row0, int st) {
    using T = CMTile<R, D>;
    const char *p = reinterpret_cast<const char *>(tile) + lanebase + row0 * 16 + 2 * st * T::CS;
    return *reinterpret_cast<const bf16x8 *>(p);
}

// Transposed fragment (MFMA operand with dims on lanes): dim 32 dt + (l % 32), rows
// row0 + {4g..4g+3, 8+4g..8+4g+3} (g = l / 32), read by two ds_read_b64_tr_b16.  Within each
// 16-lane group that instruction hands lane j element j % 4 of the 8 bytes read by lanes
// j / 4, 4 + j / 4, 8 + j / 4 and 12 + j / 4, so lane m of a group reads row 4g + m / 4 at
// dims 4 (m % 4) + 0..3 of the group's 16.
// `lanebase` = (4g + (i >> 2)) * 16 + 8 (i & 1) + (2 half + ((i & 3) >> 1)) * CS, i = l % 16,
// half = (l / 16) % 2.
template <int R, int D>
DEVI bf16x8 tr_frag(const u32x4 *tile, uint32_t lanebase, int row0, int dt) {
    using T = CMTile<R, D>;
    const char *p = reinterpret_cast<const char *>(tile) + lanebase + row0 * 16 + 4 * dt * T::CS;
    const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4 *)(p));
    const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) s16x4 *)(p + 8 * 16));
    const s16x4 cat[2] = {lo, hi};
    return __builtin_bit_cast(bf16x8, cat);
}

template <int R, int D>
DEVI uint32_t row_lanebase(int lane) {
    return (uint32_t)((lane & 31) * 16 + (lane >> 5) * CMTile<R, D>::CS);
}
template <int R, int D>
DEVI uint32_t tr_lanebase(int lane) {
    const int i = lane & 15, half = (lane >> 4) & 1, g = lane >> 5;
    return (uint32_t)((4 * g + (i >> 2)) * 16 + 8 * (i & 1) + (2 * half + ((i & 3) >> 1)) * CMTile<R, D>::CS);
}

// Logical block index: blocks are dealt to the 8 XCDs round-robin, so consecutive logical
// indices are spread to land on the same XCD (whose L2 then holds their shared K/V or Q/dO).
DEVI int logical_block() {
    const int n = gridDim.x, w = blockIdx.x;
    return (n & 7) == 0 ? (w & 7) * (n >> 3) + (w >> 3) : w;
}

}  // namespace
}  // namespace dc
