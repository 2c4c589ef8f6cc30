// gemv_rows_common.h -- activation staging shared by the row-split decode
// GEMV (gemv_rows.hip) and the chained decode launch (chain.hip): both
// stage a K block's activations with the same lane layout and the same
// exact three-part bf16 split, so a row's arithmetic, and with it its bits,
// is the same in either kernel.
#pragma once

#include "q35mm_device.h"
#include "q35mm_internal.h"

namespace q35mm {
namespace rows {

// The activations of one K block for all m tokens.  MT = m rounded up to a
// power of two (1, 2, 4, 8); lane l serves token l / L (L = 64/MT lanes per
// token) and G = 2*MT of the block's columns, so every lane does the same
// share of the split whatever m is: for G >= 4 the groups of four columns
// 4*(l % L) + 4*L*i, i < G/4, so that one 16-byte load per lane reads whole
// 128-byte lines (L lanes x 16 bytes of one token's row; lanes holding G
// consecutive columns instead made each load touch four times the lines,
// and the layer step at m = 8 ran 9% slower); for G = 2 the pair 2*l.
// Loads are unconditional (token and columns clamped), so the waits before
// each block stay static; stage_xblock masks what is not real.
template <uint32_t MT>
struct XBlock {
    static constexpr uint32_t kG = 2 * MT;          // columns per lane
    static constexpr uint32_t kLanesPerToken = 64 / MT;
    float v[kG];
};

// Block column of element e of a lane's share.
template <uint32_t MT>
__device__ __forceinline__ uint32_t xcol(uint32_t lane, uint32_t e) {
    constexpr uint32_t G = XBlock<MT>::kG, L = XBlock<MT>::kLanesPerToken;
    if constexpr (G >= 4) return 4 * (lane % L) + 4 * L * (e / 4) + (e % 4);
    return (lane % L) * G + e;
}

template <bool VEC, uint32_t MT>
__device__ __forceinline__ void load_xblock(XBlock<MT> &xb, const float *x, uint32_t ldx, uint32_t m, uint32_t k,
                                            uint32_t kb, uint32_t lane) {
    constexpr uint32_t G = XBlock<MT>::kG;
    const uint32_t t = min(lane / XBlock<MT>::kLanesPerToken, m - 1);
    const uint32_t kg = kb * kBlock;
    const float *row = x + (size_t)t * ldx;
    if constexpr (VEC) {
        // Rows 16-byte aligned and k % 8 == 0: every group of min(G, 4)
        // columns is wholly inside or wholly past the row, so clamping each
        // group on its own keeps the valid ones in place.
        if constexpr (G == 2) {
            const float2 a = *reinterpret_cast<const float2 *>(row + min(kg + xcol<MT>(lane, 0), k - 2));
            xb.v[0] = a.x; xb.v[1] = a.y;
        } else {
#pragma unroll
            for (uint32_t i = 0; i < G / 4; i++) {
                const float4 a = *reinterpret_cast<const float4 *>(row + min(kg + xcol<MT>(lane, 4 * i), k - 4));
                xb.v[4 * i] = a.x; xb.v[4 * i + 1] = a.y; xb.v[4 * i + 2] = a.z; xb.v[4 * i + 3] = a.w;
            }
        }
    } else {
#pragma unroll
        for (uint32_t e = 0; e < G; e++) xb.v[e] = row[min(kg + xcol<MT>(lane, e), k - 1)];
    }
}

// Split a block's activations into an A-operand slot of 256*R bytes:
//   byte offset(c, q, ai, h) = (((c*2 + q) * R + ai) * 2 + h) * 16
// for chunk c < 4, MFMA q < 2, A row ai = part*m + token, h = lane/32 of
// the reading lane; the 16 bytes hold block columns c*32 + 16h + 8q + 0..7.
// A lane writes its share of those 16-byte units: per part 4 bytes (G = 2)
// or 8 bytes per group of four columns.  Columns >= k are staged as zero;
// only a partial last block (a wavefront-uniform test) pays for the masks.
// Returns (the same for every lane) whether the block holds a wide value
// and was staged multiplied by kActShift: its scale is then taken times
// kActUnshift.
template <uint32_t MT>
__device__ __forceinline__ bool stage_xblock(const XBlock<MT> &xb, uint8_t *slot, uint32_t m, uint32_t R, uint32_t k,
                                             uint32_t kb, uint32_t lane) {
    constexpr uint32_t G = XBlock<MT>::kG;
    const uint32_t t = lane / XBlock<MT>::kLanesPerToken;
    float xv[G];
#pragma unroll
    for (uint32_t e = 0; e < G; e++) xv[e] = xb.v[e];
    if (kb * kBlock + kBlock > k) {
#pragma unroll
        for (uint32_t e = 0; e < G; e++) xv[e] = kb * kBlock + xcol<MT>(lane, e) < k ? xb.v[e] : 0.0f;
    }
    const bool wide = __builtin_amdgcn_ballot_w64(t < m && max_abs(xv) >= kActWide) != 0;
    if (t >= m) return wide;
    if (__builtin_expect(wide, 0)) {
#pragma unroll
        for (uint32_t e = 0; e < G; e++) xv[e] *= kActShift;
    }
    uint32_t pr[3][G / 2];   // per part, packed bf16 pairs
#pragma unroll
    for (uint32_t e = 0; e < G / 2; e++) split3_bf16x2(xv[2 * e], xv[2 * e + 1], pr[0][e], pr[1][e], pr[2][e]);
    if (__builtin_expect(wide, 0)) {
#pragma unroll
        for (uint32_t e = 0; e < G / 2; e++) split3_fix_inf(pr[0][e], pr[1][e], pr[2][e]);
    }
#pragma unroll
    for (uint32_t part = 0; part < 3; part++) {
        const uint32_t ai = part * m + t;
#pragma unroll
        for (uint32_t i = 0; i < (G + 3) / 4; i++) {   // groups of four columns (one pair for G = 2)
            const uint32_t col = xcol<MT>(lane, 4 * i);
            const uint32_t c = col >> 5, h = (col >> 4) & 1, q = (col >> 3) & 1, e0 = col & 7;
            uint8_t *dst = slot + (((c * 2 + q) * R + ai) * 2 + h) * 16 + e0 * 2;
            if constexpr (G == 2)
                *reinterpret_cast<uint32_t *>(dst) = pr[part][0];
            else
                *reinterpret_cast<u32x2_t *>(dst) = u32x2_t{pr[part][2 * i], pr[part][2 * i + 1]};
        }
    }
    return wide;
}

}  // namespace rows
}  // namespace q35mm
