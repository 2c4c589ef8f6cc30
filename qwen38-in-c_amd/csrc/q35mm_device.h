// q35mm_device.h -- gfx950 device helpers shared by the q35mm kernels.
//
// Resident weight layout ("lane-order tiles").  A weight of R rows and C
// columns is zero-padded to NB*128 rows and KB*128 columns and stored as
//
//   offset(nb, kb, sub, j, lane, e) =
//       ((((nb * KB + kb) * 4 + sub) * 4 + j) * 64 + lane) * 16 + e
//   row = nb*128 + sub*32 + (lane % 32)
//   col = kb*128 + j*32 + (lane / 32)*16 + e          (e < 16)
//
// i.e. one 128x128 block is 16 KiB contiguous, made of four 32-row
// sub-tiles of 4 KiB, each made of four 1 KiB "chunks" of 32 columns.  A
// chunk is exactly what one wavefront loads with one 16-byte load per lane,
// and lane l receives 16 consecutive codes of row (l % 32): the B operand of
// two v_mfma_f32_32x32x16_bf16 (bytes 0-7 -> first MFMA, 8-15 -> second).
//
// MFMA 32x32x16 bf16 operand layout (per lane l of the wavefront):
//   A: 8 bf16, row m = l % 32, k-slot = 8*(l/32) + i
//   B: 8 bf16, col n = l % 32, k-slot = 8*(l/32) + i
//   D: 16 fp32, col n = l % 32, reg r -> row 8*(r/4) + 4*(l/32) + (r%4)
// For chunk j the k-slots of the first MFMA map to columns j*32 + 16h + i
// and those of the second to j*32 + 16h + 8 + i, h = l/32; activations are
// laid out with the same mapping so A and B pair the same column.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "q35mm_internal.h"

namespace q35mm {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t f32_bits(float f) { return __builtin_bit_cast(uint32_t, f); }
__device__ __forceinline__ float bits_f32(uint32_t u) { return __builtin_bit_cast(float, u); }

// Two e4m3fn codes (bytes 0,1 of w if HI is false, bytes 2,3 if true) to
// two fp32.  gfx950 decodes the OCP e4m3fn format; every finite code is
// exact in fp32, 0x7F / 0xFF decode to NaN.
template <bool HI>
__device__ __forceinline__ f32x2_t e4m3x2_to_f32(uint32_t w) {
    return __builtin_amdgcn_cvt_pk_f32_fp8(w, HI);
}

// Four e4m3 codes -> four bf16 packed in two dwords (element 0 in the low
// half of the first dword).  Every finite e4m3 value has at most 4
// significant bits and an exponent within bf16 range, so truncating the
// exact fp32 to its top 16 bits is exact.
__device__ __forceinline__ u32x2_t e4m3x4_to_bf16x4(uint32_t w) {
    f32x2_t lo = e4m3x2_to_f32<false>(w);
    f32x2_t hi = e4m3x2_to_f32<true>(w);
    u32x2_t r;
    // v_perm_b32: selector bytes 0-3 pick from the second source, 4-7 from
    // the first; 0x07060302 keeps the upper halves of (src1, src0).
    r.x = __builtin_amdgcn_perm(f32_bits(lo.y), f32_bits(lo.x), 0x07060302u);
    r.y = __builtin_amdgcn_perm(f32_bits(hi.y), f32_bits(hi.x), 0x07060302u);
    return r;
}

// Eight e4m3 codes (two dwords) -> bf16x8 MFMA operand.
__device__ __forceinline__ bf16x8_t e4m3x8_to_bf16x8(uint32_t w0, uint32_t w1) {
    u32x2_t a = e4m3x4_to_bf16x4(w0);
    u32x2_t b = e4m3x4_to_bf16x4(w1);
    u32x4_t v = {a.x, a.y, b.x, b.y};
    return __builtin_bit_cast(bf16x8_t, v);
}

// Eight e4m3 codes -> bf16x8 with gfx950's v_cvt_scalef32_pk_bf16_fp8 (two
// codes per instruction; half the VALU of the path above).  The instruction
// scales by 2^exponent(scale) only (E8M0 semantics: 1.5 acts as 1, 0 as
// 2^-127).  With scale 1.0 every finite e4m3 value is exact in bf16, so the
// result equals the one above (checked for all 256 codes); 0x7F / 0xFF give
// NaN.
__device__ __forceinline__ bf16x8_t e4m3x8_to_bf16x8_cvt(uint32_t w0, uint32_t w1, float pow2_scale) {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    const bf16x2_t a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, pow2_scale, false);
    const bf16x2_t b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, pow2_scale, true);
    const bf16x2_t c = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, pow2_scale, false);
    const bf16x2_t d = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, pow2_scale, true);
    const u32x4_t v = {__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b),
                       __builtin_bit_cast(uint32_t, c), __builtin_bit_cast(uint32_t, d)};
    return __builtin_bit_cast(bf16x8_t, v);
}

// fp32 -> bf16 bits, round to nearest even (finite inputs).
__device__ __forceinline__ uint32_t f32_to_bf16_rne(float f) {
    uint32_t u = f32_bits(f);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return u >> 16;
}

__device__ __forceinline__ float bf16_to_f32(uint32_t b) { return bits_f32(b << 16); }

// Exact three-way split of an fp32 into bf16 parts: x == p0 + p1 + p2 for
// every normal x (each residual is exact in fp32 and has at most 16, then 8,
// significant bits).
__device__ __forceinline__ void split3_bf16(float x, uint32_t &p0, uint32_t &p1, uint32_t &p2) {
    p0 = f32_to_bf16_rne(x);
    float r1 = x - bf16_to_f32(p0);
    p1 = f32_to_bf16_rne(r1);
    float r2 = r1 - bf16_to_f32(p1);
    p2 = f32_to_bf16_rne(r2);
}

__device__ __forceinline__ f32x16_t mfma32x32x16(bf16x8_t a, bf16x8_t b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

}  // namespace q35mm
