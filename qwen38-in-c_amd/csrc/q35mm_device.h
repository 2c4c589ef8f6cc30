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

// Eight e4m3 codes (two dwords) -> bf16x8 MFMA operand with gfx950's
// v_cvt_scalef32_pk_bf16_fp8 (two codes per instruction).  The instruction
// scales by 2^exponent(scale) only (E8M0 semantics: 1.5 acts as 1, 0 as
// 2^-127).  Every finite e4m3 value has at most 4 significant bits and an
// exponent within bf16 range, so at scale 1.0 the conversion is exact
// (decode_bf16_kernel exposes it; checked for all 256 codes); 0x7F / 0xFF
// give NaN.
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

typedef __bf16 bf16x2v_t __attribute__((ext_vector_type(2)));
typedef float f32x2v_t __attribute__((ext_vector_type(2)));

// Two fp32 -> packed bf16 (a in the low half), round to nearest even: one
// v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t f32x2_to_bf16x2_rne(float a, float b) {
    const f32x2v_t v = {a, b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2v_t));
}

__device__ __forceinline__ float bf16_to_f32(uint32_t b) { return bits_f32(b << 16); }

// An activation about to be rounded to bf16 for the prefill GEMM: finite
// values beyond bf16's range saturate to its largest finite value instead of
// rounding to infinity (the reference's fp32 products of such x stay
// finite); infinities and NaN pass unchanged.
__device__ __forceinline__ float bf16_saturate(float v) {
    return __builtin_fabsf(v) < __builtin_inff() ? __builtin_fminf(__builtin_fmaxf(v, -0x1.FEp127f), 0x1.FEp127f)
                                                 : v;
}

// Exact three-way split of two fp32 values into bf16 parts, packed in pairs:
// x == p0 + p1 + p2 for every normal x (each residual is exact in fp32 and has
// at most 16, then 8, significant bits).  Each part is a round-to-nearest-even
// conversion; about 5.5 instructions per value.  Blocks holding wide values
// or infinities are shifted first and fixed up by split3_fix_inf (below).
__device__ __forceinline__ void split3_bf16x2(float a, float b, uint32_t &p0, uint32_t &p1, uint32_t &p2) {
#pragma clang fp contract(off)
    const f32x2v_t x = {a, b};
    const bf16x2v_t b0 = __builtin_convertvector(x, bf16x2v_t);
    const f32x2v_t r1 = x - __builtin_convertvector(b0, f32x2v_t);
    const bf16x2v_t b1 = __builtin_convertvector(r1, bf16x2v_t);
    const f32x2v_t r2 = r1 - __builtin_convertvector(b1, f32x2v_t);
    p0 = __builtin_bit_cast(uint32_t, b0);
    p1 = __builtin_bit_cast(uint32_t, b1);
    p2 = __builtin_bit_cast(uint32_t, __builtin_convertvector(r2, bf16x2v_t));
}

// Wide activations.  A K block's raw partial sum_k x_k * code_k (codes up
// to +-448, 128 terms) can overflow fp32 once |x| reaches ~2^112, where the
// reference's products (code * scale) * x stay finite.  A block (row-split
// GEMV) or a workgroup's range (stream-K) holding a value of magnitude
// kActWide or more is therefore staged multiplied by kActShift, and its
// block scales are taken multiplied by kActUnshift: both factors are powers
// of two, so fmaf(scale * 2^64, part * 2^-64, acc) rounds exactly as
// fmaf(scale, part, acc) would, and the bits are those of the plain path
// (values below 2^-62 in magnitude in such a block lose bits as subnormals).
// NaN is ignored by the test (every part of a NaN is NaN, and the output is
// NaN as the reference's fmaf chain gives it).
constexpr float kActWide = 0x1.0p96f;
constexpr float kActShift = 0x1.0p-64f;
constexpr float kActUnshift = 0x1.0p64f;

// After split3_bf16x2 of two values of a shifted block (finite values are
// below 2^64 there and split exactly): an infinity passes whole in part 0
// with zero residuals, so inf * w gives +-inf (NaN for w = 0), as
// fmaf(w, x, acc) does (qwen35-c/src/q35_mm.c:110-111) -- the plain split
// forms inf - inf = NaN in the residuals.  In a shifted block part 0 is a
// bf16 infinity exactly when the value is one, so the test reads part 0.
__device__ __forceinline__ void split3_fix_inf(uint32_t p0, uint32_t &p1, uint32_t &p2) {
    const uint32_t keep = ((p0 & 0x7FFFu) == 0x7F80u ? 0xFFFF0000u : 0xFFFFFFFFu) &
                          ((p0 & 0x7FFF0000u) == 0x7F800000u ? 0x0000FFFFu : 0xFFFFFFFFu);
    p1 &= keep;
    p2 &= keep;
}

// Largest |x| of n values (NaN ignored): v_max3_f32 with abs modifiers.
template <uint32_t N>
__device__ __forceinline__ float max_abs(const float (&v)[N]) {
    float mx = 0.0f;
#pragma unroll
    for (uint32_t e = 0; e < N; e++) mx = __builtin_fmaxf(mx, __builtin_fabsf(v[e]));
    return mx;
}

__device__ __forceinline__ f32x16_t mfma32x32x16(bf16x8_t a, bf16x8_t b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// ---- MLP neighbours, one element (qwen35-c/src/q35_kern.c) ----------------
// Each operation rounds on its own (no contraction), as the reference's
// q35_kern.c is compiled; division and square root are correctly rounded.

// exp evaluated in double precision and rounded once to float.
__device__ __forceinline__ float exp_rounded_once(float v) { return (float)exp((double)v); }

// silu(g) * u as (g * (1 / (1 + exp(-g)))) * u  (q35_kern.c:70-73, :137-145).
__device__ __forceinline__ float swiglu1(float g, float u) {
#pragma clang fp contract(off)
    const float sig = 1.0f / (1.0f + exp_rounded_once(-g));
    const float t = g * sig;
    return t * u;
}

// (x * inv) * (1 + w)  (q35_kern.c:77-86).
__device__ __forceinline__ float rmsnorm1(float x, float inv, float w) {
#pragma clang fp contract(off)
    const float t = x * inv;
    return t * (1.0f + w);
}

// 1 / sqrtf(s / n + eps) from a lane-folded sum of squares (q35_kern.c:80-81).
__device__ __forceinline__ float rms_inverse(float s, uint32_t n, float eps) {
#pragma clang fp contract(off)
    const float mean = s / (float)n;
    return 1.0f / sqrtf(mean + eps);
}

// acc + s[0] + s[1] + ... + s[cnt-1], added one at a time in that order
// (one lane of the reference's sum of squares).  s is 16-byte aligned LDS.
// Blocks of 32 values alternate between two register sets, the reads of the
// next block issued before the adds of the current one.
__device__ __forceinline__ void add32_in_order(float &acc, const float4 (&v)[8]) {
#pragma clang fp contract(off)
#pragma unroll
    for (int k = 0; k < 8; k++) {
        acc = acc + v[k].x;
        acc = acc + v[k].y;
        acc = acc + v[k].z;
        acc = acc + v[k].w;
    }
}

__device__ __forceinline__ void read32(float4 (&v)[8], const float4 *s4, uint32_t blk) {
#pragma unroll
    for (int k = 0; k < 8; k++) v[k] = s4[blk * 8 + k];
}

__device__ __forceinline__ float lane_sum_in_order(const float *s, uint32_t cnt, float acc) {
#pragma clang fp contract(off)
    const float4 *s4 = reinterpret_cast<const float4 *>(s);
    const uint32_t n32 = cnt / 32;
    float4 a[8], b[8];
    if (n32) read32(a, s4, 0);
    uint32_t blk = 0;
    for (; blk + 2 <= n32; blk += 2) {
        read32(b, s4, blk + 1);
        __builtin_amdgcn_sched_barrier(0);
        add32_in_order(acc, a);
        read32(a, s4, min(blk + 2, n32 - 1));   // the last pass re-reads a block: unused
        __builtin_amdgcn_sched_barrier(0);
        add32_in_order(acc, b);
    }
    if (blk < n32) add32_in_order(acc, a);
    for (uint32_t t = n32 * 32; t < cnt; t++) acc = acc + s[t];
    return acc;
}

}  // namespace q35mm
