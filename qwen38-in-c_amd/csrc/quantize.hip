// quantize.hip -- load-time FP8 quantizer on the device: 128x128 blocks,
// scale = amax / 448 rounded to bf16, codes = nearest e4m3 of w / scale.
//
// Replaces the loader's quantization of the BF16 DeltaNet in_proj_a/b
// weights (qwen35-c/src/q35_model.c:302-350, bind_ab) and its encoder
// (:31-57, f32_bf16 and the exhaustive nearest-code search f32_e4m3), so a
// BF16 checkpoint tensor goes from the file to resident FP8 without a host
// pass.  Results are the reference's, code for code:
//  - amax ignores NaN (the reference keeps the running max only when a
//    value compares greater), and the max of the rest is order-independent;
//  - scale = amax / 448 (correctly rounded fp32 divide), rounded to bf16 by
//    the reference's bit formula u + 0x7FFF + ((u >> 16) & 1);
//  - a block whose bf16 scale is 0 keeps all-zero codes;
//  - code = nearest e4m3 magnitude of |w / scale| over the 127 finite codes,
//    an exact tie going to the even code, sign from w < 0, NaN -> 0x7F.
// The search's distances |a - m| are rounded to fp32; for a below 2^20 the
// two candidates around a are within a factor of two of a, so their
// distances are exact and farther ones differ by at least one code step:
// the search is then round-to-nearest-even on the e4m3 grid, saturating at
// 448, which is computed directly.  Larger a (only reachable through
// infinities) runs the search itself.
#include "q35mm_device.h"
#include "q35mm_internal.h"

namespace q35mm {

namespace {

constexpr uint32_t kQuantThreads = 256;

__device__ __forceinline__ float e4m3_magnitude(uint32_t i) {
    const uint32_t e = i >> 3, m = i & 7;
    return e == 0 ? (float)m * 0.001953125f : ldexpf(1.0f + (float)m * 0.125f, (int)e - 7);
}

__device__ __forceinline__ uint32_t e4m3_nearest(float v) {
    if (v != v) return 0x7Fu;
    const float a = fabsf(v);
    const uint32_t sign = v < 0.0f ? 0x80u : 0u;
    uint32_t idx;
    if (a < 1048576.0f) {
        if (a >= 448.0f) {
            idx = 126;
        } else if (a < 0.015625f) {                   // below 2^-6: step 2^-9
            idx = (uint32_t)rintf(a * 512.0f);        // 0 .. 8
        } else {
            const int e = (int)((f32_bits(a) >> 23) & 255u) - 127;   // -6 .. 8
            const float r = rintf(ldexpf(a, 3 - e));                 // 8 .. 16, ties to even
            idx = (uint32_t)((e + 7) * 8) + (uint32_t)r - 8u;
            idx = idx > 126u ? 126u : idx;
        }
    } else {
        float best_d = 1e30f;
        idx = 0;
        for (uint32_t i = 0; i < 127; i++) {
            const float d = fabsf(a - e4m3_magnitude(i));
            if (d < best_d || (d == best_d && !(i & 1u) && (idx & 1u))) {
                best_d = d;
                idx = i;
            }
        }
    }
    return sign | idx;
}

__device__ __forceinline__ float load_w(const float *w, size_t i) { return w[i]; }
__device__ __forceinline__ float load_w(const uint16_t *w, size_t i) { return bits_f32((uint32_t)w[i] << 16); }

}  // namespace

// One workgroup per 128x128 block (partial at the edges).  Thread t covers
// column c0 + (t & 127) of rows r0 + (t >> 7) + 2k: each row is read and
// written contiguously.
template <typename T>
__global__ __launch_bounds__(kQuantThreads) void quantize_kernel(const T *__restrict__ w, uint32_t rows,
                                                                 uint32_t cols, uint32_t kb_total,
                                                                 uint8_t *__restrict__ codes,
                                                                 uint16_t *__restrict__ scale_bf16,
                                                                 float *__restrict__ scale_f32) {
    __shared__ float s_max[kQuantThreads / 64];
    const uint32_t bi = blockIdx.x / kb_total, bj = blockIdx.x - bi * kb_total;
    const uint32_t r0 = bi * kBlock, c = bj * kBlock + (threadIdx.x & 127);
    const uint32_t r1 = min(r0 + kBlock, rows);
    const bool col_ok = c < cols;

    float m = 0.0f;
    for (uint32_t r = r0 + (threadIdx.x >> 7); r < r1; r += 2) {
        const float a = col_ok ? fabsf(load_w(w, (size_t)r * cols + c)) : 0.0f;
        m = a > m ? a : m;   // NaN never replaces the running max
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const float o = __shfl_xor(m, off);
        m = o > m ? o : m;
    }
    if ((threadIdx.x & 63) == 0) s_max[threadIdx.x >> 6] = m;
    __syncthreads();
    float amax = s_max[0];
#pragma unroll
    for (uint32_t i = 1; i < kQuantThreads / 64; i++) amax = s_max[i] > amax ? s_max[i] : amax;

    const float raw = amax / 448.0f;
    uint32_t u = f32_bits(raw);
    u += 0x7FFFu + ((u >> 16) & 1u);
    const uint32_t sb = u >> 16;
    const float s = bits_f32(sb << 16);
    if (threadIdx.x == 0) {
        if (scale_bf16) scale_bf16[blockIdx.x] = (uint16_t)sb;
        if (scale_f32) scale_f32[blockIdx.x] = s;
    }
    if (!col_ok) return;
    for (uint32_t r = r0 + (threadIdx.x >> 7); r < r1; r += 2) {
        const size_t i = (size_t)r * cols + c;
        codes[i] = s == 0.0f ? (uint8_t)0 : (uint8_t)e4m3_nearest(load_w(w, i) / s);
    }
}

template <typename T>
static hipError_t launch_quantize_t(const T *w, uint32_t rows, uint32_t cols, uint8_t *codes, uint16_t *scale_bf16,
                                    float *scale_f32, hipStream_t stream) {
    if (rows == 0 || cols == 0) return hipSuccess;
    const uint32_t nb = (rows + kBlock - 1) / kBlock, kb = (cols + kBlock - 1) / kBlock;
    hipLaunchKernelGGL(quantize_kernel<T>, dim3(nb * kb), dim3(kQuantThreads), 0, stream, w, rows, cols, kb, codes,
                       scale_bf16, scale_f32);
    return hipGetLastError();
}

hipError_t launch_quantize_f32(const float *w, uint32_t rows, uint32_t cols, uint8_t *codes, uint16_t *scale_bf16,
                               float *scale_f32, hipStream_t stream) {
    return launch_quantize_t(w, rows, cols, codes, scale_bf16, scale_f32, stream);
}

hipError_t launch_quantize_bf16(const uint16_t *w, uint32_t rows, uint32_t cols, uint8_t *codes,
                                uint16_t *scale_bf16, float *scale_f32, hipStream_t stream) {
    return launch_quantize_t(w, rows, cols, codes, scale_bf16, scale_f32, stream);
}

}  // namespace q35mm
