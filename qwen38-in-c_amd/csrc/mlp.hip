// mlp.hip -- the device-resident neighbours of the FP8 matmuls in one MLP
// block: the zero-centred RMSNorm before gate/up, SwiGLU between gate/up and
// down, and the residual add after down.
//
// Replaces qwen35-c/src/q35_kern.c:26-48,77-108 (sumsq_fixed,
// q35_kern_rmsnorm), :70-73,137-166 (sigmoidf_, q35_kern_swiglu) and the
// residual loop of qwen35-c/src/q35_model.c:939 / :977, so the MLP's
// activations stay in HBM between the matmuls.
//
// Numerics follow the reference operation by operation.  FP contraction is
// off in every function here (the reference compiles q35_kern.c with
// FP_CONTRACT OFF), so each multiply, add, divide and square root rounds on
// its own; division and square root are the correctly rounded ones (hipcc's
// default for fp32).
//  - RMSNorm: the sum of squares runs in the reference's eight lanes
//    (element i into lane i mod 8, in increasing i), lanes folded 0..7,
//    mean = s / n, inv = 1 / sqrtf(mean + eps), y = (x * inv) * (1 + w):
//    bit-identical to the reference.
//  - SwiGLU: y = (g * (1 / (1 + e))) * u with e = exp(-g) evaluated in
//    double precision and rounded once to float.  libm's expf is not
//    correctly rounded; for about 4 in 100 000 inputs it differs from the
//    correctly rounded value by one ulp, and y then differs by 1 to 4 ulps
//    (1 + e can round to a neighbour whose ulp is 2-4 times that of e).
//    Every other input gives the reference's bits.
//  - Residual add: x = x + y, one rounding, identical.
#include "q35mm_device.h"
#include "q35mm_internal.h"

namespace q35mm {

namespace {

// Columns of one row handled per pass: kNormThreads threads x kNormPer
// columns, a multiple of 8 so that lane i mod 8 is fixed across passes.
// Thread t holds columns t + kNormThreads*j (j < kNormPer) in registers, so a
// pass costs one memory round trip.  Squares go to LDS lane-major,
// [8][kNormChunk/8 + 4]: the sequential lane reads four consecutive squares
// per access and the +4 pad spreads the eight lanes' rows over the banks.
constexpr uint32_t kNormThreads = 512;
constexpr uint32_t kNormPer = 16;
constexpr uint32_t kNormChunk = kNormThreads * kNormPer;   // 8192
constexpr uint32_t kNormLaneStride = kNormChunk / 8 + 4;

}  // namespace

// One workgroup per row.  The eight lanes' sums are the only sequential part
// (n/8 dependent adds each, on lanes 0..7 of wavefront 0); the squares are
// formed by all threads and handed over through LDS.  Rows of up to
// kNormChunk columns keep x and w in registers from the first load to the
// store; longer rows read them again for the output pass.
__global__ __launch_bounds__(kNormThreads) void rmsnorm_kernel(const float *x, uint32_t ldx,
                                                               const float *__restrict__ w, float *y,
                                                               uint32_t ldy, uint32_t n, float eps) {
#pragma clang fp contract(off)
    __shared__ __align__(16) float sq[8 * kNormLaneStride];
    __shared__ float lanes[8];
    const float *xr = x + (size_t)blockIdx.x * ldx;
    float *yr = y + (size_t)blockIdx.x * ldy;
    const uint32_t tid = threadIdx.x;

    float xv[kNormPer], wv[kNormPer];
    float acc = 0.0f;   // lane tid of the reference's eight (tid < 8)
    for (uint32_t c0 = 0; c0 < n; c0 += kNormChunk) {
        const uint32_t len = min(kNormChunk, n - c0);
#pragma unroll
        for (uint32_t j = 0; j < kNormPer; j++) {
            const uint32_t i = tid + j * kNormThreads;
            xv[j] = i < len ? xr[c0 + i] : 0.0f;
        }
        if (c0 == 0) {   // w for the output pass of a single-pass row, early
#pragma unroll
            for (uint32_t j = 0; j < kNormPer; j++) {
                const uint32_t i = tid + j * kNormThreads;
                wv[j] = i < len ? w[i] : 0.0f;
            }
        }
        // Columns past the row's end square to +0.0f, which leaves every
        // lane sum unchanged.
#pragma unroll
        for (uint32_t j = 0; j < kNormPer; j++) {
            const uint32_t i = tid + j * kNormThreads;
            sq[(i & 7) * kNormLaneStride + (i >> 3)] = xv[j] * xv[j];
        }
        __syncthreads();
        if (tid < 8) acc = lane_sum_in_order(sq + tid * kNormLaneStride, (len + 7) >> 3, acc);
        __syncthreads();
    }
    if (tid < 8) lanes[tid] = acc;
    __syncthreads();
    float s = lanes[0];
#pragma unroll
    for (int j = 1; j < 8; j++) s = s + lanes[j];
    const float inv = rms_inverse(s, n, eps);
    if (n <= kNormChunk) {
#pragma unroll
        for (uint32_t j = 0; j < kNormPer; j++) {
            const uint32_t i = tid + j * kNormThreads;
            if (i < n) yr[i] = rmsnorm1(xv[j], inv, wv[j]);
        }
        return;
    }
    for (uint32_t i = tid; i < n; i += kNormThreads) yr[i] = rmsnorm1(xr[i], inv, w[i]);
}

// The same RMSNorm written straight into the prefill GEMM's activations:
// bf16 in the lane-order layout of act_to_bf16_kernel (per 32 rows x 128
// columns, unit u = 64*jq + 32*h + r of 16 bytes holds row r, columns
// 32*(jq/2) + 16*h + 8*(jq%2) .. +7), rounded as that kernel rounds --
// the bits of rmsnorm_kernel followed by act_to_bf16_kernel, without the
// fp32 rows in between.  One workgroup per row of the padded tile rows;
// thread t owns the groups of eight columns t and t + kNormThreads, whose
// squares go to the reference's eight lanes (column 8g + e to lane e) and
// whose outputs fill one 16-byte unit each.  Rows past m and the columns
// of a partial last K block are written as zeros.  n % 8 == 0, n <=
// kNormBf16MaxCols, x rows and w 16-byte aligned (the host checks).
__global__ __launch_bounds__(kNormThreads) void rmsnorm_bf16_kernel(const float *x, uint32_t ldx,
                                                                    const float *__restrict__ w, uint32_t m,
                                                                    uint32_t n, uint32_t kb_total, float eps,
                                                                    uint8_t *xb) {
#pragma clang fp contract(off)
    constexpr uint32_t G = kNormBf16MaxCols / (8 * kNormThreads);   // groups per thread
    __shared__ __align__(16) float sq[8 * kNormLaneStride];
    __shared__ float lanes[8];
    const uint32_t row = blockIdx.x, tid = threadIdx.x;
    const uint32_t ng = n / 8, gp = kb_total * (kBlock / 8);   // groups with data / in the layout
    uint8_t *const base = xb + (size_t)(row / 32) * kb_total * 8 * kChunkBytes;
    auto unit = [&](uint32_t g) {
        const uint32_t c = (g % 16) * 8;   // column within its K block
        const uint32_t u = ((c >> 5) * 2 + ((c >> 3) & 1)) * 64 + ((c >> 4) & 1) * 32 + row % 32;
        return reinterpret_cast<u32x4_t *>(base + (size_t)(g / 16) * 8 * kChunkBytes + u * 16);
    };
    if (row >= m) {
#pragma unroll
        for (uint32_t j = 0; j < G; j++) {
            const uint32_t g = tid + j * kNormThreads;
            if (g < gp) *unit(g) = u32x4_t{0u, 0u, 0u, 0u};
        }
        return;
    }
    const float *xr = x + (size_t)row * ldx;
    float xv[G][8], wv[G][8];
#pragma unroll
    for (uint32_t j = 0; j < G; j++) {
        const uint32_t g = tid + j * kNormThreads;
        if (g < ng) {
            const float4 a = *reinterpret_cast<const float4 *>(xr + 8 * g);
            const float4 b = *reinterpret_cast<const float4 *>(xr + 8 * g + 4);
            const float4 c = *reinterpret_cast<const float4 *>(w + 8 * g);
            const float4 d = *reinterpret_cast<const float4 *>(w + 8 * g + 4);
            xv[j][0] = a.x; xv[j][1] = a.y; xv[j][2] = a.z; xv[j][3] = a.w;
            xv[j][4] = b.x; xv[j][5] = b.y; xv[j][6] = b.z; xv[j][7] = b.w;
            wv[j][0] = c.x; wv[j][1] = c.y; wv[j][2] = c.z; wv[j][3] = c.w;
            wv[j][4] = d.x; wv[j][5] = d.y; wv[j][6] = d.z; wv[j][7] = d.w;
        } else {
#pragma unroll
            for (uint32_t e = 0; e < 8; e++) xv[j][e] = wv[j][e] = 0.0f;
        }
    }
#pragma unroll
    for (uint32_t j = 0; j < G; j++) {
        const uint32_t g = tid + j * kNormThreads;
        if (g < ng) {
#pragma unroll
            for (uint32_t e = 0; e < 8; e++) sq[e * kNormLaneStride + g] = xv[j][e] * xv[j][e];
        }
    }
    __syncthreads();
    if (tid < 8) lanes[tid] = lane_sum_in_order(sq + tid * kNormLaneStride, ng, 0.0f);
    __syncthreads();
    float s = lanes[0];
#pragma unroll
    for (int j = 1; j < 8; j++) s = s + lanes[j];
    const float inv = rms_inverse(s, n, eps);
#pragma unroll
    for (uint32_t j = 0; j < G; j++) {
        const uint32_t g = tid + j * kNormThreads;
        if (g >= gp) continue;
        float v[8];
#pragma unroll
        for (uint32_t e = 0; e < 8; e++) v[e] = g < ng ? bf16_saturate(rmsnorm1(xv[j][e], inv, wv[j][e])) : 0.0f;
        *unit(g) = u32x4_t{f32x2_to_bf16x2_rne(v[0], v[1]), f32x2_to_bf16x2_rne(v[2], v[3]),
                           f32x2_to_bf16x2_rne(v[4], v[5]), f32x2_to_bf16x2_rne(v[6], v[7])};
    }
}

__global__ void swiglu_kernel(const float *g, const float *u, float *y, size_t n) {
#pragma clang fp contract(off)
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) y[i] = swiglu1(g[i], u[i]);
}

__global__ void add_inplace_kernel(float *x, const float *y, size_t n) {
#pragma clang fp contract(off)
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) x[i] = x[i] + y[i];
}

hipError_t launch_rmsnorm(const float *x, uint32_t ldx, const float *w, float *y, uint32_t ldy,
                          uint32_t rows, uint32_t n, float eps, hipStream_t stream) {
    if (rows == 0 || n == 0) return hipSuccess;
    hipLaunchKernelGGL(rmsnorm_kernel, dim3(rows), dim3(kNormThreads), 0, stream, x, ldx, w, y, ldy, n, eps);
    return hipGetLastError();
}

bool rmsnorm_bf16_fits(const float *x, uint32_t ldx, const float *w, uint32_t n) {
    return n > 0 && n % 8 == 0 && n <= kNormBf16MaxCols && ldx % 4 == 0 &&
           reinterpret_cast<uintptr_t>(x) % 16 == 0 && reinterpret_cast<uintptr_t>(w) % 16 == 0;
}

hipError_t launch_rmsnorm_bf16(const float *x, uint32_t ldx, const float *w, uint32_t m, uint32_t n, float eps,
                               uint32_t rows_pad, uint32_t kb, uint16_t *xb, hipStream_t stream) {
    if (!rmsnorm_bf16_fits(x, ldx, w, n) || rows_pad % 32 != 0 || rows_pad < m || kb * kBlock < n)
        return hipErrorInvalidValue;
    if (rows_pad == 0) return hipSuccess;
    hipLaunchKernelGGL(rmsnorm_bf16_kernel, dim3(rows_pad), dim3(kNormThreads), 0, stream, x, ldx, w, m, n, kb, eps,
                       reinterpret_cast<uint8_t *>(xb));
    return hipGetLastError();
}

namespace {
uint32_t elementwise_grid(size_t n) {
    // up to 16 workgroups of 256 per CU; grid-stride beyond that
    const size_t wgs = (n + 255) / 256;
    return (uint32_t)(wgs < 4096 ? wgs : 4096);
}
}  // namespace

hipError_t launch_swiglu(const float *g, const float *u, float *y, size_t n, hipStream_t stream) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(swiglu_kernel, dim3(elementwise_grid(n)), dim3(256), 0, stream, g, u, y, n);
    return hipGetLastError();
}

hipError_t launch_add_inplace(float *x, const float *y, size_t n, hipStream_t stream) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(add_inplace_kernel, dim3(elementwise_grid(n)), dim3(256), 0, stream, x, y, n);
    return hipGetLastError();
}

}  // namespace q35mm
