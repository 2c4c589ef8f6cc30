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
