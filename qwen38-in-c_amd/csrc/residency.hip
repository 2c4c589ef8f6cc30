// residency.hip -- weight residency kernels: repack row-major e4m3 codes
// into the lane-order tile layout (q35mm_device.h), bit-exact dequant to
// fp32, and the e4m3 -> bf16 conversion the matrix-core kernels use.
//
// The reference binds the checkpoint's e4m3 bytes and bf16 scales zero-copy
// from a file mapping (qwen35-c/src/q35_model.c:253-273) and dequantises
// inside the matmul loop (qwen35-c/src/q35_mm.c:99,110-111,120); here the
// codes are uploaded once and repacked on the device.
#include <algorithm>

#include "q35mm_device.h"
#include "q35mm_internal.h"

namespace q35mm {

namespace {

// Decompose a 16-byte unit index of the tiled layout.
struct TileCoord {
    uint32_t row, col;   // of the unit's first byte
};

__device__ __forceinline__ TileCoord unit_coord(uint32_t u, uint32_t kb_total) {
    const uint32_t lane = u & 63;
    const uint32_t j = (u >> 6) & 3;
    const uint32_t sub = (u >> 8) & 3;
    const uint32_t blk = u >> 10;                 // nb * KB + kb
    const uint32_t kb = blk % kb_total;
    const uint32_t nb = blk / kb_total;
    TileCoord c;
    c.row = nb * kBlock + sub * kSubRows + (lane & 31);
    c.col = kb * kBlock + j * 32 + (lane >> 5) * 16;
    return c;
}

}  // namespace

__global__ __launch_bounds__(256) void repack_kernel(const uint8_t *__restrict__ raw, uint32_t rows,
                                                     uint32_t cols, uint32_t kb_total, uint32_t units,
                                                     uint8_t *__restrict__ tiled) {
    const uint32_t u = blockIdx.x * blockDim.x + threadIdx.x;
    if (u >= units) return;
    const TileCoord c = unit_coord(u, kb_total);
    uint32_t w[4] = {0u, 0u, 0u, 0u};
    if (c.row < rows) {
        const uint8_t *src = raw + (size_t)c.row * cols + c.col;
#pragma unroll
        for (int e = 0; e < 16; e++) {
            const uint32_t b = (c.col + e < cols) ? src[e] : 0u;
            w[e >> 2] |= b << (8 * (e & 3));
        }
    }
    u32x4_t o = {w[0], w[1], w[2], w[3]};
    *reinterpret_cast<u32x4_t *>(tiled + (size_t)u * 16) = o;
}

// out[r][c] = e4m3(W[r][c]) * scale[r/128][c/128], one rounded fp32 multiply,
// exactly the reference's lut[b] * s (qwen35-c/src/q35_mm.c:110-111,120).
__global__ __launch_bounds__(256) void dequant_f32_kernel(const uint8_t *__restrict__ tiled,
                                                          const float *__restrict__ scale,
                                                          uint32_t rows, uint32_t cols,
                                                          uint32_t kb_total, uint32_t units,
                                                          float *__restrict__ out) {
    const uint32_t u = blockIdx.x * blockDim.x + threadIdx.x;
    if (u >= units) return;
    const TileCoord c = unit_coord(u, kb_total);
    if (c.row >= rows || c.col >= cols) return;
    const u32x4_t q = *reinterpret_cast<const u32x4_t *>(tiled + (size_t)u * 16);
    const float s = scale[(size_t)(c.row / kBlock) * kb_total + c.col / kBlock];
    float v[16];
#pragma unroll
    for (int d = 0; d < 4; d++) {
        const f32x2_t lo = e4m3x2_to_f32<false>(q[d]);
        const f32x2_t hi = e4m3x2_to_f32<true>(q[d]);
        v[4 * d + 0] = lo.x * s;
        v[4 * d + 1] = lo.y * s;
        v[4 * d + 2] = hi.x * s;
        v[4 * d + 3] = hi.y * s;
    }
    float *dst = out + (size_t)c.row * cols + c.col;
#pragma unroll
    for (int e = 0; e < 16; e++)
        if (c.col + e < cols) dst[e] = v[e];
}

// out[r][c] = bf16 bits of e4m3(W[r][c]), unscaled: the operand conversion
// of the GEMV and GEMM kernels (e4m3x8_to_bf16x8_cvt at scale 1.0).
__global__ __launch_bounds__(256) void decode_bf16_kernel(const uint8_t *__restrict__ tiled,
                                                          uint32_t rows, uint32_t cols,
                                                          uint32_t kb_total, uint32_t units,
                                                          uint16_t *__restrict__ out) {
    const uint32_t u = blockIdx.x * blockDim.x + threadIdx.x;
    if (u >= units) return;
    const TileCoord c = unit_coord(u, kb_total);
    if (c.row >= rows || c.col >= cols) return;
    const u32x4_t q = *reinterpret_cast<const u32x4_t *>(tiled + (size_t)u * 16);
    const bf16x8_t lo = e4m3x8_to_bf16x8_cvt(q[0], q[1], 1.0f);
    const bf16x8_t hi = e4m3x8_to_bf16x8_cvt(q[2], q[3], 1.0f);
    const u32x4_t l4 = __builtin_bit_cast(u32x4_t, lo);
    const u32x4_t h4 = __builtin_bit_cast(u32x4_t, hi);
    uint16_t v[16];
#pragma unroll
    for (int d = 0; d < 4; d++) {
        v[2 * d] = (uint16_t)(l4[d] & 0xFFFFu);
        v[2 * d + 1] = (uint16_t)(l4[d] >> 16);
        v[8 + 2 * d] = (uint16_t)(h4[d] & 0xFFFFu);
        v[8 + 2 * d + 1] = (uint16_t)(h4[d] >> 16);
    }
    uint16_t *dst = out + (size_t)c.row * cols + c.col;
#pragma unroll
    for (int e = 0; e < 16; e++)
        if (c.col + e < cols) dst[e] = v[e];
}

static uint32_t tile_units(uint32_t nb, uint32_t kb) { return nb * kb * (kBlockBytes / 16); }

hipError_t launch_repack(const uint8_t *raw, uint32_t rows, uint32_t cols, uint32_t nb, uint32_t kb,
                         uint8_t *tiled, hipStream_t stream) {
    const uint32_t units = tile_units(nb, kb);
    hipLaunchKernelGGL(repack_kernel, dim3((units + 255) / 256), dim3(256), 0, stream,
                       raw, rows, cols, kb, units, tiled);
    return hipGetLastError();
}

hipError_t launch_dequant_f32(const Weight &w, float *out, hipStream_t stream) {
    const uint32_t units = tile_units(w.nb, w.kb);
    hipLaunchKernelGGL(dequant_f32_kernel, dim3((units + 255) / 256), dim3(256), 0, stream,
                       w.codes, w.scale, w.rows, w.cols, w.kb, units, out);
    return hipGetLastError();
}

hipError_t launch_decode_bf16(const Weight &w, uint16_t *out, hipStream_t stream) {
    const uint32_t units = tile_units(w.nb, w.kb);
    hipLaunchKernelGGL(decode_bf16_kernel, dim3((units + 255) / 256), dim3(256), 0, stream,
                       w.codes, w.rows, w.cols, w.kb, units, out);
    return hipGetLastError();
}

// ---------------------------------------------------------------------
// Completion flag of a host-pointer call: runs after the call's kernels on
// the same stream (so after their completion and end-of-kernel release) and
// stores v into pinned host memory, where the calling thread waits for it.
__global__ __launch_bounds__(64) void done_flag_kernel(uint32_t *flag, uint32_t v) {
    if (threadIdx.x == 0) {
        __threadfence_system();
        __hip_atomic_store(flag, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    }
}

hipError_t launch_done_flag(uint32_t *flag, uint32_t v, hipStream_t stream) {
    hipLaunchKernelGGL(done_flag_kernel, dim3(1), dim3(64), 0, stream, flag, v);
    return hipGetLastError();
}

// ---------------------------------------------------------------------
// BF16 matvec y[r] = sum_c bf16(W[r][c]) * x[c] (qwen35-c/src/q35_mm.c:211-246),
// fp32 accumulation.  One wavefront per row; each lane streams 16-byte
// loads (8 bf16) strided by 1 KiB and the wavefront reduces with a
// butterfly of cross-lane adds.
// ---------------------------------------------------------------------
// ---- BF16 matvec (q35_mm_bf16) ----------------------------------------
// The reference's order exactly (qwen35-c/src/q35_mm.c:211-246): for each
// row, eight fmaf chains acc[n % 8] over the columns in increasing order,
// then y = ((0 + acc[0]) + acc[1]) + ... + acc[7].  One lane per row holds
// the eight chains (independent, so the FMAs pipeline), so the result is the
// reference's bit for bit.
//
// Vector path (cols % 8 == 0, W 16-byte aligned): a wavefront owns 64 rows
// and walks K in tiles of 64 columns.  A tile (64 rows x 128 bytes) is read
// with coalesced 16-byte loads (8 rows x 128 contiguous bytes per
// instruction), kD tiles ahead in registers, and passed through LDS
// (row stride 144 bytes: conflict-free 16-byte reads) so that each lane gets
// its own row; the tile's 64 activations are broadcast from LDS.  Columns
// >= cols are zeroed (a zero product leaves every chain unchanged).
namespace {
constexpr uint32_t kBf16Tile = 64;                 // columns per tile
constexpr uint32_t kBf16Stride = 144;              // LDS bytes per row
constexpr uint32_t kBf16WaveLds = kBf16Tile * kBf16Stride + kBf16Tile * 4;
// Tiles in flight per wavefront: with non-temporal weight loads two run
// 1.5% faster than three or four on 248320 x 5120.
constexpr uint32_t kBf16Depth = 2;
}  // namespace

__global__ __launch_bounds__(256) void bf16_gemv_vec_kernel(const uint16_t *__restrict__ w, uint32_t rows,
                                                            uint32_t cols, const float *__restrict__ x,
                                                            float *__restrict__ y) {
    __shared__ __align__(16) uint8_t lds[4 * kBf16WaveLds];
    const uint32_t lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    uint8_t *const tl = lds + wv * kBf16WaveLds;          // this wavefront's tile
    float *const xl = reinterpret_cast<float *>(tl + kBf16Tile * kBf16Stride);
    const uint32_t r0 = (blockIdx.x * 4 + wv) * 64;
    const uint32_t ntiles = (cols + kBf16Tile - 1) / kBf16Tile;
    const uint32_t lr = lane >> 3, lc = lane & 7;         // load role: row lr + 8i, 16-byte chunk lc

    u32x4_t wt[kBf16Depth][8];
    float xt[kBf16Depth];
    auto load = [&](uint32_t slot, uint32_t t) {
        const uint32_t col = min(t * kBf16Tile + lc * 8, cols - 8);   // in bounds; masked later
#pragma unroll
        for (uint32_t i = 0; i < 8; i++) {
            const uint32_t row = min(r0 + lr + 8 * i, rows - 1);
            // read once per call: non-temporal (+9% against plain loads)
            wt[slot][i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t *>(w + (size_t)row * cols + col));
        }
        xt[slot] = x[min(t * kBf16Tile + lane, cols - 1)];
    };
#pragma unroll
    for (uint32_t d = 0; d + 1 < kBf16Depth; d++) load(d, min(d, ntiles - 1));

    float acc[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
    for (uint32_t t0 = 0; t0 < ntiles; t0 += kBf16Depth) {
#pragma unroll
        for (uint32_t d = 0; d < kBf16Depth; d++) {
            const uint32_t t = t0 + d;
            load((d + kBf16Depth - 1) % kBf16Depth, min(t + kBf16Depth - 1, ntiles - 1));
            if (t < ntiles) {
                const bool wlive = t * kBf16Tile + lc * 8 < cols;
#pragma unroll
                for (uint32_t i = 0; i < 8; i++) {
                    const u32x4_t v = wlive ? wt[d][i] : u32x4_t{0u, 0u, 0u, 0u};
                    *reinterpret_cast<u32x4_t *>(tl + (lr + 8 * i) * kBf16Stride + lc * 16) = v;
                }
                xl[lane] = t * kBf16Tile + lane < cols ? xt[d] : 0.0f;
                // Same wavefront: LDS operations complete in order.
#pragma unroll
                for (uint32_t c = 0; c < 8; c++) {
                    const u32x4_t q = *reinterpret_cast<const u32x4_t *>(tl + lane * kBf16Stride + c * 16);
                    const float4 xa = reinterpret_cast<const float4 *>(xl)[2 * c];
                    const float4 xb = reinterpret_cast<const float4 *>(xl)[2 * c + 1];
                    const float xv[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
#pragma unroll
                    for (uint32_t e = 0; e < 4; e++) {
                        acc[2 * e] = __builtin_fmaf(bits_f32(q[e] << 16), xv[2 * e], acc[2 * e]);
                        acc[2 * e + 1] = __builtin_fmaf(bits_f32(q[e] & 0xFFFF0000u), xv[2 * e + 1], acc[2 * e + 1]);
                    }
                }
            }
        }
    }
    const uint32_t row = r0 + lane;
    if (row < rows) {
        float sum = 0.0f;
#pragma unroll
        for (uint32_t j = 0; j < 8; j++) sum += acc[j];
        y[row] = sum;
    }
}

// Any cols / alignment: one thread per row, same order, element loads.
__global__ __launch_bounds__(256) void bf16_gemv_any_kernel(const uint16_t *__restrict__ w, uint32_t rows,
                                                            uint32_t cols, const float *__restrict__ x,
                                                            float *__restrict__ y) {
    const uint32_t row = blockIdx.x * 256 + threadIdx.x;
    if (row >= rows) return;
    const uint16_t *wr = w + (size_t)row * cols;
    float acc[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
    for (uint32_t c = 0; c < cols; c++) acc[c & 7] = __builtin_fmaf(bits_f32((uint32_t)wr[c] << 16), x[c], acc[c & 7]);
    float sum = 0.0f;
#pragma unroll
    for (uint32_t j = 0; j < 8; j++) sum += acc[j];
    y[row] = sum;
}

hipError_t launch_bf16_gemv(const uint16_t *w, uint32_t rows, uint32_t cols, const float *x, float *y,
                            hipStream_t stream) {
    if (cols % 8 == 0 && (reinterpret_cast<uintptr_t>(w) & 15u) == 0)
        hipLaunchKernelGGL(bf16_gemv_vec_kernel, dim3((rows + 255) / 256), dim3(256), 0, stream, w, rows, cols, x, y);
    else
        hipLaunchKernelGGL(bf16_gemv_any_kernel, dim3((rows + 255) / 256), dim3(256), 0, stream, w, rows, cols, x, y);
    return hipGetLastError();
}

}  // namespace q35mm
