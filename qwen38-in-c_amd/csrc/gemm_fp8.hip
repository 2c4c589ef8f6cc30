// gemm_fp8.hip -- prefill GEMM for FP8-E4M3 weights with 128x128 fp32 block
// scales: Y[t][n] = sum_k bf16(x[t][k]) * e4m3(W[n][k]) * s[n/128][k/128].
//
// Replaces the batched path of qwen35-c/src/q35_mm.c:158-172
// (q35_mm_fp8_batch) for m >= 64 tokens, where the work is a dense
// contraction: bf16 MFMA (v_mfma_f32_32x32x16_bf16) with fp32 accumulation.
//
//  - Activations are rounded to bf16 once per call by act_to_bf16_kernel,
//    which writes them in the same lane-order layout as the weights (32-row
//    tiles, 1 KiB per MFMA operand load).
//  - e4m3 -> bf16 is exact, so weights are converted in registers after the
//    LDS read; the block scale is never folded into bf16 weights (that
//    would round).  Per 128-wide K block the MFMA accumulators hold the raw
//    block product, then each output gets acc += scale * block (fp32 fmaf).
//  - A workgroup computes a 128x128 output tile (one scale row-block, so the
//    scale is uniform across the tile for each K block) with four
//    wavefronts of 64x64; tiles of A (32 KiB bf16) and B (16 KiB e4m3) per K
//    block are staged through LDS, the next block's global loads are in
//    flight while the current one is multiplied.
//  - Split-K with a deterministic last-arriver fixup when there are too few
//    output tiles to occupy the device.
#include "q35mm_device.h"
#include "q35mm_internal.h"

namespace q35mm {

namespace {

constexpr uint32_t kGemmThreads = 256;
constexpr uint32_t kAPieces = 32;   // 4 m32 tiles x 4 chunks x 2 MFMA halves
constexpr uint32_t kBPieces = 16;   // 4 n32 tiles x 4 chunks
constexpr uint32_t kPiecesPerWave = (kAPieces + kBPieces) / 4;

__device__ __forceinline__ u32x4_t ld16(const void *p) {
    return *reinterpret_cast<const u32x4_t *>(p);
}

}  // namespace

// X fp32 [m][ldx] -> bf16 (round to nearest even) in lane order:
//   unit u = ((m32 * KB + kb) * 8 + j*2 + q) * 64 + lane, 16 bytes each,
//   row = m32*32 + lane%32, columns kb*128 + j*32 + (lane/32)*16 + q*8 + e.
// Rows >= m and columns >= k are zero.
__global__ __launch_bounds__(256) void act_to_bf16_kernel(const float *__restrict__ x, uint32_t ldx,
                                                          uint32_t m, uint32_t k, uint32_t kb_total,
                                                          uint32_t units, uint16_t *__restrict__ xb) {
    const uint32_t u = blockIdx.x * blockDim.x + threadIdx.x;
    if (u >= units) return;
    const uint32_t lane = u & 63;
    const uint32_t jq = (u >> 6) & 7;
    const uint32_t rest = u >> 9;            // m32 * KB + kb
    const uint32_t kb = rest % kb_total;
    const uint32_t m32 = rest / kb_total;
    const uint32_t row = m32 * 32 + (lane & 31);
    const uint32_t col = kb * kBlock + (jq >> 1) * 32 + (lane >> 5) * 16 + (jq & 1) * 8;
    uint32_t b[8];
    const float *xp = x + (size_t)row * ldx + col;
#pragma unroll
    for (int e = 0; e < 8; e++) {
        const float v = (row < m && col + e < k) ? xp[e] : 0.0f;
        b[e] = f32_to_bf16_rne(v);
    }
    u32x4_t o = {b[0] | (b[1] << 16), b[2] | (b[3] << 16), b[4] | (b[5] << 16), b[6] | (b[7] << 16)};
    *reinterpret_cast<u32x4_t *>(xb + (size_t)u * 8) = o;
}

__global__ __launch_bounds__(kGemmThreads) void gemm_fp8_kernel(GemmParams p) {
    __shared__ __align__(16) uint8_t lds_a[kAPieces * kChunkBytes];
    __shared__ __align__(16) uint8_t lds_b[kBPieces * kChunkBytes];
    __shared__ uint32_t s_ticket;

    const uint32_t S = p.nslices;
    const uint32_t tile = blockIdx.x / S;
    const uint32_t s = blockIdx.x - tile * S;
    const uint32_t mt = tile % p.mtiles;
    const uint32_t nt = tile / p.mtiles;
    const uint32_t KB = p.kb;
    const uint32_t kb0 = (s * KB) / S;
    const uint32_t kb1 = ((s + 1) * KB) / S;

    const uint32_t lane = threadIdx.x & 63;
    const uint32_t wv = threadIdx.x >> 6;
    const uint32_t wm = wv & 1, wn = wv >> 1;

    // Global sources for the pieces this wavefront copies.  Piece P < 32 is
    // A piece (m32 = P/8, chunk-half = P%8); P >= 32 is B piece P-32.
    const uint8_t *xa = reinterpret_cast<const uint8_t *>(p.xb);
    const size_t a_tile_stride = (size_t)KB * 8 * kChunkBytes;   // one m32 row of tiles
    u32x4_t stage[kPiecesPerWave];
    auto load_stage = [&](uint32_t kb) {
#pragma unroll
        for (uint32_t u = 0; u < kPiecesPerWave; u++) {
            const uint32_t P = wv + 4 * u;
            const uint8_t *src;
            if (P < kAPieces) {
                const uint32_t m32 = mt * 4 + P / 8;
                src = xa + m32 * a_tile_stride + (size_t)kb * 8 * kChunkBytes + (P % 8) * kChunkBytes;
            } else {
                src = p.codes + ((size_t)nt * KB + kb) * kBlockBytes + (P - kAPieces) * kChunkBytes;
            }
            stage[u] = ld16(src + lane * 16);
        }
    };
    auto store_stage = [&]() {
#pragma unroll
        for (uint32_t u = 0; u < kPiecesPerWave; u++) {
            const uint32_t P = wv + 4 * u;
            uint8_t *dst = P < kAPieces ? lds_a + P * kChunkBytes : lds_b + (P - kAPieces) * kChunkBytes;
            *reinterpret_cast<u32x4_t *>(dst + lane * 16) = stage[u];
        }
    };

    f32x16_t acc[2][2] = {};
    const f32x16_t zero = {};
    const float *srow = p.scale + (size_t)nt * KB;

    load_stage(kb0);
    for (uint32_t kb = kb0; kb < kb1; kb++) {
        __syncthreads();
        store_stage();
        __syncthreads();
        if (kb + 1 < kb1) load_stage(kb + 1);

        f32x16_t part[2][2];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            u32x4_t braw[2];
#pragma unroll
            for (int jn = 0; jn < 2; jn++)
                braw[jn] = ld16(lds_b + ((2 * wn + jn) * 4 + j) * kChunkBytes + lane * 16);
#pragma unroll
            for (int q = 0; q < 2; q++) {
                bf16x8_t bop[2];
#pragma unroll
                for (int jn = 0; jn < 2; jn++)
                    bop[jn] = e4m3x8_to_bf16x8(braw[jn][2 * q], braw[jn][2 * q + 1]);
#pragma unroll
                for (int i = 0; i < 2; i++) {
                    const bf16x8_t aop = __builtin_bit_cast(
                        bf16x8_t, ld16(lds_a + ((2 * wm + i) * 8 + j * 2 + q) * kChunkBytes + lane * 16));
#pragma unroll
                    for (int jn = 0; jn < 2; jn++)
                        part[i][jn] = mfma32x32x16(aop, bop[jn], (j == 0 && q == 0) ? zero : part[i][jn]);
                }
            }
        }
        const float sc = srow[kb];
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int jn = 0; jn < 2; jn++)
#pragma unroll
                for (int r = 0; r < 16; r++) acc[i][jn][r] = __builtin_fmaf(sc, part[i][jn][r], acc[i][jn][r]);
    }

    // Output coordinates of accumulator element (i, jn, r) of this lane.
    auto out_row = [&](int i, int r) -> uint32_t {
        return (2 * wm + i) * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
    };
    auto out_col = [&](int jn) -> uint32_t { return (2 * wn + jn) * 32 + (lane & 31); };

    if (S == 1) {
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int jn = 0; jn < 2; jn++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const uint32_t mrow = mt * kGemmTile + out_row(i, r);
                    const uint32_t ncol = nt * kGemmTile + out_col(jn);
                    if (mrow < p.m && ncol < p.rows) p.y[(size_t)mrow * p.ldy + ncol] = acc[i][jn][r];
                }
        return;
    }

    float *ws = p.ws + ((size_t)tile * S + s) * kGemmTile * kGemmTile;
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int jn = 0; jn < 2; jn++)
#pragma unroll
            for (int r = 0; r < 16; r++) ws[out_row(i, r) * kGemmTile + out_col(jn)] = acc[i][jn][r];
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) s_ticket = atomicAdd(p.cnt + tile, 1u);
    __syncthreads();
    if (s_ticket != S - 1) return;

    __threadfence();
    const float *base = p.ws + (size_t)tile * S * kGemmTile * kGemmTile;
    for (uint32_t e = threadIdx.x; e < kGemmTile * kGemmTile; e += blockDim.x) {
        float sum = __builtin_nontemporal_load(base + e);
        for (uint32_t s2 = 1; s2 < S; s2++)
            sum += __builtin_nontemporal_load(base + (size_t)s2 * kGemmTile * kGemmTile + e);
        const uint32_t mrow = mt * kGemmTile + e / kGemmTile;
        const uint32_t ncol = nt * kGemmTile + e % kGemmTile;
        if (mrow < p.m && ncol < p.rows) p.y[(size_t)mrow * p.ldy + ncol] = sum;
    }
    if (threadIdx.x == 0) p.cnt[tile] = 0u;
}

uint32_t gemm_slices(uint32_t mtiles, uint32_t ntiles, uint32_t kb) {
    // Split K only when the output tiles cannot occupy a 256-CU device.
    const uint32_t tiles = mtiles * ntiles;
    uint32_t s = 1;
    while (tiles * s < 256 && s * 2 <= kb / 4) s *= 2;
    return s;
}

hipError_t launch_act_to_bf16(const float *x, uint32_t ldx, uint32_t m, uint32_t k,
                              uint32_t mtiles, uint32_t kb, uint16_t *xb, hipStream_t stream) {
    const uint32_t units = mtiles * 4 * kb * 8 * 64;
    hipLaunchKernelGGL(act_to_bf16_kernel, dim3((units + 255) / 256), dim3(256), 0, stream,
                       x, ldx, m, k, kb, units, xb);
    return hipGetLastError();
}

hipError_t launch_gemm(const GemmParams &p, hipStream_t stream) {
    const uint32_t grid = p.mtiles * p.ntiles * p.nslices;
    hipLaunchKernelGGL(gemm_fp8_kernel, dim3(grid), dim3(kGemmThreads), 0, stream, p);
    return hipGetLastError();
}

}  // namespace q35mm
