// q35mm_probe.hip -- ceilings the kernels are measured against (not part of
// libq35mm.so; built by build.py as lib/q35mm_probe).
//
//   q35mm_probe read [pool_MB]
//     Raw read time of e4m3 weights of the decode projection shapes in the
//     lane-order tiled layout (16 KiB per 128x128 block), no arithmetic:
//       tiles  -- the row-split GEMV's decomposition: one workgroup per 32-row
//                 sub-tile, four wavefronts splitting K, each loading one
//                 1 KiB chunk per lane-order load through a ring of 2 or 3
//                 K blocks (non-temporal loads, as the GEMV);
//       linear -- the same bytes as one contiguous stream, 256 workgroups,
//                 1 KiB per wavefront load, 8 loads in flight.
//     Each launch reads a different copy of the weight from a pool of
//     pool_MB (default 1536) so no cache holds it.  Prints us and GB/s.
//
//   q35mm_probe lds
//     LDS read rate of ds_read_b128 (conflict-free: lane l reads 16 bytes at
//     l*16 of a 1 KiB row) from 256 workgroups of 8 wavefronts, each
//     wavefront issuing 8 independent reads per iteration; prints bytes per
//     clock per CU (core clock from s_memtime against s_memrealtime).
//
//   q35mm_probe mfma
//     Issue rate of v_mfma_f32_32x32x16_bf16: 256 workgroups of four
//     wavefronts (one per SIMD), each wavefront issuing 8 independent
//     accumulator chains of back-to-back MFMAs; also the core clock under
//     that load (s_memtime ticks against s_memrealtime's 100 MHz).  Prints
//     TFLOP/s and cycles per MFMA.
//
//   q35mm_probe mfma_rand | mfma_order
//     The same on operands that change like real activations and weights
//     (mfma_order: the prefill GEMM's 4 x 2 tile pattern in three issue
//     orders, one or two wavefronts per SIMD).
//
//   q35mm_probe mix
//     MFMA issue with VALU work (rescale multiplies, e4m3 conversions)
//     beside it, spread or in bursts.
//
//   q35mm_probe launch
//     Cost of one more launch in a sequence of dependent launches (empty
//     kernel, on a stream and as a graph).
//
//   q35mm_probe sync [spin]
//     Host round trip of launch + wait: hipStreamSynchronize,
//     hipEventSynchronize, or spinning on a flag the kernel stores into
//     pinned memory (spin: hipDeviceScheduleSpin first).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#define CK(x)                                                                                  \
    do {                                                                                       \
        hipError_t e_ = (x);                                                                   \
        if (e_ != hipSuccess) {                                                                \
            fprintf(stderr, "%s failed: %s (line %d)\n", #x, hipGetErrorString(e_), __LINE__); \
            exit(1);                                                                           \
        }                                                                                      \
    } while (0)

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// ---- read: row-split decomposition ---------------------------------------
template <int D>
__global__ __launch_bounds__(256) void read_tiles(const uint8_t *codes, uint32_t kb, float *out) {
    const uint32_t lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const uint32_t sub = blockIdx.x, g = sub >> 2, s = sub & 3;
    const uint32_t k0 = wv * kb / 4, n = (wv + 1) * kb / 4 - k0;
    const uint8_t *b = codes + ((size_t)g * kb * 4 + s) * 4096 + (size_t)k0 * 16384 + lane * 16;
    u32x4 buf[D][4];
    uint32_t acc = 0;
#pragma unroll
    for (int d = 0; d < D; d++)
#pragma unroll
        for (int j = 0; j < 4; j++)
            buf[d][j] = __builtin_nontemporal_load((const u32x4 *)(b + (size_t)min((uint32_t)d, n - 1) * 16384 + j * 1024));
    for (uint32_t i = 0; i < n; i += D) {
#pragma unroll
        for (int d = 0; d < D; d++)
#pragma unroll
            for (int j = 0; j < 4; j++) {
                if (i + d < n) acc += buf[d][j].x ^ buf[d][j].w;
                buf[d][j] = __builtin_nontemporal_load(
                    (const u32x4 *)(b + (size_t)min(i + d + D, n - 1) * 16384 + j * 1024));
            }
    }
    if (lane == 0) out[blockIdx.x * 4 + wv] = (float)acc;
}

// read_tiles<2> behind NOPS s_nop instructions before the first load: what
// a longer stretch of code at the start of a kernel costs (at one
// instruction per cycle, 1600 s_nop take 0.8 us; more means the code is
// fetched cold).
template <int NOPS>
__global__ __launch_bounds__(256) void read_tiles_pad(const uint8_t *codes, uint32_t kb, float *out) {
    if constexpr (NOPS == 400) asm volatile(".rept 400\n s_nop 0\n .endr");
    if constexpr (NOPS == 1600) asm volatile(".rept 1600\n s_nop 0\n .endr");
    const uint32_t lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const uint32_t sub = blockIdx.x, g = sub >> 2, s = sub & 3;
    const uint32_t k0 = wv * kb / 4, n = (wv + 1) * kb / 4 - k0;
    const uint8_t *b = codes + ((size_t)g * kb * 4 + s) * 4096 + (size_t)k0 * 16384 + lane * 16;
    u32x4 buf[2][4];
    uint32_t acc = 0;
#pragma unroll
    for (int d = 0; d < 2; d++)
#pragma unroll
        for (int j = 0; j < 4; j++)
            buf[d][j] = __builtin_nontemporal_load((const u32x4 *)(b + (size_t)min((uint32_t)d, n - 1) * 16384 + j * 1024));
    for (uint32_t i = 0; i < n; i += 2) {
#pragma unroll
        for (int d = 0; d < 2; d++)
#pragma unroll
            for (int j = 0; j < 4; j++) {
                if (i + d < n) acc += buf[d][j].x ^ buf[d][j].w;
                buf[d][j] = __builtin_nontemporal_load((const u32x4 *)(b + (size_t)min(i + d + 2, n - 1) * 16384 + j * 1024));
            }
    }
    if (lane == 0) out[blockIdx.x * 4 + wv] = (float)acc;
}

// read_tiles with timestamps (s_memrealtime, 100 MHz): entry, first block
// consumed, end; wavefront 0 of each workgroup writes them to st[3 * wg].
template <int D>
__global__ __launch_bounds__(256) void read_tiles_st(const uint8_t *codes, uint32_t kb, float *out, uint32_t *st) {
    const uint32_t t0 = (uint32_t)__builtin_amdgcn_s_memrealtime();
    uint32_t t1 = 0;
    const uint32_t lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const uint32_t sub = blockIdx.x, g = sub >> 2, s = sub & 3;
    const uint32_t k0 = wv * kb / 4, n = (wv + 1) * kb / 4 - k0;
    const uint8_t *b = codes + ((size_t)g * kb * 4 + s) * 4096 + (size_t)k0 * 16384 + lane * 16;
    u32x4 buf[D][4];
    uint32_t acc = 0;
#pragma unroll
    for (int d = 0; d < D; d++)
#pragma unroll
        for (int j = 0; j < 4; j++)
            buf[d][j] = __builtin_nontemporal_load((const u32x4 *)(b + (size_t)min((uint32_t)d, n - 1) * 16384 + j * 1024));
    for (uint32_t i = 0; i < n; i += D) {
#pragma unroll
        for (int d = 0; d < D; d++) {
#pragma unroll
            for (int j = 0; j < 4; j++) {
                if (i + d < n) acc += buf[d][j].x ^ buf[d][j].w;
                buf[d][j] = __builtin_nontemporal_load((const u32x4 *)(b + (size_t)min(i + d + D, n - 1) * 16384 + j * 1024));
            }
            if (i + d == 0) t1 = (uint32_t)__builtin_amdgcn_s_memrealtime() + (acc & 1) * 0;
        }
    }
    if (lane == 0) out[blockIdx.x * 4 + wv] = (float)acc;
    const uint32_t t2 = (uint32_t)__builtin_amdgcn_s_memrealtime();
    if (wv == 0 && lane == 0) {
        st[3 * blockIdx.x] = t0;
        st[3 * blockIdx.x + 1] = t1;
        st[3 * blockIdx.x + 2] = t2;
    }
}

// read_tiles<3> whose unrolled loop carries NOPS s_nop per block copy
// (executed every block, in the shadow of the memory wait): what a larger
// loop body costs once per launch when its code is fetched cold.
template <int NOPS>
__global__ __launch_bounds__(256) void read_tiles_fat(const uint8_t *codes, uint32_t kb, float *out) {
    const uint32_t lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const uint32_t sub = blockIdx.x, g = sub >> 2, s = sub & 3;
    const uint32_t k0 = wv * kb / 4, n = (wv + 1) * kb / 4 - k0;
    const uint8_t *b = codes + ((size_t)g * kb * 4 + s) * 4096 + (size_t)k0 * 16384 + lane * 16;
    constexpr int D = 3;
    u32x4 buf[D][4];
    uint32_t acc = 0;
#pragma unroll
    for (int d = 0; d < D; d++)
#pragma unroll
        for (int j = 0; j < 4; j++)
            buf[d][j] = __builtin_nontemporal_load((const u32x4 *)(b + (size_t)min((uint32_t)d, n - 1) * 16384 + j * 1024));
    for (uint32_t i = 0; i < n; i += D) {
#pragma unroll
        for (int d = 0; d < D; d++) {
#pragma unroll
            for (int j = 0; j < 4; j++) {
                if (i + d < n) acc += buf[d][j].x ^ buf[d][j].w;
                buf[d][j] = __builtin_nontemporal_load((const u32x4 *)(b + (size_t)min(i + d + D, n - 1) * 16384 + j * 1024));
            }
            if constexpr (NOPS == 64) asm volatile(".rept 64\n s_nop 0\n .endr");
            if constexpr (NOPS == 256) asm volatile(".rept 256\n s_nop 0\n .endr");
        }
    }
    if (lane == 0) out[blockIdx.x * 4 + wv] = (float)acc;
}

// ---- read: S sub-tiles per workgroup, W wavefronts splitting K -------------------
// S = 2: 64 rows per workgroup, S = 4: a whole 128-row group (16 KiB per K
// block).  SM: the weight as if stored sub-tile-major (each 32-row
// sub-tile's K blocks contiguous, 4 KiB apart) instead of block-major.
template <int D, int S, int W, bool SM>
__global__ __launch_bounds__(64 * W) void read_group(const uint8_t *codes, uint32_t kb, float *out) {
    const uint32_t lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const uint32_t sub0 = blockIdx.x * S;
    const uint32_t k0 = wv * kb / W, n = (wv + 1) * kb / W - k0;
    auto addr = [&](uint32_t s, uint32_t k, uint32_t j) -> const u32x4 * {
        const uint32_t sub = sub0 + s, g = sub >> 2, t = sub & 3;
        const size_t o = SM ? ((size_t)sub * kb + k) * 4096 : ((size_t)g * kb * 4 + (size_t)k * 4 + t) * 4096;
        return (const u32x4 *)(codes + o + j * 1024 + lane * 16);
    };
    uint32_t acc = 0;
    if (n) {
        u32x4 buf[D][S][4];
#pragma unroll
        for (int d = 0; d < D; d++)
#pragma unroll
            for (int s = 0; s < S; s++)
#pragma unroll
                for (int j = 0; j < 4; j++) buf[d][s][j] = __builtin_nontemporal_load(addr(s, k0 + min((uint32_t)d, n - 1), j));
        for (uint32_t i = 0; i < n; i += D) {
#pragma unroll
            for (int d = 0; d < D; d++)
#pragma unroll
                for (int s = 0; s < S; s++)
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        if (i + d < n) acc += buf[d][s][j].x ^ buf[d][s][j].w;
                        buf[d][s][j] = __builtin_nontemporal_load(addr(s, k0 + min(i + d + D, n - 1), j));
                    }
        }
    }
    if (lane == 0) out[blockIdx.x * W + wv] = (float)acc;
}

// ---- decode layer step of raw reads, with the next weight's first blocks
// fetched ahead on a second stream (step) ------------------------------------
// prefetch_head<D>: for every 32-row sub-tile and each of the four
// wavefront K ranges of the row-split decomposition, the first D K blocks
// (what a read_tiles launch on the same weight loads first), with plain
// loads so they stay in the caches; grid-stride over (sub-tile, range).
template <int D>
__global__ __launch_bounds__(256) void prefetch_head(const uint8_t *codes, uint32_t kb, uint32_t subs, float *out) {
    const uint32_t lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    uint32_t acc = 0;
    for (uint32_t u = blockIdx.x * 4 + wv; u < subs * 4; u += gridDim.x * 4) {
        const uint32_t sub = u >> 2, w = u & 3, g = sub >> 2, t = sub & 3;
        const uint32_t k0 = w * kb / 4, n = (w + 1) * kb / 4 - k0;
        u32x4 v[D][4];
#pragma unroll
        for (int d = 0; d < D; d++)
#pragma unroll
            for (int j = 0; j < 4; j++)
                v[d][j] = *(const u32x4 *)(codes + ((size_t)g * kb * 4 + (size_t)(k0 + min((uint32_t)d, n - 1)) * 4 + t) * 4096 +
                                           j * 1024 + lane * 16);
#pragma unroll
        for (int d = 0; d < D; d++)
#pragma unroll
            for (int j = 0; j < 4; j++) acc += v[d][j].x ^ v[d][j].w;
    }
    if (lane == 0) out[blockIdx.x * 4 + wv] = (float)acc;
}

// ---- read: one contiguous stream -------------------------------------------
__global__ __launch_bounds__(256) void read_linear(const uint8_t *codes, size_t bytes, float *out) {
    const uint32_t lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const uint64_t L = bytes / 1024;
    const uint64_t l0 = (uint64_t)blockIdx.x * L / gridDim.x, l1 = (uint64_t)(blockIdx.x + 1) * L / gridDim.x;
    const uint64_t w0 = l0 + wv * (l1 - l0) / 4, w1 = l0 + (wv + 1) * (l1 - l0) / 4;
    uint32_t acc = 0;
    if (w1 > w0) {
        const uint32_t n = (uint32_t)(w1 - w0);
        const uint8_t *b = codes + w0 * 1024 + lane * 16;
        constexpr int D = 8;
        u32x4 buf[D];
#pragma unroll
        for (int d = 0; d < D; d++) buf[d] = __builtin_nontemporal_load((const u32x4 *)(b + (size_t)min((uint32_t)d, n - 1) * 1024));
        for (uint32_t i = 0; i < n; i += D) {
#pragma unroll
            for (int d = 0; d < D; d++) {
                if (i + d < n) acc += buf[d].x ^ buf[d].w;
                buf[d] = __builtin_nontemporal_load((const u32x4 *)(b + (size_t)min(i + d + D, n - 1) * 1024));
            }
        }
    }
    if (lane == 0) out[blockIdx.x * 4 + wv] = (float)acc;
}

// ---- MFMA issue rate ------------------------------------------------------
__global__ __launch_bounds__(256) void mfma_rate(uint32_t iters, float *out, uint64_t *clocks) {
    const uint32_t lane = threadIdx.x & 63;
    bf16x8 a, b;
    for (int i = 0; i < 8; i++) {
        a[i] = (__bf16)(float)((lane + i) & 7);
        b[i] = (__bf16)(float)((lane * 3 + i) & 7);
    }
    f32x16 acc[8] = {};
    const uint64_t t0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
    for (uint32_t it = 0; it < iters; it++) {
#pragma unroll
        for (int c = 0; c < 8; c++) acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc[c], 0, 0, 0);
    }
    const uint64_t t1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
    float s = 0.0f;
    for (int c = 0; c < 8; c++) s += acc[c][lane & 15];
    out[blockIdx.x * 256 + threadIdx.x] = s;
    if (threadIdx.x == 0) {
        clocks[blockIdx.x * 2] = t1 - t0;
        clocks[blockIdx.x * 2 + 1] = r1 - r0;
    }
}

// ---- MFMA issue rate on data that changes -------------------------------------
// As mfma_rate, but each MFMA takes one of 8 A and 8 B operand sets of
// pseudo-random finite bf16 values (random signs, exponents within 2^-8..2^8,
// random mantissas), so the matrix datapath toggles as it does on real
// activations and weights.  The clock the chip holds then can lie well below
// the one it holds on near-constant operands.
template <bool E4M3B>
__global__ __launch_bounds__(256) void mfma_rand(uint32_t iters, uint32_t seed, float *out, uint64_t *clocks) {
    const uint32_t lane = threadIdx.x & 63;
    u32x4 av[8], bv[8];
    uint32_t h = seed ^ (blockIdx.x * 0x9e3779b9u) ^ (threadIdx.x * 0x85ebca6bu);
    // wide: exponents 2^-8..2^7, 7 random mantissa bits; e4m3: a code's value
    // (3 mantissa bits, exponents 2^-6..2^8) as the GEMM's widened weights are
    auto rnd_bf16x2 = [&](bool e4m3) {
        uint32_t r = 0;
        for (int k = 0; k < 2; k++) {
            h ^= h << 13; h ^= h >> 17; h ^= h << 5;
            const uint32_t sign = (h >> 31) & 1, ex = (e4m3 ? 121 : 119) + ((h >> 20) & 15) % (e4m3 ? 15 : 16),
                           man = e4m3 ? (h & 0x70) : (h & 127);
            r |= ((sign << 15) | (ex << 7) | man) << (16 * k);
        }
        return r;
    };
    for (int c = 0; c < 8; c++)
        for (int j = 0; j < 4; j++) {
            av[c][j] = rnd_bf16x2(false);
            bv[c][j] = rnd_bf16x2(E4M3B);
        }
    f32x16 acc[8] = {};
    __syncthreads();
    const uint64_t t0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
    // eight iterations per trip (iters is a multiple of 8), so every operand
    // index is a compile-time constant: a B index depending on the loop
    // counter compiles to s_set_gpr_idx and four v_mov per MFMA
    for (uint32_t it = 0; it < iters; it += 8) {
#pragma unroll
        for (int u = 0; u < 8; u++)
#pragma unroll
            for (int c = 0; c < 8; c++)
                acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, av[c]),
                                                                   __builtin_bit_cast(bf16x8, bv[(c + u) & 7]), acc[c],
                                                                   0, 0, 0);
    }
    __syncthreads();
    const uint64_t t1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
    float s = 0.0f;
    for (int c = 0; c < 8; c++) s += acc[c][lane & 15];
    out[blockIdx.x * 256 + threadIdx.x] = s;
    if (threadIdx.x == 0) {
        clocks[blockIdx.x * 2] = t1 - t0;
        clocks[blockIdx.x * 2 + 1] = r1 - r0;
    }
}

// ---- MFMA issue order on operands that change (mfma_order) ----------------
// The prefill GEMM's operand pattern for one 32-column chunk of a 128 x 64
// wavefront tile: A tiles i < 4 and B tiles jn < 2, each in two k-halves q,
// 16 MFMAs on 8 accumulators (acc[4*jn + i] += A[i][q] * B[jn][q]).  Two
// operand sets of random bf16 A and e4m3-valued B alternate chunk by chunk.
// ORD 0 "pairs": accumulator by accumulator, both halves back to back
//   (A and B change at every MFMA);
// ORD 1 "b-hold": q, then jn, then i (B held for four MFMAs, A changes);
// ORD 2 "a-hold": q, then i, then jn (A held for two MFMAs, B alternates).
// Bit-identical orders for the GEMM: each accumulator still adds half 0,
// then half 1.
template <int ORD, int WPS>
__global__ __launch_bounds__(256 * WPS) void mfma_order(uint32_t iters, uint32_t seed, float *out, uint64_t *clocks) {
    const uint32_t lane = threadIdx.x & 63;
    u32x4 av[2][4][2], bv[2][2][2];
    uint32_t h = seed ^ (blockIdx.x * 0x9e3779b9u) ^ (threadIdx.x * 0x85ebca6bu);
    auto rnd_bf16x2 = [&](bool e4m3) {
        uint32_t r = 0;
        for (int k = 0; k < 2; k++) {
            h ^= h << 13; h ^= h >> 17; h ^= h << 5;
            const uint32_t sign = (h >> 31) & 1, ex = (e4m3 ? 121 : 119) + ((h >> 20) & 15) % (e4m3 ? 15 : 16),
                           man = e4m3 ? (h & 0x70) : (h & 127);
            r |= ((sign << 15) | (ex << 7) | man) << (16 * k);
        }
        return r;
    };
    for (int st = 0; st < 2; st++)
        for (int q = 0; q < 2; q++)
            for (int j = 0; j < 4; j++) {
                for (int i = 0; i < 4; i++) av[st][i][q][j] = rnd_bf16x2(false);
                for (int jn = 0; jn < 2; jn++) bv[st][jn][q][j] = rnd_bf16x2(true);
            }
    f32x16 acc[8] = {};
    __syncthreads();
    const uint64_t t0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
    for (uint32_t it = 0; it < iters; it += 2) {
#pragma unroll
        for (int st = 0; st < 2; st++)
#pragma unroll
            for (int t = 0; t < 16; t++) {
                int i, jn, q;
                if (ORD == 0) { const int a = t >> 1; q = t & 1; i = a & 3; jn = a >> 2; }
                else if (ORD == 1) { q = t >> 3; jn = (t >> 2) & 1; i = t & 3; }
                else { q = t >> 3; i = (t >> 1) & 3; jn = t & 1; }
                acc[4 * jn + i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                    __builtin_bit_cast(bf16x8, av[st][i][q]), __builtin_bit_cast(bf16x8, bv[st][jn][q]),
                    acc[4 * jn + i], 0, 0, 0);
                __builtin_amdgcn_sched_barrier(0);   // keep the order as written
            }
    }
    __syncthreads();
    const uint64_t t1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
    float s = 0.0f;
    for (int c = 0; c < 8; c++) s += acc[c][lane & 15];
    out[blockIdx.x * 256 * WPS + threadIdx.x] = s;
    if (threadIdx.x == 0) {
        clocks[blockIdx.x * 2] = t1 - t0;
        clocks[blockIdx.x * 2 + 1] = r1 - r0;
    }
}

// ---- launch gap (launch) -----------------------------------------------------
// Back-to-back launches of a kernel that does nothing (one store per
// workgroup, so it is not optimised away), on one stream and as a captured
// graph: what one more launch in a sequence of dependent launches costs.
__global__ __launch_bounds__(256) void empty_kernel(float *out) {
    if (threadIdx.x == 0 && out) out[blockIdx.x] = 0.0f;
}

// ---- MFMA issue rate with VALU work beside it ------------------------------
// WPS wavefronts per SIMD, each running 8 accumulators of
// v_mfma_f32_32x32x16_bf16 with, after every MFMA:
//   MUL 1: two v_mul_f32 on an accumulator two MFMAs old (the GEMM's per-K-block
//          rescale, spread evenly: 2 per MFMA);
//   MUL 2: the same work in bursts: all 16 values of one accumulator after
//          every eighth MFMA;
//   CVT c: c v_cvt_scalef32_pk_bf16_fp8 building the B operand of the next
//          group of four MFMAs (1 per MFMA = the GEMM's e4m3 -> bf16 widening
//          for 128 x 64 wavefront tiles); CVT 8: eight after every eighth MFMA.
// ORD 0 interleaves the accumulators (c = 0..7, each two MFMAs apart from
// nothing it depends on); ORD 1 issues each accumulator's MFMAs in pairs
// back to back (a dependent MFMA right after the one it accumulates onto).
// Cycles are the workgroup's (barriers around the timed loop) per MFMA per
// SIMD: 32 means the VALU work hides entirely.
template <int WPS, int MUL, int CVT, int ORD>
__global__ __launch_bounds__(256 * WPS, 2) void mfma_mix(uint32_t iters, float r, float *out, uint64_t *clocks) {
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    const uint32_t lane = threadIdx.x & 63;
    bf16x8 a;
    u32x4 bw[2];
    for (int i = 0; i < 8; i++) a[i] = (__bf16)(float)((lane + i) & 7);
    for (int j = 0; j < 4; j++) {
        bw[0][j] = 0x3f803f80u + lane;
        bw[1][j] = 0x3f803f80u + lane * 3;
    }
    const uint32_t codes = 0x38383838u ^ (lane << 8);
    uint32_t side = 0;
    f32x16 acc[8] = {};
    __syncthreads();
    const uint64_t t0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
    for (uint32_t it = 0; it < iters; it++) {
#pragma unroll
        for (int u = 0; u < 8; u++)   // eight rounds unrolled: static element indices
#pragma unroll
            for (int c = 0; c < 8; c++) {
                const int ac = ORD ? ((c >> 1) + 4 * (u & 1)) : c;   // ORD 1: pairs on one accumulator
                acc[ac] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, __builtin_bit_cast(bf16x8, bw[c >> 2]),
                                                                    acc[ac], 0, 0, 0);
                if constexpr (MUL == 1) {
                    const int e = (2 * u) & 15;
                    const int t = ORD ? ((((c >> 1) + 2) & 3) + 4 * (u & 1)) : ((c + 6) & 7);
                    acc[t][e] *= r;
                    acc[t][e + 1] *= r;
                } else if constexpr (MUL == 2) {
                    if (c == 1) acc[ORD ? (3 + 4 * (u & 1)) : 7] *= r;
                }
                if constexpr (CVT == 8) {
                    if (c == 1) {
#pragma unroll
                        for (int k = 0; k < 8; k++) {
                            const uint32_t w = codes ^ (it * 64 + u * 8 + k);
                            const bf16x2 v = (k & 1) ? __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, true)
                                                     : __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, false);
                            if (k < 4)
                                bw[1][k] = __builtin_bit_cast(uint32_t, v);
                            else
                                side ^= __builtin_bit_cast(uint32_t, v);
                        }
                    }
                } else {
#pragma unroll
                    for (int k = 0; k < CVT; k++) {
                        const uint32_t w = codes ^ (it * 64 + u * 8 + c);
                        const bf16x2 v = (k & 1) ? __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, true)
                                                 : __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, false);
                        if (k == 0)
                            bw[(c >> 2) ^ 1][c & 3] = __builtin_bit_cast(uint32_t, v);
                        else
                            side ^= __builtin_bit_cast(uint32_t, v);
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
            }
    }
    __syncthreads();
    const uint64_t t1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
    float s = (float)side;
    for (int c = 0; c < 8; c++) s += acc[c][lane & 15];
    out[blockIdx.x * 256 * WPS + threadIdx.x] = s;
    if (threadIdx.x == 0) {
        clocks[blockIdx.x * 2] = t1 - t0;
        clocks[blockIdx.x * 2 + 1] = r1 - r0;
    }
}

// ---- LDS read rate -------------------------------------------------------
__global__ __launch_bounds__(512) void lds_rate(uint32_t iters, float *out, uint64_t *clocks) {
    __shared__ __align__(16) uint8_t buf[64 * 1024];
    const uint32_t lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    for (uint32_t i = threadIdx.x; i < 64 * 1024 / 16; i += 512)
        reinterpret_cast<u32x4 *>(buf)[i] = u32x4{i, i * 3u, i * 5u, i * 7u};
    __syncthreads();
    u32x4 acc = {0, 0, 0, 0};
    const uint64_t t0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
    for (uint32_t it = 0; it < iters; it++) {
        u32x4 v[8];
#pragma unroll
        for (int j = 0; j < 8; j++)   // rows (it*8 + j + wv) % 64 of 1 KiB: always inside buf
            v[j] = *reinterpret_cast<const u32x4 *>(buf + ((it * 8 + j + wv) & 63) * 1024 + lane * 16);
#pragma unroll
        for (int j = 0; j < 8; j++) acc ^= v[j];
    }
    const uint64_t t1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
    out[blockIdx.x * 512 + threadIdx.x] = (float)(acc.x ^ acc.y ^ acc.z ^ acc.w);
    if (threadIdx.x == 0) {
        clocks[blockIdx.x * 2] = t1 - t0;
        clocks[blockIdx.x * 2 + 1] = r1 - r0;
    }
}

static float time_ms(hipEvent_t a, hipEvent_t b) {
    float ms = 0.0f;
    CK(hipEventElapsedTime(&ms, a, b));
    return ms;
}

static int run_read(size_t pool_mb) {
    struct Shape { const char *name; uint32_t k, n; };
    const Shape shapes[] = {{"qkv 5120->6144", 5120, 6144},     {"o_proj 4096->5120", 4096, 5120},
                            {"gate+up 5120->34816", 5120, 34816}, {"down 17408->5120", 17408, 5120},
                            {"single 5120->5120", 5120, 5120}};
    float *out;
    CK(hipMalloc(&out, 1 << 20));
    hipEvent_t e0, e1;
    CK(hipEventCreate(&e0));
    CK(hipEventCreate(&e1));
    hipStream_t gst;
    CK(hipStreamCreate(&gst));
    for (const Shape &sh : shapes) {
        const uint32_t nb = (sh.n + 127) / 128, kb = (sh.k + 127) / 128;
        const size_t bytes = (size_t)nb * kb * 16384;
        const int copies = std::max<int>(4, (int)(pool_mb * 1000000 / bytes));
        uint8_t *pool;
        CK(hipMalloc(&pool, bytes * copies));
        CK(hipMemset(pool, 0x35, bytes * copies));
        const uint32_t subs = (sh.n + 31) / 32;
        static const char *const vname[] = {"tiles/2", "tiles/3", "linear", "sm/2", "g2w4/2", "g2w8/2", "g4w8/2",
                                            "g4w16/2", "g2w4sm/2", "t2+400nop", "t2+1600nop", "t3+64nop/blk",
                                            "t3+256nop/blk"};
        const int nvar = getenv("Q35MM_PROBE_READ_PAD") ? 13 : 9;
        for (int variant = 0; variant < nvar; variant++) {
            if (nvar == 13 && variant > 1 && variant < 9) continue;
            if (variant >= 4 && subs % 4) continue;
            auto launch_on = [&](int i, hipStream_t s) {
                const uint8_t *c = pool + (size_t)(i % copies) * bytes;
                if (variant == 0) hipLaunchKernelGGL(read_tiles<2>, dim3(subs), dim3(256), 0, s, c, kb, out);
                else if (variant == 1) hipLaunchKernelGGL(read_tiles<3>, dim3(subs), dim3(256), 0, s, c, kb, out);
                else if (variant == 2) hipLaunchKernelGGL(read_linear, dim3(256), dim3(256), 0, s, c, bytes, out);
                else if (variant == 3) hipLaunchKernelGGL((read_group<2, 1, 4, true>), dim3(subs), dim3(256), 0, s, c, kb, out);
                else if (variant == 4) hipLaunchKernelGGL((read_group<2, 2, 4, false>), dim3(subs / 2), dim3(256), 0, s, c, kb, out);
                else if (variant == 5) hipLaunchKernelGGL((read_group<2, 2, 8, false>), dim3(subs / 2), dim3(512), 0, s, c, kb, out);
                else if (variant == 6) hipLaunchKernelGGL((read_group<2, 4, 8, false>), dim3(subs / 4), dim3(512), 0, s, c, kb, out);
                else if (variant == 7) hipLaunchKernelGGL((read_group<2, 4, 16, false>), dim3(subs / 4), dim3(1024), 0, s, c, kb, out);
                else if (variant == 8) hipLaunchKernelGGL((read_group<2, 2, 4, true>), dim3(subs / 2), dim3(256), 0, s, c, kb, out);
                else if (variant == 9) hipLaunchKernelGGL(read_tiles_pad<400>, dim3(subs), dim3(256), 0, s, c, kb, out);
                else if (variant == 10) hipLaunchKernelGGL(read_tiles_pad<1600>, dim3(subs), dim3(256), 0, s, c, kb, out);
                else if (variant == 11) hipLaunchKernelGGL(read_tiles_fat<64>, dim3(subs), dim3(256), 0, s, c, kb, out);
                else hipLaunchKernelGGL(read_tiles_fat<256>, dim3(subs), dim3(256), 0, s, c, kb, out);
            };
            auto launch = [&](int i) { launch_on(i, 0); };
            for (int i = 0; i < 8; i++) launch(i);
            CK(hipDeviceSynchronize());
            const int reps = 200;
            CK(hipEventRecord(e0));
            for (int i = 0; i < reps; i++) launch(i);
            CK(hipEventRecord(e1));
            CK(hipEventSynchronize(e1));
            const double us = time_ms(e0, e1) * 1e3 / reps;
            // the same launches captured once and replayed as a graph (as the
            // benchmark launches its kernels): each launch costs less there
            hipGraph_t g;
            hipGraphExec_t ge;
            CK(hipStreamBeginCapture(gst, hipStreamCaptureModeGlobal));
            for (int i = 0; i < reps; i++) launch_on(i, gst);
            CK(hipStreamEndCapture(gst, &g));
            CK(hipGraphInstantiate(&ge, g, nullptr, nullptr, 0));
            CK(hipGraphLaunch(ge, gst));
            CK(hipStreamSynchronize(gst));
            CK(hipEventRecord(e0, gst));
            CK(hipGraphLaunch(ge, gst));
            CK(hipEventRecord(e1, gst));
            CK(hipEventSynchronize(e1));
            const double us_g = time_ms(e0, e1) * 1e3 / reps;
            CK(hipGraphExecDestroy(ge));
            CK(hipGraphDestroy(g));
            printf("read %-22s %-8s %8.2f us %7.0f GB/s; graph %8.2f us %7.0f GB/s (%zu bytes, %d copies)\n",
                   sh.name, vname[variant], us, bytes / us / 1e3,
                   us_g, bytes / us_g / 1e3, bytes, copies);
            fflush(stdout);
        }
        CK(hipFree(pool));
    }
    return 0;
}

static int run_mfma() {
    const uint32_t blocks = 256, iters = 4096;
    float *out;
    uint64_t *clk;
    CK(hipMalloc(&out, blocks * 256 * sizeof(float)));
    CK(hipMalloc(&clk, blocks * 2 * sizeof(uint64_t)));
    hipEvent_t e0, e1;
    CK(hipEventCreate(&e0));
    CK(hipEventCreate(&e1));
    hipLaunchKernelGGL(mfma_rate, dim3(blocks), dim3(256), 0, 0, 64u, out, clk);
    CK(hipDeviceSynchronize());
    CK(hipEventRecord(e0));
    hipLaunchKernelGGL(mfma_rate, dim3(blocks), dim3(256), 0, 0, iters, out, clk);
    CK(hipEventRecord(e1));
    CK(hipEventSynchronize(e1));
    const double s = time_ms(e0, e1) * 1e-3;
    std::vector<uint64_t> c(blocks * 2);
    CK(hipMemcpy(c.data(), clk, c.size() * sizeof(uint64_t), hipMemcpyDeviceToHost));
    double cyc = 0, real = 0;
    for (uint32_t b = 0; b < blocks; b++) {
        cyc += (double)c[2 * b];
        real += (double)c[2 * b + 1];
    }
    const double mfmas = (double)blocks * 4 * iters * 8;
    const double flops = mfmas * 32 * 32 * 16 * 2;
    const double clock_ghz = cyc / real * 0.1;   // s_memrealtime ticks at 100 MHz
    printf("mfma 32x32x16 bf16: %.1f TFLOP/s over %.3f ms; core clock under load %.2f GHz; "
           "%.1f cycles per MFMA per SIMD\n",
           flops / s / 1e12, s * 1e3, clock_ghz, cyc / blocks / (iters * 8.0));
    return 0;
}

template <int WPS, int MUL, int CVT, int ORD = 0>
static void mix_case(float *out, uint64_t *clk) {
    const uint32_t blocks = 256, iters = 256;   // x 64 MFMAs per wavefront
    hipLaunchKernelGGL((mfma_mix<WPS, MUL, CVT, ORD>), dim3(blocks), dim3(256 * WPS), 0, 0, 8u, 0.999f, out, clk);
    CK(hipDeviceSynchronize());
    hipLaunchKernelGGL((mfma_mix<WPS, MUL, CVT, ORD>), dim3(blocks), dim3(256 * WPS), 0, 0, iters, 0.999f, out,
                       clk);
    CK(hipDeviceSynchronize());
    std::vector<uint64_t> c(blocks * 2);
    CK(hipMemcpy(c.data(), clk, c.size() * sizeof(uint64_t), hipMemcpyDeviceToHost));
    double cyc = 0;
    for (uint32_t b = 0; b < blocks; b++) cyc += (double)c[2 * b];
    cyc /= blocks;
    printf("mix waves/SIMD %d  order %-11s  rescale %-6s  cvt %s:  %.1f cycles per MFMA per SIMD\n", WPS,
           ORD ? "pairs" : "interleaved", MUL == 0 ? "none" : MUL == 1 ? "spread" : "burst",
           CVT == 8 ? "burst 8/8" : CVT == 2 ? "2/MFMA" : CVT == 1 ? "1/MFMA" : "none",
           cyc / (iters * 64.0 * WPS));
}

static int run_mix() {
    float *out;
    uint64_t *clk;
    CK(hipMalloc(&out, 256 * 512 * sizeof(float)));
    CK(hipMalloc(&clk, 256 * 2 * sizeof(uint64_t)));
    mix_case<1, 0, 0>(out, clk);
    mix_case<1, 1, 0>(out, clk);
    mix_case<1, 2, 0>(out, clk);
    mix_case<1, 0, 1>(out, clk);
    mix_case<1, 0, 8>(out, clk);
    mix_case<1, 1, 1>(out, clk);
    mix_case<1, 2, 8>(out, clk);
    mix_case<1, 0, 0, 1>(out, clk);
    mix_case<1, 1, 1, 1>(out, clk);
    mix_case<2, 0, 0>(out, clk);
    mix_case<2, 1, 0>(out, clk);
    mix_case<2, 2, 0>(out, clk);
    mix_case<2, 0, 1>(out, clk);
    mix_case<2, 0, 8>(out, clk);
    mix_case<2, 1, 1>(out, clk);
    mix_case<2, 2, 8>(out, clk);
    mix_case<2, 0, 0, 1>(out, clk);
    mix_case<2, 1, 1, 1>(out, clk);
    return 0;
}

static int run_mfma_rand() {
    const uint32_t blocks = 256;
    float *out;
    uint64_t *clk;
    CK(hipMalloc(&out, blocks * 256 * sizeof(float)));
    CK(hipMalloc(&clk, blocks * 2 * sizeof(uint64_t)));
    hipEvent_t e0, e1;
    CK(hipEventCreate(&e0));
    CK(hipEventCreate(&e1));
    for (int e4m3 = 0; e4m3 < 2; e4m3++)
    for (uint32_t iters : {4096u, 65536u}) {   // ~0.6 ms and ~10 ms of MFMAs
        auto kern = e4m3 ? mfma_rand<true> : mfma_rand<false>;
        hipLaunchKernelGGL(kern, dim3(blocks), dim3(256), 0, 0, 64u, 1u, out, clk);
        CK(hipDeviceSynchronize());
        CK(hipEventRecord(e0));
        hipLaunchKernelGGL(kern, dim3(blocks), dim3(256), 0, 0, iters, 7u, out, clk);
        CK(hipEventRecord(e1));
        CK(hipEventSynchronize(e1));
        const double sec = time_ms(e0, e1) * 1e-3;
        std::vector<uint64_t> c(blocks * 2);
        CK(hipMemcpy(c.data(), clk, c.size() * sizeof(uint64_t), hipMemcpyDeviceToHost));
        double cyc = 0, real = 0;
        for (uint32_t b = 0; b < blocks; b++) {
            cyc += (double)c[2 * b];
            real += (double)c[2 * b + 1];
        }
        const double flops = (double)blocks * 4 * iters * 8 * 32 * 32 * 16 * 2;
        printf("mfma 32x32x16 bf16, random A, %s B: %.1f TFLOP/s over %.3f ms; core clock %.2f GHz; "
               "%.1f cycles per MFMA per SIMD\n", e4m3 ? "e4m3-valued" : "random",
               flops / sec / 1e12, sec * 1e3, cyc / real * 0.1, cyc / blocks / (iters * 8.0));
    }
    return 0;
}

template <int ORD, int WPS>
static void order_case(float *out, uint64_t *clk, hipEvent_t e0, hipEvent_t e1, uint32_t iters) {
    const uint32_t blocks = 256;
    hipLaunchKernelGGL((mfma_order<ORD, WPS>), dim3(blocks), dim3(256 * WPS), 0, 0, 64u, 1u, out, clk);
    CK(hipDeviceSynchronize());
    CK(hipEventRecord(e0));
    hipLaunchKernelGGL((mfma_order<ORD, WPS>), dim3(blocks), dim3(256 * WPS), 0, 0, iters, 7u, out, clk);
    CK(hipEventRecord(e1));
    CK(hipEventSynchronize(e1));
    const double sec = time_ms(e0, e1) * 1e-3;
    std::vector<uint64_t> c(blocks * 2);
    CK(hipMemcpy(c.data(), clk, c.size() * sizeof(uint64_t), hipMemcpyDeviceToHost));
    double cyc = 0, real = 0;
    for (uint32_t b = 0; b < blocks; b++) {
        cyc += (double)c[2 * b];
        real += (double)c[2 * b + 1];
    }
    const double mfmas_per_simd = (double)iters * 16 * WPS;
    const double flops = (double)blocks * 4 * mfmas_per_simd * 32 * 32 * 16 * 2;
    printf("mfma order %-11s waves/SIMD %d: %.1f TFLOP/s over %.3f ms; core clock %.2f GHz; %.1f cycles per MFMA "
           "per SIMD\n", ORD == 0 ? "pairs" : ORD == 1 ? "b-hold" : "a-hold", WPS, flops / sec / 1e12, sec * 1e3,
           cyc / real * 0.1, cyc / blocks / mfmas_per_simd);
    fflush(stdout);
}

static int run_mfma_order() {
    float *out;
    uint64_t *clk;
    CK(hipMalloc(&out, 256 * 512 * sizeof(float)));
    CK(hipMalloc(&clk, 256 * 2 * sizeof(uint64_t)));
    hipEvent_t e0, e1;
    CK(hipEventCreate(&e0));
    CK(hipEventCreate(&e1));
    for (uint32_t iters : {4096u, 32768u}) {   // x 16 MFMAs per wavefront: ~0.6 ms and ~5 ms
        order_case<0, 1>(out, clk, e0, e1, iters);
        order_case<1, 1>(out, clk, e0, e1, iters);
        order_case<2, 1>(out, clk, e0, e1, iters);
        order_case<0, 2>(out, clk, e0, e1, iters / 2);
        order_case<1, 2>(out, clk, e0, e1, iters / 2);
        order_case<2, 2>(out, clk, e0, e1, iters / 2);
    }
    return 0;
}

static int run_launch() {
    float *out;
    CK(hipMalloc(&out, 4096 * sizeof(float)));
    hipStream_t st;
    CK(hipStreamCreate(&st));
    hipEvent_t e0, e1;
    CK(hipEventCreate(&e0));
    CK(hipEventCreate(&e1));
    const int n = 400;
    for (uint32_t blocks : {1u, 256u, 1024u}) {
        for (int i = 0; i < 20; i++) hipLaunchKernelGGL(empty_kernel, dim3(blocks), dim3(256), 0, st, out);
        CK(hipStreamSynchronize(st));
        CK(hipEventRecord(e0, st));
        for (int i = 0; i < n; i++) hipLaunchKernelGGL(empty_kernel, dim3(blocks), dim3(256), 0, st, out);
        CK(hipEventRecord(e1, st));
        CK(hipEventSynchronize(e1));
        const double us_stream = time_ms(e0, e1) * 1e3 / n;
        hipGraph_t g;
        hipGraphExec_t ge;
        CK(hipStreamBeginCapture(st, hipStreamCaptureModeGlobal));
        for (int i = 0; i < n; i++) hipLaunchKernelGGL(empty_kernel, dim3(blocks), dim3(256), 0, st, out);
        CK(hipStreamEndCapture(st, &g));
        CK(hipGraphInstantiate(&ge, g, nullptr, nullptr, 0));
        CK(hipGraphLaunch(ge, st));
        CK(hipStreamSynchronize(st));
        CK(hipEventRecord(e0, st));
        CK(hipGraphLaunch(ge, st));
        CK(hipEventRecord(e1, st));
        CK(hipEventSynchronize(e1));
        const double us_graph = time_ms(e0, e1) * 1e3 / n;
        printf("launch empty kernel, %4u workgroups: %.2f us per launch on a stream, %.2f us in a graph\n", blocks,
               us_stream, us_graph);
        fflush(stdout);
        CK(hipGraphExecDestroy(ge));
        CK(hipGraphDestroy(g));
    }
    return 0;
}

// Host round trip of one launch: launch, then wait for it on the host, as a
// synchronous library call does.  "sync": hipStreamSynchronize; "event":
// hipEventSynchronize on an event recorded after the launch; "flag": the
// kernel's last store goes to pinned host memory and the host spins on it.
__global__ __launch_bounds__(64) void flag_kernel(volatile uint32_t *flag, uint32_t v) {
    if (threadIdx.x == 0) {
        __threadfence_system();
        *flag = v;
    }
}

// The empty kernel whose last workgroup to finish stores the flag: each
// workgroup's thread 0 makes its stores visible system-wide, then counts
// itself in; the last one resets the counter and stores v.
__global__ __launch_bounds__(256) void empty_flag_kernel(float *out, uint32_t *count, uint32_t *flag, uint32_t v) {
    if (threadIdx.x == 0) {
        if (out) out[blockIdx.x] = 0.0f;
        __threadfence_system();
        const uint32_t prev = __hip_atomic_fetch_add(count, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
        if (prev == gridDim.x - 1) {
            __hip_atomic_store(count, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __threadfence_system();
            __hip_atomic_store(flag, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        }
    }
}

static int run_sync(bool spin) {
    if (spin) CK(hipSetDeviceFlags(hipDeviceScheduleSpin));
    hipStream_t st;
    CK(hipStreamCreate(&st));
    float *out;
    CK(hipMalloc(&out, 4096 * sizeof(float)));
    uint32_t *flag;
    CK(hipHostMalloc(&flag, 64, hipHostMallocDefault));
    *flag = 0;
    hipEvent_t ev;
    CK(hipEventCreateWithFlags(&ev, hipEventDisableTiming));
    const int n = 2000;
    // spins give up after a second: a missing store ends the probe, not the box
    auto spin_for = [&](uint32_t v) {
        const auto ts = std::chrono::steady_clock::now();
        for (uint32_t j = 0; __atomic_load_n(flag, __ATOMIC_ACQUIRE) != v; j++) {
            __builtin_ia32_pause();
            if ((j & 1023) == 1023 && std::chrono::steady_clock::now() - ts > std::chrono::seconds(1)) {
                fprintf(stderr, "flag %u never came\n", v);
                exit(1);
            }
        }
    };
    uint32_t *count;
    CK(hipMalloc(&count, 64));
    CK(hipMemset(count, 0, 64));
    CK(hipDeviceSynchronize());
    for (int mode = 0; mode < 6; mode++) {
        double best = 1e30;
        for (int rep = 0; rep < 3; rep++) {
            auto t0 = std::chrono::steady_clock::now();
            for (int i = 0; i < n; i++) {
                const uint32_t v = (uint32_t)(mode * 3 * n + rep * n + i + 1);
                if (mode == 2) {
                    hipLaunchKernelGGL(flag_kernel, dim3(1), dim3(64), 0, st, (volatile uint32_t *)flag, v);
                    spin_for(v);
                } else if (mode == 3) {
                    hipLaunchKernelGGL(empty_kernel, dim3(160), dim3(256), 0, st, out);
                    hipLaunchKernelGGL(flag_kernel, dim3(1), dim3(64), 0, st, (volatile uint32_t *)flag, v);
                    spin_for(v);
                } else if (mode == 5) {
                    hipLaunchKernelGGL(empty_flag_kernel, dim3(160), dim3(256), 0, st, out, count, flag, v);
                    spin_for(v);
                } else if (mode == 4) {
                    hipLaunchKernelGGL(empty_kernel, dim3(160), dim3(256), 0, st, out);
                    CK(hipStreamWriteValue32(st, flag, v, 0));
                    spin_for(v);
                } else {
                    hipLaunchKernelGGL(empty_kernel, dim3(160), dim3(256), 0, st, out);
                    if (mode == 0) {
                        CK(hipStreamSynchronize(st));
                    } else {
                        CK(hipEventRecord(ev, st));
                        CK(hipEventSynchronize(ev));
                    }
                }
            }
            CK(hipStreamSynchronize(st));
            const double us = std::chrono::duration<double, std::micro>(std::chrono::steady_clock::now() - t0).count() / n;
            best = std::min(best, us);
        }
        printf("host round trip (%s scheduling), %s: %.2f us\n", spin ? "spin" : "default",
               mode == 0   ? "launch + hipStreamSynchronize"
               : mode == 1 ? "launch + hipEventSynchronize"
               : mode == 2 ? "flag-kernel launch + spin on the pinned flag"
               : mode == 3 ? "launch + flag-kernel launch + spin"
               : mode == 4 ? "launch + hipStreamWriteValue32 of the flag + spin"
                           : "launch of a kernel whose last workgroup stores the flag + spin",
               best);
        fflush(stdout);
    }
    return 0;
}

// Decode layer step of raw reads (qkv, o_proj, gate+up, down) over 8 layer
// copies, 64 steps replayed as a graph.  PF = 0: reads only; PF = D > 0:
// before each read, a prefetch_head<D> of the next launch's weight on a
// second stream, depending (like the read) on the previous read only, so
// the two run at the same time; REREAD: every weight read twice in a row
// (the second read finds what the caches kept).
static int run_step() {
    struct Shape { uint32_t k, n; int depth; };
    const Shape shapes[] = {{5120, 6144, 2}, {4096, 5120, 2}, {5120, 34816, 2}, {17408, 5120, 3}};
    const int layers = 8, steps = 64;
    std::vector<uint8_t *> w(layers * 4);
    size_t step_bytes = 0;
    for (int s = 0; s < 4; s++) step_bytes += (size_t)(shapes[s].n / 128) * (shapes[s].k / 128) * 16384;
    for (int l = 0; l < layers; l++)
        for (int s = 0; s < 4; s++) {
            const size_t b = (size_t)(shapes[s].n / 128) * (shapes[s].k / 128) * 16384;
            CK(hipMalloc(&w[l * 4 + s], b));
            CK(hipMemset(w[l * 4 + s], 0x35, b));
        }
    float *out, *out2;
    CK(hipMalloc(&out, 1 << 20));
    CK(hipMalloc(&out2, 1 << 20));
    hipStream_t a, b;
    CK(hipStreamCreate(&a));
    CK(hipStreamCreate(&b));
    const int nev = steps * 4 + 1;
    std::vector<hipEvent_t> ev(nev), evb(1);
    for (auto &e : ev) CK(hipEventCreateWithFlags(&e, hipEventDisableTiming));
    CK(hipEventCreateWithFlags(&evb[0], hipEventDisableTiming));
    hipEvent_t t0, t1;
    CK(hipEventCreate(&t0));
    CK(hipEventCreate(&t1));
    auto read = [&](int i, hipStream_t st) {
        const int s = i % 4, l = (i / 4) % layers;
        const uint32_t kb = shapes[s].k / 128, subs = shapes[s].n / 32;
        if (shapes[s].depth == 3)
            hipLaunchKernelGGL(read_tiles<3>, dim3(subs), dim3(256), 0, st, w[l * 4 + s], kb, out);
        else
            hipLaunchKernelGGL(read_tiles<2>, dim3(subs), dim3(256), 0, st, w[l * 4 + s], kb, out);
    };
    auto prefetch = [&](int i, int D, uint32_t grid, hipStream_t st) {
        const int s = i % 4, l = (i / 4) % layers;
        const uint32_t kb = shapes[s].k / 128, subs = shapes[s].n / 32;
        if (D == 1) hipLaunchKernelGGL(prefetch_head<1>, dim3(grid), dim3(256), 0, st, w[l * 4 + s], kb, subs, out2);
        else if (D == 2) hipLaunchKernelGGL(prefetch_head<2>, dim3(grid), dim3(256), 0, st, w[l * 4 + s], kb, subs, out2);
        else hipLaunchKernelGGL(prefetch_head<4>, dim3(grid), dim3(256), 0, st, w[l * 4 + s], kb, subs, out2);
    };
    struct Case { const char *name; int pf; uint32_t grid; bool reread; };
    const Case cases[] = {{"reads only", 0, 0, false},          {"reads, each twice", 0, 0, true},
                          {"prefetch 1 block, 64 wg", 1, 64, false}, {"prefetch 2 blocks, 64 wg", 2, 64, false},
                          {"prefetch 2 blocks, 128 wg", 2, 128, false}, {"prefetch 4 blocks, 64 wg", 4, 64, false},
                          {"reads only", 0, 0, false}};
    for (const Case &c : cases) {
        hipGraph_t g;
        hipGraphExec_t ge;
        CK(hipStreamBeginCapture(a, hipStreamCaptureModeGlobal));
        const int n = steps * 4;
        for (int i = 0; i < n; i++) {
            if (c.pf && i + 1 < n) {
                // the prefetch of launch i+1 waits for launch i-1, as launch i does
                if (i > 0) CK(hipStreamWaitEvent(b, ev[i - 1], 0));
                else {
                    CK(hipEventRecord(evb[0], a));
                    CK(hipStreamWaitEvent(b, evb[0], 0));
                }
                prefetch(i + 1, c.pf, c.grid, b);
            }
            read(i, a);
            if (c.reread) read(i, a);
            CK(hipEventRecord(ev[i], a));
        }
        if (c.pf) {
            CK(hipEventRecord(ev[n], b));
            CK(hipStreamWaitEvent(a, ev[n], 0));
        }
        CK(hipStreamEndCapture(a, &g));
        CK(hipGraphInstantiate(&ge, g, nullptr, nullptr, 0));
        CK(hipGraphLaunch(ge, a));
        CK(hipStreamSynchronize(a));
        double best = 1e30;
        for (int r = 0; r < 3; r++) {
            CK(hipEventRecord(t0, a));
            CK(hipGraphLaunch(ge, a));
            CK(hipEventRecord(t1, a));
            CK(hipEventSynchronize(t1));
            best = std::min(best, (double)time_ms(t0, t1) * 1e3 / steps);
        }
        printf("step of raw reads, %-26s %7.2f us per step  %6.0f GB/s\n", c.name, best,
               step_bytes * (c.reread ? 2 : 1) / best / 1e3);
        fflush(stdout);
        CK(hipGraphExecDestroy(ge));
        CK(hipGraphDestroy(g));
    }
    return 0;
}

// One decode layer step of raw reads with timestamps (after 16 warm-up
// steps, launched back to back on one stream): per launch, the spread of
// workgroup starts, time to the first block, end spread, gaps.
static int run_stampread() {
    struct Shape { const char *name; uint32_t k, n; int depth; };
    const Shape shapes[] = {{"qkv", 5120, 6144, 2}, {"o_proj", 4096, 5120, 2}, {"gate+up", 5120, 34816, 2},
                            {"down", 17408, 5120, 3}};
    const int layers = 8;
    std::vector<uint8_t *> w(layers * 4);
    for (int l = 0; l < layers; l++)
        for (int s = 0; s < 4; s++) {
            const size_t b = (size_t)(shapes[s].n / 128) * (shapes[s].k / 128) * 16384;
            CK(hipMalloc(&w[l * 4 + s], b));
            CK(hipMemset(w[l * 4 + s], 0x35, b));
        }
    float *out;
    CK(hipMalloc(&out, 1 << 20));
    uint32_t *st[4];
    for (int s = 0; s < 4; s++) CK(hipMalloc(&st[s], 3 * 1088 * sizeof(uint32_t)));
    for (int it = 0; it < 17; it++)
        for (int s = 0; s < 4; s++) {
            const uint32_t kb = shapes[s].k / 128, subs = shapes[s].n / 32;
            const uint8_t *c = w[(it % layers) * 4 + s];
            if (shapes[s].depth == 3) hipLaunchKernelGGL(read_tiles_st<3>, dim3(subs), dim3(256), 0, 0, c, kb, out, st[s]);
            else hipLaunchKernelGGL(read_tiles_st<2>, dim3(subs), dim3(256), 0, 0, c, kb, out, st[s]);
        }
    CK(hipDeviceSynchronize());
    std::vector<std::vector<uint32_t>> h(4);
    uint64_t base = ~0ull;
    for (int s = 0; s < 4; s++) {
        const uint32_t subs = shapes[s].n / 32;
        h[s].resize(3 * subs);
        CK(hipMemcpy(h[s].data(), st[s], 3 * subs * sizeof(uint32_t), hipMemcpyDeviceToHost));
        for (uint32_t i = 0; i < subs; i++) base = std::min<uint64_t>(base, h[s][3 * i]);
    }
    for (int s = 0; s < 4; s++) {
        const uint32_t subs = shapes[s].n / 32;
        std::vector<double> a(subs), f(subs), e(subs);
        for (uint32_t i = 0; i < subs; i++) {
            a[i] = (h[s][3 * i] - base) * 10.0;
            f[i] = (h[s][3 * i + 1] - (double)h[s][3 * i]) * 10.0;
            e[i] = (h[s][3 * i + 2] - base) * 10.0;
        }
        std::vector<double> fs = f;
        std::sort(fs.begin(), fs.end());
        printf("raw %-8s start %6.0f..%6.0f ns  first block med %5.0f max %5.0f  end %6.0f..%6.0f ns\n", shapes[s].name,
               *std::min_element(a.begin(), a.end()), *std::max_element(a.begin(), a.end()), fs[subs / 2], fs.back(),
               *std::min_element(e.begin(), e.end()), *std::max_element(e.begin(), e.end()));
    }
    return 0;
}

static int run_lds() {
    const uint32_t blocks = 256, iters = 4096;
    float *out;
    uint64_t *clk;
    CK(hipMalloc(&out, blocks * 512 * sizeof(float)));
    CK(hipMalloc(&clk, blocks * 2 * sizeof(uint64_t)));
    hipLaunchKernelGGL(lds_rate, dim3(blocks), dim3(512), 0, 0, 64u, out, clk);
    CK(hipDeviceSynchronize());
    hipLaunchKernelGGL(lds_rate, dim3(blocks), dim3(512), 0, 0, iters, out, clk);
    CK(hipDeviceSynchronize());
    std::vector<uint64_t> c(blocks * 2);
    CK(hipMemcpy(c.data(), clk, c.size() * sizeof(uint64_t), hipMemcpyDeviceToHost));
    double cyc = 0, real = 0;
    for (uint32_t b = 0; b < blocks; b++) {
        cyc += (double)c[2 * b];
        real += (double)c[2 * b + 1];
    }
    cyc /= blocks;
    real /= blocks;
    const double bytes_per_cu = 8.0 * iters * 8 * 1024;   // 8 wavefronts x iters x 8 reads x 1 KiB
    printf("lds ds_read_b128: %.1f bytes per clock per CU (%.0f cycles per workgroup, core clock %.2f GHz)\n",
           bytes_per_cu / cyc, cyc, cyc / real * 0.1);
    return 0;
}

int main(int argc, char **argv) {
    if (argc >= 2 && !strcmp(argv[1], "read")) return run_read(argc >= 3 ? strtoul(argv[2], nullptr, 10) : 1536);
    if (argc >= 2 && !strcmp(argv[1], "mfma")) return run_mfma();
    if (argc >= 2 && !strcmp(argv[1], "lds")) return run_lds();
    if (argc >= 2 && !strcmp(argv[1], "mix")) return run_mix();
    if (argc >= 2 && !strcmp(argv[1], "mfma_rand")) return run_mfma_rand();
    if (argc >= 2 && !strcmp(argv[1], "mfma_order")) return run_mfma_order();
    if (argc >= 2 && !strcmp(argv[1], "launch")) return run_launch();
    if (argc >= 2 && !strcmp(argv[1], "step")) return run_step();
    if (argc >= 2 && !strcmp(argv[1], "stampread")) return run_stampread();
    if (argc >= 2 && !strcmp(argv[1], "sync")) return run_sync(argc >= 3 && !strcmp(argv[2], "spin"));
    fprintf(stderr, "usage: %s read [pool_MB] | lds | mfma | mfma_rand | mfma_order | mix | launch | sync [spin] | step | stampread\n", argv[0]);
    return 2;
}
