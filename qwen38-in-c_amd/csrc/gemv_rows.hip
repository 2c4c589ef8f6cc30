// gemv_rows.hip -- decode GEMV, m <= 8 tokens, row-split decomposition for
// weights of at least a few thousand rows and a moderate K.
//
// Replaces the same hot loop as gemv_fp8.hip (qwen35-c/src/q35_mm.c:88-198,
// mm_fp8_row under q35_mm_fp8 / q35_mm_fp8_batch / q35_mm_fp8_multi4) for
// the shapes gemv_rows_shape() selects, e.g. 5120->6144, 4096->5120,
// 5120->17408 and 17408->5120.
//
// Decomposition.  Each workgroup owns a range of at most 32 consecutive
// rows of one weight, and its NW (4 or 8) wavefronts split K into
// contiguous ranges of K blocks.  Each wavefront streams its K range of
// those rows (lane l loads row r0 + l%32 of the lane-order tiles, 16 bytes
// per 32-column chunk) through a ring of DEPTH blocks; the wavefront
// partials are added through LDS in wavefront order at the end.  No partial
// output leaves the workgroup, so there are no tickets, no workspace and no
// second pass: that is the whole point against stream-K, whose split-group
// protocol costs a few microseconds per launch, as much as streaming these
// weights takes.
//
// Ranges (gemv_rows_plan).  One workgroup per 32-row sub-tile, whatever
// the launch's size: each load is a whole 1 KiB chunk, which the memory
// system streams fastest (a raw-read probe of 5120 x 17408 codes: 15.2 us as
// sub-tiles on 160 CUs against 17.5 us as 256 ranges of 20 rows, whose
// loads read 320-byte pieces of each chunk).  A small launch leaves most
// CUs idle that way and is still no slower than spreading its rows over
// every CU in ranges of 4 rows: 1024 x 5120 6.05 against 6.48 us, 256 x
// 17408 14.0 against 14.3 us; such a launch is bound by each wavefront's
// chain of K blocks (about 0.35 us of instructions per block at one
// wavefront per SIMD), not by how many CUs stream.

// Arithmetic is the stream-K kernel's: e4m3 -> bf16 exactly, activations
// split exactly into three bf16 parts (A-operand rows m = token + 8*part),
// v_mfma_f32_32x32x16_bf16 per K block (weight row r0 + n is MFMA column
// n), the block's fp32 scale applied with one fmaf per output.  A row's
// summation order depends only on K (K ranges per wavefront, wavefronts in
// order), not on which range holds it, so a batch of m tokens gives exactly
// the bits of m single-token calls, and a weight gives the same bits alone
// or in a multi-weight launch.
//
// Activations.  Each K block's activations ride the weight ring one block
// ahead: the slot that brings the weights of block b brings the activations
// of block b+1, which are split into the wavefront's second A-operand slot
// in LDS while block b's MFMAs run.  Nothing is staged up front and no
// barrier is needed before the stream: each wavefront only reads LDS it
// wrote itself (LDS operations of one wavefront complete in order).
#include <algorithm>

#include "gemv_rows_common.h"
#include "q35mm_device.h"
#include "q35mm_internal.h"

namespace q35mm {

using namespace rows;

namespace {

// K blocks in flight per wavefront (the ring depth DEPTH), chosen by the
// host from m and the launch's workgroup count; the summation order does
// not depend on it, so results stay those of any other depth.
// Three for a launch of one round of workgroups at m <= 2; two (fewer
// registers: four wavefronts per SIMD instead of three) for launches of
// several rounds, where more resident workgroups hide the latency, and for
// m > 2, where each block's larger split hides it.  Layer step at m = 1 /
// 4 / 8 against four blocks everywhere: +6% / +10% / +19%.
constexpr uint32_t kRsDepthShort = 2, kRsDepthLong = 3;

// Wavefronts per SIMD the register allocator must leave room for: four
// (128 registers, accumulators included) for one token on a ring of two
// blocks -- the gate+up launch, several rounds of workgroups -- which the
// plain kernel fits; the rest as many as their registers allow.
constexpr uint32_t rows_min_waves(uint32_t mt, uint32_t depth, uint32_t nw) {
    return mt == 1 && depth == 2 && nw == 4 ? 4 : 1;
}

}  // namespace

// MT = m rounded up to a power of two; DEPTH = ring depth; NW = wavefronts.
// MODE: kRowsPlain -- rows of up to four weights, y (+ resid) per segment;
// kRowsPair -- the MLP's gate (segment 0) and up (segment 1) together,
// writing silu(gate) * up; kRowsPairNorm -- the same on RMSNorm(x).
template <bool VEC, uint32_t MT, uint32_t DEPTH, uint32_t NW, uint32_t MODE = kRowsPlain>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(rows_min_waves(MT, DEPTH, NW), 8)))
void gemv_rows_kernel(GemvParams p) {
    constexpr bool PAIR = MODE != kRowsPlain, NORM = MODE == kRowsPairNorm;
    static_assert(!NORM || MT == 1, "the fused RMSNorm is for one token");
    extern __shared__ __align__(16) uint8_t lds[];
    __shared__ float red[NW][kGemvMaxM][kSubRows];

    uint32_t si = 0;
    if constexpr (!PAIR) {
#pragma unroll
        for (uint32_t i = 1; i < 4; i++)
            if (i < p.nseg && blockIdx.x >= p.seg[i].cta_begin) si = i;
    }
    const GemvSeg &sg = p.seg[si];
    // Rows [r0, r1) of the segment: workgroup c owns sub-tile c.  Pair
    // mode: workgroup c owns rows [16c, 16c + 16) of both weights; MFMA
    // column n < 16 is gate row 16c + n, column 16 + n up row 16c + n, so
    // silu(gate) * up is formed from the workgroup's own sums.
    const uint32_t c = blockIdx.x - sg.cta_begin;
    const uint32_t unit = PAIR ? kPairRows : kSubRows;
    const uint32_t r0 = c * unit, r1 = min(r0 + unit, sg.rows);
    const uint32_t KB = p.kb, M = p.m, R = stage_rows(M);

    const uint32_t lane = threadIdx.x & 63;
    const uint32_t wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // K blocks of this wavefront: kbof(i) = k0 + i for i < n (KB >= waves).
    // (Interleaving the wavefronts over K instead measured the same.)
    const uint32_t k0 = wv * KB / NW, n = (wv + 1) * KB / NW - k0;
    auto kbof = [&](uint32_t i) { return k0 + i; };

    // This wavefront's LDS: two A-operand slots and a 16-byte zero slot.
    // Lanes whose A row carries no token (t >= m, or rows 24..31) read the
    // zero slot, so every lane issues the same LDS reads.
    uint8_t *const wbase = lds + wv * gemv_rows_wave_lds(M);
    const uint32_t mrow = lane & 31, hh = lane >> 5;
    const uint32_t tt = mrow & 7, pp = mrow >> 3;
    const bool a_active = tt < M && pp < 3;
    const uint8_t *const arow = a_active ? wbase + ((pp * M + tt) * 2 + hh) * 16 : wbase + 512 * R;
    const uint32_t a_slot = a_active ? 256 * R : 0;
    const uint32_t a_step = a_active ? R * 32 : 0;
    if (lane < 4) reinterpret_cast<uint32_t *>(wbase + 512 * R)[lane] = 0u;

    // ---- block scales of the (at most two) 128-row groups the range
    // touches: lane i holds block kbof(i)'s (a wavefront has at most 64
    // blocks); v_readlane picks them per block, so no scalar load shares the
    // LDS counter with the operand reads inside the loop.  An output lane
    // (column mrow = row r0 + mrow) takes its row's group ----
    // (Pair mode: a = gate's group, b = up's same group; lanes of columns
    // 16..31 take up's.)
    const uint32_t ga = r0 >> 7, gb = PAIR ? ga : (r1 - 1) >> 7;
    const float *const scale_b = PAIR ? p.seg[1].scale : sg.scale;
    const float sca_lane = sg.scale[(size_t)ga * KB + kbof(min(lane, n - 1))];
    const float scb_lane = scale_b[(size_t)gb * KB + kbof(min(lane, n - 1))];
    const bool out_in_a = PAIR ? mrow < kPairRows : ((r0 + mrow) >> 7) == ga;

    // ---- ring: slot d holds the weights of block b and the activations of
    // block b+1 (clamped into the range).  Weights are read once per call:
    // non-temporal loads keep them from displacing cached data (layer step
    // +3.4% against plain loads) ----
    // lane l: row r0 + l%32 (clamped into the range; the extra columns are
    // never written), its sub-tile and place in the 1 KiB chunks
    const uint32_t rl = min(r0 + (PAIR ? mrow % kPairRows : mrow), r1 - 1);
    const uint8_t *const codes_w = PAIR && mrow >= kPairRows ? p.seg[1].codes : sg.codes;
    const uint8_t *codes = codes_w + ((size_t)(rl >> 7) * KB * 4 + ((rl >> 5) & 3)) * kSubBytes + hh * 512 +
                           (rl & 31) * 16;
    u32x4_t buf[DEPTH][4];
    XBlock<MT> xr[DEPTH], wr[NORM ? DEPTH : 1];   // wr: RMSNorm weights of the same columns
    auto load = [&](uint32_t d, uint32_t i) {
        const uint8_t *src = codes + (size_t)kbof(i) * kBlockBytes;
#pragma unroll
        for (uint32_t j = 0; j < 4; j++)
            buf[d][j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t *>(src + j * kChunkBytes));
        load_xblock<VEC, MT>(xr[d], p.x, p.ldx, M, p.k, kbof(min(i + 1, n - 1)), lane);
        if constexpr (NORM) load_xblock<VEC, MT>(wr[d], p.norm_w, 0, 1, p.k, kbof(min(i + 1, n - 1)), lane);
    };
    // RMSNorm: the row's whole x, squared into LDS for the reference's
    // eight sequential lane sums (loaded first, so waiting for it waits for
    // nothing else)
    constexpr uint32_t kNormPer = NORM ? kPairNormMaxCols / (64 * NW) : 1;
    float xs[kNormPer];
    if constexpr (NORM) {
#pragma unroll
        for (uint32_t j = 0; j < kNormPer; j++) {
            const uint32_t i = threadIdx.x + j * 64 * NW;
            xs[j] = i < p.k ? p.x[i] : 0.0f;
        }
    }
    XBlock<MT> x0, w0;
    load_xblock<VEC, MT>(x0, p.x, p.ldx, M, p.k, kbof(0), lane);
    if constexpr (NORM) load_xblock<VEC, MT>(w0, p.norm_w, 0, 1, p.k, kbof(0), lane);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (uint32_t d = 0; d + 1 < DEPTH; d++) load(d, min(d, n - 1));
    __builtin_amdgcn_sched_barrier(0);
    // The scale 1 / sqrt(mean(x^2) + eps) of the row, computed by every
    // workgroup while its first weight loads are in flight: resident
    // workgroups run their chains of n/8 dependent adds side by side, so a
    // launch pays one chain per round of workgroups, not one per workgroup
    float inv = 1.0f;
    if constexpr (NORM) {
        __shared__ float s_inv;
        float *const sq = reinterpret_cast<float *>(lds + NW * gemv_rows_wave_lds(1));
        const uint32_t kStride = pair_norm_stride(p.k);
        const uint32_t kpad = (p.k + 7) & ~7u;   // squares the lane sums read; past the row +0, no change
#pragma unroll
        for (uint32_t j = 0; j < kNormPer; j++) {
            const uint32_t i = threadIdx.x + j * 64 * NW;
            if (i < kpad) sq[(i & 7) * kStride + (i >> 3)] = xs[j] * xs[j];
        }
        __syncthreads();
        if (threadIdx.x < 8) red[0][0][threadIdx.x] = lane_sum_in_order(sq + threadIdx.x * kStride, (p.k + 7) >> 3, 0.0f);
        __syncthreads();
        if (threadIdx.x == 0) {
            float sum = red[0][0][0];
#pragma unroll
            for (uint32_t j = 1; j < 8; j++) sum = sum + red[0][0][j];
            s_inv = rms_inverse(sum, p.k, p.eps);
        }
        __syncthreads();
        inv = s_inv;
#pragma unroll
        for (uint32_t e = 0; e < XBlock<MT>::kG; e++) x0.v[e] = rmsnorm1(x0.v[e], inv, w0.v[e]);
    }
    // A block staged shifted (wide activations) takes its scale times
    // kActUnshift: lane i holds block i's scales, so only that lane changes.
    float sca_l = sca_lane, scb_l = scb_lane;
    auto unshift_scale = [&](uint32_t i) {
        if (lane == i) {
            sca_l *= kActUnshift;
            scb_l *= kActUnshift;
        }
    };
    // waits for x0 only: loads complete in order
    if (__builtin_expect(stage_xblock<MT>(x0, wbase, M, R, p.k, kbof(0), lane), 0)) unshift_scale(0);

    // ---- stream ----
    f32x16_t acc = {};
    const f32x16_t zero = {};
    for (uint32_t b = 0; b < n; b += DEPTH) {
#pragma unroll
        for (uint32_t d = 0; d < DEPTH; d++) {
            const uint32_t bb = b + d;
            load((d + DEPTH - 1) % DEPTH, min(bb + DEPTH - 1, n - 1));
            // keep the scheduler from sinking these loads below block bb's math
            __builtin_amdgcn_sched_barrier(0);
            if (bb < n) {
                const uint32_t par = bb & 1;
                u32x4_t araw[8];
#pragma unroll
                for (uint32_t i = 0; i < 8; i++)
                    araw[i] = *reinterpret_cast<const u32x4_t *>(arow + par * a_slot + i * a_step);
                if constexpr (NORM) {
#pragma unroll
                    for (uint32_t e = 0; e < XBlock<MT>::kG; e++) xr[d].v[e] = rmsnorm1(xr[d].v[e], inv, wr[d].v[e]);
                }
                if (bb + 1 < n &&
                    __builtin_expect(stage_xblock<MT>(xr[d], wbase + (par ^ 1) * 256 * R, M, R, p.k, kbof(bb + 1), lane), 0))
                    unshift_scale(bb + 1);
                __builtin_amdgcn_sched_barrier(0);
                f32x16_t part;
#pragma unroll
                for (uint32_t j = 0; j < 4; j++)
#pragma unroll
                    for (uint32_t q = 0; q < 2; q++) {
                        const bf16x8_t bop = e4m3x8_to_bf16x8_cvt(buf[d][j][2 * q], buf[d][j][2 * q + 1], 1.0f);
                        const bf16x8_t aop = __builtin_bit_cast(bf16x8_t, araw[j * 2 + q]);
                        part = mfma32x32x16(aop, bop, (j == 0 && q == 0) ? zero : part);
                    }
                const float sca =
                    __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, sca_l), bb));
                const float scb =
                    __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, scb_l), bb));
                const float sc = out_in_a ? sca : scb;
                // acc[r + 4p] holds part p of token 4h + (r & 3): only tokens
                // below MT are scaled; rows 24..31 carry nothing (regs 12..15)
#pragma unroll
                for (uint32_t r = 0; r < 12; r++)
                    if ((r & 3) < MT) acc[r] = __builtin_fmaf(sc, part[r], acc[r]);
            }
        }
    }

    // ---- wavefront partials -> outputs, wavefronts added in order ----
    // Lane (h, n) holds token 4h + r of row n in acc[r] (part 0), acc[r + 4]
    // (part 1) and acc[r + 8] (part 2).
#pragma unroll
    for (uint32_t r = 0; r < 4; r++) {
        const uint32_t t = 4 * hh + r;
        if (t < M) red[wv][t][mrow] = (acc[r] + acc[r + 4]) + acc[r + 8];
    }
    __syncthreads();
    if constexpr (PAIR) {
        // gate and up of row r0 + col, wavefronts added in order as for one
        // weight, then silu(gate) * up (the bits of the separate kernels)
        if (threadIdx.x < kPairRows * M) {
            const uint32_t t = threadIdx.x / kPairRows, col = threadIdx.x % kPairRows;
            float g = red[0][t][col], u = red[0][t][col + kPairRows];
#pragma unroll
            for (uint32_t w = 1; w < NW; w++) {
                g += red[w][t][col];
                u += red[w][t][col + kPairRows];
            }
            const uint32_t row = r0 + col;
            if (row < r1) sg.y[(size_t)t * sg.ldy + row] = swiglu1(g, u);
        }
        return;
    }
    if (threadIdx.x < kSubRows * M) {
        const uint32_t t = threadIdx.x >> 5, col = threadIdx.x & 31;
        float sum = red[0][t][col];
#pragma unroll
        for (uint32_t w = 1; w < NW; w++) sum += red[w][t][col];
        const uint32_t row = r0 + col;
        if (row < r1) {
            const size_t o = (size_t)t * sg.ldy + row;
            const float v = sg.resid ? sg.resid[o] + sum : sum;
            if (p.done_word)
                __hip_atomic_store(sg.y + o, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            else
                sg.y[o] = v;
        }
    }
    // Host-pointer calls: the last workgroup to finish stores the call's
    // completion word (pinned host memory the calling thread polls), in
    // place of a flag kernel queued after this one.  The outputs were
    // stored at system scope (through to memory, no cache keeps them); every
    // wavefront waits for its stores to complete before the workgroup
    // counts itself, so when the count completes every output of the launch
    // has reached memory.  The counter returns to zero.
    if (p.done_word) {
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (threadIdx.x == 0) {
            if (__hip_atomic_fetch_add(p.done_cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == p.nctas - 1) {
                __hip_atomic_store(p.done_cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(p.done_word, p.done_value, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            }
        }
    }
}

bool gemv_rows_shape(uint32_t kb, uint32_t waves) { return kb >= waves && kb <= kGemvRsMaxKb && kb <= 64 * waves; }

void gemv_rows_plan(const uint32_t *rows, uint32_t nseg, uint32_t *nctas) {
    for (uint32_t s = 0; s < nseg; s++) nctas[s] = (rows[s] + kSubRows - 1) / kSubRows;
}

namespace {
using RowsKernel = void (*)(GemvParams);

template <uint32_t NW>
RowsKernel rows_kernel(uint32_t depth, uint32_t vec_mt) {
#define Q35_RK(D)                                                                                          \
    {gemv_rows_kernel<false, 1, D, NW>, gemv_rows_kernel<false, 2, D, NW>, gemv_rows_kernel<false, 4, D, NW>, \
     gemv_rows_kernel<false, 8, D, NW>, gemv_rows_kernel<true, 1, D, NW>,  gemv_rows_kernel<true, 2, D, NW>,  \
     gemv_rows_kernel<true, 4, D, NW>,  gemv_rows_kernel<true, 8, D, NW>}
    static const RowsKernel k[3][8] = {Q35_RK(2), Q35_RK(3), Q35_RK(4)};
#undef Q35_RK
    return k[depth - 2][vec_mt];
}
using PairKernel = void (*)(GemvParams);
PairKernel pair_kernel(bool norm, uint32_t depth, uint32_t vec_mt) {
#define Q35_PK(D)                                                                                       \
    {gemv_rows_kernel<false, 1, D, 4, kRowsPair>, gemv_rows_kernel<false, 2, D, 4, kRowsPair>,          \
     gemv_rows_kernel<false, 4, D, 4, kRowsPair>, gemv_rows_kernel<false, 8, D, 4, kRowsPair>,          \
     gemv_rows_kernel<true, 1, D, 4, kRowsPair>,  gemv_rows_kernel<true, 2, D, 4, kRowsPair>,           \
     gemv_rows_kernel<true, 4, D, 4, kRowsPair>,  gemv_rows_kernel<true, 8, D, 4, kRowsPair>}
    static const PairKernel k[2][8] = {Q35_PK(2), Q35_PK(3)};
#undef Q35_PK
    static const PairKernel kn[2][2] = {{gemv_rows_kernel<false, 1, 2, 4, kRowsPairNorm>,
                                         gemv_rows_kernel<true, 1, 2, 4, kRowsPairNorm>},
                                        {gemv_rows_kernel<false, 1, 3, 4, kRowsPairNorm>,
                                         gemv_rows_kernel<true, 1, 3, 4, kRowsPairNorm>}};
    return norm ? kn[depth - 2][vec_mt >> 2] : k[depth - 2][vec_mt];
}
}  // namespace

hipError_t launch_gemv_pair(const GemvParams &pin, bool norm, uint32_t cus, hipStream_t stream) {
    GemvParams p = pin;
    const GemvSeg &g = p.seg[0], &u = p.seg[1];
    if (p.xmode != kXPlain || p.m == 0 || p.m > kGemvMaxM || !gemv_rows_shape(p.kb, 4) || p.nseg != 2 ||
        g.rows != u.rows || g.nb != u.nb || g.rows == 0 || g.cta_begin != 0)
        return hipErrorInvalidValue;
    if (norm && (p.m != 1 || p.k > kPairNormMaxCols || !p.norm_w)) return hipErrorInvalidValue;
    p.nctas = (g.rows + kPairRows - 1) / kPairRows;
    size_t lds = 4 * (size_t)gemv_rows_wave_lds(p.m);
    if (norm) lds += 8 * pair_norm_stride(p.k) * sizeof(float);   // the squares of x, lane-major
    const uint32_t mt = p.m <= 1 ? 0 : p.m <= 2 ? 1 : p.m <= 4 ? 2 : 3;
    const uint32_t depth = p.m <= 2 && p.nctas <= cus ? kRsDepthLong : kRsDepthShort;
    const PairKernel k = pair_kernel(norm, depth, (p.x_vec ? 4 : 0) + mt);
    static bool attr_set = false;
    if (!attr_set) {
        for (bool nm : {false, true})
            for (uint32_t d : {2u, 3u})
                for (uint32_t v = 0; v < 8; v++) {
                    if (nm && (v & 3)) continue;
                    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(pair_kernel(nm, d, v)),
                                                             hipFuncAttributeMaxDynamicSharedMemorySize, 64 * 1024);
                    if (e != hipSuccess) return e;
                }
        attr_set = true;
    }
    hipLaunchKernelGGL(k, dim3(p.nctas), dim3(256), lds, stream, p);
    return hipGetLastError();
}

hipError_t launch_gemv_rows(const GemvParams &pin, uint32_t cus, uint32_t waves, uint32_t depth,
                            hipStream_t stream) {
    GemvParams p = pin;
    if (p.xmode != kXPlain || p.m == 0 || p.m > kGemvMaxM || (waves != 4 && waves != 8) ||
        !gemv_rows_shape(p.kb, waves) || p.nseg == 0 || p.nseg > 4)
        return hipErrorInvalidValue;
    for (uint32_t s = 0; s < p.nseg; s++) {
        const GemvSeg &g = p.seg[s];
        if (g.rows == 0 || g.nctas != (g.rows + kSubRows - 1) / kSubRows)
            return hipErrorInvalidValue;   // one workgroup per 32-row sub-tile
    }
    const size_t lds = (size_t)waves * gemv_rows_wave_lds(p.m);
    const uint32_t mt = p.m <= 1 ? 0 : p.m <= 2 ? 1 : p.m <= 4 ? 2 : 3;   // log2 of MT
    if (depth == 0) depth = p.m <= 2 && p.nctas <= cus ? kRsDepthLong : kRsDepthShort;
    depth = std::min(std::max(depth, 2u), 4u);
    const uint32_t vm = (p.x_vec ? 4 : 0) + mt;
    const RowsKernel k = waves == 8 ? rows_kernel<8>(depth, vm) : rows_kernel<4>(depth, vm);
    hipLaunchKernelGGL(k, dim3(p.nctas), dim3(64 * waves), lds, stream, p);
    return hipGetLastError();
}

}  // namespace q35mm
