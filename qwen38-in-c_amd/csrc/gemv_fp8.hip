// gemv_fp8.hip -- decode GEMV, m <= 8 tokens, FP8-E4M3 weights with
// 128x128 fp32 block scales, fp32-accurate.
//
// Replaces the hot loop of qwen35-c/src/q35_mm.c:88-198 (mm_fp8_row called
// by q35_mm_fp8 / q35_mm_fp8_batch / q35_mm_fp8_multi4).
//
// Arithmetic.  Weights are converted e4m3 -> bf16 in registers (exact, two
// codes per v_cvt_scalef32_pk_bf16_fp8 at scale 1.0) and
// fed to v_mfma_f32_32x32x16_bf16.  Activations are fp32; each is split
// exactly into three bf16 parts x = p0 + p1 + p2, and the A-operand rows are
// m = t + 8p (token t < 8, part p < 3), so one MFMA forms the three partial
// dot products of up to eight tokens.  Products e4m3*bf16 are exact in fp32;
// the only rounding is fp32 accumulation.  Per 128-column K block the MFMA
// accumulator holds the raw block dot product, which is multiplied by the
// block's fp32 scale and added to the running sum (one fmaf per output and
// block).
//
// Decomposition (stream-K).  A weight is a sequence of T = NB*KB 16 KiB
// blocks (128-row group g, K block kb) in (g, kb) order.  Its grid is a
// fixed P workgroups (one per CU by default); workgroup c takes the
// contiguous block range [c*T/P, (c+1)*T/P), so every CU streams the same
// number of bytes whatever the shape.  Several weights sharing K (the
// reference's multi4) get one grid each, concatenated into one launch.
// Wavefront w of a workgroup owns 32-row sub-tile w of every block, streams
// it with one 16-byte load per lane per 1 KiB chunk (the lane-order tile
// layout makes every load a contiguous 1 KiB) and keeps a ring of
// kGemvDepth blocks in flight across group boundaries.
//
// A group wholly inside one range is written to y directly.  A group split
// between ranges is finished by its last contributor to arrive: each
// contributor publishes its partial outputs, takes a ticket, and the last
// one adds the partials in range order.  That order is fixed by the shape,
// so results do not depend on timing, and P depends only on the shape, so a
// batch of m tokens gives exactly the bits of m single-token calls.
//
// Fused neighbours (qwen35-c/src/q35_model.c:927-939).  The staged
// activations can be the RMSNorm of x (kXRmsNorm: every workgroup forms the
// sum of squares of the whole row in the reference's eight-lane order, then
// normalises the columns it stages) or SwiGLU of two inputs (kXSwiGLU), and
// the output can be added to a residual (y = resid + product).  Each is the
// same arithmetic as the separate kernels in mlp.hip, so a fused launch gives
// the bits of the unfused sequence.
#include <algorithm>

#include "q35mm_device.h"
#include "q35mm_internal.h"

namespace q35mm {

namespace {

// Weight codes: read once per call, so non-temporal (+4% against plain
// loads on the decode shapes).
__device__ __forceinline__ u32x4_t ld16(const uint8_t *p) {
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4_t *>(p));
}

// Activation staging.  The three-part bf16 split of the activations for the
// workgroup's blocks goes to LDS in MFMA A-operand order.  Slot i holds K
// block (b0 + i) mod KB:
//   byte offset(c, q, ai, h) = (((c*2 + q) * R + ai) * 2 + h) * 16
// where c = i*4 + chunk, q selects the first or second MFMA of the chunk,
// ai = part*m + t, R = 3m rounded up to odd, h = lane/32, and the 16 bytes
// hold columns
// kb*128 + chunk*32 + 16h + 8q + (0..7).  An odd R keeps the 16 (c, q, h)
// positions of one K block in 16 different 16-byte bank groups (an even R
// puts a 256-byte multiple between consecutive (c, q) and the staging
// writes of a wavefront pile onto two bank groups).
//
// Work item v (< m * nblk * 16) is one 8-column vector of one token.  The
// loads of a thread's first kStagePre items are split from the rest so they
// can be issued before the weight prologue: memory loads complete in issue
// order, so anything issued before the weights can be waited for without
// waiting for the weights.
constexpr uint32_t kStagePre = 2;
constexpr uint32_t kStageBatch = 4;

struct StageItem {
    uint32_t t, kk, kg;   // token, slot-relative column, global column
};

__device__ __forceinline__ StageItem stage_item(uint32_t i, uint32_t per_t, uint32_t kb_total, uint32_t b0) {
    StageItem it;
    it.t = i / per_t;
    const uint32_t v = i - it.t * per_t;
    const uint32_t slot = v >> 4;
    it.kk = slot * kBlock + (v & 15) * 8;
    it.kg = ((b0 + slot) % kb_total) * kBlock + (v & 15) * 8;
    return it;
}

// Eight consecutive columns of one row at the clamped column min(kg, k - 8)
// (vec: two 16-byte loads; the row is 16-byte aligned and k % 8 == 0) or
// min(kg + e, k - 1) (eight 4-byte loads).  Unconditional, so no branch sits
// between them and the weight prologue; columns >= k are zeroed later.
template <bool VEC>
__device__ __forceinline__ void load8(float (&v)[8], const float *row, uint32_t kg, uint32_t k) {
    if constexpr (VEC) {
        const float4 *q = reinterpret_cast<const float4 *>(row + min(kg, k - 8));
        const float4 a = q[0], b = q[1];
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
        v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
#pragma unroll
        for (int e = 0; e < 8; e++) v[e] = row[min(kg + e, k - 1)];
    }
}

// Raw inputs of one item: x, plus up (kXSwiGLU) or the norm weight
// (kXRmsNorm).  vec requires every input row to be 16-byte aligned.
template <uint32_t XM>
struct StageIn {
    float x[8];
    float a[8];
};

template <uint32_t XM, bool VEC>
__device__ __forceinline__ void stage_load(StageIn<XM> &in, const GemvParams &p, const StageItem &it) {
    load8<VEC>(in.x, p.x + (size_t)it.t * p.ldx, it.kg, p.k);
    if constexpr (XM == kXSwiGLU) load8<VEC>(in.a, p.x2 + (size_t)it.t * p.ldx, it.kg, p.k);
    if constexpr (XM == kXRmsNorm) load8<VEC>(in.a, p.norm_w, it.kg, p.k);
}

// The staged values: the transform of the raw inputs, columns >= k zeroed.
template <uint32_t XM>
__device__ __forceinline__ void stage_finish(float (&xv)[8], const StageIn<XM> &in, uint32_t k, const StageItem &it,
                                             const float *s_inv) {
#pragma unroll
    for (int e = 0; e < 8; e++) {
        float v = in.x[e];
        if constexpr (XM == kXSwiGLU) v = swiglu1(in.x[e], in.a[e]);
        if constexpr (XM == kXRmsNorm) v = rmsnorm1(in.x[e], s_inv[it.t], in.a[e]);
        xv[e] = (it.kg + e < k) ? v : 0.0f;
    }
}

// SHIFT: the workgroup's range holds a wide value (kActWide): every staged
// value is multiplied by kActShift and the block scales by kActUnshift.
template <bool SHIFT>
__device__ __forceinline__ void stage_store(uint8_t *lds, uint32_t m, const StageItem &it, const float (&xv)[8]) {
    const uint32_t R = stage_rows(m);
    uint32_t p0[4], p1[4], p2[4];   // packed pairs of columns
#pragma unroll
    for (int e = 0; e < 4; e++) {
        if constexpr (SHIFT) {
            const float a = xv[2 * e] * kActShift, b = xv[2 * e + 1] * kActShift;
            split3_bf16x2(a, b, p0[e], p1[e], p2[e]);
            split3_fix_inf(p0[e], p1[e], p2[e]);
        } else {
            split3_bf16x2(xv[2 * e], xv[2 * e + 1], p0[e], p1[e], p2[e]);
        }
    }
    const uint32_t c = it.kk >> 5, h = (it.kk >> 4) & 1, q = (it.kk >> 3) & 1;
    const uint32_t base = (c * 2 + q) * R;
    const u32x4_t w0 = {p0[0], p0[1], p0[2], p0[3]};
    const u32x4_t w1 = {p1[0], p1[1], p1[2], p1[3]};
    const u32x4_t w2 = {p2[0], p2[1], p2[2], p2[3]};
    *reinterpret_cast<u32x4_t *>(lds + ((base + 0 * m + it.t) * 2 + h) * 16) = w0;
    *reinterpret_cast<u32x4_t *>(lds + ((base + 1 * m + it.t) * 2 + h) * 16) = w1;
    *reinterpret_cast<u32x4_t *>(lds + ((base + 2 * m + it.t) * 2 + h) * 16) = w2;
}

// The workgroup whose range holds a given block: the largest c with
// floor(c*T/P) <= block.
__device__ __forceinline__ uint32_t range_of(uint64_t block, uint32_t T, uint32_t P) {
    return (uint32_t)(((block + 1) * P + T - 1) / T) - 1;
}

// ---- RMSNorm prologue (kXRmsNorm) ----
// The m rows of x are loaded once, kNormBatch float4s per thread (float4
// slot v = token * slots + column/4; the host uses this mode only when
// m * k fits), before the weight prologue.  Their squares go to LDS
// lane-major, lane row (t*8 + j) holding columns j, j+8, ... of token t,
// row stride norm_cols/8 + 4 floats.  Lane 8t + j of wavefront 0 then adds
// its row in order; lanes are folded 0..7 per token.

struct NormBatch {
    float4 v[kGemvNormBatch];
};

// Loads are unconditional (addresses clamped into the row) and the values
// are used only by norm_store, which masks columns past the row's end: a
// load under a branch, or a use right after the loads, would make the
// compiler wait for them before the weight prologue is issued.
__device__ __forceinline__ void norm_load(NormBatch &nb, const GemvParams &p, uint32_t slots) {
    const uint32_t n4 = p.m * slots, k = p.k;
#pragma unroll
    for (uint32_t u = 0; u < kGemvNormBatch; u++) {
        const uint32_t v = min(u * kGemvThreads + threadIdx.x, n4 - 1);
        const uint32_t t = v / slots, q = v - t * slots;
        const float *row = p.x + (size_t)t * p.ldx;
        if (p.x_vec) {   // k % 8 == 0: a slot is wholly inside or wholly past the row
            nb.v[u] = *reinterpret_cast<const float4 *>(row + min(4 * q, k - 4));
        } else {
            nb.v[u].x = row[min(4 * q + 0, k - 1)];
            nb.v[u].y = row[min(4 * q + 1, k - 1)];
            nb.v[u].z = row[min(4 * q + 2, k - 1)];
            nb.v[u].w = row[min(4 * q + 3, k - 1)];
        }
    }
}

__device__ __forceinline__ void norm_store(const NormBatch &nb, float *sq, uint32_t stride, uint32_t slots,
                                           uint32_t k, uint32_t n4) {
#pragma clang fp contract(off)
#pragma unroll
    for (uint32_t u = 0; u < kGemvNormBatch; u++) {
        const uint32_t v = u * kGemvThreads + threadIdx.x;
        // every loaded value is consumed here, repeats of a clamped slot too,
        // so no load stays in flight past this point
        const float4 x = nb.v[u];
        const uint32_t t = min(v, n4 - 1) / slots, q = min(v, n4 - 1) - t * slots;
        const uint32_t c = 4 * q;   // columns c .. c+3; past k they square to +0.0f
        const float e0 = c + 0 < k ? x.x : 0.0f, e1 = c + 1 < k ? x.y : 0.0f;
        const float e2 = c + 2 < k ? x.z : 0.0f, e3 = c + 3 < k ? x.w : 0.0f;
        const float q0 = e0 * e0, q1 = e1 * e1, q2 = e2 * e2, q3 = e3 * e3;
        if (v < n4) {
            // lanes (c & 7) + 0..3 of token t, position q / 2
            float *d = sq + (t * 8 + (c & 7)) * stride + (q >> 1);
            d[0 * stride] = q0;
            d[1 * stride] = q1;
            d[2 * stride] = q2;
            d[3 * stride] = q3;
        }
    }
}

// Lane 8t + j of wavefront 0 adds lane row 8t + j of the squares in order;
// s_inv[t] = 1 / sqrtf(mean_t + eps) for t < m.
__device__ __forceinline__ void norm_finish(const GemvParams &p, const float *sq, uint32_t stride, uint32_t cnt,
                                            float *s_lane, float *s_inv) {
#pragma clang fp contract(off)
    const uint32_t tid = threadIdx.x;
    if (tid < 8 * p.m) s_lane[tid] = lane_sum_in_order(sq + tid * stride, cnt, 0.0f);
    __syncthreads();
    if (tid < p.m) {
        float s = s_lane[8 * tid];
#pragma unroll
        for (int j = 1; j < 8; j++) s = s + s_lane[8 * tid + j];
        s_inv[tid] = rms_inverse(s, p.k, p.eps);
    }
    __syncthreads();
}

}  // namespace

template <uint32_t XM, bool VEC>
__global__ __launch_bounds__(kGemvThreads) void gemv_fp8_kernel(GemvParams p) {
    extern __shared__ __align__(16) uint8_t lds[];
    __shared__ uint32_t s_ticket;
    __shared__ float s_lane[8 * kGemvMaxM];   // kXRmsNorm: lane sums
    __shared__ float s_inv[kGemvMaxM];        // kXRmsNorm: 1/rms per token

    // ---- segment and block range of this workgroup ----
    uint32_t si = 0;
#pragma unroll
    for (uint32_t i = 1; i < 4; i++)
        if (i < p.nseg && blockIdx.x >= p.seg[i].cta_begin) si = i;
    const GemvSeg &sg = p.seg[si];
    const uint32_t c = blockIdx.x - sg.cta_begin;
    const uint32_t KB = p.kb, M = p.m;
    const uint32_t P = sg.nctas, T = sg.nb * KB;
    const uint32_t b0 = (uint32_t)(((uint64_t)c * T) / P);
    const uint32_t b1 = (uint32_t)(((uint64_t)(c + 1) * T) / P);
    const uint32_t nblk = b1 - b0;                 // >= 1 (P <= T)

    // ---- per-lane roles ----
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t wv = threadIdx.x >> 6;          // 32-row sub-tile
    const uint32_t mrow = lane & 31, hh = lane >> 5;
    const uint32_t tt = mrow & 7, pp = mrow >> 3;  // A row = token + 8*part
    const bool a_active = (tt < M) && (pp < 3);
    const uint32_t R = stage_rows(M);
    // A-operand address = a_base + (chunk*2 + q) * a_step.  Rows that carry
    // no token (t >= m, or the unused rows 24..31) read a 16-byte zero slot
    // placed after the stage, so every lane issues the same LDS read.
    const uint32_t zero_off = nblk * 256 * R;
    const uint32_t a_base = a_active ? ((pp * M + tt) * 2 + hh) * 16 : zero_off;
    const uint32_t a_step = a_active ? R * 32 : 0;
    const uint32_t lane_off = wv * kSubBytes + lane * 16;

    // ---- weight stream: a ring of kGemvDepth blocks in registers ----
    // Loads are unconditional (block index clamped into the range; the few
    // repeated tail loads hit in cache) so that the wait before each block is
    // a static vmcnt and kGemvDepth-1 blocks stay in flight.  The range's
    // block scales sit one per lane (lane i: block b0 + i) and v_readlane
    // picks each, so no scalar load shares the LDS counter with the operand
    // reads in the loop.
    static_assert(kGemvMaxRangeBlocks <= 64, "a range's block scales sit one per lane");
    u32x4_t buf[kGemvDepth][4];
    float sc_lane = 0.0f;
    const uint8_t *codes = sg.codes + lane_off;
    auto load = [&](u32x4_t (&dst)[4], uint32_t b) {
        const uint8_t *src = codes + (size_t)b * kBlockBytes;   // block b = g*KB + kb
#pragma unroll
        for (int j = 0; j < 4; j++) dst[j] = ld16(src + j * kChunkBytes);
    };

    // ---- prologue: activation loads, then the first weight blocks ----
    const uint32_t per_t = nblk * 16;
    const uint32_t nvec = M * per_t;
    StageIn<XM> xpre[kStagePre];
    auto stage_pre_load = [&]() {
#pragma unroll
        for (uint32_t u = 0; u < kStagePre; u++)   // index clamped: loads are unconditional
            stage_load<XM, VEC>(xpre[u], p, stage_item(min(threadIdx.x + u * kGemvThreads, nvec - 1), per_t, KB, b0));
    };
    auto ring_prologue = [&]() {
        sc_lane = sg.scale[min(b0 + lane, b1 - 1)];
#pragma unroll
        for (uint32_t d = 0; d + 1 < kGemvDepth; d++) load(buf[d], min(b0 + d, b1 - 1));
    };
    if constexpr (XM == kXRmsNorm) {
        // x rows first, alone: their squares go to LDS (the stage takes it
        // over afterwards) before any weight load competes with them.  Then
        // the stage and weight loads, whose latency hides behind the
        // sequential sums.
        const uint32_t slots = ((p.k + 7) & ~7u) / 4, stride = p.norm_cols / 8 + 4;
        float *sq = reinterpret_cast<float *>(lds);
        NormBatch nb;
        norm_load(nb, p, slots);
        norm_store(nb, sq, stride, slots, p.k, M * slots);
        __syncthreads();
        stage_pre_load();
        __builtin_amdgcn_sched_barrier(0);
        ring_prologue();
        __builtin_amdgcn_sched_barrier(0);
        norm_finish(p, sq, stride, slots / 2, s_lane, s_inv);
    } else {
        stage_pre_load();
        __builtin_amdgcn_sched_barrier(0);
        ring_prologue();
        __builtin_amdgcn_sched_barrier(0);
    }
    // Split and stage while the weight blocks are in flight.  wide: a
    // staged value of this thread reached kActWide.
    bool wide = false;
#pragma unroll
    for (uint32_t u = 0; u < kStagePre; u++) {
        const uint32_t i = threadIdx.x + u * kGemvThreads;
        const StageItem it = stage_item(min(i, nvec - 1), per_t, KB, b0);
        float xv[8];
        stage_finish(xv, xpre[u], p.k, it, s_inv);
        if (i < nvec) {
            wide |= max_abs(xv) >= kActWide;
            stage_store<false>(lds, M, it, xv);
        }
    }
    // The rest (m > 1) in batches of kStageBatch items per thread: the loads
    // of a batch are all issued before any is used (the scheduling barrier
    // keeps the compiler from sinking them to their uses), one memory round
    // trip per batch.
    for (uint32_t i0 = threadIdx.x + kStagePre * kGemvThreads; i0 < nvec; i0 += kStageBatch * kGemvThreads) {
        StageIn<XM> in[kStageBatch];
#pragma unroll
        for (uint32_t u = 0; u < kStageBatch; u++)   // index clamped: loads are unconditional
            stage_load<XM, VEC>(in[u], p, stage_item(min(i0 + u * kGemvThreads, nvec - 1), per_t, KB, b0));
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (uint32_t u = 0; u < kStageBatch; u++) {
            const uint32_t i = i0 + u * kGemvThreads;
            const StageItem it = stage_item(min(i, nvec - 1), per_t, KB, b0);
            float xv[8];
            stage_finish(xv, in[u], p.k, it, s_inv);
            if (i < nvec) {
                wide |= max_abs(xv) >= kActWide;
                stage_store<false>(lds, M, it, xv);
            }
        }
    }
    if (threadIdx.x < 4) reinterpret_cast<uint32_t *>(lds + zero_off)[threadIdx.x] = 0u;
    if (__builtin_expect(__syncthreads_or(wide), 0)) {
        // Rare: the range holds a wide value or an infinity.  Stage it all
        // again, shifted, and take the block scales times kActUnshift.
        for (uint32_t i = threadIdx.x; i < nvec; i += kGemvThreads) {
            const StageItem it = stage_item(i, per_t, KB, b0);
            StageIn<XM> in;
            stage_load<XM, VEC>(in, p, it);
            float xv[8];
            stage_finish(xv, in, p.k, it, s_inv);
            stage_store<true>(lds, M, it, xv);
        }
        sc_lane *= kActUnshift;
        __syncthreads();
    }

    f32x16_t acc = {};
    const f32x16_t zero = {};

    auto compute = [&](const u32x4_t (&wq)[4], float sc, uint32_t slot) {
        const uint32_t cbase = slot * 4;
        // All eight A-operand reads of the block first: their latency is paid
        // once per block.
        u32x4_t araw[8];
#pragma unroll
        for (int i = 0; i < 8; i++)
            araw[i] = *reinterpret_cast<const u32x4_t *>(lds + a_base + (cbase * 2 + i) * a_step);
        __builtin_amdgcn_sched_barrier(0);
        f32x16_t part;
#pragma unroll
        for (int j = 0; j < 4; j++) {
#pragma unroll
            for (int q = 0; q < 2; q++) {
                const bf16x8_t bop = e4m3x8_to_bf16x8_cvt(wq[j][2 * q], wq[j][2 * q + 1], 1.0f);
                const bf16x8_t aop = __builtin_bit_cast(bf16x8_t, araw[j * 2 + q]);
                part = mfma32x32x16(aop, bop, (j == 0 && q == 0) ? zero : part);
            }
        }
        // Rows 24..31 of the A operand are never used (regs 12..15).
#pragma unroll
        for (int r = 0; r < 12; r++) acc[r] = __builtin_fmaf(sc, part[r], acc[r]);
    };

    // ---- finishing a group segment [gs, ge) of this range ----
    // Only the first and the last segment of a range can be part of a split
    // group; pend* remember split groups this workgroup arrived last at.
    // They are reduced after the stream so the ring is not held up.
    bool pend0 = false, pend1 = false;
    uint32_t pg0 = 0, pg1 = 0;
    auto flush = [&](uint32_t G, uint32_t gs, uint32_t ge, bool first) {
        float yv[4];
#pragma unroll
        for (int r = 0; r < 4; r++) yv[r] = (acc[r] + acc[r + 4]) + acc[r + 8];
        const uint32_t rl = wv * 32 + mrow;
        const uint32_t row = G * kBlock + rl;
        if (ge - gs == KB) {   // the whole group is in this range
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const uint32_t t = 4 * hh + r;
                if (t < M && row < sg.rows) {
                    const size_t o = (size_t)t * sg.ldy + row;
                    sg.y[o] = sg.resid ? sg.resid[o] + yv[r] : yv[r];
                }
            }
            return;
        }
        // Publish the partial with device-scope atomic stores (they reach the
        // coherence point instead of staying dirty in this XCD's L2, so no L2
        // writeback is needed), wait until they are complete, take a ticket.
        const uint32_t cfirst = range_of((uint64_t)G * KB, T, P);
        const uint32_t clast = range_of((uint64_t)G * KB + KB - 1, T, P);
        float *slot = p.ws + sg.ws_off + ((size_t)G * sg.maxc + (c - cfirst)) * (kGemvMaxM * kBlock);
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const uint32_t t = 4 * hh + r;
            if (t < M)
                __hip_atomic_store(slot + t * kBlock + rl, yv[r], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (threadIdx.x == 0)
            s_ticket = __hip_atomic_fetch_add(p.cnt + sg.cnt_off + G, 1u, __ATOMIC_RELAXED,
                                              __HIP_MEMORY_SCOPE_AGENT);
        __syncthreads();
        if (s_ticket == clast - cfirst) {
            if (first) {
                pend0 = true;
                pg0 = G;
            } else {
                pend1 = true;
                pg1 = G;
            }
        }
    };

    uint32_t gcur = b0 / KB, gstart = b0;
    bool first_seg = true;
    for (uint32_t b = b0; b < b1; b += kGemvDepth) {
#pragma unroll
        for (uint32_t d = 0; d < kGemvDepth; d++) {
            const uint32_t bb = b + d;
            constexpr uint32_t nx = kGemvDepth - 1;
            load(buf[(d + nx) % kGemvDepth], min(bb + nx, b1 - 1));
            // Keep the scheduler from sinking these loads below the math of
            // block bb (it would, to reuse their registers).
            __builtin_amdgcn_sched_barrier(0);
            if (bb < b1) {
                const uint32_t G = bb / KB;
                if (G != gcur) {
                    flush(gcur, gstart, bb, first_seg);
                    first_seg = false;
                    gcur = G;
                    gstart = bb;
                    acc = zero;
                }
                compute(buf[d], __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, sc_lane), bb - b0)),
                        bb - b0);
            }
        }
    }
    flush(gcur, gstart, b1, first_seg);

    // ---- ordered sums of split groups this workgroup finished last ----
    // Device-scope loads read the coherence point; each thread owns up to
    // four outputs and fetches their partials four contributions at a time,
    // adding them in range order.
    auto reduce = [&](uint32_t G) {
        const uint32_t cfirst = range_of((uint64_t)G * KB, T, P);
        const uint32_t nc = range_of((uint64_t)G * KB + KB - 1, T, P) - cfirst + 1;
        const uint32_t per_c = M * kBlock;
        const float *base = p.ws + sg.ws_off + (size_t)G * sg.maxc * (kGemvMaxM * kBlock);
        constexpr uint32_t kOut = kGemvMaxM * kBlock / kGemvThreads;   // 4
        float sum[kOut];
#pragma unroll
        for (uint32_t o = 0; o < kOut; o++) sum[o] = 0.0f;
        for (uint32_t c0 = 0; c0 < nc; c0 += 4) {
            float v[4][kOut];
#pragma unroll
            for (uint32_t u = 0; u < 4; u++)
#pragma unroll
                for (uint32_t o = 0; o < kOut; o++) {
                    const uint32_t i = threadIdx.x + o * kGemvThreads;
                    const uint32_t j = min(c0 + u, nc - 1);
                    v[u][o] = i < per_c ? __hip_atomic_load(base + (size_t)j * kGemvMaxM * kBlock + i,
                                                            __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                                        : 0.0f;
                }
#pragma unroll
            for (uint32_t u = 0; u < 4; u++)
#pragma unroll
                for (uint32_t o = 0; o < kOut; o++)
                    if (c0 + u < nc) sum[o] = (c0 + u == 0) ? v[u][o] : sum[o] + v[u][o];
        }
#pragma unroll
        for (uint32_t o = 0; o < kOut; o++) {
            const uint32_t i = threadIdx.x + o * kGemvThreads;
            const uint32_t t = i >> 7, r2 = G * kBlock + (i & 127);
            if (i < per_c && r2 < sg.rows) {
                const size_t o2 = (size_t)t * sg.ldy + r2;
                sg.y[o2] = sg.resid ? sg.resid[o2] + sum[o] : sum[o];
            }
        }
        if (threadIdx.x == 0)
            __hip_atomic_store(p.cnt + sg.cnt_off + G, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    };
    if (pend0) reduce(pg0);
    if (pend1) reduce(pg1);
}

uint32_t gemv_ctas(uint32_t nblocks, uint32_t cus, uint32_t per_cu) {
    // A whole number of workgroups per CU keeps every CU's byte count equal;
    // ranges are capped at kGemvMaxRangeBlocks (LDS stage at m = 8).
    uint32_t P = cus * per_cu;
    const uint32_t need = (nblocks + kGemvMaxRangeBlocks - 1) / kGemvMaxRangeBlocks;
    if (P < need) P = ((need + cus - 1) / cus) * cus;
    if (P > nblocks) P = nblocks;
    return P;
}

uint32_t gemv_max_contrib(uint32_t nblocks, uint32_t nctas, uint32_t kb) {
    // Ranges have at least floor(T/P) blocks, so a group of kb blocks meets
    // at most ceil((kb - 1) / floor(T/P)) + 1 of them.
    const uint32_t minlen = nblocks / nctas;
    return (kb - 1 + minlen - 1) / minlen + 1;
}

size_t gemv_lds_bytes(uint32_t m, uint32_t range_blocks) {
    return (size_t)range_blocks * 256 * stage_rows(m) + 16;   // + zero slot
}

bool gemv_norm_fits(uint32_t m, uint32_t k) {
    return m >= 1 && m <= kGemvMaxM && (uint64_t)m * ((k + 7) & ~7u) <= kGemvThreads * kGemvNormBatch * 4;
}

uint32_t gemv_norm_cols(uint32_t k) { return (k + 31) & ~31u; }

size_t gemv_norm_lds_bytes(uint32_t m, uint32_t norm_cols) {
    return (size_t)m * 8 * (norm_cols / 8 + 4) * sizeof(float);
}

hipError_t launch_gemv(const GemvParams &p, hipStream_t stream) {
    using Kernel = void (*)(GemvParams);
    static const Kernel kernels[6] = {gemv_fp8_kernel<kXPlain, false>,   gemv_fp8_kernel<kXRmsNorm, false>,
                                      gemv_fp8_kernel<kXSwiGLU, false>,  gemv_fp8_kernel<kXPlain, true>,
                                      gemv_fp8_kernel<kXRmsNorm, true>,  gemv_fp8_kernel<kXSwiGLU, true>};
    static bool attr_set = false;
    if (!attr_set) {
        for (Kernel k : kernels) {
            hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(k),
                                               hipFuncAttributeMaxDynamicSharedMemorySize, (int)kGemvMaxLds);
            if (e != hipSuccess) return e;
        }
        attr_set = true;
    }
    if (p.xmode > kXSwiGLU || p.m == 0 || p.m > kGemvMaxM) return hipErrorInvalidValue;
    size_t lds = gemv_lds_bytes(p.m, p.max_range);
    if (p.xmode == kXRmsNorm) {
        if (!gemv_norm_fits(p.m, p.k) || p.norm_cols != gemv_norm_cols(p.k)) return hipErrorInvalidValue;
        lds = std::max(lds, gemv_norm_lds_bytes(p.m, p.norm_cols));
    }
    if (lds > kGemvMaxLds) return hipErrorInvalidValue;
    hipLaunchKernelGGL(kernels[p.xmode + (p.x_vec ? 3 : 0)], dim3(p.nctas), dim3(kGemvThreads), lds, stream, p);
    return hipGetLastError();
}

}  // namespace q35mm
