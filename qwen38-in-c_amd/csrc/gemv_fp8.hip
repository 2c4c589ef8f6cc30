// gemv_fp8.hip -- decode GEMV, m <= 8 tokens, FP8-E4M3 weights with
// 128x128 fp32 block scales, fp32-accurate.
//
// Replaces the hot loop of qwen35-c/src/q35_mm.c:88-198 (mm_fp8_row called
// by q35_mm_fp8 / q35_mm_fp8_batch / q35_mm_fp8_multi4).
//
// Work decomposition.  A workgroup of four wavefronts owns one 128-row group
// (one scale row-block) and a slice of the K blocks; wavefront w owns the
// 32-row sub-tile w.  Each wavefront streams its weights with one 16-byte
// load per lane per 1 KiB chunk (the lane-order tile layout makes every load
// a contiguous 1 KiB), converts e4m3 -> bf16 in registers (exact) and feeds
// v_mfma_f32_32x32x16_bf16.
//
// Activations are fp32.  To keep fp32 accuracy on a bf16 matrix core, every
// activation is split exactly into three bf16 parts x = p0 + p1 + p2; the A
// operand rows are m = t + 8p (token t < 8, part p < 3), so one MFMA computes
// the three partial dot products of up to eight tokens at once.  The
// products e4m3*bf16 are exact in fp32; the only rounding is the fp32
// accumulation.  Per 128-column K block the MFMA accumulator holds the raw
// block dot product, which is then multiplied by the block's fp32 scale and
// added to the running sum (one fmaf per output and block).
//
// Split-K: when a slice does not cover all K blocks, each workgroup writes
// its partial outputs to a workspace, and the last workgroup of a row group
// to arrive (device-scope atomic ticket) adds the partials in slice order
// and writes y.  The order is fixed, so results do not depend on timing, and
// the slice count depends only on the weight shape, so a batch of m tokens
// gives exactly the bits of m single-token calls.
#include "q35mm_device.h"
#include "q35mm_internal.h"

namespace q35mm {

namespace {

__device__ __forceinline__ u32x4_t ld16(const uint8_t *p) {
    return *reinterpret_cast<const u32x4_t *>(p);
}

// Stage the three-part bf16 split of x[t][kb0*128 .. (kb0+nkb)*128) for
// t < m into LDS in MFMA A-operand order:
//   byte offset(c, q, ai, h) = (((c*2 + q) * R + ai) * 2 + h) * 16
// where c is the slice-relative 32-column chunk, q selects the first or the
// second MFMA of the chunk, ai = part*m + t, R = 3m, h = lane/32, and the 16
// bytes hold columns c*32 + 16h + 8q + (0..7).
__device__ void stage_split_x(uint8_t *lds, const float *x, uint32_t ldx, uint32_t m,
                              uint32_t k, uint32_t kb0, uint32_t nkb) {
    const uint32_t R = 3 * m;
    const uint32_t per_t = nkb * 16;               // 8-column vectors per token
    const uint32_t nvec = m * per_t;
    for (uint32_t i = threadIdx.x; i < nvec; i += blockDim.x) {
        const uint32_t t = i / per_t;
        const uint32_t kk = (i - t * per_t) * 8;   // slice-relative column
        const uint32_t kg = kb0 * kBlock + kk;     // global column
        const float *xp = x + (size_t)t * ldx + kg;
        float v[8];
#pragma unroll
        for (int e = 0; e < 8; e++) v[e] = (kg + e < k) ? xp[e] : 0.0f;
        uint32_t p0[8], p1[8], p2[8];
#pragma unroll
        for (int e = 0; e < 8; e++) split3_bf16(v[e], p0[e], p1[e], p2[e]);
        const uint32_t c = kk >> 5, h = (kk >> 4) & 1, q = (kk >> 3) & 1;
        const uint32_t base = (c * 2 + q) * R;
        u32x4_t w0 = {p0[0] | (p0[1] << 16), p0[2] | (p0[3] << 16),
                      p0[4] | (p0[5] << 16), p0[6] | (p0[7] << 16)};
        u32x4_t w1 = {p1[0] | (p1[1] << 16), p1[2] | (p1[3] << 16),
                      p1[4] | (p1[5] << 16), p1[6] | (p1[7] << 16)};
        u32x4_t w2 = {p2[0] | (p2[1] << 16), p2[2] | (p2[3] << 16),
                      p2[4] | (p2[5] << 16), p2[6] | (p2[7] << 16)};
        *reinterpret_cast<u32x4_t *>(lds + ((base + 0 * m + t) * 2 + h) * 16) = w0;
        *reinterpret_cast<u32x4_t *>(lds + ((base + 1 * m + t) * 2 + h) * 16) = w1;
        *reinterpret_cast<u32x4_t *>(lds + ((base + 2 * m + t) * 2 + h) * 16) = w2;
    }
}

}  // namespace

__global__ __launch_bounds__(kGemvThreads) void gemv_fp8_kernel(GemvParams p) {
    extern __shared__ __align__(16) uint8_t lds[];
    __shared__ uint32_t s_ticket;

    // ---- which segment / row group / K slice ----
    const uint32_t b = blockIdx.x;
    uint32_t si = 0;
#pragma unroll
    for (uint32_t i = 1; i < 4; i++)
        if (i < p.nseg && b >= p.seg[i].cta_begin) si = i;
    const GemvSeg sg = p.seg[si];
    const uint32_t S = sg.nslices;
    const uint32_t local = b - sg.cta_begin;
    const uint32_t g = local / S;
    const uint32_t s = local - g * S;
    const uint32_t KB = p.kb;
    const uint32_t kb0 = (s * KB) / S;
    const uint32_t kb1 = ((s + 1) * KB) / S;
    const uint32_t M = p.m;

    stage_split_x(lds, p.x, p.ldx, M, p.k, kb0, kb1 - kb0);
    __syncthreads();

    // ---- per-lane roles ----
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t wv = threadIdx.x >> 6;         // 32-row sub-tile
    const uint32_t mrow = lane & 31, hh = lane >> 5;
    const uint32_t tt = mrow & 7, pp = mrow >> 3;  // A row = token + 8*part
    const bool a_active = (tt < M) && (pp < 3);
    const uint32_t R = 3 * M;
    const uint32_t a_lane_off = ((pp * M + tt) * 2 + hh) * 16;

    const uint8_t *wbase = sg.codes + (size_t)g * KB * kBlockBytes + wv * kSubBytes + lane * 16;
    const float *srow = sg.scale + (size_t)g * KB;

    f32x16_t acc = {};
    const f32x16_t zero = {};

    auto compute = [&](const u32x4_t (&wq)[4], uint32_t kb) {
        const uint32_t cbase = (kb - kb0) * 4;
        f32x16_t part;
#pragma unroll
        for (int j = 0; j < 4; j++) {
#pragma unroll
            for (int q = 0; q < 2; q++) {
                const bf16x8_t bop = e4m3x8_to_bf16x8(wq[j][2 * q], wq[j][2 * q + 1]);
                u32x4_t araw = {0u, 0u, 0u, 0u};
                if (a_active)
                    araw = *reinterpret_cast<const u32x4_t *>(
                        lds + ((cbase + j) * 2 + q) * R * 32 + a_lane_off);
                const bf16x8_t aop = __builtin_bit_cast(bf16x8_t, araw);
                part = mfma32x32x16(aop, bop, (j == 0 && q == 0) ? zero : part);
            }
        }
        const float sc = srow[kb];
        // Rows 24..31 of the A operand are never used (regs 12..15).
#pragma unroll
        for (int r = 0; r < 12; r++) acc[r] = __builtin_fmaf(sc, part[r], acc[r]);
    };

    // ---- stream the slice, one K block of loads ahead ----
    u32x4_t wa[4], wb[4];
    auto load = [&](u32x4_t (&dst)[4], uint32_t kb) {
        const uint8_t *src = wbase + (size_t)kb * kBlockBytes;
#pragma unroll
        for (int j = 0; j < 4; j++) dst[j] = ld16(src + j * kChunkBytes);
    };
    load(wa, kb0);
    for (uint32_t kb = kb0; kb < kb1; kb += 2) {
        if (kb + 1 < kb1) load(wb, kb + 1);
        compute(wa, kb);
        if (kb + 1 < kb1) {
            if (kb + 2 < kb1) load(wa, kb + 2);
            compute(wb, kb + 1);
        }
    }

    // ---- combine the three parts: token t = 4*hh + r ----
    float yv[4];
#pragma unroll
    for (int r = 0; r < 4; r++) yv[r] = (acc[r] + acc[r + 4]) + acc[r + 8];
    const uint32_t row_local = wv * 32 + mrow;
    const uint32_t row = g * kBlock + row_local;

    if (S == 1) {
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const uint32_t t = 4 * hh + r;
            if (t < M && row < sg.rows) sg.y[(size_t)t * sg.ldy + row] = yv[r];
        }
        return;
    }

    float *ws = p.ws + sg.ws_off;
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const uint32_t t = 4 * hh + r;
        if (t < M) ws[(((size_t)g * S + s) * kGemvMaxM + t) * kBlock + row_local] = yv[r];
    }
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) s_ticket = atomicAdd(p.cnt + sg.cnt_off + g, 1u);
    __syncthreads();
    if (s_ticket != S - 1) return;

    // Last workgroup of this row group: every other slice has published.
    __threadfence();
    for (uint32_t i = threadIdx.x; i < M * kBlock; i += blockDim.x) {
        const uint32_t t = i >> 7, rl = i & 127;
        const float *src = ws + ((size_t)g * S * kGemvMaxM + t) * kBlock + rl;
        float sum = __builtin_nontemporal_load(src);
        for (uint32_t s2 = 1; s2 < S; s2++)
            sum += __builtin_nontemporal_load(src + (size_t)s2 * kGemvMaxM * kBlock);
        const uint32_t r2 = g * kBlock + rl;
        if (r2 < sg.rows) sg.y[(size_t)t * sg.ldy + r2] = sum;
    }
    if (threadIdx.x == 0) p.cnt[sg.cnt_off + g] = 0u;
}

uint32_t gemv_slices(uint32_t nb, uint32_t kb) {
    // Aim for about two workgroups per CU on a 256-CU part, keep every slice
    // at most kGemvMaxSliceKb blocks (LDS stage) and at least two blocks.
    const uint32_t target = 512;
    uint32_t s = (target + nb - 1) / nb;
    const uint32_t s_min = (kb + kGemvMaxSliceKb - 1) / kGemvMaxSliceKb;
    const uint32_t s_max = kb >= 2 ? kb / 2 : 1;
    if (s > s_max) s = s_max;
    if (s < s_min) s = s_min;
    if (s < 1) s = 1;
    if (s > kb) s = kb;
    return s;
}

hipError_t launch_gemv(const GemvParams &p, uint32_t grid, uint32_t max_slice_kb,
                       hipStream_t stream) {
    const size_t lds = (size_t)max_slice_kb * kBlock * 3 * p.m * 2;
    hipLaunchKernelGGL(gemv_fp8_kernel, dim3(grid), dim3(kGemvThreads), lds, stream, p);
    return hipGetLastError();
}

}  // namespace q35mm
