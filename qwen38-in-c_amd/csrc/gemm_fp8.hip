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
//  - A workgroup computes a 256x256 output tile with eight wavefronts of
//    128 (tokens) x 64 (weight rows), two per SIMD: 8 accumulators of 32x32,
//    128 VGPRs, so the per-block rescale below is a plain v_mul.  (64 x 128
//    wavefront tiles read 20% fewer LDS bytes per MFMA but convert twice the
//    e4m3 codes; they ran 4% slower.)  Up to 128 tokens the tile is 128 x 512
//    (the eight wavefronts side by side along the rows, same per-wavefront
//    code), so a short batch is not three quarters padding.
//  - K advances in stages of 64 columns (two 32-column chunks).  A stage is
//    48 KiB of LDS: A as bf16 (32 KiB) and B still as e4m3 (16 KiB); B is
//    widened to bf16 after the LDS read, exactly.  Stages are copied straight
//    from global memory into a three-deep LDS ring with global_load_lds
//    (no register staging), issued two stages ahead.
//  - Block scales: a wavefront's 64 output columns lie in one 128-row scale
//    block, so for each 128-wide K block its scale s is one number.  The
//    accumulator is kept in units of the last nonzero scale: before block kb
//    it is multiplied by s_prev / s_kb, after the last block by s_last.  One
//    v_mul per accumulator and K block, and the scale is never folded into
//    bf16 weights (that would round).  The multiplies and the conversions are
//    spread over the MFMAs (at most five and one per MFMA), never in bursts.
//  - Work split: whole rounds of tiles unsplit; the tiles of a last partial
//    round either cut into 64x64 tiles, run by the whole-tile workgroups
//    after their own tile while its stores drain (or by gemm_tail_kernel
//    when there is no whole round), or cut along K, their partial tiles added
//    in slice order by a second kernel (deterministic, spread over the whole
//    device).
//  - Two weights of one shape (the MLP's gate and up) run as paired tiles:
//    the first half of a tile's rows from one, the same rows of the other in
//    the second half, so each output of one sits in the same workgroup as the
//    same output of the other.  The MLP block uses that to form silu(gate) *
//    up in the epilogue and write it, rounded to bf16, as the down GEMM's
//    activations.
#include <algorithm>
#include <cstdlib>
#include <type_traits>
#include <utility>

#include "q35mm_device.h"
#include "q35mm_internal.h"

namespace q35mm {

namespace {

typedef __attribute__((address_space(3))) uint8_t lds_u8;

constexpr uint32_t kStageK = 64;                          // two 32-column chunks
constexpr uint32_t kStageA = kGemmTile * kStageK * 2;     // 32 KiB bf16
constexpr uint32_t kStageB = kGemmTile * kStageK;         // 16 KiB e4m3
constexpr uint32_t kStageBytes = kStageA + kStageB;       // 48 KiB
constexpr uint32_t kRing = 3;
constexpr uint32_t kScaleOff = kRing * kStageBytes;       // 144 KiB: [2][kGemmMaxSliceKb] fp32
constexpr uint32_t kGemmLds = kScaleOff + 2 * kGemmMaxSliceKb * 4;
constexpr uint32_t kALoads = 4;    // 1 KiB pieces of A per wavefront per stage
constexpr uint32_t kBLoads = 2;    // 1 KiB pieces of B per wavefront per stage
constexpr uint32_t kStageLoads = kALoads + kBLoads;
static_assert(8 * kALoads * kChunkBytes == kStageA, "A pieces");
static_assert(8 * kBLoads * kChunkBytes == kStageB, "B pieces");

// Tile geometry.  The standard tile is 256 tokens x 256 weight rows; for
// m <= 128 the narrow tile is 128 tokens x 512 rows, so a short batch does
// not run a mostly empty 256-token tile.  Either way each of the eight
// wavefronts computes 128 tokens x 64 rows, a stage is 48 KiB and every
// wavefront issues six copies per stage; only the split of a stage between
// A and B and the wavefronts' places in the tile differ.
template <bool NARROW>
struct GemmGeo {
    static constexpr uint32_t kTM = NARROW ? 128 : kGemmTile;        // tokens per tile
    static constexpr uint32_t kTR = NARROW ? 4 * 128 : kGemmTile;    // weight rows per tile
    static constexpr uint32_t kA = kTM * kStageK * 2;                // A bytes per stage
    static constexpr uint32_t kAL = kA / kChunkBytes / 8;            // A pieces per wavefront per stage
    static constexpr uint32_t kBL = kTR * kStageK / kChunkBytes / 8; // B pieces per wavefront per stage
    static constexpr uint32_t kGroups = kTR / kBlock;                // 128-row scale groups per tile
    static constexpr uint32_t kSliceKb = 2 * kGemmMaxSliceKb / kGroups;   // scale table per group
};
static_assert(GemmGeo<true>::kAL + GemmGeo<true>::kBL == kStageLoads, "six copies per stage");
static_assert(GemmGeo<true>::kA + GemmGeo<true>::kTR * kStageK == kStageBytes, "48 KiB stage");
static_assert(GemmGeo<true>::kTM * GemmGeo<true>::kTR == kGemmTile * kGemmTile, "partial tiles of one size");
static_assert(kGemmLds <= 160 * 1024, "LDS");

// One wavefront copies 1 KiB: lane l's 16 bytes at g go to LDS l*16 past l.
// The LDS address must be the same for all lanes (it goes through M0).
// s_waitcnt immediate that waits only for vmcnt <= n (gfx9 encoding:
// vmcnt[3:0] in bits 3:0, vmcnt[5:4] in 15:14, expcnt 6:4, lgkmcnt 11:8).
constexpr uint32_t waitcnt_vm(uint32_t n) { return (n & 15u) | ((n >> 4) << 14) | (7u << 4) | (15u << 8); }
constexpr uint32_t kWaitLgkm0 = 15u | (3u << 14) | (7u << 4);   // lgkmcnt(0) only

// Plain s_barrier.  __syncthreads() adds workgroup fences that wait for every
// outstanding global load (vmcnt(0)), which would drain the copies in flight
// for the next stages; the caller waits for exactly the copies it needs.  The
// barrier is a memory side effect to the compiler, so no LDS access moves
// across it.
__device__ __forceinline__ void lds_barrier() { __builtin_amdgcn_s_barrier(); }

__device__ __forceinline__ void dma_1k(const uint8_t *g, lds_u8 *l) {
    __builtin_amdgcn_global_load_lds(g, l, 16, 0, 0);
}

// The segment (weight) of a tile and the tile's position in it.  MULTI is a
// compile-time choice: a single-weight launch indexes segment 0 statically,
// which keeps the main kernel's registers as they are without segments.
struct TileAt {
    uint32_t seg, mt, nt;
};
template <bool MULTI>
__device__ __forceinline__ TileAt tile_at(const GemmParams &p, uint32_t tile) {
    uint32_t s = 0;
    if constexpr (MULTI) {
#pragma unroll
        for (uint32_t i = 1; i < 4; i++)
            if (i < p.nseg && tile >= p.seg[i].tile0) s = i;
    }
    const uint32_t lt = MULTI ? tile - p.seg[s].tile0 : tile;
    return {s, lt % p.mtiles, lt / p.mtiles};
}

// s_waitcnt immediate that waits only for lgkmcnt <= n.
constexpr uint32_t waitcnt_lgkm(uint32_t n) { return 15u | (3u << 14) | (7u << 4) | ((n & 15u) << 8); }

// One v_cvt_scalef32_pk_bf16_fp8: codes 0,1 (HI false) or 2,3 (HI true) of w
// to two bf16, packed.
template <bool HI>
__device__ __forceinline__ uint32_t cvt_pk(uint32_t w, float keep) {
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, keep, HI));
}

// f(std::integral_constant<uint32_t, I>) for I = 0..N-1, each call its own
// code (indices known at compile time, whatever the unroller decides).
template <class F, uint32_t... I>
__device__ __forceinline__ void static_for_impl(F &&f, std::integer_sequence<uint32_t, I...>) {
    (f(std::integral_constant<uint32_t, I>{}), ...);
}
template <uint32_t N, class F>
__device__ __forceinline__ void static_for(F &&f) {
    static_for_impl(f, std::make_integer_sequence<uint32_t, N>{});
}

// Where the per-K-block rescale goes.  Accumulator a runs MFMAs
// 2a and 2a+1 of every 16-MFMA phase, so between its last MFMA of block kb
// (slot 2a+1 of the block's last phase) and its first of block kb+1 (slot 2a
// of the next phase) lie 14 slots; its 16 values are multiplied in slots
// 2a+3 .. 2a+15 of the 32 (last phase: g = t, next phase: g = 16 + t), at
// most five multiplies per slot, earliest window first.  Issued in one burst
// after one MFMA, 16 multiplies hold back the wavefront's next MFMA by ~64
// cycles; five fit beside the 32-cycle MFMA.
struct RescalePlan {
    uint8_t cnt[32][8];
    uint8_t first[32][8];
};
constexpr uint32_t kRescaleCap = 5;
constexpr RescalePlan make_rescale_plan() {
    RescalePlan pl{};
    uint32_t done[8] = {};
    for (uint32_t g = 0; g < 32; g++) {
        uint32_t cap = kRescaleCap;
        for (uint32_t a = 0; a < 8; a++) {
            pl.cnt[g][a] = 0;
            pl.first[g][a] = 0;
            if (g < 2 * a + 3 || g > 2 * a + 15 || cap == 0) continue;
            const uint32_t n = cap < 16 - done[a] ? cap : 16 - done[a];
            pl.cnt[g][a] = (uint8_t)n;
            pl.first[g][a] = (uint8_t)done[a];
            done[a] += n;
            cap -= n;
        }
    }
    return pl;
}
constexpr RescalePlan kRescale = make_rescale_plan();
constexpr bool rescale_plan_complete() {
    uint32_t tot[8] = {};
    for (uint32_t g = 0; g < 32; g++)
        for (uint32_t a = 0; a < 8; a++) tot[a] += kRescale.cnt[g][a];
    for (uint32_t a = 0; a < 8; a++)
        if (tot[a] != 16) return false;
    return true;
}
static_assert(rescale_plan_complete(), "every accumulator value rescaled once per K block");

}  // namespace

// X fp32 [m][ldx] -> bf16 (round to nearest even) in lane order.  Output
// unit u = ((m32 * KB + kb) * 8 + j*2 + q) * 64 + lane holds 16 bytes:
//   row = m32*32 + lane%32, columns kb*128 + j*32 + (lane/32)*16 + q*8 + e.
// One workgroup converts one 32-row x 128-column block: coalesced row reads
// (512 B per row), a transpose through LDS, and 8 KiB of contiguous writes.
// Rows >= m and columns >= k are zero.  With SWIGLU the converted value is
// silu(x) * x2 (q35_kern_swiglu's arithmetic, swiglu1) of two inputs with the
// same layout: the bits of swiglu_kernel followed by the plain conversion,
// without writing and re-reading the fp32 product.
template <bool SWIGLU>
__global__ __launch_bounds__(256) void act_to_bf16_kernel(const float *__restrict__ x,
                                                          const float *__restrict__ x2, uint32_t ldx,
                                                          uint32_t m, uint32_t k, uint32_t kb_total,
                                                          uint16_t *__restrict__ xb) {
    __shared__ __align__(16) uint16_t t[32][128 + 8];     // +8: spread rows over banks
    const uint32_t kb = blockIdx.x % kb_total;
    const uint32_t m32 = blockIdx.x / kb_total;
    // Each thread's four 16-byte pieces (32 rows x 32 float4): all loads are
    // issued before the first is used, one memory round trip instead of four
    // (the whole kernel is a few microseconds).  Pieces past k or unaligned
    // take the element path below.
    auto piece = [&](uint32_t i, uint32_t &r, uint32_t &c4, uint32_t &row, uint32_t &col) {
        const uint32_t idx = threadIdx.x + 256 * i;
        r = idx >> 5;
        c4 = idx & 31;
        row = m32 * 32 + r;
        col = kb * kBlock + c4 * 4;
    };
    float4 fa[4], fb[4];
    bool fast[4];
#pragma unroll
    for (uint32_t i = 0; i < 4; i++) {
        uint32_t r, c4, row, col;
        piece(i, r, c4, row, col);
        const size_t o = (size_t)row * ldx + col;
        fast[i] = row < m && col + 4 <= k && ((reinterpret_cast<uintptr_t>(x + o) & 15) == 0) &&
                  (!SWIGLU || ((reinterpret_cast<uintptr_t>(x2 + o) & 15) == 0));
        if (fast[i]) {
            fa[i] = *reinterpret_cast<const float4 *>(x + o);
            if constexpr (SWIGLU) fb[i] = *reinterpret_cast<const float4 *>(x2 + o);
        }
    }
#pragma unroll
    for (uint32_t i = 0; i < 4; i++) {
        uint32_t r, c4, row, col;
        piece(i, r, c4, row, col);
        float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        if (row < m) {
            const size_t o = (size_t)row * ldx + col;
            float a[4] = {0.0f, 0.0f, 0.0f, 0.0f}, b[4] = {0.0f, 0.0f, 0.0f, 0.0f};
            if (fast[i]) {
                a[0] = fa[i].x; a[1] = fa[i].y; a[2] = fa[i].z; a[3] = fa[i].w;
                if constexpr (SWIGLU) {
                    b[0] = fb[i].x; b[1] = fb[i].y; b[2] = fb[i].z; b[3] = fb[i].w;
                }
            } else {
#pragma unroll
                for (uint32_t e = 0; e < 4; e++)
                    if (col + e < k) {
                        a[e] = x[o + e];
                        if constexpr (SWIGLU) b[e] = x2[o + e];
                    }
            }
#pragma unroll
            for (uint32_t e = 0; e < 4; e++) {
                if constexpr (SWIGLU)
                    v[e] = col + e < k ? swiglu1(a[e], b[e]) : 0.0f;
                else
                    v[e] = a[e];
                v[e] = bf16_saturate(v[e]);
            }
        }
        u32x2_t w = {f32x2_to_bf16x2_rne(v[0], v[1]), f32x2_to_bf16x2_rne(v[2], v[3])};
        *reinterpret_cast<u32x2_t *>(&t[r][c4 * 4]) = w;
    }
    __syncthreads();
    uint8_t *out = reinterpret_cast<uint8_t *>(xb) + ((size_t)m32 * kb_total + kb) * 8 * kChunkBytes;
#pragma unroll
    for (uint32_t i = 0; i < 2; i++) {
        const uint32_t u = threadIdx.x + 256 * i;           // 0..511
        const uint32_t lane = u & 63, jq = u >> 6;
        const uint32_t r = lane & 31, c = (jq >> 1) * 32 + (lane >> 5) * 16 + (jq & 1) * 8;
        const u32x4_t v = *reinterpret_cast<const u32x4_t *>(&t[r][c]);
        *reinterpret_cast<u32x4_t *>(out + u * 16) = v;
    }
}

// ---- the tail of a partial last round as 64x64 output tiles ----
// When the tiles of the last round are few (at most one per 16 CUs), each
// is cut into sixteen 64x64 output tiles, one workgroup per small tile.
// Its eight wavefronts split K into contiguous K-block ranges and stream
// their operands from memory straight into registers (nothing is shared
// between wavefronts, so no LDS staging), each accumulating the whole 64x64
// tile (2x2 MFMA tiles of 32x32) with the main kernel's arithmetic: bf16
// operands, the accumulator kept in units of the last live block scale.
// The eight partial tiles are added through LDS in wavefront order.  Against
// K slices of whole 256x256 tiles this writes and re-reads no partial tiles
// (64 MB for the 16 leftover tiles of a 512 x 34816 x 5120 product) and
// needs no reduction kernel.
// Activation t, column c of the lane-order bf16 layout act_to_bf16_kernel
// writes (per 32 tokens x 128 columns 8 KiB; unit 64*jq + 32*h + t%32 of
// 16 bytes holds columns 32*(jq/2) + 16*h + 8*(jq%2) .. +7), rounded as that
// kernel rounds.
__device__ __forceinline__ void store_act_bf16(uint16_t *act, uint32_t act_kb, uint32_t t, uint32_t c, float v) {
    const uint32_t cc = c % kBlock;
    const uint32_t u = ((cc >> 5) * 2 + ((cc >> 3) & 1)) * 64 + ((cc >> 4) & 1) * 32 + t % 32;
    act[((size_t)(t / 32) * act_kb + c / kBlock) * (4 * kChunkBytes) + u * 8 + (cc & 7)] =
        (uint16_t)(f32x2_to_bf16x2_rne(v, 0.0f) & 0xFFFFu);
}

// silu(g) * u of a paired tile, as act_to_bf16_kernel<true> forms it before
// rounding.
__device__ __forceinline__ float paired_swiglu(float g, float u) { return bf16_saturate(swiglu1(g, u)); }

constexpr uint32_t kTailTile = 64;
constexpr uint32_t kTailPerTile = (kGemmTile / kTailTile) * (kGemmTile / kTailTile);   // 16
constexpr uint32_t kTailDepth = 4;                                                      // chunks in flight
constexpr uint32_t kTailLds = (kGemmThreads / 64) * kTailTile * kTailTile * 4;          // 128 KiB
static_assert(kTailLds <= 160 * 1024, "LDS");

// PM (paired segments, GemmParams::pair): 0 -- no pairing; 1 -- the small
// tile holds 32 rows of segment 0 and the same 32 rows of segment 1, fp32
// outputs; 2 -- the same, writing silu(segment 0) * segment 1 as bf16
// activations.
template <bool MULTI, uint32_t PM>
__device__ __forceinline__ void tail_tile(const GemmParams &p, uint32_t idx, uint8_t *lds) {
    static_assert(!(MULTI && PM), "paired tiles come from two segments of one shape");
    const uint32_t tile = p.tail_tile0 + idx / kTailPerTile, st = idx % kTailPerTile;
    const TileAt ta = tile_at<MULTI>(p, tile);
    const GemmSeg &sg = p.seg[ta.seg];
    const uint32_t row0 = ta.mt * kGemmTile + (st & 3) * kTailTile;   // token rows
    // weight rows: 64 of one weight, or (paired) 32 of each segment
    const uint32_t col0 = PM ? ta.nt * (kGemmTile / 2) + (st >> 2) * (kTailTile / 2)
                             : ta.nt * kGemmTile + (st >> 2) * kTailTile;
    if (col0 >= sg.nb * kBlock) return;   // the whole workgroup: no work
    if (row0 >= p.m) {
        if constexpr (PM == 2) {   // padding tokens of the activation layout: zeros
#pragma unroll
            for (uint32_t k = 0; k < 4; k++) {
                const uint32_t q = threadIdx.x * 4 + k;   // 64 tokens x 32 columns
                store_act_bf16(p.act_out, p.act_kb, row0 + q / 32, col0 + q % 32, 0.0f);
            }
        }
        return;
    }

    const uint32_t lane = threadIdx.x & 63;
    const uint32_t wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t KB = p.kb;
    const uint32_t nw = kGemmThreads / 64;
    const uint32_t k0 = wv * KB / nw, k1 = (wv + 1) * KB / nw;        // empty when KB < nw
    const uint32_t g = col0 / kBlock, s0 = (col0 % kBlock) / kSubRows; // weight group, first sub-tile
    const uint32_t m32 = row0 / kSubRows;
    const uint8_t *xa = reinterpret_cast<const uint8_t *>(p.xb) + lane * 16;
    // B of MFMA column tile ni: sub-tile s0 + ni of the weight, or (paired)
    // sub-tile s0 of segment ni; one scale track per weight read.
    constexpr uint32_t NS = PM ? 2 : 1;
    const uint8_t *wb[NS];
    const float *sc_g[NS];
#pragma unroll
    for (uint32_t z = 0; z < NS; z++) {
        const GemmSeg &bs = PM ? p.seg[z] : sg;
        wb[z] = bs.codes + (size_t)g * KB * kBlockBytes + s0 * kSubBytes + lane * 16;
        sc_g[z] = bs.scale + (size_t)g * KB;
    }

    // Chunk c = 4 * (kb - k0) + j (32 columns): A for the two 32-row token
    // sub-tiles and both MFMA halves, B (16 e4m3 codes per lane) for the
    // two 32-row weight sub-tiles.
    struct Chunk {
        u32x4_t a[2][2];
        u32x4_t b[2];
    };
    auto load = [&](Chunk &ch, uint32_t c) {
        const uint32_t kb = k0 + c / 4, j = c % 4;
#pragma unroll
        for (uint32_t mi = 0; mi < 2; mi++)
#pragma unroll
            for (uint32_t q = 0; q < 2; q++)
                ch.a[mi][q] = *reinterpret_cast<const u32x4_t *>(
                    xa + ((size_t)((m32 + mi) * KB + kb) * 8 + j * 2 + q) * kChunkBytes);
#pragma unroll
        for (uint32_t ni = 0; ni < 2; ni++)
            ch.b[ni] = *reinterpret_cast<const u32x4_t *>(wb[PM ? ni : 0] + (size_t)kb * kBlockBytes +
                                                           (PM ? 0 : ni) * kSubBytes + j * kChunkBytes);
    };

    f32x16_t acc[2][2] = {};
    float s_prev[NS] = {};   // units of the accumulators (0: nothing live yet)
    if (k1 > k0) {
        const uint32_t nc = (k1 - k0) * 4;
        Chunk ring[kTailDepth];
#pragma unroll
        for (uint32_t d = 0; d + 1 < kTailDepth; d++) load(ring[d], min(d, nc - 1));
        float keep[NS], sc_next[NS];
#pragma unroll
        for (uint32_t z = 0; z < NS; z++) {
            keep[z] = 1.0f;
            sc_next[z] = sc_g[z][k0];
        }
        for (uint32_t c0 = 0; c0 < nc; c0 += kTailDepth) {
#pragma unroll
            for (uint32_t d = 0; d < kTailDepth; d++) {
                const uint32_t c = c0 + d;
                load(ring[(d + kTailDepth - 1) % kTailDepth], min(c + kTailDepth - 1, nc - 1));
                __builtin_amdgcn_sched_barrier(0);
                if (c < nc) {
                    if ((c & 3) == 0) {
                        // a new K block: bring the accumulator into its units
                        // (block scale 0: the conversion scale 0 acts as
                        // 2^-127, as in the main kernel)
                        const uint32_t kb = k0 + c / 4;
#pragma unroll
                        for (uint32_t z = 0; z < NS; z++) {
                            const float sc = sc_next[z];
                            sc_next[z] = sc_g[z][min(kb + 1, k1 - 1)];
                            const bool live = sc != 0.0f;
                            keep[z] = live ? 1.0f : 0.0f;
                            const float r = live ? (s_prev[z] != 0.0f ? s_prev[z] / sc : 0.0f) : 1.0f;
#pragma unroll
                            for (uint32_t mi = 0; mi < 2; mi++)
#pragma unroll
                                for (uint32_t ni = 0; ni < 2; ni++)
                                    if (!PM || ni == z) acc[mi][ni] *= r;
                            s_prev[z] = live ? sc : s_prev[z];
                        }
                    }
                    const Chunk &ch = ring[d];
#pragma unroll
                    for (uint32_t q = 0; q < 2; q++) {
                        bf16x8_t bw[2];
#pragma unroll
                        for (uint32_t ni = 0; ni < 2; ni++)
                            bw[ni] = e4m3x8_to_bf16x8_cvt(ch.b[ni][2 * q], ch.b[ni][2 * q + 1], keep[PM ? ni : 0]);
#pragma unroll
                        for (uint32_t mi = 0; mi < 2; mi++)
#pragma unroll
                            for (uint32_t ni = 0; ni < 2; ni++)
                                acc[mi][ni] = mfma32x32x16(__builtin_bit_cast(bf16x8_t, ch.a[mi][q]), bw[ni],
                                                           acc[mi][ni]);
                    }
                }
            }
        }
    }

    // ---- partial tiles -> LDS (lane-major, 16 values per lane and MFMA
    // tile), then added in wavefront order ----
    float *red = reinterpret_cast<float *>(lds);
#pragma unroll
    for (uint32_t a = 0; a < 4; a++) {
        f32x16_t v = acc[a >> 1][a & 1] * s_prev[PM ? (a & 1) : 0];
#pragma unroll
        for (uint32_t r4 = 0; r4 < 4; r4++)
            *reinterpret_cast<float4 *>(red + ((wv * 4 + a) * 64 + lane) * 16 + 4 * r4) =
                make_float4(v[4 * r4], v[4 * r4 + 1], v[4 * r4 + 2], v[4 * r4 + 3]);
    }
    __syncthreads();
    // thread t: MFMA tile a = (t / 64) % 4, lane l = t % 64, values 8h..8h+7
    const uint32_t l = threadIdx.x & 63, a = (threadIdx.x >> 6) & 3, h = threadIdx.x >> 8;
    float sum[8];
#pragma unroll
    for (uint32_t w = 0; w < kGemmThreads / 64; w++) {
        const float *src = red + ((w * 4 + a) * 64 + l) * 16 + 8 * h;
        const float4 u0 = *reinterpret_cast<const float4 *>(src);
        const float4 u1 = *reinterpret_cast<const float4 *>(src + 4);
        const float v[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
#pragma unroll
        for (uint32_t e = 0; e < 8; e++) sum[e] = w == 0 ? v[e] : sum[e] + v[e];
    }
    const uint32_t mi = a >> 1, ni = a & 1;
    auto row_of = [&](uint32_t e) {
        const uint32_t r = 8 * h + e;
        return row0 + mi * 32 + 8 * (r >> 2) + 4 * (l >> 5) + (r & 3);
    };
    if constexpr (PM == 2) {
        // silu(segment 0) * segment 1: the segment-1 threads hand their sums
        // to the segment-0 threads of the same lane and values through LDS
        float *xu = reinterpret_cast<float *>(lds) + (mi * 64 + l) * 16 + 8 * h;
        __syncthreads();   // every thread is done reading the partial tiles
        if (ni == 1) {
#pragma unroll
            for (uint32_t e = 0; e < 8; e++) xu[e] = sum[e];
        }
        __syncthreads();
        if (ni == 0) {
            const uint32_t col = col0 + (l & 31);
#pragma unroll
            for (uint32_t e = 0; e < 8; e++) {
                const uint32_t row = row_of(e);
                const float y = row < p.m && col < sg.rows ? paired_swiglu(sum[e], xu[e]) : 0.0f;
                store_act_bf16(p.act_out, p.act_kb, row, col, y);
            }
        }
        return;
    }
    const GemmSeg &os = PM ? p.seg[ni] : sg;
    const uint32_t col = col0 + (PM ? 0 : ni * 32) + (l & 31);
    if (col < os.rows) {
#pragma unroll
        for (uint32_t e = 0; e < 8; e++) {
            const uint32_t row = row_of(e);
            if (row < p.m) {
                const size_t o = (size_t)row * os.ldy + col;
                os.y[o] = os.resid ? os.resid[o] + sum[e] : sum[e];
            }
        }
    }
}

template <bool MULTI, uint32_t PM>
__global__ __launch_bounds__(kGemmThreads) void gemm_tail_kernel(GemmParams p) {
    extern __shared__ __align__(16) uint8_t lds[];
    tail_tile<MULTI, PM>(p, blockIdx.x, lds);
}

// PM (paired segments, GemmParams::pair): 0 -- none; 1 -- each tile holds
// kTR/2 rows of segment 0 in its first half and the same rows of segment 1
// in its second, fp32 outputs; 2 -- the same, writing silu(segment 0) *
// segment 1 as bf16 activations (split tiles publish partials as usual and
// gemm_reduce_kernel<..., 2> forms the products).
template <bool MULTI, bool NARROW, uint32_t PM = 0>
__global__ __launch_bounds__(kGemmThreads) void gemm_fp8_kernel(GemmParams p) {
    static_assert(!(MULTI && PM), "paired tiles come from two segments of one shape");
    constexpr uint32_t kTM = 4, kTN = 2;   // 32x32 MFMA tiles per wavefront: 128 tokens x 64 rows
    using Geo = GemmGeo<NARROW>;
    extern __shared__ __align__(16) uint8_t lds[];
    lds_u8 *const ring = (lds_u8 *)lds;

    const bool split = blockIdx.x >= p.split_tile0;
    const uint32_t S = split ? p.nslices : 1;
    const uint32_t u = split ? blockIdx.x - p.split_tile0 : 0;
    const uint32_t tile = split ? p.split_tile0 + u / S : blockIdx.x;
    const uint32_t sl = split ? u % S : 0;
    const TileAt ta = tile_at<MULTI>(p, tile);
    const GemmSeg &sg = p.seg[ta.seg];
    const uint32_t mt = ta.mt, nt = ta.nt;
    const uint32_t KB = p.kb;
    const uint32_t kb0 = (sl * KB) / S, kb1 = ((sl + 1) * KB) / S;
    const uint32_t st0 = 2 * kb0, st1 = 2 * kb1;   // stages of 64 columns

    const uint32_t lane = threadIdx.x & 63;
    const uint32_t wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // standard: 2 x 4 wavefronts of 128 x 64; narrow: 1 x 8
    const uint32_t wm = NARROW ? 0 : wv & 1, wn = NARROW ? wv : wv >> 1;
    constexpr uint32_t kHW = (NARROW ? 8 : 4) / 2;   // paired: wn < kHW hold segment 0's rows

    // ---- global sources of this wavefront's pieces ----
    // A piece P (0 .. 4*kTM/32 - 1): token rows (mt*kTM/32 + P/4)*32..,
    // piece (h*4 + P%4) of the K block's eight (h = stage half); wavefront w
    // copies pieces w*kAL ...  B piece Q: weight rows (nt*kTR/32 + Q/2)*32..,
    // chunk 2h + Q%2; wavefront w copies w*kBL ...  A missing row group
    // (NB not a multiple of the tile's groups) reads the last group instead;
    // those columns are never stored.
    const uint8_t *xa = reinterpret_cast<const uint8_t *>(p.xb);
    // Byte offsets (32-bit: the host keeps both operands under 4 GiB) that are
    // wavefront-uniform, so they live in scalar registers; each copy adds the
    // lane's 16 bytes and uses the global_load_lds saddr + voffset form.
    uint32_t aoff[Geo::kAL], boff[Geo::kBL];
    const uint32_t lane16 = lane * 16;
#pragma unroll
    for (uint32_t i = 0; i < Geo::kAL; i++) {
        const uint32_t P = wv * Geo::kAL + i;
        aoff[i] = (mt * (Geo::kTM / 32) + P / 4) * (KB * 8 * kChunkBytes) + (P % 4) * kChunkBytes;
    }
#pragma unroll
    for (uint32_t i = 0; i < Geo::kBL; i++) {
        const uint32_t Q = wv * Geo::kBL + i;
        const uint32_t n32 = Q / 2;
        // paired: 32-row groups [0, kTR/64) of segment 0, then the same of 1
        const uint32_t n32p = PM && n32 >= Geo::kTR / 64 ? n32 - Geo::kTR / 64 : n32;
        const uint32_t nbk = PM ? min(nt * (Geo::kGroups / 2) + n32p / 4, sg.nb - 1)
                                : min(nt * Geo::kGroups + n32 / 4, sg.nb - 1);
        boff[i] = nbk * KB * kBlockBytes + (n32p % 4) * kSubBytes + (Q % 2) * kChunkBytes;
    }
    // paired: the groups one wavefront copies all lie in one segment's half
    const uint8_t *bcodes = PM ? p.seg[wv * Geo::kBL / 2 >= Geo::kTR / 64 ? 1 : 0].codes : sg.codes;
    // Copy k of stage st into ring slot buf: k < kAL an A piece, then the
    // B pieces.
    auto issue_piece = [&](uint32_t st, uint32_t buf, uint32_t k) {
        const uint32_t kb = st >> 1, h = st & 1;
        lds_u8 *la = ring + buf * kStageBytes;
        if (k < Geo::kAL) {
            dma_1k(xa + (aoff[k] + kb * 8 * kChunkBytes + h * 4 * kChunkBytes + lane16),
                   la + (wv * Geo::kAL + k) * kChunkBytes);
        } else {
            const uint32_t i = k - Geo::kAL;
            dma_1k(bcodes + (boff[i] + kb * kBlockBytes + h * 2 * kChunkBytes + lane16),
                   la + Geo::kA + (wv * Geo::kBL + i) * kChunkBytes);
        }
    };
    auto issue = [&](uint32_t st, uint32_t buf) {
#pragma unroll
        for (uint32_t k = 0; k < kStageLoads; k++) issue_piece(st, buf, k);
    };

    // ---- block scales of the tile's row groups, staged in LDS ----
    // The loop takes them from registers (one K block per lane, refilled
    // every 64 blocks), so no LDS read of a scale sits between its MFMAs and
    // nothing waits for one there.  The table is copied global -> LDS like
    // the stages (4-byte global_load_lds, issued just before the first
    // stages' copies), so its latency is the copies' and no register waits
    // for it: loaded into registers first, one round trip at a time behind a
    // branch, it held back the first copy by a memory round trip or two.
    // Entries past the slice's K range repeat its last block (never read);
    // a row group past the weight's last repeats that group's scales (its
    // rows are never stored).
    constexpr uint32_t kScPer = 2 * kGemmMaxSliceKb / kGemmThreads;
    float *sc_lds = reinterpret_cast<float *>(lds + kScaleOff);
    {
        const uint32_t nkb = kb1 > kb0 ? kb1 - kb0 : 1u;
#pragma unroll
        for (uint32_t i = 0; i < kScPer; i++) {
            const uint32_t j0 = wv * 64 + i * kGemmThreads;   // the wavefront's first entry
            const uint32_t j = j0 + lane;
            const uint32_t g = j / Geo::kSliceKb, kk = min(j % Geo::kSliceKb, nkb - 1);
            const uint32_t gs = PM && g >= Geo::kGroups / 2 ? 1 : 0;   // paired: the group's segment
            const uint32_t nbg = PM ? min(nt * (Geo::kGroups / 2) + g - gs * (Geo::kGroups / 2), sg.nb - 1)
                                    : min(nt * Geo::kGroups + g, sg.nb - 1);
            const float *gsc = PM ? (gs ? p.seg[1].scale : p.seg[0].scale) : sg.scale;
            __builtin_amdgcn_global_load_lds(gsc + (size_t)nbg * KB + kb0 + kk, (lds_u8 *)(lds + kScaleOff) + j0 * 4,
                                             4, 0, 0);
        }
    }
    issue(st0, 0);
    issue(min(st0 + 1, st1 - 1), 1);
    issue(min(st0 + 2, st1 - 1), 2);
    const float *my_sc = sc_lds + (wn >> 1) * Geo::kSliceKb - kb0;   // indexed by kb
    uint32_t sc_base = kb0;                                           // lane i holds block sc_base + i
    float sc_lane = 0.0f;   // read once the table has landed (below)
    auto scale_of = [&](uint32_t kb) {   // kb in [sc_base, sc_base + 64)
        return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, sc_lane), kb - sc_base));
    };

    f32x16_t acc[kTM][kTN] = {};
    float s_prev = 0.0f;

    // Operands of one 32-column chunk: A for this wavefront's 4 token
    // sub-tiles x 2 MFMA halves (bf16), B for its 2 weight sub-tiles (16 e4m3
    // codes per lane, both halves).  Read from LDS one 1 KiB piece at a time.
    struct Frags {
        bf16x8_t a[kTM][2];
        u32x4_t b[kTN];
    };
    constexpr uint32_t kPieces = 2 * kTM + kTN;   // 10
    static_assert(kStageLoads + kPieces == 16, "one copy or read per MFMA of a phase");
    auto read_a = [&](Frags &f, uint32_t buf, uint32_t jj, uint32_t i, uint32_t q) {
        const uint8_t *la = lds + buf * kStageBytes;
        f.a[i][q] = *reinterpret_cast<const bf16x8_t *>(la + (((wm * kTM + i) * 2 + jj) * 2 + q) * kChunkBytes +
                                                        lane * 16);
    };
    auto read_b = [&](Frags &f, uint32_t buf, uint32_t jj, uint32_t jn) {
        const uint8_t *la = lds + buf * kStageBytes;
        f.b[jn] = *reinterpret_cast<const u32x4_t *>(la + Geo::kA + ((wn * kTN + jn) * 2 + jj) * kChunkBytes +
                                                     lane * 16);
    };
    // ---- pipeline ----
    // LDS ring of three stages (64 columns each, two per K block).  Stage s:
    // its first chunk's operands are in registers (f0) when it starts; the
    // second chunk's are read (f1) during the first chunk's MFMAs.  Then,
    // once every wavefront has read all of stage s and stage s+1 has landed
    // (one barrier), stage s+3 is copied into s's slot and stage s+1's first
    // chunk is read during the second chunk's MFMAs.  Every wavefront issues
    // exactly kStageLoads copies per stage (clamped to the last stage past
    // the end), so "vmcnt <= kStageLoads" means: all but the newest stage
    // have landed.
    //
    // Block scales: the accumulator is kept in units of the last live block
    // scale.  Before the MFMAs of block kb+1 it is multiplied by r = s_prev /
    // s_{kb+1}, after its last MFMA of block kb and before its first of block
    // kb+1, so each accumulator sees the same products in the same order as
    // with one multiply at the block boundary.  A block with scale 0 runs
    // with keep = 0 and r = 1, so the accumulator keeps its units.  keep is
    // the conversion's power-of-two scale: 1.0 (exact) for a live block, 0.0
    // (= 2^-127) for a block whose scale is 0, which then adds at most
    // 2^-127 * 448 * |x| per term (and NaN for a NaN code, as lut[code] * 0
    // does).  No branches around the MFMAs.  (The scale table and the first
    // three stages were issued above: vmcnt <= 2 * kStageLoads means the
    // table and stage st0 have landed.)
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(2 * kStageLoads));
    lds_barrier();
    sc_lane = my_sc[min(sc_base + lane, kb1 - 1)];
    Frags f0, f1;
    uint32_t buf = 0;
    // B first, so the next phase's first B sub-tile can be converted
    // while this phase's second half runs
    read_b(f0, 0, 0, 0);
    read_b(f0, 0, 0, 1);
#pragma unroll
    for (uint32_t k = 0; k < 2 * kTM; k++) read_a(f0, 0, 0, k >> 1, k & 1);
    __builtin_amdgcn_s_waitcnt(kWaitLgkm0);   // f0 and the first scales
    const float sc0 = scale_of(kb0);
    const bool live = sc0 != 0.0f;
    float keep = live ? 1.0f : 0.0f;
    float r = live ? 0.0f : 1.0f;            // the accumulator is still zero
    s_prev = live ? sc0 : 0.0f;              // units of the accumulator after this block

    // Each phase runs its 16 MFMAs accumulator by accumulator, both
    // halves of a chunk back to back (slot t: accumulator a = t / 2,
    // half q = t % 2; a = 4 jn + i, so B sub-tile 0 serves slots 0..7 and
    // sub-tile 1 slots 8..15).  Beside MFMA t, pinned there
    // (sched_barrier), at most one piece of each kind of other work:
    //  - t < 8: one conversion of this phase's B sub-tile 1 (needed from
    //    slot 8);  t >= 8: one conversion of the next phase's sub-tile 0
    //    (needed at its slot 0; its LDS read was the phase's first);
    //  - t < 10: the next phase's LDS reads (B sub-tiles, then A);
    //    t >= 10 in a stage's second phase: the stage copies;
    //  - in a K block's last phase and the next block's first, the
    //    rescale plan's multiplies.
    // No burst of VALU work holds back an MFMA: a wavefront's 16
    // multiplies after one MFMA, or 8 conversions before one, delay its
    // next MFMA by 30-60 cycles.
    u32x4_t bw0[2], bw1[2];   // converted B sub-tiles 0 (this phase) and 1, halves q
    auto cvt_part = [&](u32x4_t (&bw)[2], const u32x4_t &raw, uint32_t c, float kp) {
        const uint32_t q = c >> 2, part = c & 3, w = raw[2 * q + (part >> 1)];
        bw[q][part] = (part & 1) ? cvt_pk<true>(w, kp) : cvt_pk<false>(w, kp);
    };
#pragma unroll
    for (uint32_t c = 0; c < 8; c++) cvt_part(bw0, f0.b[0], c, keep);
    // phase: f = this phase's operands, fn = the next phase's (read into);
    // g0 = rescale plan offset (0: last phase of a block, 16: first
    // phase of a block, 32: none); second = the stage's second phase
    // (copies of stage st_copy into ring slot cbuf).
    auto phase = [&](const Frags &f, Frags &fn, uint32_t nbuf, uint32_t njj, float kp, float kp_next,
                     auto g0c, float rr, auto secondc, uint32_t st_copy, uint32_t cbuf) {
        constexpr uint32_t g0 = decltype(g0c)::value;
        constexpr bool second = decltype(secondc)::value;
        static_for<16>([&](auto tc) {
            constexpr uint32_t t = decltype(tc)::value;
            constexpr uint32_t a = t >> 1, q = t & 1, i = a & 3, jn = a >> 2;
            if constexpr (jn == 0)
                acc[i][0] = mfma32x32x16(f.a[i][q], __builtin_bit_cast(bf16x8_t, bw0[q]), acc[i][0]);
            else
                acc[i][1] = mfma32x32x16(f.a[i][q], __builtin_bit_cast(bf16x8_t, bw1[q]), acc[i][1]);
            if constexpr (t < 8) {
                cvt_part(bw1, f.b[1], t, kp);
            } else {
                if constexpr (t == 8) __builtin_amdgcn_s_waitcnt(waitcnt_lgkm(7));   // fn.b[0]: read first
                cvt_part(bw0, fn.b[0], t - 8, kp_next);
            }
            if constexpr (t < 2)
                read_b(fn, nbuf, njj, t);
            else if constexpr (t < kPieces)
                read_a(fn, nbuf, njj, (t - 2) >> 1, t & 1);
            else if constexpr (second)
                issue_piece(st_copy, cbuf, t - kPieces);
            if constexpr (g0 < 32) {
                static_for<8>([&](auto acc_c) {
                    constexpr uint32_t ac = decltype(acc_c)::value;
                    constexpr uint32_t n = kRescale.cnt[g0 + t][ac], e0 = kRescale.first[g0 + t][ac];
                    static_for<n>([&](auto ec) { acc[ac & 3][ac >> 2][e0 + decltype(ec)::value] *= rr; });
                });
            }
            __builtin_amdgcn_sched_barrier(0);
        });
    };
    for (uint32_t kb = kb0; kb < kb1; kb++) {
        if (kb + 1 == sc_base + 64) {
            sc_base += 64;
            sc_lane = my_sc[min(sc_base + lane, kb1 - 1)];
            __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
        }
        const bool live_n = kb + 1 < kb1 && scale_of(min(kb + 1, kb1 - 1)) != 0.0f;
        const float sc_n = live_n ? scale_of(kb + 1) : 1.0f;
        const float keep_n = live_n ? 1.0f : 0.0f;
        const float r_n = live_n ? (s_prev != 0.0f ? s_prev / sc_n : 0.0f) : 1.0f;
        const float s_prev_n = live_n ? sc_n : s_prev;
        __builtin_amdgcn_sched_barrier(0);
        static_for<2>([&](auto hc) {
            constexpr uint32_t h = decltype(hc)::value;
            const uint32_t st = 2 * kb + h;
            using G0a = std::integral_constant<uint32_t, h == 0 ? 16 : 32>;   // a block's first phase
            using G0b = std::integral_constant<uint32_t, h == 1 ? 0 : 32>;    // a block's last phase
            __builtin_amdgcn_s_waitcnt(kWaitLgkm0);   // f0 was read during the previous phase
            phase(f0, f1, buf, 1, keep, keep, G0a{}, r, std::false_type{}, 0, 0);
            __builtin_amdgcn_s_waitcnt(waitcnt_vm(kStageLoads));
            __builtin_amdgcn_s_waitcnt(kWaitLgkm0);   // f1 is in registers: slot st is free
            lds_barrier();
            const uint32_t nb = buf == 2 ? 0 : buf + 1;
            // past the end the reads of f0 are unused (in bounds)
            phase(f1, f0, nb, 0, keep, h == 1 ? keep_n : keep, G0b{}, r_n, std::true_type{},
                  min(st + 3, st1 - 1), buf);
            buf = nb;
        });
        keep = keep_n;
        r = r_n;
        s_prev = s_prev_n;
    }
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));   // no copy outlives the loop
#pragma unroll
    for (uint32_t i = 0; i < kTM; i++)
#pragma unroll
        for (uint32_t jn = 0; jn < kTN; jn++) acc[i][jn] *= s_prev;

    // Output coordinates of accumulator element (i, jn, r) of this lane.
    auto out_row = [&](uint32_t i, uint32_t r) -> uint32_t {
        return wm * (32 * kTM) + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
    };
    auto out_col = [&](uint32_t jn) -> uint32_t { return wn * (32 * kTN) + jn * 32 + (lane & 31); };

    if (!split) {
        if constexpr (PM == 0) {
#pragma unroll
            for (uint32_t i = 0; i < kTM; i++)
#pragma unroll
                for (uint32_t jn = 0; jn < kTN; jn++)
#pragma unroll
                    for (uint32_t e = 0; e < 16; e++) {
                        const uint32_t mrow = mt * Geo::kTM + out_row(i, e);
                        const uint32_t ncol = nt * Geo::kTR + out_col(jn);
                        if (mrow < p.m && ncol < sg.rows) {
                            const size_t o = (size_t)mrow * sg.ldy + ncol;
                            __builtin_nontemporal_store(sg.resid ? sg.resid[o] + acc[i][jn][e] : acc[i][jn][e],
                                                        sg.y + o);
                        }
                    }
        } else {
            // Paired: this wavefront holds rows of segment hs; its column
            // within that segment's half of the tile.
            const uint32_t hs = wn >= kHW ? 1 : 0;
            auto pcol = [&](uint32_t jn) {
                return nt * (Geo::kTR / 2) + (wn - hs * kHW) * 64 + jn * 32 + (lane & 31);
            };
            if constexpr (PM == 1) {
                float *oy = hs ? p.seg[1].y : p.seg[0].y;
#pragma unroll
                for (uint32_t i = 0; i < kTM; i++)
#pragma unroll
                    for (uint32_t jn = 0; jn < kTN; jn++)
#pragma unroll
                        for (uint32_t e = 0; e < 16; e++) {
                            const uint32_t mrow = mt * Geo::kTM + out_row(i, e);
                            const uint32_t ncol = pcol(jn);
                            if (mrow < p.m && ncol < sg.rows)
                                __builtin_nontemporal_store(acc[i][jn][e], oy + (size_t)mrow * sg.ldy + ncol);
                        }
            } else {
                // silu(segment 0) * segment 1.  The wavefronts (wm, wn) and
                // (wm, wn + kHW) hold the same outputs of the two segments;
                // segment 0's forms token sub-tiles 0 and 1 of the pair,
                // segment 1's sub-tiles 2 and 3, each handing the other the
                // accumulators it needs through LDS (the ring is free).
                float *xch = reinterpret_cast<float *>(lds);
                const uint32_t pi = wm * kHW + (wn - hs * kHW);
                auto xat = [&](uint32_t side, uint32_t t4, uint32_t e) -> float & {
                    return xch[(((pi * 2 + side) * 4 + t4) * 16 + e) * 64 + lane];
                };
                auto hand_over = [&](auto basec) {   // accumulators basec, basec + 1 into side hs
                    constexpr uint32_t base = decltype(basec)::value;
#pragma unroll
                    for (uint32_t ii = 0; ii < 2; ii++)
#pragma unroll
                        for (uint32_t jn = 0; jn < kTN; jn++)
#pragma unroll
                            for (uint32_t e = 0; e < 16; e++) xat(hs, ii * 2 + jn, e) = acc[base + ii][jn][e];
                };
                auto form = [&](auto basec) {   // sub-tiles basec, basec + 1 with the other side's values
                    constexpr uint32_t base = decltype(basec)::value;
#pragma unroll
                    for (uint32_t ii = 0; ii < 2; ii++)
#pragma unroll
                        for (uint32_t jn = 0; jn < kTN; jn++)
#pragma unroll
                            for (uint32_t e = 0; e < 16; e++) {
                                const float own = acc[base + ii][jn][e], other = xat(1 - hs, ii * 2 + jn, e);
                                const uint32_t mrow = mt * Geo::kTM + out_row(base + ii, e);
                                const uint32_t ncol = pcol(jn);
                                if (ncol < p.act_kb * kBlock)
                                    store_act_bf16(p.act_out, p.act_kb, mrow, ncol,
                                                   mrow < p.m && ncol < sg.rows
                                                       ? paired_swiglu(hs ? other : own, hs ? own : other)
                                                       : 0.0f);
                            }
                };
                __syncthreads();   // every wavefront is done reading the ring
                if (hs)
                    hand_over(std::integral_constant<uint32_t, 0>{});
                else
                    hand_over(std::integral_constant<uint32_t, 2>{});
                __syncthreads();
                if (hs)
                    form(std::integral_constant<uint32_t, 2>{});
                else
                    form(std::integral_constant<uint32_t, 0>{});
            }
        }
        // One 64x64 tile of the last round's tail, while these stores drain
        // (every workgroup reaches this point at about the same time, when
        // the device's write bandwidth bounds the stores).
        if constexpr (!NARROW) {
            if (blockIdx.x < p.tail_fused) {
                __syncthreads();   // the ring is free: every wavefront is past its last LDS read
                tail_tile<MULTI, PM>(p, blockIdx.x, lds);
            }
        }
        return;
    }

    // ---- split tile: publish this slice's partial ----
    // Stored in the accumulator layout, float4 q of thread t (q = (i*2 + jn)*4
    // + r/4) at (q*512 + t)*16 bytes of the slice's 256 KiB, so every store is
    // a coalesced 16-byte access; gemm_reduce maps it back to (row, column).
    // A float4 holds four consecutive token rows; one whose first row is past
    // m holds padding only and is neither stored nor read back (at m = 64 on
    // 128-token tiles, half of every partial).
    const size_t slot = (size_t)(tile - p.split_tile0) * S + sl;
    float4 *part = reinterpret_cast<float4 *>(p.ws + slot * kGemmTile * kGemmTile);
#pragma unroll
    for (uint32_t q = 0; q < 32; q++) {
        const uint32_t i = q / (4 * kTN), jn = (q / 4) % kTN, r4 = q & 3;
        if (mt * Geo::kTM + out_row(i, 4 * r4) < p.m)
            part[q * kGemmThreads + threadIdx.x] = make_float4(acc[i][jn][4 * r4], acc[i][jn][4 * r4 + 1],
                                                               acc[i][jn][4 * r4 + 2], acc[i][jn][4 * r4 + 3]);
    }
}

// Ordered sum of the K slices of split tiles: y = ((p_0 + p_1) + p_2) + ...
// One thread per float4 of a partial tile (16384 per tile); the layout is
// the one gemm_fp8_kernel publishes.  Runs after it on the same stream, so
// the partials are visible without any device-scope protocol.  PM = 1:
// paired tiles (fp32 outputs), whose second half of columns belongs to
// segment 1; PM = 2: the same tiles forming silu(segment 0) * segment 1 as
// bf16 activations.
template <bool MULTI, bool NARROW, uint32_t PM = 0>
__global__ __launch_bounds__(256) void gemm_reduce_kernel(GemmParams p) {
    using Geo = GemmGeo<NARROW>;
    constexpr uint32_t kTileQuads = kGemmTile * kGemmTile / 4;
    const uint32_t f = blockIdx.x * 256 + threadIdx.x;
    const uint32_t st = f / kTileQuads;                 // split tile index
    const uint32_t fq = f - st * kTileQuads;
    const uint32_t tile = p.split_tile0 + st;
    const uint32_t S = p.nslices;
    // accumulator layout -> output coordinates (as out_row / out_col)
    const uint32_t t = fq % kGemmThreads, q = fq / kGemmThreads;
    const uint32_t lane = t & 63, wv = t >> 6, wm = NARROW ? 0 : wv & 1, wn = NARROW ? wv : wv >> 1;
    const uint32_t i = q >> 3, jn = (q >> 2) & 1, r4 = q & 3;
    const TileAt ta = tile_at<MULTI>(p, tile);
    const uint32_t row0 = ta.mt * Geo::kTM + wm * 128 + i * 32 + 8 * r4 + 4 * (lane >> 5);
    constexpr uint32_t kHW = (NARROW ? 8 : 4) / 2;
    if constexpr (PM == 2) {
        // The threads of segment 0's columns sum both segments' partials
        // (segment 1's float4 of the same outputs sits kGemmThreads / 2
        // threads further in the layout), in slice order as below, and
        // write four tokens of one column; padding tokens and columns past
        // the weight's rows as zeros.
        if (wn >= kHW) return;
        const uint32_t col = ta.nt * (Geo::kTR / 2) + wn * 64 + jn * 32 + (lane & 31);
        if (col >= p.act_kb * kBlock) return;
        float y[4] = {};
        if (row0 < p.m && col < p.seg[0].rows) {
            const float4 *pg = reinterpret_cast<const float4 *>(p.ws) + (size_t)st * S * kTileQuads + fq;
            const float4 *pu = pg + kGemmThreads / 2;
            float4 vg[4], vu[4];
            float4 tg = pg[0], tu = pu[0];
            for (uint32_t s0 = 1; s0 < S; s0 += 4) {
#pragma unroll
                for (uint32_t b = 0; b < 4; b++)
                    if (s0 + b < S) {
                        vg[b] = pg[(size_t)(s0 + b) * kTileQuads];
                        vu[b] = pu[(size_t)(s0 + b) * kTileQuads];
                    }
#pragma unroll
                for (uint32_t b = 0; b < 4; b++)
                    if (s0 + b < S) {
                        tg.x += vg[b].x;
                        tg.y += vg[b].y;
                        tg.z += vg[b].z;
                        tg.w += vg[b].w;
                        tu.x += vu[b].x;
                        tu.y += vu[b].y;
                        tu.z += vu[b].z;
                        tu.w += vu[b].w;
                    }
            }
            const float g4[4] = {tg.x, tg.y, tg.z, tg.w}, u4[4] = {tu.x, tu.y, tu.z, tu.w};
#pragma unroll
            for (uint32_t e = 0; e < 4; e++)
                if (row0 + e < p.m) y[e] = paired_swiglu(g4[e], u4[e]);
        }
#pragma unroll
        for (uint32_t e = 0; e < 4; e++) store_act_bf16(p.act_out, p.act_kb, row0 + e, col, y[e]);
        return;
    }
    if (row0 >= p.m) return;   // padding rows: never stored by the slices
    const uint32_t hs = PM && wn >= kHW ? 1 : 0;
    const GemmSeg &sg = p.seg[PM ? hs : ta.seg];
    const uint32_t col = PM ? ta.nt * (Geo::kTR / 2) + (wn - hs * kHW) * 64 + jn * 32 + (lane & 31)
                            : ta.nt * Geo::kTR + wn * 64 + jn * 32 + (lane & 31);
    // The residuals (y may be the residual, updated in place) are loaded
    // first, all four together with the rows and the column clamped in
    // bounds: loaded one by one between the stores, each waited for the
    // store before it (the compiler cannot tell y from the residual).
    float rv[4] = {};
    if (sg.resid) {
        const uint32_t c = min(col, sg.rows - 1);
#pragma unroll
        for (uint32_t e = 0; e < 4; e++) rv[e] = sg.resid[(size_t)min(row0 + e, p.m - 1) * sg.ldy + c];
    }
    const float4 *part = reinterpret_cast<const float4 *>(p.ws) + (size_t)st * S * kTileQuads + fq;
    // Up to eight slices' loads in flight, each behind a uniform test (S is
    // the launch's) rather than clamped to the last slice: a clamped load
    // still costs its 16 bytes per lane of cache bandwidth.
    float4 v[8];
    float4 tot = part[0];
    for (uint32_t s0 = 1; s0 < S; s0 += 8) {
#pragma unroll
        for (uint32_t b = 0; b < 8; b++)
            if (s0 + b < S) v[b] = part[(size_t)(s0 + b) * kTileQuads];
#pragma unroll
        for (uint32_t b = 0; b < 8; b++)
            if (s0 + b < S) {
                tot.x += v[b].x;
                tot.y += v[b].y;
                tot.z += v[b].z;
                tot.w += v[b].w;
            }
    }
    const float tv[4] = {tot.x, tot.y, tot.z, tot.w};
    if (col < sg.rows) {
#pragma unroll
        for (uint32_t e = 0; e < 4; e++)
            if (row0 + e < p.m) {
                const size_t o = (size_t)(row0 + e) * sg.ldy + col;
                sg.y[o] = sg.resid ? rv[e] + tv[e] : tv[e];
            }
    }
}

GemmPlan gemm_plan(uint32_t m, uint32_t ntiles, uint32_t kb, uint32_t cus, bool narrow) {
    // Whole rounds of tiles run unsplit; the tiles of the last, partial round
    // are cut so that round fills the device too:
    //  - into 64x64 tiles when those fit one round (gemm_tail_kernel);
    //  - otherwise along K, as many slices as fill the CUs (a slice keeps at
    //    least two K blocks, four pipeline stages).
    // (Just over half a round -- 136 tiles of a 512 x 17408 x 5120 product
    // -- runs one slice per tile: cutting half a round's tiles in two and the
    // rest into 64x64 tiles took the main kernel from 110 to 80 us, but the
    // slice reduction and the tail added 33 us.)
    // A K range longer than the LDS scale table (kGemmMaxSliceKb blocks)
    // splits every tile along K.
    // Narrow tiles (m <= 128) have no 64x64 tail: their partial round is cut
    // along K, and their scale table holds half as many K blocks per group.
    GemmPlan pl{};
    pl.narrow = narrow;
    const uint32_t tm = narrow ? GemmGeo<true>::kTM : GemmGeo<false>::kTM;
    const uint32_t slice_kb = narrow ? GemmGeo<true>::kSliceKb : GemmGeo<false>::kSliceKb;
    pl.mtiles = (m + tm - 1) / tm;
    pl.ntiles = ntiles;
    const uint32_t tiles = pl.mtiles * pl.ntiles;
    pl.tail_tile0 = tiles;
    pl.nslices = 1;
    const uint32_t smin = (kb + slice_kb - 1) / slice_kb;
    if (smin > 1) {
        pl.split_tile0 = 0;
        pl.nslices = smin;
        return pl;
    }
    const uint32_t whole = tiles / cus * cus;
    const uint32_t rest = tiles - whole;
    pl.split_tile0 = tiles;
    if (!rest) return pl;
    if (!narrow && rest * kTailPerTile <= cus) {
        pl.split_tile0 = pl.tail_tile0 = whole;
        return pl;
    }
    const uint32_t s = std::min(cus / rest, std::max(1u, kb / 2));
    if (s > 1) {
        pl.split_tile0 = whole;
        pl.nslices = s;
    }
    return pl;
}

hipError_t launch_act_to_bf16(const float *x, const float *x2, uint32_t ldx, uint32_t m, uint32_t k,
                              uint32_t m32_tiles, uint32_t kb, uint16_t *xb, hipStream_t stream) {
    if (x2)
        hipLaunchKernelGGL(act_to_bf16_kernel<true>, dim3(m32_tiles * kb), dim3(256), 0, stream, x, x2, ldx, m, k,
                           kb, xb);
    else
        hipLaunchKernelGGL(act_to_bf16_kernel<false>, dim3(m32_tiles * kb), dim3(256), 0, stream, x, x2, ldx, m, k,
                           kb, xb);
    return hipGetLastError();
}

static bool fuse_tail() {
    static const bool on = [] {
        const char *v = getenv("Q35MM_GEMM_FUSE_TAIL");
        return !(v && v[0] == '0');
    }();
    return on;
}

template <bool MULTI, bool NARROW, uint32_t PM = 0>
static hipError_t launch_gemm_t(const GemmParams &p, hipStream_t stream) {
    static bool attr_set = false;
    if (!attr_set) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(gemm_fp8_kernel<MULTI, NARROW, PM>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)kGemmLds);
        if (e == hipSuccess && !NARROW)
            e = hipFuncSetAttribute(reinterpret_cast<const void *>(gemm_tail_kernel<MULTI, PM>),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, (int)kTailLds);
        if (e != hipSuccess) return e;
        attr_set = true;
    }
    if (NARROW && p.tail_tile0 != p.mtiles * p.ntiles) return hipErrorInvalidValue;   // no 64x64 tail
    const uint32_t tiles = p.mtiles * p.ntiles;
    const uint32_t nsplit = p.tail_tile0 - p.split_tile0;   // tiles cut along K
    const uint32_t grid = p.split_tile0 + nsplit * p.nslices;
    const uint32_t ntail = (tiles - p.tail_tile0) * kTailPerTile;   // 64x64 tiles
    GemmParams q = p;
    // the 64x64 tiles run in the whole-tile workgroups, after their stores
    q.tail_fused = (ntail && !nsplit && p.split_tile0 >= ntail && fuse_tail()) ? ntail : 0;
    if (grid)
        hipLaunchKernelGGL((gemm_fp8_kernel<MULTI, NARROW, PM>), dim3(grid), dim3(kGemmThreads), kGemmLds, stream, q);
    if (nsplit) {
        const uint32_t quads = nsplit * (kGemmTile * kGemmTile / 4);
        hipLaunchKernelGGL((gemm_reduce_kernel<MULTI, NARROW, PM>), dim3(quads / 256), dim3(256), 0, stream, p);
    }
    if constexpr (!NARROW) {
        if (ntail && !q.tail_fused)
            hipLaunchKernelGGL((gemm_tail_kernel<MULTI, PM>), dim3(ntail), dim3(kGemmThreads), kTailLds, stream, q);
    }
    return hipGetLastError();
}

hipError_t launch_gemm(const GemmParams &p, hipStream_t stream) {
    if (p.nseg == 0 || p.nseg > 4) return hipErrorInvalidValue;
    if (p.pair) {
        const GemmSeg &a = p.seg[0], &b = p.seg[1];
        if (p.nseg != 2 || a.rows != b.rows || a.nb != b.nb || a.ldy != b.ldy || a.resid || b.resid)
            return hipErrorInvalidValue;
        if (p.act_out) {
            if (p.act_kb != a.nb) return hipErrorInvalidValue;
            return p.narrow ? launch_gemm_t<false, true, 2>(p, stream) : launch_gemm_t<false, false, 2>(p, stream);
        }
        return p.narrow ? launch_gemm_t<false, true, 1>(p, stream) : launch_gemm_t<false, false, 1>(p, stream);
    }
    if (p.narrow) return p.nseg > 1 ? launch_gemm_t<true, true>(p, stream) : launch_gemm_t<false, true>(p, stream);
    return p.nseg > 1 ? launch_gemm_t<true, false>(p, stream) : launch_gemm_t<false, false>(p, stream);
}

}  // namespace q35mm
