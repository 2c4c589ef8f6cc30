// q35mm_internal.h -- interfaces between the host runtime (runtime.cpp) and
// the kernel translation units.  Not installed; no C ABI here.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace q35mm {

// Geometry of the lane-order tile layout (described in q35mm_device.h).
constexpr uint32_t kBlock = 128;         // scale block edge
constexpr uint32_t kSubRows = 32;        // rows per MFMA sub-tile
constexpr uint32_t kChunkBytes = 1024;   // one wavefront load
constexpr uint32_t kSubBytes = 4096;     // 32 rows x 128 columns
constexpr uint32_t kBlockBytes = 16384;  // 128 x 128

// A resident FP8 weight: lane-order tiled codes + fp32 block scales.
struct Weight {
    uint8_t *codes = nullptr;   // NB*128 x KB*128 bytes, layout in q35mm_device.h
    float *scale = nullptr;     // [NB][KB] fp32 (padded blocks are 0)
    uint32_t rows = 0, cols = 0;
    uint32_t nb = 0, kb = 0;    // ceil(rows/128), ceil(cols/128)
    // Live (nonzero) block scales of some 128-row group span more than
    // kGemmScaleSpan: the prefill GEMM, which keeps its accumulator in units
    // of the current block scale, could overflow, so such a weight runs on
    // the decode GEMV (one fmaf per block and output) at any m.
    bool wide_scales = false;
};
constexpr float kGemmScaleSpan = 0x1.0p64f;

// ---- decode GEMV (m <= 8 tokens) -------------------------------------
// Stream-K decomposition: the weight's NB*KB 16 KiB blocks, taken in
// (row group, K block) order and concatenated over up to four segments that
// share K, are split into P equal contiguous ranges, one per workgroup.
constexpr uint32_t kGemvMaxM = 8;
constexpr uint32_t kGemvMaxRangeBlocks = 24;  // bounds the LDS stage (147 KiB at m = 8)
constexpr uint32_t kGemvCtasPerCu = 1;        // default P = one workgroup per CU
// Dynamic LDS cap: gfx950 gives a workgroup 160 KiB in total; 1 KiB stays
// for the kernel's static LDS.
constexpr uint32_t kGemvMaxLds = 159 * 1024;
constexpr uint32_t kGemvThreads = 256;    // 4 wavefronts = one 128-row group
constexpr uint32_t kGemvDepth = 4;        // K blocks of weights per wavefront ring
constexpr uint32_t kGemvMaxPending = 4;   // groups one workgroup may have to reduce

// Each segment (one weight) gets the grid it would get alone, so multi-weight
// launches return exactly the bits of single-weight calls.
struct GemvSeg {
    const uint8_t *codes;
    const float *scale;
    float *y;            // token-major [m][ldy]
    const float *resid;  // optional [m][ldy]: y = resid + product (may equal y)
    uint32_t rows;
    uint32_t ldy;
    uint32_t nb;         // 128-row groups
    uint32_t cta_begin;  // first workgroup of this segment's grid
    uint32_t nctas;      // P: workgroups of this segment
    uint32_t maxc;       // contributions per group the workspace holds
    uint32_t ws_off;     // float offset of the segment's partials [nb][maxc][8][128]
    uint32_t cnt_off;    // offset of the segment's arrival counters [nb]
};

// What the staged activations are, per column k of token t:
//   kXPlain    x[t][k]
//   kXRmsNorm  (x[t][k] * inv_t) * (1 + norm_w[k]), inv_t the RMSNorm scale of
//              row t of x, computed by every workgroup (q35_kern_rmsnorm)
//   kXSwiGLU   silu(x[t][k]) * x2[t][k]  (q35_kern_swiglu; x = gate, x2 = up)
constexpr uint32_t kXPlain = 0, kXRmsNorm = 1, kXSwiGLU = 2;

struct GemvParams {
    GemvSeg seg[4];
    const float *x;      // [m][ldx] fp32
    const float *x2;     // kXSwiGLU: up [m][ldx]
    const float *norm_w; // kXRmsNorm: [k]
    float eps;           // kXRmsNorm
    uint32_t xmode;
    uint32_t norm_cols;  // kXRmsNorm: k rounded up to 32
    float *ws;           // partial outputs
    uint32_t *cnt;       // arrival counters, zero between launches
    uint32_t ldx;
    uint32_t m;
    uint32_t k;          // valid columns
    uint32_t kb;         // KB
    uint32_t nseg;
    uint32_t nctas;      // total workgroups
    uint32_t max_range;  // longest range of any segment, in blocks
    uint32_t x_vec;      // x 16-byte aligned, ldx % 4 == 0, k % 8 == 0: vector staging loads
    // Row-split launches of host-pointer calls: the launch's last workgroup
    // stores done_value into *done_word (null: nothing); done_cnt counts
    // finished workgroups and is zero between launches.
    uint32_t *done_word;
    uint32_t *done_cnt;
    uint32_t done_value;
};

// A-operand rows of the GEMV's staged activations: token x bf16 part (3m),
// rounded up to an odd count for conflict-free LDS staging writes.
__host__ __device__ constexpr uint32_t stage_rows(uint32_t m) { return (3 * m) | 1u; }

// P for T blocks on a device with cus compute units; depends only on the
// weight shape, so a batch of m tokens gives exactly the bits of m single
// calls.
uint32_t gemv_ctas(uint32_t nblocks, uint32_t cus, uint32_t per_cu);
// Most workgroups (P ranges) that can cover one group of kb blocks.
uint32_t gemv_max_contrib(uint32_t nblocks, uint32_t nctas, uint32_t kb);
size_t gemv_lds_bytes(uint32_t m, uint32_t range_blocks);
// kXRmsNorm holds the m rows of x in registers, kGemvNormBatch float4s per
// thread: usable when m * k (k rounded up to 8) fits.  norm_cols = k rounded
// up to 32 sets the LDS layout of the squares.
constexpr uint32_t kGemvNormBatch = 8;
bool gemv_norm_fits(uint32_t m, uint32_t k);
uint32_t gemv_norm_cols(uint32_t k);
size_t gemv_norm_lds_bytes(uint32_t m, uint32_t norm_cols);
hipError_t launch_gemv(const GemvParams &p, hipStream_t stream);

// Row-split decode GEMV (gemv_rows.hip): each workgroup owns a range of at
// most 32 rows of one weight, its wavefronts (4 or 8) splitting K; no
// partial outputs between workgroups.  Used for the weights
// gemv_rows_shape() selects (by K only, so batch and multi-weight results
// stay those of single calls); activations plain (kXPlain), optional
// residual.  Segments: nctas from gemv_rows_plan (cta_begin consecutive);
// ws, cnt, max_range unused.
constexpr uint32_t kGemvRsMaxWaves = 8;
// Every row-split workgroup splits all m*K activations of its wavefronts'
// K ranges itself, so that redundant work grows with K*m; beyond 160 K
// blocks stream-K is kept.
constexpr uint32_t kGemvRsMaxKb = 160;
// Per wavefront: two A-operand slots of 256 * stage_rows(m) bytes + a zero slot.
__host__ __device__ constexpr uint32_t gemv_rows_wave_lds(uint32_t m) { return 512 * stage_rows(m) + 16; }
// K blocks and wavefronts per workgroup the kernel accepts (a wavefront's
// block scales sit one per lane: at most 64 blocks each).
bool gemv_rows_shape(uint32_t kb, uint32_t waves);
// Workgroups of one launch over weights of rows[0..nseg) rows: one per
// 32-row sub-tile (whole 1 KiB chunks per load).
void gemv_rows_plan(const uint32_t *rows, uint32_t nseg, uint32_t *nctas);
// waves: 4 or 8; depth: ring depth 2..4 (0: by launch shape).
hipError_t launch_gemv_rows(const GemvParams &p, uint32_t cus, uint32_t waves, uint32_t depth, hipStream_t stream);

// Row-split kernel modes: plain rows of up to four weights, or the MLP's
// gate (seg[0]) and up (seg[1]) paired -- kPairRows rows of each per
// workgroup, one MFMA tile -- writing silu(gate) * up to seg[0].y, on x as
// given (kRowsPair) or on RMSNorm(x) with p.norm_w / p.eps (kRowsPairNorm,
// one token, k <= kPairNormMaxCols: every workgroup forms the row's scale).
constexpr uint32_t kRowsPlain = 0, kRowsPair = 1, kRowsPairNorm = 2;
constexpr uint32_t kPairRows = 16;
constexpr uint32_t kPairNormMaxCols = 8192;
// Floats per lane row of the fused RMSNorm's squares in LDS ([8][stride]):
// k/8 rounded up to whole float4, + 4 to spread the eight rows over banks.
__host__ __device__ constexpr uint32_t pair_norm_stride(uint32_t k) { return (((k + 7) / 8 + 3) & ~3u) + 4; }
hipError_t launch_gemv_pair(const GemvParams &p, bool norm, uint32_t cus, hipStream_t stream);

// ---- chained decode GEMVs (chain.hip) ---------------------------------
// One step: a row-split GEMV over 1..4 weights sharing x.  seg[i].cta_begin
// is the first item (32-row sub-tile) of weight i within the step,
// seg[i].nctas its item count; ws_off, cnt_off and maxc are unused.
struct ChainStep {
    GemvSeg seg[4];
    const float *x;      // [m][ldx] fp32
    uint32_t ldx, k, kb, nseg;
    uint32_t items;      // sub-tiles of all segments
    uint32_t count;      // 1: a later step waits for this one, so its items are counted
                         // and its ready flags set (the last step's are not)
    uint32_t wait;       // 1: x or resid are outputs of earlier steps (wait until those have completed)
    uint32_t x_mode;     // how x and resid are read: kChainX*
};
// kChainXPlain: cached loads, allowed when no earlier step of the launch
// read x's or resid's bytes and at most one wrote them; kChainXCoherent:
// agent-scope loads at the coherence point.
constexpr uint32_t kChainXPlain = 0, kChainXCoherent = 2;
// Counters and flags sit kChainCtrStride bytes apart, each step's ready
// flags in kChainFlags copies, so that neither atomics nor polls pile onto
// one cache line.
constexpr uint32_t kChainFlags = 64;
constexpr uint32_t kChainCtrStride = 256;
// Zero floats the activation loads of a block whose inputs are not known
// to be complete read instead (reloaded once they are).
constexpr uint32_t kChainZeroFloats = 1024;
struct ChainParams {
    const ChainStep *steps;   // device memory, [nsteps]
    const uint32_t *wg_off;   // [nwg + 1]: workgroup w's items are wg_items[wg_off[w] .. wg_off[w + 1])
    const uint32_t *wg_items; // (step << 16) | item, in step order
    const float *zero;        // kChainZeroFloats zeros
    uint8_t *done;            // step s: uint32 at s * stride, parts finished (zero between launches)
    uint8_t *ready;           // step s, copy c: uint32 at (s * kChainFlags + c) * stride (zero between launches)
    uint32_t *exit_cnt;       // workgroups finished, zero between launches
    uint32_t *err;            // set to 1 when a wait gave up
    uint32_t nsteps;
    uint32_t m;
    uint32_t nwg;             // one workgroup per CU
    uint32_t spin_limit;      // polls before a wait gives up
    uint32_t coherent;        // some step's x_mode is kChainXCoherent: every step reads that way
};
// Dynamic LDS of a chain launch: the wavefronts' A-operand slots, padded so
// that one workgroup fills a CU (kChainLds).
constexpr size_t kChainLds = 96 * 1024;
hipError_t launch_chain(const ChainParams &p, hipStream_t stream);

// ---- prefill GEMM (bf16 MFMA) ----------------------------------------
constexpr uint32_t kGemmTile = 256;       // BM = BN = 256 per workgroup
constexpr uint32_t kGemmThreads = 512;    // 8 wavefronts of 128 x 64
constexpr uint32_t kGemmMaxSliceKb = 1024;  // K blocks one workgroup may cover

// Work split.  Tiles (mt, nt) are numbered tile = nt * mtiles + mt, in three
// consecutive ranges: tiles below split_tile0 are whole (one workgroup,
// written straight to y); tiles in [split_tile0, tail_tile0) are cut into
// nslices K slices each, whose partial tiles go to ws and are added in slice
// order by gemm_reduce; tiles from tail_tile0 on run as sixteen 64x64 tiles
// each (gemm_tail_kernel).  Workgroup b < split_tile0 of gemm_fp8_kernel owns
// tile b; workgroup split_tile0 + u owns slice u % nslices of tile
// split_tile0 + u / nslices.  With whole tiles first, the split and tail
// workgroups fill the CUs the last round of whole tiles leaves idle.
// One weight of a GEMM launch: several weights sharing K (the reference's
// gate and up) run as one launch over the concatenation of their tiles;
// segment s owns tiles [tile0, tile0 + mtiles * ((nb + 1) / 2)).
struct GemmSeg {
    const uint8_t *codes;
    const float *scale;
    float *y;            // token-major [m][ldy]
    const float *resid;  // optional [m][ldy]: y = resid + product (may equal y)
    uint32_t rows;
    uint32_t ldy;
    uint32_t nb;         // 128-row groups of the weight
    uint32_t tile0;
};

struct GemmParams {
    GemmSeg seg[4];
    const uint16_t *xb;  // lane-order bf16 activations, mtiles*256 rows
    float *ws;           // partial tiles of split tiles, 256 KiB each
    uint32_t nseg;
    uint32_t m;
    uint32_t kb;
    uint32_t mtiles;
    uint32_t ntiles;     // 256-row weight tiles over all segments
    uint32_t split_tile0;
    uint32_t nslices;    // K slices of each split tile (>= 2 when any tile is split)
    uint32_t tail_tile0; // first tile of the 64x64 tail (= mtiles * ntiles: none)
    uint32_t tail_fused; // 64x64 tiles run by the first whole-tile workgroups after their own tile
    uint32_t narrow;     // tiles of 128 tokens x 512 rows (m <= 128) instead of 256 x 256
    // Paired segments (nseg == 2, equal shapes): each tile holds rows r..r+T/2
    // of segment 0 in its first half and the same rows of segment 1 in its
    // second (ntiles counts such tiles).  With act_out the tiles (or, for
    // tiles cut along K, the slice sum) write silu(seg 0) * seg 1 as bf16 in
    // the lane-order activation layout of act_kb K blocks instead of fp32 y.
    uint32_t pair;
    uint16_t *act_out;
    uint32_t act_kb;
};

struct GemmPlan {
    bool narrow;
    uint32_t mtiles, ntiles, split_tile0, nslices, tail_tile0;
    size_t ws_bytes() const {
        return nslices > 1 ? (size_t)(tail_tile0 - split_tile0) * nslices * kGemmTile * kGemmTile * 4 : 0;
    }
};
// ntiles: weight tiles of all segments together (256 rows, or 512 narrow)
GemmPlan gemm_plan(uint32_t m, uint32_t ntiles, uint32_t kb, uint32_t cus, bool narrow);
// Narrow tiles: 128 tokens x 512 weight rows, for m <= kGemmNarrowMaxM.
constexpr uint32_t kGemmNarrowMaxM = 128, kGemmNarrowRows = 512;
// X [m][ldx] fp32 -> lane-order bf16 [rows_pad][kb*128 cols], rows_pad a
// multiple of 32 (m32 tiles = rows_pad / 32).  With x2: silu(x) * x2 first.
hipError_t launch_act_to_bf16(const float *x, const float *x2, uint32_t ldx, uint32_t m, uint32_t k,
                              uint32_t m32_tiles, uint32_t kb, uint16_t *xb, hipStream_t stream);
// gemm_fp8_kernel, then gemm_reduce (K-split tail) or gemm_tail_kernel (64x64 tail)
hipError_t launch_gemm(const GemmParams &p, hipStream_t stream);

// ---- residency / conversions -----------------------------------------
// Row-major raw codes (device) -> lane-order tiles (device).
hipError_t launch_repack(const uint8_t *raw, uint32_t rows, uint32_t cols,
                         uint32_t nb, uint32_t kb, uint8_t *tiled,
                         hipStream_t stream);
hipError_t launch_dequant_f32(const Weight &w, float *out, hipStream_t stream);
hipError_t launch_decode_bf16(const Weight &w, uint16_t *out, hipStream_t stream);
// Stores v into *flag (pinned host memory) once everything queued before it
// on the stream has completed.
hipError_t launch_done_flag(uint32_t *flag, uint32_t v, hipStream_t stream);

// ---- BF16 matvec (q35_mm_bf16) ---------------------------------------
hipError_t launch_bf16_gemv(const uint16_t *w, uint32_t rows, uint32_t cols,
                            const float *x, float *y, hipStream_t stream);

// ---- allocation-free scratch (noalloc.hip) -----------------------------
// q35mm_matmul_noalloc's scratch: counters first (zero between launches),
// then one region for split partials and staged activations.
constexpr size_t kNoAllocCntBytes = 64u << 10;
constexpr size_t kNoAllocBytes = 16u << 20;
// Once per device, with the device current: resolve the scratch array's
// address and clear its counters (synchronises stream).
hipError_t noalloc_setup(int device, hipStream_t stream);
// The device address of the array (nullptr before noalloc_setup).
uint8_t *noalloc_scratch(int device);

// ---- load-time quantizer (quantize.hip) --------------------------------
// w [rows][cols] (fp32, or bf16 bits) -> row-major e4m3 codes and the
// [ceil(rows/128)][ceil(cols/128)] block scales as bf16 bits and/or fp32
// (either pointer may be null).
hipError_t launch_quantize_f32(const float *w, uint32_t rows, uint32_t cols, uint8_t *codes, uint16_t *scale_bf16,
                               float *scale_f32, hipStream_t stream);
hipError_t launch_quantize_bf16(const uint16_t *w, uint32_t rows, uint32_t cols, uint8_t *codes,
                                uint16_t *scale_bf16, float *scale_f32, hipStream_t stream);

// ---- MLP neighbours (mlp.hip) -----------------------------------------
// RMSNorm of rows rows of n (row strides ldx, ldy; y may alias x), SwiGLU
// y = silu(g) * u, residual x += y.
hipError_t launch_rmsnorm(const float *x, uint32_t ldx, const float *w, float *y, uint32_t ldy,
                          uint32_t rows, uint32_t n, float eps, hipStream_t stream);
// RMSNorm of rows 0..m-1 of x straight into launch_act_to_bf16's layout
// (rows_pad rows, a multiple of 32, zeros past m; kb K blocks of 128, zeros
// past n): the bits of launch_rmsnorm followed by launch_act_to_bf16.  For
// rmsnorm_bf16_fits: n % 8 == 0, n <= kNormBf16MaxCols, rows of x and w
// 16-byte aligned.
constexpr uint32_t kNormBf16MaxCols = 8192;
bool rmsnorm_bf16_fits(const float *x, uint32_t ldx, const float *w, uint32_t n);
hipError_t launch_rmsnorm_bf16(const float *x, uint32_t ldx, const float *w, uint32_t m, uint32_t n, float eps,
                               uint32_t rows_pad, uint32_t kb, uint16_t *xb, hipStream_t stream);
hipError_t launch_swiglu(const float *g, const float *u, float *y, size_t n, hipStream_t stream);
hipError_t launch_add_inplace(float *x, const float *y, size_t n, hipStream_t stream);

}  // namespace q35mm
