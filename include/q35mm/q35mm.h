/*
 * q35mm.h -- additive device-side API of libq35mm.so (no counterpart in the
 * reference; the reference's q35_mm_* calls take host pointers only).
 *
 * It exposes what the drop-in entry points of q35/q35_mm.h do internally,
 * for callers that keep activations in HBM and chain launches on their own
 * stream (the benchmark, tests, and a device-resident model forward):
 *
 *   - weight residency: upload e4m3 codes + bf16 block scales once; the
 *     library keeps them in HBM in a tiled, zero-padded layout with fp32
 *     scales (see the layout notes in the implementation);
 *   - matmuls on device pointers, asynchronous on a caller stream;
 *   - bit-exact dequantisation to fp32 (e4m3 -> fp32, times the fp32 scale);
 *   - explicit release of resident copies the drop-in path created.
 *
 * All functions return 0 on success and a negative Q35MM_E* code on failure;
 * q35mm_last_error() describes the last failure of the calling thread.
 * Streams are hipStream_t passed as void*; NULL is HIP's null stream.
 *
 * Concurrency: scratch memory between a call's kernels (split-K partials
 * and counters, the GEMM's bf16 activations, the MLP block's intermediates)
 * is kept per stream, so calls on different streams may overlap on the GPU.
 * Calls on one stream run in order.  Host threads may call concurrently
 * (calls are serialised on a library lock while they queue work).
 */
#ifndef Q35MM_H
#define Q35MM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    Q35MM_OK = 0,
    Q35MM_EINVAL = -1,    /* bad argument (null pointer, size out of range) */
    Q35MM_EHIP = -2,      /* a HIP runtime call failed */
    Q35MM_ENOMEM = -3,    /* device or host allocation failed */
    Q35MM_ENODEV = -4,    /* no usable gfx950 device */
    Q35MM_EIO = -5,       /* a checkpoint file cannot be opened or read */
    Q35MM_EFORMAT = -6,   /* bad safetensors header, unknown dtype, range out of file */
    Q35MM_ENOTFOUND = -7, /* no tensor of that name */
    Q35MM_ESHAPE = -8     /* tensor dtype / rank / shape differs from what was asked */
};

typedef struct q35mm_weight q35mm_weight;

/* Selects and initialises the device (default: HIP device 0, or the
 * Q35MM_DEVICE environment variable).  Called implicitly by every entry
 * point that needs the GPU. */
int q35mm_init(int device);

/* Uploads W [rows][cols] e4m3 and scale_bf16 [ceil(rows/128)][ceil(cols/128)]
 * to HBM.  The host buffers may be freed afterwards. */
int q35mm_weight_create(const uint8_t *W, const uint16_t *scale_bf16,
                        uint32_t rows, uint32_t cols, q35mm_weight **out);
/* Same, with fp32 block scales (any finite value; not expressible through
 * the reference ABI). */
int q35mm_weight_create_f32scale(const uint8_t *W, const float *scale_f32,
                                 uint32_t rows, uint32_t cols,
                                 q35mm_weight **out);
void q35mm_weight_destroy(q35mm_weight *w);
int q35mm_weight_shape(const q35mm_weight *w, uint32_t *rows, uint32_t *cols);
/* Bytes of HBM held by the resident copy (codes + scales, padded). */
size_t q35mm_weight_bytes(const q35mm_weight *w);

/* Y[t][r] for t < m, X [m][cols] fp32, Y [m][rows] fp32, device pointers.
 * Dispatch by m: m <= 8 -> decode GEMV; 8 < m < Q35MM_GEMM_MIN_M -> decode
 * GEMV over groups of 8 tokens; m >= Q35MM_GEMM_MIN_M -> bf16 MFMA GEMM. */
int q35mm_matmul(const q35mm_weight *w, uint32_t m, const float *dX, float *dY,
                 void *stream);
/* q35mm_matmul without any allocation.  No counterpart in the reference:
 * it is for callers that cannot allocate (code under HIP graph capture,
 * tight serving loops).  Same dispatch, kernels and results (bit for bit)
 * as q35mm_matmul, with one exception: a GEMM of at most 128 tokens whose
 * narrow-tile K-slice partials would not fit runs on 256 x 256 tiles
 * instead (results within the GEMM bars, not the same bits).  The scratch
 * its kernels need between launches (stream-K partials and arrival
 * counters, the GEMM's bf16 activations and K-slice partials) comes from
 * one fixed device array of 16 MiB plus 64 KiB of counters that the library
 * holds on each device until the process ends.  Calls that need more fail
 * with Q35MM_EINVAL: every decode GEMV fits; a GEMM fits when its bf16
 * activations (m rounded up to 256 rows x K x 2 bytes) and K-slice
 * partials do.  q35mm_init must have run (it resolves the
 * array's address); nothing here calls an allocator.  Every call on a device
 * shares that device's array and leaves its contents behind: calls whose
 * kernels overlap on one device (different streams) race. */
int q35mm_matmul_noalloc(const q35mm_weight *w, uint32_t m, const float *dX,
                         float *dY, void *stream);
/* Decode GEMV for any m (groups of 8 tokens), fp32-accurate. */
int q35mm_gemv(const q35mm_weight *w, uint32_t m, const float *dX, float *dY,
               void *stream);
/* Prefill GEMM for any m: activations rounded to bf16, bf16 MFMA with fp32
 * accumulation, fp32 block scale applied per 128-wide K step.  The bf16
 * activations (m rounded up to 256 rows) and the resident weight must each
 * stay under 4 GiB, and the live block scales of every 128-row group must
 * lie within a factor of 2^64 of each other (Q35MM_EINVAL otherwise;
 * q35mm_matmul then uses the GEMV). */
int q35mm_gemm(const q35mm_weight *w, uint32_t m, const float *dX, float *dY,
               void *stream);
/* Up to four weights sharing cols and X, one launch (rows may differ);
 * dY[s] is [m][rows_s].  Same results as q35mm_matmul per segment. */
int q35mm_matmul_multi(const q35mm_weight *const *w, uint32_t nseg, uint32_t m,
                       const float *dX, float *const *dY, void *stream);

/* out [rows][cols] fp32 = e4m3(W) * scale, bit-exact. */
int q35mm_dequant_f32(const q35mm_weight *w, float *dOut, void *stream);
/* out [rows][cols] bf16 bits = e4m3(W) unscaled: the exact conversion the
 * matrix-core kernels feed to MFMA. */
int q35mm_decode_bf16(const q35mm_weight *w, uint16_t *dOut, void *stream);

/* BF16 weights for q35_mm_bf16 on device pointers: W [rows][cols] bf16. */
int q35mm_bf16_gemv(const uint16_t *dW, uint32_t rows, uint32_t cols,
                    const float *dx, float *dy, void *stream);

/* ---- MLP neighbours on device pointers (qwen35-c/src/q35_kern.c) ---- */

/* Zero-centred RMSNorm of rows rows of n fp32: dY[r][i] = (dX[r][i] * inv_r)
 * * (1 + dW[i]), inv_r = 1 / sqrtf(mean_r + eps), mean_r = (sum of squares in
 * the reference's eight lanes) / n.  Bit-identical to q35_kern_rmsnorm
 * (qwen35-c/src/q35_kern.c:88-108, sumsq_fixed :26-48) row by row.  dY may
 * equal dX (in place, as q35_kern_qk_norm uses it). */
int q35mm_rmsnorm(const float *dX, const float *dW, float *dY, uint32_t rows,
                  uint32_t n, float eps, void *stream);
/* dY[i] = (g * (1 / (1 + exp(-g)))) * dUp[i], g = dGate[i]: q35_kern_swiglu
 * (qwen35-c/src/q35_kern.c:147-166).  exp is rounded once from double
 * precision; libm's expf differs from that by one ulp for ~4e-5 of inputs,
 * where dY differs from the reference by 1 to 4 ulps.  dY may equal dGate
 * or dUp. */
int q35mm_swiglu(const float *dGate, const float *dUp, float *dY, size_t n,
                 void *stream);
/* One MLP block on m tokens, in place on the residual stream dX [m][H]
 * (H = gate cols = down rows, I = gate rows = up rows = down cols):
 *   xn = rmsnorm(dX, dNormW, eps); g = gate(xn); u = up(xn);
 *   dX += down(swiglu(g, u))
 * as qwen35-c/src/q35_model.c:927-939 (one token) and :964-978 (a batch).
 * The matmuls dispatch by m as q35mm_matmul (gate and up in one launch on
 * the GEMV path).  Intermediates live in a library workspace. */
int q35mm_mlp(const q35mm_weight *gate, const q35mm_weight *up,
              const q35mm_weight *down, const float *dNormW, float eps,
              uint32_t m, float *dX, void *stream);

/* ---- checkpoint -> HBM (safetensors) ---------------------------------- */

/* The loader-side quantizer of qwen35-c/src/q35_model.c:302-350 (bind_ab) on
 * device pointers: dW [rows][cols] fp32 -> dCodes [rows][cols] row-major e4m3
 * and dScale [ceil(rows/128)][ceil(cols/128)] bf16 bits.  Per 128x128 block:
 * scale = bf16(amax / 448); codes = nearest e4m3 of w / scale (ties to the
 * even code, saturating at 448, NaN -> 0x7F); blocks with scale 0 keep zero
 * codes.  Code-for-code equal to the reference. */
int q35mm_quantize_f32(const float *dW, uint32_t rows, uint32_t cols,
                       uint8_t *dCodes, uint16_t *dScale, void *stream);

/* A safetensors checkpoint: one .safetensors file, or a directory whose
 * files with ".safetensors" in the name (and not "json") are its shards
 * (qwen35-c/include/q35/q35_st.h:44-53).  Opening parses and validates every
 * header (Q35MM_EFORMAT / Q35MM_EIO on failure); tensor bytes are read on
 * demand. */
typedef struct q35mm_st q35mm_st;
int q35mm_st_open(const char *path, q35mm_st **out);
void q35mm_st_close(q35mm_st *st);
uint32_t q35mm_st_count(const q35mm_st *st);
const char *q35mm_st_name(const q35mm_st *st, uint32_t i);
/* dtype is one of "F8_E4M3", "BF16", "F32", "F16", "I64". */
int q35mm_st_info(const q35mm_st *st, const char *name, const char **dtype,
                  uint32_t *ndim, uint32_t shape[8], uint64_t *nbytes);
/* The tensor's bytes into host memory dst (cap >= its size). */
int q35mm_st_read(const q35mm_st *st, const char *name, void *dst, uint64_t cap);
/* bind_fp8 (qwen35-c/src/q35_model.c:253-273): F8_E4M3 `name` [rows][cols]
 * and BF16 `name`_scale_inv [ceil(rows/128)][ceil(cols/128)] -> a resident
 * weight, read in chunks into pinned memory, copied to HBM and repacked on
 * the device.  Q35MM_ENOTFOUND / Q35MM_ESHAPE as the reference's checks. */
int q35mm_st_load_fp8(q35mm_st *st, const char *name, uint32_t rows,
                      uint32_t cols, q35mm_weight **out);
/* bind_ab (qwen35-c/src/q35_model.c:302-350): as q35mm_st_load_fp8 when the
 * tensor is F8_E4M3; a BF16 [rows][cols] tensor is quantized on the device
 * (as q35mm_quantize_f32). */
int q35mm_st_load_ab(q35mm_st *st, const char *name, uint32_t rows,
                     uint32_t cols, q35mm_weight **out);
/* A BF16 [rows][cols] tensor (the lm_head of q35_mm_bf16) into a new device
 * buffer *dOut, released with q35mm_free. */
int q35mm_st_load_bf16(q35mm_st *st, const char *name, uint32_t rows,
                       uint32_t cols, uint16_t **dOut);
void q35mm_free(void *dptr);

/* Drop the resident copy that the q35_mm_* entry points made for host
 * pointer W (no-op if none).  q35mm_release_all drops every such copy. */
void q35mm_release(const void *W);
void q35mm_release_all(void);
/* Frees every device resource of the library. */
void q35mm_shutdown(void);

/* Chained decode GEMVs: a sequence of projections, each reading what
 * earlier ones wrote (the model's decode calls them one after another,
 * qwen35-c/src/q35_model.c:877-947), run as ONE persistent launch.  Each
 * step's weights start streaming before the previous step's outputs are
 * ready; a step reads its activations only once every earlier step has
 * completed.  Outputs are bit-identical to calling q35mm_matmul_multi step
 * by step.
 *
 * A step: nw (1..4) weights sharing cols and the device activations x
 * [m][cols] (the reference's multi4), outputs y[i] [m][rows of w[i]], and
 * optional residuals resid[i] (y = resid + product; may equal y).  Every
 * weight must run on the row-split GEMV (cols of 4..160 blocks of 128, as
 * every projection of the model); m is 1..8 tokens.  x, y and resid may be
 * outputs of earlier steps.
 *
 * q35mm_chain_create uploads the step table once (it allocates);
 * q35mm_chain_run launches it on a stream and allocates nothing (it may be
 * captured into a HIP graph); buffers and weights must outlive the chain.
 * The launch holds every workgroup slot of the device while it runs, and a
 * step's workgroups wait (bounded) for earlier steps: chain launches on
 * different streams must not run at the same time -- a wait that gives up
 * is reported by q35mm_chain_status (which waits for the device).
 * No counterpart in the reference (its calls return one at a time). */
typedef struct q35mm_chain q35mm_chain;
typedef struct q35mm_chain_step {
    uint32_t nw;
    const q35mm_weight *w[4];
    const float *x;
    float *y[4];
    const float *resid[4];
} q35mm_chain_step;
int q35mm_chain_create(const q35mm_chain_step *steps, uint32_t nsteps, uint32_t m, q35mm_chain **out);
int q35mm_chain_run(q35mm_chain *chain, void *stream);
int q35mm_chain_status(q35mm_chain *chain);
/* Workgroups of one launch (all resident on the device at once). */
uint32_t q35mm_chain_workgroups(const q35mm_chain *chain);
void q35mm_chain_destroy(q35mm_chain *chain);

/* Scratch of one stream.  Each stream the device API is called on gets its
 * own scratch set (split partials, counters, staged activations, the MLP
 * block's intermediates: tens to hundreds of MB at prefill sizes), kept
 * until this call or q35mm_shutdown.  A caller that creates and destroys
 * streams calls it before destroying one (after waiting for the device).
 * A set that a captured HIP graph used is never freed before
 * q35mm_shutdown, so graphs stay valid: its buffers are moved aside instead.
 * No counterpart in the reference (its calls keep no state). */
int q35mm_stream_release(void *stream);

/* Debug: after waiting for the device, the number of nonzero words among
 * the arrival counters of `stream`'s scratch (noalloc = 0) or of the
 * allocation-free entry point's fixed scratch (noalloc = 1), and how many
 * words there are.  Every launch returns the counters it takes to zero, so
 * both read 0 nonzero words between calls.  No counterpart in the
 * reference. */
int q35mm_debug_counters(void *stream, int noalloc, uint64_t *nonzero, uint64_t *words);

const char *q35mm_last_error(void);

/* Number of resident copies the drop-in entry points currently hold. */
size_t q35mm_resident_count(void);

#ifdef __cplusplus
}
#endif

#endif
