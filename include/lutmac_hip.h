/*
 * lutmac_hip.h -- C ABI of the MI355X (gfx950) bit-serial LUT-GEMV path.
 *
 * Drop-in boundary for LutMac's kernel API (include/lutmac/lut_gemm.hpp in
 * the LutMac tree).  Plain pointers and sizes only; every entry point
 * returns an lmx_status and never throws.  On failure lmx_last_error()
 * returns a thread-local message describing the last failing call.
 *
 * Weights are immutable device handles created once at load time (repacked
 * from the reference's AoS blocks or from canonical bit-planes), so they can
 * be shared between threads.  A GEMV on one handle uses the handle's split-K
 * scratch: calls on the same handle must be ordered (one stream, or
 * externally serialised); calls on different handles are independent.
 *
 * Activation/output pointers passed to lmx_gemv/lmx_linear and the debug
 * kernels are DEVICE pointers; the host-pointer wrappers with the
 * reference's exact signatures live in lutmac_hip_compat.h.
 */
#ifndef LUTMAC_HIP_H
#define LUTMAC_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
  LMX_OK = 0,
  LMX_ERR_INVALID_ARGUMENT = 1,
  LMX_ERR_UNSUPPORTED_FORMAT = 2,
  LMX_ERR_NO_DEVICE = 3,
  LMX_ERR_OUT_OF_MEMORY = 4,
  LMX_ERR_LAUNCH_FAILED = 5,
  LMX_ERR_HIP = 6
} lmx_status;

/* Weight formats.  Plane semantics (canonical planes, see lmx_planes_desc):
 *   TERNARY  planes 0 sign (1 = negative), 1 zero (1 = zero)    BitPlaneBlock
 *   BINARY   plane 0: 1 -> +1, 0 -> -1                          BinaryBlock
 *   RRQ2     planes 0,1: stage i bit; v = sum_i (b_i ? +s_i : -s_i)  Int2Block
 *   RRQ3     planes 0,1,2 (three residual stages; no reference block)
 *   INT3     plane b = bit b of q in [0,7];  v = (q - 4) * s    Int3Block
 *   INT4     plane b = bit b of q in [0,15]; v = (q - 8) * s    Int4Block
 *   INT8     plane b = bit b of (uint8)q;    v = (int8)q * s    Int8Block   */
typedef enum {
  LMX_FMT_TERNARY = 1,
  LMX_FMT_BINARY = 2,
  LMX_FMT_RRQ2 = 3,
  LMX_FMT_RRQ3 = 4,
  LMX_FMT_INT3 = 5,
  LMX_FMT_INT4 = 6,
  LMX_FMT_INT8 = 7
} lmx_format;

/* Activation rotation applied inside the GEMV before the table build. */
#define LMX_ROTATE_NONE 0u
/* Blockwise FWHT-256 with 1/16 scaling over the zero-padded activations,
 * src/kernels/transform_simd.cpp:26-110 (scalar branch). */
#define LMX_ROTATE_FWHT256 1u
/* Orthonormal length-K Walsh-Hadamard transform H_K/sqrt(K); K must be a
 * power of two <= 16384.  (no reference counterpart.) */
#define LMX_ROTATE_FWHT_FULL 2u

typedef struct lmx_weight lmx_weight;

/* Canonical bit-plane source (host memory).
 *   planes: [P][rows][cols/8] bytes; weight k of a row is bit 7-(k%8) of byte
 *           k/8 (the reference's MSB-first plane order, types.hpp:140-149).
 *   scales: [S][rows][ceil(cols/group)] fp32 (S = stages: 2 RRQ2, 3 RRQ3,
 *           else 1).  group is a multiple of 128, or 0 for one scale per row.
 *   cols must be a multiple of 8. */
typedef struct {
  int format;
  size_t rows;
  size_t cols;
  size_t group;
  const uint8_t *planes;
  const float *scales;
} lmx_planes_desc;

/* ---- status / library ---------------------------------------------------*/
const char *lmx_status_string(int status);
const char *lmx_last_error(void);
/* Number of visible GPUs (0 and LMX_ERR_NO_DEVICE when none). */
int lmx_device_count(int *count);
/* Library version as MAJOR*10000 + MINOR*100 + PATCH. */
int lmx_version(void);

/* ---- host-only helpers (no GPU needed) ----------------------------------*/
/* Planes and scale stages of a format. */
int lmx_format_info(int format, int *planes, int *stages);
/* Bytes of one reference AoS block of `format` (68/36/72/100/132/260). */
int lmx_block_bytes(int format, size_t *bytes);
/* Reference AoS blocks -> canonical planes + scales, group 256
 * (replaces reading PackedTensor blocks, types.hpp:126-465).
 * blocks: rows*ceil(cols/256) blocks; planes: [P][rows][Kp/8] with
 * Kp = ceil(cols/256)*256; scales: [S][rows][Kp/256]. */
int lmx_blocks_to_planes(int format, const void *blocks, size_t num_blocks,
                         size_t rows, size_t cols, uint8_t *planes,
                         float *scales);
/* Inverse of lmx_blocks_to_planes (bit-exact round trip). */
int lmx_planes_to_blocks(int format, const uint8_t *planes,
                         const float *scales, size_t rows, size_t cols,
                         void *blocks, size_t num_blocks);
/* Size in bytes of the device tile layout for rows x cols. */
int lmx_tile_bytes(int format, size_t rows, size_t cols, size_t *bytes);
/* Canonical planes [P][rows][cols/8] -> device tile layout (host buffer of
 * lmx_tile_bytes): [Kp/128][P][Npad][16 B], Npad = rows rounded up to 64,
 * Kp = cols rounded up to 256.  Padded columns hold the format's code for 0
 * (ternary zero flag set, int3 q=4, int4 q=8, int8 q=0; binary/RRQ bits 0),
 * padded rows are zero. */
int lmx_tile_planes(int format, const uint8_t *planes, size_t rows,
                    size_t cols, uint8_t *tiles);
/* Inverse of lmx_tile_planes. */
int lmx_untile_planes(int format, const uint8_t *tiles, size_t rows,
                      size_t cols, uint8_t *planes);
/* Canonical scales [S][rows][ceil(cols/group)] (group as in lmx_planes_desc)
 * -> the device scale layout [S][n_groups][Npad] fp32 (n_groups = Kp/group,
 * or 1 per row; padded rows and groups 0).  With out == NULL only *bytes is
 * set to the layout's size; otherwise *bytes must equal it.  No reference
 * counterpart (the reference keeps one scale inside each block). */
int lmx_tile_scales(int format, const float *scales, size_t rows, size_t cols,
                    size_t group, float *out, size_t *bytes);

/* ---- weights ------------------------------------------------------------*/
/* Repack + upload canonical planes (BASELINE synthetic formats). */
int lmx_weight_create(const lmx_planes_desc *desc, lmx_weight **out);
/* Repack + upload reference AoS blocks: the device side of a PackedTensor
 * (types.hpp:470-492); group 256, rows = M, cols = K. */
int lmx_weight_from_blocks(int format, const void *blocks, size_t num_blocks,
                           size_t rows, size_t cols, lmx_weight **out);
int lmx_weight_destroy(lmx_weight *w);
/* Format, shape and device bytes (planes + scales) of a handle. */
int lmx_weight_info(const lmx_weight *w, int *format, size_t *rows,
                    size_t *cols, size_t *device_bytes);
/* Kernel plan chosen for a handle at creation: full-K configuration
 * (0 = split-K kernel, 1..6 = LMX_FULLK values), split-K k-slice, and
 * whether the full-K kernel stages its weight loads.  Diagnostic only; the
 * environment variables LMX_FULLK, LMX_KSLICE, LMX_WAVES, LMX_STAGED and
 * LMX_REDUCE, read when a handle is created, override the plan.  No
 * reference counterpart (the reference has one CPU kernel per format). */
int lmx_weight_kernel_config(const lmx_weight *w, int *fullk, int *kslice,
                             int *staged);
/* Copy the device tile layout back to the host (bit-exact repack check). */
int lmx_weight_read_tiles(const lmx_weight *w, uint8_t *tiles, size_t bytes);

/* ---- compute (device pointers, asynchronous on `stream`; NULL = default) */
/* y[b*rows + r] = sum_k W[r,k] * R(x[b*cols + .])[k] for b < batch, where R is
 * the rotation selected by flags.  x holds `cols` floats per batch row (the
 * kernel zero-extends to the padded width).  With batch >= 4 (x 16-byte
 * aligned, cols % 4 == 0) groups of 16/8/4 rows share one pass over the
 * weights, through scratch allocated with the handle (no call allocates,
 * so calls can be captured into a HIP graph).  Replaces the raw per-format
 * dispatchers lut_gemv / lut_gemv_binary / int2_gemv / int3_gemv /
 * int4_gemv / int8_gemv (lut_gemm.hpp:172-408). */
int lmx_gemv(const lmx_weight *w, const float *x, float *y, size_t batch,
             unsigned flags, void *stream);
/* lut_linear (lut_gemm.hpp:419-420, lut_gemm_scalar.cpp:68-180): rotation
 * FWHT-256 for TERNARY/BINARY/RRQ2/RRQ3 as the reference does for
 * quant_bits <= 2, none otherwise; then y += bias when bias is not NULL. */
int lmx_linear(const lmx_weight *w, const float *bias, const float *x,
               float *y, size_t batch, void *stream);
/* In-place blockwise FWHT-256 (transform.hpp:19 apply_hadamard_rotation);
 * n a multiple of 256 (whole chunks only, as the reference). */
int lmx_fwht256(float *x, size_t n, void *stream);
/* Device table build (lut_gemm.hpp:53-58 precompute_luts): luts[n/4][16],
 * bit-identical to the reference's order of additions; flags may request a
 * FWHT-256 of x first (then n must be a multiple of 256). */
int lmx_precompute_luts(const float *x, size_t n, unsigned flags, float *luts,
                        void *stream);
/* Device index generation (lut_gemm.hpp:79-99 extract_indices) for n_groups
 * groups of canonical sign/zero plane bytes; one pos/neg byte per group. */
int lmx_extract_indices(const uint8_t *sign_plane, const uint8_t *zero_plane,
                        size_t n_groups, uint8_t *pos_idx, uint8_t *neg_idx,
                        void *stream);

/* The GEMV of lmx_gemv without a weight handle, for callers that cannot
 * allocate: code under HIP graph capture, serving loops with a fixed memory
 * budget.  No counterpart in the reference.  Weights are the caller's DEVICE
 * buffers: tiles in the lmx_tile_planes layout (16-byte aligned), scales in
 * the lmx_tile_scales layout; format, rows, cols, group, x, y, batch, flags
 * and stream mean what they mean for lmx_gemv, with the same kernel plan, so
 * y is bit-identical to lmx_gemv's (batches run one vector at a time).  It
 * allocates nothing: the split-K partials, ticket counters and the staging
 * copy of x live in an 8 MiB device array that each GPU holds until the
 * process ends: a fixed 64 KiB of split-K ticket counters (one per 64-row
 * block), then the staging copy of x (Kp*4 B), then the split-K partials
 * ((Kp/kslice)*Npad*4 B); shapes needing more return
 * LMX_ERR_INVALID_ARGUMENT.  The first call on a device looks the array up,
 * zeroes it with a kernel on `stream` and waits for that kernel before it
 * returns or launches anything else, so make it outside graph capture; every
 * later call, on any stream or thread, then finds the counters zeroed.  Calls
 * on one GPU share the array: calls that overlap in time on one GPU race, so
 * order them (e.g. one stream, or an event between streams). */
int lmx_gemv_tiles_noalloc(int format, const void *tiles, const float *scales,
                           size_t rows, size_t cols, size_t group,
                           const float *x, float *y, size_t batch,
                           unsigned flags, void *stream);

/* ---- measurement -------------------------------------------------------*/
/* Achievable-bandwidth yardstick: one plain streaming read of `bytes` device
 * bytes at `buf` (16-byte aligned, a multiple of 16), asynchronous on
 * `stream`; `sink` is a device word it may write.  Timing it beside a GEMV
 * of the same bytes gives the GEMV's fraction of what the memory system
 * delivers at that size.  No reference counterpart (the reference has no
 * device and no roofline). */
int lmx_hbm_read_probe(const void *buf, size_t bytes, unsigned *sink,
                       void *stream);
/* The same read with its launch shape chosen: `workgroups` workgroups of
 * 1024 lanes, each lane with `loads_in_flight` (1, 2, 4, 8 or 16) 16-byte
 * loads issued before their data is used (lmx_hbm_read_probe is 2 on 512).
 * A sweep over shapes gives the fastest plain read at a size. */
int lmx_hbm_read_probe_shape(const void *buf, size_t bytes, int loads_in_flight,
                             int workgroups, unsigned *sink, void *stream);
/* A read of a weight's device tiles and scales (the lmx_tile_planes /
 * lmx_tile_scales layouts of format x rows x cols x group, K <= 16384) with
 * the load schedule of the interleaved full-K GEMV: 32 rows per 1024-lane
 * workgroup, each lane loading its row's plane words of two 128-chunks per
 * step and their scales -- every step's loads issued at once, so each CU's
 * whole share of the matrix is requested before any of it is used. */
int lmx_hbm_read_probe_tiles(const void *tiles, const float *scales, int format,
                             size_t rows, size_t cols, size_t group,
                             unsigned *sink, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* LUTMAC_HIP_H */
