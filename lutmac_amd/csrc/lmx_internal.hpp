// lmx_internal.hpp -- shared definitions of the LUT-GEMV library (not part
// of the C ABI).
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>

#include "lutmac_hip.h"

namespace lmx {

constexpr int kChunk = 128;        // k per chunk: one uint4 per plane per row
constexpr int kRotChunk = 256;     // FWHT-256 block and device K padding
constexpr int kWave = 64;          // lanes per wavefront (one row per lane)

inline size_t round_up(size_t v, size_t m) { return (v + m - 1) / m * m; }

struct FormatInfo {
  int planes;
  int stages;
  size_t block_bytes;  // reference AoS block size; 0 = no reference block
};

bool format_info(int fmt, FormatInfo *fi);

// Sets the thread-local error message and returns `status`.
int fail(int status, const char *fmt, ...);
void clear_error();

// ---- host repack (lmx_repack.cpp) ----------------------------------------
int blocks_to_planes(int fmt, const uint8_t *blocks, size_t rows, size_t cols,
                     uint8_t *planes, float *scales);
int planes_to_blocks(int fmt, const uint8_t *planes, const float *scales,
                     size_t rows, size_t cols, uint8_t *blocks);
// planes: [P][rows][row_bytes]; tiles: [Kp/128][P][Npad][16].  Columns past
// row_bytes*8 get the format's pad code (pad_byte), rows past `rows` zero.
uint8_t pad_byte(int fmt, int plane);
void tile_planes(int fmt, const uint8_t *planes, size_t rows, size_t row_bytes,
                 size_t Npad, size_t Kp, uint8_t *tiles);
void untile_planes(int fmt, const uint8_t *tiles, size_t rows, size_t row_bytes,
                   size_t Npad, size_t Kp, uint8_t *planes);
// 4-bit planes [4][rows][row_bytes] -> the matrix-core kernel's code layout
// [Kp/128][Npad][4 lane groups kq][8 k-blocks][2 bytes]: byte b of k-block
// kb, group kq holds codes k = 16 kb + 4 kq + 2b (low nibble) and + 1 (high
// nibble) of the chunk; columns past row_bytes*8 and rows past `rows` hold
// code 8 (value 0).
void nibble_tiles(const uint8_t *planes, size_t rows, size_t row_bytes, size_t Npad, size_t Kp, uint8_t *out);

// ---- device launches (lmx_kernels.hip) -----------------------------------
struct GemvArgs {
  const void *planes;      // tiled planes
  const void *nib;         // int4 codes in the matrix-core layout (nibble_tiles), or null
  const float *scales;     // [S][n_groups][Npad]
  const float *x;          // [cols]
  float *y;                // [rows]
  const float *bias;       // [rows] or null
  const float *resid;      // batched kernel: [batch][rows] added to y (may alias y), or null
  float *partials;         // [splits][Npad]
  unsigned *counters;      // [row_blocks]
  int rows, Npad, cols, Kp;
  int group_chunks;        // chunks per scale group
  int gshift;              // log2(group_chunks) when it is a power of two, else -1
  int n_groups;
  int kslice;              // k per workgroup (multiple of 256, divides Kp)
  unsigned rotate;         // LMX_ROTATE_NONE / LMX_ROTATE_FWHT256
  int reduce;              // split-K reduction strategy (kReduce*)
  int waves;               // wavefronts (64-row slabs) per workgroup: 1, 2 or 4
  int fullk;               // 0: split-K kernel; else a kFullK_* configuration
  int kfamily;             // full-K kernel family for plain activations (kKernel*)
  int staged;              // full-K: issue part of the weight loads after the table prologue
  int xmode;               // activation transform fused into the table prologue (kXMode*)
  const float *xw;         // kXModeRmsNorm: norm weight [cols]
  float eps;               // kXModeRmsNorm: epsilon
  unsigned long long *amax;  // when set: per-wave argmax keys of y (gemv_argmax_slots of them)
  const unsigned *pcount;  // with amax, or null: occurrences of each row's token in the history; the
                           // argmax keys then rank repetition-penalised values (penalised_logit)
  float penalty;           // repetition penalty applied pcount[row] times
  int epi;                 // output epilogue (kEpi*)
  float *y2;               // kEpiNormOut: RMSNorm of y with weight xw [rows] (batched GEMV only)
};

// Output epilogues of the full-K kernels:
//   kEpiStore:     y[r] = (W x')[r] (+ bias[r])
//   kEpiSiluPair:  rows = 2h (a fused gate|up weight): y[j] = silu(g_j) * u_j for
//                  j < h, g_j = row j, u_j = row h + j (each + bias); a
//                  workgroup computes gate rows and the matching up rows
//                  (model.cpp:36,413-416), so the activation of the down
//                  projection leaves the gate|up launch already formed
//   kEpiNormOut:   (batched GEMV) y as kEpiStore (+ resid), and y2 = the
//                  RMSNorm of each y row with weight xw and epsilon eps
//                  (norm.cpp:18-34), the next linear's input
//   kEpiPartials:  (batched GEMV, exactly one group of 4/8/16 vectors) no
//                  reduction: the split sums stay in a.partials
//                  [nb][splits][Npad] (batched_launch_splits of them) for a
//                  consumer that sums them in split order itself (the decode
//                  attention reads its q/k/v rows that way)
constexpr int kEpiStore = 0;
constexpr int kEpiSiluPair = 1;
constexpr int kEpiNormOut = 2;
constexpr int kEpiPartials = 3;
constexpr int kNormOutMaxRows = 8192;   // kEpiNormOut keeps a whole row in LDS

// Activation transforms applied while the tables are built:
//   kXModeRmsNorm:  x'[k] = x[k] * inv_rms * xw[k], inv_rms = 1/sqrt(sum x^2 / cols + eps)
//                   (norm.cpp:18-34), the sum taken over x[0..cols) by every workgroup
//   kXModeSiluMul:  x'[k] = silu(x[k]) * x[cols + k]  (model.cpp:36,413-416: gate and
//                   up halves of one fused gate|up output)
// (both applied by xform4 after the load)
constexpr int kXModeNone = 0;
constexpr int kXModeRmsNorm = 1;
constexpr int kXModeSiluMul = 2;
constexpr int kAttnChunk = 64;

// Full-K kernel configurations (waves x k-slices per wave x chunks per slice):
// the workgroup holds the tables of the whole K and reduces in LDS.
enum {
  kFullK_None = 0,
  kFullK_16x2x2 = 1,  // 32 rows, 32 slices of 256: K <= 8192
  kFullK_16x2x3 = 2,  // 32 rows, 32 slices of 384: K <= 12288 (LDS-bound ~9472)
  kFullK_8x2x1 = 3,   // 32 rows, 16 slices of 128: K <= 2048
  kFullK_16x1x1 = 4,  // 64 rows, 16 slices of 128: K <= 2048
  kFullK_16x4x1 = 5,  // 16 rows, 64 slices of 128: K <= 8192
  kFullK_4x4x1 = 6,   // 16 rows, 16 slices of 128: K <= 2048
  kFullK_8x8x1 = 7,   // 8 rows, 64 slices of 128: K <= 8192
  kFullK_8x8x2L = 8   // 8 rows, 64 slices x 2 layered chunks (slice s: chunks s, s + 64): 4-bit,
                      // the lean kernel only, K <= 8960 (tables of 70 chunks back to back)
};

constexpr size_t kMaxLdsBytes = 160 * 1024;  // LDS per workgroup on gfx950

// LDS of a full-K launch: x sums + slice partials (rounded to 256 B), then
// one table region of cps*2048 + 256 B per slice that holds chunks.
// A staggered chunk block rounded up to 256 B (v_perm keeps only bytes 1-2
// of a table base), the stride of chunks whose tables sit back to back.
constexpr uint32_t kIplChunkBytes = 2304;

// LDS of a layered launch (kFullK_8x8x2L): the prefix, then Kc chunk blocks.
inline size_t layered_lds_bytes(int waves, int h, int cps, size_t Kc) {
  return (size_t(waves * h * cps + waves * kWave) * 4 + 255) / 256 * 256 + Kc * kIplChunkBytes;
}

inline size_t fullk_lds_bytes(int waves, int h, int cps, size_t Kc) {
  const size_t prefix = (size_t(waves * h * cps + waves * kWave) * 4 + 255) / 256 * 256;
  const size_t used = (Kc + cps - 1) / cps;
  return prefix + used * (size_t(cps) * 2048 + 256);
}

struct FullKShape { int waves, h, cps; };
inline FullKShape fullk_shape(int cfg) {
  switch (cfg) {
  case kFullK_16x2x2: return {16, 2, 2};
  case kFullK_16x2x3: return {16, 2, 3};
  case kFullK_8x2x1: return {8, 2, 1};
  case kFullK_16x1x1: return {16, 1, 1};
  case kFullK_16x4x1: return {16, 4, 1};
  case kFullK_4x4x1: return {4, 4, 1};
  case kFullK_8x8x1: return {8, 8, 1};
  case kFullK_8x8x2L: return {8, 8, 2};
  }
  return {0, 0, 0};
}

// Full-K kernel families for plain activations (no fused transform, no
// argmax): the interleaved table-build/lookup kernel where it applies and
// measured faster (two k-slices and at least two steps per wave, its tables
// fit, not RRQ-3), else the lean kernel, else the generic one (which also
// serves every fused transform).  LMX_KERNEL forces one for tests:
// 1 generic, 2 lean.
constexpr int kKernelAuto = 0;
constexpr int kKernelGeneric = 1;
constexpr int kKernelLean = 2;

// Split-K reduction strategies.
constexpr int kReduceTicket = 0;    // last workgroup of a row block sums (one release per group)
constexpr int kReduceFenceAll = 1;  // same, with a device fence in every thread
constexpr int kReduceTwoPass = 2;   // partials, then a separate reduce kernel

int launch_gemv(int fmt, const GemvArgs &a, void *stream);
// Plane split of unrotated 4-bit lean launches (LMX_PS, read per call): 1
// the 4 x 4 x 1 and 16 x 4 x 1 plans (default), 2 the 4 x 4 x 1 plan only,
// 0 neither.
int plane_split_level();
// Batched unrotated 4-bit GEMVs of 8 or 16 vectors, and of 4 except for
// split partials left to a consumer, on the matrix cores (LMX_MFMA, read per
// call): 1 (default), 0 the lookup-table kernel.
int mfma_batched();
// Rows of one output half a workgroup covers with kEpiSiluPair for these
// arguments (format, plan, transform), 0 when that epilogue is not served.
int silu_pair_rows(int fmt, const GemvArgs &a);
// nb (2, 4, 8, 16) vectors at a.x + n*cols -> a.y + n*rows; a.partials holds
// nb * (Kp/256) * Npad floats.
int launch_gemv_batch(int fmt, const GemvArgs &a, int nb, void *stream);
// k-slices of the batched kernel for a weight: 256-wide, or 128-wide where
// the 256-wide grid at 64 rows per workgroup has fewer than kBatchMinGrid128
// workgroups (CUs idle); the batched partials hold 16 x this x Npad floats.
constexpr size_t kBatchMinGrid128 = 256;
inline size_t batched_slice_splits(size_t Npad, size_t Kp) {
  const size_t s256 = Kp / kRotChunk;
  return (Npad / kWave) * s256 < kBatchMinGrid128 ? 2 * s256 : s256;
}
// The k-slices a batched launch actually uses: batched_slice_splits, or the
// 256-wide ones when LMX_BATCH_S128=0 turns the 128-wide slices off.
int batched_launch_splits(size_t Npad, size_t Kp);

// Exactly 4 vectors (a.x [4][cols], a.y [4][rows], a.resid [4][rows]) in one
// full-K launch with the transform a.xmode (none or RMSNorm with a.xw) and
// epilogue a.epi (store or SiLU pair); returns 1, launching nothing, when
// the handle's plan has no such form (split-K plans, K above 2048, more than
// one round of workgroups; quad_serves tells beforehand).
int launch_gemv_quad(int fmt, const GemvArgs &a, void *stream);
bool quad_serves(const GemvArgs &a);
// Number of argmax key slots a launch with these arguments writes.
size_t gemv_argmax_slots(const GemvArgs &a);
int launch_fwht256(float *x, size_t n, void *stream);
int launch_stage_x(const float *x, size_t n, float *out, size_t n_pad, void *stream);
int launch_fwht_full(const float *x, float *out, size_t n, void *stream);
int launch_precompute_luts(const float *x, size_t n, unsigned flags,
                           float *luts, void *stream);
int launch_extract_indices(const uint8_t *s, const uint8_t *z, size_t n_groups,
                           uint8_t *pos, uint8_t *neg, void *stream);

}  // namespace lmx

// Device weight handle (opaque to C callers).
struct lmx_weight {
  int format = 0;
  int device = 0;
  size_t rows = 0, cols = 0;
  size_t Npad = 0, Kp = 0;
  size_t group = 0;        // scale group in k on the device (multiple of 128)
  size_t n_groups = 0;     // Kp / group
  size_t tile_bytes = 0;
  size_t scale_bytes = 0;
  int kslice = 0;          // chosen k-slice per workgroup
  int reduce = 0;          // split-K reduction strategy
  int waves = 4;           // wavefronts per workgroup
  int fullk = 0;           // full-K kernel configuration (kFullK_*), 0 = split-K
  int kfamily = 0;         // full-K kernel family for plain activations (kKernel*)
  int staged = 1;          // full-K: later chunks' weight loads after the prologue
  void *d_planes = nullptr;
  float *d_scales = nullptr;
  float *d_partials = nullptr;
  unsigned *d_counters = nullptr;
  float *d_xrot = nullptr;  // staging for LMX_ROTATE_FWHT_FULL (cols floats)
  bool batched = true;           // batch >= 2 through the batched kernel (LMX_BATCHED=0: one GEMV per vector)
  float *d_bpartials = nullptr;  // batched partials [16][Kp/256][Npad], allocated with the handle
  void *d_nib = nullptr;         // int4 with the matrix-core kernel: codes in nibble_tiles layout
  size_t bpartials_cap = 0;      // floats
};

namespace lmx {
// Fills a handle's shape, layout sizes and kernel plan for (fmt, rows, cols,
// group) as lmx_weight_create does; allocates nothing, sets no pointers.
void plan_weight(lmx_weight *w, int fmt, size_t rows, size_t cols, size_t group);
// lmx_gemv after its handle check: y = W x for `batch` vectors with the
// handle's pointers (planes, scales, partials, counters, staging).
int gemv_impl(const lmx_weight *w, const float *x, float *y, size_t batch, unsigned flags, void *stream);
// Kernel arguments of a handle (x, y, bias, rotation and transform unset).
GemvArgs weight_args(const lmx_weight *w);
// Vectors x[0..batch) in groups of 16/8/4 through the batched kernel (a.bias
// per row, a.resid per vector row); *done = the vectors it covered (none
// below 4).
int gemv_batched(const lmx_weight *w, GemvArgs a, const float *x, float *y, size_t batch, void *stream,
                 size_t *done);
// Whether gemv_batched serves epilogue epi (kEpi*) for `batch` vectors of w
// with no vector left to the single-vector path (x 16-byte aligned assumed).
bool batched_epilogue_ok(const lmx_weight *w, int epi, size_t batch);
}  // namespace lmx
