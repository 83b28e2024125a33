// lmx_capi.cpp -- the C ABI (include/lutmac_hip.h): argument validation,
// weight handles (repack + upload), launch configuration.  Nothing here
// throws across the ABI; every failure returns an lmx_status and records a
// thread-local message.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <new>
#include <vector>

#include "lmx_internal.hpp"

namespace lmx {

namespace {
thread_local char g_err[512] = "";
}

int fail(int status, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return status;
}

void clear_error() { g_err[0] = '\0'; }

namespace {

int hip_fail(hipError_t e, const char *what) {
  if (e == hipErrorOutOfMemory) return fail(LMX_ERR_OUT_OF_MEMORY, "%s: %s", what, hipGetErrorString(e));
  if (e == hipErrorNoDevice || e == hipErrorInvalidDevice)
    return fail(LMX_ERR_NO_DEVICE, "%s: %s", what, hipGetErrorString(e));
  return fail(LMX_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

int require_device(int *dev) {
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess || n <= 0) return fail(LMX_ERR_NO_DEVICE, "no HIP device visible");
  e = hipGetDevice(dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  return LMX_OK;
}

int env_int(const char *name, int dflt) {
  const char *s = std::getenv(name);
  return s ? std::atoi(s) : dflt;
}


int choose_waves() {
  const int env = env_int("LMX_WAVES", 4);
  return (env == 1 || env == 2 || env == 4) ? env : 4;
}

// k-slice per workgroup: 512 when K is above 4096, the padded K allows it
// and the grid still has at least 4 workgroups per CU, else 256 (measured on
// MI355X: the LM heads, K 1536 and 2048, run 3-4 % faster at 256).
// LMX_KSLICE overrides.
int choose_kslice(size_t Npad, size_t Kp, int waves) {
  const int env = env_int("LMX_KSLICE", 0);
  if ((env == 256 || env == 512) && Kp % size_t(env) == 0) return env;
  const size_t row_blocks = (Npad + kWave * waves - 1) / (kWave * waves);
  if (Kp > 4096 && Kp % 512 == 0 && row_blocks * (Kp / 512) >= 1024) return 512;
  return 256;
}

// Full-K configuration for a shape, or kFullK_None for the split-K kernel.
// A configuration must cover all Kc chunks with its k-slices, fit the LDS
// and keep its weight words in registers.  LMX_FULLK: 0 forces split-K,
// 1..6 forces a configuration (when it fits).
int choose_fullk(int fmt, size_t Npad, size_t Kp, int kfamily) {
  const int env = env_int("LMX_FULLK", -1);
  const size_t Kc = Kp / kChunk;
  FormatInfo fi;
  format_info(fmt, &fi);
  auto fits = [&](int cfg) {
    const FullKShape f = fullk_shape(cfg);
    if (cfg == kFullK_8x8x2L)   // the lean kernel only, which serves every 4-bit transform
      return fmt == LMX_FMT_INT4 && kfamily != kKernelGeneric && size_t(f.waves * f.h * f.cps) >= Kc &&
             layered_lds_bytes(f.waves, f.h, f.cps, Kc) <= kMaxLdsBytes;
    // Weight words stay in registers (no spills): up to 8 plane words per
    // lane in the generic kernel; 16 (int8 over two steps) in the
    // interleaved kernel, which always serves 16x2x2 when it is allowed.
    const bool regs = f.cps * fi.planes <= 8 ||
                      (cfg == kFullK_16x2x2 && f.cps * fi.planes <= 16 && kfamily == kKernelAuto);
    if (!regs) return false;
    return size_t(f.waves * f.h * f.cps) >= Kc && fullk_lds_bytes(f.waves, f.h, f.cps, Kc) <= kMaxLdsBytes;
  };
  if (env >= 0) return (env == 0 || !fits(env)) ? kFullK_None : env;
  const bool wide = env_int("LMX_FULLK_WIDE", 1) != 0;   // 0: auto never picks 8 rows x 64 slices
  // 4-bit: the 16 x 4 x 1 plan splits its planes over two lanes (unrotated
  // launches), 8 rows per workgroup
  const bool ps16 = fmt == LMX_FMT_INT4 && plane_split_level() == 1;
  auto workgroups = [&](int cfg) {
    const size_t rows = size_t(kWave / fullk_shape(cfg).h) / (ps16 && cfg == kFullK_16x4x1 ? 2 : 1);
    return Npad / rows;
  };
  // Measured on MI355X (4-bit, decode shapes):
  //  * K <= 2048: 4 waves x 16 rows per workgroup wins from N = 256 up to
  //    ~8k rows (latency-bound small GEMVs want many small workgroups); up
  //    to ~32k rows 8 waves x 32 rows (16384 x 2048: 6.7 against 7.5 us);
  //    beyond that (LM heads) every workgroup rebuilding the tables costs
  //    more than the split-K handoff.
  //  * larger K: the configuration with the most workgroups that still
  //    leaves at most one per CU (each holds up to 160 KB of tables);
  //    split-K when none does.
  if (Kc <= 16) {
    if (fits(kFullK_4x4x1) && workgroups(kFullK_4x4x1) <= 512) return kFullK_4x4x1;
    if (fits(kFullK_8x2x1) && workgroups(kFullK_8x2x1) <= 1024) return kFullK_8x2x1;
    return kFullK_None;
  }
  int best = kFullK_None;
  size_t best_wg = 0, best_slots = 0;
  for (int cfg = kFullK_16x2x2; cfg <= kFullK_8x8x2L; ++cfg) {
    if ((cfg == kFullK_8x8x1 || cfg == kFullK_8x8x2L) && !wide) continue;
    if (!fits(cfg)) continue;
    const FullKShape f = fullk_shape(cfg);
    const size_t wg = workgroups(cfg), slots = size_t(f.waves * f.h * f.cps);
    if (wg > 256) continue;
    if (wg > best_wg || (wg == best_wg && slots < best_slots)) best = cfg, best_wg = wg, best_slots = slots;
  }
  return best;
}

int choose_staged() {
  const int env = env_int("LMX_STAGED", 1);
  return env;
}

int choose_reduce() {
  const int env = env_int("LMX_REDUCE", kReduceTicket);
  return (env == kReduceTwoPass || env == kReduceFenceAll) ? env : kReduceTicket;
}

}  // namespace

int plane_split_level() { return env_int("LMX_PS", 1); }
int mfma_batched() { return env_int("LMX_MFMA", 1); }

void plan_weight(lmx_weight *w, int fmt, size_t rows, size_t cols, size_t group) {
  FormatInfo fi;
  format_info(fmt, &fi);
  w->format = fmt;
  w->rows = rows;
  w->cols = cols;
  w->Npad = round_up(rows, kWave);
  w->Kp = round_up(cols, kRotChunk);
  w->group = group ? group : w->Kp;
  w->n_groups = (w->Kp + w->group - 1) / w->group;
  w->tile_bytes = (w->Kp / kChunk) * fi.planes * w->Npad * 16;
  w->scale_bytes = size_t(fi.stages) * w->n_groups * w->Npad * sizeof(float);
  w->waves = choose_waves();
  w->kslice = choose_kslice(w->Npad, w->Kp, w->waves);
  w->reduce = choose_reduce();
  {
    const int fam = env_int("LMX_KERNEL", kKernelAuto);
    w->kfamily = (fam == kKernelGeneric || fam == kKernelLean) ? fam : kKernelAuto;
  }
  w->fullk = choose_fullk(fmt, w->Npad, w->Kp, w->kfamily);
  w->staged = choose_staged();
  w->batched = env_int("LMX_BATCHED", 1) != 0;
}

namespace {

void free_weight(lmx_weight *w) {
  if (!w) return;
  if (w->d_planes) (void)hipFree(w->d_planes);
  if (w->d_scales) (void)hipFree(w->d_scales);
  if (w->d_partials) (void)hipFree(w->d_partials);
  if (w->d_counters) (void)hipFree(w->d_counters);
  if (w->d_xrot) (void)hipFree(w->d_xrot);
  if (w->d_bpartials) (void)hipFree(w->d_bpartials);
  if (w->d_nib) (void)hipFree(w->d_nib);
  delete w;
}

// Shared tail of both constructors: canonical planes/scales on the host ->
// device tile layout, scales transposed to [S][n_groups][Npad].
int upload(int fmt, size_t rows, size_t cols, size_t group, const uint8_t *planes, size_t row_bytes,
           const float *scales, size_t ng_src, lmx_weight **out) {
  FormatInfo fi;
  format_info(fmt, &fi);
  int dev = 0;
  int st = require_device(&dev);
  if (st) return st;
  lmx_weight *w = new (std::nothrow) lmx_weight;
  if (!w) return fail(LMX_ERR_OUT_OF_MEMORY, "host allocation failed");
  plan_weight(w, fmt, rows, cols, group);
  w->device = dev;

  std::vector<uint8_t> tiles;
  std::vector<float> sc;
  try {
    tiles.resize(w->tile_bytes);
    sc.assign(w->scale_bytes / sizeof(float), 0.0f);
  } catch (const std::bad_alloc &) {
    delete w;
    return fail(LMX_ERR_OUT_OF_MEMORY, "host staging allocation failed");
  }
  tile_planes(fmt, planes, rows, row_bytes, w->Npad, w->Kp, tiles.data());
  for (int s = 0; s < fi.stages; ++s)
    for (size_t r = 0; r < rows; ++r)
      for (size_t g = 0; g < ng_src && g < w->n_groups; ++g)
        sc[(size_t(s) * w->n_groups + g) * w->Npad + r] = scales[(size_t(s) * rows + r) * ng_src + g];

  const size_t row_blocks = w->Npad / kWave;  // enough counters for any waves-per-group choice
  const size_t max_splits = w->Kp / kRotChunk;
  hipError_t e;
  if ((e = hipMalloc(&w->d_planes, w->tile_bytes)) != hipSuccess ||
      (e = hipMalloc(reinterpret_cast<void **>(&w->d_scales), w->scale_bytes)) != hipSuccess ||
      (e = hipMalloc(reinterpret_cast<void **>(&w->d_partials), max_splits * w->Npad * sizeof(float))) != hipSuccess ||
      (e = hipMalloc(reinterpret_cast<void **>(&w->d_counters), row_blocks * sizeof(unsigned))) != hipSuccess ||
      (e = hipMalloc(reinterpret_cast<void **>(&w->d_xrot), w->Kp * sizeof(float))) != hipSuccess) {
    free_weight(w);
    return hip_fail(e, "hipMalloc (weight)");
  }
  // Batched partials for the largest vector group (16), allocated with the
  // handle so that no GEMV call allocates (graph capture stays possible).
  if (w->batched) {
    // 128-wide k-slices (twice the splits) where 256-wide ones give the
    // batched kernel less than a workgroup per CU (batched_slice_splits)
    const size_t n = 16 * batched_slice_splits(w->Npad, w->Kp) * w->Npad;
    if ((e = hipMalloc(reinterpret_cast<void **>(&w->d_bpartials), n * sizeof(float))) != hipSuccess) {
      free_weight(w);
      return hip_fail(e, "hipMalloc (batched partials)");
    }
    w->bpartials_cap = n;
    // 4-bit: the codes once more in the matrix-core kernel's layout (groups
    // of 4, 8 and 16 vectors; the same 4 bits per weight as the planes)
    if (fmt == LMX_FMT_INT4 && mfma_batched()) {
      std::vector<uint8_t> nib;
      try {
        nib.resize(w->Kp * w->Npad / 2);
      } catch (const std::bad_alloc &) {
        free_weight(w);
        return fail(LMX_ERR_OUT_OF_MEMORY, "host staging allocation failed");
      }
      nibble_tiles(planes, rows, row_bytes, w->Npad, w->Kp, nib.data());
      if ((e = hipMalloc(&w->d_nib, nib.size())) != hipSuccess ||
          (e = hipMemcpy(w->d_nib, nib.data(), nib.size(), hipMemcpyHostToDevice)) != hipSuccess) {
        free_weight(w);
        return hip_fail(e, "hipMalloc (matrix-core codes)");
      }
    }
  }
  if ((e = hipMemcpy(w->d_planes, tiles.data(), w->tile_bytes, hipMemcpyHostToDevice)) != hipSuccess ||
      (e = hipMemcpy(w->d_scales, sc.data(), w->scale_bytes, hipMemcpyHostToDevice)) != hipSuccess ||
      (e = hipMemset(w->d_counters, 0, row_blocks * sizeof(unsigned))) != hipSuccess ||
      (e = hipDeviceSynchronize()) != hipSuccess) {
    free_weight(w);
    return hip_fail(e, "upload (weight)");
  }
  *out = w;
  return LMX_OK;
}

int check_weight(const lmx_weight *w) {
  if (!w) return fail(LMX_ERR_INVALID_ARGUMENT, "weight handle is NULL");
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  if (dev != w->device)
    return fail(LMX_ERR_INVALID_ARGUMENT, "weight lives on device %d, current device is %d", w->device, dev);
  return LMX_OK;
}

bool is_pow2(size_t n) { return n && !(n & (n - 1)); }

// The GEMV kernel reads x with aligned float4 loads; an unaligned x or a
// length that is not a multiple of 4 is first copied, zero-padded, into the
// handle's staging buffer.
int stage_if_needed(const lmx_weight *w, GemvArgs &a, void *stream) {
  if (reinterpret_cast<size_t>(a.x) % 16 == 0 && w->cols % 4 == 0) return LMX_OK;
  int st = launch_stage_x(a.x, w->cols, w->d_xrot, w->Kp, stream);
  if (st) return st;
  a.x = w->d_xrot;
  a.cols = int(w->Kp);
  return LMX_OK;
}

}  // namespace

// Batched vectors in groups of 16/8/4 through the batched kernel (weights
// read once per group; below 4 vectors one GEMV per vector is faster), a
// group of 4 through the four-vector full-K kernel where the handle's plan
// has one; returns the number of vectors done.  Needs x
// 16-byte aligned with cols % 4 == 0 (every vector then is).  Uses the
// handle's batched partials, allocated with the handle.
int gemv_batched(const lmx_weight *w, GemvArgs a, const float *x, float *y, size_t batch, void *stream,
                 size_t *done) {
  *done = 0;
  if (a.epi != kEpiStore && !batched_epilogue_ok(w, a.epi, batch))
    return fail(LMX_ERR_INVALID_ARGUMENT, "batched epilogue %d does not cover %zu vectors of a %zu x %zu weight", a.epi,
                batch, w->rows, w->cols);
  if (!w->batched || batch < 4 || reinterpret_cast<size_t>(x) % 16 || w->cols % 4) return LMX_OK;
  const float *resid = a.resid;  // [batch][rows] residual rows, offset with the vectors
  float *y2 = a.y2;               // kEpiNormOut: [batch][rows]
  const size_t out_rows = a.epi == kEpiSiluPair ? w->rows / 2 : w->rows;
  while (batch - *done >= 4) {
    const size_t left = batch - *done;
    const int nb = left >= 16 ? 16 : left >= 8 ? 8 : 4;
    if (size_t(nb) * batched_slice_splits(w->Npad, w->Kp) * w->Npad > w->bpartials_cap)
      return fail(LMX_ERR_INVALID_ARGUMENT, "batched partials of %zu floats hold no group of %d", w->bpartials_cap, nb);
    a.x = x + *done * w->cols;
    a.y = y + *done * out_rows;
    a.y2 = y2 ? y2 + *done * w->rows : nullptr;
    a.resid = resid ? resid + *done * w->rows : nullptr;
    a.cols = int(w->cols);
    a.partials = w->d_bpartials;
    a.nib = w->d_nib;
    if (nb == 4 && a.epi != kEpiNormOut && a.epi != kEpiPartials) {   // one full-K launch where the plan allows
      const int q = launch_gemv_quad(w->format, a, stream);
      if (q != 1) {
        if (q) return q;
        *done += 4;
        continue;
      }
    }
    int st = launch_gemv_batch(w->format, a, nb, stream);   // RMSNorm in groups of 4 only
    if (st) return st;
    *done += size_t(nb);
  }
  return LMX_OK;
}

bool batched_epilogue_ok(const lmx_weight *w, int epi, size_t batch) {
  if (!w->batched || batch < 4 || batch % 4 || w->cols % 4) return false;   // every vector in a group of 16/8/4
  if (epi == kEpiSiluPair) return w->rows % 8 == 0;
  if (epi == kEpiNormOut) return w->rows <= size_t(kNormOutMaxRows);
  if (epi == kEpiPartials) return batch == 4 || batch == 8 || batch == 16;   // one group: one set of partials
  return epi == kEpiStore;
}

GemvArgs weight_args(const lmx_weight *w) {
  GemvArgs a{};
  a.planes = w->d_planes;
  a.scales = w->d_scales;
  a.partials = w->d_partials;
  a.counters = w->d_counters;
  a.rows = int(w->rows);
  a.Npad = int(w->Npad);
  a.cols = int(w->cols);
  a.Kp = int(w->Kp);
  a.group_chunks = int(w->group / kChunk);
  a.gshift = -1;
  for (int sh = 0; sh < 31; ++sh)
    if ((1 << sh) == a.group_chunks) a.gshift = sh;
  a.n_groups = int(w->n_groups);
  a.kslice = w->kslice;
  a.reduce = w->reduce;
  a.waves = w->waves;
  a.fullk = w->fullk;
  a.kfamily = w->kfamily;
  a.staged = w->staged;
  a.xmode = kXModeNone;
  return a;
}

}  // namespace lmx

using namespace lmx;

extern "C" {

const char *lmx_status_string(int status) {
  switch (status) {
  case LMX_OK: return "ok";
  case LMX_ERR_INVALID_ARGUMENT: return "invalid argument";
  case LMX_ERR_UNSUPPORTED_FORMAT: return "unsupported format";
  case LMX_ERR_NO_DEVICE: return "no device";
  case LMX_ERR_OUT_OF_MEMORY: return "out of memory";
  case LMX_ERR_LAUNCH_FAILED: return "launch failed";
  case LMX_ERR_HIP: return "HIP runtime error";
  }
  return "unknown status";
}

const char *lmx_last_error(void) { return g_err; }

int lmx_version(void) { return 100; }

int lmx_device_count(int *count) {
  if (!count) return fail(LMX_ERR_INVALID_ARGUMENT, "count is NULL");
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  *count = (e == hipSuccess && n > 0) ? n : 0;
  if (*count == 0) return fail(LMX_ERR_NO_DEVICE, "no HIP device visible");
  return LMX_OK;
}

int lmx_format_info(int format, int *planes, int *stages) {
  FormatInfo fi;
  if (!format_info(format, &fi)) return fail(LMX_ERR_UNSUPPORTED_FORMAT, "unknown format %d", format);
  if (planes) *planes = fi.planes;
  if (stages) *stages = fi.stages;
  return LMX_OK;
}

int lmx_block_bytes(int format, size_t *bytes) {
  FormatInfo fi;
  if (!format_info(format, &fi)) return fail(LMX_ERR_UNSUPPORTED_FORMAT, "unknown format %d", format);
  if (!fi.block_bytes) return fail(LMX_ERR_UNSUPPORTED_FORMAT, "format %d has no reference block", format);
  if (!bytes) return fail(LMX_ERR_INVALID_ARGUMENT, "bytes is NULL");
  *bytes = fi.block_bytes;
  return LMX_OK;
}

int lmx_blocks_to_planes(int format, const void *blocks, size_t num_blocks, size_t rows, size_t cols,
                         uint8_t *planes, float *scales) {
  FormatInfo fi;
  if (!format_info(format, &fi) || !fi.block_bytes)
    return fail(LMX_ERR_UNSUPPORTED_FORMAT, "format %d has no reference block", format);
  if (!blocks || !planes || !scales || rows == 0 || cols == 0)
    return fail(LMX_ERR_INVALID_ARGUMENT, "NULL pointer or empty shape");
  if (num_blocks != rows * ((cols + 255) / 256))
    return fail(LMX_ERR_INVALID_ARGUMENT, "num_blocks %zu != rows*ceil(cols/256) = %zu", num_blocks,
                rows * ((cols + 255) / 256));
  return blocks_to_planes(format, static_cast<const uint8_t *>(blocks), rows, cols, planes, scales);
}

int lmx_planes_to_blocks(int format, const uint8_t *planes, const float *scales, size_t rows, size_t cols,
                         void *blocks, size_t num_blocks) {
  FormatInfo fi;
  if (!format_info(format, &fi) || !fi.block_bytes)
    return fail(LMX_ERR_UNSUPPORTED_FORMAT, "format %d has no reference block", format);
  if (!blocks || !planes || !scales || rows == 0 || cols == 0)
    return fail(LMX_ERR_INVALID_ARGUMENT, "NULL pointer or empty shape");
  if (num_blocks != rows * ((cols + 255) / 256))
    return fail(LMX_ERR_INVALID_ARGUMENT, "num_blocks %zu != rows*ceil(cols/256)", num_blocks);
  return planes_to_blocks(format, planes, scales, rows, cols, static_cast<uint8_t *>(blocks));
}

int lmx_tile_bytes(int format, size_t rows, size_t cols, size_t *bytes) {
  FormatInfo fi;
  if (!format_info(format, &fi)) return fail(LMX_ERR_UNSUPPORTED_FORMAT, "unknown format %d", format);
  if (!bytes || rows == 0 || cols == 0) return fail(LMX_ERR_INVALID_ARGUMENT, "NULL pointer or empty shape");
  *bytes = (round_up(cols, kRotChunk) / kChunk) * fi.planes * round_up(rows, kWave) * 16;
  return LMX_OK;
}

int lmx_tile_planes(int format, const uint8_t *planes, size_t rows, size_t cols, uint8_t *tiles) {
  FormatInfo fi;
  if (!format_info(format, &fi)) return fail(LMX_ERR_UNSUPPORTED_FORMAT, "unknown format %d", format);
  if (!planes || !tiles || rows == 0 || cols == 0 || cols % 8)
    return fail(LMX_ERR_INVALID_ARGUMENT, "NULL pointer, empty shape or cols not a multiple of 8");
  tile_planes(format, planes, rows, cols / 8, round_up(rows, kWave), round_up(cols, kRotChunk), tiles);
  return LMX_OK;
}

int lmx_untile_planes(int format, const uint8_t *tiles, size_t rows, size_t cols, uint8_t *planes) {
  FormatInfo fi;
  if (!format_info(format, &fi)) return fail(LMX_ERR_UNSUPPORTED_FORMAT, "unknown format %d", format);
  if (!planes || !tiles || rows == 0 || cols == 0 || cols % 8)
    return fail(LMX_ERR_INVALID_ARGUMENT, "NULL pointer, empty shape or cols not a multiple of 8");
  untile_planes(format, tiles, rows, cols / 8, round_up(rows, kWave), round_up(cols, kRotChunk), planes);
  return LMX_OK;
}

int lmx_tile_scales(int format, const float *scales, size_t rows, size_t cols, size_t group, float *out,
                    size_t *bytes) {
  FormatInfo fi;
  if (!format_info(format, &fi)) return fail(LMX_ERR_UNSUPPORTED_FORMAT, "unknown format %d", format);
  if (!bytes) return fail(LMX_ERR_INVALID_ARGUMENT, "bytes is NULL");
  if (rows == 0 || cols == 0 || cols % 8)
    return fail(LMX_ERR_INVALID_ARGUMENT, "rows/cols must be > 0 and cols a multiple of 8");
  if (group >= round_up(cols, kRotChunk)) group = 0;
  if (group && group % kChunk)
    return fail(LMX_ERR_INVALID_ARGUMENT, "group %zu must be a multiple of 128 (or 0 = per row)", group);
  lmx_weight w;
  plan_weight(&w, format, rows, cols, group);
  if (!out) {
    *bytes = w.scale_bytes;
    return LMX_OK;
  }
  if (!scales) return fail(LMX_ERR_INVALID_ARGUMENT, "scales is NULL");
  if (*bytes != w.scale_bytes) return fail(LMX_ERR_INVALID_ARGUMENT, "bytes %zu != %zu", *bytes, w.scale_bytes);
  const size_t ng_src = group ? (cols + group - 1) / group : 1;
  std::fill(out, out + w.scale_bytes / sizeof(float), 0.0f);
  for (int s = 0; s < fi.stages; ++s)
    for (size_t r = 0; r < rows; ++r)
      for (size_t g = 0; g < ng_src && g < w.n_groups; ++g)
        out[(size_t(s) * w.n_groups + g) * w.Npad + r] = scales[(size_t(s) * rows + r) * ng_src + g];
  return LMX_OK;
}

int lmx_weight_create(const lmx_planes_desc *d, lmx_weight **out) {
  if (!d || !out) return fail(LMX_ERR_INVALID_ARGUMENT, "desc or out is NULL");
  *out = nullptr;
  FormatInfo fi;
  if (!format_info(d->format, &fi)) return fail(LMX_ERR_UNSUPPORTED_FORMAT, "unknown format %d", d->format);
  if (!d->planes || !d->scales) return fail(LMX_ERR_INVALID_ARGUMENT, "planes or scales is NULL");
  if (d->rows == 0 || d->cols == 0 || d->cols % 8)
    return fail(LMX_ERR_INVALID_ARGUMENT, "rows/cols must be > 0 and cols a multiple of 8");
  if (d->rows > (1u << 30) || d->cols > (1u << 28))
    return fail(LMX_ERR_INVALID_ARGUMENT, "shape %zu x %zu too large", d->rows, d->cols);
  size_t group = d->group;
  if (group >= round_up(d->cols, kRotChunk)) group = 0;
  if (group && group % kChunk)
    return fail(LMX_ERR_INVALID_ARGUMENT, "group %zu must be a multiple of 128 (or 0 = per row)", d->group);
  const size_t ng_src = group ? (d->cols + group - 1) / group : 1;
  return upload(d->format, d->rows, d->cols, group, d->planes, d->cols / 8, d->scales, ng_src, out);
}

int lmx_weight_from_blocks(int format, const void *blocks, size_t num_blocks, size_t rows, size_t cols,
                           lmx_weight **out) {
  if (!out) return fail(LMX_ERR_INVALID_ARGUMENT, "out is NULL");
  *out = nullptr;
  FormatInfo fi;
  if (!format_info(format, &fi) || !fi.block_bytes)
    return fail(LMX_ERR_UNSUPPORTED_FORMAT, "format %d has no reference block", format);
  if (!blocks || rows == 0 || cols == 0) return fail(LMX_ERR_INVALID_ARGUMENT, "NULL blocks or empty shape");
  const size_t bpr = (cols + 255) / 256;
  if (num_blocks != rows * bpr)
    return fail(LMX_ERR_INVALID_ARGUMENT, "num_blocks %zu != rows*ceil(cols/256) = %zu", num_blocks, rows * bpr);
  std::vector<uint8_t> planes;
  std::vector<float> scales;
  try {
    planes.resize(size_t(fi.planes) * rows * bpr * 32);
    scales.resize(size_t(fi.stages) * rows * bpr);
  } catch (const std::bad_alloc &) {
    return fail(LMX_ERR_OUT_OF_MEMORY, "host staging allocation failed");
  }
  int st = blocks_to_planes(format, static_cast<const uint8_t *>(blocks), rows, cols, planes.data(), scales.data());
  if (st) return st;
  return upload(format, rows, cols, 256, planes.data(), bpr * 32, scales.data(), bpr, out);
}

int lmx_weight_destroy(lmx_weight *w) {
  free_weight(w);
  return LMX_OK;
}

int lmx_weight_info(const lmx_weight *w, int *format, size_t *rows, size_t *cols, size_t *device_bytes) {
  if (!w) return fail(LMX_ERR_INVALID_ARGUMENT, "weight handle is NULL");
  if (format) *format = w->format;
  if (rows) *rows = w->rows;
  if (cols) *cols = w->cols;
  if (device_bytes) *device_bytes = w->tile_bytes + w->scale_bytes;
  return LMX_OK;
}

int lmx_weight_kernel_config(const lmx_weight *w, int *fullk, int *kslice, int *staged) {
  if (!w) return fail(LMX_ERR_INVALID_ARGUMENT, "weight handle is NULL");
  if (fullk) *fullk = w->fullk;
  if (kslice) *kslice = w->kslice;
  if (staged) *staged = w->staged;
  return LMX_OK;
}

int lmx_weight_read_tiles(const lmx_weight *w, uint8_t *tiles, size_t bytes) {
  int st = check_weight(w);
  if (st) return st;
  if (!tiles || bytes != w->tile_bytes)
    return fail(LMX_ERR_INVALID_ARGUMENT, "tiles NULL or bytes %zu != %zu", bytes, w->tile_bytes);
  hipError_t e = hipMemcpy(tiles, w->d_planes, bytes, hipMemcpyDeviceToHost);
  if (e != hipSuccess) return hip_fail(e, "hipMemcpy (read tiles)");
  return LMX_OK;
}

int lmx_gemv(const lmx_weight *w, const float *x, float *y, size_t batch, unsigned flags, void *stream) {
  int st = check_weight(w);
  if (st) return st;
  return gemv_impl(w, x, y, batch, flags, stream);
}

}  // extern "C"

namespace lmx {
int gemv_impl(const lmx_weight *w, const float *x, float *y, size_t batch, unsigned flags, void *stream) {
  int st;
  if (!x || !y) return fail(LMX_ERR_INVALID_ARGUMENT, "x or y is NULL");
  if (reinterpret_cast<size_t>(x) % 4 || reinterpret_cast<size_t>(y) % 4)
    return fail(LMX_ERR_INVALID_ARGUMENT, "x and y must be 4-byte aligned");
  if (batch == 0) return LMX_OK;
  if (flags != LMX_ROTATE_NONE && flags != LMX_ROTATE_FWHT256 && flags != LMX_ROTATE_FWHT_FULL)
    return fail(LMX_ERR_INVALID_ARGUMENT, "unknown flags 0x%x", flags);
  if (flags == LMX_ROTATE_FWHT_FULL && (!is_pow2(w->cols) || w->cols < 256 || w->cols > 16384))
    return fail(LMX_ERR_INVALID_ARGUMENT, "length-K FWHT needs cols a power of two in [256, 16384], got %zu",
                w->cols);
  GemvArgs a = weight_args(w);
  size_t b0 = 0;
  if (flags != LMX_ROTATE_FWHT_FULL) {
    a.rotate = flags == LMX_ROTATE_FWHT256 ? LMX_ROTATE_FWHT256 : LMX_ROTATE_NONE;
    if ((st = gemv_batched(w, a, x, y, batch, stream, &b0))) return st;
  }
  for (size_t b = b0; b < batch; ++b) {
    a.x = x + b * w->cols;
    a.y = y + b * w->rows;
    a.cols = int(w->cols);
    a.partials = w->d_partials;
    a.rotate = flags == LMX_ROTATE_FWHT256 ? LMX_ROTATE_FWHT256 : LMX_ROTATE_NONE;
    if (flags == LMX_ROTATE_FWHT_FULL) {
      st = launch_fwht_full(a.x, w->d_xrot, w->cols, stream);
      if (st) return st;
      a.x = w->d_xrot;
    } else if ((st = stage_if_needed(w, a, stream)) != LMX_OK) {
      return st;
    }
    st = launch_gemv(w->format, a, stream);
    if (st) return st;
  }
  return LMX_OK;
}
}  // namespace lmx

extern "C" {

int lmx_linear(const lmx_weight *w, const float *bias, const float *x, float *y, size_t batch, void *stream) {
  int st = check_weight(w);
  if (st) return st;
  if (!x || !y) return fail(LMX_ERR_INVALID_ARGUMENT, "x or y is NULL");
  if (batch == 0) return LMX_OK;
  const bool rotate = w->format == LMX_FMT_TERNARY || w->format == LMX_FMT_BINARY ||
                      w->format == LMX_FMT_RRQ2 || w->format == LMX_FMT_RRQ3;
  GemvArgs a = weight_args(w);
  a.bias = bias;
  a.rotate = rotate ? LMX_ROTATE_FWHT256 : LMX_ROTATE_NONE;
  size_t b0 = 0;
  if ((st = gemv_batched(w, a, x, y, batch, stream, &b0))) return st;
  for (size_t b = b0; b < batch; ++b) {
    a.x = x + b * w->cols;
    a.y = y + b * w->rows;
    a.cols = int(w->cols);
    a.partials = w->d_partials;
    if ((st = stage_if_needed(w, a, stream)) != LMX_OK) return st;
    st = launch_gemv(w->format, a, stream);
    if (st) return st;
  }
  return LMX_OK;
}

int lmx_fwht256(float *x, size_t n, void *stream) {
  if (!x) return fail(LMX_ERR_INVALID_ARGUMENT, "x is NULL");
  if (n % kRotChunk) return fail(LMX_ERR_INVALID_ARGUMENT, "n %zu is not a multiple of 256", n);
  if (reinterpret_cast<size_t>(x) % 16) return fail(LMX_ERR_INVALID_ARGUMENT, "x must be 16-byte aligned");
  int dev;
  int st = require_device(&dev);
  if (st) return st;
  return launch_fwht256(x, n, stream);
}

int lmx_precompute_luts(const float *x, size_t n, unsigned flags, float *luts, void *stream) {
  if (!x || !luts) return fail(LMX_ERR_INVALID_ARGUMENT, "x or luts is NULL");
  if (flags != LMX_ROTATE_NONE && flags != LMX_ROTATE_FWHT256)
    return fail(LMX_ERR_INVALID_ARGUMENT, "flags must be NONE or FWHT256");
  if (flags == LMX_ROTATE_FWHT256 && n % kRotChunk)
    return fail(LMX_ERR_INVALID_ARGUMENT, "rotated table build needs n a multiple of 256");
  if (n > (size_t(1) << 30)) return fail(LMX_ERR_INVALID_ARGUMENT, "n too large");
  int dev;
  int st = require_device(&dev);
  if (st) return st;
  return launch_precompute_luts(x, n, flags, luts, stream);
}

int lmx_extract_indices(const uint8_t *sign_plane, const uint8_t *zero_plane, size_t n_groups, uint8_t *pos_idx,
                        uint8_t *neg_idx, void *stream) {
  if (!sign_plane || !zero_plane || !pos_idx || !neg_idx)
    return fail(LMX_ERR_INVALID_ARGUMENT, "NULL pointer");
  int dev;
  int st = require_device(&dev);
  if (st) return st;
  return launch_extract_indices(sign_plane, zero_plane, n_groups, pos_idx, neg_idx, stream);
}

}  // extern "C"
