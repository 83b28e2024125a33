// lut_gemm_compat.cpp -- host-pointer drop-ins with the reference's kernel
// API semantics (include/lutmac/lut_gemm.hpp, include/lutmac/transform.hpp),
// implemented over the device C ABI.
//
// Every function takes and returns HOST memory exactly like the reference's
// scalar kernels: activations in, outputs overwritten.  The reference's
// weights are immutable after load, so the first call with a given block
// array repacks and uploads it once; later calls reuse the device handle
// (keyed by block pointer, count, shape and format).  Activations/outputs go
// through per-thread device staging buffers on a per-thread stream.
//
// The reference functions return void and have no error channel; these
// entry points return an lmx_status, and the C++ wrappers in
// include/lutmac_hip_compat.h abort with the message on failure (never a silent CPU
// fallback).
#include <hip/hip_runtime.h>

#include <cstring>
#include <map>
#include <mutex>
#include <tuple>
#include <vector>

#include "lmx_internal.hpp"
#include "lutmac_hip_compat.h"

namespace {

using Key = std::tuple<const void *, size_t, size_t, size_t, int>;

struct WeightCache {
  std::mutex mu;
  std::map<Key, lmx_weight *> handles;
  ~WeightCache() {
    for (auto &kv : handles) lmx_weight_destroy(kv.second);
  }
};

WeightCache &cache() {
  static WeightCache c;
  return c;
}

int get_weight(int fmt, const void *blocks, size_t num_blocks, size_t M, size_t K, lmx_weight **out) {
  WeightCache &c = cache();
  std::lock_guard<std::mutex> lock(c.mu);
  const Key key{blocks, num_blocks, M, K, fmt};
  auto it = c.handles.find(key);
  if (it != c.handles.end()) {
    *out = it->second;
    return LMX_OK;
  }
  lmx_weight *w = nullptr;
  int st = lmx_weight_from_blocks(fmt, blocks, num_blocks, M, K, &w);
  if (st) return st;
  c.handles.emplace(key, w);
  *out = w;
  return LMX_OK;
}

// Per-thread device staging (the reference's lut_linear keeps a
// static thread_local pad buffer; this is its device counterpart).
struct Staging {
  hipStream_t stream = nullptr;
  float *d_in = nullptr, *d_out = nullptr, *d_bias = nullptr;
  size_t n_in = 0, n_out = 0, n_bias = 0;
  ~Staging() {
    if (d_in) (void)hipFree(d_in);
    if (d_out) (void)hipFree(d_out);
    if (d_bias) (void)hipFree(d_bias);
    if (stream) (void)hipStreamDestroy(stream);
  }
};

thread_local Staging g_stage;

int ensure(float **p, size_t *have, size_t need) {
  if (*have >= need) return LMX_OK;
  if (*p) (void)hipFree(*p);
  *p = nullptr;
  *have = 0;
  hipError_t e = hipMalloc(reinterpret_cast<void **>(p), need * sizeof(float));
  if (e != hipSuccess) return lmx::fail(LMX_ERR_OUT_OF_MEMORY, "staging hipMalloc: %s", hipGetErrorString(e));
  *have = need;
  return LMX_OK;
}

int stage_stream() {
  if (g_stage.stream) return LMX_OK;
  hipError_t e = hipStreamCreateWithFlags(&g_stage.stream, hipStreamNonBlocking);
  if (e != hipSuccess) return lmx::fail(LMX_ERR_HIP, "hipStreamCreate: %s", hipGetErrorString(e));
  return LMX_OK;
}

int h2d(float *d, const float *h, size_t n) {
  hipError_t e = hipMemcpyAsync(d, h, n * sizeof(float), hipMemcpyHostToDevice, g_stage.stream);
  return e == hipSuccess ? LMX_OK : lmx::fail(LMX_ERR_HIP, "H2D copy: %s", hipGetErrorString(e));
}

int d2h_sync(float *h, const float *d, size_t n) {
  hipError_t e = hipMemcpyAsync(h, d, n * sizeof(float), hipMemcpyDeviceToHost, g_stage.stream);
  if (e == hipSuccess) e = hipStreamSynchronize(g_stage.stream);
  return e == hipSuccess ? LMX_OK : lmx::fail(LMX_ERR_HIP, "D2H copy: %s", hipGetErrorString(e));
}

// Shared body of the raw per-format kernels and lut_linear.
int host_run(int fmt, const void *blocks, size_t num_blocks, const float *bias, const float *input, float *output,
             size_t M, size_t K, size_t batch, bool linear) {
  if (!blocks || !input || !output) return lmx::fail(LMX_ERR_INVALID_ARGUMENT, "NULL pointer");
  if (M == 0 || K == 0 || batch == 0) return LMX_OK;
  lmx_weight *w = nullptr;
  int st = get_weight(fmt, blocks, num_blocks, M, K, &w);
  if (st) return st;
  if ((st = stage_stream()) || (st = ensure(&g_stage.d_in, &g_stage.n_in, K * batch)) ||
      (st = ensure(&g_stage.d_out, &g_stage.n_out, M * batch)))
    return st;
  const float *d_bias = nullptr;
  if (bias) {
    if ((st = ensure(&g_stage.d_bias, &g_stage.n_bias, M)) || (st = h2d(g_stage.d_bias, bias, M))) return st;
    d_bias = g_stage.d_bias;
  }
  if ((st = h2d(g_stage.d_in, input, K * batch))) return st;
  st = linear ? lmx_linear(w, d_bias, g_stage.d_in, g_stage.d_out, batch, g_stage.stream)
              : lmx_gemv(w, g_stage.d_in, g_stage.d_out, batch, LMX_ROTATE_NONE, g_stage.stream);
  if (st) return st;
  return d2h_sync(output, g_stage.d_out, M * batch);
}

}  // namespace

extern "C" {

int lmx_host_gemv(int format, const void *blocks, size_t num_blocks, const float *activations, float *output,
                  size_t M, size_t K) {
  return host_run(format, blocks, num_blocks, nullptr, activations, output, M, K, 1, false);
}

int lmx_host_lut_linear(int format, const void *blocks, size_t num_blocks, const float *bias, const float *input,
                        float *output, size_t M, size_t K, size_t batch_size) {
  return host_run(format, blocks, num_blocks, bias, input, output, M, K, batch_size, true);
}

int lmx_host_apply_hadamard_rotation(float *data, size_t n) {
  if (!data) return lmx::fail(LMX_ERR_INVALID_ARGUMENT, "NULL pointer");
  const size_t whole = n / 256 * 256;  // whole 256-chunks only (transform_simd.cpp:105-109)
  if (whole == 0) return LMX_OK;
  int st;
  if ((st = stage_stream()) || (st = ensure(&g_stage.d_in, &g_stage.n_in, whole)) ||
      (st = h2d(g_stage.d_in, data, whole)) || (st = lmx_fwht256(g_stage.d_in, whole, g_stage.stream)))
    return st;
  return d2h_sync(data, g_stage.d_in, whole);
}

int lmx_host_precompute_luts(const float *activations, size_t n, float *luts) {
  if (!activations || !luts) return lmx::fail(LMX_ERR_INVALID_ARGUMENT, "NULL pointer");
  const size_t groups = n / 4;
  if (groups == 0) return LMX_OK;
  int st;
  if ((st = stage_stream()) || (st = ensure(&g_stage.d_in, &g_stage.n_in, n)) ||
      (st = ensure(&g_stage.d_out, &g_stage.n_out, groups * 16)) || (st = h2d(g_stage.d_in, activations, n)) ||
      (st = lmx_precompute_luts(g_stage.d_in, n, LMX_ROTATE_NONE, g_stage.d_out, g_stage.stream)))
    return st;
  return d2h_sync(luts, g_stage.d_out, groups * 16);
}

}  // extern "C"
