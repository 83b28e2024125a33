// lmx_noalloc.hip -- lmx_gemv_tiles_noalloc: the GEMV of lmx_gemv for a
// caller that cannot allocate (code under HIP graph capture, serving loops
// with a fixed memory budget).  The weights are the caller's own device
// buffers in the device tile layout (lmx_tile_planes / lmx_tile_scales), x
// and y are the caller's; every buffer the kernels need beyond those -- the
// split-K ticket counters, the staging copy of x and the split-K partial
// sums -- lives in `scratch`, a file-scope device array of kScratchBytes
// that each GPU holds for the life of the process.  Nothing here calls
// hipMalloc, hipFree or any allocating routine.
//
// Scratch layout (byte offsets, each region 256-byte aligned):
//   [0, 64 KiB)   ticket counters, one per 64-row block of a split-K plan: a
//                 fixed region, so no other call's staging or partials ever
//                 land on a counter (up to 16384 row blocks, Npad <= 1 Mi rows)
//   [64 KiB, +X)  staging copy of x (unaligned x, length-K FWHT)   X = Kp * 4
//   [.., ...)     split-K partials [Kp/kslice][Npad] fp32 (split-K plans only)
// The counters must read zero when a call starts: the first call on a
// device zeroes the whole array with a fill kernel and waits for it before
// any call may use the array, and every split-K launch leaves each counter
// it used at zero again (its last workgroup resets it).  Calls on one GPU
// share the array, so calls that overlap in time on one GPU (two streams,
// two threads) race; order them.
#include <hip/hip_runtime.h>

#include <mutex>

#include "lmx_internal.hpp"

constexpr size_t kScratchBytes = size_t(8) << 20;   // 8 MiB per GPU
constexpr size_t kCounterBytes = size_t(64) << 10;  // fixed ticket-counter region at offset 0

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace lmx {
namespace {

constexpr int kMaxDevices = 64;

__global__ __launch_bounds__(256) void zero_scratch_kernel(uint32_t *p, size_t n) {
  for (size_t i = size_t(blockIdx.x) * 256 + threadIdx.x; i < n; i += size_t(gridDim.x) * 256) p[i] = 0u;
}

std::mutex g_mu;
void *g_ptr[kMaxDevices] = {};   // each device's address of `scratch`, set once

// The device address of this device's `scratch` (never the host-side name),
// set up on the first call on the device: the zero fill is waited for before
// the address is published, so a call on any stream or thread that starts
// after this one returned finds zeroed counters.
int scratch_ptr(int dev, void *stream, unsigned char **out) {
  if (dev < 0 || dev >= kMaxDevices) return fail(LMX_ERR_NO_DEVICE, "device %d outside 0..%d", dev, kMaxDevices - 1);
  std::lock_guard<std::mutex> lock(g_mu);
  if (!g_ptr[dev]) {
    void *p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(LMX_ERR_HIP, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
    hipStream_t st = static_cast<hipStream_t>(stream);
    zero_scratch_kernel<<<dim3(1024), dim3(256), 0, st>>>(static_cast<uint32_t *>(p), kScratchBytes / 4);
    e = hipGetLastError();
    if (e != hipSuccess) return fail(LMX_ERR_LAUNCH_FAILED, "scratch zero fill: %s", hipGetErrorString(e));
    e = hipStreamSynchronize(st);
    if (e != hipSuccess) return fail(LMX_ERR_HIP, "scratch zero fill: %s", hipGetErrorString(e));
    g_ptr[dev] = p;
  }
  *out = static_cast<unsigned char *>(g_ptr[dev]);
  return LMX_OK;
}

}  // namespace
}  // namespace lmx

extern "C" int lmx_gemv_tiles_noalloc(int format, const void *tiles, const float *scales, size_t rows, size_t cols,
                                      size_t group, const float *x, float *y, size_t batch, unsigned flags,
                                      void *stream) {
  using namespace lmx;
  FormatInfo fi;
  if (!format_info(format, &fi)) return fail(LMX_ERR_UNSUPPORTED_FORMAT, "unknown format %d", format);
  if (!tiles || !scales) return fail(LMX_ERR_INVALID_ARGUMENT, "tiles or scales is NULL");
  if (rows == 0 || cols == 0 || cols % 8)
    return fail(LMX_ERR_INVALID_ARGUMENT, "rows/cols must be > 0 and cols a multiple of 8");
  if (rows > (1u << 30) || cols > (1u << 28))
    return fail(LMX_ERR_INVALID_ARGUMENT, "shape %zu x %zu too large", rows, cols);
  if (group >= round_up(cols, kRotChunk)) group = 0;
  if (group && group % kChunk)
    return fail(LMX_ERR_INVALID_ARGUMENT, "group %zu must be a multiple of 128 (or 0 = per row)", group);
  if (reinterpret_cast<size_t>(tiles) % 16 || reinterpret_cast<size_t>(scales) % 4)
    return fail(LMX_ERR_INVALID_ARGUMENT, "tiles must be 16-byte and scales 4-byte aligned");
  lmx_weight w;   // the plan lmx_weight_create would choose, over the caller's buffers
  plan_weight(&w, format, rows, cols, group);
  w.batched = false;   // one vector at a time: the batched kernel's partials would not fit
  const size_t row_blocks = w.Npad / kWave;
  const size_t staging = round_up(w.Kp * sizeof(float), 256);
  // split-K plans, and the layered full-K plan (which runs the split-K
  // kernel where it has no kernel form), need partials and ticket counters
  const bool splitk = !w.fullk || w.fullk == kFullK_8x8x2L;
  const size_t partials = splitk ? (w.Kp / size_t(w.kslice)) * w.Npad * sizeof(float) : 0;
  if ((splitk && row_blocks * sizeof(unsigned) > kCounterBytes) || kCounterBytes + staging + partials > kScratchBytes)
    return fail(LMX_ERR_INVALID_ARGUMENT,
                "%zu x %zu needs %zu B of scratch (ticket counters %zu B of %zu, x staging, split-K partials); "
                "lmx_gemv_tiles_noalloc holds %zu B per GPU: use a weight handle (lmx_gemv)",
                rows, cols, kCounterBytes + staging + partials, splitk ? row_blocks * sizeof(unsigned) : size_t(0),
                kCounterBytes, kScratchBytes);
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(LMX_ERR_NO_DEVICE, "hipGetDevice: %s", hipGetErrorString(e));
  unsigned char *base = nullptr;
  int st = scratch_ptr(dev, stream, &base);
  if (st) return st;
  w.device = dev;
  w.d_planes = const_cast<void *>(tiles);
  w.d_scales = const_cast<float *>(scales);
  w.d_counters = reinterpret_cast<unsigned *>(base);
  w.d_xrot = reinterpret_cast<float *>(base + kCounterBytes);
  w.d_partials = reinterpret_cast<float *>(base + kCounterBytes + staging);
  return gemv_impl(&w, x, y, batch, flags, stream);
}
