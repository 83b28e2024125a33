// lmx_probe.hip -- achievable-bandwidth yardstick: a plain streaming read of
// a device buffer (16-byte non-temporal loads, 512 workgroups of 1024
// threads, two loads in flight per thread; the fastest plain-read shape
// measured on MI355X at the 16-70 MB GEMV sizes).  It does no arithmetic
// beyond an XOR that keeps the loads live, so its time is what the memory
// system needs to deliver the same bytes a GEMV streams.
#include <hip/hip_runtime.h>

#include "lmx_internal.hpp"

namespace lmx {
namespace {

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(1024) void read_probe_kernel(const u32x4 *__restrict__ p, size_t n16,
                                                          unsigned *__restrict__ sink) {
  const size_t nt = size_t(gridDim.x) * blockDim.x;
  size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
  unsigned acc = 0;
  for (; i + nt < n16; i += 2 * nt) {
    const u32x4 a = __builtin_nontemporal_load(p + i), b = __builtin_nontemporal_load(p + i + nt);
    acc ^= a.x ^ a.y ^ a.z ^ a.w ^ b.x ^ b.y ^ b.z ^ b.w;
  }
  for (; i < n16; i += nt) {
    const u32x4 a = p[i];
    acc ^= a.x ^ a.y ^ a.z ^ a.w;
  }
  if (acc == 0x9E3779B9u) sink[0] = acc;   // practically never: keeps the loads
}

}  // namespace
}  // namespace lmx

extern "C" int lmx_hbm_read_probe(const void *buf, size_t bytes, unsigned *sink, void *stream) {
  using namespace lmx;
  if (!buf || !sink) return fail(LMX_ERR_INVALID_ARGUMENT, "NULL argument");
  if (reinterpret_cast<size_t>(buf) % 16 || bytes % 16)
    return fail(LMX_ERR_INVALID_ARGUMENT, "buffer and size must be 16-byte multiples");
  if (bytes == 0) return LMX_OK;
  read_probe_kernel<<<dim3(512), dim3(1024), 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const u32x4 *>(buf), bytes / 16, sink);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? LMX_OK : fail(LMX_ERR_LAUNCH_FAILED, "read probe launch: %s", hipGetErrorString(e));
}
