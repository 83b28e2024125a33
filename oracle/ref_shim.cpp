// ref_shim.cpp -- extern "C" entry points onto the reference's own kernels.
//
// TEST INFRASTRUCTURE ONLY.  oracle/Makefile compiles this file together with
// the reference's kernel sources where they lie (src/kernels/*.cpp under the
// LutMac tree, headers from its include/) into oracle/_ref/libref.so.  It lets
// the tests and tests/golden/gen_golden.py run the reference's x86 path on the
// same bytes the HIP path consumes.  Nothing of the reference is copied here:
// this file only marshals raw AoS block bytes into the reference's types and
// calls its functions.
#include "lutmac/lut_gemm.hpp"
#include "lutmac/quantize.hpp"
#include "lutmac/transform.hpp"
#include "lutmac/types.hpp"

#include <cstring>
#include <vector>

using namespace lutmac;

namespace {
template <typename B> std::vector<B> to_blocks(const void *p, size_t n) {
  std::vector<B> v(n);
  std::memcpy(v.data(), p, n * sizeof(B));
  return v;
}
template <typename B> size_t from_blocks(const std::vector<B> &v, void *out, size_t cap) {
  size_t n = v.size() * sizeof(B);
  if (out && cap >= n) std::memcpy(out, v.data(), n);
  return n;
}
} // namespace

extern "C" {

size_t ref_sizeof_block(int fmt) {
  switch (fmt) {
  case 1: return sizeof(BitPlaneBlock);
  case 2: return sizeof(BinaryBlock);
  case 3: return sizeof(Int2Block);
  case 5: return sizeof(Int3Block);
  case 6: return sizeof(Int4Block);
  case 7: return sizeof(Int8Block);
  }
  return 0;
}

void ref_precompute_luts(const float *x, size_t n, float *luts) { precompute_luts(x, n, luts); }

void ref_extract_indices(const uint8_t *s, const uint8_t *z, size_t g, uint8_t *pos, uint8_t *neg) {
  uint8_t p = 0, q = 0;
  extract_indices(s, z, g, p, q);
  *pos = p;
  *neg = q;
}

void ref_fwht_256(float *d) { fwht_256(d); }
void ref_apply_hadamard_rotation(float *d, size_t n) { apply_hadamard_rotation(d, n); }

void ref_pack_to_bitplanes(const int8_t *t, size_t n, uint8_t *s, uint8_t *z) {
  std::vector<TernaryValue> tv(n);
  for (size_t i = 0; i < n; ++i) tv[i] = static_cast<TernaryValue>(t[i]);
  pack_to_bitplanes(tv.data(), n, s, z);
}

void ref_unpack_from_bitplanes(const uint8_t *s, const uint8_t *z, size_t n, int8_t *t) {
  std::vector<TernaryValue> tv(n);
  unpack_from_bitplanes(s, z, n, tv.data());
  for (size_t i = 0; i < n; ++i) t[i] = static_cast<int8_t>(tv[i]);
}

// Raw dispatchers, exactly as the callers in model.cpp / tests reach them.
void ref_gemv(int fmt, const void *blocks, size_t num_blocks, const float *x, float *y, size_t M,
              size_t K) {
  switch (fmt) {
  case 1: lut_gemv(static_cast<const BitPlaneBlock *>(blocks), num_blocks, x, y, M, K); break;
  case 2: lut_gemv_binary(static_cast<const BinaryBlock *>(blocks), num_blocks, x, y, M, K); break;
  case 3: int2_gemv(static_cast<const Int2Block *>(blocks), num_blocks, x, y, M, K); break;
  case 5: int3_gemv(static_cast<const Int3Block *>(blocks), num_blocks, x, y, M, K); break;
  case 6: int4_gemv(static_cast<const Int4Block *>(blocks), num_blocks, x, y, M, K); break;
  case 7: int8_gemv(static_cast<const Int8Block *>(blocks), num_blocks, x, y, M, K); break;
  }
}

// lut_linear over a PackedTensor assembled from raw blocks.
int ref_lut_linear(int fmt, const void *blocks, size_t num_blocks, const float *bias, const float *x,
                   float *y, size_t M, size_t K, size_t batch) {
  PackedTensor w;
  w.shape = {M, K};
  w.is_quantized = true;
  switch (fmt) {
  case 1: w.quant_bits = 2; w.blocks = to_blocks<BitPlaneBlock>(blocks, num_blocks); break;
  case 2: w.quant_bits = 1; w.binary_blocks = to_blocks<BinaryBlock>(blocks, num_blocks); break;
  case 3: w.quant_bits = 2; w.int2_blocks = to_blocks<Int2Block>(blocks, num_blocks); break;
  case 5: w.quant_bits = 3; w.int3_blocks = to_blocks<Int3Block>(blocks, num_blocks); break;
  case 6: w.quant_bits = 4; w.int4_blocks = to_blocks<Int4Block>(blocks, num_blocks); break;
  case 7: w.quant_bits = 8; w.int8_blocks = to_blocks<Int8Block>(blocks, num_blocks); break;
  default: return -1;
  }
  lut_linear(w, bias, x, y, batch);
  return 0;
}

// Reference quantizers (quantize.hpp) for fixture generation.  Returns the
// byte size of the block array; copies it when cap is large enough.
size_t ref_quantize(int fmt, const float *data, size_t M, size_t K, void *out, size_t cap) {
  std::vector<size_t> shape = {M, K};
  switch (fmt) {
  case 1: return from_blocks(quantize_tensor(data, shape).blocks, out, cap);
  case 2: return from_blocks(quantize_tensor_binary(data, shape).binary_blocks, out, cap);
  case 3: return from_blocks(quantize_tensor_int2(data, shape).int2_blocks, out, cap);
  case 5: return from_blocks(quantize_tensor_int3(data, shape).int3_blocks, out, cap);
  case 6: return from_blocks(quantize_tensor_int4(data, shape).int4_blocks, out, cap);
  case 7: return from_blocks(quantize_tensor_int8(data, shape).int8_blocks, out, cap);
  }
  return 0;
}

// Dequantized weight w[i] of block b via the reference accessors (get()).
float ref_block_get(int fmt, const void *blocks, size_t b, size_t i) {
  switch (fmt) {
  case 1: return static_cast<const BitPlaneBlock *>(blocks)[b].get(i);
  case 2: return static_cast<const BinaryBlock *>(blocks)[b].get(i);
  case 3: return static_cast<const Int2Block *>(blocks)[b].get(i);
  case 5: return static_cast<const Int3Block *>(blocks)[b].get(i);
  case 6: return static_cast<const Int4Block *>(blocks)[b].get(i);
  case 7: return static_cast<const Int8Block *>(blocks)[b].get(static_cast<int>(i));
  }
  return 0.0f;
}

} // extern "C"
