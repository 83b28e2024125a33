/*
 * lutmac_hip_compat.h -- host-pointer drop-ins for LutMac's kernel API.
 *
 * The extern "C" functions keep the argument meaning of the reference's
 * scalar kernels: host activations in, host outputs overwritten, weights as
 * the reference's AoS block arrays (BitPlaneBlock / BinaryBlock / Int2Block /
 * Int3Block / Int4Block / Int8Block).  Each returns an lmx_status.  The
 * reference reads the blocks on every call; here a block array is repacked
 * and uploaded on first use and cached by (pointer, count, M, K, format),
 * guarded by a fingerprint of its count and of up to 256 whole blocks spread
 * over the array, rechecked on every call: a mismatch re-uploads.  Call
 * lmx_host_forget(blocks) before freeing an array or rewriting part of it
 * (a change the sample cannot see), so no later call reuses stale device
 * weights; or set LMX_HOST_HASH=all in the environment, and every call
 * hashes the whole array (every rewrite is seen, at a host pass over the
 * array per call).  Calls from several threads are safe; calls that share one
 * weight are serialised on it.
 *
 * The C++ section maps the reference's names onto them (namespace
 * lutmac_hip); on a failing status it prints lmx_last_error() and aborts, the
 * reference's functions having no error channel.
 */
#ifndef LUTMAC_HIP_COMPAT_H
#define LUTMAC_HIP_COMPAT_H

#include <stddef.h>
#include <stdint.h>

#include "lutmac_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Raw per-format GEMV: activations hold ceil(K/256)*256 floats, already
 * zero-padded and rotated where the format needs it; output[M] overwritten.
 * Replaces lut_gemv (lut_gemm.hpp:189-204), lut_gemv_binary (172-184),
 * int2_gemv (280-292), int3_gemv (322-334), int4_gemv (238-250),
 * int8_gemv (396-408). */
int lmx_host_gemv(int format, const void *blocks, size_t num_blocks,
                  const float *activations, float *output, size_t M, size_t K);

/* lut_linear (lut_gemm.hpp:419-420, lut_gemm_scalar.cpp:68-180): per batch
 * row, zero-pad to ceil(K/256)*256, FWHT-256 for ternary/binary/2-bit,
 * GEMV, then + bias when bias is not NULL. */
int lmx_host_lut_linear(int format, const void *blocks, size_t num_blocks,
                        const float *bias, const float *input, float *output,
                        size_t M, size_t K, size_t batch_size);

/* Drops the cached device weights of the block array at `blocks` (all
 * shapes and formats), and every cached weight.  No reference counterpart:
 * the reference reads its blocks per call, so it has no copy to invalidate;
 * these tie the device copy's lifetime to the caller's PackedTensor. */
int lmx_host_forget(const void *blocks);
int lmx_host_cache_clear(void);

/* apply_hadamard_rotation (transform.hpp:19, transform_simd.cpp:101-110):
 * in place, whole 256-chunks only. */
int lmx_host_apply_hadamard_rotation(float *data, size_t n);

/* precompute_luts (lut_gemm.hpp:53-58): luts[n/4][16]. */
int lmx_host_precompute_luts(const float *activations, size_t n, float *luts);

/* precompute_lut (lut_gemm.hpp:30-44): the 16-entry table of one group of
 * 4 activations, lut[m] = sum of a_j over the set bits (3-j) of m. */
int lmx_host_precompute_lut(const float *activations, float *lut);

/* extract_indices (lut_gemm.hpp:79-99): group group_idx of a ternary
 * block's sign/zero planes (byte group_idx/2, high nibble for even groups)
 * -> pos_idx = non-zero and positive, neg_idx = non-zero and negative. */
int lmx_host_extract_indices(const uint8_t *sign_plane, const uint8_t *zero_plane, size_t group_idx,
                             uint8_t *pos_idx, uint8_t *neg_idx);

#ifdef __cplusplus
}  /* extern "C" */

#include <cstdio>
#include <cstdlib>

namespace lutmac_hip {

inline void check_or_abort(int status, const char *what) {
  if (status != LMX_OK) {
    std::fprintf(stderr, "lutmac_hip: %s failed: %s (%s)\n", what, lmx_status_string(status), lmx_last_error());
    std::abort();
  }
}

inline void lut_gemv(const void *blocks, size_t num_blocks, const float *activations, float *output, size_t M,
                     size_t K) {
  check_or_abort(lmx_host_gemv(LMX_FMT_TERNARY, blocks, num_blocks, activations, output, M, K), "lut_gemv");
}
inline void lut_gemv_binary(const void *blocks, size_t num_blocks, const float *activations, float *output,
                            size_t M, size_t K) {
  check_or_abort(lmx_host_gemv(LMX_FMT_BINARY, blocks, num_blocks, activations, output, M, K), "lut_gemv_binary");
}
inline void int2_gemv(const void *blocks, size_t num_blocks, const float *activations, float *output, size_t M,
                      size_t K) {
  check_or_abort(lmx_host_gemv(LMX_FMT_RRQ2, blocks, num_blocks, activations, output, M, K), "int2_gemv");
}
inline void int3_gemv(const void *blocks, size_t num_blocks, const float *activations, float *output, size_t M,
                      size_t K) {
  check_or_abort(lmx_host_gemv(LMX_FMT_INT3, blocks, num_blocks, activations, output, M, K), "int3_gemv");
}
inline void int4_gemv(const void *blocks, size_t num_blocks, const float *activations, float *output, size_t M,
                      size_t K) {
  check_or_abort(lmx_host_gemv(LMX_FMT_INT4, blocks, num_blocks, activations, output, M, K), "int4_gemv");
}
inline void int8_gemv(const void *blocks, size_t num_blocks, const float *activations, float *output, size_t M,
                      size_t K) {
  check_or_abort(lmx_host_gemv(LMX_FMT_INT8, blocks, num_blocks, activations, output, M, K), "int8_gemv");
}
inline void apply_hadamard_rotation(float *data, size_t n) {
  check_or_abort(lmx_host_apply_hadamard_rotation(data, n), "apply_hadamard_rotation");
}
inline void fwht_256(float *data) { apply_hadamard_rotation(data, 256); }
inline void precompute_luts(const float *activations, size_t n, float *luts) {
  check_or_abort(lmx_host_precompute_luts(activations, n, luts), "precompute_luts");
}
inline void precompute_lut(const float *activations, float *lut) {
  check_or_abort(lmx_host_precompute_lut(activations, lut), "precompute_lut");
}
inline void extract_indices(const uint8_t *sign_plane, const uint8_t *zero_plane, size_t group_idx,
                            uint8_t &pos_idx, uint8_t &neg_idx) {
  check_or_abort(lmx_host_extract_indices(sign_plane, zero_plane, group_idx, &pos_idx, &neg_idx),
                 "extract_indices");
}

/* lut_linear over the reference's PackedTensor (or any type with the same
 * members): the format is chosen exactly as lut_gemm_scalar.cpp:115-156
 * does -- quant_bits together with the non-empty block vector, ternary
 * (`blocks`) otherwise.  5/6-bit and raw fp32 tensors are not on this path
 * and abort. */
template <class PackedTensorT>
inline void lut_linear(const PackedTensorT &w, const float *bias, const float *input, float *output,
                       size_t batch_size = 1) {
  if (w.shape.size() != 2) return;  // the reference returns silently (lut_gemm_scalar.cpp:70-71)
  const size_t M = w.shape[0], K = w.shape[1];
  int fmt = 0;
  const void *blocks = nullptr;
  size_t n = 0;
  if (!w.is_quantized) {
    check_or_abort(LMX_ERR_UNSUPPORTED_FORMAT, "lut_linear (raw fp32 weights)");
  } else if (w.quant_bits == 4 && !w.int4_blocks.empty()) {
    fmt = LMX_FMT_INT4, blocks = w.int4_blocks.data(), n = w.int4_blocks.size();
  } else if (w.quant_bits == 8 && !w.int8_blocks.empty()) {
    fmt = LMX_FMT_INT8, blocks = w.int8_blocks.data(), n = w.int8_blocks.size();
  } else if (w.quant_bits == 1 && !w.binary_blocks.empty()) {
    fmt = LMX_FMT_BINARY, blocks = w.binary_blocks.data(), n = w.binary_blocks.size();
  } else if (w.quant_bits == 2 && !w.int2_blocks.empty()) {
    fmt = LMX_FMT_RRQ2, blocks = w.int2_blocks.data(), n = w.int2_blocks.size();
  } else if (w.quant_bits == 3 && !w.int3_blocks.empty()) {
    fmt = LMX_FMT_INT3, blocks = w.int3_blocks.data(), n = w.int3_blocks.size();
  } else if ((w.quant_bits == 5 && !w.int5_blocks.empty()) || (w.quant_bits == 6 && !w.int6_blocks.empty())) {
    check_or_abort(LMX_ERR_UNSUPPORTED_FORMAT, "lut_linear (5/6-bit weights)");
  } else {
    fmt = LMX_FMT_TERNARY, blocks = w.blocks.data(), n = w.blocks.size();
  }
  check_or_abort(lmx_host_lut_linear(fmt, blocks, n, bias, input, output, M, K, batch_size), "lut_linear");
}

}  /* namespace lutmac_hip */
#endif /* __cplusplus */

#endif /* LUTMAC_HIP_COMPAT_H */
