/*
 * lutmac_synth.h -- producer-side helpers: 4-bit quantization of fp32
 * weights into canonical planes, and the seeded Gaussian weights the
 * benchmarks and tests quantize (BASELINE configs 4 and 5: N(0, 0.02)).
 *
 * Host-only; no GPU needed.  Both run row-parallel on up to 16 threads and
 * give the same bytes for any thread count.
 */
#ifndef LUTMAC_SYNTH_H
#define LUTMAC_SYNTH_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* fp32 w[rows][cols] -> canonical 4-bit planes [4][rows][cols/8] and scales
 * [rows][cols/group], the reference's 4-bit rule applied per `group`
 * weights (include/lutmac/quantize.hpp:437-461: scale = absmax/7, q =
 * round(w / scale) clamped to [-7, 7] or 0 when scale <= 1e-10, code q + 8),
 * evaluated as the reference's -ffast-math build does (absmax * (1/7),
 * w / scale), so the output is bit-identical to its quantize_tensor_int4.
 * group must be a multiple of 8 dividing cols. */
int lmx_quantize_int4(const float *w, size_t rows, size_t cols, size_t group,
                      uint8_t *planes, float *scales);

/* The same applied to seeded Gaussian weights N(0, stddev^2) without
 * materialising them: element (r, c) of matrix `stream` is a Box-Muller
 * normal drawn from a counter-based generator keyed by (seed, stream,
 * r*cols + c). */
int lmx_synth_int4_normal(uint64_t seed, uint64_t stream, size_t rows,
                          size_t cols, float stddev, size_t group,
                          uint8_t *planes, float *scales);
/* The Gaussian values themselves (fp32 w[rows][cols]), for checks. */
int lmx_synth_normal(uint64_t seed, uint64_t stream, size_t rows, size_t cols,
                     float stddev, float *w);

#ifdef __cplusplus
}
#endif
#endif /* LUTMAC_SYNTH_H */
