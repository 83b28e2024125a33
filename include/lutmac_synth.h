/*
 * lutmac_synth.h -- producer-side helpers: quantization of fp32 weights
 * into canonical planes for every kernel format (ternary, binary, 2-bit,
 * RRQ-3, 4-bit; optional weight FWHT), and the seeded Gaussian weights the
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

/* lmx_quantize flags. */
/* FWHT-256 of the weights first, over the row-major tensor in whole
 * 256-chunks, as tools/lutmac-quantize.cpp:426-447 does for <= 2-bit formats
 * (lut_linear rotates those formats' activations, so (W H)(H x) = W x). */
#define LMX_QUANT_ROTATE 1u
/* RRQ2: binarise the residual of stage 1 again (a real stage-2 scale)
 * instead of the reference's quantize_tensor_int2 rule, whose stage-2 scale
 * is always 0 (quantize.hpp:951). */
#define LMX_QUANT_RESIDUAL 2u

/* fp32 w[rows][cols] -> canonical planes [P][rows][cols/8] and scales
 * [S][rows][ceil(cols/group)] (the lmx_planes_desc layout) with the
 * reference's rules per `group` weights (a multiple of 8; 0 = one scale per
 * row, ternary only):
 *   TERNARY  quantize_tensor's 2-D rule (quantize.hpp:193-281): threshold t =
 *            mean |w| of the whole tensor, 0 where |w| < t/2, else the sign;
 *            scale = mean of the |w| >= t (1 when none);
 *   BINARY   quantize_tensor_binary (725-823): sign bit, scale = mean |w|;
 *   RRQ2     quantize_tensor_int2 (918-975): s = absmax/2, q = round(w/s) in
 *            [-2, 1] stored as (stage-1, stage-2) bits of q + 2, stage-2
 *            scale 0; with LMX_QUANT_RESIDUAL two residual binary stages;
 *   RRQ3     three residual binary stages (no reference rule);
 *   INT3     quantize_tensor_int3 (982-1041): s = absmax/4, q = round(w/s)
 *            in [-4, 3] (0 when s <= 1e-10), code q + 4 (no flags);
 *   INT4     lmx_quantize_int4 (no flags);
 *   INT8     quantize_tensor_int8 / Int8Block::set (833-912, types.hpp:441-460):
 *            s = absmax/127, q = round(w/s) in [-127, 127] (all 0 when s == 0),
 *            two's-complement code (no flags).
 * INT3, INT4 and INT8 need a group (a multiple of 8) dividing cols.  At
 * group 256 the ternary, binary, 2-bit, 3-bit and 8-bit outputs, repacked
 * with lmx_planes_to_blocks, are byte-identical to the reference
 * quantizers' blocks for the same (optionally rotated) weights. */
int lmx_quantize(int format, const float *w, size_t rows, size_t cols,
                 size_t group, unsigned flags, uint8_t *planes, float *scales);

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
