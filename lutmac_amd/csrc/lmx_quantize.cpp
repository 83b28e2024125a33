// lmx_quantize.cpp -- the producer side (lutmac_synth.h lmx_quantize): fp32
// weights -> canonical planes + scales for every format the kernels run,
// per scale group of any multiple of 8 weights (the reference's rules use
// 256-weight blocks; group 256 reproduces them exactly).
//
// Rules (include/lutmac/quantize.hpp in the LutMac tree):
//   TERNARY  quantize_tensor, 2-D path (193-281): threshold t = mean |w| over
//            the whole tensor (double sum); weight 0 where |w| < t/2, else
//            its sign; group scale = mean of the |w| >= t (a float sum, as
//            the 2-D path keeps it), 1 when no weight reaches t.
//   BINARY   quantize_tensor_binary (725-823): bit = (w >= 0), group scale =
//            mean |w| over the group's valid weights (double sum).
//   RRQ2     quantize_tensor_int2 (918-975): s = absmax / 2, q = round(w / s)
//            clamped to [-2, 1], stored q + 2 as (stage-1 bit, stage-2 bit);
//            the reference never sets the stage-2 scale, so it is 0.  With
//            LMX_QUANT_RESIDUAL instead each stage binarises the residual
//            of the previous ones with the binary rule (real stage-2 scale).
//   RRQ3     residual binarisation over three stages (no reference rule).
//   INT3     quantize_tensor_int3 (982-1041): s = absmax / 4, q = round(w * (1/s))
//            clamped to [-4, 3] (0 when s <= 1e-10), code q + 4 over three
//            planes (bit p of the code in plane p).
//   INT4     quantize_tensor_int4 (437-461), as lmx_quantize_int4.
//   INT8     quantize_tensor_int8 (833-912) with Int8Block::set (types.hpp:441-460):
//            s = absmax * (1/127) (the -ffast-math build's form of absmax / 127),
//            q = round(clamp(w * (1/s), -127, 127)), all 0 when s == 0; the
//            code's two's-complement bits over eight planes.
// LMX_QUANT_ROTATE first applies the blockwise FWHT-256 to the weights, over
// the row-major tensor in whole 256-chunks (apply_hadamard_rotation on the
// tensor's data, as tools/lutmac-quantize.cpp:426-447 does for <= 2-bit
// formats; the activations of those formats are rotated by lut_linear, so
// (W H)(H x) = W x).  The butterflies are the scalar branch's, bit-exact.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <thread>
#include <vector>

#include "lmx_internal.hpp"
#include "lutmac_synth.h"

namespace {

using lmx::fail;

// transform_simd.cpp:14-23,26-45,94-97 (scalar branch): stages h = 1..128 of
// (a + b, a - b), then x 1/16.
void fwht256(float *d) {
  for (int h = 1; h < 256; h <<= 1)
    for (int i = 0; i < 256; i += 2 * h)
      for (int j = i; j < i + h; ++j) {
        const float a = d[j], b = d[j + h];
        d[j] = a + b;
        d[j + h] = a - b;
      }
  for (int i = 0; i < 256; ++i) d[i] *= 0.0625f;
}

void set_bit(uint8_t *plane_row, size_t k, bool on) {
  if (on) plane_row[k / 8] |= uint8_t(0x80u >> (k % 8));
}

// Per-row work spread over threads; rows are independent, so the output does
// not depend on the thread count.
template <class F>
void for_rows(size_t rows, F f) {
  const size_t nt = std::max<size_t>(1, std::min<size_t>(std::thread::hardware_concurrency(), (rows + 63) / 64));
  if (nt == 1) {
    for (size_t r = 0; r < rows; ++r) f(r);
    return;
  }
  std::vector<std::thread> th;
  for (size_t t = 0; t < nt; ++t)
    th.emplace_back([&, t] {
      for (size_t r = t; r < rows; r += nt) f(r);
    });
  for (auto &x : th) x.join();
}

// Binary stage of one group: bits (w >= 0) and scale mean |w| (double sum),
// quantize.hpp:773-793.  Returns the scale.
float binary_group(const float *v, size_t n, uint8_t *plane_row, size_t k0) {
  double sum_abs = 0.0;
  for (size_t i = 0; i < n; ++i) sum_abs += std::abs(v[i]);
  const float s = n ? static_cast<float>(sum_abs / double(n)) : 0.0f;
  for (size_t i = 0; i < n; ++i) set_bit(plane_row, k0 + i, v[i] >= 0.0f);
  return s;
}

// INT3 / INT8: one group's absmax scale and codes, the bits of each code
// spread over the format's planes (planes [P][rows][cols/8]).
int quantize_uniform(int format, const float *w, size_t rows, size_t cols, size_t G, uint8_t *planes,
                     float *scales) {
  const int P = format == LMX_FMT_INT3 ? 3 : 8;
  const size_t ng = cols / G, rb = cols / 8;
  std::memset(planes, 0, size_t(P) * rows * rb);
  for_rows(rows, [&](size_t r) {
    const float *v = w + r * cols;
    for (size_t g = 0; g < ng; ++g) {
      const size_t k0 = g * G;
      float absmax = 0.0f;
      for (size_t i = 0; i < G; ++i) absmax = std::max(absmax, std::abs(v[k0 + i]));
      float s;
      if (format == LMX_FMT_INT3) {
        s = absmax / 4.0f;
        const float inv = s > 1e-10f ? 1.0f / s : 0.0f;
        for (size_t i = 0; i < G; ++i) {
          int q = static_cast<int>(std::round(v[k0 + i] * inv));
          q = std::max(-4, std::min(3, q));
          const unsigned code = unsigned(q + 4);
          for (int p = 0; p < 3; ++p) set_bit(planes + (size_t(p) * rows + r) * rb, k0 + i, (code >> p) & 1u);
        }
      } else {
        s = absmax * (1.0f / 127.0f);
        if (s != 0.0f) {
          const float inv = 1.0f / s;
          for (size_t i = 0; i < G; ++i) {
            const float val = std::max(-127.0f, std::min(127.0f, v[k0 + i] * inv));
            const unsigned code = unsigned(uint8_t(int8_t(std::round(val))));
            for (int p = 0; p < 8; ++p) set_bit(planes + (size_t(p) * rows + r) * rb, k0 + i, (code >> p) & 1u);
          }
        }
      }
      scales[r * ng + g] = s;
    }
  });
  return LMX_OK;
}

}  // namespace

extern "C" int lmx_quantize(int format, const float *w, size_t rows, size_t cols, size_t group, unsigned flags,
                            uint8_t *planes, float *scales) {
  if (!w || !planes || !scales) return fail(LMX_ERR_INVALID_ARGUMENT, "NULL argument");
  if (rows == 0 || cols == 0 || cols % 8) return fail(LMX_ERR_INVALID_ARGUMENT, "cols must be a positive multiple of 8");
  if (flags & ~(LMX_QUANT_ROTATE | LMX_QUANT_RESIDUAL)) return fail(LMX_ERR_INVALID_ARGUMENT, "unknown flags 0x%x", flags);
  if (format == LMX_FMT_INT4) {
    if (flags) return fail(LMX_ERR_INVALID_ARGUMENT, "int4 takes no flags (the reference never rotates 4-bit)");
    if (group == 0 || group % 8 || cols % group)
      return fail(LMX_ERR_INVALID_ARGUMENT, "int4 group must be a multiple of 8 dividing cols");
    return lmx_quantize_int4(w, rows, cols, group, planes, scales);
  }
  if (format == LMX_FMT_INT3 || format == LMX_FMT_INT8) {
    if (flags) return fail(LMX_ERR_INVALID_ARGUMENT, "int3/int8 take no flags (the tool never rotates them)");
    if (group == 0 || group % 8 || cols % group)
      return fail(LMX_ERR_INVALID_ARGUMENT, "int3/int8 group must be a multiple of 8 dividing cols");
    return quantize_uniform(format, w, rows, cols, group, planes, scales);
  }
  if (format != LMX_FMT_TERNARY && format != LMX_FMT_BINARY && format != LMX_FMT_RRQ2 && format != LMX_FMT_RRQ3)
    return fail(LMX_ERR_UNSUPPORTED_FORMAT, "lmx_quantize: format %d (ternary, binary, rrq2, rrq3, int3, int4, int8)",
                format);
  if ((flags & LMX_QUANT_RESIDUAL) && format != LMX_FMT_RRQ2)
    return fail(LMX_ERR_INVALID_ARGUMENT, "LMX_QUANT_RESIDUAL applies to rrq2 (rrq3 is always residual)");
  if (group == 0 && format != LMX_FMT_TERNARY)
    return fail(LMX_ERR_INVALID_ARGUMENT, "one scale per row (group 0) is a ternary rule");
  const size_t G = group ? group : cols;
  if (G % 8) return fail(LMX_ERR_INVALID_ARGUMENT, "group %zu is not a multiple of 8", group);
  const size_t ng = (cols + G - 1) / G, rb = cols / 8;
  const int P = format == LMX_FMT_RRQ3 ? 3 : (format == LMX_FMT_BINARY ? 1 : 2);
  const int S = format == LMX_FMT_RRQ3 ? 3 : (format == LMX_FMT_RRQ2 ? 2 : 1);

  // Rotated copy (whole 256-chunks of the row-major tensor; a tail is left as is).
  std::vector<float> rot;
  const float *src = w;
  if (flags & LMX_QUANT_ROTATE) {
    try {
      rot.assign(w, w + rows * cols);
    } catch (const std::bad_alloc &) {
      return fail(LMX_ERR_OUT_OF_MEMORY, "rotated copy of %zu weights", rows * cols);
    }
    const size_t chunks = rows * cols / 256;
    for (size_t c = 0; c < chunks; ++c) fwht256(rot.data() + c * 256);
    src = rot.data();
  }
  std::memset(planes, 0, size_t(P) * rows * rb);

  if (format == LMX_FMT_TERNARY) {
    double abs_sum = 0.0;   // quantize.hpp:93-99 over the whole tensor
    for (size_t i = 0; i < rows * cols; ++i) abs_sum += std::abs(src[i]);
    const float thr = static_cast<float>(abs_sum / double(rows * cols));
    const float zero_below = 0.5f * thr;
    for_rows(rows, [&](size_t r) {
      const float *v = src + r * cols;
      uint8_t *sign = planes + r * rb, *zero = planes + (rows + r) * rb;
      for (size_t g = 0; g < ng; ++g) {
        const size_t k0 = g * G, n = std::min(G, cols - k0);
        size_t count = 0;
        for (size_t i = 0; i < n; ++i) {
          const float x = v[k0 + i];
          if (std::abs(x) < zero_below) {
            set_bit(zero, k0 + i, true);
          } else if (!(x > 0.0f)) {
            set_bit(sign, k0 + i, true);
          }
          count += std::abs(x) >= thr;
        }
        // The float sum of the |w| >= t in the order the reference's
        // (-O3 -ffast-math -mavx2) build evaluates it: per 32 weights, the
        // four 8-weight slices A..D of masked |w| are added lane-wise as
        // (A + B) + (C + D) into one 8-lane accumulator, whose lanes are
        // finally added as ((a0+a4)+(a2+a6)) + ((a1+a5)+(a3+a7)) -- the
        // reference's scales are reproduced bit for bit.  Weights past the
        // last whole 32 are added one by one after that.
        float acc[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
        auto m = [&](size_t i) { const float a = std::abs(v[k0 + i]); return a >= thr ? a : 0.0f; };
        const size_t n32 = n / 32 * 32;
        for (size_t t = 0; t < n32; t += 32)
          for (int j = 0; j < 8; ++j)
            acc[j] += (m(t + j) + m(t + 8 + j)) + (m(t + 16 + j) + m(t + 24 + j));
        float scale_sum = ((acc[0] + acc[4]) + (acc[2] + acc[6])) + ((acc[1] + acc[5]) + (acc[3] + acc[7]));
        for (size_t i = n32; i < n; ++i) scale_sum += m(i);
        scales[r * ng + g] = count > 0 ? scale_sum / float(count) : 1.0f;
      }
    });
    return LMX_OK;
  }
  if (format == LMX_FMT_RRQ2 && !(flags & LMX_QUANT_RESIDUAL)) {
    for_rows(rows, [&](size_t r) {
      const float *v = src + r * cols;
      uint8_t *b1 = planes + r * rb, *b2 = planes + (rows + r) * rb;
      for (size_t g = 0; g < ng; ++g) {
        const size_t k0 = g * G, n = std::min(G, cols - k0);
        float absmax = 0.0f;
        for (size_t i = 0; i < n; ++i) absmax = std::max(absmax, std::abs(v[k0 + i]));
        const float s = absmax / 2.0f;
        const float inv = s > 1e-10f ? 1.0f / s : 0.0f;
        for (size_t i = 0; i < n; ++i) {
          int q = static_cast<int>(std::round(v[k0 + i] * inv));
          q = std::max(-2, std::min(1, q));
          const unsigned uq = unsigned(q + 2);   // (stage-1 bit, stage-2 bit), types.hpp:236-241
          set_bit(b1, k0 + i, (uq >> 1) & 1u);
          set_bit(b2, k0 + i, uq & 1u);
        }
        scales[r * ng + g] = s;
        scales[(rows + r) * ng + g] = 0.0f;   // the reference leaves scale2 at 0 (quantize.hpp:951)
      }
    });
    return LMX_OK;
  }
  // BINARY, residual RRQ2, RRQ3: stage i binarises what the earlier stages left.
  for_rows(rows, [&](size_t r) {
    std::vector<float> res(src + r * cols, src + (r + 1) * cols);
    for (int st = 0; st < S; ++st) {
      uint8_t *row = planes + (size_t(st) * rows + r) * rb;
      for (size_t g = 0; g < ng; ++g) {
        const size_t k0 = g * G, n = std::min(G, cols - k0);
        const float s = binary_group(res.data() + k0, n, row, k0);
        scales[(size_t(st) * rows + r) * ng + g] = s;
        for (size_t i = 0; i < n; ++i) res[k0 + i] -= res[k0 + i] >= 0.0f ? s : -s;
      }
    }
  });
  return LMX_OK;
}
