// lmx_synth.cpp -- 4-bit producer and seeded Gaussian weights (lutmac_synth.h).
#include <algorithm>
#include <cmath>
#include <cstring>
#include <thread>
#include <vector>

#include "lmx_internal.hpp"
#include "lutmac_synth.h"

namespace {

// splitmix64 finaliser: a counter-based generator (one 64-bit draw per key).
inline uint64_t mix64(uint64_t z) {
  z += 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

// Normal pair number i of (seed, stream) by Box-Muller in double precision.
inline void normal_pair(uint64_t seed, uint64_t stream, uint64_t i, double *z0, double *z1) {
  const uint64_t key = mix64(seed ^ mix64(stream + 0x632BE59BD9B4E019ull));
  const uint64_t a = mix64(key ^ (2 * i)), b = mix64(key ^ (2 * i + 1));
  const double u1 = (double(a >> 11) + 1.0) * (1.0 / 9007199254740992.0);   // (0, 1]
  const double u2 = double(b >> 11) * (1.0 / 9007199254740992.0);           // [0, 1)
  const double r = std::sqrt(-2.0 * std::log(u1));
  *z0 = r * std::cos(6.283185307179586 * u2);
  *z1 = r * std::sin(6.283185307179586 * u2);
}

// Row of Gaussian values (cols even or odd; pairs are keyed by element index / 2).
void normal_row(uint64_t seed, uint64_t stream, size_t r, size_t cols, float stddev, float *out) {
  const uint64_t base = uint64_t(r) * cols;
  for (size_t c = 0; c < cols;) {
    const uint64_t idx = base + c;
    double z0, z1;
    normal_pair(seed, stream, idx / 2, &z0, &z1);
    if (idx % 2 == 0) {
      out[c++] = float(z0) * stddev;
      if (c < cols) out[c++] = float(z1) * stddev;
    } else {
      out[c++] = float(z1) * stddev;
    }
  }
}

// quantize.hpp:437-461 for one row, per `group` weights.
void quantize_row(const float *w, size_t r, size_t rows, size_t cols, size_t group, uint8_t *planes, float *scales) {
  const size_t rb = cols / 8, ng = cols / group;
  for (size_t g = 0; g < ng; ++g) {
    const float *v = w + g * group;
    float absmax = 0.0f;
    for (size_t i = 0; i < group; ++i) absmax = std::max(absmax, std::abs(v[i]));
    // The arithmetic of the reference's -ffast-math build of this rule:
    // absmax / 7 becomes absmax * (1/7), and w * (1 / scale) becomes
    // w / scale; the outputs are bit-identical to its quantize_tensor_int4.
    const float scale = absmax * (1.0f / 7.0f);
    const bool live = scale > 1e-10f;
    scales[r * ng + g] = scale;
    for (size_t i = 0; i < group; i += 8) {
      uint8_t b[4] = {0, 0, 0, 0};
      for (int j = 0; j < 8; ++j) {
        int q = live ? int(std::round(v[i + j] / scale)) : 0;
        q = std::max(-7, std::min(7, q));
        const unsigned u = unsigned(q + 8);
        for (int p = 0; p < 4; ++p) b[p] |= uint8_t(((u >> p) & 1u) << (7 - j));
      }
      const size_t byte = (g * group + i) / 8;
      for (int p = 0; p < 4; ++p) planes[(size_t(p) * rows + r) * rb + byte] = b[p];
    }
  }
}

template <class F>
void parallel_rows(size_t rows, F f) {
  const unsigned hw = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
  const size_t nt = std::min<size_t>(hw, std::max<size_t>(1, rows / 64));
  if (nt <= 1) {
    f(size_t(0), rows);
    return;
  }
  std::vector<std::thread> ts;
  const size_t per = (rows + nt - 1) / nt;
  for (size_t t = 0; t < nt; ++t) {
    const size_t a = t * per, b = std::min(rows, a + per);
    if (a < b) ts.emplace_back(f, a, b);
  }
  for (auto &t : ts) t.join();
}

int check_args(size_t rows, size_t cols, size_t group, const void *planes, const float *scales) {
  if (!planes || !scales) return lmx::fail(LMX_ERR_INVALID_ARGUMENT, "NULL output");
  if (!rows || !cols || !group || group % 8 || cols % group)
    return lmx::fail(LMX_ERR_INVALID_ARGUMENT, "group %zu must be a multiple of 8 dividing cols %zu", group, cols);
  return LMX_OK;
}

}  // namespace

extern "C" {

int lmx_quantize_int4(const float *w, size_t rows, size_t cols, size_t group, uint8_t *planes, float *scales) {
  int st = check_args(rows, cols, group, planes, scales);
  if (st) return st;
  if (!w) return lmx::fail(LMX_ERR_INVALID_ARGUMENT, "NULL weights");
  parallel_rows(rows, [&](size_t a, size_t b) {
    for (size_t r = a; r < b; ++r) quantize_row(w + r * cols, r, rows, cols, group, planes, scales);
  });
  return LMX_OK;
}

int lmx_synth_int4_normal(uint64_t seed, uint64_t stream, size_t rows, size_t cols, float stddev, size_t group,
                          uint8_t *planes, float *scales) {
  int st = check_args(rows, cols, group, planes, scales);
  if (st) return st;
  parallel_rows(rows, [&](size_t a, size_t b) {
    std::vector<float> row(cols);
    for (size_t r = a; r < b; ++r) {
      normal_row(seed, stream, r, cols, stddev, row.data());
      quantize_row(row.data(), r, rows, cols, group, planes, scales);
    }
  });
  return LMX_OK;
}

int lmx_synth_normal(uint64_t seed, uint64_t stream, size_t rows, size_t cols, float stddev, float *w) {
  if (!w || !rows || !cols) return lmx::fail(LMX_ERR_INVALID_ARGUMENT, "bad arguments");
  parallel_rows(rows, [&](size_t a, size_t b) {
    for (size_t r = a; r < b; ++r) normal_row(seed, stream, r, cols, stddev, w + r * cols);
  });
  return LMX_OK;
}

}  // extern "C"
