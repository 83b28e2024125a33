/*
 * lutmac_oracle.c -- CPU restatement of LutMac's bit-serial LUT-GEMV path.
 *
 * TEST INFRASTRUCTURE ONLY (the parity checker and the "port" CPU baseline);
 * the product path never links or loads it.  Written from the reference's
 * documented semantics; each function cites the reference file:line it
 * restates.  Built with plain -O2 (no -ffast-math) so that its own summation
 * order is the literal k order.
 */
#include "lutmac_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

int orc_format_planes(int fmt) {
  switch (fmt) {
  case ORC_FMT_TERNARY: return 2;
  case ORC_FMT_BINARY: return 1;
  case ORC_FMT_RRQ2: return 2;
  case ORC_FMT_RRQ3: return 3;
  case ORC_FMT_INT3: return 3;
  case ORC_FMT_INT4: return 4;
  case ORC_FMT_INT8: return 8;
  default: return 0;
  }
}

int orc_format_stages(int fmt) {
  if (fmt == ORC_FMT_RRQ2) return 2;
  if (fmt == ORC_FMT_RRQ3) return 3;
  return orc_format_planes(fmt) ? 1 : 0;
}

size_t orc_block_bytes(int fmt) {
  switch (fmt) {
  case ORC_FMT_TERNARY: return 68;
  case ORC_FMT_BINARY: return 36;
  case ORC_FMT_RRQ2: return 72;
  case ORC_FMT_INT3: return 100;
  case ORC_FMT_INT4: return 132;
  case ORC_FMT_INT8: return 260;
  default: return 0;
  }
}

static float rd_f32(const uint8_t *p) {
  float f;
  memcpy(&f, p, 4);
  return f;
}

/* ---- tables and indices --------------------------------------------------*/

/* lut_gemm.hpp:30-44: entry m sums a_j for each set bit (3-j) of m, adding in
 * the order a0, a1, a2, a3 to a running sum that starts at +0. */
void orc_precompute_lut(const float *a, float *lut) {
  lut[0] = 0.0f;
  for (int i = 1; i < 16; ++i) {
    float sum = 0.0f;
    if (i & 8) sum += a[0];
    if (i & 4) sum += a[1];
    if (i & 2) sum += a[2];
    if (i & 1) sum += a[3];
    lut[i] = sum;
  }
}

/* lut_gemm.hpp:53-58 */
void orc_precompute_luts(const float *x, size_t n, float *luts) {
  for (size_t g = 0; g < n / 4; ++g) orc_precompute_lut(x + 4 * g, luts + 16 * g);
}

/* lut_gemm.hpp:79-99: group g lives in byte g/2, high nibble for even g. */
void orc_extract_indices(const uint8_t *sign_plane, const uint8_t *zero_plane,
                         size_t group_idx, uint8_t *pos_idx, uint8_t *neg_idx) {
  size_t byte_idx = group_idx / 2;
  unsigned shift = 4u - (unsigned)(group_idx % 2) * 4u;
  uint8_t s = (uint8_t)((sign_plane[byte_idx] >> shift) & 0x0F);
  uint8_t z = (uint8_t)((zero_plane[byte_idx] >> shift) & 0x0F);
  uint8_t nz = (uint8_t)(~z & 0x0F);
  *pos_idx = (uint8_t)(nz & (uint8_t)~s);
  *neg_idx = (uint8_t)(nz & s);
}

/* ---- Walsh-Hadamard ------------------------------------------------------*/

/* transform_simd.cpp:14-23 (stride h butterflies over one 256-chunk) */
static void fwht_pass(float *d, size_t h) {
  for (size_t i = 0; i < 256; i += 2 * h)
    for (size_t j = i; j < i + h; ++j) {
      float x = d[j], y = d[j + h];
      d[j] = x + y;
      d[j + h] = x - y;
    }
}

/* transform_simd.cpp:26-99, scalar branch (56-63, 94-97): strides 1..128 in
 * increasing order, then x (1/16).  The AVX2 branch (46-55) is not followed:
 * it skips half of every stride>=4 stage and writes past the chunk. */
void orc_fwht_256(float *data) {
  for (size_t h = 1; h < 256; h <<= 1) fwht_pass(data, h);
  for (size_t i = 0; i < 256; ++i) data[i] *= (1.0f / 16.0f);
}

/* transform_simd.cpp:101-110: whole 256-chunks only. */
void orc_apply_hadamard_rotation(float *data, size_t n) {
  for (size_t i = 0; i + 256 <= n; i += 256) orc_fwht_256(data + i);
}

void orc_fwht_full(float *data, size_t n) {
  for (size_t h = 1; h < n; h <<= 1)
    for (size_t i = 0; i < n; i += 2 * h)
      for (size_t j = i; j < i + h; ++j) {
        float x = data[j], y = data[j + h];
        data[j] = x + y;
        data[j + h] = x - y;
      }
  float s = (float)(1.0 / sqrt((double)n));
  for (size_t i = 0; i < n; ++i) data[i] *= s;
}

/* ---- ternary bit-plane packing -------------------------------------------*/

/* quantize.hpp:135-154 */
void orc_pack_to_bitplanes(const int8_t *t, size_t n, uint8_t *sign_plane,
                           uint8_t *zero_plane) {
  for (size_t i = 0; i < n; i += 8) {
    uint8_t sb = 0, zb = 0;
    for (size_t j = 0; j < 8 && i + j < n; ++j) {
      if (t[i + j] < 0) sb |= (uint8_t)(1u << (7 - j));
      if (t[i + j] == 0) zb |= (uint8_t)(1u << (7 - j));
    }
    sign_plane[i / 8] = sb;
    zero_plane[i / 8] = zb;
  }
}

/* quantize.hpp:158-180 */
void orc_unpack_from_bitplanes(const uint8_t *sign_plane,
                               const uint8_t *zero_plane, size_t n, int8_t *t) {
  for (size_t i = 0; i < n; i += 8)
    for (size_t j = 0; j < 8 && i + j < n; ++j) {
      int neg = (sign_plane[i / 8] >> (7 - j)) & 1;
      int zero = (zero_plane[i / 8] >> (7 - j)) & 1;
      t[i + j] = (int8_t)(zero ? 0 : (neg ? -1 : 1));
    }
}

/* ---- scalar GEMVs over reference AoS blocks ------------------------------*/

static size_t blocks_per_row(size_t K) { return (K + 255) / 256; }

/* lut_gemm_scalar.cpp:7-61 */
void orc_ternary_gemv(const uint8_t *blocks, const float *x, float *y, size_t M,
                      size_t K) {
  size_t bpr = blocks_per_row(K);
  for (size_t r = 0; r < M; ++r) {
    float acc = 0.0f;
    for (size_t b = 0; b < bpr; ++b) {
      const uint8_t *blk = blocks + (r * bpr + b) * 68;
      const float *xb = x + b * 256;
      float bs = 0.0f;
      for (size_t i = 0; i < 32; ++i)
        for (int j = 0; j < 8; ++j) {
          int bit = 7 - j;
          int z = (blk[32 + i] >> bit) & 1, s = (blk[i] >> bit) & 1;
          if (!z) {
            if (s) bs -= xb[i * 8 + j];
            else bs += xb[i * 8 + j];
          }
        }
      acc += bs * rd_f32(blk + 64);
    }
    y[r] = acc;
  }
}

/* lut_gemm_scalar.cpp:228-259 (row-parallel in the reference; the per-row
 * arithmetic is what is restated here) */
void orc_binary_gemv(const uint8_t *blocks, const float *x, float *y, size_t M,
                     size_t K) {
  size_t bpr = blocks_per_row(K);
  for (size_t r = 0; r < M; ++r) {
    float acc = 0.0f;
    for (size_t b = 0; b < bpr; ++b) {
      const uint8_t *blk = blocks + (r * bpr + b) * 36;
      const float *xb = x + b * 256;
      float bs = 0.0f;
      for (size_t i = 0; i < 32; ++i)
        for (int j = 0; j < 8; ++j) {
          int bit = (blk[i] >> (7 - j)) & 1;
          float v = xb[i * 8 + j];
          bs += bit ? v : -v;
        }
      acc += bs * rd_f32(blk + 32);
    }
    y[r] = acc;
  }
}

/* lut_gemm_scalar.cpp:186-222; even index in the high nibble (types.hpp:184-191) */
void orc_int4_gemv(const uint8_t *blocks, const float *x, float *y, size_t M,
                   size_t K) {
  size_t bpr = blocks_per_row(K);
  for (size_t r = 0; r < M; ++r) {
    float acc = 0.0f;
    for (size_t b = 0; b < bpr; ++b) {
      const uint8_t *blk = blocks + (r * bpr + b) * 132;
      const float *xb = x + b * 256;
      float bs = 0.0f;
      for (size_t i = 0; i < 256; ++i) {
        uint8_t byte = blk[i / 2];
        int nib = (i % 2 == 0) ? (byte >> 4) : (byte & 0x0F);
        bs += (float)(nib - 8) * xb[i];
      }
      acc += bs * rd_f32(blk + 128);
    }
    y[r] = acc;
  }
}

/* types.hpp:217-234: 2-bit field i at bits (7-2(i%4))..(6-2(i%4)) of byte i/4;
 * field bit 1 = primary sign, bit 0 = residual sign. */
static float int2_get(const uint8_t *blk, size_t i) {
  uint8_t v = (uint8_t)((blk[i / 4] >> (6 - (i % 4) * 2)) & 3);
  float s1 = rd_f32(blk + 64), s2 = rd_f32(blk + 68);
  float v1 = (v >> 1) ? s1 : -s1;
  float v2 = (v & 1) ? s2 : -s2;
  return v1 + v2;
}

/* lut_gemm_scalar.cpp:298-321 */
void orc_int2_gemv(const uint8_t *blocks, const float *x, float *y, size_t M,
                   size_t K) {
  size_t bpr = blocks_per_row(K);
  for (size_t r = 0; r < M; ++r) {
    float acc = 0.0f;
    for (size_t b = 0; b < bpr; ++b) {
      const uint8_t *blk = blocks + (r * bpr + b) * 72;
      const float *xb = x + b * 256;
      float s = rd_f32(blk + 64), bs = 0.0f;
      for (size_t i = 0; i < 256; ++i) bs += int2_get(blk, i) * xb[i] / s;
      acc += bs * s;
    }
    y[r] = acc;
  }
}

/* types.hpp:256-268: 3-bit big-endian stream, q at bits [3i, 3i+3). */
static int int3_q(const uint8_t *blk, size_t i) {
  size_t bit = i * 3, byte = bit / 8, off = bit % 8;
  unsigned w = (unsigned)blk[byte] << 8;
  if (byte + 1 < 96) w |= blk[byte + 1];
  return (int)((w >> (13 - off)) & 7);
}

/* lut_gemm_scalar.cpp:327-350 */
void orc_int3_gemv(const uint8_t *blocks, const float *x, float *y, size_t M,
                   size_t K) {
  size_t bpr = blocks_per_row(K);
  for (size_t r = 0; r < M; ++r) {
    float acc = 0.0f;
    for (size_t b = 0; b < bpr; ++b) {
      const uint8_t *blk = blocks + (r * bpr + b) * 100;
      const float *xb = x + b * 256;
      float s = rd_f32(blk + 96), bs = 0.0f;
      for (size_t i = 0; i < 256; ++i)
        bs += ((float)(int3_q(blk, i) - 4) * s) * xb[i] / s;
      acc += bs * s;
    }
    y[r] = acc;
  }
}

/* lut_gemm_scalar.cpp:265-292; scale first, then int8[256] (types.hpp:434-465) */
void orc_int8_gemv(const uint8_t *blocks, const float *x, float *y, size_t M,
                   size_t K) {
  size_t bpr = blocks_per_row(K);
  for (size_t r = 0; r < M; ++r) {
    float acc = 0.0f;
    for (size_t b = 0; b < bpr; ++b) {
      const uint8_t *blk = blocks + (r * bpr + b) * 260;
      const float *xb = x + b * 256;
      float bs = 0.0f;
      for (size_t i = 0; i < 256; ++i) bs += (float)(int8_t)blk[4 + i] * xb[i];
      acc += bs * rd_f32(blk);
    }
    y[r] = acc;
  }
}

/* lut_gemm_scalar.cpp:68-180 */
int orc_lut_linear(int fmt, const uint8_t *blocks, const float *bias,
                   const float *x, float *y, size_t M, size_t K, size_t batch) {
  size_t Ka = blocks_per_row(K) * 256;
  /* lut_gemm_scalar.cpp:92-93: rotate for quant_bits 1..2 or ternary blocks */
  int rotate = (fmt == ORC_FMT_TERNARY || fmt == ORC_FMT_BINARY || fmt == ORC_FMT_RRQ2);
  if (!(fmt == ORC_FMT_TERNARY || fmt == ORC_FMT_BINARY || fmt == ORC_FMT_RRQ2 ||
        fmt == ORC_FMT_INT3 || fmt == ORC_FMT_INT4 || fmt == ORC_FMT_INT8))
    return -1;
  float *buf = (float *)malloc(Ka * sizeof(float));
  if (!buf) return -1;
  for (size_t b = 0; b < batch; ++b) {
    memcpy(buf, x + b * K, K * sizeof(float));
    memset(buf + K, 0, (Ka - K) * sizeof(float));
    if (rotate) orc_apply_hadamard_rotation(buf, Ka);
    float *yo = y + b * M;
    switch (fmt) {
    case ORC_FMT_TERNARY: orc_ternary_gemv(blocks, buf, yo, M, K); break;
    case ORC_FMT_BINARY: orc_binary_gemv(blocks, buf, yo, M, K); break;
    case ORC_FMT_RRQ2: orc_int2_gemv(blocks, buf, yo, M, K); break;
    case ORC_FMT_INT3: orc_int3_gemv(blocks, buf, yo, M, K); break;
    case ORC_FMT_INT4: orc_int4_gemv(blocks, buf, yo, M, K); break;
    case ORC_FMT_INT8: orc_int8_gemv(blocks, buf, yo, M, K); break;
    }
    if (bias)
      for (size_t i = 0; i < M; ++i) yo[i] += bias[i];
  }
  free(buf);
  return 0;
}

/* ---- AoS blocks -> canonical planes --------------------------------------*/

static void set_plane_bit(uint8_t *planes, size_t M, size_t Kp, int p, size_t r,
                          size_t k, int bit) {
  uint8_t *byte = planes + ((size_t)p * M + r) * (Kp / 8) + k / 8;
  uint8_t m = (uint8_t)(1u << (7 - k % 8));
  if (bit) *byte |= m;
  else *byte &= (uint8_t)~m;
}

static int get_plane_bit(const uint8_t *planes, size_t M, size_t Kp, int p,
                         size_t r, size_t k) {
  return (planes[((size_t)p * M + r) * (Kp / 8) + k / 8] >> (7 - k % 8)) & 1;
}

int orc_blocks_to_planes(int fmt, const uint8_t *blocks, size_t M, size_t K,
                         uint8_t *planes, float *scales) {
  size_t bpr = blocks_per_row(K), Kp = bpr * 256, bb = orc_block_bytes(fmt);
  int P = orc_format_planes(fmt);
  if (!bb || !P) return -1;
  memset(planes, 0, (size_t)P * M * (Kp / 8));
  for (size_t r = 0; r < M; ++r)
    for (size_t b = 0; b < bpr; ++b) {
      const uint8_t *blk = blocks + (r * bpr + b) * bb;
      size_t gi = r * bpr + b, stride = M * bpr;
      for (size_t i = 0; i < 256; ++i) {
        size_t k = b * 256 + i;
        switch (fmt) {
        case ORC_FMT_TERNARY: /* types.hpp:140-149 */
          set_plane_bit(planes, M, Kp, 0, r, k, (blk[i / 8] >> (7 - i % 8)) & 1);
          set_plane_bit(planes, M, Kp, 1, r, k, (blk[32 + i / 8] >> (7 - i % 8)) & 1);
          break;
        case ORC_FMT_BINARY: /* types.hpp:404-411 */
          set_plane_bit(planes, M, Kp, 0, r, k, (blk[i / 8] >> (7 - i % 8)) & 1);
          break;
        case ORC_FMT_RRQ2: { /* types.hpp:217-234 */
          int v = (blk[i / 4] >> (6 - (i % 4) * 2)) & 3;
          set_plane_bit(planes, M, Kp, 0, r, k, v >> 1);
          set_plane_bit(planes, M, Kp, 1, r, k, v & 1);
          break;
        }
        case ORC_FMT_INT3: { /* types.hpp:256-268 */
          int q = int3_q(blk, i);
          for (int p = 0; p < 3; ++p) set_plane_bit(planes, M, Kp, p, r, k, (q >> p) & 1);
          break;
        }
        case ORC_FMT_INT4: { /* types.hpp:184-191 */
          int q = (i % 2 == 0) ? (blk[i / 2] >> 4) : (blk[i / 2] & 0x0F);
          for (int p = 0; p < 4; ++p) set_plane_bit(planes, M, Kp, p, r, k, (q >> p) & 1);
          break;
        }
        case ORC_FMT_INT8: { /* types.hpp:464 */
          int q = blk[4 + i];
          for (int p = 0; p < 8; ++p) set_plane_bit(planes, M, Kp, p, r, k, (q >> p) & 1);
          break;
        }
        }
      }
      switch (fmt) {
      case ORC_FMT_TERNARY: scales[gi] = rd_f32(blk + 64); break;
      case ORC_FMT_BINARY: scales[gi] = rd_f32(blk + 32); break;
      case ORC_FMT_RRQ2:
        scales[gi] = rd_f32(blk + 64);
        scales[stride + gi] = rd_f32(blk + 68);
        break;
      case ORC_FMT_INT3: scales[gi] = rd_f32(blk + 96); break;
      case ORC_FMT_INT4: scales[gi] = rd_f32(blk + 128); break;
      case ORC_FMT_INT8: scales[gi] = rd_f32(blk); break;
      }
    }
  return 0;
}

int orc_plane_value(int fmt, const uint8_t *planes, size_t M, size_t Kp,
                    size_t r, size_t k, int stage) {
  int q = 0;
  switch (fmt) {
  case ORC_FMT_TERNARY:
    if (get_plane_bit(planes, M, Kp, 1, r, k)) return 0;
    return get_plane_bit(planes, M, Kp, 0, r, k) ? -1 : 1;
  case ORC_FMT_BINARY:
    return get_plane_bit(planes, M, Kp, 0, r, k) ? 1 : -1;
  case ORC_FMT_RRQ2:
  case ORC_FMT_RRQ3:
    return get_plane_bit(planes, M, Kp, stage, r, k) ? 1 : -1;
  case ORC_FMT_INT3:
    for (int p = 0; p < 3; ++p) q |= get_plane_bit(planes, M, Kp, p, r, k) << p;
    return q - 4;
  case ORC_FMT_INT4:
    for (int p = 0; p < 4; ++p) q |= get_plane_bit(planes, M, Kp, p, r, k) << p;
    return q - 8;
  case ORC_FMT_INT8:
    for (int p = 0; p < 8; ++p) q |= get_plane_bit(planes, M, Kp, p, r, k) << p;
    return (int)(int8_t)(uint8_t)q;
  }
  return 0;
}

/* Integer values of the 8 weights of byte `byte` of row r (stage st). */
static void byte_values(int fmt, const uint8_t *planes, size_t M, size_t Kp,
                        size_t r, size_t byte, int st, int *v) {
  const size_t rb = Kp / 8;
  int P = orc_format_planes(fmt);
  uint8_t b[8];
  for (int p = 0; p < P; ++p) b[p] = planes[((size_t)p * M + r) * rb + byte];
  for (int j = 0; j < 8; ++j) {
    int bit = 7 - j, q = 0;
    switch (fmt) {
    case ORC_FMT_TERNARY:
      v[j] = ((b[1] >> bit) & 1) ? 0 : (((b[0] >> bit) & 1) ? -1 : 1);
      break;
    case ORC_FMT_BINARY:
      v[j] = ((b[0] >> bit) & 1) ? 1 : -1;
      break;
    case ORC_FMT_RRQ2:
    case ORC_FMT_RRQ3:
      v[j] = ((b[st] >> bit) & 1) ? 1 : -1;
      break;
    default:
      for (int p = 0; p < P; ++p) q |= ((b[p] >> bit) & 1) << p;
      v[j] = fmt == ORC_FMT_INT3 ? q - 4 : fmt == ORC_FMT_INT4 ? q - 8 : (int)(int8_t)(uint8_t)q;
    }
  }
}

void orc_planes_gemv(int fmt, const uint8_t *planes, const float *scales,
                     size_t M, size_t Kp, size_t G, const float *x, float *y) {
  int S = orc_format_stages(fmt);
  size_t ng = Kp / G;
  /* rows are independent: spread over threads, each row's sum unchanged */
#pragma omp parallel for schedule(static)
  for (size_t r = 0; r < M; ++r) {
    int v[8];
    float acc = 0.0f;
    for (int st = 0; st < S; ++st) {
      const float *sc = scales + ((size_t)st * M + r) * ng;
      for (size_t g = 0; g < ng; ++g) {
        float gs = 0.0f;
        for (size_t byte = g * G / 8; byte < (g + 1) * G / 8; ++byte) {
          byte_values(fmt, planes, M, Kp, r, byte, st, v);
          for (int j = 0; j < 8; ++j) gs += (float)v[j] * x[byte * 8 + j];
        }
        acc += gs * sc[g];
      }
    }
    y[r] = acc;
  }
}

/* ---- decoder forward (src/model.cpp:47-453) ------------------------------ */

/* src/layers/norm.cpp:18-34 */
static void rms_norm(const float *in, const float *w, float *out, size_t n, float eps) {
  float ss = 0.0f;
  for (size_t i = 0; i < n; ++i) ss += in[i] * in[i];
  float rms = sqrtf(ss / (float)n + eps);
  float inv = 1.0f / rms;
  for (size_t i = 0; i < n; ++i) out[i] = in[i] * inv * w[i];
}

/* Frequencies of the rotary embedding: theta^(-2d/hd) as
 * src/layers/embedding.cpp:46 computes it, or with the published Llama-3
 * frequency scaling (computed in double, rounded to float). */
static float rope_freq(const orc_model *m, size_t d) {
  size_t hd = m->head_dim;
  if (m->rope_mode == 0) return 1.0f / powf(m->rope_theta, (2.0f * (float)d) / (float)hd);
  double inv = 1.0 / pow((double)m->rope_theta, 2.0 * (double)d / (double)hd);
  double lo_wl = (double)m->rope_orig_max_pos / m->rope_low_freq_factor;
  double hi_wl = (double)m->rope_orig_max_pos / m->rope_high_freq_factor;
  double wl = 2.0 * 3.14159265358979323846 / inv;
  if (wl < hi_wl) return (float)inv;
  if (wl > lo_wl) return (float)(inv / m->rope_factor);
  double sm = ((double)m->rope_orig_max_pos / wl - m->rope_low_freq_factor) /
              (m->rope_high_freq_factor - m->rope_low_freq_factor);
  return (float)((1.0 - sm) * inv / m->rope_factor + sm * inv);
}

void orc_rope_freqs(const orc_model *m, float *out) {
  for (size_t d = 0; d < m->head_dim / 2; ++d) out[d] = rope_freq(m, d);
}

/* src/layers/embedding.cpp:36-75 (rotate-half pairs d, d + hd/2) */
static void rope(const orc_model *m, float *v, size_t n_heads, size_t pos) {
  size_t hd = m->head_dim, half = hd / 2;
  float pf = m->rope_mode == 0 ? (float)pos / m->rope_factor : (float)pos;
  for (size_t h = 0; h < n_heads; ++h) {
    float *x = v + h * hd;
    for (size_t d = 0; d < half; ++d) {
      float angle = pf * rope_freq(m, d);
      float c = cosf(angle), s = sinf(angle);
      float a = x[d], b = x[d + half];
      x[d] = a * c - b * s;
      x[d + half] = a * s + b * c;
    }
  }
}

/* lut_linear's rotation rule (lut_gemm_scalar.cpp:88-96): activations of
 * ternary and 1-2 bit weights (binary, RRQ-2, RRQ-3) are FWHT-256-rotated,
 * in a copy, before the GEMV; cols is a multiple of 256 here. */
static void linear(const orc_matrix *w, const float *x, float *y) {
  const int rot = w->fmt == ORC_FMT_TERNARY || w->fmt == ORC_FMT_BINARY || w->fmt == ORC_FMT_RRQ2 ||
                  w->fmt == ORC_FMT_RRQ3;
  if (!rot) {
    orc_planes_gemv(w->fmt, w->planes, w->scales, w->rows, w->cols, w->group, x, y);
    return;
  }
  float *xr = malloc(w->cols * sizeof(float));
  if (!xr) return;
  memcpy(xr, x, w->cols * sizeof(float));
  orc_apply_hadamard_rotation(xr, w->cols);
  orc_planes_gemv(w->fmt, w->planes, w->scales, w->rows, w->cols, w->group, xr, y);
  free(xr);
}

static float silu(float x) { return x / (1.0f + expf(-x)); } /* model.cpp:36 */

int orc_decode_step(const orc_model *m, int token, size_t pos, float *logits) {
  const size_t h = m->hidden, nh = m->n_heads, nkv = m->n_kv_heads, hd = m->head_dim;
  const size_t qd = nh * hd, kvd = nkv * hd, ffn = m->ffn;
  if (pos >= m->max_seq || token < 0 || (size_t)token >= m->vocab) return -1;
  float *hs = malloc(h * 4), *nrm = malloc(h * 4), *qkv = malloc((qd + 2 * kvd) * 4);
  float *att = malloc(qd * 4), *tmp = malloc(h * 4), *gu = malloc(2 * ffn * 4);
  float *inter = malloc(ffn * 4), *wall = malloc(nh * (pos + 1) * 4);
  if (!hs || !nrm || !qkv || !att || !tmp || !gu || !inter || !wall) return -2;

  /* embedding row (model.cpp:58-85, per-group scales of the tied table) */
  {
    const orc_matrix *e = &m->head;
    size_t ng = e->cols / e->group;
    int v[8];
    for (size_t byte = 0; byte < h / 8; ++byte) {
      byte_values(e->fmt, e->planes, e->rows, e->cols, (size_t)token, byte, 0, v);
      for (int j = 0; j < 8; ++j) {
        size_t k = byte * 8 + j;
        hs[k] = (float)v[j] * e->scales[(size_t)token * ng + k / e->group];
      }
    }
  }
  const float scale = 1.0f / sqrtf((float)hd); /* model.cpp:337 */
  const size_t group = nh / nkv;
  for (size_t l = 0; l < m->n_layers; ++l) {
    float *kc = m->kcache + l * m->max_seq * kvd, *vc = m->vcache + l * m->max_seq * kvd;
    rms_norm(hs, m->in_norm + l * h, nrm, h, m->rms_eps);
    linear(&m->qkv[l], nrm, qkv);
    if (m->qkv_bias)
      for (size_t j = 0; j < qd + 2 * kvd; ++j) qkv[j] += m->qkv_bias[l * (qd + 2 * kvd) + j];
    rope(m, qkv, nh, pos);
    rope(m, qkv + qd, nkv, pos);
    memcpy(kc + pos * kvd, qkv + qd, kvd * 4);
    memcpy(vc + pos * kvd, qkv + qd + kvd, kvd * 4);
    memset(att, 0, qd * 4);
    /* heads are independent (own score row w[hh], own output slice) */
#pragma omp parallel for schedule(static)
    for (size_t hh = 0; hh < nh; ++hh) { /* model.cpp:341-372 */
      float *w = wall + hh * (pos + 1);
      size_t kvh = hh / group;
      const float *q = qkv + hh * hd;
      for (size_t t = 0; t <= pos; ++t) {
        const float *k = kc + t * kvd + kvh * hd;
        float sc = 0.0f;
        for (size_t d = 0; d < hd; ++d) sc += q[d] * k[d];
        w[t] = sc * scale;
      }
      float mx = w[0], sum = 0.0f; /* attention.cpp:23-42 */
      for (size_t t = 1; t <= pos; ++t) mx = w[t] > mx ? w[t] : mx;
      for (size_t t = 0; t <= pos; ++t) { w[t] = expf(w[t] - mx); sum += w[t]; }
      float inv = 1.0f / sum;
      for (size_t t = 0; t <= pos; ++t) w[t] *= inv;
      float *o = att + hh * hd;
      for (size_t t = 0; t <= pos; ++t) {
        const float *v = vc + t * kvd + kvh * hd;
        for (size_t d = 0; d < hd; ++d) o[d] += w[t] * v[d];
      }
    }
    linear(&m->o[l], att, tmp);
    for (size_t j = 0; j < h; ++j) hs[j] += tmp[j];
    rms_norm(hs, m->post_norm + l * h, nrm, h, m->rms_eps);
    linear(&m->gate_up[l], nrm, gu);
    for (size_t j = 0; j < ffn; ++j) inter[j] = silu(gu[j]) * gu[ffn + j];
    linear(&m->down[l], inter, tmp);
    for (size_t j = 0; j < h; ++j) hs[j] += tmp[j];
  }
  rms_norm(hs, m->final_norm, nrm, h, m->rms_eps);
  linear(&m->head, nrm, logits);
  free(hs); free(nrm); free(qkv); free(att); free(tmp); free(gu); free(inter); free(wall);
  return 0;
}
