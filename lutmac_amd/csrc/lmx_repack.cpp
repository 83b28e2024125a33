// lmx_repack.cpp -- host-side repack between LutMac's AoS weight blocks, the
// canonical bit-plane form and the device tile layout.
//
// The reference stores each 256-weight block as one struct (types.hpp:126-465).
// The GPU kernels want every bit-plane as its own stream, tiled so that one
// wavefront (64 rows) reads 64 x 16 contiguous bytes per plane per 128-k
// chunk.  The canonical plane form sits in between: plane p of row r is a
// byte string in the reference's MSB-first order (weight k at bit 7-(k%8) of
// byte k/8), so a plane byte is bit-identical to the reference's sign/zero/
// data bytes wherever the reference already stores planes.
#include <cstring>
#include <algorithm>
#include <vector>

#include "lmx_internal.hpp"

namespace lmx {

namespace {

float rd_f32(const uint8_t *p) {
  float f;
  std::memcpy(&f, p, 4);
  return f;
}
void wr_f32(uint8_t *p, float f) { std::memcpy(p, &f, 4); }

// Decode the per-weight field of one block into q[256] (integer formats) or
// the 2-bit RRQ field (Int2Block), following the accessors in types.hpp.
void decode_block(int fmt, const uint8_t *blk, uint8_t *q) {
  switch (fmt) {
  case LMX_FMT_RRQ2:  // types.hpp:217-234: field (b1<<1)|b2, MSB-first
    for (int i = 0; i < 256; ++i) q[i] = (blk[i / 4] >> (6 - 2 * (i % 4))) & 3;
    break;
  case LMX_FMT_INT3:  // types.hpp:256-268: 3-bit big-endian stream
    for (int i = 0; i < 256; ++i) {
      int bit = 3 * i, byte = bit / 8, off = bit % 8;
      unsigned w = unsigned(blk[byte]) << 8;
      if (byte + 1 < 96) w |= blk[byte + 1];
      q[i] = (w >> (13 - off)) & 7;
    }
    break;
  case LMX_FMT_INT4:  // types.hpp:184-191: even index in the high nibble
    for (int i = 0; i < 256; ++i) q[i] = (i % 2 == 0) ? (blk[i / 2] >> 4) : (blk[i / 2] & 15);
    break;
  case LMX_FMT_INT8:  // types.hpp:434-465: scale first, then int8[256]
    for (int i = 0; i < 256; ++i) q[i] = blk[4 + i];
    break;
  }
}

void encode_block(int fmt, const uint8_t *q, uint8_t *blk) {
  switch (fmt) {
  case LMX_FMT_RRQ2:
    std::memset(blk, 0, 64);
    for (int i = 0; i < 256; ++i) blk[i / 4] |= uint8_t((q[i] & 3) << (6 - 2 * (i % 4)));
    break;
  case LMX_FMT_INT3:
    std::memset(blk, 0, 96);
    for (int i = 0; i < 256; ++i) {
      int bit = 3 * i;
      for (int j = 0; j < 3; ++j, ++bit)
        if ((q[i] >> (2 - j)) & 1) blk[bit / 8] |= uint8_t(0x80u >> (bit % 8));
    }
    break;
  case LMX_FMT_INT4:
    for (int i = 0; i < 128; ++i) blk[i] = uint8_t((q[2 * i] << 4) | (q[2 * i + 1] & 15));
    break;
  case LMX_FMT_INT8:
    std::memcpy(blk + 4, q, 256);
    break;
  }
}

// Bit `plane` of q[8m..8m+7] gathered MSB-first into one byte.
inline uint8_t gather_plane_byte(const uint8_t *q8, int plane) {
  unsigned b = 0;
  for (int j = 0; j < 8; ++j) b |= ((q8[j] >> plane) & 1u) << (7 - j);
  return uint8_t(b);
}

// RRQ2 stores the primary sign in field bit 1 and the residual in bit 0;
// canonical plane 0 is the primary stage, plane 1 the residual.
inline int field_bit_of_plane(int fmt, int plane) {
  return fmt == LMX_FMT_RRQ2 ? 1 - plane : plane;
}

}  // namespace

bool format_info(int fmt, FormatInfo *fi) {
  switch (fmt) {
  case LMX_FMT_TERNARY: *fi = {2, 1, 68}; return true;
  case LMX_FMT_BINARY: *fi = {1, 1, 36}; return true;
  case LMX_FMT_RRQ2: *fi = {2, 2, 72}; return true;
  case LMX_FMT_RRQ3: *fi = {3, 3, 0}; return true;
  case LMX_FMT_INT3: *fi = {3, 1, 100}; return true;
  case LMX_FMT_INT4: *fi = {4, 1, 132}; return true;
  case LMX_FMT_INT8: *fi = {8, 1, 260}; return true;
  }
  return false;
}

int blocks_to_planes(int fmt, const uint8_t *blocks, size_t rows, size_t cols,
                     uint8_t *planes, float *scales) {
  FormatInfo fi;
  if (!format_info(fmt, &fi) || fi.block_bytes == 0)
    return fail(LMX_ERR_UNSUPPORTED_FORMAT, "format %d has no reference block layout", fmt);
  const size_t bpr = (cols + 255) / 256, row_bytes = bpr * 32;
  const size_t plane_stride = rows * row_bytes, stage_stride = rows * bpr;
  uint8_t q[256];
  for (size_t r = 0; r < rows; ++r) {
    for (size_t b = 0; b < bpr; ++b) {
      const uint8_t *blk = blocks + (r * bpr + b) * fi.block_bytes;
      uint8_t *dst = planes + r * row_bytes + b * 32;
      const size_t si = r * bpr + b;
      switch (fmt) {
      case LMX_FMT_TERNARY:  // sign[32], zero[32], scale (types.hpp:126-166)
        std::memcpy(dst, blk, 32);
        std::memcpy(dst + plane_stride, blk + 32, 32);
        scales[si] = rd_f32(blk + 64);
        break;
      case LMX_FMT_BINARY:  // data[32], scale (types.hpp:394-423)
        std::memcpy(dst, blk, 32);
        scales[si] = rd_f32(blk + 32);
        break;
      default: {
        decode_block(fmt, blk, q);
        for (int p = 0; p < fi.planes; ++p) {
          int fb = field_bit_of_plane(fmt, p);
          for (int m = 0; m < 32; ++m) dst[p * plane_stride + m] = gather_plane_byte(q + 8 * m, fb);
        }
        if (fmt == LMX_FMT_RRQ2) {
          scales[si] = rd_f32(blk + 64);
          scales[stage_stride + si] = rd_f32(blk + 68);
        } else if (fmt == LMX_FMT_INT8) {
          scales[si] = rd_f32(blk);
        } else {
          scales[si] = rd_f32(blk + (fmt == LMX_FMT_INT3 ? 96 : 128));
        }
      }
      }
    }
  }
  return LMX_OK;
}

int planes_to_blocks(int fmt, const uint8_t *planes, const float *scales,
                     size_t rows, size_t cols, uint8_t *blocks) {
  FormatInfo fi;
  if (!format_info(fmt, &fi) || fi.block_bytes == 0)
    return fail(LMX_ERR_UNSUPPORTED_FORMAT, "format %d has no reference block layout", fmt);
  const size_t bpr = (cols + 255) / 256, row_bytes = bpr * 32;
  const size_t plane_stride = rows * row_bytes, stage_stride = rows * bpr;
  uint8_t q[256];
  for (size_t r = 0; r < rows; ++r) {
    for (size_t b = 0; b < bpr; ++b) {
      uint8_t *blk = blocks + (r * bpr + b) * fi.block_bytes;
      const uint8_t *src = planes + r * row_bytes + b * 32;
      const size_t si = r * bpr + b;
      switch (fmt) {
      case LMX_FMT_TERNARY:
        std::memcpy(blk, src, 32);
        std::memcpy(blk + 32, src + plane_stride, 32);
        wr_f32(blk + 64, scales[si]);
        break;
      case LMX_FMT_BINARY:
        std::memcpy(blk, src, 32);
        wr_f32(blk + 32, scales[si]);
        break;
      default: {
        std::memset(q, 0, sizeof(q));
        for (int p = 0; p < fi.planes; ++p) {
          int fb = field_bit_of_plane(fmt, p);
          for (int i = 0; i < 256; ++i)
            q[i] |= uint8_t(((src[p * plane_stride + i / 8] >> (7 - i % 8)) & 1u) << fb);
        }
        encode_block(fmt, q, blk);
        if (fmt == LMX_FMT_RRQ2) {
          wr_f32(blk + 64, scales[si]);
          wr_f32(blk + 68, scales[stage_stride + si]);
        } else if (fmt == LMX_FMT_INT8) {
          wr_f32(blk, scales[si]);
        } else {
          wr_f32(blk + (fmt == LMX_FMT_INT3 ? 96 : 128), scales[si]);
        }
      }
      }
    }
  }
  return LMX_OK;
}

uint8_t pad_byte(int fmt, int plane) {
  // Columns past `cols` hold the code of the value 0 where the format has one
  // (ternary zero flag, int3 q=4, int4 q=8, int8 q=0), as the reference's
  // quantizers pad their last block (quantize.hpp:244-263,429-440).  Binary
  // and RRQ codes have no 0; their padding bits are 0.
  if ((fmt == LMX_FMT_TERNARY && plane == 1) || (fmt == LMX_FMT_INT3 && plane == 2) ||
      (fmt == LMX_FMT_INT4 && plane == 3))
    return 0xFF;
  return 0x00;
}

void nibble_tiles(const uint8_t *planes, size_t rows, size_t row_bytes, size_t Npad, size_t Kp, uint8_t *out) {
  const size_t Kc = Kp / kChunk;
  // spread[b]: the 8 bits of a plane byte (MSB first: k = 8m + j at bit 7 - j,
  // quantize.hpp:135-180) at bit 4j of a word of 8 nibbles
  static const std::vector<uint32_t> spread = [] {
    std::vector<uint32_t> t(256);
    for (unsigned b = 0; b < 256; ++b)
      for (int j = 0; j < 8; ++j) t[b] |= ((b >> (7 - j)) & 1u) << (4 * j);
    return t;
  }();
  std::vector<uint8_t> q(Kp);
  for (size_t r = 0; r < Npad; ++r) {
    // the row's codes q = sum_p bit_p << p, 8 (value 0) past the columns
    std::fill(q.begin(), q.end(), uint8_t(8));
    if (r < rows) {
      for (size_t m = 0; m < row_bytes; ++m) {
        uint32_t v = 0;
        for (int p = 0; p < 4; ++p) v |= spread[planes[(size_t(p) * rows + r) * row_bytes + m]] << p;
        for (int j = 0; j < 8; ++j) q[8 * m + j] = uint8_t((v >> (4 * j)) & 15u);
      }
    }
    for (size_t c = 0; c < Kc; ++c) {
      uint8_t *dst = out + (c * Npad + r) * 64;
      const uint8_t *qc = q.data() + c * kChunk;
      for (int kq = 0; kq < 4; ++kq)
        for (int kb = 0; kb < 8; ++kb)
          for (int b = 0; b < 2; ++b) {
            const int k = 16 * kb + 4 * kq + 2 * b;
            dst[kq * 16 + kb * 2 + b] = uint8_t(qc[k] | (qc[k + 1] << 4));
          }
    }
  }
}

void tile_planes(int fmt, const uint8_t *planes, size_t rows, size_t row_bytes,
                 size_t Npad, size_t Kp, uint8_t *tiles) {
  FormatInfo fi;
  format_info(fmt, &fi);
  const int P = fi.planes;
  const size_t Kc = Kp / kChunk;
  for (size_t c = 0; c < Kc; ++c) {
    const size_t off = c * 16;
    const size_t n = off >= row_bytes ? 0 : (row_bytes - off < 16 ? row_bytes - off : 16);
    for (int p = 0; p < P; ++p) {
      uint8_t *dst = tiles + ((c * P + p) * Npad) * 16;
      const uint8_t *src = planes + size_t(p) * rows * row_bytes + off;
      const uint8_t pad = pad_byte(fmt, p);
      for (size_t r = 0; r < rows; ++r) {
        if (n) std::memcpy(dst + r * 16, src + r * row_bytes, n);
        if (n < 16) std::memset(dst + r * 16 + n, pad, 16 - n);
      }
      std::memset(dst + rows * 16, 0, (Npad - rows) * 16);
    }
  }
}

void untile_planes(int fmt, const uint8_t *tiles, size_t rows, size_t row_bytes,
                   size_t Npad, size_t Kp, uint8_t *planes) {
  FormatInfo fi;
  format_info(fmt, &fi);
  const int P = fi.planes;
  const size_t Kc = Kp / kChunk;
  for (size_t c = 0; c < Kc; ++c) {
    const size_t off = c * 16;
    if (off >= row_bytes) break;
    const size_t n = row_bytes - off < 16 ? row_bytes - off : 16;
    for (int p = 0; p < P; ++p) {
      const uint8_t *src = tiles + ((c * P + p) * Npad) * 16;
      uint8_t *dst = planes + size_t(p) * rows * row_bytes + off;
      for (size_t r = 0; r < rows; ++r) std::memcpy(dst + r * row_bytes, src + r * 16, n);
    }
  }
}

}  // namespace lmx
