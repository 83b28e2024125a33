// lmx_device.hpp -- device-side building blocks shared by the LUT-GEMV
// kernels (included by the .hip sources only): format traits and per-format
// identities, the table layout and lookups, the register FWHT-256, the group
// table build, activation loads and fused transforms, argmax keys and the
// workgroup RMS norm.
#ifndef LMX_DEVICE_HPP
#define LMX_DEVICE_HPP

#include <hip/hip_runtime.h>

#include "lmx_internal.hpp"
#include "lmx_lanes.hpp"

namespace lmx {

typedef __attribute__((address_space(3))) float lds_f32;
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float lds_load(uint32_t byte_addr) {
  return *(const lds_f32 *)(size_t)byte_addr;
}

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) f32x2 lds_f32x2;
typedef __attribute__((address_space(3))) f32x4 lds_f32x4;

// 8 / 16 bytes at an 8 / 16-byte aligned LDS byte address.
__device__ __forceinline__ f32x2 lds_load2(uint32_t byte_addr) {
  return *(const lds_f32x2 *)(size_t)byte_addr;
}
__device__ __forceinline__ f32x4 lds_load4(uint32_t byte_addr) {
  return *(const lds_f32x4 *)(size_t)byte_addr;
}

__device__ __forceinline__ uint32_t lds_addr(const float *p) {
  return (uint32_t)(size_t)(const lds_f32 *)p;
}

// ---------------------------------------------------------------------------
// Format traits: loaded planes P, accumulators NA, scale stages S.
template <int FMT> struct Fmt;
template <> struct Fmt<LMX_FMT_TERNARY> { static constexpr int P = 2, NA = 2, S = 1; static constexpr bool XS = false; };
template <> struct Fmt<LMX_FMT_BINARY> { static constexpr int P = 1, NA = 1, S = 1; static constexpr bool XS = true; };
template <> struct Fmt<LMX_FMT_RRQ2> { static constexpr int P = 2, NA = 2, S = 2; static constexpr bool XS = true; };
template <> struct Fmt<LMX_FMT_RRQ3> { static constexpr int P = 3, NA = 3, S = 3; static constexpr bool XS = true; };
template <> struct Fmt<LMX_FMT_INT3> { static constexpr int P = 3, NA = 3, S = 1; static constexpr bool XS = false; };
template <> struct Fmt<LMX_FMT_INT4> { static constexpr int P = 4, NA = 4, S = 1; static constexpr bool XS = false; };
template <> struct Fmt<LMX_FMT_INT8> { static constexpr int P = 8, NA = 8, S = 1; static constexpr bool XS = false; };

// Plane words -> lookup words (one per accumulator).
template <int FMT>
__device__ __forceinline__ void lookup_words(const uint32_t *w, uint32_t *v) {
  if constexpr (FMT == LMX_FMT_TERNARY) {
    v[0] = ~(w[0] | w[1]);   // non-zero and positive
    v[1] = w[0] & ~w[1];     // non-zero and negative
  } else if constexpr (FMT == LMX_FMT_INT3) {
    v[0] = w[0]; v[1] = w[1]; v[2] = ~w[2];
  } else if constexpr (FMT == LMX_FMT_INT4) {
    v[0] = w[0]; v[1] = w[1]; v[2] = w[2]; v[3] = ~w[3];
  } else {
#pragma unroll
    for (int p = 0; p < Fmt<FMT>::P; ++p) v[p] = w[p];
  }
}

// Chunk sums -> row accumulator.
template <int FMT>
__device__ __forceinline__ float finish_chunk(const float *A, float xs, const float *sc, float acc) {
  if constexpr (FMT == LMX_FMT_TERNARY) {
    return fmaf(sc[0], A[0] - A[1], acc);
  } else if constexpr (FMT == LMX_FMT_BINARY) {
    return fmaf(sc[0], 2.0f * A[0] - xs, acc);
  } else if constexpr (FMT == LMX_FMT_RRQ2 || FMT == LMX_FMT_RRQ3) {
#pragma unroll
    for (int i = 0; i < Fmt<FMT>::S; ++i) acc = fmaf(sc[i], 2.0f * A[i] - xs, acc);
    return acc;
  } else if constexpr (FMT == LMX_FMT_INT3) {
    return fmaf(sc[0], (A[0] + 2.0f * A[1]) - 4.0f * A[2], acc);
  } else if constexpr (FMT == LMX_FMT_INT4) {
    return fmaf(sc[0], ((A[0] + 2.0f * A[1]) + 4.0f * A[2]) - 8.0f * A[3], acc);
  } else {
    float s = A[0];
#pragma unroll
    for (int b = 1; b < 7; ++b) s = fmaf(float(1 << b), A[b], s);
    return fmaf(sc[0], fmaf(-128.0f, A[7], s), acc);
  }
}


// The 8 lookups of one 32-bit lookup word (word i of a 128-k chunk = groups
// 8i..8i+7).  Addresses come from v_perm (table base bytes 1-2, 4*nibble in
// byte 0, plus an optional bank shift in bits 6-7); the group's table offset
// is the ds_read immediate.  All 64 lanes read the same 16-entry table at a
// time: 16 consecutive dwords, no bank conflicts.  word_reads issues the
// reads, word_sum adds them as a balanced tree.
// Byte offset of group g's table inside a chunk's table block.  Packed:
// 64*g.  Staggered (STAG): each table starts 16 B later than its
// predecessor's slot within a run of 4 (4 runs per 16 groups), and each
// block of 16 groups is padded by 64 B, so the 64 lanes of one table-write
// instruction (lane = group) start in 16 different 4-bank groups: the
// prologue's 16-byte writes are bank-conflict free, and every table is
// still 16 contiguous dwords for the lookups.
template <bool STAG>
__host__ __device__ constexpr uint32_t group_offset(int g) {
  return STAG ? uint32_t(64 * g + 16 * ((g >> 2) & 3) + 64 * (g >> 4)) : uint32_t(64 * g);
}
constexpr uint32_t kStagChunkBytes = 2176;
static_assert(kIplChunkBytes >= group_offset<true>(31) + 64 + 64, "a staggered chunk block and its 64-byte slice shift");
// One k-slice of CPS staggered chunk blocks plus 64 B (room for the H = 4
// slice shift), rounded up to 256 B so every slice base is 256-byte aligned.
__host__ __device__ constexpr uint32_t stag_slice_bytes(int cps) { return (cps * kStagChunkBytes + 64 + 255) / 256 * 256; }

// cbase must be 256-byte aligned (v_perm keeps its bytes 1-2 only); coff is
// a compile-time chunk offset folded into the ds_read immediate.
template <bool STAG = false>
__device__ __forceinline__ void word_reads(uint32_t v, int i, uint32_t cbase, uint32_t shift, float *t,
                                           uint32_t coff = 0) {
  const uint32_t hi = ((v >> 2) & 0x3C3C3C3Cu) | shift;  // byte b: 4*nibble of group 8i+2b
  const uint32_t lo = ((v << 2) & 0x3C3C3C3Cu) | shift;  // byte b: 4*nibble of group 8i+2b+1
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    t[2 * b] = lds_load(__builtin_amdgcn_perm(cbase, hi, 0x0C060500u | b) + (coff + group_offset<STAG>(8 * i + 2 * b)));
    t[2 * b + 1] =
        lds_load(__builtin_amdgcn_perm(cbase, lo, 0x0C060500u | b) + (coff + group_offset<STAG>(8 * i + 2 * b + 1)));
  }
}

__device__ __forceinline__ float word_sum(const float *t) {
  return ((t[0] + t[1]) + (t[2] + t[3])) + ((t[4] + t[5]) + (t[6] + t[7]));
}

template <bool STAG = false>
__device__ __forceinline__ float word_lookups(uint32_t v, int i, uint32_t cbase, uint32_t shift, uint32_t coff = 0) {
  float t[8];
  word_reads<STAG>(v, i, cbase, shift, t, coff);
  return word_sum(t);
}

// Table lookups of one 128-k chunk for one lane: NA accumulators over the
// 32 groups of the chunk.
template <int FMT, bool STAG = false>
__device__ __forceinline__ void chunk_lookups(const u32x4 *wc, uint32_t cbase, uint32_t shift, float *A,
                                              uint32_t coff = 0) {
  constexpr int P = Fmt<FMT>::P, NA = Fmt<FMT>::NA;
  if constexpr (FMT != LMX_FMT_TERNARY) {
    // Accumulator q reads plane q only.  Software pipeline over the NA*4
    // words: the reads of word n+1 are in flight while word n is summed
    // (workgroups with one wave per SIMD would otherwise wait out the LDS
    // latency once per word).
    float t[2][8];
    auto word_of = [&](int n) {
      uint32_t wi[P], v[NA];
#pragma unroll
      for (int p = 0; p < P; ++p) wi[p] = wc[p][n & 3];
      lookup_words<FMT>(wi, v);
      return v[n >> 2];
    };
    word_reads<STAG>(word_of(0), 0, cbase, shift, t[0], coff);
#pragma unroll
    for (int n = 0; n < NA * 4; ++n) {
      if (n + 1 < NA * 4) word_reads<STAG>(word_of(n + 1), (n + 1) & 3, cbase, shift, t[(n + 1) & 1], coff);
      A[n >> 2] += word_sum(t[n & 1]);
    }
    return;
  }
  if constexpr (FMT == LMX_FMT_TERNARY) {
    // Both accumulators need both planes: word-outer.
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint32_t wi[P], v[NA];
#pragma unroll
      for (int p = 0; p < P; ++p) wi[p] = wc[p][i];
      lookup_words<FMT>(wi, v);
#pragma unroll
      for (int q = 0; q < NA; ++q) A[q] += word_lookups<STAG>(v[q], i, cbase, shift, coff);
    }
  }
}

// ---------------------------------------------------------------------------
// Register FWHT-256: lane l holds x[4l..4l+3] of one 256-chunk.  Strides 1
// and 2 are in-lane, strides 4..128 pair lane l with lane l^(h/4).  Every
// output is produced by the same sequence of (a+b, a-b) as the reference's
// scalar stage loop (transform_simd.cpp:14-23,26-45) followed by x(1/16),
// so the result is bit-identical.
// One butterfly stage between lanes l and l ^ D: the lower lane keeps
// own + partner, the upper lane partner - own.  For D = 16, 32 both lanes
// read the pair as (lo, hi) and form lo + hi or lo - hi: the same operands.
template <int D>
__device__ __forceinline__ void fwht_lane_stage(float &x0, float &x1, float &x2, float &x3, int lane) {
  const bool top = (lane & D) == 0;
  if constexpr (D >= 16) {
    float l0, h0, l1, h1, l2, h2, l3, h3;
    lane_pair<D>(x0, l0, h0);
    lane_pair<D>(x1, l1, h1);
    lane_pair<D>(x2, l2, h2);
    lane_pair<D>(x3, l3, h3);
    x0 = top ? l0 + h0 : l0 - h0;
    x1 = top ? l1 + h1 : l1 - h1;
    x2 = top ? l2 + h2 : l2 - h2;
    x3 = top ? l3 + h3 : l3 - h3;
  } else {
    const float p0 = lane_xor<D>(x0, lane), p1 = lane_xor<D>(x1, lane);
    const float p2 = lane_xor<D>(x2, lane), p3 = lane_xor<D>(x3, lane);
    x0 = top ? x0 + p0 : p0 - x0;
    x1 = top ? x1 + p1 : p1 - x1;
    x2 = top ? x2 + p2 : p2 - x2;
    x3 = top ? x3 + p3 : p3 - x3;
  }
}

// The cross-lane stages exchange through DPP and permlane swaps (VALU), not
// through the LDS, which the table reads keep busy.
__device__ __forceinline__ void fwht256_regs(float &x0, float &x1, float &x2, float &x3, int lane) {
  float a0 = x0 + x1, a1 = x0 - x1, a2 = x2 + x3, a3 = x2 - x3;   // h = 1
  x0 = a0 + a2; x2 = a0 - a2; x1 = a1 + a3; x3 = a1 - a3;          // h = 2
  fwht_lane_stage<1>(x0, x1, x2, x3, lane);                        // h = 4
  fwht_lane_stage<2>(x0, x1, x2, x3, lane);
  fwht_lane_stage<4>(x0, x1, x2, x3, lane);
  fwht_lane_stage<8>(x0, x1, x2, x3, lane);
  fwht_lane_stage<16>(x0, x1, x2, x3, lane);
  fwht_lane_stage<32>(x0, x1, x2, x3, lane);                       // h = 128
  x0 *= 0.0625f; x1 *= 0.0625f; x2 *= 0.0625f; x3 *= 0.0625f;
}

// 16 partial sums of (a0,a1,a2,a3), entry m adding a_j for set bit (3-j) in
// the order a0,a1,a2,a3 from +0 (lut_gemm.hpp:30-44): bit-identical entries.
__device__ __forceinline__ void group_table(float a0, float a1, float a2, float a3, float *t) {
  const float s01 = a0 + a1, s02 = a0 + a2, s12 = a1 + a2, s23 = a2 + a3;
  const float s012 = s01 + a2;
  t[0] = 0.0f;   t[1] = a3;          t[2] = a2;          t[3] = s23;
  t[4] = a1;     t[5] = a1 + a3;     t[6] = s12;         t[7] = s12 + a3;
  t[8] = a0;     t[9] = a0 + a3;     t[10] = s02;        t[11] = s02 + a3;
  t[12] = s01;   t[13] = s01 + a3;   t[14] = s012;       t[15] = s012 + a3;
}

// Loads the lane's 4 activations of a 256-chunk starting at k0, zero past
// cols.  The caller guarantees x is 16-byte aligned and cols % 4 == 0 (the
// host stages x otherwise), so this is one clamped float4 load and a select:
// no branch, which keeps the wait for x separate from the weight stream.
__device__ __forceinline__ void load_x4(const float *__restrict__ x, int k0, int cols, int lane,
                                        float &x0, float &x1, float &x2, float &x3) {
  const int k = k0 + 4 * lane;
  const float4 v = *reinterpret_cast<const float4 *>(x + min(k, cols - 4));
  const bool in = k < cols;
  x0 = in ? v.x : 0.0f;
  x1 = in ? v.y : 0.0f;
  x2 = in ? v.z : 0.0f;
  x3 = in ? v.w : 0.0f;
}

// load_x4 in two halves: the raw (clamped) load, and the zeroing of lanes
// past cols, applied where the values are first used so that no
// instruction between the load and the weight stream waits for the data.
__device__ __forceinline__ float4 load_x4_raw(const float *__restrict__ x, int k0, int cols, int lane) {
  return *reinterpret_cast<const float4 *>(x + min(k0 + 4 * lane, cols - 4));
}

__device__ __forceinline__ void mask_x4(const float4 v, int k0, int cols, int lane, float &x0, float &x1, float &x2,
                                        float &x3) {
  const bool in = k0 + 4 * lane < cols;
  x0 = in ? v.x : 0.0f;
  x1 = in ? v.y : 0.0f;
  x2 = in ? v.z : 0.0f;
  x3 = in ? v.w : 0.0f;
}

// Second operand of the fused activation transform for the lane's 4
// activations at k0 + 4*lane: the norm weights (kXModeRmsNorm) or the up
// half of a gate|up vector (kXModeSiluMul).  Other modes load x[0..3] in
// every lane (one cache line, result unused), so the load needs no branch.
// Clamped in bounds like load_x4.
__device__ __forceinline__ void load_aux4(const GemvArgs &a, int k0, int lane, float *aux) {
  const bool used = a.xmode == kXModeRmsNorm || a.xmode == kXModeSiluMul;
  const float *p = a.xmode == kXModeRmsNorm ? a.xw : a.xmode == kXModeSiluMul ? a.x + a.cols : a.x;
  const float4 v = *reinterpret_cast<const float4 *>(p + (used ? min(k0 + 4 * lane, a.cols - 4) : 0));
  aux[0] = v.x; aux[1] = v.y; aux[2] = v.z; aux[3] = v.w;
}

__device__ __forceinline__ float silu(float g) { return g / (1.0f + expf(-g)); }   // model.cpp:36

__device__ __forceinline__ void xform4(int mode, float inv_rms, const float *aux, float &x0, float &x1, float &x2,
                                       float &x3) {
  if (mode == kXModeRmsNorm) {   // input * inv_rms * weight, in that order (norm.cpp:31)
    x0 = x0 * inv_rms * aux[0]; x1 = x1 * inv_rms * aux[1];
    x2 = x2 * inv_rms * aux[2]; x3 = x3 * inv_rms * aux[3];
  } else if (mode == kXModeSiluMul) {
    x0 = silu(x0) * aux[0]; x1 = silu(x1) * aux[1];
    x2 = silu(x2) * aux[2]; x3 = silu(x3) * aux[3];
  }
}

// Greedy-sampling fold: the key (orderable value bits << 32 | ~row) of the
// largest y over the wave's valid lanes.  Larger value wins; equal values
// keep the lower row, as the reference's first-maximum scan does
// (model.cpp:480-490).  NaN never wins; -0 counts as +0.  Every lane of the
// wave must call it; every lane gets the wave's key (0 = no valid row).
__device__ __forceinline__ unsigned long long wave_argmax_key(float v, int row, bool valid) {
  unsigned long long key = 0;
  if (valid && !__builtin_isnan(v)) {
    uint32_t u = __float_as_uint(v + 0.0f);
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    key = (static_cast<unsigned long long>(u) << 32) | (0xFFFFFFFFu - uint32_t(row));
  }
  return wave_max_key(key, threadIdx.x & (kWave - 1));
}

// Repetition penalty of Model::sample (model.cpp:458-469): once per
// occurrence of the token in the history, a positive logit is divided by the
// penalty and any other multiplied by it; the sign never changes, so n
// occurrences are n of the same step, applied one after another as there.
__device__ __forceinline__ float penalised_logit(float v, unsigned n, float penalty) {
  for (unsigned i = 0; i < n; ++i) v = v > 0.0f ? v / penalty : v * penalty;
  return v;
}

// The value the greedy pick ranks for row `row` of a GEMV with an argmax
// epilogue: y itself, or y penalised when the launch carries token counts.
__device__ __forceinline__ float argmax_value(const GemvArgs &a, float v, int row, bool valid) {
  return a.pcount && valid ? penalised_logit(v, a.pcount[row], a.penalty) : v;
}

// Writes the wave's key into its slot: one slot per wave of the launch
// (every slot is written on every launch, so the reader sees no stale keys).
__device__ __forceinline__ void wave_argmax(unsigned long long *slots, int slot, float v, int row, bool valid) {
  const unsigned long long key = wave_argmax_key(v, row, valid);
  if ((threadIdx.x & (kWave - 1)) == 0) slots[slot] = key;
}

// 1/sqrt(sum(x[0..cols)^2)/cols + eps) (norm.cpp:20-28) from per-thread
// partial sums.  Every workgroup sums in the same fixed order, so every
// workgroup gets the same bits.  red: NT/64 floats of LDS.
template <int NT>
__device__ float wg_inv_rms_from(float s, int cols, float eps, float *red) {
  s = lane_sum<32>(s, threadIdx.x & (kWave - 1));
  if ((threadIdx.x & (kWave - 1)) == 0) red[threadIdx.x / kWave] = s;
  __syncthreads();
  float t = 0.0f;
#pragma unroll
  for (int i = 0; i < NT / kWave; ++i) t += red[i];
  __syncthreads();
  return 1.0f / sqrtf(t / float(cols) + eps);
}

// The same over all of x read from memory (workgroups that hold a k-slice).
template <int NT>
__device__ float wg_inv_rms(const float *__restrict__ x, int cols, float eps, float *red) {
  float s = 0.0f;
  for (int k = 4 * int(threadIdx.x); k < cols; k += 4 * NT) {
    const float4 v = *reinterpret_cast<const float4 *>(x + k);
    s += (v.x * v.x + v.y * v.y) + (v.z * v.z + v.w * v.w);
  }
  return wg_inv_rms_from<NT>(s, cols, eps, red);
}

// One FWHT butterfly stage at lane distance D = 16 or 32 for two values a, b
// held by every lane: new a = (a_lo + a_hi, a_lo - a_hi) in the (lower, upper)
// lane of each pair (l, l ^ D), the same for b.  Two permlane swaps, one add
// and one subtract for the two values.
template <int D>
__device__ __forceinline__ void lane_pair_stage(float &a, float &b) {
  static_assert(D == 16 || D == 32, "permlane swap distance");
  uint32_t ua = __float_as_uint(a), ub = __float_as_uint(b);
  {
    const auto r = D == 16 ? __builtin_amdgcn_permlane16_swap(ua, ub, false, false)
                           : __builtin_amdgcn_permlane32_swap(ua, ub, false, false);
    ua = r[0];
    ub = r[1];
  }
  const float lo = __uint_as_float(ua), hi = __uint_as_float(ub);
  const uint32_t sum = __float_as_uint(lo + hi), dif = __float_as_uint(lo - hi);
  const auto r = D == 16 ? __builtin_amdgcn_permlane16_swap(sum, dif, false, false)
                         : __builtin_amdgcn_permlane32_swap(sum, dif, false, false);
  a = __uint_as_float(r[0]);
  b = __uint_as_float(r[1]);
}

// FWHT-256 of the lane's 4 values without the final 1/16: every output is
// exactly 16x the reference's (the butterflies are the same exact sums and
// differences, and a power-of-two scale commutes with rounding), so the
// caller folds 1/16 into the group scale.  Cross-lane butterflies are
// fma(sgn, own, partner) with sgn = +1 in the lower lane of a pair (own +
// partner) and -1 in the upper lane (partner - own): the same roundings as
// the reference's a + b and a - b.
__device__ __forceinline__ void fwht256_regs_x16(float &x0, float &x1, float &x2, float &x3, int lane) {
  float a0 = x0 + x1, a1 = x0 - x1, a2 = x2 + x3, a3 = x2 - x3;   // h = 1
  x0 = a0 + a2; x2 = a0 - a2; x1 = a1 + a3; x3 = a1 - a3;          // h = 2
#define LMX_XSTAGE(D)                                                           \
  {                                                                             \
    const float sg = (lane & (D)) ? -1.0f : 1.0f;                               \
    const float p0 = lane_xor<D>(x0, lane), p1 = lane_xor<D>(x1, lane);         \
    const float p2 = lane_xor<D>(x2, lane), p3 = lane_xor<D>(x3, lane);         \
    x0 = fmaf(sg, x0, p0); x1 = fmaf(sg, x1, p1);                               \
    x2 = fmaf(sg, x2, p2); x3 = fmaf(sg, x3, p3);                               \
  }
  LMX_XSTAGE(1) LMX_XSTAGE(2) LMX_XSTAGE(4) LMX_XSTAGE(8)
#undef LMX_XSTAGE
  // Lane distance 16 / 32 on two values per swap pair: after swap(a, b) the
  // lower half of every pair of lane groups holds (a_lo, a_hi) and the upper
  // half (b_lo, b_hi); their sum and difference, swapped back, are the new a
  // (lo + hi, lo - hi) and the new b.
  lane_pair_stage<16>(x0, x1);
  lane_pair_stage<16>(x2, x3);
  lane_pair_stage<32>(x0, x1);
  lane_pair_stage<32>(x2, x3);
}

}  // namespace lmx

#endif  // LMX_DEVICE_HPP
