// lmx_kernels.hip -- gfx950 kernels of the bit-serial LUT-GEMV path.
//
// One GEMV is one launch of a full-K kernel where its tables fit, or
// lut_gemv_kernel (split-K, last-workgroup reduction) elsewhere.  Full-K
// launches with plain activations run lut_gemv_ipl_kernel (interleaved table
// build and lookups) or lut_gemv_plain_kernel (lean front end); fused
// transforms and the argmax epilogue run lut_gemv_fullk_kernel.  All share:
//   * a fused prologue: each wavefront takes 256-chunks of x, rotates them
//     with an in-register FWHT-256 (cross-lane butterflies via shuffles)
//     when asked, and writes the 16-entry partial-sum table of every group
//     of 4 activations straight into LDS (lane l owns group l of a chunk);
//   * the lookup loop: every lane streams one row's bit-planes (one 16-byte
//     non-temporal load per plane per 128-k chunk, 1 KiB contiguous per
//     wavefront), turns each plane nibble into an LDS address with one
//     v_perm and accumulates the looked-up partial sums in fp32.  All 64
//     lanes read the same 16-entry table at a time, so a lookup touches 16
//     consecutive dwords: no bank conflicts;
//   * deterministic reductions (fixed slice order, no float atomics).
// Full-K: a workgroup owns 64/H rows and the whole K (tables of the whole K
// in LDS), k-slices spread over its lanes, slice partials summed in LDS.
// Split-K: a workgroup owns 64*WAVES rows x one k-slice and writes one
// partial per row; a second kernel (or the last workgroup) sums them.
//
// Per-format identities (T = group table, m_p = plane-p nibble, ~ = 4-bit
// complement, xs = sum of the chunk's activations):
//   ternary  T[~s&~z] - T[s&~z]                    (lut_gemm.hpp:79-99)
//   binary   2*T[m] - T[15]
//   RRQ-k    sum_i s_i * (2*T[m_i] - T[15])        (Int2Block::get generalised)
//   int3     T[m0] + 2T[m1] - 4T[~m2]              ((q-4) with q = 4b2+2b1+b0)
//   int4     T[m0] + 2T[m1] + 4T[m2] - 8T[~m3]     ((q-8))
//   int8     sum_{b<7} 2^b T[m_b] - 128 T[m7]      (two's complement)
#include <hip/hip_runtime.h>

#include "lmx_internal.hpp"
#include "lmx_lanes.hpp"

namespace lmx {

typedef __attribute__((address_space(3))) float lds_f32;
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float lds_load(uint32_t byte_addr) {
  return *(const lds_f32 *)(size_t)byte_addr;
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
constexpr uint32_t kStagChunkBytes = 2176;   // group_offset<true>(31) + 64, 16-byte multiple
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

// ---------------------------------------------------------------------------
template <int FMT, int CHUNKS, int WAVES>
__global__ __launch_bounds__(WAVES * kWave) void lut_gemv_kernel(GemvArgs a, int row_blocks, int splits) {
  constexpr int P = Fmt<FMT>::P, NA = Fmt<FMT>::NA, S = Fmt<FMT>::S;
  constexpr int KS = CHUNKS * kChunk;
  constexpr int ROWS = WAVES * kWave;
  constexpr int C2 = KS / kRotChunk;  // 256-chunks of the slice
  __shared__ __attribute__((aligned(16))) float tables[KS / 4 * 16];
  __shared__ float xsum[CHUNKS];
  __shared__ float xred[WAVES];
  __shared__ unsigned ticket;

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int rb = blockIdx.x % row_blocks;
  const int split = blockIdx.x / row_blocks;
  const int k0 = split * KS;
  const int row = rb * ROWS + wave * kWave + lane;
  const bool active = rb * ROWS + wave * kWave < a.Npad;  // whole wavefronts

  // ---- loads: this wave's activations first, then the lane's plane and
  // scale words, so the table build below only waits for x while the weight
  // stream is still in flight (vector loads retire in issue order).  Loads
  // are unconditional (indices clamped in bounds) so no branch splits them.
  constexpr int XJ = (C2 + WAVES - 1) / WAVES;
  float xv[XJ][4], aux[XJ][4];
#pragma unroll
  for (int j = 0; j < XJ; ++j) {
    const int c2 = min(wave + j * WAVES, C2 - 1);
    load_x4(a.x, k0 + c2 * kRotChunk, a.cols, lane, xv[j][0], xv[j][1], xv[j][2], xv[j][3]);
  }
  if (a.xmode == kXModeRmsNorm || a.xmode == kXModeSiluMul) {
#pragma unroll
    for (int j = 0; j < XJ; ++j) load_aux4(a, k0 + min(wave + j * WAVES, C2 - 1) * kRotChunk, lane, aux[j]);
  }
  __builtin_amdgcn_sched_barrier(0);  // keep the x loads ahead of the weight stream
  u32x4 w[CHUNKS][P];
  float sc[CHUNKS][S];
  {
    const u32x4 *__restrict__ pl = reinterpret_cast<const u32x4 *>(a.planes);
    const size_t Npad = size_t(a.Npad);
    const int c0 = k0 / kChunk;
    const int lr = min(row, a.Npad - 1);
#pragma unroll
    for (int c = 0; c < CHUNKS; ++c) {
#pragma unroll
      for (int p = 0; p < P; ++p)
        w[c][p] = __builtin_nontemporal_load(pl + (size_t(c0 + c) * P + p) * Npad + lr);
      const int g = (c0 + c) / a.group_chunks;
#pragma unroll
      for (int s = 0; s < S; ++s) sc[c][s] = a.scales[(size_t(s) * a.n_groups + g) * Npad + lr];
    }
  }

  // ---- prologue: (transform) -> (FWHT-256) -> 16-entry group tables ------
  // Lane l of the wave owning a 256-chunk holds activations 4l..4l+3 = group
  // l of the chunk and writes that group's table.
  const float inv_rms = a.xmode == kXModeRmsNorm ? wg_inv_rms<ROWS>(a.x, a.cols, a.eps, xred) : 1.0f;
#pragma unroll
  for (int j = 0; j < XJ; ++j) {
    const int c2 = wave + j * WAVES;
    if (c2 >= C2) break;   // wave-uniform
    float x0 = xv[j][0], x1 = xv[j][1], x2 = xv[j][2], x3 = xv[j][3];
    xform4(a.xmode, inv_rms, aux[j], x0, x1, x2, x3);
    if (a.rotate == LMX_ROTATE_FWHT256) fwht256_regs(x0, x1, x2, x3, lane);
    float t[16];
    group_table(x0, x1, x2, x3, t);
    float4 *dst = reinterpret_cast<float4 *>(tables + (c2 * 64 + lane) * 16);
    dst[0] = make_float4(t[0], t[1], t[2], t[3]);
    dst[1] = make_float4(t[4], t[5], t[6], t[7]);
    dst[2] = make_float4(t[8], t[9], t[10], t[11]);
    dst[3] = make_float4(t[12], t[13], t[14], t[15]);
    if constexpr (Fmt<FMT>::XS) {
      float s = t[15];
      s = lane_sum<16>(s, lane);
      if ((lane & 31) == 0) xsum[c2 * 2 + (lane >> 5)] = s;
    }
  }
  __syncthreads();

  // ---- lookups: one row per lane ------------------------------------------
  // All 64 lanes read the same 16-entry table at a time: 16 consecutive
  // dwords, no bank conflicts.  v_perm turns a byte of the pre-shifted plane
  // word into the table offset 4*nibble; the group's table offset is an
  // immediate of the ds_read.
  float acc = 0.0f;
  if (active) {
    const uint32_t tbase = lds_addr(tables);
#pragma unroll
    for (int c = 0; c < CHUNKS; ++c) {
      float A[NA];
#pragma unroll
      for (int i = 0; i < NA; ++i) A[i] = 0.0f;
      chunk_lookups<FMT>(w[c], tbase + c * (32 * 64), 0u, A);
      float xs = 0.0f;
      if constexpr (Fmt<FMT>::XS) xs = xsum[c];
      acc = finish_chunk<FMT>(A, xs, sc[c], acc);
    }
  }

  // ---- split-K reduction --------------------------------------------------
  if (splits == 1) {
    const float out = a.bias && active && row < a.rows ? acc + a.bias[row] : acc;
    if (active && row < a.rows) a.y[row] = out;
    if (a.amax) wave_argmax(a.amax, blockIdx.x * WAVES + wave, out, row, active && row < a.rows);
    return;
  }
  float *part = a.partials + size_t(split) * a.Npad;
  if (a.reduce == kReduceTwoPass) {
    if (active) part[row] = acc;
    return;
  }
  if (a.reduce == kReduceFenceAll) {
    if (active) part[row] = acc;
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) ticket = atomicAdd(a.counters + rb, 1u);
    __syncthreads();
    if (ticket != unsigned(splits - 1)) return;
    __threadfence();
  } else {
    // Partials travel as agent-scope (device-coherent) relaxed atomic stores
    // and loads, which bypass the non-coherent per-XCD L2 state, so no L2
    // writeback or invalidate is needed.  Each thread waits for its store to
    // complete before the barrier; the ticket is taken after the barrier, so
    // the workgroup that draws the last ticket sees every partial.
    if (active) __hip_atomic_store(part + row, acc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0)
      ticket = __hip_atomic_fetch_add(a.counters + rb, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (ticket != unsigned(splits - 1)) return;
  }
  const int r = rb * ROWS + threadIdx.x;
  float out = 0.0f;
  if (r < a.rows) {
    // Sum the partials in split order; loads go out 32 at a time so their
    // latencies overlap (one round trip up to 32 splits, K = 8192 at
    // 256-wide slices).
    float s = 0.0f;
    const float *pr = a.partials + r;
    for (int k0s = 0; k0s < splits; k0s += 32) {
      float v[32];
#pragma unroll
      for (int j = 0; j < 32; ++j)
        v[j] = k0s + j < splits
                   ? __hip_atomic_load(pr + size_t(k0s + j) * a.Npad, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                   : 0.0f;
#pragma unroll
      for (int j = 0; j < 32; ++j) s += v[j];
    }
    out = a.bias ? s + a.bias[r] : s;
    a.y[r] = out;
  }
  if (a.amax) wave_argmax(a.amax, rb * WAVES + wave, out, r, r < a.rows);
  if (threadIdx.x == 0) __hip_atomic_store(a.counters + rb, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Second pass of the two-pass split-K reduction: y[r] = sum_s partials[s][r]
// (+ bias).  A workgroup covers 64 rows; its 4 wavefronts each sum a quarter
// of the splits with independent loads, then wave 0 adds the four quarters
// in a fixed order.
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float *__restrict__ partials, int splits, int Npad,
                                                            int rows, const float *__restrict__ bias,
                                                            float *__restrict__ y, unsigned long long *amax) {
  __shared__ float q[4][kWave];
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  const int r = blockIdx.x * kWave + lane;
  float s = 0.0f;
  if (r < Npad)
    for (int k = wave; k < splits; k += 4) s += partials[size_t(k) * Npad + r];
  q[wave][lane] = s;
  __syncthreads();
  if (wave == 0) {
    float t = (q[0][lane] + q[1][lane]) + (q[2][lane] + q[3][lane]);
    if (r < rows) {
      t = bias ? t + bias[r] : t;
      y[r] = t;
    }
    if (amax) wave_argmax(amax, blockIdx.x, t, r, r < rows);
  }
}

// ---------------------------------------------------------------------------
// Full-K variant: a workgroup owns RW = 64/H output rows and the whole
// padded K, so no partial sums leave the workgroup.  The WAVES*H k-slices of
// CPS chunks each are spread over the lanes: lane l of wave w serves row
// l % RW of the workgroup and k-slice w*H + l/RW.  The tables of the whole K
// sit in LDS (16 B per activation); each 256-chunk is rotated by one wave.
// Slice s keeps its tables at s*(CPS*2048 + 256) bytes; with H = 4, two
// quarter-wave slices share an LDS pass, so odd slices are shifted by 64 B
// into other banks (the shift rides in bits 6-7 of the nibble byte).  At the
// end the NS = WAVES*H slice partials of each row are summed in slice order.
template <int WAVES, int H, int CPS>
constexpr uint32_t fullk_prefix_bytes() {
  return (uint32_t(WAVES * H * CPS + WAVES * kWave) * 4 + 255) / 256 * 256;
}

template <int H>
__device__ __forceinline__ uint32_t slice_shift(int s) {
  return (H == 4 && (s & 1)) ? 64u : 0u;
}

template <int FMT, int WAVES, int H, int CPS, bool STAGED>
__global__ __launch_bounds__(WAVES * kWave) void lut_gemv_fullk_kernel(GemvArgs a) {
  constexpr int P = Fmt<FMT>::P, NA = Fmt<FMT>::NA, S = Fmt<FMT>::S;
  constexpr int RW = kWave / H;
  constexpr int NS = WAVES * H;
  constexpr uint32_t SSTRIDE = CPS * 32 * 64 + 256;
  // Wave w owns the 128-chunks of its k-slices, [w*H*CPS, (w+1)*H*CPS), and
  // builds exactly their tables (XJ 256-chunks), so no other wave waits on it.
  constexpr int XJ = H * CPS >= 2 ? H * CPS / 2 : 1;
  constexpr uint32_t PREFIX = fullk_prefix_bytes<WAVES, H, CPS>();
  extern __shared__ __attribute__((aligned(256))) float lds[];
  const int Kc = a.Kp / kChunk;
  const int used = (Kc + CPS - 1) / CPS;                      // slices holding chunks
  float *xsum = lds;                                          // [NS*CPS]
  float *red = lds + NS * CPS;                                // [NS][RW]
  char *tables = reinterpret_cast<char *>(lds) + PREFIX;      // slice s at s*SSTRIDE

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int sub = lane / RW;
  const int s = wave * H + sub;
  const int rl = lane % RW;
  const int row = blockIdx.x * RW + rl;
  const int lr = min(row, a.Npad - 1);

  // ---- loads: activations for this wave's 256-chunks, then the weights ----
  const int C2n = a.Kp / kRotChunk;
  const int own0 = wave * H * CPS, own1 = own0 + H * CPS;   // owned 128-chunks [own0, own1)
  const int c2base = own0 / 2;
  float4 xr[XJ];
  float aux[XJ][4];
#pragma unroll
  for (int j = 0; j < XJ; ++j) {
    const int c2 = min(c2base + j, C2n - 1);
    xr[j] = load_x4_raw(a.x, c2 * kRotChunk, a.cols, lane);
    load_aux4(a, c2 * kRotChunk, lane, aux[j]);
  }
  __builtin_amdgcn_sched_barrier(0);
  // A CU returns vector loads roughly in issue order, so every wave's x
  // requests go out before any wave's weight requests (the barrier does not
  // wait for the loads): no wave's tables wait behind the weight stream.
  __builtin_amdgcn_s_barrier();
  // Weight loads.  STAGED (CPS > 1 only) issues chunk 0 before the table
  // prologue and the later chunks after it, so that HBM serves chunk 0 of
  // every wave first and chunk 1 streams in while chunk 0 is looked up.
  u32x4 w[CPS][P];
  float sc[CPS][S];
  const u32x4 *__restrict__ pl = reinterpret_cast<const u32x4 *>(a.planes);
  const size_t Npad = size_t(a.Npad);
  auto load_planes = [&](int c) {
    const int ch = min(s * CPS + c, Kc - 1);                   // clamped; masked below
#pragma unroll
    for (int p = 0; p < P; ++p) w[c][p] = __builtin_nontemporal_load(pl + (size_t(ch) * P + p) * Npad + lr);
  };
#pragma unroll
  for (int c = 0; c < CPS; ++c) {
    const int ch = min(s * CPS + c, Kc - 1);
    const int g = ch / a.group_chunks;
    if (!STAGED || c == 0) load_planes(c);
#pragma unroll
    for (int t = 0; t < S; ++t) sc[c][t] = a.scales[(size_t(t) * a.n_groups + g) * Npad + lr];
  }
  if constexpr (STAGED) __builtin_amdgcn_sched_barrier(0);

  // ---- prologue: (transform) -> (FWHT-256) -> this wave's group tables ---
  // Lanes 0-31 / 32-63 hold the first / second 128-chunk of a 256-chunk; a
  // lane's values count (norm, tables) only where the wave owns that chunk,
  // which partitions x exactly, so the norm needs no second read of x.
  float inv_rms = 1.0f;
  if (a.xmode == kXModeRmsNorm) {
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < XJ; ++j) {
      const int ch = (c2base + j) * 2 + (lane >> 5);
      float x0, x1, x2, x3;
      mask_x4(xr[j], (c2base + j) * kRotChunk, a.cols, lane, x0, x1, x2, x3);
      if (ch >= own0 && ch < own1 && c2base + j < C2n) ss += (x0 * x0 + x1 * x1) + (x2 * x2 + x3 * x3);
    }
    inv_rms = wg_inv_rms_from<WAVES * kWave>(ss, a.cols, a.eps, red);
  }
#pragma unroll
  for (int j = 0; j < XJ; ++j) {
    const int c2 = c2base + j;
    if (c2 >= C2n) break;   // wave-uniform
    float x0, x1, x2, x3;
    mask_x4(xr[j], c2 * kRotChunk, a.cols, lane, x0, x1, x2, x3);
    xform4(a.xmode, inv_rms, aux[j], x0, x1, x2, x3);
    if (a.rotate == LMX_ROTATE_FWHT256) fwht256_regs(x0, x1, x2, x3, lane);
    float t[16];
    group_table(x0, x1, x2, x3, t);
    const int ch = c2 * 2 + (lane >> 5);                      // 128-chunk of this group
    const bool mine = ch >= own0 && ch < own1;
    const int ts = ch / CPS;                                  // its k-slice
    float4 *dst = reinterpret_cast<float4 *>(tables + ts * SSTRIDE + slice_shift<H>(ts) + (ch % CPS) * 2048 +
                                             (lane & 31) * 64);
    if (mine) {
      dst[0] = make_float4(t[0], t[1], t[2], t[3]);
      dst[1] = make_float4(t[4], t[5], t[6], t[7]);
      dst[2] = make_float4(t[8], t[9], t[10], t[11]);
      dst[3] = make_float4(t[12], t[13], t[14], t[15]);
    }
    if constexpr (Fmt<FMT>::XS) {
      float xs = t[15];
      xs = lane_sum<16>(xs, lane);
      if ((lane & 31) == 0 && mine) xsum[ch] = xs;
    }
  }
  if constexpr (STAGED) {
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int c = 1; c < CPS; ++c) load_planes(c);
  }
  // Each wave reads only the tables it wrote: a wave-scope fence (LDS
  // operations of a wave complete in order) instead of a workgroup barrier,
  // so every wave starts its lookups as soon as its own data is in.
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();

  // ---- lookups over this lane's k-slice -----------------------------------
  float acc = 0.0f;
  {
    // Lanes whose slice lies past K read slice used-1 (in bounds, possibly
    // another wave's, possibly mid-write) and discard the result.
    const uint32_t tbase = lds_addr(lds) + PREFIX + min(s, used - 1) * SSTRIDE;   // 256-byte aligned
    const uint32_t shift = slice_shift<H>(s) * 0x01010101u;   // bits 6-7 of each byte
#pragma unroll
    for (int c = 0; c < CPS; ++c) {
      float A[NA];
#pragma unroll
      for (int i = 0; i < NA; ++i) A[i] = 0.0f;
      chunk_lookups<FMT>(w[c], tbase + c * 2048, shift, A);
      const int ch = s * CPS + c;
      float xs = 0.0f;
      if constexpr (Fmt<FMT>::XS) xs = xsum[min(ch, Kc - 1)];
      const float nacc = finish_chunk<FMT>(A, xs, sc[c], acc);
      acc = ch < Kc ? nacc : acc;
    }
  }

  // ---- in-workgroup reduction over the k-slices, fixed order --------------
  red[s * RW + rl] = acc;
  __syncthreads();
  const int r = blockIdx.x * RW + threadIdx.x;
  float t = 0.0f;
  if (threadIdx.x < RW) {
#pragma unroll 8
    for (int k = 0; k < NS; ++k) t += red[k * RW + threadIdx.x];
    if (r < a.rows) {
      t = a.bias ? t + a.bias[r] : t;
      a.y[r] = t;
    }
  }
  if (a.amax && threadIdx.x < kWave) wave_argmax(a.amax, blockIdx.x, t, r, threadIdx.x < RW && r < a.rows);
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

// Full-K kernel with a lean front end: the same geometry, lookups and
// slice reduction as lut_gemv_fullk_kernel, staggered tables, weight and
// scale addresses in 32-bit offsets with a shift for the scale group, x
// rotated (ROT) without its final 1/16 (folded into the scales), every wave
// building the tables of its own 256-chunks only, and the activation
// transform XM (kXMode*) fixed at compile time.  Needs H*CPS even (each
// wave owns whole 256-chunks).  No argmax epilogue.
template <int FMT, bool ROT, int WAVES, int H, int CPS, int XM>
__global__ __launch_bounds__(WAVES * kWave) void lut_gemv_plain_kernel(GemvArgs a) {
  constexpr int P = Fmt<FMT>::P, NA = Fmt<FMT>::NA, S = Fmt<FMT>::S;
  constexpr int RW = kWave / H;
  constexpr int NS = WAVES * H;
  constexpr uint32_t SSTRIDE = stag_slice_bytes(CPS);
  constexpr int XJ = H * CPS / 2;
  static_assert(H * CPS % 2 == 0, "whole 256-chunks per wave");
  constexpr uint32_t PREFIX = fullk_prefix_bytes<WAVES, H, CPS>();
  extern __shared__ __attribute__((aligned(256))) float lds[];
  const int Kc = a.Kp / kChunk;
  const int used = (Kc + CPS - 1) / CPS;
  float *xsum = lds;
  float *red = lds + NS * CPS;
  char *tables = reinterpret_cast<char *>(lds) + PREFIX;

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int s = wave * H + lane / RW;
  const int rl = lane % RW;
  const int row = blockIdx.x * RW + rl;
  const int lr = min(row, a.Npad - 1);

  // ---- x of this wave's 256-chunks (clamped in bounds, masked below) ----
  const int C2n = a.Kp / kRotChunk;
  const int c2base = wave * XJ;
  constexpr bool AUX = XM == kXModeRmsNorm || XM == kXModeSiluMul;
  float4 xr[XJ], xa[XJ];
#pragma unroll
  for (int j = 0; j < XJ; ++j) {
    const int k = min(min(c2base + j, C2n - 1) * kRotChunk + 4 * lane, a.cols - 4);
    xr[j] = *reinterpret_cast<const float4 *>(a.x + k);
    // norm weight, or the up half of a gate|up vector
    if constexpr (AUX) xa[j] = *reinterpret_cast<const float4 *>((XM == kXModeRmsNorm ? a.xw : a.x + a.cols) + k);
  }
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_barrier();   // every wave's x requests ahead of the weight stream

  // ---- weights (chunk 0 now, the rest after the prologue) and scales ----
  u32x4 w[CPS][P];
  float sc[CPS][S];
  const u32x4 *__restrict__ pl = reinterpret_cast<const u32x4 *>(a.planes);
  const uint32_t Npad = uint32_t(a.Npad);
  auto load_planes = [&](int c) {
    const uint32_t ch = uint32_t(min(s * CPS + c, Kc - 1));
#pragma unroll
    for (int p = 0; p < P; ++p) w[c][p] = __builtin_nontemporal_load(pl + ((ch * P + p) * Npad + uint32_t(lr)));
  };
  load_planes(0);
#pragma unroll
  for (int c = 0; c < CPS; ++c) {
    const int ch = min(s * CPS + c, Kc - 1);
    const int g = a.gshift >= 0 ? ch >> a.gshift : ch / a.group_chunks;
#pragma unroll
    for (int t = 0; t < S; ++t) sc[c][t] = a.scales[(uint32_t(t * a.n_groups + g)) * Npad + uint32_t(lr)];
  }
  __builtin_amdgcn_sched_barrier(0);

  // RMSNorm: the waves' 256-chunks partition x, so the sum of squares over
  // them (zero past cols) is the norm's, summed in the same order in every
  // workgroup (norm.cpp:18-34).
  float inv_rms = 1.0f;
  if constexpr (XM == kXModeRmsNorm) {
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < XJ; ++j) {
      float x0, x1, x2, x3;
      mask_x4(xr[j], (c2base + j) * kRotChunk, a.cols, lane, x0, x1, x2, x3);
      if (c2base + j < C2n) ss += (x0 * x0 + x1 * x1) + (x2 * x2 + x3 * x3);
    }
    inv_rms = wg_inv_rms_from<WAVES * kWave>(ss, a.cols, a.eps, red);
  }

  // ---- prologue: (transform) -> (FWHT-256 x16) -> group tables of this wave's chunks ----
  const uint32_t goff = group_offset<true>(lane & 31);
#pragma unroll
  for (int j = 0; j < XJ; ++j) {
    const int c2 = c2base + j;
    if (c2 >= C2n) break;   // wave-uniform
    float x0, x1, x2, x3;
    mask_x4(xr[j], c2 * kRotChunk, a.cols, lane, x0, x1, x2, x3);
    if constexpr (AUX) {
      const float aux[4] = {xa[j].x, xa[j].y, xa[j].z, xa[j].w};
      xform4(XM, inv_rms, aux, x0, x1, x2, x3);
    }
    if constexpr (ROT) fwht256_regs_x16(x0, x1, x2, x3, lane);
    float t[16];
    group_table(x0, x1, x2, x3, t);
    const int ch = c2 * 2 + (lane >> 5);
    const int ts = ch / CPS;
    float4 *dst = reinterpret_cast<float4 *>(tables + ts * SSTRIDE + slice_shift<H>(ts) +
                                             (ch % CPS) * kStagChunkBytes + goff);
    dst[0] = make_float4(t[0], t[1], t[2], t[3]);
    dst[1] = make_float4(t[4], t[5], t[6], t[7]);
    dst[2] = make_float4(t[8], t[9], t[10], t[11]);
    dst[3] = make_float4(t[12], t[13], t[14], t[15]);
    if constexpr (Fmt<FMT>::XS) {
      float xs = t[15];
      xs = lane_sum<16>(xs, lane);
      if ((lane & 31) == 0) xsum[ch] = xs;
    }
  }
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int c = 1; c < CPS; ++c) load_planes(c);
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();

  // ---- lookups over this lane's k-slice ----------------------------------
  constexpr float kScale = ROT ? 0.0625f : 1.0f;   // the FWHT's 1/16, exact
  float acc = 0.0f;
  {
    const uint32_t tbase = lds_addr(lds) + PREFIX + min(s, used - 1) * SSTRIDE;
    const uint32_t shift = slice_shift<H>(s) * 0x01010101u;
#pragma unroll
    for (int c = 0; c < CPS; ++c) {
      float A[NA];
#pragma unroll
      for (int i = 0; i < NA; ++i) A[i] = 0.0f;
      chunk_lookups<FMT, true>(w[c], tbase, shift, A, c * kStagChunkBytes);
      const int ch = s * CPS + c;
      float xs = 0.0f;
      if constexpr (Fmt<FMT>::XS) xs = xsum[min(ch, Kc - 1)];
      float scl[S];
#pragma unroll
      for (int t = 0; t < S; ++t) scl[t] = sc[c][t] * kScale;
      const float nacc = finish_chunk<FMT>(A, xs, scl, acc);
      acc = ch < Kc ? nacc : acc;
    }
  }

  // ---- in-workgroup reduction over the k-slices, fixed order --------------
  red[s * RW + rl] = acc;
  __syncthreads();
  if (threadIdx.x < RW) {
    const int r = blockIdx.x * RW + threadIdx.x;
    float t = 0.0f;
#pragma unroll 8
    for (int k = 0; k < NS; ++k) t += red[k * RW + threadIdx.x];
    if (r < a.rows) a.y[r] = a.bias ? t + a.bias[r] : t;
  }
}

// Interleaved variant of the plain kernel (two k-slices per wave, H = 2):
// wave w owns the 256-chunks c2 = w*CPS + c, c < CPS, and at step c its
// lower / upper half-wave looks up 128-chunk 2*c2 / 2*c2 + 1, exactly the two
// halves of the 256-chunk it has just rotated.  So every step is "build the
// tables of one 256-chunk, then look them up", and the VALU-heavy table
// build of one wave overlaps the LDS-heavy lookups of the others.  Chunk ch
// keeps its (staggered) tables at ch * kIplChunkBytes, a 256-byte multiple.
constexpr uint32_t kIplChunkBytes = 2304;

template <int WAVES, int CPS>
constexpr uint32_t ipl_prefix_bytes() {
  return (uint32_t(2 * WAVES * CPS + 2 * WAVES * (kWave / 2)) * 4 + 255) / 256 * 256;
}

template <int FMT, bool ROT, int WAVES, int CPS>
__global__ __launch_bounds__(WAVES * kWave) void lut_gemv_ipl_kernel(GemvArgs a) {
  constexpr int P = Fmt<FMT>::P, NA = Fmt<FMT>::NA, S = Fmt<FMT>::S;
  constexpr int RW = kWave / 2;
  constexpr int NS = WAVES * 2;
  constexpr uint32_t PREFIX = ipl_prefix_bytes<WAVES, CPS>();
  extern __shared__ __attribute__((aligned(256))) float lds[];
  const int Kc = a.Kp / kChunk;
  float *xsum = lds;                 // [2*WAVES*CPS]
  float *red = lds + 2 * WAVES * CPS;   // [NS][RW]
  char *tables = reinterpret_cast<char *>(lds) + PREFIX;

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int h = lane >> 5;
  const int rl = lane & (RW - 1);
  const int row = blockIdx.x * RW + rl;
  const int lr = min(row, a.Npad - 1);

  const int C2n = a.Kp / kRotChunk;
  const int c2base = wave * CPS;
  float4 xr[CPS];
#pragma unroll
  for (int c = 0; c < CPS; ++c) xr[c] = load_x4_raw(a.x, min(c2base + c, C2n - 1) * kRotChunk, a.cols, lane);
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_barrier();   // every wave's x requests ahead of the weight stream

  u32x4 w[CPS][P];
  float sc[CPS][S];
  const u32x4 *__restrict__ pl = reinterpret_cast<const u32x4 *>(a.planes);
  const uint32_t Npad = uint32_t(a.Npad);
  auto chunk_of = [&](int c) { return min(2 * (c2base + c) + h, Kc - 1); };   // clamped; masked below
  auto load_planes = [&](int c) {
    const uint32_t ch = uint32_t(chunk_of(c));
#pragma unroll
    for (int p = 0; p < P; ++p) w[c][p] = __builtin_nontemporal_load(pl + ((ch * P + p) * Npad + uint32_t(lr)));
  };
  load_planes(0);
#pragma unroll
  for (int c = 0; c < CPS; ++c) {
    const int ch = chunk_of(c);
    const int g = a.gshift >= 0 ? ch >> a.gshift : ch / a.group_chunks;
#pragma unroll
    for (int t = 0; t < S; ++t) sc[c][t] = a.scales[(uint32_t(t * a.n_groups + g)) * Npad + uint32_t(lr)];
  }
  __builtin_amdgcn_sched_barrier(0);

  constexpr float kScale = ROT ? 0.0625f : 1.0f;   // the FWHT's 1/16, exact
  const uint32_t goff = group_offset<true>(lane & 31);
  const uint32_t tb = lds_addr(lds) + PREFIX;
  float acc = 0.0f;
#pragma unroll
  for (int c = 0; c < CPS; ++c) {
    const int c2 = c2base + c;
    if (c2 >= C2n) break;   // wave-uniform: no chunk of this step holds data
    // ---- tables of 256-chunk c2 (128-chunks 2*c2 and 2*c2 + 1) ----
    {
      float x0 = xr[c].x, x1 = xr[c].y, x2 = xr[c].z, x3 = xr[c].w;
      if (c2 * kRotChunk + kRotChunk > a.cols)   // wave-uniform: only the chunk holding the end of x
        mask_x4(xr[c], c2 * kRotChunk, a.cols, lane, x0, x1, x2, x3);
      if constexpr (ROT) fwht256_regs_x16(x0, x1, x2, x3, lane);
      float t[16];
      group_table(x0, x1, x2, x3, t);
      float4 *dst = reinterpret_cast<float4 *>(tables + (2 * c2 + h) * kIplChunkBytes + goff);
      dst[0] = make_float4(t[0], t[1], t[2], t[3]);
      dst[1] = make_float4(t[4], t[5], t[6], t[7]);
      dst[2] = make_float4(t[8], t[9], t[10], t[11]);
      dst[3] = make_float4(t[12], t[13], t[14], t[15]);
      if constexpr (Fmt<FMT>::XS) {
        float xs = t[15];
        xs = lane_sum<16>(xs, lane);
        if ((lane & 31) == 0) xsum[2 * c2 + h] = xs;
      }
    }
    if (c == 0) {   // later chunks stream in while this one is looked up
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int cc = 1; cc < CPS; ++cc) load_planes(cc);
      __builtin_amdgcn_sched_barrier(0);
    }
    // A wave reads only the tables it wrote; its LDS operations complete in order.
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
    // ---- lookups of 128-chunk 2*c2 + h ----
    const int ch = 2 * c2 + h;
    float A[NA];
#pragma unroll
    for (int i = 0; i < NA; ++i) A[i] = 0.0f;
    chunk_lookups<FMT, true>(w[c], tb + uint32_t(ch) * kIplChunkBytes, 0u, A);
    float xs = 0.0f;
    if constexpr (Fmt<FMT>::XS) xs = xsum[min(ch, Kc - 1)];
    float scl[S];
#pragma unroll
    for (int t = 0; t < S; ++t) scl[t] = sc[c][t] * kScale;
    const float nacc = finish_chunk<FMT>(A, xs, scl, acc);
    acc = ch < Kc ? nacc : acc;
  }

  // ---- in-workgroup reduction over the 2*WAVES slices, fixed order ----
  red[(wave * 2 + h) * RW + rl] = acc;
  __syncthreads();
  if (threadIdx.x < RW) {
    const int r = blockIdx.x * RW + threadIdx.x;
    float t = 0.0f;
#pragma unroll 8
    for (int k = 0; k < NS; ++k) t += red[k * RW + threadIdx.x];
    if (r < a.rows) a.y[r] = a.bias ? t + a.bias[r] : t;
  }
}

template <int FMT, bool ROT, int WAVES, int H, int CPS, int XM>
static int launch_plain_kernel(const GemvArgs &a, hipStream_t st) {
  const size_t Kc = size_t(a.Kp / kChunk);
  const size_t lds = fullk_prefix_bytes<WAVES, H, CPS>() + (Kc + CPS - 1) / CPS * stag_slice_bytes(CPS);
  if (lds > kMaxLdsBytes) return 1;   // staggered tables do not fit: the generic kernel serves it
  static const hipError_t attr = hipFuncSetAttribute(
      reinterpret_cast<const void *>(&lut_gemv_plain_kernel<FMT, ROT, WAVES, H, CPS, XM>),
      hipFuncAttributeMaxDynamicSharedMemorySize, int(kMaxLdsBytes));
  if (attr != hipSuccess) return fail(LMX_ERR_LAUNCH_FAILED, "hipFuncSetAttribute: %s", hipGetErrorString(attr));
  if (lds > kMaxLdsBytes) return fail(LMX_ERR_INVALID_ARGUMENT, "full-K tables need %zu B of LDS", lds);
  constexpr int RW = kWave / H;
  lut_gemv_plain_kernel<FMT, ROT, WAVES, H, CPS, XM>
      <<<dim3((a.Npad + RW - 1) / RW), dim3(WAVES * kWave), lds, st>>>(a);
  return LMX_OK;
}

template <int FMT, bool ROT, int WAVES, int CPS>
static int launch_ipl_kernel(const GemvArgs &a, hipStream_t st) {
  const size_t lds = ipl_prefix_bytes<WAVES, CPS>() + size_t(a.Kp / kRotChunk) * 2 * kIplChunkBytes;
  if (lds > kMaxLdsBytes) return 1;
  static const hipError_t attr =
      hipFuncSetAttribute(reinterpret_cast<const void *>(&lut_gemv_ipl_kernel<FMT, ROT, WAVES, CPS>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, int(kMaxLdsBytes));
  if (attr != hipSuccess) return fail(LMX_ERR_LAUNCH_FAILED, "hipFuncSetAttribute: %s", hipGetErrorString(attr));
  lut_gemv_ipl_kernel<FMT, ROT, WAVES, CPS><<<dim3((a.Npad + 31) / 32), dim3(WAVES * kWave), lds, st>>>(a);
  return LMX_OK;
}

template <int FMT, int WAVES, int H, int CPS>
static int launch_plain_cfg(const GemvArgs &a, hipStream_t st) {
  // Interleaved where it measured faster: two k-slices per wave and at least
  // two steps per wave (one step has nothing to interleave; 17920 x 1536
  // ran 40% slower that way), RRQ-3 excepted (4% slower at 8192^2).
  if (a.xmode != kXModeNone) {
    // Fused transforms on the lean kernel: the decode step's linears (4-bit,
    // unrotated); other formats take the generic kernel.
    if constexpr (FMT == LMX_FMT_INT4) {
      if (a.rotate == LMX_ROTATE_NONE) {
        switch (a.xmode) {
        case kXModeRmsNorm: return launch_plain_kernel<FMT, false, WAVES, H, CPS, kXModeRmsNorm>(a, st);
        case kXModeSiluMul: return launch_plain_kernel<FMT, false, WAVES, H, CPS, kXModeSiluMul>(a, st);
        }
      }
    }
    return 1;
  }
  if constexpr (H == 2 && CPS >= 2 && FMT != LMX_FMT_RRQ3) {
    if (a.kfamily != kKernelLean) {
      const int r = a.rotate == LMX_ROTATE_FWHT256 ? launch_ipl_kernel<FMT, true, WAVES, CPS>(a, st)
                                                   : launch_ipl_kernel<FMT, false, WAVES, CPS>(a, st);
      if (r != 1) return r;
    }
  }
  if (a.rotate == LMX_ROTATE_FWHT256) return launch_plain_kernel<FMT, true, WAVES, H, CPS, kXModeNone>(a, st);
  return launch_plain_kernel<FMT, false, WAVES, H, CPS, kXModeNone>(a, st);
}

// The plain kernel serves full-K launches without a fused transform or an
// argmax epilogue; returns 1 when the configuration is not covered.
template <int FMT>
static int launch_plain(const GemvArgs &a, hipStream_t st) {
  switch (a.fullk) {
  case kFullK_16x2x2: return launch_plain_cfg<FMT, 16, 2, 2>(a, st);
  case kFullK_16x2x3: return launch_plain_cfg<FMT, 16, 2, 3>(a, st);
  case kFullK_8x2x1: return launch_plain_cfg<FMT, 8, 2, 1>(a, st);
  case kFullK_16x4x1: return launch_plain_cfg<FMT, 16, 4, 1>(a, st);
  case kFullK_4x4x1: return launch_plain_cfg<FMT, 4, 4, 1>(a, st);
  }
  return 1;
}

template <int FMT, int WAVES, int H, int CPS, bool STAGED>
static int launch_fullk_kernel(const GemvArgs &a, hipStream_t st) {
  const size_t lds = fullk_lds_bytes(WAVES, H, CPS, a.Kp / kChunk);
  static const hipError_t attr = hipFuncSetAttribute(
      reinterpret_cast<const void *>(&lut_gemv_fullk_kernel<FMT, WAVES, H, CPS, STAGED>),
      hipFuncAttributeMaxDynamicSharedMemorySize, int(kMaxLdsBytes));
  if (attr != hipSuccess) return fail(LMX_ERR_LAUNCH_FAILED, "hipFuncSetAttribute: %s", hipGetErrorString(attr));
  if (lds > kMaxLdsBytes) return fail(LMX_ERR_INVALID_ARGUMENT, "full-K tables need %zu B of LDS", lds);
  constexpr int RW = kWave / H;
  lut_gemv_fullk_kernel<FMT, WAVES, H, CPS, STAGED>
      <<<dim3((a.Npad + RW - 1) / RW), dim3(WAVES * kWave), lds, st>>>(a);
  return LMX_OK;
}

template <int FMT, int WAVES, int H, int CPS>
static int launch_fullk_cfg(const GemvArgs &a, hipStream_t st) {
  if constexpr (CPS > 1)
    if (a.staged) return launch_fullk_kernel<FMT, WAVES, H, CPS, true>(a, st);
  return launch_fullk_kernel<FMT, WAVES, H, CPS, false>(a, st);
}

template <int FMT, int WAVES>
static void launch_waves(const GemvArgs &a, hipStream_t st) {
  const int row_blocks = (a.Npad + WAVES * kWave - 1) / (WAVES * kWave);
  const int splits = a.Kp / a.kslice;
  dim3 grid(row_blocks * splits), block(WAVES * kWave);
  if (a.kslice == 512)
    lut_gemv_kernel<FMT, 4, WAVES><<<grid, block, 0, st>>>(a, row_blocks, splits);
  else
    lut_gemv_kernel<FMT, 2, WAVES><<<grid, block, 0, st>>>(a, row_blocks, splits);
}

template <int FMT>
static int launch_fullk(const GemvArgs &a, hipStream_t st) {
  switch (a.fullk) {
  case kFullK_16x2x2: return launch_fullk_cfg<FMT, 16, 2, 2>(a, st);
  case kFullK_16x2x3: return launch_fullk_cfg<FMT, 16, 2, 3>(a, st);
  case kFullK_8x2x1: return launch_fullk_cfg<FMT, 8, 2, 1>(a, st);
  case kFullK_16x1x1: return launch_fullk_cfg<FMT, 16, 1, 1>(a, st);
  case kFullK_16x4x1: return launch_fullk_cfg<FMT, 16, 4, 1>(a, st);
  case kFullK_4x4x1: return launch_fullk_cfg<FMT, 4, 4, 1>(a, st);
  }
  return fail(LMX_ERR_INVALID_ARGUMENT, "unknown full-K configuration %d", a.fullk);
}

template <int FMT>
static int launch_fmt(const GemvArgs &a, hipStream_t st) {
  if (a.fullk) {
    int r = 1;
    if (!a.amax && a.kfamily != kKernelGeneric) r = launch_plain<FMT>(a, st);
    if (r == 1) r = launch_fullk<FMT>(a, st);
    if (r) return r;
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(LMX_ERR_LAUNCH_FAILED, "lut_gemv_fullk launch: %s", hipGetErrorString(e));
    return LMX_OK;
  }
  if (a.kslice != 256 && a.kslice != 512)
    return fail(LMX_ERR_INVALID_ARGUMENT, "unsupported k-slice %d", a.kslice);
  switch (a.waves) {
  case 1: launch_waves<FMT, 1>(a, st); break;
  case 2: launch_waves<FMT, 2>(a, st); break;
  case 4: launch_waves<FMT, 4>(a, st); break;
  default: return fail(LMX_ERR_INVALID_ARGUMENT, "unsupported waves per workgroup %d", a.waves);
  }
  const int splits = a.Kp / a.kslice;
  if (splits > 1 && a.reduce == kReduceTwoPass)
    splitk_reduce_kernel<<<dim3((a.rows + kWave - 1) / kWave), dim3(256), 0, st>>>(a.partials, splits, a.Npad,
                                                                                  a.rows, a.bias, a.y, a.amax);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(LMX_ERR_LAUNCH_FAILED, "lut_gemv launch: %s", hipGetErrorString(e));
  return LMX_OK;
}

size_t gemv_argmax_slots(const GemvArgs &a) {
  if (a.fullk) return size_t((a.Npad + kWave / fullk_shape(a.fullk).h - 1) / (kWave / fullk_shape(a.fullk).h));
  const int splits = a.Kp / a.kslice;
  if (splits == 1) return size_t((a.Npad + a.waves * kWave - 1) / (a.waves * kWave)) * size_t(a.waves);
  if (a.reduce == kReduceTwoPass) return size_t((a.rows + kWave - 1) / kWave);
  return size_t((a.Npad + a.waves * kWave - 1) / (a.waves * kWave)) * size_t(a.waves);
}

// ---------------------------------------------------------------------------
// Batched GEMV: y_b = W x_b for NB activation vectors with the weights read
// once (replaces lut_linear's per-row loop, lut_gemm_scalar.cpp:76-79).  A
// workgroup owns 256 rows and a k-slice of 256 with 4 * NB/VG waves: wave w
// serves row group w % 4 (one row per lane) for vectors (w / 4)*VG ..
// (w / 4)*VG + VG - 1, so the LDS lookups of many vectors have enough waves
// to hide their latency (the weight words of a row group are read by NB/VG
// waves: one HBM read, the rest cache hits).  The tables of a vector group
// sit interleaved per group in LDS, table (chunk c, vector group v, group g,
// vector b of the group) at (((c*NB/VG + v)*32 + g)*VG + b)*64 bytes, so
// every group block starts 256-byte aligned, one v_perm address serves a
// wave's VG vectors and the vector picks the ds_read immediate.  Partials
// [NB][splits][Npad] go through batched_reduce_kernel.
template <int VG>
__device__ __forceinline__ void word_lookups_batch(uint32_t v, int i, uint32_t cbase, float *out) {
  const uint32_t hi = (v >> 2) & 0x3C3C3C3Cu, lo = (v << 2) & 0x3C3C3C3Cu;
  uint32_t ad[8];
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    ad[2 * b] = __builtin_amdgcn_perm(cbase, hi, 0x0C060500u | b);
    ad[2 * b + 1] = __builtin_amdgcn_perm(cbase, lo, 0x0C060500u | b);
  }
#pragma unroll
  for (int n = 0; n < VG; ++n) {
    float t[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) t[j] = lds_load(ad[j] + ((8 * i + j) * VG + n) * 64);
    out[n] += ((t[0] + t[1]) + (t[2] + t[3])) + ((t[4] + t[5]) + (t[6] + t[7]));
  }
}

template <int NB, int VG>
constexpr int batch_waves() { return 4 * (NB / VG); }

template <int FMT, int NB, int VG>
__global__ __launch_bounds__((kWave * batch_waves<NB, VG>())) void lut_gemv_batch_kernel(GemvArgs a, int row_blocks,
                                                                                      int splits) {
  constexpr int P = Fmt<FMT>::P, NA = Fmt<FMT>::NA, S = Fmt<FMT>::S;
  constexpr int CH = kRotChunk / kChunk;   // 2 chunks of 128 per slice
  constexpr int NW = batch_waves<NB, VG>();
  constexpr int NVG = NB / VG;
  static_assert(NB % VG == 0 && NW <= 16, "whole vector groups, at most 1024 threads");
  __shared__ __attribute__((aligned(256))) float tables[CH * 32 * NB * 16];
  __shared__ float xsum[NB][CH];
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  const int rg = wave & 3, vg = wave >> 2;
  const int rb = blockIdx.x % row_blocks, split = blockIdx.x / row_blocks;
  const int k0 = split * kRotChunk;
  const int row = rb * 256 + rg * kWave + lane;
  const bool active = rb * 256 + rg * kWave < a.Npad;
  const int lr = min(row, a.Npad - 1);

  // activations: wave w builds the tables of vectors w, w + NW, ...
  constexpr int XV = (NB + NW - 1) / NW;
  float xv[XV][4];
#pragma unroll
  for (int j = 0; j < XV; ++j) {
    const int n = min(wave + NW * j, NB - 1);
    load_x4(a.x + size_t(n) * a.cols, k0, a.cols, lane, xv[j][0], xv[j][1], xv[j][2], xv[j][3]);
  }
  __builtin_amdgcn_sched_barrier(0);
  u32x4 w[CH][P];
  float sc[CH][S];
  {
    const u32x4 *__restrict__ pl = reinterpret_cast<const u32x4 *>(a.planes);
    const size_t Npad = size_t(a.Npad);
    const int c0 = k0 / kChunk;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
#pragma unroll
      for (int p = 0; p < P; ++p) {
        const u32x4 *src = pl + (size_t(c0 + c) * P + p) * Npad + lr;
        // one wave per row group streams; the others re-read through the caches
        w[c][p] = NW == 4 ? __builtin_nontemporal_load(src) : *src;
      }
      const int g = (c0 + c) / a.group_chunks;
#pragma unroll
      for (int t = 0; t < S; ++t) sc[c][t] = a.scales[(size_t(t) * a.n_groups + g) * Npad + lr];
    }
  }
#pragma unroll
  for (int j = 0; j < XV; ++j) {
    const int n = wave + NW * j;
    if (n >= NB) break;   // wave-uniform
    float x0 = xv[j][0], x1 = xv[j][1], x2 = xv[j][2], x3 = xv[j][3];
    if (a.rotate == LMX_ROTATE_FWHT256) fwht256_regs(x0, x1, x2, x3, lane);
    float t[16];
    group_table(x0, x1, x2, x3, t);
    const int c = lane >> 5, g = lane & 31;
    float4 *dst = reinterpret_cast<float4 *>(tables + (((c * NVG + n / VG) * 32 + g) * VG + n % VG) * 16);
    dst[0] = make_float4(t[0], t[1], t[2], t[3]);
    dst[1] = make_float4(t[4], t[5], t[6], t[7]);
    dst[2] = make_float4(t[8], t[9], t[10], t[11]);
    dst[3] = make_float4(t[12], t[13], t[14], t[15]);
    if constexpr (Fmt<FMT>::XS) {
      float xs = t[15];
      xs = lane_sum<16>(xs, lane);
      if ((lane & 31) == 0) xsum[n][c] = xs;
    }
  }
  __syncthreads();
  if (!active) return;   // whole wavefronts; no barrier follows

  const int n0 = vg * VG;   // this wave's first vector
  float acc[VG];
#pragma unroll
  for (int n = 0; n < VG; ++n) acc[n] = 0.0f;
  const uint32_t tbase = lds_addr(tables) + uint32_t(vg) * (32 * VG * 64);   // 256-byte aligned
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    float A[NA][VG];
#pragma unroll
    for (int q = 0; q < NA; ++q)
#pragma unroll
      for (int n = 0; n < VG; ++n) A[q][n] = 0.0f;
    const uint32_t cbase = tbase + c * (NVG * 32 * VG * 64);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint32_t wi[P], v[NA];
#pragma unroll
      for (int p = 0; p < P; ++p) wi[p] = w[c][p][i];
      lookup_words<FMT>(wi, v);
#pragma unroll
      for (int q = 0; q < NA; ++q) word_lookups_batch<VG>(v[q], i, cbase, A[q]);
    }
#pragma unroll
    for (int n = 0; n < VG; ++n) {
      float An[NA];
#pragma unroll
      for (int q = 0; q < NA; ++q) An[q] = A[q][n];
      float xs = 0.0f;
      if constexpr (Fmt<FMT>::XS) xs = xsum[n0 + n][c];
      acc[n] = finish_chunk<FMT>(An, xs, sc[c], acc[n]);
    }
  }
#pragma unroll
  for (int n = 0; n < VG; ++n) a.partials[(size_t(n0 + n) * splits + split) * a.Npad + row] = acc[n];
}

// y[n*rows + r] = sum_s partials[n][s][r] (+ bias[r]) (+ resid[n*rows + r])
// in split order; resid may be y itself (each element is read and written
// by one thread).
__global__ __launch_bounds__(64) void batched_reduce_kernel(const float *__restrict__ partials, int splits, int Npad,
                                                            int rows, const float *__restrict__ bias,
                                                            const float *resid, float *y) {
  const int r = blockIdx.x * kWave + threadIdx.x, n = blockIdx.y;
  if (r >= rows) return;
  const float *p = partials + size_t(n) * splits * Npad + r;
  float s = 0.0f;
  for (int k0 = 0; k0 < splits; k0 += 32) {   // 32 loads in flight, summed in split order
    float v[32];
#pragma unroll
    for (int j = 0; j < 32; ++j) v[j] = k0 + j < splits ? p[size_t(k0 + j) * Npad] : 0.0f;
#pragma unroll
    for (int j = 0; j < 32; ++j) s += v[j];
  }
  if (bias) s += bias[r];
  if (resid) s += resid[size_t(n) * rows + r];
  y[size_t(n) * rows + r] = s;
}

template <int FMT, int NB>
static int launch_batch_nb(const GemvArgs &a, hipStream_t st) {
  const int row_blocks = (a.Npad + 255) / 256, splits = a.Kp / kRotChunk;
  constexpr int VG = NB >= 4 ? NB / 4 : 1;   // vectors per wave: 16 waves from 4 vectors up
  lut_gemv_batch_kernel<FMT, NB, VG>
      <<<dim3(row_blocks * splits), dim3(kWave * batch_waves<NB, VG>()), 0, st>>>(a, row_blocks, splits);
  batched_reduce_kernel<<<dim3((a.rows + kWave - 1) / kWave, NB), dim3(kWave), 0, st>>>(a.partials, splits, a.Npad,
                                                                                     a.rows, a.bias, a.resid, a.y);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? LMX_OK : fail(LMX_ERR_LAUNCH_FAILED, "batched lut_gemv launch: %s", hipGetErrorString(e));
}

template <int FMT>
static int launch_batch_fmt(const GemvArgs &a, int nb, hipStream_t st) {
  switch (nb) {
  case 2: return launch_batch_nb<FMT, 2>(a, st);
  case 4: return launch_batch_nb<FMT, 4>(a, st);
  case 8: return launch_batch_nb<FMT, 8>(a, st);
  case 16: return launch_batch_nb<FMT, 16>(a, st);
  }
  return fail(LMX_ERR_INVALID_ARGUMENT, "batch group %d (2, 4, 8 or 16)", nb);
}

int launch_gemv_batch(int fmt, const GemvArgs &a, int nb, void *stream) {
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (fmt) {
  case LMX_FMT_TERNARY: return launch_batch_fmt<LMX_FMT_TERNARY>(a, nb, st);
  case LMX_FMT_BINARY: return launch_batch_fmt<LMX_FMT_BINARY>(a, nb, st);
  case LMX_FMT_RRQ2: return launch_batch_fmt<LMX_FMT_RRQ2>(a, nb, st);
  case LMX_FMT_RRQ3: return launch_batch_fmt<LMX_FMT_RRQ3>(a, nb, st);
  case LMX_FMT_INT3: return launch_batch_fmt<LMX_FMT_INT3>(a, nb, st);
  case LMX_FMT_INT4: return launch_batch_fmt<LMX_FMT_INT4>(a, nb, st);
  case LMX_FMT_INT8: return launch_batch_fmt<LMX_FMT_INT8>(a, nb, st);
  }
  return fail(LMX_ERR_UNSUPPORTED_FORMAT, "unknown format %d", fmt);
}

int launch_gemv(int fmt, const GemvArgs &a, void *stream) {
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (fmt) {
  case LMX_FMT_TERNARY: return launch_fmt<LMX_FMT_TERNARY>(a, st);
  case LMX_FMT_BINARY: return launch_fmt<LMX_FMT_BINARY>(a, st);
  case LMX_FMT_RRQ2: return launch_fmt<LMX_FMT_RRQ2>(a, st);
  case LMX_FMT_RRQ3: return launch_fmt<LMX_FMT_RRQ3>(a, st);
  case LMX_FMT_INT3: return launch_fmt<LMX_FMT_INT3>(a, st);
  case LMX_FMT_INT4: return launch_fmt<LMX_FMT_INT4>(a, st);
  case LMX_FMT_INT8: return launch_fmt<LMX_FMT_INT8>(a, st);
  }
  return fail(LMX_ERR_UNSUPPORTED_FORMAT, "unknown format %d", fmt);
}

// ---------------------------------------------------------------------------
// Copies x[n] into an aligned buffer zero-padded to n_pad (used when the
// caller's x is not 16-byte aligned or n % 4 != 0).
__global__ __launch_bounds__(256) void stage_x_kernel(const float *__restrict__ x, size_t n, float *__restrict__ out,
                                                      size_t n_pad) {
  const size_t i = size_t(blockIdx.x) * 256 + threadIdx.x;
  if (i < n_pad) out[i] = i < n ? x[i] : 0.0f;
}

int launch_stage_x(const float *x, size_t n, float *out, size_t n_pad, void *stream) {
  stage_x_kernel<<<dim3((n_pad + 255) / 256), dim3(256), 0, static_cast<hipStream_t>(stream)>>>(x, n, out, n_pad);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(LMX_ERR_LAUNCH_FAILED, "stage_x launch: %s", hipGetErrorString(e));
  return LMX_OK;
}

// ---------------------------------------------------------------------------
// Standalone FWHT-256 (apply_hadamard_rotation): one wavefront per chunk.
__global__ __launch_bounds__(256) void fwht256_kernel(float *x, size_t n_chunks) {
  const size_t c = size_t(blockIdx.x) * 4 + threadIdx.x / kWave;
  const int lane = threadIdx.x & (kWave - 1);
  if (c >= n_chunks) return;
  float4 *p = reinterpret_cast<float4 *>(x + c * kRotChunk) + lane;
  float4 v = *p;
  fwht256_regs(v.x, v.y, v.z, v.w, lane);
  *p = v;
}

int launch_fwht256(float *x, size_t n, void *stream) {
  const size_t chunks = n / kRotChunk;
  if (chunks == 0) return LMX_OK;
  fwht256_kernel<<<dim3((chunks + 3) / 4), dim3(256), 0, static_cast<hipStream_t>(stream)>>>(x, chunks);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(LMX_ERR_LAUNCH_FAILED, "fwht256 launch: %s", hipGetErrorString(e));
  return LMX_OK;
}

// Length-n orthonormal FWHT (n a power of two, 256 <= n <= 16384) in one
// workgroup through LDS: out = H_n x / sqrt(n).
__global__ __launch_bounds__(1024) void fwht_full_kernel(const float *x, float *out, int n, float scale) {
  __shared__ float buf[16384];
  for (int i = threadIdx.x; i < n; i += blockDim.x) buf[i] = x[i];
  __syncthreads();
  for (int h = 1; h < n; h <<= 1) {
    for (int t = threadIdx.x; t < n / 2; t += blockDim.x) {
      const int j = (t / h) * 2 * h + (t % h);
      const float u = buf[j], v = buf[j + h];
      buf[j] = u + v;
      buf[j + h] = u - v;
    }
    __syncthreads();
  }
  for (int i = threadIdx.x; i < n; i += blockDim.x) out[i] = buf[i] * scale;
}

int launch_fwht_full(const float *x, float *out, size_t n, void *stream) {
  fwht_full_kernel<<<dim3(1), dim3(1024), 0, static_cast<hipStream_t>(stream)>>>(
      x, out, int(n), float(1.0 / __builtin_sqrt(double(n))));
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(LMX_ERR_LAUNCH_FAILED, "fwht_full launch: %s", hipGetErrorString(e));
  return LMX_OK;
}

// ---------------------------------------------------------------------------
// precompute_luts on the device with the GEMV's own table code.
__global__ __launch_bounds__(256) void luts_kernel(const float *x, size_t n, unsigned rotate, float *luts) {
  const size_t c = size_t(blockIdx.x) * 4 + threadIdx.x / kWave;  // 256-chunk
  const int lane = threadIdx.x & (kWave - 1);
  if (c * kRotChunk >= n) return;
  float x0, x1, x2, x3;
  const size_t k = c * kRotChunk + 4 * lane;
  if (rotate == LMX_ROTATE_FWHT256) {  // n % 256 == 0 and x aligned (checked by the host)
    load_x4(x, int(c * kRotChunk), int(n), lane, x0, x1, x2, x3);
    fwht256_regs(x0, x1, x2, x3, lane);
  } else {
    if (k + 3 >= n) return;  // whole groups only, as precompute_luts
    x0 = x[k]; x1 = x[k + 1]; x2 = x[k + 2]; x3 = x[k + 3];
  }
  float t[16];
  group_table(x0, x1, x2, x3, t);
  float *dst = luts + (k / 4) * 16;
#pragma unroll
  for (int m = 0; m < 16; ++m) dst[m] = t[m];
}

int launch_precompute_luts(const float *x, size_t n, unsigned flags, float *luts, void *stream) {
  const size_t chunks = (n + kRotChunk - 1) / kRotChunk;
  if (chunks == 0) return LMX_OK;
  luts_kernel<<<dim3((chunks + 3) / 4), dim3(256), 0, static_cast<hipStream_t>(stream)>>>(x, n, flags, luts);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(LMX_ERR_LAUNCH_FAILED, "precompute_luts launch: %s", hipGetErrorString(e));
  return LMX_OK;
}

// ---------------------------------------------------------------------------
// extract_indices on the device, with the same lookup-word and nibble
// arithmetic the ternary GEMV uses (32-bit little-endian words of canonical
// plane bytes; group 2j in the high nibble of byte j).
__global__ __launch_bounds__(256) void indices_kernel(const uint8_t *s, const uint8_t *z, size_t n_groups,
                                                      uint8_t *pos, uint8_t *neg) {
  const size_t g = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (g >= n_groups) return;
  const uint32_t w[2] = {uint32_t(s[g / 2]), uint32_t(z[g / 2])};
  uint32_t v[2];
  lookup_words<LMX_FMT_TERNARY>(w, v);
  const uint32_t sh = (g & 1) ? 0u : 4u;
  pos[g] = uint8_t((v[0] >> sh) & 15u);
  neg[g] = uint8_t((v[1] >> sh) & 15u);
}

int launch_extract_indices(const uint8_t *s, const uint8_t *z, size_t n_groups, uint8_t *pos, uint8_t *neg,
                           void *stream) {
  if (n_groups == 0) return LMX_OK;
  indices_kernel<<<dim3((n_groups + 255) / 256), dim3(256), 0, static_cast<hipStream_t>(stream)>>>(
      s, z, n_groups, pos, neg);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(LMX_ERR_LAUNCH_FAILED, "extract_indices launch: %s", hipGetErrorString(e));
  return LMX_OK;
}

}  // namespace lmx
