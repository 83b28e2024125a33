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
// in LDS), k-slices spread over its lanes, slice partials summed in LDS (a
// lane butterfly inside each wave, then the waves in order).
// Batched (lut_gemv_batch_kernel): NB = 4/8/16 vectors, 4 per wave, each
// table entry of a wave's 4 vectors side by side so that one 16-byte LDS
// read serves all 4; split-K partials summed by batched_reduce_kernel (or
// its SiLU-pair / RMSNorm-out variants).
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

#include <cstdlib>

#include "lmx_device.hpp"

namespace lmx {

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
    if (a.amax)
      wave_argmax(a.amax, blockIdx.x * WAVES + wave, argmax_value(a, out, row, active && row < a.rows), row,
                  active && row < a.rows);
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
    // Sum the partials in split order; loads go out 48 at a time so their
    // latencies overlap (one round trip up to 48 splits, K = 12288 at
    // 256-wide slices).
    constexpr int RL = 48;
    float s = 0.0f;
    const float *pr = a.partials + r;
    for (int k0s = 0; k0s < splits; k0s += RL) {
      float v[RL];
#pragma unroll
      for (int j = 0; j < RL; ++j)
        v[j] = k0s + j < splits
                   ? __hip_atomic_load(pr + size_t(k0s + j) * a.Npad, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                   : 0.0f;
#pragma unroll
      for (int j = 0; j < RL; ++j) s += v[j];
    }
    out = a.bias ? s + a.bias[r] : s;
    a.y[r] = out;
  }
  if (a.amax) wave_argmax(a.amax, rb * WAVES + wave, argmax_value(a, out, r, r < a.rows), r, r < a.rows);
  if (threadIdx.x == 0) __hip_atomic_store(a.counters + rb, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Second pass of the two-pass split-K reduction: y[r] = sum_s partials[s][r]
// (+ bias).  A workgroup covers 64 rows; its 4 wavefronts each sum a quarter
// of the splits with independent loads, then wave 0 adds the four quarters
// in a fixed order.
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float *__restrict__ partials, int splits, int Npad,
                                                            int rows, const float *__restrict__ bias,
                                                            float *__restrict__ y, unsigned long long *amax,
                                                            const unsigned *__restrict__ pcount, float penalty) {
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
    if (amax)
      wave_argmax(amax, blockIdx.x, pcount && r < rows ? penalised_logit(t, pcount[r], penalty) : t, r, r < rows);
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
// into other banks (the shift rides in bits 6-7 of the nibble byte); with
// H = 8 four slices share a pass and the same shift halves their overlap.  At the
// end the NS = WAVES*H slice partials of each row are summed in slice order.
template <int WAVES, int H, int CPS>
constexpr uint32_t fullk_prefix_bytes() {
  return (uint32_t(WAVES * H * CPS + WAVES * kWave) * 4 + 255) / 256 * 256;
}

// The lean kernel's prefix: as fullk_prefix_bytes, or with a plane split
// only the WAVES x (rows per workgroup) slice sums it writes (the layered
// plan's 70 chunk blocks leave 2.5 KB of the 160 KB)
template <int WAVES, int H, int CPS, bool PS>
constexpr uint32_t plain_prefix_bytes() {
  if constexpr (PS) return (uint32_t(WAVES * H * CPS + WAVES * (kWave / H / 2)) * 4 + 255) / 256 * 256;
  return fullk_prefix_bytes<WAVES, H, CPS>();
}

template <int H>
__device__ __forceinline__ uint32_t slice_shift(int s) {
  return ((H == 4 || H == 8) && (s & 1)) ? 64u : 0u;
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
  if (a.amax && threadIdx.x < kWave)
    wave_argmax(a.amax, blockIdx.x, argmax_value(a, t, r, threadIdx.x < RW && r < a.rows), r,
                threadIdx.x < RW && r < a.rows);
}

// Full-K kernel with a lean front end: the same geometry, lookups and
// slice reduction as lut_gemv_fullk_kernel, staggered tables, weight and
// scale addresses in 32-bit offsets with a shift for the scale group, x
// rotated (ROT) without its final 1/16 (folded into the scales), every wave
// building the tables of its own 256-chunks only, and the activation
// transform XM (kXMode*) and the epilogue EPI (kEpi*) fixed at compile
// time.  Needs H*CPS even (each wave owns whole 256-chunks).  No argmax
// epilogue.
// LAY (layered): slice s owns chunks s, s + NS, s + 2 NS, ... (not CPS
// consecutive ones), and chunk ch keeps its tables at ch * kIplChunkBytes,
// back to back: the last layer may be ragged (K = 8960 = 70 chunks on 64
// slices: 6 slices do two chunks), and 70 chunks' tables fit the LDS.
template <int FMT, bool ROT, int WAVES, int H, int CPS, int XM, int EPI = kEpiStore, bool LAY = false, bool PS = false>
__global__ __launch_bounds__(WAVES * kWave) void lut_gemv_plain_kernel(GemvArgs a) {
  constexpr int P = Fmt<FMT>::P, NA = Fmt<FMT>::NA, S = Fmt<FMT>::S;
  // PS (4-bit): the four planes of a row's chunk split over two lanes, planes
  // 0-1 and 2-3 (half the lookups per lane, half the rows per workgroup)
  static_assert(!PS || (FMT == LMX_FMT_INT4 && EPI == kEpiStore), "plane split: 4-bit, plain store");
  constexpr int RW = kWave / H / (PS ? 2 : 1);
  constexpr bool PAIR = EPI == kEpiSiluPair;
  constexpr int HR = RW / 2;   // PAIR: gate rows (then as many up rows) per workgroup
  constexpr int NS = WAVES * H;
  constexpr uint32_t SSTRIDE = stag_slice_bytes(CPS);
  constexpr int XJ = H * CPS / 2;
  static_assert(!LAY || H % 2 == 0, "layered: whole 256-chunks per wave and layer");
  static_assert(H * CPS % 2 == 0, "whole 256-chunks per wave");
  constexpr uint32_t PREFIX = plain_prefix_bytes<WAVES, H, CPS, PS>();
  extern __shared__ __attribute__((aligned(256))) float lds[];
  const int Kc = a.Kp / kChunk;
  const int used = (Kc + CPS - 1) / CPS;
  float *xsum = lds;
  float *red = lds + NS * CPS;
  char *tables = reinterpret_cast<char *>(lds) + PREFIX;

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int s = wave * H + (PS ? (lane / RW) >> 1 : lane / RW);
  const int part = PS ? (lane / RW) & 1 : 0;   // PS: planes 2*part, 2*part + 1
  const int rl = lane % RW;
  // PAIR: the workgroup's rows are gate rows blockIdx.x*HR + [0, HR) and the
  // up rows rows/2 + blockIdx.x*HR + [0, HR) (the host checks rows/2 % HR == 0)
  const int row = PAIR ? (rl < HR ? 0 : a.rows / 2 - HR) + blockIdx.x * HR + rl : blockIdx.x * RW + rl;
  const int lr = min(row, a.Npad - 1);

  // ---- x of this wave's 256-chunks (clamped in bounds, masked below) ----
  const int C2n = a.Kp / kRotChunk;
  const int c2base = wave * XJ;
  // the wave's j-th 256-chunk (increasing in j)
  const auto c2_of = [&](int j) { return LAY ? (j / (H / 2)) * (NS / 2) + wave * (H / 2) + j % (H / 2) : c2base + j; };
  // the chunk that slice s looks up at its step c
  const auto chunk_of = [&](int c) { return LAY ? c * NS + s : s * CPS + c; };
  constexpr bool AUX = XM == kXModeRmsNorm || XM == kXModeSiluMul;
  float4 xr[XJ], xa[XJ];
#pragma unroll
  for (int j = 0; j < XJ; ++j) {
    const int k = min(min(c2_of(j), C2n - 1) * kRotChunk + 4 * lane, a.cols - 4);
    xr[j] = *reinterpret_cast<const float4 *>(a.x + k);
    // norm weight, or the up half of a gate|up vector
    if constexpr (AUX) xa[j] = *reinterpret_cast<const float4 *>((XM == kXModeRmsNorm ? a.xw : a.x + a.cols) + k);
  }
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_barrier();   // every wave's x requests ahead of the weight stream

  // ---- weights (chunk 0 now, the rest after the prologue) and scales ----
  constexpr int PL = PS ? 2 : P;   // planes a lane loads
  u32x4 w[CPS][PL];
  float sc[CPS][S];
  const u32x4 *__restrict__ pl = reinterpret_cast<const u32x4 *>(a.planes);
  const uint32_t Npad = uint32_t(a.Npad);
  auto load_planes = [&](int c) {
    const uint32_t ch = uint32_t(min(chunk_of(c), Kc - 1));
#pragma unroll
    for (int p = 0; p < PL; ++p)
      w[c][p] = __builtin_nontemporal_load(pl + ((ch * P + uint32_t(PS ? 2 * part + p : p)) * Npad + uint32_t(lr)));
  };
  load_planes(0);
#pragma unroll
  for (int c = 0; c < CPS; ++c) {
    const int ch = min(chunk_of(c), Kc - 1);
    const int g = a.gshift >= 0 ? ch >> a.gshift : ch / a.group_chunks;
#pragma unroll
    for (int t = 0; t < S; ++t) sc[c][t] = a.scales[(uint32_t(t * a.n_groups + g)) * Npad + uint32_t(lr)];
  }
  // the epilogue thread's bias term (the decoder's residual rides there),
  // requested with the weights so that its round trip overlaps the lookups
  // (not for the SiLU pair, whose gate|up carries no residual: two live
  // registers there cost a workgroup per CU)
  float eb0 = 0.0f;
  if constexpr (!PAIR) {
    if (threadIdx.x < RW && a.bias) {
      const int r = blockIdx.x * RW + threadIdx.x;
      if (r < a.rows) eb0 = a.bias[r];
    }
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
      mask_x4(xr[j], c2_of(j) * kRotChunk, a.cols, lane, x0, x1, x2, x3);
      if (c2_of(j) < C2n) ss += (x0 * x0 + x1 * x1) + (x2 * x2 + x3 * x3);
    }
    inv_rms = wg_inv_rms_from<WAVES * kWave>(ss, a.cols, a.eps, red);
  }

  // ---- prologue: (transform) -> (FWHT-256 x16) -> group tables of this wave's chunks ----
  const uint32_t goff = group_offset<true>(lane & 31);
#pragma unroll
  for (int j = 0; j < XJ; ++j) {
    const int c2 = c2_of(j);
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
    const int ts = LAY ? ch % NS : ch / CPS;   // the slice that looks it up
    float4 *dst = reinterpret_cast<float4 *>(
        tables + (LAY ? ch * kIplChunkBytes : ts * SSTRIDE + (ch % CPS) * kStagChunkBytes) + slice_shift<H>(ts) + goff);
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
    const uint32_t tbase = lds_addr(lds) + PREFIX + (LAY ? 0u : min(s, used - 1) * SSTRIDE);
    const uint32_t shift = slice_shift<H>(s) * 0x01010101u;
#pragma unroll
    for (int c = 0; c < CPS; ++c) {
      const int ch = chunk_of(c);
      float scl[S];
#pragma unroll
      for (int t = 0; t < S; ++t) scl[t] = sc[c][t] * kScale;
      if constexpr (PS) {
        // two planes as a 2-plane format; the third plane of the 4-bit
        // identity enters inverted, and the part's terms of
        // ((A0 + 2 A1) + 4 A2) - 8 A3 weight its two sums
        u32x4 wl[2] = {w[c][0], w[c][1]};
        const uint32_t inv = part ? 0xFFFFFFFFu : 0u;
        wl[1].x ^= inv;
        wl[1].y ^= inv;
        wl[1].z ^= inv;
        wl[1].w ^= inv;
        float A2[2] = {0.0f, 0.0f};
        if constexpr (LAY)
          chunk_lookups<LMX_FMT_RRQ2, true>(wl, tbase + uint32_t(min(chunk_of(c), Kc - 1)) * kIplChunkBytes, shift, A2);
        else
          chunk_lookups<LMX_FMT_RRQ2, true>(wl, tbase, shift, A2, c * kStagChunkBytes);
        const float c0 = part ? 4.0f : 1.0f, c1 = part ? -8.0f : 2.0f;
        const float nacc = fmaf(scl[0], c0 * A2[0] + c1 * A2[1], acc);
        acc = ch < Kc ? nacc : acc;
      } else {
        float A[NA];
#pragma unroll
        for (int i = 0; i < NA; ++i) A[i] = 0.0f;
        if constexpr (LAY)
          chunk_lookups<FMT, true>(w[c], tbase + uint32_t(min(chunk_of(c), Kc - 1)) * kIplChunkBytes, shift, A);
        else
          chunk_lookups<FMT, true>(w[c], tbase, shift, A, c * kStagChunkBytes);
        float xs = 0.0f;
        if constexpr (Fmt<FMT>::XS) xs = xsum[min(ch, Kc - 1)];
        const float nacc = finish_chunk<FMT>(A, xs, scl, acc);
        acc = ch < Kc ? nacc : acc;
      }
    }
  }

  // ---- in-workgroup reduction: a wave's H slices of a row by a lane
  // butterfly, then the waves in order (fixed, so deterministic) -----------
  {
    const float wsum = strided_sum<RW>(acc, lane);
    if (lane < RW) red[wave * RW + rl] = wsum;
  }
  __syncthreads();
  if constexpr (PAIR) {
    if (threadIdx.x < HR) {
      const int j = blockIdx.x * HR + threadIdx.x;
      float g = 0.0f, u = 0.0f;
#pragma unroll 8
      for (int k = 0; k < WAVES; ++k) {
        g += red[k * RW + threadIdx.x];
        u += red[k * RW + HR + threadIdx.x];
      }
      if (a.bias) g += a.bias[j], u += a.bias[a.rows / 2 + j];
      a.y[j] = silu(g) * u;
    }
  } else if (threadIdx.x < RW) {
    const int r = blockIdx.x * RW + threadIdx.x;
    float t = 0.0f;
#pragma unroll 8
    for (int k = 0; k < WAVES; ++k) t += red[k * RW + threadIdx.x];
    if (r < a.rows) a.y[r] = a.bias ? t + eb0 : t;
  }
}

// Interleaved variant of the plain kernel (two k-slices per wave, H = 2):
// wave w owns the 256-chunks c2 = w*CPS + c, c < CPS, and at step c its
// lower / upper half-wave looks up 128-chunk 2*c2 / 2*c2 + 1, exactly the two
// halves of the 256-chunk it has just rotated.  So every step is "build the
// tables of one 256-chunk, then look them up", and the VALU-heavy table
// build of one wave overlaps the LDS-heavy lookups of the others.  Chunk ch
// keeps its (staggered) tables at ch * kIplChunkBytes, a 256-byte multiple.

template <int WAVES, int CPS>
constexpr uint32_t ipl_prefix_bytes() {
  return (uint32_t(2 * WAVES * CPS + 2 * WAVES * (kWave / 2)) * 4 + 255) / 256 * 256;
}

template <int FMT, bool ROT, int WAVES, int CPS>
__global__ __launch_bounds__(WAVES * kWave) void lut_gemv_ipl_kernel(GemvArgs a) {
  constexpr int P = Fmt<FMT>::P, NA = Fmt<FMT>::NA, S = Fmt<FMT>::S;
  constexpr int RW = kWave / 2;
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
  // A wave still on its first step outranks the waves past it (priority 1,
  // dropped once its later steps' loads are out).  The SIMD otherwise serves
  // its oldest waves first, so the youngest wave of each SIMD looked up its
  // first step last and only then requested the rest: its late loads and a
  // tail of lookups alone on the SIMD ended the kernel (measured: int4 8192^2
  // -4.5 %, ternary -8.7 %, binary -5 %, same bits).
  // AGE: past the first step the younger waves outrank the older ones
  // (priority wave / 4, the first step at 3), so the wave whose weights
  // came last is not also served last; measured int4 -1.1 %, int8 -1.6 %,
  // RRQ-2 -1.9 %, RRQ-3 -2.5 %, but ternary +1.3 % and binary +2.2 %.
  constexpr bool AGE = FMT != LMX_FMT_TERNARY && FMT != LMX_FMT_BINARY;
  if constexpr (AGE)
    __builtin_amdgcn_s_setprio(3);
  else
    __builtin_amdgcn_s_setprio(1);
  const int wave_s = __builtin_amdgcn_readfirstlane(wave);
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
    // A wave reads only the tables it wrote; its LDS operations complete in order.
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
    // ---- lookups of 128-chunk 2*c2 + h ----
    const int ch = 2 * c2 + h;
    float A[NA];
#pragma unroll
    for (int i = 0; i < NA; ++i) A[i] = 0.0f;
    chunk_lookups<FMT, true>(w[c], tb + uint32_t(ch) * kIplChunkBytes, 0u, A);
    if (c == 0) {
      // The later chunks' loads go out only now: a wave whose load issue
      // stalls on a full memory queue cannot run its lookups, so issuing them
      // before this chunk's lookups held those lookups back until the HBM
      // stream drained (measured: int4 8192^2 -0.5 us, ternary -0.35 us).
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int cc = 1; cc < CPS; ++cc) load_planes(cc);
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (AGE) {
        // priority wave / 4, in one asm block: a branch on the wave index
        // here splits the unrolled step loop and the compiler spills
        asm volatile(
            "s_setprio 0\n"
            "s_cmp_ge_u32 %0, 4\n"
            "s_cbranch_scc0 1f\n"
            "s_setprio 1\n"
            "s_cmp_ge_u32 %0, 8\n"
            "s_cbranch_scc0 1f\n"
            "s_setprio 2\n"
            "s_cmp_ge_u32 %0, 12\n"
            "s_cbranch_scc0 1f\n"
            "s_setprio 3\n"
            "1:" ::"s"(wave_s)
            : "scc");
      } else {
        __builtin_amdgcn_s_setprio(0);
      }
    }
    float xs = 0.0f;
    if constexpr (Fmt<FMT>::XS) xs = xsum[min(ch, Kc - 1)];
    float scl[S];
#pragma unroll
    for (int t = 0; t < S; ++t) scl[t] = sc[c][t] * kScale;
    const float nacc = finish_chunk<FMT>(A, xs, scl, acc);
    acc = ch < Kc ? nacc : acc;
  }

  // ---- in-workgroup reduction: the two half-wave slices of a row by a
  // lane swap, then the waves in order (fixed, so deterministic) ----------
  {
    const float wsum = strided_sum<RW>(acc, lane);
    if (h == 0) red[wave * RW + rl] = wsum;
  }
  __syncthreads();
  if (threadIdx.x < RW) {
    const int r = blockIdx.x * RW + threadIdx.x;
    float t = 0.0f;
#pragma unroll 8
    for (int k = 0; k < WAVES; ++k) t += red[k * RW + threadIdx.x];
    if (r < a.rows) a.y[r] = a.bias ? t + a.bias[r] : t;
  }
}

template <int WAVES, int H, int CPS, bool LAY = false, bool PS = false>
constexpr size_t plain_lds_bytes(size_t Kc) {
  return plain_prefix_bytes<WAVES, H, CPS, PS>() +
         (LAY ? Kc * kIplChunkBytes : (Kc + CPS - 1) / CPS * stag_slice_bytes(CPS));
}

template <int FMT, bool ROT, int WAVES, int H, int CPS, int XM, int EPI = kEpiStore, bool LAY = false, bool PS = false>
static int launch_plain_kernel(const GemvArgs &a, hipStream_t st) {
  const size_t lds = plain_lds_bytes<WAVES, H, CPS, LAY, PS>(size_t(a.Kp / kChunk));
  if (lds > kMaxLdsBytes) return 1;   // staggered tables do not fit: the generic kernel serves it
  static const hipError_t attr = hipFuncSetAttribute(
      reinterpret_cast<const void *>(&lut_gemv_plain_kernel<FMT, ROT, WAVES, H, CPS, XM, EPI, LAY, PS>),
      hipFuncAttributeMaxDynamicSharedMemorySize, int(kMaxLdsBytes));
  if (attr != hipSuccess) return fail(LMX_ERR_LAUNCH_FAILED, "hipFuncSetAttribute: %s", hipGetErrorString(attr));
  constexpr int RW = kWave / H / (PS ? 2 : 1);
  const int blocks = EPI == kEpiSiluPair ? a.rows / RW : (a.Npad + RW - 1) / RW;
  lut_gemv_plain_kernel<FMT, ROT, WAVES, H, CPS, XM, EPI, LAY, PS><<<dim3(blocks), dim3(WAVES * kWave), lds, st>>>(a);
  return LMX_OK;
}

// Unrotated 4-bit launches of the 4 x 4 x 1 and 16 x 4 x 1 plans split each
// chunk's planes over two lanes (plane_split_level(): 1, the default; 2 the
// 4 x 4 x 1 plan only; 0 neither).  Splitting the 8 x 8 x 1 plan as well
// (4 rows per workgroup, each building the whole K's tables) measured 9 %
// slower in Llama decode, so the plan chooser takes 16 x 4 x 1 with 8 rows
// per workgroup there instead (choose_fullk).
template <int WAVES, int H, int CPS, bool LAY>
static bool plane_split_plan() {
  if constexpr (LAY || CPS != 1) return false;
  if constexpr (WAVES == 4 && H == 4) return plane_split_level() >= 1;
  if constexpr (WAVES == 16 && H == 4) return plane_split_level() == 1;
  return false;
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

template <int FMT, int WAVES, int H, int CPS, bool LAY = false>
static int launch_plain_cfg(const GemvArgs &a, hipStream_t st) {
  // Interleaved where it measured faster: two k-slices per wave and at least
  // two steps per wave (one step has nothing to interleave; 17920 x 1536
  // ran 40% slower that way).  RRQ-3 too since the first-step priority
  // (8192^2 -1.6 %; it had been 4 % slower).
  if (a.epi == kEpiSiluPair) {
    // gate|up of the decode step: RMSNorm in, SiLU(gate)*up out (4-bit, unrotated)
    if constexpr (FMT == LMX_FMT_INT4)
      if (a.rotate == LMX_ROTATE_NONE && a.xmode == kXModeRmsNorm && a.rows % (kWave / H) == 0)
        return launch_plain_kernel<FMT, false, WAVES, H, CPS, kXModeRmsNorm, kEpiSiluPair, LAY>(a, st);
    return 1;
  }
  if (a.xmode != kXModeNone) {
    // Fused transforms on the lean kernel: the decode step's linears (4-bit,
    // unrotated); other formats take the generic kernel.
    if constexpr (FMT == LMX_FMT_INT4) {
      if (a.rotate == LMX_ROTATE_NONE) {
        if constexpr (!LAY && CPS == 1)
          if (a.xmode == kXModeRmsNorm && plane_split_plan<WAVES, H, CPS, LAY>())
            return launch_plain_kernel<FMT, false, WAVES, H, CPS, kXModeRmsNorm, kEpiStore, LAY, true>(a, st);
        switch (a.xmode) {
        case kXModeRmsNorm: return launch_plain_kernel<FMT, false, WAVES, H, CPS, kXModeRmsNorm, kEpiStore, LAY>(a, st);
        case kXModeSiluMul: return launch_plain_kernel<FMT, false, WAVES, H, CPS, kXModeSiluMul, kEpiStore, LAY>(a, st);
        }
      }
    }
    return 1;
  }
  if constexpr (!LAY && H == 2 && CPS >= 2) {
    if (a.kfamily != kKernelLean) {
      const int r = a.rotate == LMX_ROTATE_FWHT256 ? launch_ipl_kernel<FMT, true, WAVES, CPS>(a, st)
                                                   : launch_ipl_kernel<FMT, false, WAVES, CPS>(a, st);
      if (r != 1) return r;
    }
  }
  if (a.rotate == LMX_ROTATE_FWHT256) return launch_plain_kernel<FMT, true, WAVES, H, CPS, kXModeNone, kEpiStore, LAY>(a, st);
  if constexpr (FMT == LMX_FMT_INT4 && !LAY && CPS == 1)
    if (plane_split_plan<WAVES, H, CPS, LAY>())
      return launch_plain_kernel<FMT, false, WAVES, H, CPS, kXModeNone, kEpiStore, LAY, true>(a, st);
  return launch_plain_kernel<FMT, false, WAVES, H, CPS, kXModeNone, kEpiStore, LAY>(a, st);
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
  case kFullK_8x8x1: return launch_plain_cfg<FMT, 8, 8, 1>(a, st);
  case kFullK_8x8x2L:
    if constexpr (FMT == LMX_FMT_INT4) {
      // unrotated, plain store: 16 waves x 4 slices x 2 layered chunks with
      // the planes split over two lanes (the same 8 rows per workgroup and
      // chunk tables; four waves per SIMD, half the lookups per lane)
      if (a.rotate == LMX_ROTATE_NONE && a.epi == kEpiStore && plane_split_level() == 1) {
        switch (a.xmode) {
        case kXModeNone: return launch_plain_kernel<FMT, false, 16, 4, 2, kXModeNone, kEpiStore, true, true>(a, st);
        case kXModeRmsNorm: return launch_plain_kernel<FMT, false, 16, 4, 2, kXModeRmsNorm, kEpiStore, true, true>(a, st);
        case kXModeSiluMul: return launch_plain_kernel<FMT, false, 16, 4, 2, kXModeSiluMul, kEpiStore, true, true>(a, st);
        }
      }
      return launch_plain_cfg<FMT, 8, 8, 2, true>(a, st);
    }
    return 1;
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
  case kFullK_8x8x1: return launch_fullk_cfg<FMT, 8, 8, 1>(a, st);
  case kFullK_8x8x2L:
    return fail(LMX_ERR_INVALID_ARGUMENT, "the layered 8 x 8 x 2 plan has no form for this format and transform");
  }
  return fail(LMX_ERR_INVALID_ARGUMENT, "unknown full-K configuration %d", a.fullk);
}

template <int FMT>
static int launch_fmt(const GemvArgs &a, hipStream_t st) {
  if (a.epi != kEpiStore && silu_pair_rows(FMT, a) == 0)
    return fail(LMX_ERR_INVALID_ARGUMENT, "the SiLU-pair epilogue is not served for this weight and transform");
  if (a.fullk) {
    int r = 1;
    if (!a.amax && a.kfamily != kKernelGeneric) r = launch_plain<FMT>(a, st);
    if (r == 1 && a.fullk == kFullK_8x8x2L) {
      // the layered plan has no generic form (argmax epilogue, a transform
      // with rotation): the split-K kernel, whose scratch every handle holds
      GemvArgs b = a;
      b.fullk = kFullK_None;
      return launch_fmt<FMT>(b, st);
    }
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
                                                                                  a.rows, a.bias, a.y, a.amax,
                                                                                  a.pcount, a.penalty);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(LMX_ERR_LAUNCH_FAILED, "lut_gemv launch: %s", hipGetErrorString(e));
  return LMX_OK;
}

int silu_pair_rows(int fmt, const GemvArgs &a) {
  if (fmt != LMX_FMT_INT4 || a.rotate != LMX_ROTATE_NONE || a.xmode != kXModeRmsNorm || a.amax ||
      a.kfamily == kKernelGeneric)
    return 0;
  const size_t Kc = size_t(a.Kp / kChunk);
  size_t lds = 0;
  switch (a.fullk) {
  case kFullK_16x2x2: lds = plain_lds_bytes<16, 2, 2>(Kc); break;
  case kFullK_16x2x3: lds = plain_lds_bytes<16, 2, 3>(Kc); break;
  case kFullK_8x2x1: lds = plain_lds_bytes<8, 2, 1>(Kc); break;
  case kFullK_16x4x1: lds = plain_lds_bytes<16, 4, 1>(Kc); break;
  case kFullK_4x4x1: lds = plain_lds_bytes<4, 4, 1>(Kc); break;
  case kFullK_8x8x1: lds = plain_lds_bytes<8, 8, 1>(Kc); break;
  case kFullK_8x8x2L: lds = plain_lds_bytes<8, 8, 2, true>(Kc); break;
  default: return 0;   // split-K, or a configuration only the generic kernel serves
  }
  const int rw = kWave / fullk_shape(a.fullk).h;
  return lds <= kMaxLdsBytes && a.rows % rw == 0 ? rw / 2 : 0;
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
// workgroup owns 64*RG rows and a k-slice of 256 with RG * NB/VG waves: wave
// w serves row group w % RG (one row per lane) for vectors (w / RG)*VG ..
// (w / RG)*VG + VG - 1, so the LDS lookups of many vectors have enough waves
// to hide their latency (the weight words of a row group are read by NB/VG
// waves: one HBM read, the rest cache hits).  RG (1, 2 or 4) is the largest
// that still gives the grid a workgroup per CU, so small matrices spread
// over the chip.  The tables of a vector group sit together per group:
// group g of (chunk c, vector group v) starts at batch_chunk_bytes<VG>() *
// (c*NB/VG + v) + g*GS, GS = VG*64 + 16 (every chunk base 256-byte aligned),
// and holds entry m of its vector b at m*4*VG + 4*b, so one v_perm address
// (nibble * 4*VG) and one 8- or 16-byte LDS read serve a wave's VG vectors;
// the 16 B pad spreads the table writes of consecutive groups over the
// banks.  Partials [NB][splits][Npad] go through batched_reduce_kernel.
constexpr int kBatchMinGrid = 256;   // workgroups: one per CU

template <int VG>
constexpr uint32_t batch_group_stride() { return uint32_t(VG) * 64 + 16; }
template <int VG>
constexpr uint32_t batch_chunk_bytes() { return 32 * batch_group_stride<VG>(); }   // a multiple of 256

template <int VG>
__device__ __forceinline__ void word_lookups_batch(uint32_t v, int i, uint32_t cbase, float *out) {
  constexpr uint32_t GS = batch_group_stride<VG>();
  if constexpr (VG == 1) {
    const uint32_t hi = (v >> 2) & 0x3C3C3C3Cu, lo = (v << 2) & 0x3C3C3C3Cu;
    float t[8];
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      t[2 * b] = lds_load(__builtin_amdgcn_perm(cbase, hi, 0x0C060500u | b) + uint32_t(8 * i + 2 * b) * GS);
      t[2 * b + 1] = lds_load(__builtin_amdgcn_perm(cbase, lo, 0x0C060500u | b) + uint32_t(8 * i + 2 * b + 1) * GS);
    }
    out[0] += ((t[0] + t[1]) + (t[2] + t[3])) + ((t[4] + t[5]) + (t[6] + t[7]));
  } else {
    // entry m of the group's VG vectors sits at m * 4*VG: the nibble times
    // 4*VG is the byte offset, and one 8- or 16-byte read returns the entry
    // of every vector of the group
    constexpr uint32_t SH = VG == 2 ? 1 : 0;   // nibble << 3 (VG 2) or << 4 (VG 4)
    constexpr uint32_t MASK = VG == 2 ? 0x78787878u : 0xF0F0F0F0u;
    const uint32_t hi = (v >> SH) & MASK, lo = (v << (4 - SH)) & MASK;
    uint32_t ad[8];
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      ad[2 * b] = __builtin_amdgcn_perm(cbase, hi, 0x0C060500u | b) + uint32_t(8 * i + 2 * b) * GS;
      ad[2 * b + 1] = __builtin_amdgcn_perm(cbase, lo, 0x0C060500u | b) + uint32_t(8 * i + 2 * b + 1) * GS;
    }
    float t[8][VG];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if constexpr (VG == 2) {
        const f32x2 e = lds_load2(ad[j]);
        t[j][0] = e.x, t[j][1] = e.y;
      } else {
        const f32x4 e = lds_load4(ad[j]);
        t[j][0] = e.x, t[j][1] = e.y, t[j][2] = e.z, t[j][3] = e.w;
      }
    }
#pragma unroll
    for (int n = 0; n < VG; ++n)
      out[n] += ((t[0][n] + t[1][n]) + (t[2][n] + t[3][n])) + ((t[4][n] + t[5][n]) + (t[6][n] + t[7][n]));
  }
}

template <int NB, int VG, int RG>
constexpr int batch_waves() { return RG * (NB / VG); }

// XM = kXModeRmsNorm (groups of 4 vectors): each wave also reads the whole
// row of its vectors for the sum of squares (every workgroup, so the
// k-slices need no exchange) and the tables take x * inv_rms * xw
// (norm.cpp:18-34).
// CH = 2: 256-wide k-slices; CH = 1: 128-wide (twice the workgroups for
// small matrices), the workgroup rotating the 256-chunk that holds its slice
// and keeping the tables of its half.
template <int FMT, int NB, int VG, int RG, int XM = kXModeNone, int CH = 2>
__global__ __launch_bounds__((kWave * batch_waves<NB, VG, RG>())) void lut_gemv_batch_kernel(GemvArgs a,
                                                                                          int row_blocks,
                                                                                          int splits) {
  constexpr int P = Fmt<FMT>::P, NA = Fmt<FMT>::NA, S = Fmt<FMT>::S;
  static_assert(CH == 1 || CH == 2, "128- or 256-wide k-slices");
  constexpr int NW = batch_waves<NB, VG, RG>();
  constexpr int NVG = NB / VG;
  constexpr int ROWS = RG * kWave;
  constexpr uint32_t GS = batch_group_stride<VG>(), CB = batch_chunk_bytes<VG>();
  static_assert(NB % VG == 0 && NW <= 16, "whole vector groups, at most 1024 threads");
  __shared__ __attribute__((aligned(256))) char tables[CH * NVG * CB];
  __shared__ float xsum[NB][CH];
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  const int rg = wave % RG, vg = wave / RG;
  const int rb = blockIdx.x % row_blocks, split = blockIdx.x / row_blocks;
  const int c0 = split * CH;                        // the slice's first 128-chunk
  const int k0 = (c0 / 2) * kRotChunk;              // the 256-chunk that holds it
  const int row = rb * ROWS + rg * kWave + lane;
  const bool active = rb * ROWS + rg * kWave < a.Npad;
  const int lr = min(row, a.Npad - 1);

  // activations: wave w builds the tables of vectors w, w + NW, ...
  constexpr int XV = (NB + NW - 1) / NW;
  constexpr bool NORM = XM == kXModeRmsNorm;
  constexpr int RL = NORM ? 8 : 1;   // row loads in flight per lane and vector (2048 columns)
  static_assert(XM == kXModeNone || (NORM && NB == 4), "RMSNorm for groups of 4 vectors");
  float xv[XV][4], xw[4];
  float4 rv[NORM ? XV : 1][RL];
#pragma unroll
  for (int j = 0; j < XV; ++j) {
    const int n = min(wave + NW * j, NB - 1);
    load_x4(a.x + size_t(n) * a.cols, k0, a.cols, lane, xv[j][0], xv[j][1], xv[j][2], xv[j][3]);
    if constexpr (NORM) {
#pragma unroll
      for (int u = 0; u < RL; ++u)
        rv[j][u] = *reinterpret_cast<const float4 *>(a.x + size_t(n) * a.cols + min(u * kRotChunk + 4 * lane, a.cols - 4));
    }
  }
  if constexpr (NORM) load_x4(a.xw, k0, a.cols, lane, xw[0], xw[1], xw[2], xw[3]);
  __builtin_amdgcn_sched_barrier(0);
  u32x4 w[CH][P];
  float sc[CH][S];
  {
    const u32x4 *__restrict__ pl = reinterpret_cast<const u32x4 *>(a.planes);
    const size_t Npad = size_t(a.Npad);
#pragma unroll
    for (int c = 0; c < CH; ++c) {
#pragma unroll
      for (int p = 0; p < P; ++p) {
        const u32x4 *src = pl + (size_t(c0 + c) * P + p) * Npad + lr;
        // one wave per row group streams; the others re-read through the caches
        w[c][p] = NVG == 1 ? __builtin_nontemporal_load(src) : *src;
      }
      const int g = (c0 + c) / a.group_chunks;
#pragma unroll
      for (int t = 0; t < S; ++t) sc[c][t] = a.scales[(size_t(t) * a.n_groups + g) * Npad + lr];
    }
  }
  // RMSNorm: the sum of squares of each vector's whole row (the loads above
  // cover 2048 columns, later rounds the rest)
  float inv_rms[XV];
#pragma unroll
  for (int j = 0; j < XV; ++j) inv_rms[j] = 1.0f;
  if constexpr (NORM) {
#pragma unroll
    for (int j = 0; j < XV; ++j) {
      const int n = min(wave + NW * j, NB - 1);
      float ss = 0.0f;
      for (int r0 = 0; r0 < a.cols; r0 += RL * kRotChunk) {
        if (r0 > 0) {
#pragma unroll
          for (int u = 0; u < RL; ++u)
            rv[j][u] = *reinterpret_cast<const float4 *>(a.x + size_t(n) * a.cols +
                                                         min(r0 + u * kRotChunk + 4 * lane, a.cols - 4));
        }
#pragma unroll
        for (int u = 0; u < RL; ++u) {
          const float4 v = rv[j][u];
          if (r0 + u * kRotChunk + 4 * lane < a.cols) ss += (v.x * v.x + v.y * v.y) + (v.z * v.z + v.w * v.w);
        }
      }
      ss = lane_sum<32>(ss, lane);
      inv_rms[j] = 1.0f / sqrtf(ss / float(a.cols) + a.eps);
    }
  }
#pragma unroll
  for (int j = 0; j < XV; ++j) {
    const int n = wave + NW * j;
    if (n >= NB) break;   // wave-uniform
    float x0 = xv[j][0], x1 = xv[j][1], x2 = xv[j][2], x3 = xv[j][3];
    if constexpr (NORM) xform4(kXModeRmsNorm, inv_rms[j], xw, x0, x1, x2, x3);
    if (a.rotate == LMX_ROTATE_FWHT256) fwht256_regs(x0, x1, x2, x3, lane);
    float t[16];
    group_table(x0, x1, x2, x3, t);
    const int half = lane >> 5, g = lane & 31;
    const int c = CH == 2 ? half : 0;              // table slot
    const bool keep = CH == 2 || half == (c0 & 1);   // CH = 1: the slice's half only
    if (keep) {
      if constexpr (VG == 1) {
        float4 *dst = reinterpret_cast<float4 *>(tables + (c * NVG + n / VG) * CB + g * GS);
        dst[0] = make_float4(t[0], t[1], t[2], t[3]);
        dst[1] = make_float4(t[4], t[5], t[6], t[7]);
        dst[2] = make_float4(t[8], t[9], t[10], t[11]);
        dst[3] = make_float4(t[12], t[13], t[14], t[15]);
      } else {
        float *dst = reinterpret_cast<float *>(tables + (c * NVG + n / VG) * CB + g * GS) + n % VG;
#pragma unroll
        for (int m = 0; m < 16; ++m) dst[m * VG] = t[m];
      }
    }
    if constexpr (Fmt<FMT>::XS) {
      float xs = t[15];
      xs = lane_sum<16>(xs, lane);
      if ((lane & 31) == 0 && keep) xsum[n][c] = xs;
    }
  }
  __syncthreads();
  if (!active) return;   // whole wavefronts; no barrier follows

  const int n0 = vg * VG;   // this wave's first vector
  float acc[VG];
#pragma unroll
  for (int n = 0; n < VG; ++n) acc[n] = 0.0f;
  const uint32_t tbase = lds_addr(reinterpret_cast<const float *>(tables)) + uint32_t(vg) * CB;   // 256-byte aligned
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    float A[NA][VG];
#pragma unroll
    for (int q = 0; q < NA; ++q)
#pragma unroll
      for (int n = 0; n < VG; ++n) A[q][n] = 0.0f;
    const uint32_t cbase = tbase + uint32_t(c * NVG) * CB;
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

// Batched 4-bit GEMV on the matrix cores (int4, unrotated, up to 16
// vectors): the same k-slices, grid and partials as lut_gemv_batch_kernel,
// so its reductions and epilogues consume them unchanged.  A wave owns 16
// rows of the slice; v_mfma_f32_16x16x16_bf16 takes A = the 16 rows' codes
// plus 16 (16..31: bf16 0x4180 | q << 3, exact) and B = the vectors split
// into three bf16 parts (x = hi + mid + lo exactly: hi and mid the top 8
// significant bits of x and of x - hi, lo the at most 8 bits left), so every
// product is exact and the sums accumulate in fp32; each 128-chunk's sum
// less 24 times the chunk's sum of x is scaled by its group scale in fp32
// (int4_gemv, lut_gemm_scalar.cpp:186-222: y = sum_b s_b sum_i (q_i - 8) x_i).  Lane (i, kq) of a 16 x 16 x 16 step
// holds row i's codes of 4 k (A) and vector i's 4 activations (B), lane
// layout A[i][k] -> lane i + 16 (k / 4), item k % 4; B[k][j] -> lane
// j + 16 (k / 4); D[i][j] -> lane j + 16 (i / 4), item i % 4.  k-block
// kb = 2m + h of a slice takes the 4-groups g = 8m + 2kq + h: lane kq's
// byte kq of word m of each plane holds its nibbles of both h, and item e
// is k = 4g + 3 - e (the nibble's bit e, MSB-first planes).
// NIB: the codes come from the handle's nibble_tiles copy (a.nib): lane
// (i, kq) reads its 16 bytes of each 128-chunk in one load, k-block kb's
// items e = 0..3 are k = 16 kb + 4 kq + e (bytes 2 kb, 2 kb + 1: two codes
// each), and bf16(q + 16) of a byte's two codes is one multiply by 0x8008
// and one and-or, no transpose.
template <int NB, int CH, int NW, int RT, bool NIB = false>
__global__ __launch_bounds__(kWave * NW) void lut_gemv_mfma_kernel(GemvArgs a, int row_blocks, int splits, int xmap) {
  typedef short v4s __attribute__((ext_vector_type(4)));
  typedef float v4f __attribute__((ext_vector_type(4)));
  constexpr int KB = 8 * CH;   // 16-k blocks per slice
  static_assert(NB >= 1 && NB <= 16 && (CH == 1 || CH == 2) && (RT == 1 || RT == 2),
                "up to 16 vectors, 128- or 256-wide slices, 1 or 2 row tiles per wave");
  __shared__ uint2 bfrag[KB * 3][kWave];   // B fragments: [k-block][part][lane], 4 bf16 each
  __shared__ float xsb[KB][16];            // sum of each k-block's activations per vector
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  int rb = blockIdx.x % row_blocks, split = blockIdx.x / row_blocks;
  if (xmap) {
    // XCD-aware: workgroup i runs on XCD i % 8, and XCD x takes the slices
    // congruent to x mod 8 (every row block of them), so a slice's
    // activations are fetched into one XCD's L2 instead of all eight
    const int q = int(blockIdx.x) / 8;
    split = int(blockIdx.x) % 8 + 8 * (q / row_blocks);
    rb = q % row_blocks;
    if (split >= splits) return;   // padding: the whole workgroup, before any barrier
  }
  const int c0 = split * CH;
  const int kq = lane >> 4, li = lane & 15;
  // tile t of the wave: rows row0[t] .. + 15; tiles past Npad redo the last
  // one and are not stored
  int row0[RT];
  bool live[RT];
#pragma unroll
  for (int t = 0; t < RT; ++t) {
    const int r = (rb * NW + wave) * 16 * RT + 16 * t;
    row0[t] = min(r, a.Npad - 16);
    live[t] = r < a.Npad;   // wave-uniform
  }
  const uint32_t Npad = uint32_t(a.Npad);

  // ---- the rows' planes or codes (row li of each tile) and the D rows' scales ----
  u32x4 w[RT][CH][NIB ? 1 : 4];
  if constexpr (NIB) {
    const u32x4 *__restrict__ nb = reinterpret_cast<const u32x4 *>(a.nib);
#pragma unroll
    for (int t = 0; t < RT; ++t)
#pragma unroll
      for (int c = 0; c < CH; ++c)
        w[t][c][0] = __builtin_nontemporal_load(nb + ((uint32_t(c0 + c) * Npad + uint32_t(row0[t] + li)) * 4 + kq));
  } else {
    const u32x4 *__restrict__ pl = reinterpret_cast<const u32x4 *>(a.planes);
#pragma unroll
    for (int t = 0; t < RT; ++t)
#pragma unroll
      for (int c = 0; c < CH; ++c)
#pragma unroll
        for (int p = 0; p < 4; ++p)
          w[t][c][p] = __builtin_nontemporal_load(pl + (uint32_t((c0 + c) * 4 + p) * Npad + uint32_t(row0[t] + li)));
  }
  float4 sc[RT][CH];
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int g = a.gshift >= 0 ? (c0 + c) >> a.gshift : (c0 + c) / a.group_chunks;
#pragma unroll
    for (int t = 0; t < RT; ++t)
      sc[t][c] = *reinterpret_cast<const float4 *>(a.scales + uint32_t(g) * Npad + uint32_t(row0[t] + 4 * kq));
  }

  // ---- B fragments of the slice: wave w splits k-blocks w, w + NW, ... ----
  // Every activation load of the wave is requested before any split (fewer
  // registers than splitting each block as it arrives).
  constexpr int KBW = (KB + NW - 1) / NW;   // k-blocks per wave
  float4 xv[KBW];
#pragma unroll
  for (int i = 0; i < KBW; ++i) {
    const int kb = wave + i * NW;
    // plane layout: item e of k-block kb is k = 4g + 3 - e, g = 8 (kb / 2) + 2 kq + kb % 2;
    // NIB: k = 16 kb + 4 kq + e
    const int k = c0 * kChunk + (NIB ? 16 * kb + 4 * kq : 4 * (8 * (kb >> 1) + 2 * kq + (kb & 1)));
    xv[i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (kb < KB && li < NB && k < a.cols) xv[i] = *reinterpret_cast<const float4 *>(a.x + size_t(li) * a.cols + k);
  }
#pragma unroll
  for (int i = 0; i < KBW; ++i) {
    const int kb = wave + i * NW;
    if (kb >= KB) break;   // wave-uniform
    const float4 v = xv[i];
    float xe[4] = {v.w, v.z, v.y, v.x};
    if constexpr (NIB) xe[0] = v.x, xe[1] = v.y, xe[2] = v.z, xe[3] = v.w;
    {
      float xs = (v.x + v.y) + (v.z + v.w);
      xs += __shfl_xor(xs, 16, kWave);
      xs += __shfl_xor(xs, 32, kWave);
      if (kq == 0) xsb[kb][li] = xs;
    }
    uint32_t part[3][4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float r = xe[e];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const uint32_t h = __float_as_uint(r) & 0xFFFF0000u;   // the top 8 significant bits
        part[t][e] = h;
        r -= __uint_as_float(h);   // exact
      }
      part[2][e] = __float_as_uint(r);   // at most 8 significant bits left: exact in bf16
    }
#pragma unroll
    for (int t = 0; t < 3; ++t)
      bfrag[kb * 3 + t][lane] = make_uint2(__builtin_amdgcn_perm(part[t][1], part[t][0], 0x07060302u),
                                           __builtin_amdgcn_perm(part[t][3], part[t][2], 0x07060302u));
  }
  __syncthreads();

  // ---- the tiles: per 128-chunk, 8 k-blocks of 3 products, then the scale ----
  const uint32_t sel01 = uint32_t(kq) | uint32_t(4 + kq) << 8 | 0x0C0C0000u;
  const uint32_t sel23 = 0x00000C0Cu | uint32_t(kq) << 16 | uint32_t(4 + kq) << 24;
  if (!live[0]) return;   // after the barrier; no barrier follows
  v4f y[RT];
#pragma unroll
  for (int t = 0; t < RT; ++t) y[t] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    // one accumulator per tile and activation part: independent product chains
    v4f acc[RT][3];
#pragma unroll
    for (int t = 0; t < RT; ++t)
#pragma unroll
      for (int u = 0; u < 3; ++u) acc[t][u] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
    if constexpr (NIB) {
#pragma unroll
      for (int kb8 = 0; kb8 < 8; ++kb8) {
        const int kb = 8 * c + kb8;
        v4s bv[3];
#pragma unroll
        for (int u = 0; u < 3; ++u) bv[u] = __builtin_bit_cast(v4s, bfrag[kb * 3 + u][lane]);
#pragma unroll
        for (int t = 0; t < RT; ++t) {
          const uint32_t wd = w[t][c][0][kb8 >> 1] >> (16 * (kb8 & 1));
          // byte (q0 | q1 << 4) * 0x8008: q0 at bits 3-6, q1 at bits 19-22
          const uint32_t a01 = ((wd & 0xFFu) * 0x8008u & 0x00780078u) | 0x41804180u;
          const uint32_t a23 = (((wd >> 8) & 0xFFu) * 0x8008u & 0x00780078u) | 0x41804180u;
          const v4s av = __builtin_bit_cast(v4s, make_uint2(a01, a23));
#pragma unroll
          for (int u = 0; u < 3; ++u) acc[t][u] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(av, bv[u], acc[t][u], 0, 0, 0);
        }
      }
    } else {
#pragma unroll
    for (int mm = 0; mm < 4; ++mm) {
      // byte kq of word mm of planes 0..3 -> bytes 0..3 (high nibbles group
      // 8m + 2kq, low nibbles group 8m + 2kq + 1), then both nibble halves'
      // 4 x 4 bit transposes at once: bit e of byte p (plane p, item e) ->
      // bit p of byte e (in the same half)
      uint32_t T[RT];
#pragma unroll
      for (int t = 0; t < RT; ++t) {
        uint32_t M = __builtin_amdgcn_perm(w[t][c][1][mm], w[t][c][0][mm], sel01) |
                     __builtin_amdgcn_perm(w[t][c][3][mm], w[t][c][2][mm], sel23);
        const uint32_t t1 = ((M >> 14) ^ M) & 0x0000CCCCu;
        M ^= t1 ^ (t1 << 14);
        const uint32_t t2 = ((M >> 7) ^ M) & 0x00AA00AAu;
        M ^= t2 ^ (t2 << 7);
        T[t] = M;
      }
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int kb = 2 * (4 * c + mm) + h;
        v4s bv[3];
#pragma unroll
        for (int u = 0; u < 3; ++u) bv[u] = __builtin_bit_cast(v4s, bfrag[kb * 3 + u][lane]);
#pragma unroll
        for (int t = 0; t < RT; ++t) {
          // byte e's nibble h = code q of item e; A item = bf16(q + 16) = 0x4180 | q << 3
          const uint32_t p01 = __builtin_amdgcn_perm(0u, T[t], 0x0C010C00u);
          const uint32_t p23 = __builtin_amdgcn_perm(0u, T[t], 0x0C030C02u);
          const uint32_t a01 = ((h == 0 ? p01 >> 1 : p01 << 3) & 0x00780078u) | 0x41804180u;
          const uint32_t a23 = ((h == 0 ? p23 >> 1 : p23 << 3) & 0x00780078u) | 0x41804180u;
          const v4s av = __builtin_bit_cast(v4s, make_uint2(a01, a23));
#pragma unroll
          for (int u = 0; u < 3; ++u) acc[t][u] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(av, bv[u], acc[t][u], 0, 0, 0);
        }
      }
    }
    }   // NIB
    const int ch = c0 + c;
    if (ch < a.Kp / kChunk) {
      float xs = 0.0f;   // the chunk's sum of vector li's activations
#pragma unroll
      for (int kb = 8 * c; kb < 8 * c + 8; ++kb) xs += xsb[kb][li];
#pragma unroll
      for (int t = 0; t < RT; ++t) {
        const v4f s = ((acc[t][0] + acc[t][1]) + acc[t][2]) - 24.0f * xs;
        y[t][0] = fmaf(sc[t][c].x, s[0], y[t][0]);
        y[t][1] = fmaf(sc[t][c].y, s[1], y[t][1]);
        y[t][2] = fmaf(sc[t][c].z, s[2], y[t][2]);
        y[t][3] = fmaf(sc[t][c].w, s[3], y[t][3]);
      }
    }
  }
  // D[i][j]: lane j + 16 (i / 4), item i % 4 -> rows row0 + 4 kq + e of vector li
#pragma unroll
  for (int t = 0; t < RT; ++t)
    if (li < NB && live[t])
      *reinterpret_cast<float4 *>(a.partials + (size_t(li) * splits + split) * Npad + uint32_t(row0[t] + 4 * kq)) =
          make_float4(y[t][0], y[t][1], y[t][2], y[t][3]);
}

// y[n*rows + r] = sum_s partials[n][s][r] (+ bias[r]) (+ resid[n*rows + r])
// in split order; resid may be y itself (each element is read and written
// by one thread).  A thread sums 4 consecutive rows with 16-byte loads (Npad
// is a multiple of 64, so the 4 rows of any r0 < rows lie inside the padded
// partials), RL split loads in flight per round: 16, or 48 where K has more
// than 16 slices (K = 8960: one round trip instead of three).
constexpr int kReduceThreads = 256;

// The bias and residual terms of rows r0..r0+3 of vector n (0 past the rows
// or without the operand), loaded before the partials and before any store:
// resid may alias y, so a load placed after a store to y waits for the
// loads before it, one memory round trip per row.
__device__ __forceinline__ void load_row_terms(const float *__restrict__ bias, const float *resid, int n, int rows,
                                               int r0, float (&b)[4], float (&rs)[4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = r0 + i;
    b[i] = bias && r < rows ? bias[r] : 0.0f;
    rs[i] = resid && r < rows ? resid[size_t(n) * rows + r] : 0.0f;
  }
}

template <int RL>
__global__ __launch_bounds__(kReduceThreads) void batched_reduce_kernel(const float *__restrict__ partials,
                                                                        int splits, int Npad, int rows,
                                                                        const float *__restrict__ bias,
                                                                        const float *resid, float *y) {
  const int r0 = 4 * int(blockIdx.x * kReduceThreads + threadIdx.x), n = blockIdx.y;
  if (r0 >= rows) return;
  float b[4], rs[4];
  load_row_terms(bias, resid, n, rows, r0, b, rs);
  const float4 *p = reinterpret_cast<const float4 *>(partials + size_t(n) * splits * Npad + r0);
  const size_t step = size_t(Npad) / 4;
  float4 s = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  for (int k0 = 0; k0 < splits; k0 += RL) {   // RL loads in flight, summed in split order
    float4 v[RL];
#pragma unroll
    for (int j = 0; j < RL; ++j) v[j] = k0 + j < splits ? p[size_t(k0 + j) * step] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
    for (int j = 0; j < RL; ++j) s.x += v[j].x, s.y += v[j].y, s.z += v[j].z, s.w += v[j].w;
  }
  const float t[4] = {s.x, s.y, s.z, s.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = r0 + i;
    if (r >= rows) break;
    float v = t[i];
    if (bias) v += b[i];
    if (resid) v += rs[i];
    y[size_t(n) * rows + r] = v;
  }
}

// kEpiSiluPair: act[n*h + j] = silu(g) * u with g / u the split-order sums
// of rows j / h + j (+ bias), h = rows / 2 (h % 4 == 0: the up half's rows
// keep the 16-byte alignment); the same expression as silu_mul_rows_kernel.
__global__ __launch_bounds__(kReduceThreads) void batched_reduce_pair_kernel(const float *__restrict__ partials,
                                                                             int splits, int Npad, int h,
                                                                             const float *__restrict__ bias,
                                                                             float *__restrict__ act) {
  const int j0 = 4 * int(blockIdx.x * kReduceThreads + threadIdx.x), n = blockIdx.y;
  if (j0 >= h) return;
  float bg[4], bu[4];   // the bias terms, loaded before the partials
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    bg[i] = bias && j0 + i < h ? bias[j0 + i] : 0.0f;
    bu[i] = bias && j0 + i < h ? bias[h + j0 + i] : 0.0f;
  }
  const float4 *pg = reinterpret_cast<const float4 *>(partials + size_t(n) * splits * Npad + j0);
  const float4 *pu = reinterpret_cast<const float4 *>(partials + size_t(n) * splits * Npad + h + j0);
  const size_t step = size_t(Npad) / 4;
  float4 g = make_float4(0.0f, 0.0f, 0.0f, 0.0f), u = g;
  for (int k0 = 0; k0 < splits; k0 += 8) {   // 16 loads in flight, summed in split order
    float4 vg[8], vu[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const bool in = k0 + k < splits;
      vg[k] = in ? pg[size_t(k0 + k) * step] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      vu[k] = in ? pu[size_t(k0 + k) * step] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      g.x += vg[k].x, g.y += vg[k].y, g.z += vg[k].z, g.w += vg[k].w;
      u.x += vu[k].x, u.y += vu[k].y, u.z += vu[k].z, u.w += vu[k].w;
    }
  }
  const float gs[4] = {g.x, g.y, g.z, g.w}, us[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int j = j0 + i;
    if (j >= h) break;
    float a = gs[i], b = us[i];
    if (bias) a += bg[i], b += bu[i];
    act[size_t(n) * h + j] = a / (1.0f + expf(-a)) * b;
  }
}

// kEpiNormOut: one workgroup per vector n: y[n] = split-order sums (+ bias)
// (+ resid[n], which may be y itself), kept in LDS, then y2[n] = RMSNorm of
// y[n] with weight w computed exactly as rmsnorm_rows_kernel does (its 256
// threads' element assignment, sum order and expression, norm.cpp:18-34), so
// the fused and the separate forms give the same bits.  The row sums take
// kNormReduceThreads threads, 4 rows each, with up to kNormReduceLoads split
// loads in flight per thread (a whole 2048-row vector and 48 splits, K up to
// 12288, in one round trip).
constexpr int kNormReduceThreads = 512;
constexpr int kNormReduceLoads = 48;
__global__ __launch_bounds__(kNormReduceThreads) void batched_reduce_norm_kernel(
    const float *__restrict__ partials, int splits, int Npad, int rows, const float *__restrict__ bias,
    const float *resid, float *y, const float *__restrict__ w, float eps, float *__restrict__ y2) {
  constexpr int NT = 256;   // rmsnorm_rows_kernel's threads
  static_assert(kNormReduceThreads % NT == 0, "the norm runs on the first 256 threads");
  constexpr int WJ = 4;   // norm weights a thread loads up front: rows up to 4 * kNormReduceThreads
  extern __shared__ float row[];   // [rows]
  __shared__ float red[NT / kWave];
  const int n = blockIdx.x;
  const float *pn = partials + size_t(n) * splits * Npad;
  const size_t step = size_t(Npad) / 4;
  float wk[WJ];
#pragma unroll
  for (int j = 0; j < WJ; ++j) {
    const int k = int(threadIdx.x) + j * kNormReduceThreads;
    wk[j] = k < rows ? w[k] : 0.0f;
  }
  for (int r0 = 4 * int(threadIdx.x); r0 < rows; r0 += 4 * kNormReduceThreads) {
    float b[4], rs[4];
    load_row_terms(bias, resid, n, rows, r0, b, rs);
    const float4 *p = reinterpret_cast<const float4 *>(pn + r0);
    float4 s = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (int k0 = 0; k0 < splits; k0 += kNormReduceLoads) {
      float4 v[kNormReduceLoads];
#pragma unroll
      for (int k = 0; k < kNormReduceLoads; ++k)
        v[k] = k0 + k < splits ? p[size_t(k0 + k) * step] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
      for (int k = 0; k < kNormReduceLoads; ++k) s.x += v[k].x, s.y += v[k].y, s.z += v[k].z, s.w += v[k].w;
    }
    const float t[4] = {s.x, s.y, s.z, s.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = r0 + i;
      if (r >= rows) break;
      float v = t[i];
      if (bias) v += b[i];
      if (resid) v += rs[i];
      y[size_t(n) * rows + r] = v;
      row[r] = v;
    }
  }
  __syncthreads();
  float ss = 0.0f;
  if (threadIdx.x < NT)
    for (int k = threadIdx.x; k < rows; k += NT) ss += row[k] * row[k];
  ss = lane_sum<32>(ss, threadIdx.x & (kWave - 1));
  if (threadIdx.x < NT && (threadIdx.x & (kWave - 1)) == 0) red[threadIdx.x / kWave] = ss;
  __syncthreads();
  const float inv = 1.0f / sqrtf(((red[0] + red[1]) + (red[2] + red[3])) / float(rows) + eps);
#pragma unroll
  for (int j = 0; j < WJ; ++j) {
    const int k = int(threadIdx.x) + j * kNormReduceThreads;
    if (k < rows) y2[size_t(n) * rows + k] = row[k] * inv * wk[j];
  }
  for (int k = int(threadIdx.x) + WJ * kNormReduceThreads; k < rows; k += kNormReduceThreads)
    y2[size_t(n) * rows + k] = row[k] * inv * w[k];
}

// Four vectors through the full-K geometry of the lean kernel (CPS 1): a
// workgroup owns RW = 64/H rows (PAIR: RW/2 gate rows and the matching up
// rows) and the whole K, lane l serving row l % RW and 128-chunk
// wave*H + l/RW.  The tables of the 4 vectors sit side by side (entry m of
// group g of chunk ch at ch*batch_chunk_bytes<4>() + g*272 + m*16, vector n
// at +4n, as in the batched kernel), so one v_perm address and one 16-byte
// LDS read serve the 4 lookups of a weight nibble.  The activation
// transform (RMSNorm per vector) is fused into the table build and the
// k-slice sums end in the workgroup, so a group of 4 vectors costs one
// launch and no partials; the lean kernel's rules apply (each wave builds
// the tables its own lanes read).
constexpr uint32_t kQuadChunkBytes = batch_chunk_bytes<4>();
constexpr int kQuadMaxBlocks = 256;   // MI355X CUs

constexpr uint32_t quad_prefix_bytes(int waves, int h) {
  // xsum [waves*h][4], red [waves][64/h][4], per-wave norm sums [waves][4]
  return (uint32_t(waves * h * 4 + waves * (kWave / h) * 4 + waves * 4) * 4 + 255) / 256 * 256;
}

template <int FMT, bool ROT, int WAVES, int H, int XM, int EPI, bool PS = false>
__global__ __launch_bounds__(WAVES * kWave) void lut_gemv_quad_kernel(GemvArgs a) {
  constexpr int P = Fmt<FMT>::P, NA = Fmt<FMT>::NA, S = Fmt<FMT>::S;
  // PS (4-bit, unrotated): a row's chunk split over two lanes by planes, as
  // in the lean kernel
  static_assert(!PS || (FMT == LMX_FMT_INT4 && !ROT && EPI == kEpiStore), "plane split: 4-bit, plain store");
  constexpr int RW = kWave / H / (PS ? 2 : 1);
  constexpr int NS = WAVES * H;
  constexpr int XJ = H / 2;
  constexpr bool PAIR = EPI == kEpiSiluPair;
  constexpr int HR = RW / 2;
  static_assert(H % 2 == 0, "whole 256-chunks per wave");
  constexpr uint32_t PREFIX = quad_prefix_bytes(WAVES, H);
  extern __shared__ __attribute__((aligned(256))) float lds[];
  float *xsum = lds;                      // [NS][4]
  float *red = lds + NS * 4;              // [WAVES][RW][4]
  float *nrm = red + WAVES * RW * 4;      // [WAVES][4]
  char *tables = reinterpret_cast<char *>(lds) + PREFIX;
  const int Kc = a.Kp / kChunk;
  const int C2n = a.Kp / kRotChunk;
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  const int s = wave * H + (PS ? (lane / RW) >> 1 : lane / RW);   // this lane's 128-chunk
  const int part = PS ? (lane / RW) & 1 : 0;                       // PS: planes 2*part, 2*part + 1
  const int rl = lane % RW;
  const int row = PAIR ? (rl < HR ? 0 : a.rows / 2 - HR) + blockIdx.x * HR + rl : blockIdx.x * RW + rl;
  const int lr = min(row, a.Npad - 1);
  const int c2base = wave * XJ;

  // ---- x of the wave's 256-chunks for the 4 vectors, then the weights ----
  float4 xr[XJ][4], xa[XJ];
#pragma unroll
  for (int j = 0; j < XJ; ++j) {
    const int k0 = min(c2base + j, C2n - 1) * kRotChunk;
#pragma unroll
    for (int n = 0; n < 4; ++n) xr[j][n] = load_x4_raw(a.x + size_t(n) * a.cols, k0, a.cols, lane);
    if constexpr (XM == kXModeRmsNorm) xa[j] = load_x4_raw(a.xw, k0, a.cols, lane);
  }
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_barrier();   // every wave's x requests ahead of the weight stream
  constexpr int PL = PS ? 2 : P;   // planes a lane loads
  u32x4 w[PL];
  float sc[S];
  {
    const u32x4 *__restrict__ pl = reinterpret_cast<const u32x4 *>(a.planes);
    const uint32_t Npad = uint32_t(a.Npad);
    const uint32_t ch = uint32_t(min(s, Kc - 1));
#pragma unroll
    for (int p = 0; p < PL; ++p)
      w[p] = __builtin_nontemporal_load(pl + ((ch * P + uint32_t(PS ? 2 * part + p : p)) * Npad + uint32_t(lr)));
    const int g = a.gshift >= 0 ? int(ch) >> a.gshift : int(ch) / a.group_chunks;
#pragma unroll
    for (int t = 0; t < S; ++t) sc[t] = a.scales[(uint32_t(t * a.n_groups + g)) * Npad + uint32_t(lr)];
  }
  // the epilogue thread's bias and residual terms, requested behind the
  // weights so their round trip overlaps the lookups
  float eb0 = 0.0f, eb1 = 0.0f, er = 0.0f;
  if constexpr (PAIR) {
    if (threadIdx.x < HR * 4 && a.bias) {
      const int j = blockIdx.x * HR + threadIdx.x % HR;
      eb0 = a.bias[j], eb1 = a.bias[a.rows / 2 + j];
    }
  } else if (threadIdx.x < RW * 4) {
    const int r = blockIdx.x * RW + threadIdx.x % RW, n = threadIdx.x / RW;
    if (r < a.rows) {
      if (a.bias) eb0 = a.bias[r];
      if (a.resid) er = a.resid[size_t(n) * a.rows + r];   // read before this thread stores y (resid may be y)
    }
  }
  __builtin_amdgcn_sched_barrier(0);

  // RMSNorm of each vector: the waves' 256-chunks partition x (norm.cpp:18-34)
  float inv_rms[4] = {1.0f, 1.0f, 1.0f, 1.0f};
  if constexpr (XM == kXModeRmsNorm) {
#pragma unroll
    for (int n = 0; n < 4; ++n) {
      float ss = 0.0f;
#pragma unroll
      for (int j = 0; j < XJ; ++j) {
        float x0, x1, x2, x3;
        mask_x4(xr[j][n], (c2base + j) * kRotChunk, a.cols, lane, x0, x1, x2, x3);
        if (c2base + j < C2n) ss += (x0 * x0 + x1 * x1) + (x2 * x2 + x3 * x3);
      }
      ss = lane_sum<32>(ss, lane);
      if (lane == 0) nrm[wave * 4 + n] = ss;
    }
    __syncthreads();
#pragma unroll
    for (int n = 0; n < 4; ++n) {
      float t = 0.0f;
#pragma unroll
      for (int i = 0; i < WAVES; ++i) t += nrm[i * 4 + n];
      inv_rms[n] = 1.0f / sqrtf(t / float(a.cols) + a.eps);
    }
  }

  // ---- tables of the wave's chunks, the 4 vectors side by side ----
#pragma unroll
  for (int j = 0; j < XJ; ++j) {
    const int c2 = c2base + j;
    if (c2 >= C2n) break;   // wave-uniform
    const int ch = c2 * 2 + (lane >> 5), g = lane & 31;
    float *dst = reinterpret_cast<float *>(tables + uint32_t(ch) * kQuadChunkBytes + uint32_t(g) * batch_group_stride<4>());
#pragma unroll
    for (int n = 0; n < 4; ++n) {
      float x0, x1, x2, x3;
      mask_x4(xr[j][n], c2 * kRotChunk, a.cols, lane, x0, x1, x2, x3);
      if constexpr (XM == kXModeRmsNorm) {
        const float aux[4] = {xa[j].x, xa[j].y, xa[j].z, xa[j].w};
        xform4(XM, inv_rms[n], aux, x0, x1, x2, x3);
      }
      if constexpr (ROT) fwht256_regs(x0, x1, x2, x3, lane);
      float t[16];
      group_table(x0, x1, x2, x3, t);
#pragma unroll
      for (int m = 0; m < 16; ++m) dst[m * 4 + n] = t[m];
      if constexpr (Fmt<FMT>::XS) {
        float xs = t[15];
        xs = lane_sum<16>(xs, lane);
        if ((lane & 31) == 0) xsum[ch * 4 + n] = xs;
      }
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();

  // ---- lookups over this lane's chunk for the 4 vectors ----
  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  if constexpr (PS) {
    // the two planes of this lane's part; the 4-bit identity's third plane
    // enters inverted, and the part's terms of ((A0 + 2 A1) + 4 A2) - 8 A3
    // weight the two sums
    const int ch = min(s, Kc - 1);
    const uint32_t cbase = lds_addr(lds) + PREFIX + uint32_t(ch) * kQuadChunkBytes;
    const uint32_t inv = part ? 0xFFFFFFFFu : 0u;
    float A[2][4];
#pragma unroll
    for (int q = 0; q < 2; ++q)
#pragma unroll
      for (int n = 0; n < 4; ++n) A[q][n] = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t v[2] = {w[0][i], w[1][i] ^ inv};
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        word_lookups_batch<4>(v[q], i, cbase, A[q]);
#pragma unroll
        for (int n = 0; n < 4; ++n) asm volatile("" : "+v"(A[q][n]));
      }
    }
    const float c0 = part ? 4.0f : 1.0f, c1 = part ? -8.0f : 2.0f;
#pragma unroll
    for (int n = 0; n < 4; ++n) acc[n] = s < Kc ? fmaf(sc[0], c0 * A[0][n] + c1 * A[1][n], 0.0f) : 0.0f;
  } else {
    const int ch = min(s, Kc - 1);
    const uint32_t cbase = lds_addr(lds) + PREFIX + uint32_t(ch) * kQuadChunkBytes;   // 256-byte aligned
    float A[NA][4];
#pragma unroll
    for (int q = 0; q < NA; ++q)
#pragma unroll
      for (int n = 0; n < 4; ++n) A[q][n] = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint32_t wi[P], v[NA];
#pragma unroll
      for (int p = 0; p < P; ++p) wi[p] = w[p][i];
      lookup_words<FMT>(wi, v);
#pragma unroll
      for (int q = 0; q < NA; ++q) {
        word_lookups_batch<4>(v[q], i, cbase, A[q]);
        // the sums of one word complete before the next word's reads: left
        // free, the compiler sinks every add to the chunk's end (the chunk
        // is this lane's only one) and holds all 64 read results, spilling
#pragma unroll
        for (int n = 0; n < 4; ++n) asm volatile("" : "+v"(A[q][n]));
      }
    }
#pragma unroll
    for (int n = 0; n < 4; ++n) {
      float An[NA];
#pragma unroll
      for (int q = 0; q < NA; ++q) An[q] = A[q][n];
      float xs = 0.0f;
      if constexpr (Fmt<FMT>::XS) xs = xsum[ch * 4 + n];
      const float nacc = finish_chunk<FMT>(An, xs, sc, 0.0f);
      acc[n] = s < Kc ? nacc : 0.0f;
    }
  }

  // ---- the wave's H slices by a lane butterfly, then the waves in order ----
#pragma unroll
  for (int n = 0; n < 4; ++n) {
    const float wsum = strided_sum<RW>(acc[n], lane);
    if (lane < RW) red[(wave * RW + rl) * 4 + n] = wsum;
  }
  __syncthreads();
  if constexpr (PAIR) {
    if (threadIdx.x < HR * 4) {
      const int t = threadIdx.x % HR, n = threadIdx.x / HR;
      const int j = blockIdx.x * HR + t, h = a.rows / 2;
      float g = 0.0f, u = 0.0f;
#pragma unroll
      for (int k = 0; k < WAVES; ++k) {
        g += red[(k * RW + t) * 4 + n];
        u += red[(k * RW + HR + t) * 4 + n];
      }
      if (a.bias) g += eb0, u += eb1;
      a.y[size_t(n) * h + j] = silu(g) * u;
    }
  } else if (threadIdx.x < RW * 4) {
    const int t = threadIdx.x % RW, n = threadIdx.x / RW;
    const int r = blockIdx.x * RW + t;
    float v = 0.0f;
#pragma unroll
    for (int k = 0; k < WAVES; ++k) v += red[(k * RW + t) * 4 + n];
    if (r < a.rows) {
      if (a.bias) v += eb0;
      if (a.resid) v += er;
      a.y[size_t(n) * a.rows + r] = v;
    }
  }
}

template <int FMT, bool ROT, int WAVES, int H, int XM, int EPI, bool PS = false>
static int launch_quad_kernel(const GemvArgs &a, hipStream_t st) {
  const size_t lds = quad_prefix_bytes(WAVES, H) + size_t(a.Kp / kChunk) * kQuadChunkBytes;
  static const hipError_t attr =
      hipFuncSetAttribute(reinterpret_cast<const void *>(&lut_gemv_quad_kernel<FMT, ROT, WAVES, H, XM, EPI, PS>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, int(kMaxLdsBytes));
  if (attr != hipSuccess) return fail(LMX_ERR_LAUNCH_FAILED, "hipFuncSetAttribute: %s", hipGetErrorString(attr));
  constexpr int RW = kWave / H / (PS ? 2 : 1);
  const int blocks = EPI == kEpiSiluPair ? a.rows / RW : (a.Npad + RW - 1) / RW;
  lut_gemv_quad_kernel<FMT, ROT, WAVES, H, XM, EPI, PS><<<dim3(blocks), dim3(WAVES * kWave), lds, st>>>(a);
  return LMX_OK;
}

static int quad_max_blocks() {
  const char *e = std::getenv("LMX_QUAD_MAX_BLOCKS");
  return e ? std::atoi(e) : kQuadMaxBlocks;
}

template <int FMT, int WAVES, int H>
static int launch_quad_cfg(const GemvArgs &a, hipStream_t st) {   // quad_serves(a) holds
  const bool rot = a.rotate == LMX_ROTATE_FWHT256;
  // 4-bit 4 x 4 x 1, unrotated, store: the plane split where twice the
  // workgroups still make one round (LMX_QPS=0 turns it off)
  if constexpr (FMT == LMX_FMT_INT4 && WAVES == 4 && H == 4) {
    const char *qe = std::getenv("LMX_QPS");
    const int rw = kWave / H;
    if ((!qe || std::atoi(qe) != 0) && !rot && a.epi == kEpiStore && 2 * ((a.Npad + rw - 1) / rw) <= quad_max_blocks()) {
      if (a.xmode == kXModeRmsNorm) return launch_quad_kernel<FMT, false, WAVES, H, kXModeRmsNorm, kEpiStore, true>(a, st);
      return launch_quad_kernel<FMT, false, WAVES, H, kXModeNone, kEpiStore, true>(a, st);
    }
  }
#define LMX_QUAD(R, XMV, EPV) return launch_quad_kernel<FMT, R, WAVES, H, XMV, EPV>(a, st)
  if (a.xmode == kXModeRmsNorm) {
    if (rot) {
      if (a.epi == kEpiSiluPair) LMX_QUAD(true, kXModeRmsNorm, kEpiSiluPair);
      LMX_QUAD(true, kXModeRmsNorm, kEpiStore);
    }
    if (a.epi == kEpiSiluPair) LMX_QUAD(false, kXModeRmsNorm, kEpiSiluPair);
    LMX_QUAD(false, kXModeRmsNorm, kEpiStore);
  }
  if (rot) {
    if (a.epi == kEpiSiluPair) LMX_QUAD(true, kXModeNone, kEpiSiluPair);
    LMX_QUAD(true, kXModeNone, kEpiStore);
  }
  if (a.epi == kEpiSiluPair) LMX_QUAD(false, kXModeNone, kEpiSiluPair);
  LMX_QUAD(false, kXModeNone, kEpiStore);
#undef LMX_QUAD
}

// 1 when the handle's plan has no quad form (split-K, or tables of 4
// vectors over its K do not fit).
template <int FMT>
static int launch_quad_fmt(const GemvArgs &a, hipStream_t st) {
  int r = 1;
  switch (a.fullk) {
  case kFullK_8x2x1: r = launch_quad_cfg<FMT, 8, 2>(a, st); break;
  case kFullK_4x4x1: r = launch_quad_cfg<FMT, 4, 4>(a, st); break;
  default: return 1;
  }
  if (r) return r;
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? LMX_OK : fail(LMX_ERR_LAUNCH_FAILED, "quad lut_gemv launch: %s", hipGetErrorString(e));
}

bool quad_serves(const GemvArgs &a) {
  if (a.amax || a.kfamily == kKernelGeneric || std::getenv("LMX_NO_QUAD")) return false;
  if (a.fullk != kFullK_8x2x1 && a.fullk != kFullK_4x4x1) return false;
  const FullKShape f = fullk_shape(a.fullk);
  const int rw = kWave / f.h;
  if (a.epi != kEpiStore && a.epi != kEpiSiluPair) return false;
  if (a.epi == kEpiSiluPair && a.rows % rw) return false;
  if (a.xmode != kXModeNone && a.xmode != kXModeRmsNorm) return false;
  if (a.rotate != LMX_ROTATE_NONE && a.rotate != LMX_ROTATE_FWHT256) return false;
  const size_t lds = quad_prefix_bytes(f.waves, f.h) + size_t(a.Kp / kChunk) * kQuadChunkBytes;
  if (lds > kMaxLdsBytes || a.Kp / kChunk > f.waves * f.h) return false;
  // At most one workgroup per CU (LMX_QUAD_MAX_BLOCKS overrides): every
  // workgroup builds the 4 vectors' tables of the whole K, which past one
  // round of workgroups costs more than the batched kernel's per-slice
  // tables and reduce (Qwen gate|up 17920 x 1536, 560 workgroups: batch 4
  // decode 2222 -> 2285 tokens/s with the limit).
  const int blocks = a.epi == kEpiSiluPair ? a.rows / rw : (a.Npad + rw - 1) / rw;
  return blocks <= quad_max_blocks();
}

int launch_gemv_quad(int fmt, const GemvArgs &a, void *stream) {
  if (!quad_serves(a)) return 1;
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (fmt) {
  case LMX_FMT_TERNARY: return launch_quad_fmt<LMX_FMT_TERNARY>(a, st);
  case LMX_FMT_BINARY: return launch_quad_fmt<LMX_FMT_BINARY>(a, st);
  case LMX_FMT_RRQ2: return launch_quad_fmt<LMX_FMT_RRQ2>(a, st);
  case LMX_FMT_RRQ3: return launch_quad_fmt<LMX_FMT_RRQ3>(a, st);
  case LMX_FMT_INT3: return launch_quad_fmt<LMX_FMT_INT3>(a, st);
  case LMX_FMT_INT4: return launch_quad_fmt<LMX_FMT_INT4>(a, st);
  case LMX_FMT_INT8: return launch_quad_fmt<LMX_FMT_INT8>(a, st);
  }
  return 1;
}

template <int FMT, int NB, int RG, int CH = 2>
static void launch_batch_rg(const GemvArgs &a, int splits, hipStream_t st) {
  constexpr int VG = NB >= 4 ? 4 : 1;   // vectors per wave
  const int row_blocks = (a.Npad + RG * kWave - 1) / (RG * kWave);
  const dim3 grid(row_blocks * splits), block(kWave * batch_waves<NB, VG, RG>());
  if constexpr (NB == 4) {
    if (a.xmode == kXModeRmsNorm) {
      lut_gemv_batch_kernel<FMT, NB, VG, RG, kXModeRmsNorm, CH><<<grid, block, 0, st>>>(a, row_blocks, splits);
      return;
    }
  }
  lut_gemv_batch_kernel<FMT, NB, VG, RG, kXModeNone, CH><<<grid, block, 0, st>>>(a, row_blocks, splits);
}

int batched_launch_splits(size_t Npad, size_t Kp) {
  // 128-wide slices (one row group) where 256-wide ones would leave CUs idle
  static const bool s128 = [] {
    const char *e = std::getenv("LMX_BATCH_S128");
    return !(e && std::atoi(e) == 0);
  }();
  return int(s128 ? batched_slice_splits(Npad, Kp) : Kp / kRotChunk);
}

template <int FMT, int NB>
static int launch_batch_nb(const GemvArgs &a, hipStream_t st) {
  const int splits = batched_launch_splits(size_t(a.Npad), size_t(a.Kp));
  const bool narrow = splits != a.Kp / kRotChunk;
  // Rows per workgroup: 256 while that leaves a workgroup per CU, else fewer
  // (LMX_BATCH_RG = 1, 2 or 4 forces 64, 128 or 256).
  const auto grid = [&](int rg) { return (a.Npad + rg * kWave - 1) / (rg * kWave) * splits; };
  static const int force = [] {
    const char *e = std::getenv("LMX_BATCH_RG");
    const int v = e ? std::atoi(e) : 0;
    return v == 1 || v == 2 || v == 4 ? v : 0;
  }();
  const int rg = force              ? force
                 : grid(4) >= kBatchMinGrid ? 4
                 : grid(2) >= kBatchMinGrid ? 2
                                            : 1;
  bool mfma = false;
  if constexpr (FMT == LMX_FMT_INT4 && NB >= 4)
    mfma = a.rotate == LMX_ROTATE_NONE && mfma_batched() && a.xmode == kXModeNone && (NB >= 8 || a.epi != kEpiPartials);
  if (mfma) {
    // 8 waves of 16 rows per workgroup, the slice's activation fragments
    // built once for them, the codes from the handle's nibble copy
    // (LMX_MFMA=4: 4 waves; 2: 32 rows per wave; 3: codes from the planes)
    const int mode = mfma_batched();
    const int nw = mode == 4 ? 4 : 8, rt = mode == 2 ? 2 : 1;
    const int row_blocks = (a.Npad + 16 * nw * rt - 1) / (16 * nw * rt);
    // XCD-aware slices where there are many (each XCD's L2 would otherwise
    // fetch every slice's activations; LMX_MFMA_XCD=0 turns it off)
    static const bool xcd_env = [] {
      const char *e = std::getenv("LMX_MFMA_XCD");
      return !(e && std::atoi(e) == 0);
    }();
    const int xmap = xcd_env && splits >= 16 ? 1 : 0;
    const dim3 grid(xmap ? 8 * ((splits + 7) / 8) * row_blocks : row_blocks * splits), block(kWave * nw);
#define LMX_MFMA_LAUNCH(NW, RT)                                                                           \
  do {                                                                                                    \
    if (a.nib && mode != 3) {                                                                             \
      if (narrow) lut_gemv_mfma_kernel<NB, 1, NW, RT, true><<<grid, block, 0, st>>>(a, row_blocks, splits, xmap); \
      else lut_gemv_mfma_kernel<NB, 2, NW, RT, true><<<grid, block, 0, st>>>(a, row_blocks, splits, xmap);        \
    } else {                                                                                              \
      if (narrow) lut_gemv_mfma_kernel<NB, 1, NW, RT><<<grid, block, 0, st>>>(a, row_blocks, splits, xmap);       \
      else lut_gemv_mfma_kernel<NB, 2, NW, RT><<<grid, block, 0, st>>>(a, row_blocks, splits, xmap);              \
    }                                                                                                     \
  } while (0)
    if (mode == 4) LMX_MFMA_LAUNCH(4, 1);
    else if (mode == 2) LMX_MFMA_LAUNCH(8, 2);
    else LMX_MFMA_LAUNCH(8, 1);
#undef LMX_MFMA_LAUNCH
  } else if (narrow) {
    launch_batch_rg<FMT, NB, 1, 1>(a, splits, st);
  } else if (rg == 4) {
    launch_batch_rg<FMT, NB, 4>(a, splits, st);
  } else if (rg == 2) {
    launch_batch_rg<FMT, NB, 2>(a, splits, st);
  } else {
    launch_batch_rg<FMT, NB, 1>(a, splits, st);
  }
  if (a.epi == kEpiPartials) {
    // the consumer sums the partials
  } else if (a.epi == kEpiSiluPair) {
    const int h = a.rows / 2;
    batched_reduce_pair_kernel<<<dim3((h + 4 * kReduceThreads - 1) / (4 * kReduceThreads), NB),
                                 dim3(kReduceThreads), 0, st>>>(a.partials, splits, a.Npad, h, a.bias, a.y);
  } else if (a.epi == kEpiNormOut) {
    batched_reduce_norm_kernel<<<dim3(NB), dim3(kNormReduceThreads), size_t(a.rows) * sizeof(float), st>>>(
        a.partials, splits, a.Npad, a.rows, a.bias, a.resid, a.y, a.xw, a.eps, a.y2);
  } else {
    const dim3 grid((a.rows + 4 * kReduceThreads - 1) / (4 * kReduceThreads), NB);
    if (splits > 16)
      batched_reduce_kernel<48><<<grid, dim3(kReduceThreads), 0, st>>>(a.partials, splits, a.Npad, a.rows, a.bias,
                                                                       a.resid, a.y);
    else
      batched_reduce_kernel<16><<<grid, dim3(kReduceThreads), 0, st>>>(a.partials, splits, a.Npad, a.rows, a.bias,
                                                                       a.resid, a.y);
  }
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? LMX_OK : fail(LMX_ERR_LAUNCH_FAILED, "batched lut_gemv launch: %s", hipGetErrorString(e));
}

template <int FMT>
static int launch_batch_fmt(const GemvArgs &a, int nb, hipStream_t st) {
  if (a.xmode != kXModeNone && (a.xmode != kXModeRmsNorm || nb != 4))
    return fail(LMX_ERR_INVALID_ARGUMENT, "the batched kernel applies RMSNorm to groups of 4 vectors only");
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
