// lmx_decode.hip -- device-resident batch-1 decoder forward (lutmac_decode.h).
//
// A token step is Model::forward(token, pos) + greedy Model::sample
// (src/model.cpp:47-453, 455-490) with every op on the GPU; it starts from
// the embedding of the token at the current position in the hidden state
// (embed_kernel at reset: row `token` of the tied table, dequantized from
// the tile layout, model.cpp:58-85):
//   per layer:
//     GEMV qkv             RMSNorm(input_norm) fused into the table prologue,
//                          q|k|v rows in one weight, + bias (model.cpp:296-323)
//     attn_kernel          RoPE of q and k, KV-cache append, scores, partial
//                          softmax and weighted V sums over 64-position chunks,
//                          and the merge of the chunks by the last workgroup
//                          of each KV head (model.cpp:326-372,
//                          embedding.cpp:36-75, attention.cpp:23-42)
//     GEMV o               + residual: the hidden state is the bias and the
//                          output (model.cpp:376-388)
//     GEMV gate|up         RMSNorm(post_norm) fused (model.cpp:390-403); for
//                          4-bit weights the epilogue writes SiLU(gate)*up
//                          (gate and up rows paired in each workgroup)
//     GEMV down            on SiLU(gate)*up (else formed in its prologue from
//                          the gate|up output), + residual (model.cpp:410-426)
//   GEMV head              RMSNorm(final_norm) fused, tied table (model.cpp:433-447),
//                          each wave's first maximum folded into a 64-bit key
//                          by the GEMV's epilogue (model.cpp:480-490)
//   finish_embed_kernel    maximum of the keys -> next token, position + 1,
//                          and the next token's embedding into the hidden state
// (Batches of sequences start each step with embed_kernel and finish with
// argmax_rows_kernel; their linears run the batched GEMV, whose reductions
// also write the normed rows and SiLU(gate)*up, see step_batched.)
// The position and the token sequence live in device memory, so the same
// captured step replays for every position.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "lmx_device.hpp"
#include "lmx_internal.hpp"
#include "lmx_lanes.hpp"
#include "lutmac_decode.h"

namespace lmx {
namespace {

template <int FMT> struct EmbFmt;
template <> struct EmbFmt<LMX_FMT_TERNARY> { static constexpr int P = 2, S = 1; };
template <> struct EmbFmt<LMX_FMT_BINARY> { static constexpr int P = 1, S = 1; };
template <> struct EmbFmt<LMX_FMT_RRQ2> { static constexpr int P = 2, S = 2; };
template <> struct EmbFmt<LMX_FMT_RRQ3> { static constexpr int P = 3, S = 3; };
template <> struct EmbFmt<LMX_FMT_INT3> { static constexpr int P = 3, S = 1; };
template <> struct EmbFmt<LMX_FMT_INT4> { static constexpr int P = 4, S = 1; };
template <> struct EmbFmt<LMX_FMT_INT8> { static constexpr int P = 8, S = 1; };

// Weight value from its plane bits and scales (the block accessors of
// types.hpp: BitPlaneBlock 140-160, BinaryBlock::get 404-411, Int2Block::get
// 217-234 generalised to k stages, Int3Block 270-285, Int4Block::get 186-190,
// Int8Block::get 448-460).
template <int FMT>
__device__ __forceinline__ float weight_value(const int *b, const float *s) {
  if constexpr (FMT == LMX_FMT_TERNARY) {
    return b[1] ? 0.0f : (b[0] ? -1.0f : 1.0f) * s[0];
  } else if constexpr (FMT == LMX_FMT_BINARY) {
    return b[0] ? s[0] : -s[0];
  } else if constexpr (FMT == LMX_FMT_RRQ2 || FMT == LMX_FMT_RRQ3) {
    float v = 0.0f;
#pragma unroll
    for (int i = 0; i < EmbFmt<FMT>::S; ++i) v += b[i] ? s[i] : -s[i];
    return v;
  } else {
    int q = 0;
#pragma unroll
    for (int p = 0; p < EmbFmt<FMT>::P; ++p) q |= b[p] << p;
    if constexpr (FMT == LMX_FMT_INT3) return float(q - 4) * s[0];
    if constexpr (FMT == LMX_FMT_INT4) return float(q - 8) * s[0];
    return float(int(int8_t(uint8_t(q)))) * s[0];
  }
}

// hidden[k] = W[token][k] from the tile layout [Kp/128][P][Npad][16 B] and
// scales [S][n_groups][Npad]; one weight per thread.
template <int FMT>
__global__ __launch_bounds__(256) void embed_kernel(const uint8_t *__restrict__ planes, const float *__restrict__ scales,
                                                    int Npad, int rows, int n_groups, int group_chunks, int cols,
                                                    const int *__restrict__ tokens, const int *__restrict__ pos,
                                                    float *__restrict__ out, int tstride) {
  constexpr int P = EmbFmt<FMT>::P, S = EmbFmt<FMT>::S;
  const int k = blockIdx.x * 256 + threadIdx.x;
  if (k >= cols) return;
  // sequence blockIdx.y: its tokens at tokens[y * tstride], its row at out[y * cols]
  out += size_t(blockIdx.y) * cols;
  const int t = min(max(tokens[size_t(blockIdx.y) * tstride + *pos], 0), rows - 1);
  const int c = k / kChunk, byte = (k % kChunk) / 8, bit = 7 - k % 8;
  int b[P];
#pragma unroll
  for (int p = 0; p < P; ++p) b[p] = (planes[((size_t(c) * P + p) * Npad + t) * 16 + byte] >> bit) & 1;
  const int g = c / group_chunks;
  float s[S];
#pragma unroll
  for (int i = 0; i < S; ++i) s[i] = scales[(size_t(i) * n_groups + g) * Npad + t];
  out[k] = weight_value<FMT>(b, s);
}

// Batched decode helpers (one workgroup per sequence row).
// y[b] = x[b] * inv_rms(x[b]) * w, inv_rms = 1/sqrt(sum x^2 / n + eps)
// (norm.cpp:18-34).
__global__ __launch_bounds__(256) void rmsnorm_rows_kernel(const float *__restrict__ x, const float *__restrict__ w,
                                                           int n, float eps, float *__restrict__ y) {
  __shared__ float red[4];
  x += size_t(blockIdx.x) * n;
  y += size_t(blockIdx.x) * n;
  float s = 0.0f;
  for (int k = threadIdx.x; k < n; k += 256) s += x[k] * x[k];
  s = lane_sum<32>(s, threadIdx.x & (kWave - 1));
  if ((threadIdx.x & (kWave - 1)) == 0) red[threadIdx.x / kWave] = s;
  __syncthreads();
  const float inv = 1.0f / sqrtf(((red[0] + red[1]) + (red[2] + red[3])) / float(n) + eps);
  for (int k = threadIdx.x; k < n; k += 256) y[k] = x[k] * inv * w[k];
}

// act[b][k] = silu(gu[b][k]) * gu[b][ffn + k] (model.cpp:36, 413-416).
__global__ __launch_bounds__(256) void silu_mul_rows_kernel(const float *__restrict__ gu, int ffn,
                                                            float *__restrict__ act) {
  const int k = blockIdx.x * 256 + threadIdx.x;
  if (k >= ffn) return;
  const float *g = gu + size_t(blockIdx.y) * 2 * ffn;
  const float a = g[k];
  act[size_t(blockIdx.y) * ffn + k] = a / (1.0f + expf(-a)) * g[ffn + k];
}

constexpr int kArgmaxParts = 32;   // most workgroups per logits row
constexpr int kAttnMaxSplit = 8;   // most workgroups sharing one KV head's query heads
constexpr int kTicketPad = 32;     // unsigneds per ticket (attention, greedy pick): one 128-byte line each
constexpr int kAttnMaxParts = 16;  // most q|k|v split partials attention sums itself

// Greedy token of every sequence: the first maximum of its logits row
// (model.cpp:480-490); written unless the next position is forced.  Each
// row is scanned by gridDim.x workgroups (part blockIdx.x of sequence
// blockIdx.y), each leaving its slice's key in slots; the last of a
// sequence's workgroups (a ticket) takes the largest key, and the last
// sequence to finish (a second ticket) advances the shared position.
__global__ __launch_bounds__(1024) void argmax_rows_kernel(const float *__restrict__ logits, int vocab,
                                                           int *__restrict__ tokens, int tstride,
                                                           int *__restrict__ pos_p, int n_forced, int max_pos,
                                                           unsigned *__restrict__ ticket_p,
                                                           unsigned long long *__restrict__ slots,
                                                           unsigned *__restrict__ seq_tickets,
                                                           unsigned *__restrict__ pcount, float penalty) {
  constexpr int NT = 1024, IN = 4;   // threads, loads in flight per thread
  __shared__ unsigned long long best[16];
  const int part = blockIdx.x, parts = gridDim.x, b = blockIdx.y;
  const float *lg = logits + size_t(b) * vocab;
  unsigned *pc = pcount ? pcount + size_t(b) * vocab : nullptr;   // repetition penalty: token counts
  unsigned long long key = 0;
  // key = orderable value bits << 32 | ~index: the largest value, the lowest
  // index among equal values; NaN never wins, -0 counts as +0
  const auto fold = [&key, pc, penalty](float v, int i) {
    if (pc) v = penalised_logit(v, pc[i], penalty);
    if (__builtin_isnan(v)) return;
    uint32_t u = __float_as_uint(v + 0.0f);
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    const unsigned long long k = (static_cast<unsigned long long>(u) << 32) | (0xFFFFFFFFu - uint32_t(i));
    key = k > key ? k : key;
  };
  // this part's slice of the row: 16-byte loads (every row is 16-byte aligned
  // when the logits are and vocab % 4 == 0), else 4-byte ones
  const bool vec = vocab % 4 == 0 && reinterpret_cast<size_t>(logits) % 16 == 0;
  const int span = (vocab + 4 * parts - 1) / (4 * parts) * 4;
  const int i0 = part * span, i1 = min(vocab, i0 + span);
  if (vec) {
    const float4 *lg4 = reinterpret_cast<const float4 *>(lg);
    const int q0 = i0 / 4, q1 = i1 / 4;   // i1 is a multiple of 4 or vocab
    for (int q = q0 + int(threadIdx.x); q < q1; q += NT * IN) {
      float4 v[IN];
#pragma unroll
      for (int j = 0; j < IN; ++j) v[j] = lg4[min(q + j * NT, q1 - 1)];
#pragma unroll
      for (int j = 0; j < IN; ++j) {
        const int qq = q + j * NT;
        if (qq < q1) fold(v[j].x, 4 * qq), fold(v[j].y, 4 * qq + 1), fold(v[j].z, 4 * qq + 2), fold(v[j].w, 4 * qq + 3);
      }
    }
  } else {
    for (int i = i0 + int(threadIdx.x); i < i1; i += NT) fold(lg[i], i);
  }
  key = wave_max_key(key, threadIdx.x & (kWave - 1));
  if ((threadIdx.x & (kWave - 1)) == 0) best[threadIdx.x / kWave] = key;
  // the position, read before this part's slot and ticket: the last
  // sequence advances it only after every part has taken its ticket
  int pos = 0;
  if (threadIdx.x == 0) pos = *pos_p;
  __syncthreads();
  if (threadIdx.x != 0) return;
  for (int w = 1; w < 16; ++w) key = best[w] > key ? best[w] : key;
  if (parts > 1) {
    __hip_atomic_store(slots + size_t(b) * parts + part, key, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_s_waitcnt(0);
    const unsigned t =
        __hip_atomic_fetch_add(seq_tickets + b * kTicketPad, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (t != unsigned(parts - 1)) return;   // another part finishes the sequence
    for (int q0 = 0; q0 < parts; q0 += 16) {   // 16 slot loads in flight
      unsigned long long kv[16];
#pragma unroll
      for (int j = 0; j < 16; ++j)
        kv[j] = q0 + j < parts ? __hip_atomic_load(slots + size_t(b) * parts + q0 + j, __ATOMIC_RELAXED,
                                                   __HIP_MEMORY_SCOPE_AGENT)
                               : 0ull;
#pragma unroll
      for (int j = 0; j < 16; ++j) key = kv[j] > key ? kv[j] : key;
    }
    __hip_atomic_store(seq_tickets + b * kTicketPad, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  const int idx = key ? int(0xFFFFFFFFu - uint32_t(key)) : 0;
  if (pos + 1 >= n_forced && pos + 1 <= max_pos) {
    tokens[size_t(b) * tstride + pos + 1] = idx;
    if (pc) pc[idx] += 1u;   // the sampled token joins the history
  }
  __builtin_amdgcn_s_waitcnt(0);
  const unsigned t = __hip_atomic_fetch_add(ticket_p, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (t == gridDim.y - 1) {   // every sequence has read the position
    *pos_p = pos + 1;
    __hip_atomic_store(ticket_p, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// Greedy finish of a step fused with the next step's embedding: the token
// (the largest of the head GEMV's per-wave argmax keys; the encoding keeps
// the first maximum, model.cpp:480-490) is written unless the next position
// is forced, the position advances, and the embedding row of the next token
// (forced or chosen) becomes the hidden state the next step starts from
// (embed_kernel's dequantisation).
template <int FMT>
__global__ __launch_bounds__(1024) void finish_embed_kernel(const unsigned long long *__restrict__ slots, int n_slots,
                                                            int *__restrict__ tokens, int *__restrict__ pos_p,
                                                            int n_forced, int max_pos,
                                                            const uint8_t *__restrict__ planes,
                                                            const float *__restrict__ scales, int Npad, int rows,
                                                            int n_groups, int group_chunks, int cols,
                                                            float *__restrict__ out, unsigned *__restrict__ pcount) {
  constexpr int P = EmbFmt<FMT>::P, S = EmbFmt<FMT>::S;
  constexpr int SL = 4;   // slot loads in flight per thread
  __shared__ unsigned long long best[16];
  __shared__ int next;
  // rounds of SL slot loads per thread (clamped, then dropped past n_slots,
  // so that no load waits in a branch)
  const int last = max(n_slots - 1, 0);
  const auto round = [&](int i0, unsigned long long(&sv)[SL]) {
#pragma unroll
    for (int j = 0; j < SL; ++j) sv[j] = slots[min(i0 + j * 1024, last)];
  };
  const auto fold = [&](int i0, const unsigned long long(&sv)[SL], unsigned long long key) {
#pragma unroll
    for (int j = 0; j < SL; ++j) key = i0 + j * 1024 < n_slots && sv[j] > key ? sv[j] : key;
    return key;
  };
  unsigned long long sv[SL];
  round(int(threadIdx.x), sv);
  // the position, requested behind the first slots (its round trip no
  // longer follows the reduction); thread 0 advances it below, after every
  // read of it
  __builtin_amdgcn_sched_barrier(0);
  const int pos = *pos_p;
  __builtin_amdgcn_sched_barrier(0);
  unsigned long long key = fold(int(threadIdx.x), sv, 0ull);
  for (int i0 = int(threadIdx.x) + 1024 * SL; i0 < n_slots; i0 += 1024 * SL) {
    round(i0, sv);
    key = fold(i0, sv, key);
  }
  key = wave_max_key(key, threadIdx.x & (kWave - 1));
  if ((threadIdx.x & (kWave - 1)) == 0) best[threadIdx.x / kWave] = key;
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < 16; ++w) key = best[w] > key ? best[w] : key;
    const int idx = key ? int(0xFFFFFFFFu - uint32_t(key)) : 0;   // no finite maximum: index 0
    int t = idx;
    if (pos + 1 <= max_pos) {
      if (pos + 1 >= n_forced) {
        tokens[pos + 1] = idx;
        if (pcount) pcount[idx] += 1u;   // the sampled token joins the penalty's history
      } else {
        t = tokens[pos + 1];   // the prompt's token
      }
    }
    *pos_p = pos + 1;
    next = t;
  }
  __syncthreads();
  const int t = min(max(next, 0), rows - 1);
  // two columns per thread and round, every load of a round issued first
  for (int k0 = threadIdx.x; k0 < cols; k0 += 2048) {
    int b[2][P];
    float sc[2][S];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int k = min(k0 + 1024 * h, cols - 1);
      const int c = k / kChunk, byte = (k % kChunk) / 8, bit = 7 - k % 8;
#pragma unroll
      for (int p = 0; p < P; ++p) b[h][p] = (planes[((size_t(c) * P + p) * Npad + t) * 16 + byte] >> bit) & 1;
      const int g = c / group_chunks;
#pragma unroll
      for (int i = 0; i < S; ++i) sc[h][i] = scales[(size_t(i) * n_groups + g) * Npad + t];
    }
    // one wait for both columns: without a use here the compiler sinks the
    // second column's loads into its store's branch, after the first store
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
      for (int p = 0; p < P; ++p) asm volatile("" ::"v"(b[h][p]));
#pragma unroll
      for (int i = 0; i < S; ++i) asm volatile("" ::"v"(sc[h][i]));
    }
#pragma unroll
    for (int h = 0; h < 2; ++h)
      if (k0 + 1024 * h < cols) out[k0 + 1024 * h] = weight_value<FMT>(b[h], sc[h]);
  }
}

int hip_err(hipError_t e, const char *what) {
  if (e == hipErrorOutOfMemory) return fail(LMX_ERR_OUT_OF_MEMORY, "%s: %s", what, hipGetErrorString(e));
  return fail(LMX_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

int launch_err(const char *what) {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? LMX_OK : fail(LMX_ERR_LAUNCH_FAILED, "%s launch: %s", what, hipGetErrorString(e));
}

bool rotates(int fmt) {   // lut_gemm_scalar.cpp:88-96: ternary and 1/2-bit inputs are rotated
  return fmt == LMX_FMT_TERNARY || fmt == LMX_FMT_BINARY || fmt == LMX_FMT_RRQ2 || fmt == LMX_FMT_RRQ3;
}

// The rotation table of every position the cache holds: tab[p * half + d] =
// (cos, sin) of (p / pos_div) * freq[d] (embedding.cpp:36-75), written once
// when the decoder is created, so that attention reads a position's angles
// with its K/V rows instead of reducing large arguments for sincosf.
__global__ __launch_bounds__(256) void rope_table_kernel(const float *__restrict__ freq, float pos_div, int half,
                                                         size_t n, float2 *__restrict__ tab) {
  const size_t i = size_t(blockIdx.x) * 256 + threadIdx.x;
  if (i >= n) return;
  const int p = int(i / size_t(half)), d = int(i % size_t(half));
  const float pf = float(p) / pos_div;
  float sn, cs;
  sincosf(pf * freq[d], &sn, &cs);
  tab[i] = make_float2(cs, sn);
}

// Frequencies theta^(-2d/hd) for d < hd/2, Llama-3 scaled when asked.
std::vector<float> rope_freqs(const lmx_decoder_config &c) {
  const int hd = int(c.head_dim);
  std::vector<float> f(hd / 2);
  for (int d = 0; d < hd / 2; ++d) {
    if (c.rope_mode == LMX_ROPE_REFERENCE) {
      f[d] = 1.0f / std::pow(c.rope_theta, (2.0f * float(d)) / float(hd));   // embedding.cpp:46
      continue;
    }
    const double inv = 1.0 / std::pow(double(c.rope_theta), 2.0 * d / hd);
    const double lo_wl = double(c.rope_orig_max_pos) / c.rope_low_freq_factor;
    const double hi_wl = double(c.rope_orig_max_pos) / c.rope_high_freq_factor;
    const double wl = 2.0 * 3.14159265358979323846 / inv;
    double v;
    if (wl < hi_wl) {
      v = inv;
    } else if (wl > lo_wl) {
      v = inv / c.rope_factor;
    } else {
      const double sm = (double(c.rope_orig_max_pos) / wl - c.rope_low_freq_factor) /
                        (c.rope_high_freq_factor - c.rope_low_freq_factor);
      v = (1.0 - sm) * inv / c.rope_factor + sm * inv;
    }
    f[d] = float(v);
  }
  return f;
}

// One pass of the attention chunk merge over chunks c0 .. c0 + nb - 1 (nb <=
// 64): lane c loads chunk c0 + c's (m, l) and, in the same round trip, the o
// rows of the first MB chunks; later groups of MB follow.  Rescales the
// running (M, L, o) to the pass's new maximum and adds the pass's chunks
// weighted by e^(m_c - M) (each weight read from its lane).
template <int HD, int MB, class Load>
__device__ __forceinline__ void merge_pass(Load ld, int c0, int nb, int lane, float &M, float &L,
                                           float (&o)[HD / kWave]) {
  constexpr int VD = HD / kWave;
  const int c = c0 + lane;
  float mc = -INFINITY, lc = 0.0f;
  if (lane < nb) {
    mc = ld(size_t(c) * (HD + 4));
    lc = ld(size_t(c) * (HD + 4) + 1);
  }
  float v[MB][VD];
#pragma unroll
  for (int jj = 0; jj < MB; ++jj)
#pragma unroll
    for (int u = 0; u < VD; ++u) v[jj][u] = jj < nb ? ld(size_t(c0 + jj) * (HD + 4) + 4 + u * kWave + lane) : 0.0f;
  const float Mn = fmaxf(M, lane_max<32>(mc, lane));   // finite: chunk 0 holds position 0
  const float rs = expf(M - Mn);                        // 0 on the first pass
  L *= rs;
#pragma unroll
  for (int u = 0; u < VD; ++u) o[u] *= rs;
  M = Mn;
  const float wc = lane < nb ? expf(mc - M) : 0.0f;
  L += lane_sum<32>(wc * lc, lane);
  for (int j0 = 0; j0 < nb; j0 += MB) {
    if (j0 > 0) {
#pragma unroll
      for (int jj = 0; jj < MB; ++jj)
#pragma unroll
        for (int u = 0; u < VD; ++u)
          v[jj][u] = j0 + jj < nb ? ld(size_t(c0 + j0 + jj) * (HD + 4) + 4 + u * kWave + lane) : 0.0f;
    }
#pragma unroll
    for (int jj = 0; jj < MB; ++jj) {
      const float w = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wc), j0 + jj));
#pragma unroll
      for (int u = 0; u < VD; ++u) o[u] += w * v[jj][u];
    }
  }
}

// One query head's attention over one 64-position chunk whose K and V rows
// are in LDS (ks padded rows, vs), with the head's rotated q in LDS (qrow),
// the new key (knew, LDS) and value (vn, this lane's columns) for the chunk
// that holds the position (own): scores, a partial softmax and the weighted
// V sum (model.cpp:326-372, attention.cpp:23-42), returned as (m, l, o).
// pwrow is the wave's 64-float LDS scratch.  Every lane of the wave calls it.
// LEAN unrolls the loops partially (fewer registers, for a caller that holds
// the next chunk's rows in registers meanwhile).
template <int HD, bool LEAN = false>
__device__ __forceinline__ void chunk_attend(const float (*ks)[HD + 4], const float (*vs)[HD], const float *qrow,
                                             const float *knew, const float (&vn)[HD / kWave], float *pwrow, int t0,
                                             int pos, bool own, float scale, int lane, float &m, float &l,
                                             float (&o)[HD / kWave]) {
  constexpr int VD = HD / kWave;
  const int t = t0 + lane;
  const bool valid = t <= pos;
  const int n = min(kAttnChunk, pos - t0 + 1);
  const int jnew = own ? pos - t0 : -1;
  const int nold = own ? n - 1 : n;
  float sc = -INFINITY;
  if (valid) {
    const float *kv = lane == jnew ? knew : ks[lane];
    float acc = 0.0f;
    // Stages of SB float4 pairs: a stage's LDS reads are all requested
    // before its multiply-adds (the scheduler otherwise keeps two reads in
    // flight and the one wave per SIMD waits out the LDS latency on every
    // pair); the sum runs in the same order as one read at a time.
    constexpr int SB = LEAN ? 4 : 8;
    static_assert((HD / 4) % SB == 0, "whole stages");
#pragma unroll
    for (int d0 = 0; d0 < HD / 4; d0 += SB) {
      float4 k4[SB], q4[SB];
#pragma unroll
      for (int b = 0; b < SB; ++b) {
        k4[b] = *reinterpret_cast<const float4 *>(kv + 4 * (d0 + b));
        q4[b] = *reinterpret_cast<const float4 *>(qrow + 4 * (d0 + b));
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int b = 0; b < SB; ++b) {
        acc += q4[b].x * k4[b].x;
        acc += q4[b].y * k4[b].y;
        acc += q4[b].z * k4[b].z;
        acc += q4[b].w * k4[b].w;
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    sc = acc * scale;
  }
  m = lane_max<32>(sc, lane);
  const float e = valid ? expf(sc - m) : 0.0f;
  l = lane_sum<32>(e, lane);
  pwrow[lane] = lane < nold ? e : 0.0f;      // cached positions only
  const float enew = __shfl(e, jnew < 0 ? 0 : jnew, 64);
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
#pragma unroll
  for (int u = 0; u < VD; ++u) {
    const int d = u * kWave + lane;
    float s8[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    constexpr int kUnrollJ = LEAN ? 16 : kAttnChunk;
#pragma unroll kUnrollJ
    for (int j = 0; j < kAttnChunk; ++j) s8[j % 8] += pwrow[j] * vs[j][d];
    o[u] = ((s8[0] + s8[1]) + (s8[2] + s8[3])) + ((s8[4] + s8[5]) + (s8[6] + s8[7]));
    if (own) o[u] += enew * vn[u];
  }
}

// Attention with the chunk merge inside: one workgroup per (KV head, CPW
// consecutive 64-position chunks, a "unit", part hs of hsplit of the KV
// head's query heads), 8 waves.  All 8 waves first request the first
// chunk's cached K and V rows of the KV head (every row is in bounds: the
// cache holds whole chunks), so a chunk costs one memory round
// trip whatever the head dimension (a second chunk's rows are requested
// when the first's are in LDS, and arrive while it is attended); chunk by
// chunk the rows pass through LDS and wave w < group/hsplit serves query
// head kvh*group + hs*group/hsplit + w: RoPE of q (and of the new key in
// the chunk holding the position), scores, a partial softmax and the
// weighted V sum of the chunk (model.cpp:326-372, attention.cpp:23-42);
// the unit's chunks combine as (m, l, o[HD]) with the larger maximum.  The
// last workgroup of the KV head's part hs to finish (a device-scope ticket,
// the split-K handoff of the GEMV) merges the units up to the position in order,
// x = sum_u e^(m_u - M) o_u / sum_u e^(m_u - M) l_u with M = max_u m_u, and
// writes the heads' attention output, so the o-projection is a plain GEMV.
// Partials and tickets travel as device-scope relaxed atomics (no L2
// writeback needed); the merging workgroup clears the ticket for the next
// step.  CPW = 2 halves the workgroups where one per chunk would not all be
// resident at once (two workgroups per CU by their LDS); hsplit > 1 spreads
// a small grid's per-head work over more CUs (each part loads the rows).
// Cost follows the position, not the cache capacity (the reference loops
// to pos only, model.cpp:344-372): units below spec_units load their rows
// speculatively, before the position is known; later units read the
// position first and, when it lies before them, load nothing and take no
// ticket (the merge reads units up to the position only).
// PARTS: the q|k|v rows arrive as the batched GEMV's split partials
// qparts [batch][qsplits][qnpad] (no reduction launch before attention); the
// workgroup sums the rows it needs in split order (+ qbias), exactly as the
// batched reduction would, into LDS, loading them in the same round trip as
// the unit's K and V rows.
template <int HD, int CPW, bool PARTS>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(4))) void attn_kernel(const float *__restrict__ qkv, float *__restrict__ kc,
                                                   float *__restrict__ vc, const int *__restrict__ pos_p,
                                                   const float2 *__restrict__ rope, int n_heads,
                                                   int n_kv, int group, int max_seq, float scale,
                                                   float *__restrict__ part, int n_chunks,
                                                   unsigned *__restrict__ tickets, float *__restrict__ out,
                                                   size_t qkv_stride, size_t kv_stride, int spec_units,
                                                   int hsplit, const float *__restrict__ qparts, int qsplits,
                                                   int qnpad, const float *__restrict__ qbias) {
  constexpr int VD = HD / kWave;          // value columns per lane
  constexpr int NT = 512;
  constexpr int KV4 = kAttnChunk * HD / 4 / NT;   // float4 of K (and of V) per thread and chunk
  constexpr int UNIT = CPW * kAttnChunk;          // positions per workgroup
  static_assert(KV4 >= 1, "chunk rows cover the workgroup");
  __shared__ float ks[kAttnChunk][HD + 4];   // padded rows: lane j reads row j without bank conflicts
  __shared__ float vs[kAttnChunk][HD];
  __shared__ float qs[8][HD];
  __shared__ float pw[8][kAttnChunk];
  __shared__ float knew[HD];
  __shared__ float qkvb[PARTS ? (8 + 2) * HD : 1];   // PARTS: the summed q (up to 8 heads), k and v rows
  __shared__ unsigned ticket;
  // Every argument in SGPRs before the first wait: their loads then take one
  // round trip (left to the compiler they came in three batches, each waited
  // for, ahead of the K/V requests).
  asm volatile("" ::"s"(qkv), "s"(kc), "s"(vc), "s"(pos_p), "s"(rope), "s"(part), "s"(tickets), "s"(out));
  asm volatile("" ::"s"(n_heads), "s"(n_kv), "s"(group), "s"(max_seq), "s"(scale), "s"(n_chunks), "s"(qkv_stride),
               "s"(kv_stride), "s"(spec_units), "s"(hsplit));
  if constexpr (PARTS) asm volatile("" ::"s"(qparts), "s"(qsplits), "s"(qnpad), "s"(qbias));
  __builtin_amdgcn_sched_barrier(0);
  {
    // sequence blockIdx.y of a batch: its q|k|v row, KV cache, partials,
    // tickets and output (the position is shared)
    const size_t b = blockIdx.y;
    qkv += b * qkv_stride;
    if constexpr (PARTS) qparts += b * size_t(qsplits) * size_t(qnpad);
    kc += b * kv_stride;
    vc += b * kv_stride;
    part += b * size_t(n_heads) * n_chunks * (HD + 4);
    tickets += b * n_kv * kAttnMaxSplit * kTicketPad;
    out += b * size_t(n_heads) * HD;
  }
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  // part hs of hsplit of the KV head's query heads: hpw heads from h0
  const int hs = blockIdx.x % hsplit, kvu = blockIdx.x / hsplit;
  const int kvh = kvu % n_kv, unit = kvu / n_kv;
  const int hpw = group / hsplit, h0 = kvh * group + hs * hpw;
  const size_t row = size_t(n_kv) * HD;
  const int t0 = unit * UNIT;
  const float *kin = qkv + size_t(n_heads) * HD + kvh * HD;
  const float *vin = kin + row;
  // Past the speculative window a unit learns the position first (an
  // atomic load: never hoisted above this uniform branch, so the window's
  // units issue their loads without waiting for it).
  int pos = 0;
  bool skip = false;
  if (unit >= spec_units) {
    pos = min(__hip_atomic_load(pos_p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT), max_seq - 1);
    skip = t0 > pos;
  }
  if (!skip) {   // uniform over the workgroup

  // ---- every global operand requested before the first wait (one round
  // trip): the unit's K and V rows, the query head's q, the new key and
  // value, and the RoPE frequencies (all waves load them; in bounds) ----
  constexpr int HALF = HD / 2;
  constexpr int RP = (HALF + kWave - 1) / kWave;   // rotation pairs per lane
  float4 kr[KV4], vr[KV4];
  const auto load_rows = [&](int q) {
    // a unit's chunk past the cache's last one (odd chunk count) loads that
    // last chunk's rows and holds no position
    const int tq = min(t0 + q * kAttnChunk, (n_chunks - 1) * kAttnChunk);
#pragma unroll
    for (int i = 0; i < KV4; ++i) {
      const int f = int(threadIdx.x) + i * NT;          // float4 index in the 64 x HD chunk
      const int r = f / (HD / 4), c4 = f % (HD / 4);
      kr[i] = *reinterpret_cast<const float4 *>(kc + size_t(tq + r) * row + kvh * HD + 4 * c4);
      vr[i] = *reinterpret_cast<const float4 *>(vc + size_t(tq + r) * row + kvh * HD + 4 * c4);
    }
  };
  // The position (for the rotation table's row) is requested first and the
  // rows, q, k and v right after it, so that its wait (the loads return in
  // order) leaves them in flight.
  const int praw = __hip_atomic_load(pos_p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __builtin_amdgcn_sched_barrier(0);
  load_rows(0);
  const auto store_rows = [&]() {
#pragma unroll
    for (int i = 0; i < KV4; ++i) {
      const int f = int(threadIdx.x) + i * NT;
      const int r = f / (HD / 4), c4 = f % (HD / 4);
      *reinterpret_cast<float4 *>(&ks[r][4 * c4]) = kr[i];
      *reinterpret_cast<float4 *>(&vs[r][4 * c4]) = vr[i];
    }
  };
  const float *qin = qkv + size_t(h0 + (wave < hpw ? wave : 0)) * HD;
  float qa[RP], qb[RP], ka[RP], kb[RP], vn[VD];
  float2 rt[RP];   // (cos, sin) of the position's rotation angles
  // PARTS: value i < nval of the workgroup's q (hpw heads), k, v rows; thread
  // t sums values t, t + NT, ... (VPT of them) over the splits
  constexpr int VPT = PARTS ? ((8 + 2) * HD + NT - 1) / NT : 1;
  constexpr int NP = PARTS ? kAttnMaxParts : 1;
  const int nq = hpw * HD, nval = nq + 2 * HD;
  const auto qkv_row = [&](int i) {   // value i -> its row of the fused q|k|v output
    return i < nq ? h0 * HD + i : i < nq + HD ? (n_heads + kvh) * HD + (i - nq) : (n_heads + n_kv + kvh) * HD + (i - nq - HD);
  };
  float pv[VPT][NP], pb[VPT];
  if constexpr (PARTS) {
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      const int r = qkv_row(min(int(threadIdx.x) + j * NT, nval - 1));
#pragma unroll
      for (int t = 0; t < NP; ++t) pv[j][t] = t < qsplits ? qparts[size_t(t) * qnpad + r] : 0.0f;
      pb[j] = qbias ? qbias[r] : 0.0f;
    }
  }
  if constexpr (!PARTS) {
#pragma unroll
    for (int i = 0; i < RP; ++i) {
      const int d = min(lane + i * kWave, HALF - 1);
      qa[i] = qin[d];
      qb[i] = qin[d + HALF];
      ka[i] = kin[d];
      kb[i] = kin[d + HALF];
    }
#pragma unroll
    for (int u = 0; u < VD; ++u) vn[u] = vin[u * kWave + lane];
  }
  __builtin_amdgcn_sched_barrier(0);
  pos = min(__builtin_amdgcn_readfirstlane(praw), max_seq - 1);
#pragma unroll
  for (int i = 0; i < RP; ++i) rt[i] = rope[size_t(pos) * HALF + min(lane + i * kWave, HALF - 1)];
  // One wait for all of them: without a use of every loaded value here the
  // compiler issues the small loads after the K/V waits (a second round trip).
#pragma unroll
  for (int i = 0; i < KV4; ++i)
    asm volatile("" ::"v"(kr[i].x), "v"(kr[i].y), "v"(kr[i].z), "v"(kr[i].w), "v"(vr[i].x), "v"(vr[i].y),
                 "v"(vr[i].z), "v"(vr[i].w));
  if constexpr (PARTS) {
#pragma unroll
    for (int i = 0; i < RP; ++i) asm volatile("" ::"v"(rt[i].x), "v"(rt[i].y));
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
#pragma unroll
      for (int t = 0; t < NP; ++t) asm volatile("" ::"v"(pv[j][t]));
      asm volatile("" ::"v"(pb[j]));
    }
    // split-order sums (+ bias), the batched reduction's expression: one
    // round of 16 partials from zero, absent splits adding +0
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      const int i = int(threadIdx.x) + j * NT;
      float sum = 0.0f;
#pragma unroll
      for (int t = 0; t < NP; ++t) sum += pv[j][t];
      if (qbias) sum += pb[j];
      if (i < nval) qkvb[i] = sum;
    }
  } else {
#pragma unroll
    for (int i = 0; i < RP; ++i)
      asm volatile("" ::"v"(rt[i].x), "v"(rt[i].y), "v"(qa[i]), "v"(qb[i]), "v"(ka[i]), "v"(kb[i]));
#pragma unroll
    for (int u = 0; u < VD; ++u) asm volatile("" ::"v"(vn[u]));
  }
  store_rows();   // the first chunk's rows
  if constexpr (PARTS) {
    __syncthreads();   // the summed rows are in qkvb
    const float *qsrc = qkvb + (wave < hpw ? wave : 0) * HD;
#pragma unroll
    for (int i = 0; i < RP; ++i) {
      const int d = min(lane + i * kWave, HALF - 1);
      qa[i] = qsrc[d];
      qb[i] = qsrc[d + HALF];
      ka[i] = qkvb[nq + d];
      kb[i] = qkvb[nq + d + HALF];
    }
#pragma unroll
    for (int u = 0; u < VD; ++u) vn[u] = qkvb[nq + HD + u * kWave + lane];
  }
  const bool live = t0 <= pos;                      // the unit holds positions of the sequence
  const bool own = pos / UNIT == unit;              // the unit holds the new position
  // RoPE: pairs (d, d + HD/2) rotated by the position's angle for d
  // (embedding.cpp:36-75), its cosine and sine read from the decoder's
  // table; computed by every lane so that no load sinks into a branch
#pragma unroll
  for (int i = 0; i < RP; ++i) {
    // each product rounded, then the sum (no fused multiply-add): the
    // reference's a*c - b*s, the same bits in every instantiation
#pragma clang fp contract(off)
    const int d = lane + i * kWave;
    const float cs = rt[i].x, sn = rt[i].y;
    const float q0 = qa[i] * cs - qb[i] * sn, q1 = qa[i] * sn + qb[i] * cs;
    const float k0 = ka[i] * cs - kb[i] * sn, k1 = ka[i] * sn + kb[i] * cs;
    if (live && wave < hpw && d < HALF) {
      qs[wave][d] = q0;
      qs[wave][d + HALF] = q1;
      if (own && wave == 0) {
        knew[d] = k0;
        knew[d + HALF] = k1;
      }
    }
  }

  float o[VD], m = -INFINITY, l = 0.0f;
#pragma unroll
  for (int u = 0; u < VD; ++u) o[u] = 0.0f;
#pragma unroll
  for (int q = 0; q < CPW; ++q) {
    if (q > 0) {
      __syncthreads();   // every wave is done with the previous chunk's rows
      store_rows();
    }
    __syncthreads();
    // the next chunk's rows stream in while this one is attended
    if (q + 1 < CPW) load_rows(q + 1);
    const int tq = t0 + q * kAttnChunk;
    if (wave < hpw && tq <= pos) {   // chunk 0 of a live unit always holds positions
      float mq, lq, oq[VD];
      const bool ownq = pos / kAttnChunk == unit * CPW + q;   // the chunk holds the new position
      chunk_attend<HD, (CPW > 1)>(ks, vs, qs[wave], knew, vn, pw[wave], tq, pos, ownq, scale, lane, mq, lq, oq);
      if (q == 0) {
        m = mq, l = lq;
#pragma unroll
        for (int u = 0; u < VD; ++u) o[u] = oq[u];
      } else {   // both maxima finite: each chunk holds a position
        const float M = fmaxf(m, mq), ra = expf(m - M), rb = expf(mq - M);
        l = l * ra + lq * rb;
#pragma unroll
        for (int u = 0; u < VD; ++u) o[u] = o[u] * ra + oq[u] * rb;
        m = M;
      }
    }
  }

  if (wave < hpw) {
    const int head = h0 + wave;
    float *dst = part + (size_t(head) * n_chunks + unit) * (HD + 4);   // m, l, -, -, o[HD]
#pragma unroll
    for (int u = 0; u < VD; ++u)
      __hip_atomic_store(dst + 4 + u * kWave + lane, o[u], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (lane == 0) {
      __hip_atomic_store(dst, m, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(dst + 1, l, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (own && wave == 0 && hs == 0) {   // append the new position to the cache
#pragma unroll
      for (int u = 0; u < VD; ++u) {
        const int d = u * kWave + lane;
        kc[size_t(pos) * row + kvh * HD + d] = knew[d];
        vc[size_t(pos) * row + kvh * HD + d] = vn[u];
      }
    }
  }
  }   // !skip
  // ---- ticket: the last of the KV head's live units merges ----
  // Units past the position (skipped, or speculative ones that learn it
  // only now) take no ticket, so they never delay the merge.
  if (t0 > pos) return;   // uniform over the workgroup
  const int nlive = pos / UNIT + 1;   // units holding positions
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0)
    ticket = __hip_atomic_fetch_add(tickets + (kvh * kAttnMaxSplit + hs) * kTicketPad, 1u, __ATOMIC_RELAXED,
                                    __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  if (ticket != unsigned(nlive - 1)) return;   // uniform over the workgroup
  if (wave < hpw) {
    const int head = h0 + wave;
    const float *ph = part + size_t(head) * n_chunks * (HD + 4);
    // Passes of 64 units (lane c holds unit c0 + c) rescale a running
    // maximum; the batch of o rows loaded with the weights is sized to the
    // units in use (8 or 32).
    float M = -INFINITY, L = 0.0f, o[VD];
#pragma unroll
    for (int u = 0; u < VD; ++u) o[u] = 0.0f;
    const auto ld = [ph](size_t i) { return __hip_atomic_load(ph + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); };
    for (int c0 = 0; c0 < nlive; c0 += kWave) {
      const int nb = min(kWave, nlive - c0);
      if (nb <= 8)
        merge_pass<HD, 8>(ld, c0, nb, lane, M, L, o);
      else
        merge_pass<HD, 32>(ld, c0, nb, lane, M, L, o);
    }
    const float inv = 1.0f / L;
#pragma unroll
    for (int u = 0; u < VD; ++u) out[size_t(head) * HD + u * kWave + lane] = o[u] * inv;
  }
  if (threadIdx.x == 0)
    __hip_atomic_store(tickets + (kvh * kAttnMaxSplit + hs) * kTicketPad, 0u, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}

size_t attn_chunks(const lmx_decoder_config &c) { return (c.max_seq + kAttnChunk - 1) / kAttnChunk; }

}  // namespace
}  // namespace lmx

using namespace lmx;

struct lmx_decoder {
  lmx_decoder_config cfg{};
  int device = 0;
  size_t batch = 1;   // sequences decoded in lockstep (every per-sequence buffer is [batch][...])
  struct Layer {
    const lmx_weight *qkv = nullptr, *o = nullptr, *gate_up = nullptr, *down = nullptr;
    float *in_norm = nullptr, *post_norm = nullptr, *qkv_bias = nullptr;
  };
  std::vector<Layer> layers;
  const lmx_weight *embed = nullptr, *head = nullptr;   // equal when tied
  float *final_norm = nullptr;
  float *hidden = nullptr, *qkv = nullptr, *gate_up = nullptr, *logits = nullptr;
  float *kcache = nullptr, *vcache = nullptr, *freq = nullptr;
  float2 *rope = nullptr;                // [max_seq][head_dim / 2] (cos, sin) of each position's angles
  float *attn_part = nullptr;            // [n_heads][chunks][m, l, -, -, o[head_dim]]
  float *attn_out = nullptr;             // [n_heads * head_dim] merged attention output
  unsigned *attn_tickets = nullptr;      // [n_kv_heads][kAttnMaxSplit] unit tickets (zero between steps)
  float *normed = nullptr;   // batch > 1: RMSNorm output [hidden] rows
  float *act = nullptr;      // SiLU(gate)*up [ffn] rows
  unsigned *argmax_ticket = nullptr;         // batch > 1: argmax_rows_kernel's ticket
  unsigned long long *argmax_slots = nullptr;   // batch > 1: [batch][kArgmaxParts] keys
  unsigned *argmax_seq_tickets = nullptr;       // batch > 1: [batch] tickets, one 128-byte line each
  size_t kv_seq = 0;                         // floats of one sequence's K (or V) cache, all layers
  unsigned long long *amax = nullptr;    // per-wave argmax keys of the head GEMV
  size_t amax_slots = 0;
  int *tokens = nullptr, *pos = nullptr;
  // Repetition penalty (Model::sample, model.cpp:458-469): off at 1; else
  // pcount [batch][vocab] counts each token's occurrences in the history
  // (the prompt, then every sampled token), kept on the device.
  float penalty = 1.0f;
  unsigned *pcount = nullptr;
  unsigned *penalty_counts() const { return penalty != 1.0f ? pcount : nullptr; }
  int n_forced = 0;
  size_t host_pos = 0;
  float pos_div = 1.0f;
  // Attention chunks that load their K/V rows before the position is known
  // (LMX_ATTN_SPEC overrides; later chunks wait for the position and load
  // only when they hold positions).
  int spec_chunks = 8;
  int n_cu = 256;   // compute units of the device (attention's chunks per workgroup)
  std::vector<void *> allocs;
  hipStream_t stream = nullptr;   // capture/replay stream of lmx_decoder_generate

  int alloc(void **p, size_t bytes) {
    hipError_t e = hipMalloc(p, bytes);
    if (e != hipSuccess) return hip_err(e, "hipMalloc (decoder)");
    allocs.push_back(*p);
    e = hipMemset(*p, 0, bytes);
    return e == hipSuccess ? LMX_OK : hip_err(e, "hipMemset (decoder)");
  }
  ~lmx_decoder() {
    if (stream) (void)hipStreamDestroy(stream);
    for (void *p : allocs) (void)hipFree(p);
  }
};

namespace {

GemvArgs decode_args(const lmx_weight *w, int xmode, int epi) {
  GemvArgs a = weight_args(w);
  a.rotate = rotates(w->format) ? LMX_ROTATE_FWHT256 : LMX_ROTATE_NONE;
  a.xmode = xmode;
  a.epi = epi;
  return a;
}

// The gate|up launch writes SiLU(gate)*up itself (kEpiSiluPair) where its
// kernel plan serves that epilogue; else (or with LMX_SILU_PAIR=0) the down
// projection forms it in its table prologue.
bool gate_up_pairs(const lmx_weight *gate_up) {
  const char *e = std::getenv("LMX_SILU_PAIR");
  return (!e || std::atoi(e) != 0) && silu_pair_rows(gate_up->format, decode_args(gate_up, kXModeRmsNorm, kEpiSiluPair)) > 0;
}

int gemv(const lmx_weight *w, const float *x, float *y, const float *bias, int xmode, const float *xw, float eps,
         hipStream_t st, unsigned long long *amax = nullptr, int epi = kEpiStore, const unsigned *pcount = nullptr,
         float penalty = 1.0f) {
  GemvArgs a = weight_args(w);
  a.epi = epi;
  a.amax = amax;
  a.pcount = pcount;
  a.penalty = penalty;
  a.x = x;
  a.y = y;
  a.bias = bias;
  a.rotate = rotates(w->format) ? LMX_ROTATE_FWHT256 : LMX_ROTATE_NONE;
  a.xmode = xmode;
  a.xw = xw;
  a.eps = eps;
  return launch_gemv(w->format, a, st);
}


template <int FMT>
void launch_embed(const lmx_weight *w, const int *tokens, const int *pos, float *out, size_t batch, int tstride,
                  hipStream_t st) {
  embed_kernel<FMT><<<dim3(unsigned((w->cols + 255) / 256), unsigned(batch)), dim3(256), 0, st>>>(
      static_cast<const uint8_t *>(w->d_planes), w->d_scales, int(w->Npad), int(w->rows), int(w->n_groups),
      int(w->group / kChunk), int(w->cols), tokens, pos, out, tstride);
}

// Embedding rows of `batch` sequences (tokens of sequence b at tokens[b * tstride]).
int embed(const lmx_weight *w, const int *tokens, const int *pos, float *out, size_t batch, int tstride,
          hipStream_t st) {
  switch (w->format) {
  case LMX_FMT_TERNARY: launch_embed<LMX_FMT_TERNARY>(w, tokens, pos, out, batch, tstride, st); break;
  case LMX_FMT_BINARY: launch_embed<LMX_FMT_BINARY>(w, tokens, pos, out, batch, tstride, st); break;
  case LMX_FMT_RRQ2: launch_embed<LMX_FMT_RRQ2>(w, tokens, pos, out, batch, tstride, st); break;
  case LMX_FMT_RRQ3: launch_embed<LMX_FMT_RRQ3>(w, tokens, pos, out, batch, tstride, st); break;
  case LMX_FMT_INT3: launch_embed<LMX_FMT_INT3>(w, tokens, pos, out, batch, tstride, st); break;
  case LMX_FMT_INT4: launch_embed<LMX_FMT_INT4>(w, tokens, pos, out, batch, tstride, st); break;
  case LMX_FMT_INT8: launch_embed<LMX_FMT_INT8>(w, tokens, pos, out, batch, tstride, st); break;
  default: return fail(LMX_ERR_UNSUPPORTED_FORMAT, "embedding format %d", w->format);
  }
  return launch_err("embed");
}

template <int FMT>
void launch_finish_embed(const lmx_decoder *d, hipStream_t st) {
  const lmx_weight *w = d->embed;
  finish_embed_kernel<FMT><<<dim3(1), dim3(1024), 0, st>>>(
      d->amax, int(d->amax_slots), d->tokens, d->pos, d->n_forced, int(d->cfg.max_seq),
      static_cast<const uint8_t *>(w->d_planes), w->d_scales, int(w->Npad), int(w->rows), int(w->n_groups),
      int(w->group / kChunk), int(w->cols), d->hidden, d->penalty_counts());
}

// Greedy finish of a batch-1 step and the embedding of the next token.
int finish_embed(const lmx_decoder *d, hipStream_t st) {
  switch (d->embed->format) {
  case LMX_FMT_TERNARY: launch_finish_embed<LMX_FMT_TERNARY>(d, st); break;
  case LMX_FMT_BINARY: launch_finish_embed<LMX_FMT_BINARY>(d, st); break;
  case LMX_FMT_RRQ2: launch_finish_embed<LMX_FMT_RRQ2>(d, st); break;
  case LMX_FMT_RRQ3: launch_finish_embed<LMX_FMT_RRQ3>(d, st); break;
  case LMX_FMT_INT3: launch_finish_embed<LMX_FMT_INT3>(d, st); break;
  case LMX_FMT_INT4: launch_finish_embed<LMX_FMT_INT4>(d, st); break;
  case LMX_FMT_INT8: launch_finish_embed<LMX_FMT_INT8>(d, st); break;
  default: return fail(LMX_ERR_UNSUPPORTED_FORMAT, "embedding format %d", d->embed->format);
  }
  return launch_err("finish_embed");
}

// qparts: the q|k|v rows as the batched GEMV's split partials
// [batch][qsplits][qnpad] (kEpiPartials) with the q|k|v bias qbias, summed by
// the attention kernel itself; nullptr: the rows are in d->qkv.
int attention(lmx_decoder *d, size_t layer, hipStream_t st, const float *qparts = nullptr, int qsplits = 0,
              int qnpad = 0, const float *qbias = nullptr) {
  const lmx_decoder_config &c = d->cfg;
  const int group = int(c.n_heads / c.n_kv_heads);
  const int nch = int(attn_chunks(c));
  const int spec = min(nch, d->spec_chunks);
  const size_t per_layer = size_t(nch) * kAttnChunk * c.n_kv_heads * c.head_dim;
  float *kc = d->kcache + layer * per_layer, *vc = d->vcache + layer * per_layer;
  const float scale = 1.0f / std::sqrt(float(c.head_dim));   // model.cpp:337
  // Two chunks per workgroup where one per chunk would exceed the two
  // workgroups per CU that the LDS holds (LMX_ATTN_CPW = 1 or 2 overrides).
  const char *cp = std::getenv("LMX_ATTN_CPW");
  const size_t one = c.n_kv_heads * size_t(nch) * d->batch;
  const int cpw = cp ? (std::atoi(cp) == 2 ? 2 : 1) : (one > 2 * size_t(d->n_cu) ? 2 : 1);
  const int units = (nch + cpw - 1) / cpw, spec_units = (spec + cpw - 1) / cpw;
  // The KV head's query heads split over two workgroups (each loads the
  // unit's rows) where that keeps the grid within one workgroup per CU
  // (LMX_ATTN_HS overrides: a divisor of the group, at most 8).
  int hsplit = 1;
  const size_t wgs = c.n_kv_heads * size_t(units) * d->batch;
  if (const char *hv = std::getenv("LMX_ATTN_HS")) {
    const int v = std::atoi(hv);
    if (v >= 1 && v <= kAttnMaxSplit && group % v == 0) hsplit = v;
  } else if (group % 2 == 0 && wgs * 2 <= size_t(d->n_cu)) {
    hsplit = 2;
  }
  const dim3 grid(unsigned(c.n_kv_heads * units * hsplit), unsigned(d->batch));
  const size_t qkv_stride = (c.n_heads + 2 * c.n_kv_heads) * c.head_dim;
  if (qparts && (qsplits < 1 || qsplits > kAttnMaxParts || qnpad < int(qkv_stride)))
    return fail(LMX_ERR_INVALID_ARGUMENT, "attention over %d q|k|v partials of %d rows", qsplits, qnpad);
#define LMX_ATTN(HD, CPW, PARTS)                                                                                    \
  attn_kernel<HD, CPW, PARTS><<<grid, dim3(512), 0, st>>>(                                                         \
      d->qkv, kc, vc, d->pos, d->rope, int(c.n_heads), int(c.n_kv_heads), group, int(c.max_seq), scale, \
      d->attn_part, nch, d->attn_tickets, d->attn_out, qkv_stride, d->kv_seq, spec_units, hsplit, qparts, qsplits,  \
      qnpad, qbias)
  if (qparts) {
    if (c.head_dim == 64) {
      if (cpw == 2) LMX_ATTN(64, 2, true); else LMX_ATTN(64, 1, true);
    } else {
      if (cpw == 2) LMX_ATTN(128, 2, true); else LMX_ATTN(128, 1, true);
    }
  } else if (c.head_dim == 64) {
    if (cpw == 2) LMX_ATTN(64, 2, false); else LMX_ATTN(64, 1, false);
  } else {
    if (cpw == 2) LMX_ATTN(128, 2, false); else LMX_ATTN(128, 1, false);
  }
#undef LMX_ATTN
  return launch_err("attention");
}

int check_shape(const lmx_weight *w, size_t rows, size_t cols, const char *what) {
  if (!w) return fail(LMX_ERR_INVALID_ARGUMENT, "%s weight is NULL", what);
  if (w->rows != rows || w->cols != cols)
    return fail(LMX_ERR_INVALID_ARGUMENT, "%s weight is %zu x %zu, expected %zu x %zu", what, w->rows, w->cols, rows,
                cols);
  return LMX_OK;
}

int upload(lmx_decoder *d, float **dst, const float *src, size_t n) {
  int st = d->alloc(reinterpret_cast<void **>(dst), n * sizeof(float));
  if (st) return st;
  hipError_t e = hipMemcpy(*dst, src, n * sizeof(float), hipMemcpyHostToDevice);
  return e == hipSuccess ? LMX_OK : hip_err(e, "hipMemcpy (decoder weights)");
}

// y[b] = W x[b] (+ bias) (+ resid[b]) for the decoder's `batch` rows: groups
// of 16/8/4 through the batched kernel (weights read once per group), the
// rest one GEMV per row (the residual then rides as that row's bias).
int gemv_rows(const lmx_decoder *d, const lmx_weight *w, const float *x, float *y, const float *bias,
              const float *resid, hipStream_t st) {
  GemvArgs a = weight_args(w);
  a.rotate = rotates(w->format) ? LMX_ROTATE_FWHT256 : LMX_ROTATE_NONE;
  a.bias = bias;
  a.resid = resid;
  size_t done = 0;
  int r = gemv_batched(w, a, x, y, d->batch, st, &done);
  if (r) return r;
  a.resid = nullptr;
  for (size_t b = done; b < d->batch; ++b) {
    a.x = x + b * w->cols;
    a.y = y + b * w->rows;
    a.partials = w->d_partials;
    if (resid) a.bias = resid + b * w->rows;   // decoder rows never carry both
    if ((r = launch_gemv(w->format, a, st))) return r;
  }
  return LMX_OK;
}

// The decoder's rows through the batched kernel with a fused epilogue:
// kEpiNormOut (y = W x + resid, y2 = RMSNorm(y) with weight xw) or
// kEpiSiluPair (y = SiLU(gate)*up rows); every row must be covered
// (rows_fuse checks that first).
int gemv_rows_epi(const lmx_decoder *d, const lmx_weight *w, const float *x, float *y, const float *resid, int epi,
                  const float *xw, float *y2, hipStream_t st) {
  GemvArgs a = weight_args(w);
  a.rotate = rotates(w->format) ? LMX_ROTATE_FWHT256 : LMX_ROTATE_NONE;
  a.resid = resid;
  a.epi = epi;
  a.xw = xw;
  a.eps = d->cfg.rms_eps;
  a.y2 = y2;
  size_t done = 0;
  const int r = gemv_batched(w, a, x, y, d->batch, st, &done);
  if (r) return r;
  return done == d->batch ? LMX_OK
                          : fail(LMX_ERR_INVALID_ARGUMENT, "fused batched epilogue covered %zu of %zu rows", done,
                                 d->batch);
}

// Whether every layer's o / gate|up / down serve the fused epilogues for the
// decoder's batch (LMX_FUSED_ROWS=0: never; the norms and SiLU*up then run
// as row kernels).
bool rows_fuse(const lmx_decoder *d) {
  const char *e = std::getenv("LMX_FUSED_ROWS");
  if (e && std::atoi(e) == 0) return false;
  for (const lmx_decoder::Layer &L : d->layers)
    if (!batched_epilogue_ok(L.o, kEpiNormOut, d->batch) || !batched_epilogue_ok(L.gate_up, kEpiSiluPair, d->batch) ||
        !batched_epilogue_ok(L.down, kEpiNormOut, d->batch))
      return false;
  return true;
}

// Whether a layer's qkv projection leaves its split partials to attention
// (kEpiPartials): the decoder's rows are one batched group whose splits the
// attention kernel sums (LMX_QKV_PARTS=0: never; the batched reduction then
// writes the rows first).
bool qkv_parts(const lmx_decoder *d, const lmx_weight *qkv) {
  const char *e = std::getenv("LMX_QKV_PARTS");
  return !(e && std::atoi(e) == 0) && batched_epilogue_ok(qkv, kEpiPartials, d->batch) &&
         batched_launch_splits(qkv->Npad, qkv->Kp) <= kAttnMaxParts;
}

int rmsnorm_rows(const lmx_decoder *d, const float *x, const float *wt, float *y, hipStream_t st) {
  rmsnorm_rows_kernel<<<dim3(unsigned(d->batch)), dim3(256), 0, st>>>(x, wt, int(d->cfg.hidden), d->cfg.rms_eps, y);
  return launch_err("rmsnorm_rows");
}

int step_batched_rows(lmx_decoder *d, hipStream_t st);

// Four rows of one linear in one group (the four-vector kernel where the
// plan has it, else the batched kernel): y = W x' (+ bias) (+ resid), x' the
// RMSNorm of x with weight xw when xmode asks.
int gemv_group4(const lmx_decoder *d, const lmx_weight *w, const float *x, float *y, const float *bias,
                const float *resid, int xmode, const float *xw, int epi, hipStream_t st) {
  GemvArgs a = decode_args(w, xmode, epi);
  a.bias = bias;
  a.resid = resid;
  a.xw = xw;
  a.eps = d->cfg.rms_eps;
  size_t done = 0;
  const int r = gemv_batched(w, a, x, y, 4, st, &done);
  if (r) return r;
  return done == 4 ? LMX_OK : fail(LMX_ERR_INVALID_ARGUMENT, "a group of 4 rows covered %zu", done);
}

// Batch 4 with every layer's qkv and o on the four-vector kernel (LMX_QUAD_STEP=0:
// never): the norms ride in the kernels' table builds and the residual in
// their epilogues, so the o projection needs no reduction.
bool quad_step(const lmx_decoder *d) {
  const char *e = std::getenv("LMX_QUAD_STEP");
  if (d->batch != 4 || (e && std::atoi(e) == 0) || !d->head->batched) return false;
  for (const lmx_decoder::Layer &L : d->layers)
    if (!quad_serves(decode_args(L.qkv, kXModeRmsNorm, kEpiStore)) || !quad_serves(decode_args(L.o, kXModeNone, kEpiStore)) ||
        !L.qkv->batched || !L.o->batched || !L.gate_up->batched || !L.down->batched ||
        !batched_epilogue_ok(L.gate_up, kEpiSiluPair, 4))
      return false;
  return true;
}

// One token step of `batch` sequences in lockstep: every linear reads its
// weights once per group of sequences.  The batched GEMV splits K, so its
// table build cannot apply the RMSNorm of its input; instead the reduction
// that finishes the o and down projections also writes the normed rows, and
// the gate|up reduction writes SiLU(gate)*up (when every row is in a batched
// group; else the norms and SiLU*up run as row kernels).  Attention and the
// argmax run per sequence.
int step_batched(lmx_decoder *d, float *logits_out, hipStream_t st) {
  const lmx_decoder_config &c = d->cfg;
  const size_t B = d->batch;
  int r = embed(d->embed, d->tokens, d->pos, d->hidden, B, int(c.max_seq + 1), st);
  if (r) return r;
  float *lg = logits_out ? logits_out : d->logits;
  const bool quad = quad_step(d);
  if (quad) {
    // qkv: RMSNorm in the table build; o: + hidden in the epilogue; gate|up:
    // RMSNorm in the batched table build, SiLU(gate)*up in its reduction;
    // down: + hidden in its reduction; the head normalises its own input.
    for (size_t l = 0; l < c.n_layers; ++l) {
      const lmx_decoder::Layer &L = d->layers[l];
      if ((r = gemv_group4(d, L.qkv, d->hidden, d->qkv, L.qkv_bias, nullptr, kXModeRmsNorm, L.in_norm, kEpiStore,
                           st)) ||
          (r = attention(d, l, st)) ||
          (r = gemv_group4(d, L.o, d->attn_out, d->hidden, nullptr, d->hidden, kXModeNone, nullptr, kEpiStore, st)) ||
          (r = gemv_group4(d, L.gate_up, d->hidden, d->act, nullptr, nullptr, kXModeRmsNorm, L.post_norm,
                           kEpiSiluPair, st)) ||
          (r = gemv_group4(d, L.down, d->act, d->hidden, nullptr, d->hidden, kXModeNone, nullptr, kEpiStore, st)))
        return r;
    }
    if ((r = gemv_group4(d, d->head, d->hidden, lg, nullptr, nullptr, kXModeRmsNorm, d->final_norm, kEpiStore, st)))
      return r;
  } else if (rows_fuse(d)) {
    // The o and down reductions write the hidden rows and the next linear's
    // normed input; the gate|up reduction writes SiLU(gate)*up.
    if ((r = rmsnorm_rows(d, d->hidden, d->layers[0].in_norm, d->normed, st))) return r;
    for (size_t l = 0; l < c.n_layers; ++l) {
      const lmx_decoder::Layer &L = d->layers[l];
      const float *next_norm = l + 1 < c.n_layers ? d->layers[l + 1].in_norm : d->final_norm;
      if (qkv_parts(d, L.qkv)) {
        // the qkv split sums go straight to attention (no reduction launch)
        if ((r = gemv_rows_epi(d, L.qkv, d->normed, d->qkv, nullptr, kEpiPartials, nullptr, nullptr, st)) ||
            (r = attention(d, l, st, L.qkv->d_bpartials, batched_launch_splits(L.qkv->Npad, L.qkv->Kp),
                           int(L.qkv->Npad), L.qkv_bias)))
          return r;
      } else if ((r = gemv_rows(d, L.qkv, d->normed, d->qkv, L.qkv_bias, nullptr, st)) || (r = attention(d, l, st))) {
        return r;
      }
      if ((r = gemv_rows_epi(d, L.o, d->attn_out, d->hidden, d->hidden, kEpiNormOut, L.post_norm, d->normed, st)) ||
          (r = gemv_rows_epi(d, L.gate_up, d->normed, d->act, nullptr, kEpiSiluPair, nullptr, nullptr, st)) ||
          (r = gemv_rows_epi(d, L.down, d->act, d->hidden, d->hidden, kEpiNormOut, next_norm, d->normed, st)))
        return r;
    }
  } else {
    if ((r = step_batched_rows(d, st))) return r;
    if ((r = rmsnorm_rows(d, d->hidden, d->final_norm, d->normed, st))) return r;
  }
  if (!quad && (r = gemv_rows(d, d->head, d->normed, lg, nullptr, nullptr, st))) return r;
  // parts per row: about 256 workgroups in all (LMX_ARGMAX_PARTS overrides)
  const char *ap = std::getenv("LMX_ARGMAX_PARTS");
  const int parts = std::max(1, std::min(kArgmaxParts, ap ? std::atoi(ap) : int(256 / B)));
  argmax_rows_kernel<<<dim3(unsigned(parts), unsigned(B)), dim3(1024), 0, st>>>(
      lg, int(c.vocab), d->tokens, int(c.max_seq + 1), d->pos, d->n_forced, int(c.max_seq), d->argmax_ticket,
      d->argmax_slots, d->argmax_seq_tickets, d->penalty_counts(), d->penalty);
  return launch_err("argmax_rows");
}

// The layers of a batched step with the norms and SiLU*up as row kernels.
int step_batched_rows(lmx_decoder *d, hipStream_t st) {
  const lmx_decoder_config &c = d->cfg;
  const size_t B = d->batch;
  int r = LMX_OK;
  for (size_t l = 0; l < c.n_layers; ++l) {
    const lmx_decoder::Layer &L = d->layers[l];
    if ((r = rmsnorm_rows(d, d->hidden, L.in_norm, d->normed, st)) ||
        (r = gemv_rows(d, L.qkv, d->normed, d->qkv, L.qkv_bias, nullptr, st)) ||
        (r = attention(d, l, st)) ||
        (r = gemv_rows(d, L.o, d->attn_out, d->hidden, nullptr, d->hidden, st)) ||
        (r = rmsnorm_rows(d, d->hidden, L.post_norm, d->normed, st)) ||
        (r = gemv_rows(d, L.gate_up, d->normed, d->gate_up, nullptr, nullptr, st)))
      return r;
    silu_mul_rows_kernel<<<dim3(unsigned((c.ffn + 255) / 256), unsigned(B)), dim3(256), 0, st>>>(d->gate_up,
                                                                                                int(c.ffn), d->act);
    if ((r = launch_err("silu_mul_rows")) || (r = gemv_rows(d, L.down, d->act, d->hidden, nullptr, d->hidden, st)))
      return r;
  }
  return LMX_OK;
}

// One token step of one sequence.  The hidden state already holds the
// embedding of the token at the current position (set_position, then each
// step's finish_embed), so the step ends with the greedy finish and the next
// token's embedding in one kernel.
int step(lmx_decoder *d, float *logits_out, hipStream_t st) {
  if (d->batch > 1) return step_batched(d, logits_out, st);
  const lmx_decoder_config &c = d->cfg;
  int r = LMX_OK;
  for (size_t l = 0; l < c.n_layers; ++l) {
    const lmx_decoder::Layer &L = d->layers[l];
    if ((r = gemv(L.qkv, d->hidden, d->qkv, L.qkv_bias, kXModeRmsNorm, L.in_norm, c.rms_eps, st)) ||
        (r = attention(d, l, st)) ||
        (r = gemv(L.o, d->attn_out, d->hidden, d->hidden, kXModeNone, nullptr, 0.0f, st)))
      return r;
    if (gate_up_pairs(L.gate_up)) {
      if ((r = gemv(L.gate_up, d->hidden, d->act, nullptr, kXModeRmsNorm, L.post_norm, c.rms_eps, st, nullptr,
                    kEpiSiluPair)) ||
          (r = gemv(L.down, d->act, d->hidden, d->hidden, kXModeNone, nullptr, 0.0f, st)))
        return r;
    } else if ((r = gemv(L.gate_up, d->hidden, d->gate_up, nullptr, kXModeRmsNorm, L.post_norm, c.rms_eps, st)) ||
               (r = gemv(L.down, d->gate_up, d->hidden, d->hidden, kXModeSiluMul, nullptr, 0.0f, st))) {
      return r;
    }
  }
  float *lg = logits_out ? logits_out : d->logits;
  if ((r = gemv(d->head, d->hidden, lg, nullptr, kXModeRmsNorm, d->final_norm, c.rms_eps, st, d->amax, kEpiStore,
                d->penalty_counts(), d->penalty)))
    return r;
  return finish_embed(d, st);
}

int ready(const lmx_decoder *d) {
  if (!d) return fail(LMX_ERR_INVALID_ARGUMENT, "decoder is NULL");
  if (!d->head) return fail(LMX_ERR_INVALID_ARGUMENT, "decoder head not set");
  for (size_t l = 0; l < d->layers.size(); ++l)
    if (!d->layers[l].qkv) return fail(LMX_ERR_INVALID_ARGUMENT, "decoder layer %zu not set", l);
  return LMX_OK;
}

// tokens: [batch][n], row b the first n tokens of sequence b.
int set_position(lmx_decoder *d, const int32_t *tokens, size_t n, hipStream_t st) {
  if (n == 0 || n > d->cfg.max_seq) return fail(LMX_ERR_INVALID_ARGUMENT, "%zu tokens for max_seq %zu", n, d->cfg.max_seq);
  for (size_t i = 0; i < n * d->batch; ++i)
    if (tokens[i] < 0 || size_t(tokens[i]) >= d->cfg.vocab)
      return fail(LMX_ERR_INVALID_ARGUMENT, "token %d at %zu outside the vocabulary", tokens[i], i);
  const int zero = 0;
  hipError_t e = hipMemcpy2DAsync(d->tokens, (d->cfg.max_seq + 1) * sizeof(int32_t), tokens, n * sizeof(int32_t),
                                  n * sizeof(int32_t), d->batch, hipMemcpyHostToDevice, st);
  if (e == hipSuccess) e = hipMemcpyAsync(d->pos, &zero, sizeof(int), hipMemcpyHostToDevice, st);
  if (e != hipSuccess) return hip_err(e, "decoder reset");
  if (d->batch == 1) {   // a batch-1 step starts from the embedding of the token at its position
    const int r = embed(d->embed, d->tokens, d->pos, d->hidden, 1, int(d->cfg.max_seq + 1), st);
    if (r) return r;
  }
  std::vector<unsigned> hist;   // the penalty's history starts as the whole prompt (inference.cpp:264-268)
  if (d->penalty_counts()) {
    hist.assign(d->batch * d->cfg.vocab, 0u);
    for (size_t b = 0; b < d->batch; ++b)
      for (size_t i = 0; i < n; ++i) hist[b * d->cfg.vocab + size_t(tokens[b * n + i])] += 1u;
    e = hipMemcpyAsync(d->pcount, hist.data(), hist.size() * sizeof(unsigned), hipMemcpyHostToDevice, st);
    if (e != hipSuccess) return hip_err(e, "decoder reset (penalty counts)");
  }
  e = hipStreamSynchronize(st);
  if (e != hipSuccess) return hip_err(e, "decoder reset");
  d->n_forced = int(n);
  d->host_pos = 0;
  return LMX_OK;
}

}  // namespace

extern "C" {

int lmx_decoder_create(const lmx_decoder_config *cfg, lmx_decoder **out) {
  return lmx_decoder_create_batched(cfg, 1, out);
}

int lmx_decoder_create_batched(const lmx_decoder_config *cfg, size_t batch, lmx_decoder **out) {
  if (!cfg || !out) return fail(LMX_ERR_INVALID_ARGUMENT, "NULL argument");
  if (batch == 0 || batch > 64) return fail(LMX_ERR_INVALID_ARGUMENT, "batch %zu outside 1..64", batch);
  *out = nullptr;
  const lmx_decoder_config &c = *cfg;
  if (!c.hidden || !c.n_layers || !c.n_heads || !c.n_kv_heads || !c.ffn || !c.vocab || !c.max_seq)
    return fail(LMX_ERR_INVALID_ARGUMENT, "decoder sizes must be non-zero");
  if (c.head_dim != 64 && c.head_dim != 128) return fail(LMX_ERR_INVALID_ARGUMENT, "head_dim must be 64 or 128");
  if (c.n_heads % c.n_kv_heads || c.n_heads / c.n_kv_heads > 8)
    return fail(LMX_ERR_INVALID_ARGUMENT, "n_heads must be a multiple of n_kv_heads, at most 8 per KV head");
  if (c.hidden % 4 || c.ffn % 4 || (c.n_heads * c.head_dim) % 4)
    return fail(LMX_ERR_INVALID_ARGUMENT, "hidden, ffn and n_heads*head_dim must be multiples of 4");
  if (c.max_seq > (1u << 24)) return fail(LMX_ERR_INVALID_ARGUMENT, "max_seq too large");
  if (c.rope_mode != LMX_ROPE_REFERENCE && c.rope_mode != LMX_ROPE_LLAMA3)
    return fail(LMX_ERR_INVALID_ARGUMENT, "unknown rope mode %d", c.rope_mode);
  if (c.rope_mode == LMX_ROPE_REFERENCE && !(c.rope_factor > 0.0f))
    return fail(LMX_ERR_INVALID_ARGUMENT, "rope factor must be positive");
  if (c.rope_mode == LMX_ROPE_LLAMA3 &&
      !(c.rope_factor > 0.0f && c.rope_high_freq_factor > c.rope_low_freq_factor && c.rope_orig_max_pos > 0))
    return fail(LMX_ERR_INVALID_ARGUMENT, "invalid llama3 rope scaling parameters");
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(LMX_ERR_NO_DEVICE, "hipGetDevice: %s", hipGetErrorString(e));
  lmx_decoder *d = new (std::nothrow) lmx_decoder();
  if (!d) return fail(LMX_ERR_OUT_OF_MEMORY, "decoder allocation");
  d->cfg = c;
  d->device = dev;
  d->batch = batch;
  d->layers.resize(c.n_layers);
  d->pos_div = c.rope_mode == LMX_ROPE_REFERENCE ? c.rope_factor : 1.0f;
  if (const char *sp = std::getenv("LMX_ATTN_SPEC")) d->spec_chunks = std::max(1, std::atoi(sp));
  if (hipDeviceGetAttribute(&d->n_cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || d->n_cu < 1)
    d->n_cu = 256;
  const size_t qkv_rows = (c.n_heads + 2 * c.n_kv_heads) * c.head_dim;
  const size_t kv = c.n_layers * attn_chunks(c) * kAttnChunk * c.n_kv_heads * c.head_dim;   // whole chunks
  d->kv_seq = kv;
  const size_t B = batch;
  const std::vector<float> fr = rope_freqs(c);
  int st;
  if ((st = d->alloc(reinterpret_cast<void **>(&d->hidden), B * c.hidden * 4)) ||
      (st = d->alloc(reinterpret_cast<void **>(&d->qkv), B * qkv_rows * 4)) ||
      (st = d->alloc(reinterpret_cast<void **>(&d->gate_up), B * 2 * c.ffn * 4)) ||
      (st = d->alloc(reinterpret_cast<void **>(&d->logits), B * c.vocab * 4)) ||
      (st = d->alloc(reinterpret_cast<void **>(&d->kcache), B * kv * 4)) ||
      (st = d->alloc(reinterpret_cast<void **>(&d->vcache), B * kv * 4)) ||
      (st = d->alloc(reinterpret_cast<void **>(&d->tokens), B * (c.max_seq + 1) * 4)) ||
      (st = d->alloc(reinterpret_cast<void **>(&d->pos), 4)) ||
      (st = d->alloc(reinterpret_cast<void **>(&d->attn_part),
                     B * c.n_heads * attn_chunks(c) * (c.head_dim + 4) * sizeof(float))) ||
      (st = d->alloc(reinterpret_cast<void **>(&d->attn_out), B * c.n_heads * c.head_dim * sizeof(float))) ||
      (st = d->alloc(reinterpret_cast<void **>(&d->attn_tickets),
                     B * c.n_kv_heads * kAttnMaxSplit * kTicketPad * sizeof(unsigned))) ||
      (B > 1 && (st = d->alloc(reinterpret_cast<void **>(&d->normed), B * c.hidden * 4))) ||
      (st = d->alloc(reinterpret_cast<void **>(&d->act), B * c.ffn * 4)) ||
      (B > 1 && (st = d->alloc(reinterpret_cast<void **>(&d->argmax_ticket), sizeof(unsigned)))) ||
      (B > 1 && (st = d->alloc(reinterpret_cast<void **>(&d->argmax_slots), B * kArgmaxParts * 8))) ||
      (B > 1 && (st = d->alloc(reinterpret_cast<void **>(&d->argmax_seq_tickets),
                               B * kTicketPad * sizeof(unsigned)))) ||
      (st = upload(d, &d->freq, fr.data(), fr.size())) ||
      (st = d->alloc(reinterpret_cast<void **>(&d->rope), c.max_seq * (c.head_dim / 2) * sizeof(float2)))) {
    delete d;
    return st;
  }
  {
    const size_t n = c.max_seq * (c.head_dim / 2);
    rope_table_kernel<<<dim3(unsigned((n + 255) / 256)), dim3(256)>>>(d->freq, d->pos_div, int(c.head_dim / 2), n,
                                                                      d->rope);
    if ((st = launch_err("rope table"))) {
      delete d;
      return st;
    }
    e = hipStreamSynchronize(nullptr);
    if (e != hipSuccess) {
      delete d;
      return hip_err(e, "rope table");
    }
  }
  e = hipStreamCreateWithFlags(&d->stream, hipStreamNonBlocking);
  if (e != hipSuccess) {
    delete d;
    return hip_err(e, "hipStreamCreate (decoder)");
  }
  *out = d;
  return LMX_OK;
}

int lmx_decoder_destroy(lmx_decoder *d) {
  delete d;
  return LMX_OK;
}

int lmx_decoder_set_layer(lmx_decoder *d, size_t layer, const lmx_weight *qkv, const lmx_weight *o,
                          const lmx_weight *gate_up, const lmx_weight *down, const float *input_norm,
                          const float *post_norm, const float *qkv_bias) {
  if (!d) return fail(LMX_ERR_INVALID_ARGUMENT, "decoder is NULL");
  const lmx_decoder_config &c = d->cfg;
  if (layer >= c.n_layers) return fail(LMX_ERR_INVALID_ARGUMENT, "layer %zu >= %zu", layer, c.n_layers);
  if (!input_norm || !post_norm) return fail(LMX_ERR_INVALID_ARGUMENT, "norm weights are NULL");
  const size_t qd = c.n_heads * c.head_dim, kvd = c.n_kv_heads * c.head_dim;
  int st;
  if ((st = check_shape(qkv, qd + 2 * kvd, c.hidden, "qkv")) || (st = check_shape(o, c.hidden, qd, "o")) ||
      (st = check_shape(gate_up, 2 * c.ffn, c.hidden, "gate_up")) || (st = check_shape(down, c.hidden, c.ffn, "down")))
    return st;
  for (const lmx_weight *w : {qkv, o, gate_up, down})
    if (w->device != d->device) return fail(LMX_ERR_INVALID_ARGUMENT, "weight on another device");
  lmx_decoder::Layer &L = d->layers[layer];
  if ((st = upload(d, &L.in_norm, input_norm, c.hidden)) || (st = upload(d, &L.post_norm, post_norm, c.hidden)))
    return st;
  L.qkv_bias = nullptr;
  if (qkv_bias && (st = upload(d, &L.qkv_bias, qkv_bias, qd + 2 * kvd))) return st;
  L.qkv = qkv, L.o = o, L.gate_up = gate_up, L.down = down;
  return LMX_OK;
}

int lmx_decoder_set_head(lmx_decoder *d, const lmx_weight *embed, const lmx_weight *head, const float *final_norm) {
  if (!d) return fail(LMX_ERR_INVALID_ARGUMENT, "decoder is NULL");
  if (!final_norm) return fail(LMX_ERR_INVALID_ARGUMENT, "final norm is NULL");
  int st;
  if ((st = check_shape(embed, d->cfg.vocab, d->cfg.hidden, "embedding")) ||
      (st = check_shape(head, d->cfg.vocab, d->cfg.hidden, "head")))
    return st;
  if (embed->device != d->device || head->device != d->device)
    return fail(LMX_ERR_INVALID_ARGUMENT, "weight on another device");
  if ((st = upload(d, &d->final_norm, final_norm, d->cfg.hidden))) return st;
  const size_t slots = gemv_argmax_slots(weight_args(head));
  if ((st = d->alloc(reinterpret_cast<void **>(&d->amax), slots * sizeof(unsigned long long)))) return st;
  d->amax_slots = slots;
  d->embed = embed;
  d->head = head;
  return LMX_OK;
}

int lmx_decoder_set_repetition_penalty(lmx_decoder *d, float penalty) {
  if (!d) return fail(LMX_ERR_INVALID_ARGUMENT, "decoder is NULL");
  if (!(penalty > 0.0f) || !std::isfinite(penalty))
    return fail(LMX_ERR_INVALID_ARGUMENT, "repetition penalty %g must be positive and finite", double(penalty));
  if (penalty != 1.0f && !d->pcount) {
    const int st = d->alloc(reinterpret_cast<void **>(&d->pcount), d->batch * d->cfg.vocab * sizeof(unsigned));
    if (st) return st;
  }
  d->penalty = penalty;
  return LMX_OK;
}

int lmx_decoder_reset(lmx_decoder *d, const int32_t *tokens, size_t n) {
  int st = ready(d);
  if (st) return st;
  if (!tokens) return fail(LMX_ERR_INVALID_ARGUMENT, "tokens is NULL");
  return set_position(d, tokens, n, nullptr);
}

int lmx_decoder_step(lmx_decoder *d, float *d_logits, void *stream) {
  int st = ready(d);
  if (st) return st;
  if (d->host_pos >= d->cfg.max_seq)
    return fail(LMX_ERR_INVALID_ARGUMENT, "position %zu reached max_seq", d->host_pos);
  st = step(d, d_logits, static_cast<hipStream_t>(stream));
  if (st) return st;
  ++d->host_pos;
  return LMX_OK;
}

int lmx_decoder_tokens(lmx_decoder *d, int32_t *out, size_t n, void *stream) {
  if (!d || !out) return fail(LMX_ERR_INVALID_ARGUMENT, "NULL argument");
  if (n > d->cfg.max_seq + 1) return fail(LMX_ERR_INVALID_ARGUMENT, "n %zu > max_seq + 1", n);
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipError_t e = hipMemcpy2DAsync(out, n * sizeof(int32_t), d->tokens, (d->cfg.max_seq + 1) * sizeof(int32_t),
                                  n * sizeof(int32_t), d->batch, hipMemcpyDeviceToHost, st);
  if (e == hipSuccess) e = hipStreamSynchronize(st);
  return e == hipSuccess ? LMX_OK : hip_err(e, "decoder tokens");
}

int lmx_decoder_generate(lmx_decoder *d, const int32_t *prompt, size_t n_prompt, size_t n_new, int32_t *out_tokens,
                         float *prefill_ms, float *decode_ms, void *stream) {
  int st = ready(d);
  if (st) return st;
  if (!prompt || !out_tokens || n_prompt == 0 || n_new == 0)
    return fail(LMX_ERR_INVALID_ARGUMENT, "need a prompt, an output buffer and n_new > 0");
  if (n_prompt + n_new > d->cfg.max_seq + 1)
    return fail(LMX_ERR_INVALID_ARGUMENT, "n_prompt + n_new = %zu exceeds max_seq + 1", n_prompt + n_new);
  // The caller's stream may be the legacy default stream, which cannot be
  // captured: work runs on the decoder's own stream, ordered after the
  // caller's pending work, and this call returns when it is done.
  hipStream_t s = d->stream;
  {
    hipEvent_t dep = nullptr;
    hipError_t e0 = hipEventCreateWithFlags(&dep, hipEventDisableTiming);
    if (e0 == hipSuccess) e0 = hipEventRecord(dep, static_cast<hipStream_t>(stream));
    if (e0 == hipSuccess) e0 = hipStreamWaitEvent(s, dep, 0);
    if (dep) (void)hipEventDestroy(dep);
    if (e0 != hipSuccess) return hip_err(e0, "decoder stream ordering");
  }
  // One eager step (first-launch set-up of every kernel), then capture.
  if ((st = set_position(d, prompt, n_prompt, s)) || (st = step(d, nullptr, s))) return st;
  hipError_t e = hipStreamSynchronize(s);
  if (e != hipSuccess) return hip_err(e, "decoder warm-up step");
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  e = hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal);
  if (e != hipSuccess) return hip_err(e, "hipStreamBeginCapture");
  st = step(d, nullptr, s);
  e = hipStreamEndCapture(s, &graph);
  if (st) {
    if (graph) (void)hipGraphDestroy(graph);
    return st;
  }
  if (e != hipSuccess) return hip_err(e, "hipStreamEndCapture");
  e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
  (void)hipGraphDestroy(graph);
  if (e != hipSuccess) return hip_err(e, "hipGraphInstantiate");
  hipEvent_t ev[3] = {nullptr, nullptr, nullptr};
  for (auto &x : ev)
    if (e == hipSuccess) e = hipEventCreate(&x);
  if (e == hipSuccess && (st = set_position(d, prompt, n_prompt, s)) != LMX_OK) e = hipErrorUnknown;
  if (e == hipSuccess) e = hipEventRecord(ev[0], s);
  for (size_t i = 0; i < n_prompt && e == hipSuccess; ++i) e = hipGraphLaunch(exec, s);
  if (e == hipSuccess) e = hipEventRecord(ev[1], s);
  for (size_t i = 1; i < n_new && e == hipSuccess; ++i) e = hipGraphLaunch(exec, s);
  if (e == hipSuccess) e = hipEventRecord(ev[2], s);
  if (e == hipSuccess) e = hipEventSynchronize(ev[2]);
  float t0 = 0.0f, t1 = 0.0f;
  if (e == hipSuccess) e = hipEventElapsedTime(&t0, ev[0], ev[1]);
  if (e == hipSuccess) e = hipEventElapsedTime(&t1, ev[1], ev[2]);
  if (e == hipSuccess)
    e = hipMemcpy2D(out_tokens, (n_prompt + n_new) * sizeof(int32_t), d->tokens, (d->cfg.max_seq + 1) * sizeof(int32_t),
                    (n_prompt + n_new) * sizeof(int32_t), d->batch, hipMemcpyDeviceToHost);
  for (auto &x : ev)
    if (x) (void)hipEventDestroy(x);
  (void)hipGraphExecDestroy(exec);
  if (st) return st;
  if (e != hipSuccess) return hip_err(e, "decoder generate");
  d->host_pos = n_prompt + n_new - 1;
  if (prefill_ms) *prefill_ms = t0;
  if (decode_ms) *decode_ms = t1;
  return LMX_OK;
}

}  // extern "C"
