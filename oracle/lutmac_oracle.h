/*
 * lutmac_oracle.h -- CPU restatement of LutMac's bit-serial LUT-GEMV path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the HIP
 * path in lutmac_amd/.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it, and only as the checker or the timed CPU
 * baseline -- never as the product path.
 *
 * Every function names the reference file:line it restates (paths relative
 * to the LutMac source tree).  Block layouts are passed as raw bytes in the
 * reference's AoS formats (include/lutmac/types.hpp):
 *   BitPlaneBlock 68 B  = sign[32] zero[32] f32 scale            (126-166)
 *   BinaryBlock   36 B  = data[32] f32 scale                     (394-423)
 *   Int2Block     72 B  = data[64] f32 scale f32 scale2          (209-242)
 *   Int3Block    100 B  = data[96] f32 scale                     (249-289)
 *   Int4Block    132 B  = data[128] f32 scale                    (174-202)
 *   Int8Block    260 B  = f32 scale int8[256]                    (434-465)
 *
 * "Canonical planes" (the planar form BASELINE's synthetic weights use):
 *   planes[p][row][Kp/8] bytes, weight k of a row at bit 7-(k%8) of byte k/8
 *   (MSB-first, the reference plane convention), scales[stage][row][Kp/G].
 */
#ifndef LUTMAC_ORACLE_H
#define LUTMAC_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Format codes; equal to lmx_format in include/lutmac_hip.h. */
enum {
  ORC_FMT_TERNARY = 1, /* planes: 0 sign (1 = negative), 1 zero (1 = zero)  */
  ORC_FMT_BINARY = 2,  /* plane 0: 1 = +1, 0 = -1                           */
  ORC_FMT_RRQ2 = 3,    /* planes 0,1 = stage bits; v = sum_i (b_i?+s_i:-s_i) */
  ORC_FMT_RRQ3 = 4,    /* planes 0,1,2 = stage bits                          */
  ORC_FMT_INT3 = 5,    /* plane b = bit b of q in [0,7];  v = (q-4)*s        */
  ORC_FMT_INT4 = 6,    /* plane b = bit b of q in [0,15]; v = (q-8)*s        */
  ORC_FMT_INT8 = 7     /* plane b = bit b of (uint8)q;    v = (int8)q*s      */
};

int orc_format_planes(int fmt);
int orc_format_stages(int fmt);
size_t orc_block_bytes(int fmt); /* reference AoS block size, 0 for RRQ3 */

/* include/lutmac/lut_gemm.hpp:30-44 */
void orc_precompute_lut(const float *a, float *lut);
/* include/lutmac/lut_gemm.hpp:53-58 */
void orc_precompute_luts(const float *x, size_t n, float *luts);
/* include/lutmac/lut_gemm.hpp:79-99 */
void orc_extract_indices(const uint8_t *sign_plane, const uint8_t *zero_plane,
                         size_t group_idx, uint8_t *pos_idx, uint8_t *neg_idx);

/* src/kernels/transform_simd.cpp:14-23,26-45,56-63,94-97 (scalar branch) */
void orc_fwht_256(float *data);
/* src/kernels/transform_simd.cpp:101-110 */
void orc_apply_hadamard_rotation(float *data, size_t n);
/* Length-n orthonormal Walsh-Hadamard transform H_n/sqrt(n), n a power of 2
 * (BASELINE config 2's "length-K FWHT"; no reference counterpart). */
void orc_fwht_full(float *data, size_t n);

/* include/lutmac/quantize.hpp:135-154; ternary values as int8 {-1,0,+1} */
void orc_pack_to_bitplanes(const int8_t *t, size_t n, uint8_t *sign_plane,
                           uint8_t *zero_plane);
/* include/lutmac/quantize.hpp:158-180 */
void orc_unpack_from_bitplanes(const uint8_t *sign_plane,
                               const uint8_t *zero_plane, size_t n, int8_t *t);

/* Scalar GEMVs over reference AoS blocks; y[M] overwritten; x holds
 * ceil(K/256)*256 floats (zero-padded, already rotated when the format needs
 * it), exactly as the reference's raw kernels require. */
/* src/kernels/lut_gemm_scalar.cpp:7-61 */
void orc_ternary_gemv(const uint8_t *blocks, const float *x, float *y, size_t M,
                      size_t K);
/* src/kernels/lut_gemm_scalar.cpp:228-259 */
void orc_binary_gemv(const uint8_t *blocks, const float *x, float *y, size_t M,
                     size_t K);
/* src/kernels/lut_gemm_scalar.cpp:186-222 */
void orc_int4_gemv(const uint8_t *blocks, const float *x, float *y, size_t M,
                   size_t K);
/* src/kernels/lut_gemm_scalar.cpp:298-321 (via Int2Block::get, types.hpp:217-234) */
void orc_int2_gemv(const uint8_t *blocks, const float *x, float *y, size_t M,
                   size_t K);
/* src/kernels/lut_gemm_scalar.cpp:327-350 (via Int3Block::get, types.hpp:256-268) */
void orc_int3_gemv(const uint8_t *blocks, const float *x, float *y, size_t M,
                   size_t K);
/* src/kernels/lut_gemm_scalar.cpp:265-292 */
void orc_int8_gemv(const uint8_t *blocks, const float *x, float *y, size_t M,
                   size_t K);

/* src/kernels/lut_gemm_scalar.cpp:68-180: per batch row, copy+zero-pad x to
 * ceil(K/256)*256, FWHT-256 when the format is ternary/binary/2-bit, dispatch,
 * add bias.  fmt is one of TERNARY, BINARY, RRQ2 (Int2Block), INT3, INT4,
 * INT8.  Returns 0, or -1 for an unsupported format. */
int orc_lut_linear(int fmt, const uint8_t *blocks, const float *bias,
                   const float *x, float *y, size_t M, size_t K, size_t batch);

/* Reference AoS blocks -> canonical planes + scales (group 256), restating the
 * accessors types.hpp:140-149,184-191,217-234,256-268,404-411,464.
 * planes: [P][M][Kp/8], scales: [S][M][Kp/256], Kp = ceil(K/256)*256. */
int orc_blocks_to_planes(int fmt, const uint8_t *blocks, size_t M, size_t K,
                         uint8_t *planes, float *scales);

/* Integer weight value of one stage at (row, k) from canonical planes. */
int orc_plane_value(int fmt, const uint8_t *planes, size_t M, size_t Kp,
                    size_t row, size_t k, int stage);

/* GEMV over canonical planes with group-G scales (G | Kp, G = Kp means one
 * scale per row), two-level accumulation as the reference kernels do it:
 * per group, sum (integer value * x) in k order, then acc += sum * scale,
 * one pass per stage (RRQ = sum of binary GEMVs, cf. lut_gemm_scalar.cpp:228-259). */
void orc_planes_gemv(int fmt, const uint8_t *planes, const float *scales,
                     size_t M, size_t Kp, size_t G, const float *x, float *y);

/* ---- decoder forward ----------------------------------------------------
 * One token step of src/model.cpp:47-453 for a Llama/Qwen-style model whose
 * linears are canonical-plane matrices (cols a multiple of 256, group G | cols):
 * embedding row of the tied table, per layer RMSNorm (norm.cpp:18-34), fused
 * q|k|v rows (+ bias; every linear applies lut_linear's rule: FWHT-256 of
 * the activations for ternary, binary and RRQ weights), RoPE (embedding.cpp:36-75; rope_mode 0 = the
 * reference's (pos/factor)*theta^(-2d/hd), 1 = Llama-3 frequency scaling),
 * KV append, attention with softmax (model.cpp:326-372, attention.cpp:23-42),
 * o + residual, RMSNorm, fused gate|up, SiLU(gate)*up, down + residual;
 * final RMSNorm and the tied head.  kcache/vcache: [layer][max_seq][kv][hd],
 * caller-owned.  Returns 0, or < 0 on bad arguments / allocation failure. */
typedef struct {
  int fmt;
  const uint8_t *planes; /* [P][rows][cols/8] */
  const float *scales;   /* [S][rows][cols/group] */
  size_t rows, cols, group;
} orc_matrix;

typedef struct {
  size_t hidden, n_layers, n_heads, n_kv_heads, head_dim, ffn, vocab, max_seq;
  float rms_eps, rope_theta;
  int rope_mode;
  float rope_factor, rope_low_freq_factor, rope_high_freq_factor;
  size_t rope_orig_max_pos;
  const orc_matrix *qkv, *o, *gate_up, *down; /* [n_layers] each */
  const float *in_norm, *post_norm;           /* [n_layers][hidden] */
  const float *qkv_bias;                      /* [n_layers][qkv rows] or NULL */
  orc_matrix head;                            /* tied embedding / LM head */
  const float *final_norm;
  float *kcache, *vcache;
} orc_model;

int orc_decode_step(const orc_model *m, int token, size_t pos, float *logits);
/* The rotary frequencies the step uses (head_dim/2 floats; reads only the
 * head_dim and rope_* fields). */
void orc_rope_freqs(const orc_model *m, float *out);

#ifdef __cplusplus
}
#endif
#endif
