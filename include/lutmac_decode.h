/*
 * lutmac_decode.h -- device-resident batch-1 decoder forward over the LUT-GEMV
 * path (C ABI).
 *
 * Replaces Model::forward + greedy Model::sample of the LutMac engine
 * (src/model.cpp:47-453, 455-490) for decoder-only Llama/Qwen-style models
 * whose linear layers are LUT-GEMV weight handles (include/lutmac_hip.h).
 * Everything of a token step stays on the GPU: embedding gather from the
 * tied table, RMSNorm (fused into the next GEMV's table prologue), fused
 * q|k|v GEMV (+ bias), RoPE + KV-cache append + GQA attention in one kernel,
 * o-projection with the residual add fused, fused gate|up GEMV, SiLU(gate)*up
 * fused into the down GEMV's prologue (+ residual), final norm + tied LM head
 * GEMV, greedy argmax.  The position and the token sequence live in device
 * memory, so one captured step replays for every position (HIP graph).
 *
 * Layer weights are borrowed handles (the caller keeps them alive):
 *   qkv      rows [q: n_heads*hd | k: n_kv*hd | v: n_kv*hd] x hidden
 *   o        hidden x n_heads*hd
 *   gate_up  rows [gate: ffn | up: ffn] x hidden
 *   down     hidden x ffn
 *   head     vocab x hidden, also the embedding table (tied, model.cpp:667-689)
 * Numerics are fp32 throughout; KV cache fp32 [layer][pos][kv_head][hd]
 * (types.hpp:599-627 keeps the same per-layer layout).
 */
#ifndef LUTMAC_DECODE_H
#define LUTMAC_DECODE_H

#include <stddef.h>
#include <stdint.h>

#include "lutmac_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* RoPE variants.  REFERENCE: angle = (pos / factor) * theta^(-2d/hd), the
 * reference's apply_rope (src/layers/embedding.cpp:36-75).  LLAMA3: the
 * published Llama-3 frequency scaling of theta^(-2d/hd) (factor,
 * low/high-frequency factors, original context), angle = pos * freq. */
#define LMX_ROPE_REFERENCE 0
#define LMX_ROPE_LLAMA3 1

typedef struct {
  size_t hidden;       /* hidden size */
  size_t n_layers;
  size_t n_heads;      /* query heads */
  size_t n_kv_heads;   /* key/value heads (GQA), divides n_heads, <= 8 query heads each */
  size_t head_dim;     /* 64 or 128 */
  size_t ffn;          /* intermediate size */
  size_t vocab;
  size_t max_seq;      /* KV-cache capacity in positions */
  float rms_eps;
  float rope_theta;
  int rope_mode;       /* LMX_ROPE_* */
  float rope_factor;
  float rope_low_freq_factor;
  float rope_high_freq_factor;
  size_t rope_orig_max_pos;
} lmx_decoder_config;

typedef struct lmx_decoder lmx_decoder;

/* Allocates the device state (activations, KV cache, token buffer) on the
 * current device. */
int lmx_decoder_create(const lmx_decoder_config *cfg, lmx_decoder **out);
/* A decoder of `batch` (1..64) sequences decoded in lockstep at one shared
 * position, each with its own KV cache (no counterpart in the reference,
 * whose Model::forward takes one token; it extends inference.cpp's loop to
 * several sequences so the linears read their weights once per step for
 * all of them).  Every token array of the calls below is then [batch][n]
 * row-major and the logits of lmx_decoder_step [batch][vocab].  batch 1 is
 * lmx_decoder_create. */
int lmx_decoder_create_batched(const lmx_decoder_config *cfg, size_t batch, lmx_decoder **out);
int lmx_decoder_destroy(lmx_decoder *d);
/* Layer weights (borrowed handles) and norm weights (host, copied);
 * qkv_bias (host, n_heads*hd + 2*n_kv*hd floats) may be NULL. */
int lmx_decoder_set_layer(lmx_decoder *d, size_t layer, const lmx_weight *qkv,
                          const lmx_weight *o, const lmx_weight *gate_up,
                          const lmx_weight *down, const float *input_norm,
                          const float *post_norm, const float *qkv_bias);
/* Embedding table and LM head (borrowed; the same handle when tied, as
 * model.cpp:667-689 ties them), both vocab x hidden, and the final norm
 * weight (host). */
int lmx_decoder_set_head(lmx_decoder *d, const lmx_weight *embed,
                         const lmx_weight *head, const float *final_norm);
/* Repetition penalty of the greedy pick (Model::sample, src/model.cpp:458-469;
 * GenerationConfig::repetition_penalty, types.hpp:639).  Before each argmax
 * that picks a token, the logit of every token in the history -- the tokens
 * given to the next lmx_decoder_reset / lmx_decoder_generate, then every
 * picked token -- is divided by `penalty` when positive and multiplied by it
 * otherwise, once per occurrence, as the reference's loop over its
 * generated_tokens does.  1 (the default) turns it off.  The logits
 * lmx_decoder_step writes stay unpenalised.  Applies from the next reset or
 * generate on; the counts live on the device ([batch][vocab] 4-byte words,
 * allocated by the first call with a penalty other than 1). */
int lmx_decoder_set_repetition_penalty(lmx_decoder *d, float penalty);
/* Starts a sequence: position 0, tokens[0..n) = tokens (host).  Positions
 * below n are teacher-forced: their argmax does not overwrite the next
 * token. */
int lmx_decoder_reset(lmx_decoder *d, const int32_t *tokens, size_t n);
/* One forward step at the current position (Model::forward(token, pos)):
 * logits into d_logits (device, vocab floats) when not NULL, the greedy
 * next token into the token buffer, position + 1. */
int lmx_decoder_step(lmx_decoder *d, float *d_logits, void *stream);
/* Copies tokens[0..n) of the device token buffer to the host (synchronous). */
int lmx_decoder_tokens(lmx_decoder *d, int32_t *out, size_t n, void *stream);
/* Greedy generation as inference.cpp does it (prompt token by token, then
 * n_new tokens), with the step captured once in a HIP graph and replayed.
 * out_tokens (host) receives n_prompt + n_new tokens.  The work runs on the
 * decoder's own stream after the work already queued on `stream`; the call
 * returns when it is done.  Timings (ms, HIP events): prefill = the n_prompt
 * steps over the prompt (the last one yields the first new token), decode =
 * the n_new - 1 steps that yield the remaining tokens. */
int lmx_decoder_generate(lmx_decoder *d, const int32_t *prompt, size_t n_prompt,
                         size_t n_new, int32_t *out_tokens, float *prefill_ms,
                         float *decode_ms, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* LUTMAC_DECODE_H */
