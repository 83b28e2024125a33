// ref_model_shim.cpp -- extern "C" access to the reference's own Model::forward
// (src/model.cpp:47-453), built into oracle/_ref/libref.so with the
// reference's sources.  TEST INFRASTRUCTURE ONLY: the parity checker and the
// timed CPU decode baseline; never part of the product path.
//
// The model is assembled in memory the way load_model fills it
// (src/model.cpp:576-701): 4-bit linears as Int4Block vectors, the tied
// lm_head as a copy of the 4-bit embedding (model.cpp:667-689), norms, and
// Model::allocate() for the KV cache and buffers.
#include <algorithm>
#include <cstring>
#include <memory>

#include "lutmac/format.hpp"
#include "lutmac/model.hpp"

using namespace lutmac;

namespace {

void fill_int4(PackedTensor &t, const uint8_t *blocks, size_t n, size_t rows, size_t cols) {
  t.shape = {rows, cols};
  t.is_quantized = true;
  t.quant_bits = 4;
  t.int4_blocks.resize(n);
  for (size_t i = 0; i < n; ++i) {
    std::memcpy(t.int4_blocks[i].data, blocks + i * 132, 128);
    std::memcpy(&t.int4_blocks[i].scale, blocks + i * 132 + 128, 4);
  }
}

void fill_int8(PackedTensor &t, const uint8_t *blocks, size_t n, size_t rows, size_t cols) {
  t.shape = {rows, cols};
  t.is_quantized = true;
  t.quant_bits = 8;
  t.int8_blocks.resize(n);
  for (size_t i = 0; i < n; ++i) {   // Int8Block: f32 scale, then int8[256] (types.hpp:434-465)
    std::memcpy(&t.int8_blocks[i].scale, blocks + i * 260, 4);
    std::memcpy(t.int8_blocks[i].data, blocks + i * 260 + 4, 256);
  }
}

PackedTensor raw(const std::string &name, const float *v, size_t n) {
  PackedTensor t;
  t.name = name;
  t.shape = {n};
  t.is_quantized = false;
  t.raw_data.assign(v, v + n);
  return t;
}

PackedTensor named(const PackedTensor &src, const std::string &name) {
  PackedTensor t = src;
  t.name = name;
  return t;
}

}  // namespace

extern "C" {

void *ref_model_create(size_t hidden, size_t n_layers, size_t n_heads, size_t n_kv, size_t head_dim, size_t ffn,
                       size_t vocab, size_t max_seq, float eps, float theta, float rope_factor) {
  auto *m = new Model();
  ModelConfig &c = m->config;
  c.model_type = "llama";
  c.vocab_size = vocab;
  c.hidden_size = hidden;
  c.intermediate_size = ffn;
  c.num_hidden_layers = n_layers;
  c.num_attention_heads = n_heads;
  c.num_key_value_heads = n_kv;
  c.head_dim_val = head_dim;
  c.max_position_embeddings = max_seq;
  c.rms_norm_eps = eps;
  c.rope_theta = theta;
  c.rope_scaling_factor = rope_factor;
  c.activation = ActivationType::SILU;
  m->allocate();
  return m;
}

// which: 0 q, 1 k, 2 v, 3 o, 4 gate, 5 up, 6 down; blocks are Int4Block bytes.
void ref_model_set_linear(void *mp, size_t layer, int which, const uint8_t *blocks, size_t n, size_t rows,
                          size_t cols) {
  TransformerLayer &L = static_cast<Model *>(mp)->layers[layer];
  PackedTensor *t[] = {&L.q_proj, &L.k_proj, &L.v_proj, &L.o_proj, &L.gate_proj, &L.up_proj, &L.down_proj};
  fill_int4(*t[which], blocks, n, rows, cols);
}

void ref_model_set_norms(void *mp, size_t layer, const float *in_norm, const float *post_norm) {
  Model *m = static_cast<Model *>(mp);
  TransformerLayer &L = m->layers[layer];
  const size_t h = m->config.hidden_size;
  L.input_layernorm_weight.assign(in_norm, in_norm + h);
  L.post_attention_layernorm_weight.assign(post_norm, post_norm + h);
}

void ref_model_set_embed(void *mp, const uint8_t *blocks, size_t n, const float *final_norm) {
  Model *m = static_cast<Model *>(mp);
  fill_int4(m->embed_tokens, blocks, n, m->config.vocab_size, m->config.hidden_size);
  m->lm_head = m->embed_tokens;   // tied (model.cpp:667-689)
  m->norm_weight.assign(final_norm, final_norm + m->config.hidden_size);
}

// fmt 6 (Int4Block) or 7 (Int8Block) embedding, tied head.
void ref_model_set_embed_fmt(void *mp, int fmt, const uint8_t *blocks, size_t n, const float *final_norm) {
  Model *m = static_cast<Model *>(mp);
  if (fmt == 7) fill_int8(m->embed_tokens, blocks, n, m->config.vocab_size, m->config.hidden_size);
  else fill_int4(m->embed_tokens, blocks, n, m->config.vocab_size, m->config.hidden_size);
  m->lm_head = m->embed_tokens;
  m->norm_weight.assign(final_norm, final_norm + m->config.hidden_size);
}

void ref_model_set_biases(void *mp, size_t layer, const float *qb, const float *kb, const float *vb) {
  TransformerLayer &L = static_cast<Model *>(mp)->layers[layer];
  std::memcpy(L.q_bias.data(), qb, L.q_bias.size() * sizeof(float));
  std::memcpy(L.k_bias.data(), kb, L.k_bias.size() * sizeof(float));
  std::memcpy(L.v_bias.data(), vb, L.v_bias.size() * sizeof(float));
}

// Writes the model with the reference's own save_lutmac (format.cpp:146-290)
// under the tensor names load_model maps (model.cpp:589-660); the head is
// left out, so loaders tie it to the embedding.  with_biases: also the raw
// q/k/v bias tensors.  Returns 1 on success.
int ref_model_save(void *mp, const char *path, int with_biases) {
  Model *m = static_cast<Model *>(mp);
  const size_t h = m->config.hidden_size;
  std::vector<PackedTensor> ts;
  ts.push_back(named(m->embed_tokens, "model.embed_tokens.weight"));
  ts.push_back(raw("model.norm.weight", m->norm_weight.data(), h));
  for (size_t i = 0; i < m->layers.size(); ++i) {
    const TransformerLayer &L = m->layers[i];
    const std::string p = "model.layers." + std::to_string(i) + ".";
    ts.push_back(raw(p + "input_layernorm.weight", L.input_layernorm_weight.data(), h));
    ts.push_back(raw(p + "post_attention_layernorm.weight", L.post_attention_layernorm_weight.data(), h));
    ts.push_back(named(L.q_proj, p + "self_attn.q_proj.weight"));
    ts.push_back(named(L.k_proj, p + "self_attn.k_proj.weight"));
    ts.push_back(named(L.v_proj, p + "self_attn.v_proj.weight"));
    ts.push_back(named(L.o_proj, p + "self_attn.o_proj.weight"));
    if (with_biases) {
      ts.push_back(raw(p + "self_attn.q_proj.bias", L.q_bias.data(), L.q_bias.size()));
      ts.push_back(raw(p + "self_attn.k_proj.bias", L.k_bias.data(), L.k_bias.size()));
      ts.push_back(raw(p + "self_attn.v_proj.bias", L.v_bias.data(), L.v_bias.size()));
    }
    ts.push_back(named(L.gate_proj, p + "mlp.gate_proj.weight"));
    ts.push_back(named(L.up_proj, p + "mlp.up_proj.weight"));
    ts.push_back(named(L.down_proj, p + "mlp.down_proj.weight"));
  }
  return save_lutmac(path, m->config, ts) ? 1 : 0;
}

// The reference's own load_model (model.cpp:576-701) of a .lutmac file.
void *ref_model_load(const char *path) { return load_model(path).release(); }

void ref_model_forward(void *mp, int token, size_t pos, float *logits) {
  Model *m = static_cast<Model *>(mp);
  m->forward(token, pos);
  std::memcpy(logits, m->logits.data(), m->config.vocab_size * sizeof(float));
}

void ref_model_destroy(void *mp) { delete static_cast<Model *>(mp); }

// Model::sample (model.cpp:455-490) in its greedy form (temperature 0) over
// the given logits and token history: the repetition penalty, then the first
// maximum.  logits_out receives the penalised logits the pick ranked.
int ref_greedy_sample(const float *logits, size_t vocab, const int *history, size_t n_hist, float penalty,
                      float *logits_out) {
  Model m;
  m.config.vocab_size = vocab;
  m.logits.assign(logits, logits + vocab);
  m.generated_tokens.assign(history, history + n_hist);
  GenerationConfig g;
  g.repetition_penalty = penalty;
  g.temperature = 0.0f;
  const int t = m.sample(g);
  std::copy(m.logits.begin(), m.logits.end(), logits_out);
  return t;
}

}  // extern "C"
