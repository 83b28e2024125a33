// lmx_model.cpp -- .lutmac files onto the device decoder (lutmac_model.h).
//
// Version 1 (src/format.cpp:146-290, types.hpp:44-45): "LUTMAC01", u32
// version 1, u32 metadata size, JSON metadata {"config": {...}, "tensors":
// [{"name", "shape", "offset", "type", "num_blocks", "quant_bits"}, ...]},
// zero padding to a 256-byte boundary, then each tensor's data at
// data_start + offset: its AoS blocks, or raw fp32.
//
// Version 2 (this build's extension, no reference counterpart): the same
// container; a tensor may also be a record {"type": "planes", "format":
// "ternary" | "binary" | "rrq2" | "rrq3" | "int3" | "int4" | "int8",
// "group": G (a multiple of 128, 0 = one scale per row), "rotated": bool,
// "offset", "planes_bytes", "scales_bytes"} whose data is the canonical
// planes [P][rows][cols/8] followed by the scales [S][rows][groups] fp32
// (the lmx_planes_desc layout), so per-128-group scales and RRQ-3 -- which
// the 256-weight blocks cannot express -- have a file form.  "rotated" says
// the weights were FWHT-256-rotated when quantized (lmx_quantize with
// LMX_QUANT_ROTATE); the runtime rotates the activations of ternary, binary
// and RRQ linears (lut_linear's rule), so those formats must be rotated and
// the others not, and the embedding must not be (it is read row by row).
#include <cstdio>
#include <cstring>
#include <fstream>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "lmx_internal.hpp"
#include "lutmac_hip.h"
#include "lutmac_model.h"

namespace {

using lmx::fail;

// ---- a small JSON reader (objects, arrays, strings, numbers, literals) -----
struct JVal {
  enum Kind { Null, Bool, Num, Str, Arr, Obj } kind = Null;
  double num = 0.0;
  std::string str;
  std::vector<JVal> arr;
  std::vector<std::pair<std::string, JVal>> obj;
  const JVal *get(const char *key) const {
    for (const auto &kv : obj)
      if (kv.first == key) return &kv.second;
    return nullptr;
  }
};

struct JParser {
  const char *p, *end;
  bool ok = true;
  void ws() {
    while (p < end && (*p == ' ' || *p == '\n' || *p == '\r' || *p == '\t')) ++p;
  }
  bool lit(const char *s) {
    const size_t n = std::strlen(s);
    if (size_t(end - p) >= n && std::memcmp(p, s, n) == 0) {
      p += n;
      return true;
    }
    return false;
  }
  std::string string() {
    std::string out;
    ++p;   // opening quote
    while (p < end && *p != '"') {
      if (*p == '\\' && p + 1 < end) {
        ++p;
        switch (*p) {
        case 'n': out += '\n'; break;
        case 't': out += '\t'; break;
        case 'r': out += '\r'; break;
        case 'b': out += '\b'; break;
        case 'f': out += '\f'; break;
        case 'u': out += '?', p += (end - p > 4 ? 4 : 0); break;   // names are ASCII
        default: out += *p;
        }
        ++p;
      } else {
        out += *p++;
      }
    }
    if (p >= end) ok = false;
    else ++p;
    return out;
  }
  JVal value(int depth = 0) {
    JVal v;
    ws();
    if (p >= end || depth > 64) {
      ok = false;
      return v;
    }
    if (*p == '{') {
      v.kind = JVal::Obj;
      ++p;
      ws();
      if (p < end && *p == '}') return ++p, v;
      while (ok) {
        ws();
        if (p >= end || *p != '"') return ok = false, v;
        std::string key = string();
        ws();
        if (p >= end || *p != ':') return ok = false, v;
        ++p;
        v.obj.emplace_back(std::move(key), value(depth + 1));
        ws();
        if (p < end && *p == ',') {
          ++p;
          continue;
        }
        if (p < end && *p == '}') return ++p, v;
        ok = false;
      }
      return v;
    }
    if (*p == '[') {
      v.kind = JVal::Arr;
      ++p;
      ws();
      if (p < end && *p == ']') return ++p, v;
      while (ok) {
        v.arr.push_back(value(depth + 1));
        ws();
        if (p < end && *p == ',') {
          ++p;
          continue;
        }
        if (p < end && *p == ']') return ++p, v;
        ok = false;
      }
      return v;
    }
    if (*p == '"') {
      v.kind = JVal::Str;
      v.str = string();
      return v;
    }
    if (lit("true")) return v.kind = JVal::Bool, v.num = 1, v;
    if (lit("false")) return v.kind = JVal::Bool, v;
    if (lit("null")) return v;
    char *e = nullptr;
    std::string tok(p, size_t(std::min<ptrdiff_t>(end - p, 64)));
    v.num = std::strtod(tok.c_str(), &e);
    if (e == tok.c_str()) return ok = false, v;
    v.kind = JVal::Num;
    p += e - tok.c_str();
    return v;
  }
};

double num_or(const JVal &o, const char *key, double dflt) {
  const JVal *v = o.get(key);
  return v && v->kind == JVal::Num ? v->num : dflt;
}

// ---- tensors -----------------------------------------------------------------
struct TensorRec {
  std::string name, type;
  std::vector<size_t> shape;
  size_t offset = 0, num_blocks = 0;
  // version-2 plane records
  int format = 0;
  size_t group = 0, planes_bytes = 0, scales_bytes = 0;
  bool rotated = false;
};

int plane_format(const std::string &f) {
  struct M { const char *name; int fmt; };
  static const M table[] = {{"ternary", LMX_FMT_TERNARY}, {"binary", LMX_FMT_BINARY}, {"rrq2", LMX_FMT_RRQ2},
                            {"rrq3", LMX_FMT_RRQ3},       {"int3", LMX_FMT_INT3},     {"int4", LMX_FMT_INT4},
                            {"int8", LMX_FMT_INT8}};
  for (const M &m : table)
    if (f == m.name) return m.fmt;
  return 0;
}

bool rotated_format(int fmt) {   // lut_gemm_scalar.cpp:88-96
  return fmt == LMX_FMT_TERNARY || fmt == LMX_FMT_BINARY || fmt == LMX_FMT_RRQ2 || fmt == LMX_FMT_RRQ3;
}

// A version-2 plane record's sizes and rotation against its shape and format.
int check_planes(const TensorRec &t) {
  if (!t.format) return fail(LMX_ERR_UNSUPPORTED_FORMAT, "tensor %s: unknown plane format", t.name.c_str());
  if (t.shape.size() != 2 || t.shape[1] % 8)
    return fail(LMX_ERR_INVALID_ARGUMENT, "tensor %s: planes need [rows, cols] with cols a multiple of 8",
                t.name.c_str());
  int P = 0, S = 0;
  lmx_format_info(t.format, &P, &S);
  const size_t rows = t.shape[0], cols = t.shape[1];
  if (t.group && t.group % 128)
    return fail(LMX_ERR_INVALID_ARGUMENT, "tensor %s: group %zu is not a multiple of 128", t.name.c_str(), t.group);
  const size_t ng = t.group ? (cols + t.group - 1) / t.group : 1;
  if (t.planes_bytes != size_t(P) * rows * cols / 8 || t.scales_bytes != size_t(S) * rows * ng * sizeof(float))
    return fail(LMX_ERR_INVALID_ARGUMENT, "tensor %s: plane/scale sizes do not match its shape", t.name.c_str());
  if (t.rotated != rotated_format(t.format))
    return fail(LMX_ERR_UNSUPPORTED_FORMAT,
                "tensor %s: %s weights must %sbe FWHT-rotated (the runtime rotates the activations of ternary, "
                "binary and RRQ linears only)", t.name.c_str(), t.type.c_str(), rotated_format(t.format) ? "" : "not ");
  return LMX_OK;
}

// Reference block type -> (lmx_format, bytes per 256-weight block); 0 when
// this path has no kernel for it.
int type_format(const std::string &t, size_t *bytes) {
  struct M { const char *name; int fmt; size_t bytes; };
  static const M table[] = {{"ternary", LMX_FMT_TERNARY, 68}, {"quantized", LMX_FMT_TERNARY, 68},
                            {"binary", LMX_FMT_BINARY, 36},   {"int2", LMX_FMT_RRQ2, 72},
                            {"int3", LMX_FMT_INT3, 100},      {"int4", LMX_FMT_INT4, 132},
                            {"int8", LMX_FMT_INT8, 260}};
  for (const M &m : table)
    if (t == m.name) {
      *bytes = m.bytes;
      return m.fmt;
    }
  return 0;
}

struct File {
  std::ifstream f;
  size_t data_start = 0;
  int read(size_t off, void *dst, size_t n) {
    f.clear();
    f.seekg(std::streamoff(data_start + off));
    f.read(static_cast<char *>(dst), std::streamsize(n));
    if (!f || size_t(f.gcount()) != n) return fail(LMX_ERR_INVALID_ARGUMENT, "truncated tensor data");
    return LMX_OK;
  }
};

}  // namespace

struct lmx_model {
  lmx_decoder_config cfg{};
  lmx_decoder *dec = nullptr;
  std::vector<lmx_weight *> owned;
  struct L { lmx_weight *w[4] = {nullptr, nullptr, nullptr, nullptr}; };
  std::vector<L> layers;
  lmx_weight *embed = nullptr, *head = nullptr;
  ~lmx_model() {
    if (dec) lmx_decoder_destroy(dec);
    for (lmx_weight *w : owned) lmx_weight_destroy(w);
  }
};

namespace {

// Version-2 plane records -> one device weight: planes and scales of the
// parts concatenated row-wise, plane by plane and stage by stage (all parts
// share format, group and width).
int make_weight_planes(File &file, const std::vector<const TensorRec *> &parts, size_t cols, lmx_model *m,
                       lmx_weight **out) {
  const TensorRec &t0 = *parts[0];
  int P = 0, S = 0;
  lmx_format_info(t0.format, &P, &S);
  size_t rows = 0;
  for (const TensorRec *t : parts) {
    if (t->type != "planes" || t->format != t0.format || t->group != t0.group)
      return fail(LMX_ERR_UNSUPPORTED_FORMAT, "tensor %s: fused tensors must share one format and group",
                  t->name.c_str());
    int st = check_planes(*t);
    if (st) return st;
    if (t->shape[1] != cols)
      return fail(LMX_ERR_INVALID_ARGUMENT, "tensor %s: expected [rows, %zu]", t->name.c_str(), cols);
    rows += t->shape[0];
  }
  const size_t rb = cols / 8, ng = t0.group ? (cols + t0.group - 1) / t0.group : 1;
  std::vector<uint8_t> planes, pbuf;
  std::vector<float> scales, sbuf;
  try {
    planes.resize(size_t(P) * rows * rb);
    scales.resize(size_t(S) * rows * ng);
  } catch (const std::bad_alloc &) {
    return fail(LMX_ERR_OUT_OF_MEMORY, "host buffers for %zu rows", rows);
  }
  size_t r0 = 0;
  for (const TensorRec *t : parts) {
    const size_t tr = t->shape[0];
    pbuf.resize(t->planes_bytes);
    sbuf.resize(t->scales_bytes / sizeof(float));
    int st = file.read(t->offset, pbuf.data(), t->planes_bytes);
    if (!st) st = file.read(t->offset + t->planes_bytes, sbuf.data(), t->scales_bytes);
    if (st) return st;
    for (int p = 0; p < P; ++p)
      std::memcpy(planes.data() + (size_t(p) * rows + r0) * rb, pbuf.data() + size_t(p) * tr * rb, tr * rb);
    for (int s2 = 0; s2 < S; ++s2)
      std::memcpy(scales.data() + (size_t(s2) * rows + r0) * ng, sbuf.data() + size_t(s2) * tr * ng,
                  tr * ng * sizeof(float));
    r0 += tr;
  }
  lmx_planes_desc d{t0.format, rows, cols, t0.group, planes.data(), scales.data()};
  int st = lmx_weight_create(&d, out);
  if (st) return st;
  m->owned.push_back(*out);
  return LMX_OK;
}

// Quantized tensor(s) -> one device weight: the tensors' block arrays
// concatenated row-wise (all must share format and width).
int make_weight(File &file, const std::vector<const TensorRec *> &parts, size_t cols, lmx_model *m,
                lmx_weight **out) {
  if (parts[0]->type == "planes") return make_weight_planes(file, parts, cols, m, out);
  int fmt = 0;
  size_t bytes = 0, rows = 0, nblocks = 0;
  for (const TensorRec *t : parts) {
    size_t b = 0;
    const int f = type_format(t->type, &b);
    if (!f)
      return fail(LMX_ERR_UNSUPPORTED_FORMAT, "tensor %s has type '%s' (no LUT-GEMV kernel for it)", t->name.c_str(),
                  t->type.c_str());
    if (fmt && f != fmt)
      return fail(LMX_ERR_UNSUPPORTED_FORMAT, "tensor %s: fused tensors must share one format", t->name.c_str());
    if (t->shape.size() != 2 || t->shape[1] != cols)
      return fail(LMX_ERR_INVALID_ARGUMENT, "tensor %s: expected [rows, %zu]", t->name.c_str(), cols);
    const size_t bpr = (cols + 255) / 256;
    if (t->num_blocks != t->shape[0] * bpr)
      return fail(LMX_ERR_INVALID_ARGUMENT, "tensor %s: %zu blocks for %zu x %zu", t->name.c_str(), t->num_blocks,
                  t->shape[0], cols);
    fmt = f, bytes = b;
    rows += t->shape[0];
    nblocks += t->num_blocks;
  }
  std::vector<uint8_t> blocks;
  try {
    blocks.resize(nblocks * bytes);
  } catch (const std::bad_alloc &) {
    return fail(LMX_ERR_OUT_OF_MEMORY, "host buffer for %zu blocks", nblocks);
  }
  size_t at = 0;
  for (const TensorRec *t : parts) {
    int st = file.read(t->offset, blocks.data() + at, t->num_blocks * bytes);
    if (st) return st;
    at += t->num_blocks * bytes;
  }
  int st = lmx_weight_from_blocks(fmt, blocks.data(), nblocks, rows, cols, out);
  if (st) return st;
  m->owned.push_back(*out);
  return LMX_OK;
}

int read_raw(File &file, const TensorRec &t, size_t n, std::vector<float> &out) {
  if (!t.type.empty() && t.type != "raw")
    return fail(LMX_ERR_UNSUPPORTED_FORMAT, "tensor %s: expected raw fp32, got '%s'", t.name.c_str(), t.type.c_str());
  size_t count = 1;
  for (size_t s : t.shape) count *= s;
  if (count != n) return fail(LMX_ERR_INVALID_ARGUMENT, "tensor %s has %zu values, expected %zu", t.name.c_str(), count, n);
  out.resize(n);
  return file.read(t.offset, out.data(), n * sizeof(float));
}

bool has(const std::string &s, const char *needle) { return s.find(needle) != std::string::npos; }

}  // namespace

extern "C" {

int lmx_model_load(const char *path, size_t max_seq, lmx_model **out) {
  if (!path || !out) return fail(LMX_ERR_INVALID_ARGUMENT, "NULL argument");
  *out = nullptr;
  File file;
  file.f.open(path, std::ios::binary);
  if (!file.f) return fail(LMX_ERR_INVALID_ARGUMENT, "cannot open %s", path);
  char magic[8];
  uint32_t version = 0, header = 0;
  file.f.read(magic, 8);
  file.f.read(reinterpret_cast<char *>(&version), 4);
  file.f.read(reinterpret_cast<char *>(&header), 4);
  if (!file.f || std::memcmp(magic, "LUTMAC01", 8) != 0)
    return fail(LMX_ERR_INVALID_ARGUMENT, "%s is not a .lutmac file", path);
  if (version != 1 && version != 2)
    return fail(LMX_ERR_UNSUPPORTED_FORMAT, ".lutmac version %u (this loader reads 1 and 2)", version);
  std::string meta(header, '\0');
  file.f.read(&meta[0], std::streamsize(header));
  if (!file.f) return fail(LMX_ERR_INVALID_ARGUMENT, "truncated metadata");
  file.data_start = (16 + size_t(header) + 255) / 256 * 256;   // format.cpp:336-339

  JParser jp{meta.data(), meta.data() + meta.size()};
  const JVal root = jp.value();
  const JVal *config = root.get("config"), *tensors = root.get("tensors");
  if (!jp.ok || !config || config->kind != JVal::Obj || !tensors || tensors->kind != JVal::Arr)
    return fail(LMX_ERR_INVALID_ARGUMENT, "malformed .lutmac metadata");

  // config (format.cpp:320-345 reads the same keys)
  const JVal *mt = config->get("model_type");
  const std::string model_type = mt && mt->kind == JVal::Str ? mt->str : "llama";
  if (model_type == "gemma" || num_or(*config, "activation", 2) == 1)
    return fail(LMX_ERR_UNSUPPORTED_FORMAT, "GELU / Gemma models are not on this path");
  lmx_decoder_config c{};
  c.vocab = size_t(num_or(*config, "vocab_size", 0));
  c.hidden = size_t(num_or(*config, "hidden_size", 0));
  c.ffn = size_t(num_or(*config, "intermediate_size", 0));
  c.n_layers = size_t(num_or(*config, "num_hidden_layers", 0));
  c.n_heads = size_t(num_or(*config, "num_attention_heads", 0));
  c.n_kv_heads = size_t(num_or(*config, "num_key_value_heads", 0));
  c.head_dim = size_t(num_or(*config, "head_dim", 0));
  if (c.head_dim == 0 && c.n_heads) c.head_dim = c.hidden / c.n_heads;   // types.hpp:585-588
  c.rms_eps = float(num_or(*config, "rms_norm_eps", 1e-5));
  c.rope_theta = float(num_or(*config, "rope_theta", 10000.0));
  c.rope_mode = LMX_ROPE_REFERENCE;
  c.rope_factor = float(num_or(*config, "rope_scaling_factor", 1.0));
  if (!(c.rope_factor > 0.0f)) c.rope_factor = 1.0f;                  // format.cpp:331-332
  // KV capacity: the reference never reads max_position_embeddings back
  // (format.cpp:321-342), so its cache holds the default 2048 positions
  // (types.hpp:558, model.hpp:117); a file's 131072 would mean a multi-GB cache.
  c.max_seq = max_seq ? max_seq : 2048;
  if (!c.vocab || !c.hidden || !c.n_layers || !c.n_heads || !c.n_kv_heads)
    return fail(LMX_ERR_INVALID_ARGUMENT, "incomplete model config in %s", path);

  // tensor records
  std::vector<TensorRec> recs;
  for (const JVal &t : tensors->arr) {
    if (t.kind != JVal::Obj) continue;
    TensorRec r;
    const JVal *n = t.get("name"), *ty = t.get("type"), *sh = t.get("shape");
    r.name = n && n->kind == JVal::Str ? n->str : "";
    r.type = ty && ty->kind == JVal::Str ? ty->str : "";
    if (sh && sh->kind == JVal::Arr)
      for (const JVal &d : sh->arr) r.shape.push_back(size_t(d.num));
    r.offset = size_t(num_or(t, "offset", 0));
    r.num_blocks = size_t(num_or(t, "num_blocks", 0));
    if (r.type == "planes") {
      if (version < 2) return fail(LMX_ERR_INVALID_ARGUMENT, "tensor %s: plane records need version 2", r.name.c_str());
      const JVal *f = t.get("format"), *rot = t.get("rotated");
      r.format = f && f->kind == JVal::Str ? plane_format(f->str) : 0;
      r.group = size_t(num_or(t, "group", 0));
      r.rotated = rot && rot->kind == JVal::Bool && rot->num != 0.0;
      r.planes_bytes = size_t(num_or(t, "planes_bytes", 0));
      r.scales_bytes = size_t(num_or(t, "scales_bytes", 0));
    }
    recs.push_back(std::move(r));
  }
  // name -> record, matched as load_model matches (model.cpp:589-660)
  const TensorRec *embed = nullptr, *head = nullptr, *norm = nullptr;
  struct LayerRecs { const TensorRec *q = nullptr, *k = nullptr, *v = nullptr, *o = nullptr, *g = nullptr,
                                       *u = nullptr, *d = nullptr, *in = nullptr, *post = nullptr, *qb = nullptr,
                                       *kb = nullptr, *vb = nullptr; };
  std::vector<LayerRecs> lr(c.n_layers);
  for (const TensorRec &t : recs) {
    const std::string &n = t.name;
    if (n == "embed_tokens" || n == "token_embeddings.weight" || n == "model.embed_tokens.weight") {
      embed = &t;
    } else if (n == "norm.weight" || n == "model.norm.weight") {
      norm = &t;
    } else if (n == "lm_head.weight" || n == "output.weight") {
      head = &t;
    } else if (has(n, "layers.")) {
      const size_t a = n.find("layers.") + 7, b = n.find('.', a);
      if (b == std::string::npos) continue;
      const long li = std::strtol(n.substr(a, b - a).c_str(), nullptr, 10);
      if (li < 0 || size_t(li) >= c.n_layers) continue;
      LayerRecs &L = lr[size_t(li)];
      if (has(n, "input_layernorm.weight")) L.in = &t;
      else if (has(n, "post_attention_layernorm.weight")) L.post = &t;
      else if (has(n, "self_attn.q_proj.weight")) L.q = &t;
      else if (has(n, "self_attn.k_proj.weight")) L.k = &t;
      else if (has(n, "self_attn.v_proj.weight")) L.v = &t;
      else if (has(n, "self_attn.o_proj.weight")) L.o = &t;
      else if (has(n, "self_attn.q_proj.bias")) L.qb = &t;
      else if (has(n, "self_attn.k_proj.bias")) L.kb = &t;
      else if (has(n, "self_attn.v_proj.bias")) L.vb = &t;
      else if (has(n, "mlp.gate_proj.weight")) L.g = &t;
      else if (has(n, "mlp.up_proj.weight")) L.u = &t;
      else if (has(n, "mlp.down_proj.weight")) L.d = &t;
    }
  }
  if (!embed) return fail(LMX_ERR_INVALID_ARGUMENT, "%s has no embedding table", path);
  // Every tensor the decoder needs, checked before any device work.
  auto quantized = [](const TensorRec *t) -> int {
    size_t b = 0;
    if (t->type == "planes") return check_planes(*t);
    if (type_format(t->type, &b)) return LMX_OK;
    return fail(LMX_ERR_UNSUPPORTED_FORMAT, "tensor %s has type '%s' (no LUT-GEMV kernel for it)", t->name.c_str(),
                t->type.c_str());
  };
  {
    int st = quantized(embed);
    if (!st && embed->type == "planes" && embed->rotated)
      return fail(LMX_ERR_UNSUPPORTED_FORMAT, "the embedding must not be rotated (int3, int4 or int8 planes)");
    if (!st && head) st = quantized(head);
    for (size_t l = 0; l < c.n_layers && !st; ++l) {
      const LayerRecs &L = lr[l];
      if (!L.q || !L.k || !L.v || !L.o || !L.g || !L.u || !L.d)
        return fail(LMX_ERR_INVALID_ARGUMENT, "layer %zu is missing a projection", l);
      for (const TensorRec *t : {L.q, L.k, L.v, L.o, L.g, L.u, L.d})
        if (!st) st = quantized(t);
    }
    if (st) return st;
  }

  std::unique_ptr<lmx_model> m(new (std::nothrow) lmx_model());
  if (!m) return fail(LMX_ERR_OUT_OF_MEMORY, "model allocation");
  m->cfg = c;
  m->layers.resize(c.n_layers);
  int st = lmx_decoder_create(&c, &m->dec);
  if (st) return st;
  const size_t qd = c.n_heads * c.head_dim, kvd = c.n_kv_heads * c.head_dim;
  std::vector<float> ones(c.hidden, 1.0f);   // Model::allocate() defaults (model.hpp:74-91)
  for (size_t l = 0; l < c.n_layers; ++l) {
    const LayerRecs &L = lr[l];
    lmx_model::L &W = m->layers[l];
    if ((st = make_weight(file, {L.q, L.k, L.v}, c.hidden, m.get(), &W.w[0])) ||
        (st = make_weight(file, {L.o}, qd, m.get(), &W.w[1])) ||
        (st = make_weight(file, {L.g, L.u}, c.hidden, m.get(), &W.w[2])) ||
        (st = make_weight(file, {L.d}, c.ffn, m.get(), &W.w[3])))
      return st;
    std::vector<float> in = ones, post = ones, bias;
    if (L.in && (st = read_raw(file, *L.in, c.hidden, in))) return st;
    if (L.post && (st = read_raw(file, *L.post, c.hidden, post))) return st;
    if (L.qb || L.kb || L.vb) {
      bias.assign(qd + 2 * kvd, 0.0f);
      std::vector<float> part;
      if (L.qb && (st = read_raw(file, *L.qb, qd, part)) == LMX_OK) std::copy(part.begin(), part.end(), bias.begin());
      if (st) return st;
      if (L.kb && (st = read_raw(file, *L.kb, kvd, part)) == LMX_OK)
        std::copy(part.begin(), part.end(), bias.begin() + qd);
      if (st) return st;
      if (L.vb && (st = read_raw(file, *L.vb, kvd, part)) == LMX_OK)
        std::copy(part.begin(), part.end(), bias.begin() + qd + kvd);
      if (st) return st;
    }
    if ((st = lmx_decoder_set_layer(m->dec, l, W.w[0], W.w[1], W.w[2], W.w[3], in.data(), post.data(),
                                    bias.empty() ? nullptr : bias.data())))
      return st;
  }
  if ((st = make_weight(file, {embed}, c.hidden, m.get(), &m->embed))) return st;
  m->head = m->embed;   // tied unless the file has its own head (model.cpp:667-689)
  if (head && (st = make_weight(file, {head}, c.hidden, m.get(), &m->head))) return st;
  std::vector<float> fn = ones;
  if (norm && (st = read_raw(file, *norm, c.hidden, fn))) return st;
  if ((st = lmx_decoder_set_head(m->dec, m->embed, m->head, fn.data()))) return st;
  *out = m.release();
  return LMX_OK;
}

int lmx_model_destroy(lmx_model *m) {
  delete m;
  return LMX_OK;
}

int lmx_model_config(const lmx_model *m, lmx_decoder_config *cfg) {
  if (!m || !cfg) return fail(LMX_ERR_INVALID_ARGUMENT, "NULL argument");
  *cfg = m->cfg;
  return LMX_OK;
}

lmx_decoder *lmx_model_decoder(lmx_model *m) { return m ? m->dec : nullptr; }

int lmx_model_weight_format(const lmx_model *m, int layer, int which, int *format) {
  if (!m || !format) return fail(LMX_ERR_INVALID_ARGUMENT, "NULL argument");
  const lmx_weight *w = nullptr;
  if (layer == -1) w = m->embed;
  else if (layer == -2) w = m->head;
  else if (layer >= 0 && size_t(layer) < m->layers.size() && which >= 0 && which < 4) w = m->layers[size_t(layer)].w[which];
  if (!w) return fail(LMX_ERR_INVALID_ARGUMENT, "no weight at layer %d / %d", layer, which);
  return lmx_weight_info(w, format, nullptr, nullptr, nullptr);
}

}  // extern "C"
