// sg_gguf.cpp -- GGUF v3 model images into the library (the INT8 path of
// LoadModel / LoadModelFromBytes, internal/runtime/model.go:236-262).
//
// Restated behaviour of the reference reader (internal/gguf/reader.go:98-178,
// format.go) and loader:
//   - little-endian header: magic "GGUF", version 3 only, u64 tensor count,
//     u64 metadata count; metadata values of types 0..12 (arrays nest);
//     tensor infos (name, u32 ndim, u64 dims, u32 dtype, u64 offset);
//   - tensor data starts at the end of the infos rounded up to 32 bytes
//     (the reader ignores general.alignment); a tensor's size is
//     ceil(elements / elements_per_block) * block_bytes from the dtype table;
//   - configuration as parseConfig (model.go:424-517): architecture prefix,
//     required uint32 embedding_length / block_count / attention.head_count,
//     optional head_count_kv (default: head_count), feed_forward_length
//     (default: blk.0.ffn_up.weight dims[1], else 3 * embedding_length),
//     context_length (2048), attention.layer_norm_rms_epsilon (1e-6) and
//     rope.freq_base (10000) when float32, vocabulary = length of
//     tokenizer.ggml.tokens (else the number of tensors);
//   - token_embd.weight (or model.embed_tokens.weight) and the seven layer
//     matrices must be Q8_0 (model.go:520-552, model_int8.go:54-140);
//     attn_norm / ffn_norm are required, the q/k norms, post norms and
//     output_norm optional (their load errors are ignored); norms are F32 or
//     Q8_0 (dequantized with gguf's fp16 converter, tensor.go:114-240).
// Where the Go code would panic (a required key of another integer type, a
// tensor smaller than its shape, an embedding table shorter than the
// vocabulary), this reader returns SG_ERR_INVALID with a message instead.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include "semantica_gpu.h"
#include "sg_internal.h"

namespace {

using sgi::fail;

enum : uint32_t { M_U8, M_I8, M_U16, M_I16, M_U32, M_I32, M_F32, M_BOOL, M_STR, M_ARR, M_U64, M_I64, M_F64 };
enum : uint32_t { D_F32 = 0, D_F16 = 1, D_Q8_0 = 8 };

struct Meta {
  uint32_t type = 0;
  uint64_t u = 0;  // integer and bool payloads (raw bits for float32)
  double f = 0;    // float payloads
  std::string s;
  uint64_t arr_len = 0;
  uint32_t elem_type = 0;   // arrays: element type
  std::vector<Meta> elems;  // arrays: the elements (the tokenizer reads them)
};

struct Tensor {
  uint32_t dtype = 0;
  std::vector<uint64_t> dims;
  uint64_t offset = 0, size = 0;
};

struct Gguf {
  const uint8_t* base = nullptr;
  size_t size = 0, data_off = 0;
  uint64_t n_tensors = 0;
  std::unordered_map<std::string, Meta> meta;
  std::unordered_map<std::string, Tensor> tensors;
};

struct Cursor {
  const uint8_t* p;
  size_t n, off = 0;
  bool ok = true;
  template <typename T>
  T get() {
    T v{};
    if (!ok || n - off < sizeof(T)) {
      ok = false;
      return v;
    }
    memcpy(&v, p + off, sizeof(T));
    off += sizeof(T);
    return v;
  }
  std::string str() {
    const uint64_t len = get<uint64_t>();
    if (!ok || len > n - off) {
      ok = false;
      return {};
    }
    std::string s(reinterpret_cast<const char*>(p + off), len);
    off += len;
    return s;
  }
};

// Element bytes and elements per block of the dtypes the reader sizes
// (format.go BlockSize / ElementsPerBlock); 0 for the rest.
void dtype_block(uint32_t d, int& bytes, int& per) {
  static const int tb[21][2] = {{4, 1},  {2, 1},  {18, 16}, {20, 16}, {0, 0}, {0, 0}, {22, 16},
                                {24, 16}, {34, 32}, {36, 32}, {0, 0},  {0, 0}, {0, 0}, {0, 0},
                                {0, 0},  {0, 0},  {1, 1},   {2, 1},   {4, 1}, {8, 1}, {8, 1}};
  bytes = d < 21 ? tb[d][0] : 0;
  per = d < 21 ? tb[d][1] : 0;
}

const char* dtype_name(uint32_t d) {
  static const char* names[] = {"F32",  "F16",  "Q4_0", "Q4_1", "?",    "?",    "Q5_0", "Q5_1", "Q8_0", "Q8_1",
                                "Q2_K", "Q3_K", "Q4_K", "Q5_K", "Q6_K", "Q8_K", "I8",   "I16",  "I32",  "I64",
                                "F64"};
  return d < 21 ? names[d] : "Unknown";
}

bool read_value(Cursor& c, uint32_t type, Meta* out, int depth) {
  if (depth > 8) return false;
  switch (type) {
    case M_U8: case M_I8: case M_BOOL: { const uint8_t v = c.get<uint8_t>(); if (out) out->u = v; break; }
    case M_U16: case M_I16: { const uint16_t v = c.get<uint16_t>(); if (out) out->u = v; break; }
    case M_U32: case M_I32: { const uint32_t v = c.get<uint32_t>(); if (out) out->u = v; break; }
    case M_F32: {
      const uint32_t v = c.get<uint32_t>();
      if (out) {
        float f;
        memcpy(&f, &v, 4);
        out->u = v;
        out->f = f;
      }
      break;
    }
    case M_U64: case M_I64: { const uint64_t v = c.get<uint64_t>(); if (out) out->u = v; break; }
    case M_F64: {
      const uint64_t v = c.get<uint64_t>();
      if (out) memcpy(&out->f, &v, 8);
      break;
    }
    case M_STR: {
      std::string s = c.str();
      if (out) out->s = std::move(s);
      break;
    }
    case M_ARR: {
      const uint32_t et = c.get<uint32_t>();
      const uint64_t len = c.get<uint64_t>();
      if (!c.ok || len > c.n) return false;  // every element takes at least one byte
      if (out) {
        out->arr_len = len;
        out->elem_type = et;
        out->elems.resize(len);
      }
      for (uint64_t i = 0; i < len && c.ok; i++) {
        Meta* e = out ? &out->elems[i] : nullptr;
        if (e) e->type = et;
        if (!read_value(c, et, e, depth + 1)) return false;
      }
      break;
    }
    default:
      return false;
  }
  return c.ok;
}

// reader.go:98-178
int parse(const void* data, size_t size, Gguf& g) {
  if (!data) return fail(SG_ERR_INVALID, "NULL argument");
  if (size < 24) return fail(SG_ERR_INVALID, "file too small for header");
  Cursor c{static_cast<const uint8_t*>(data), size};
  const uint32_t magic = c.get<uint32_t>();
  if (magic != 0x46554747u) return fail(SG_ERR_INVALID, "invalid magic: 0x%08x", magic);
  const uint32_t version = c.get<uint32_t>();
  if (version != 3) return fail(SG_ERR_INVALID, "unsupported version: %u", version);
  g.base = static_cast<const uint8_t*>(data);
  g.size = size;
  g.n_tensors = c.get<uint64_t>();
  const uint64_t n_kv = c.get<uint64_t>();
  if (n_kv > size || g.n_tensors > size) return fail(SG_ERR_INVALID, "metadata or tensor count exceeds the file");
  for (uint64_t i = 0; i < n_kv; i++) {
    std::string key = c.str();
    Meta m;
    m.type = c.get<uint32_t>();
    if (!c.ok) return fail(SG_ERR_INVALID, "read metadata %llu: truncated", (unsigned long long)i);
    if (!read_value(c, m.type, &m, 0))
      return fail(SG_ERR_INVALID, "read metadata %llu (%s): bad or truncated value of type %u", (unsigned long long)i,
                  key.c_str(), m.type);
    g.meta[key] = std::move(m);
  }
  for (uint64_t i = 0; i < g.n_tensors; i++) {
    std::string name = c.str();
    Tensor t;
    const uint32_t nd = c.get<uint32_t>();
    if (!c.ok || nd > 8) return fail(SG_ERR_INVALID, "read tensor info %llu: bad dimensions", (unsigned long long)i);
    uint64_t elems = 1;
    for (uint32_t j = 0; j < nd; j++) {
      const uint64_t d = c.get<uint64_t>();
      t.dims.push_back(d);
      elems = d && elems > UINT64_MAX / d ? UINT64_MAX : elems * d;
    }
    t.dtype = c.get<uint32_t>();
    t.offset = c.get<uint64_t>();
    if (!c.ok) return fail(SG_ERR_INVALID, "read tensor info %llu: truncated", (unsigned long long)i);
    int bb, per;
    dtype_block(t.dtype, bb, per);
    if (elems > (UINT64_MAX >> 8))
      t.size = UINT64_MAX;  // cannot fit any file; rejected when its data is read
    else
      t.size = (bb > 0 && per > 0) ? (elems + per - 1) / per * (uint64_t)bb : elems * (uint64_t)bb;
    g.tensors[name] = std::move(t);
  }
  g.data_off = (c.off + 31) & ~size_t(31);
  return SG_OK;
}

const Meta* find(const Gguf& g, const std::string& k) {
  auto it = g.meta.find(k);
  return it == g.meta.end() ? nullptr : &it->second;
}

int req_u32(const Gguf& g, const std::string& k, int32_t& out) {
  const Meta* m = find(g, k);
  if (!m) return fail(SG_ERR_INVALID, "%s not found", k.c_str());
  if (m->type != M_U32) return fail(SG_ERR_INVALID, "%s has metadata type %u, want uint32", k.c_str(), m->type);
  out = (int32_t)m->u;
  return SG_OK;
}

// parseConfig, model.go:424-517
int config_of(const Gguf& g, sg_model_config& c) {
  c = sg_model_config{};
  c.norm_eps = 1e-6f;
  c.rope_base = 10000.0f;
  c.max_seq_len = 2048;
  std::string prefix;
  if (const Meta* a = find(g, "general.architecture"); a && a->type == M_STR && !a->s.empty()) prefix = a->s + ".";
  if (int r = req_u32(g, prefix + "embedding_length", c.embed_dim)) return r;
  if (int r = req_u32(g, prefix + "block_count", c.num_layers)) return r;
  if (int r = req_u32(g, prefix + "attention.head_count", c.num_heads)) return r;
  if (const Meta* m = find(g, prefix + "attention.head_count_kv")) {
    if (m->type != M_U32) return fail(SG_ERR_INVALID, "%sattention.head_count_kv is not uint32", prefix.c_str());
    c.num_kv_heads = (int32_t)m->u;
  } else {
    c.num_kv_heads = c.num_heads;
  }
  if (const Meta* m = find(g, prefix + "feed_forward_length")) {
    if (m->type != M_U32) return fail(SG_ERR_INVALID, "%sfeed_forward_length is not uint32", prefix.c_str());
    c.interm_dim = (int32_t)m->u;
  } else if (auto it = g.tensors.find("blk.0.ffn_up.weight"); it != g.tensors.end() && it->second.dims.size() >= 2) {
    c.interm_dim = (int32_t)it->second.dims[1];
  } else {
    c.interm_dim = 3 * c.embed_dim;
  }
  if (const Meta* m = find(g, prefix + "context_length")) {
    if (m->type != M_U32) return fail(SG_ERR_INVALID, "%scontext_length is not uint32", prefix.c_str());
    c.max_seq_len = (int32_t)m->u;
  }
  if (const Meta* m = find(g, prefix + "attention.layer_norm_rms_epsilon"); m && m->type == M_F32) c.norm_eps = (float)m->f;
  if (const Meta* m = find(g, prefix + "rope.freq_base"); m && m->type == M_F32) c.rope_base = (float)m->f;
  if (const Meta* m = find(g, "tokenizer.ggml.tokens"); m && m->type == M_ARR)
    c.vocab_size = (int32_t)m->arr_len;
  else
    c.vocab_size = (int32_t)g.tensors.size();
  return SG_OK;
}

// fp16 -> fp32 as gguf/tensor.go:207-240 converts (subnormals come out halved).
float f16_gguf(uint16_t h) {
  const uint32_t sign = (h >> 15) & 1u, ex = (h >> 10) & 0x1fu;
  uint32_t m = h & 0x3ffu, bits;
  if (ex == 0) {
    if (m == 0) {
      bits = sign << 31;
    } else {
      uint32_t e = 112u;
      while ((m & 0x400u) == 0) {
        m <<= 1;
        e--;
      }
      bits = (sign << 31) | (e << 23) | ((m & 0x3ffu) << 13);
    }
  } else if (ex == 0x1f) {
    bits = (sign << 31) | (0xffu << 23) | (m << 13);
  } else {
    bits = (sign << 31) | (((ex + 112u) & 0xffu) << 23) | (m << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

struct Loaded {
  sg_model_desc desc{};
  std::vector<sg_layer_desc> layers;
  std::vector<std::vector<float>> owned;  // dequantized norms
};

const uint8_t* tensor_bytes(const Gguf& g, const Tensor& t) {
  const uint64_t off = (uint64_t)g.data_off + t.offset;
  if (off < t.offset || off > g.size || t.size > g.size - off) return nullptr;
  return g.base + off;
}

// A Q8_0 matrix [rows][cols] (GGUF dims {cols, rows}).
int q8_matrix(const Gguf& g, const std::string& name, int rows, int cols, const void*& out) {
  auto it = g.tensors.find(name);
  if (it == g.tensors.end()) return fail(SG_ERR_INVALID, "tensor not found: %s", name.c_str());
  const Tensor& t = it->second;
  if (t.dtype != D_Q8_0) return fail(SG_ERR_INVALID, "expected Q8_0, got %s for %s", dtype_name(t.dtype), name.c_str());
  if (t.dims.size() < 2 || t.dims[0] != (uint64_t)cols || t.dims[1] != (uint64_t)rows)
    return fail(SG_ERR_INVALID, "%s: shape does not match [%d x %d]", name.c_str(), cols, rows);
  const uint8_t* p = tensor_bytes(g, t);
  if (!p) return fail(SG_ERR_INVALID, "tensor data out of bounds: %s", name.c_str());
  out = p;
  return SG_OK;
}

// loadTensorF32 (model.go:621-651): F32, or Q8_0 dequantized.  Returns
// SG_ERR_INVALID (with a message) when absent or unusable; optional norms
// ignore that error as the reference does.
int f32_vector(const Gguf& g, const std::string& name, int n, Loaded& L, const float*& out) {
  out = nullptr;
  auto it = g.tensors.find(name);
  if (it == g.tensors.end()) return fail(SG_ERR_INVALID, "tensor not found: %s", name.c_str());
  const Tensor& t = it->second;
  const uint8_t* p = tensor_bytes(g, t);
  if (!p) return fail(SG_ERR_INVALID, "tensor data out of bounds: %s", name.c_str());
  if (t.dims.empty() || t.dims[0] != (uint64_t)n) return fail(SG_ERR_INVALID, "%s: length is not %d", name.c_str(), n);
  std::vector<float> v(n);
  if (t.dtype == D_F32) {
    memcpy(v.data(), p, sizeof(float) * n);
  } else if (t.dtype == D_Q8_0) {
    for (int i = 0; i < n; i++) {
      const uint8_t* blk = p + (size_t)(i / 32) * 34;
      uint16_t h;
      memcpy(&h, blk, 2);
      v[i] = (float)(int8_t)blk[2 + i % 32] * f16_gguf(h);
    }
  } else {
    return fail(SG_ERR_INVALID, "unsupported dtype for conversion: %s", dtype_name(t.dtype));
  }
  L.owned.push_back(std::move(v));
  out = L.owned.back().data();
  return SG_OK;
}

int build_desc(const Gguf& g, Loaded& L) {
  sg_model_config& c = L.desc.config;
  if (int r = config_of(g, c)) return r;
  if (c.embed_dim <= 0 || c.num_heads <= 0 || c.num_layers <= 0 || c.num_kv_heads <= 0 || c.interm_dim <= 0 ||
      c.embed_dim % c.num_heads || c.embed_dim % 32 || c.interm_dim % 32)
    return fail(SG_ERR_INVALID, "unsupported model shape (d=%d, heads=%d, ff=%d)", c.embed_dim, c.num_heads,
                c.interm_dim);
  const int d = c.embed_dim, hd = d / c.num_heads, qd = c.num_heads * hd, kvd = c.num_kv_heads * hd,
            ff = c.interm_dim;
  // token embedding (loadWeights model.go:520-552)
  const char* emb_name = g.tensors.count("token_embd.weight") ? "token_embd.weight" : "model.embed_tokens.weight";
  auto it = g.tensors.find(emb_name);
  if (it == g.tensors.end()) return fail(SG_ERR_INVALID, "token embedding tensor not found");
  if (it->second.dtype != D_Q8_0)
    return fail(SG_ERR_INVALID, "expected Q8_0 embeddings, got %s", dtype_name(it->second.dtype));
  const uint8_t* emb = tensor_bytes(g, it->second);
  if (!emb) return fail(SG_ERR_INVALID, "tensor data out of bounds: %s", emb_name);
  if (c.vocab_size <= 0 || it->second.size < (uint64_t)c.vocab_size * (d / 32) * 34)
    return fail(SG_ERR_INVALID, "token embedding has fewer rows than the vocabulary (%d)", c.vocab_size);
  L.desc.token_embd = emb;
  const float* on = nullptr;
  if (f32_vector(g, "output_norm.weight", d, L, on) == SG_OK) L.desc.output_norm = on;  // optional
  L.layers.resize(c.num_layers);
  for (int l = 0; l < c.num_layers; l++) {
    const std::string p = "blk." + std::to_string(l) + ".";
    sg_layer_desc& ld = L.layers[l];
    if (int r = f32_vector(g, p + "attn_norm.weight", d, L, ld.attn_norm)) return r;
    if (int r = f32_vector(g, p + "ffn_norm.weight", d, L, ld.ffn_norm)) return r;
    f32_vector(g, p + "attn_q_norm.weight", hd, L, ld.attn_q_norm);  // optional (model_int8.go:66-69)
    f32_vector(g, p + "attn_k_norm.weight", hd, L, ld.attn_k_norm);
    f32_vector(g, p + "post_attention_norm.weight", d, L, ld.post_attention_norm);
    f32_vector(g, p + "post_ffw_norm.weight", d, L, ld.post_ffw_norm);
    if (int r = q8_matrix(g, p + "attn_q.weight", qd, d, ld.attn_q)) return r;
    if (int r = q8_matrix(g, p + "attn_k.weight", kvd, d, ld.attn_k)) return r;
    if (int r = q8_matrix(g, p + "attn_v.weight", kvd, d, ld.attn_v)) return r;
    if (int r = q8_matrix(g, p + "attn_output.weight", d, qd, ld.attn_output)) return r;
    if (int r = q8_matrix(g, p + "ffn_gate.weight", ff, d, ld.ffn_gate)) return r;
    if (int r = q8_matrix(g, p + "ffn_up.weight", ff, d, ld.ffn_up)) return r;
    if (int r = q8_matrix(g, p + "ffn_down.weight", d, ff, ld.ffn_down)) return r;
  }
  L.desc.layers = L.layers.data();
  return SG_OK;
}

}  // namespace

namespace sgi {

// LoadFromGGUF's reading of the tokenizer metadata (internal/tokenizer/
// tokenizer.go:497-598): tokens (strings, required), scores (float32 or
// float64, required), token_type (int32 / uint32 entries, others -> normal;
// optional), add_bos_token (bool, default true), add_eos_token (bool, default
// false), NFKC on, and the special ids when stored as uint32.
int gguf_tokenizer_spec(const void* data, size_t size, TokenizerSpec& out) {
  Gguf g;
  SG_TRY(parse(data, size, g));
  out = TokenizerSpec{};
  const Meta* tk = find(g, "tokenizer.ggml.tokens");
  if (!tk) return fail(SG_ERR_INVALID, "tokenizer.ggml.tokens not found");
  if (tk->type != M_ARR) return fail(SG_ERR_INVALID, "tokenizer.ggml.tokens is not an array");
  out.tokens.resize(tk->elems.size());
  for (size_t i = 0; i < tk->elems.size(); i++) {
    if (tk->elems[i].type != M_STR) return fail(SG_ERR_INVALID, "token %zu is not a string", i);
    out.tokens[i] = tk->elems[i].s;
  }
  const Meta* sc = find(g, "tokenizer.ggml.scores");
  if (!sc) return fail(SG_ERR_INVALID, "tokenizer.ggml.scores not found");
  if (sc->type != M_ARR) return fail(SG_ERR_INVALID, "tokenizer.ggml.scores is not an array");
  out.scores.resize(sc->elems.size());
  for (size_t i = 0; i < sc->elems.size(); i++) {
    const Meta& e = sc->elems[i];
    if (e.type == M_F32 || e.type == M_F64)
      out.scores[i] = (float)e.f;
    else
      return fail(SG_ERR_INVALID, "score %zu is not a number", i);
  }
  if (const Meta* ty = find(g, "tokenizer.ggml.token_type"); ty && ty->type == M_ARR) {
    out.types.resize(ty->elems.size());
    for (size_t i = 0; i < ty->elems.size(); i++) {
      const Meta& e = ty->elems[i];
      out.types[i] = (e.type == M_I32 || e.type == M_U32) ? (int32_t)(uint32_t)e.u : 1;
    }
  }
  auto get_bool = [&](const char* k, bool dflt) {
    const Meta* m = find(g, k);
    return m && m->type == M_BOOL ? m->u != 0 : dflt;
  };
  out.add_bos = get_bool("tokenizer.ggml.add_bos_token", true);
  out.add_eos = get_bool("tokenizer.ggml.add_eos_token", false);
  out.nfkc = true;
  auto get_id = [&](const char* k, int32_t& id) {
    const Meta* m = find(g, k);
    if (m && m->type == M_U32) id = (int32_t)(uint32_t)m->u;
  };
  get_id("tokenizer.ggml.bos_token_id", out.bos);
  get_id("tokenizer.ggml.eos_token_id", out.eos);
  get_id("tokenizer.ggml.unknown_token_id", out.unk);
  get_id("tokenizer.ggml.padding_token_id", out.pad);
  return SG_OK;
}

}  // namespace sgi

extern "C" {

int sg_gguf_read_config(const void* data, size_t size, sg_model_config* out) {
  if (!data || !out) return fail(SG_ERR_INVALID, "NULL argument");
  Gguf g;
  if (int r = parse(data, size, g)) return r;
  return config_of(g, *out);
}

int sg_model_load_gguf(sg_ctx* ctx, const void* data, size_t size, sg_model** out) {
  if (!ctx || !data || !out) return fail(SG_ERR_INVALID, "NULL argument");
  *out = nullptr;
  Gguf g;
  if (int r = parse(data, size, g)) return r;
  Loaded L;
  if (int r = build_desc(g, L)) return r;
  return sg_model_load(ctx, &L.desc, out);
}

int sg_model_load_gguf_file(sg_ctx* ctx, const char* path, sg_model** out) {
  if (!ctx || !path || !out) return fail(SG_ERR_INVALID, "NULL argument");
  *out = nullptr;
  const int fd = open(path, O_RDONLY);
  if (fd < 0) return fail(SG_ERR_INVALID, "open file: %s: %s", path, strerror(errno));
  struct stat st;
  if (fstat(fd, &st) != 0 || st.st_size <= 0) {
    close(fd);
    return fail(SG_ERR_INVALID, "file too small for header");
  }
  void* p = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
  close(fd);
  if (p == MAP_FAILED) return fail(SG_ERR_INVALID, "mmap file: %s", strerror(errno));
  const int r = sg_model_load_gguf(ctx, p, (size_t)st.st_size, out);
  munmap(p, (size_t)st.st_size);
  return r;
}

int sg_tokenizer_from_gguf_file(const char* path, sg_tokenizer** out) {
  if (!path || !out) return fail(SG_ERR_INVALID, "NULL argument");
  *out = nullptr;
  const int fd = open(path, O_RDONLY);
  if (fd < 0) return fail(SG_ERR_INVALID, "open file: %s: %s", path, strerror(errno));
  struct stat st;
  if (fstat(fd, &st) != 0 || st.st_size <= 0) {
    close(fd);
    return fail(SG_ERR_INVALID, "file too small for header");
  }
  void* p = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
  close(fd);
  if (p == MAP_FAILED) return fail(SG_ERR_INVALID, "mmap file: %s", strerror(errno));
  const int r = sg_tokenizer_from_gguf(p, (size_t)st.st_size, out);
  munmap(p, (size_t)st.st_size);
  return r;
}

}  // extern "C"
