// The C ABI over the GGUF index reader (gguf.h), Gemma 3 shapes from a
// file's metadata, and the load of a Gemma 3 file's tensors into a model.
// Host code only; the upload goes through frz_model_set_tensor.

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <memory>
#include <string>
#include <vector>

#include "../../include/frizzle_hip.h"
#include "gguf.h"


namespace frz {
// Sets the calling thread's message and returns `status` (backend.hip).
int fail(int status, const std::string& message);
}  // namespace frz

namespace {

using frz::fail;
using frz::gguf::Index;
using frz::gguf::Meta;
using frz::gguf::Tensor;

void to_info(const Tensor& t, frz_gguf_tensor* out) {
  std::memset(out, 0, sizeof(*out));
  std::memcpy(out->name, t.name.data(), t.name.size() < 64 ? t.name.size() : 64);
  out->type = t.type;
  out->dimensions = t.dims;
  for (int d = 0; d < 4; ++d) out->shape[d] = t.shape[d];
  out->elements = t.elements;
  out->offset = t.offset;
  out->bytes = t.bytes;
}

// An integer value of any width that fits in 32 unsigned bits.
bool as_u32(const Meta& m, uint32_t* out) {
  using namespace frz::gguf;
  switch (m.type) {
    case kU8: case kU16: case kU32: case kU64: case kBool:
      if (m.u > 0xFFFFFFFFull) return false;
      *out = (uint32_t)m.u;
      return true;
    case kI8: case kI16: case kI32: case kI64:
      if (m.i < 0 || m.i > 0xFFFFFFFFll) return false;
      *out = (uint32_t)m.i;
      return true;
    default:
      return false;
  }
}

struct RoleName {
  int role;
  const char* name;
};

// Gemma 3's tensor names by role (gemma3.cpp:21-35).
constexpr RoleName kLayerNames[] = {
    {FRZ_ROLE_Q, "attn_q.weight"},
    {FRZ_ROLE_K, "attn_k.weight"},
    {FRZ_ROLE_V, "attn_v.weight"},
    {FRZ_ROLE_O, "attn_output.weight"},
    {FRZ_ROLE_GATE, "ffn_gate.weight"},
    {FRZ_ROLE_UP, "ffn_up.weight"},
    {FRZ_ROLE_DOWN, "ffn_down.weight"},
    {FRZ_ROLE_ATTN_NORM, "attn_norm.weight"},
    {FRZ_ROLE_Q_NORM, "attn_q_norm.weight"},
    {FRZ_ROLE_K_NORM, "attn_k_norm.weight"},
    {FRZ_ROLE_POST_ATTN_NORM, "post_attention_norm.weight"},
    {FRZ_ROLE_FFN_NORM, "ffn_norm.weight"},
    {FRZ_ROLE_POST_FFN_NORM, "post_ffw_norm.weight"},
};

// The extents (ne0, ne1) a role's tensor has in a file for these shapes: a
// matrix of `rows` outputs over `cols` inputs is [cols, rows]; a norm gain
// of n values is [n].
void expected_shape(const frz_model_config& c, int role, uint64_t* ne0, uint64_t* ne1) {
  const uint64_t qw = (uint64_t)c.query_heads * c.head_dim, kvw = (uint64_t)c.kv_heads * c.head_dim;
  *ne1 = 1;
  switch (role) {
    case FRZ_ROLE_Q: *ne0 = c.hidden; *ne1 = qw; break;
    case FRZ_ROLE_K: case FRZ_ROLE_V: *ne0 = c.hidden; *ne1 = kvw; break;
    case FRZ_ROLE_O: *ne0 = qw; *ne1 = c.hidden; break;
    case FRZ_ROLE_GATE: case FRZ_ROLE_UP: *ne0 = c.hidden; *ne1 = c.ffn; break;
    case FRZ_ROLE_DOWN: *ne0 = c.ffn; *ne1 = c.hidden; break;
    case FRZ_ROLE_Q_NORM: case FRZ_ROLE_K_NORM: *ne0 = c.head_dim; break;
    case FRZ_ROLE_EMBEDDING: *ne0 = c.hidden; *ne1 = c.vocab; break;
    default: *ne0 = c.hidden; break;  // the layer norms and output_norm
  }
}

bool is_matrix(int role) { return role <= FRZ_ROLE_DOWN || role == FRZ_ROLE_EMBEDDING; }

}  // namespace

extern "C" {

int frz_gguf_read(const void* front, uint64_t resident, uint64_t file_size, frz_gguf** out,
                  uint64_t* bytes_needed) {
  if (!out || (!front && resident)) return -1;
  auto g = std::make_unique<frz_gguf>();
  const int e = frz::gguf::read_index(static_cast<const uint8_t*>(front), resident, file_size,
                                      g->index, bytes_needed);
  if (e == frz::gguf::kOk) *out = g.release();
  return e;
}

int frz_gguf_open(const char* path, frz_gguf** out) {
  if (!path || !out) return -1;
  frz::gguf::File file;
  if (!file.open(path)) return -1;
  auto g = std::make_unique<frz_gguf>();
  const int e = frz::gguf::read_file(file, g->index);
  if (e == frz::gguf::kOk) *out = g.release();
  return e;
}

void frz_gguf_free(frz_gguf* index) { delete index; }

const char* frz_gguf_error_text(int error) { return frz::gguf::error_text(error); }

int frz_gguf_format(uint32_t type, const char** name, uint32_t* block_elements,
                    uint32_t* block_bytes) {
  const frz::gguf::Layout* l = frz::gguf::layout_of(type);
  if (!l) return fail(FRZ_ERR_ARGUMENT, "frz_gguf_format: not a GGUF format number");
  if (name) *name = l->name;
  if (block_elements) *block_elements = l->elements;
  if (block_bytes) *block_bytes = l->bytes;
  return FRZ_OK;
}

uint64_t frz_gguf_tensor_count(const frz_gguf* g) { return g ? g->index.tensors.size() : 0; }

int frz_gguf_tensor_at(const frz_gguf* g, uint64_t i, frz_gguf_tensor* out) {
  if (!g || !out || i >= g->index.tensors.size())
    return fail(FRZ_ERR_ARGUMENT, "frz_gguf_tensor_at: no such tensor");
  to_info(g->index.tensors[i], out);
  return FRZ_OK;
}

int frz_gguf_find(const frz_gguf* g, const char* name, frz_gguf_tensor* out) {
  const Tensor* t = g && name ? g->index.tensor(name) : nullptr;
  if (!t || !out) return fail(FRZ_ERR_ARGUMENT, std::string("no tensor ") + (name ? name : ""));
  to_info(*t, out);
  return FRZ_OK;
}

uint64_t frz_gguf_metadata_count(const frz_gguf* g) { return g ? g->index.metadata.size() : 0; }

int frz_gguf_get_u32(const frz_gguf* g, const char* key, uint32_t* out) {
  const Meta* m = g && key ? g->index.meta(key) : nullptr;
  if (!m || !out || !as_u32(*m, out))
    return fail(FRZ_ERR_ARGUMENT, std::string("no 32-bit unsigned value for ") + (key ? key : ""));
  return FRZ_OK;
}

int frz_gguf_get_f32(const frz_gguf* g, const char* key, float* out) {
  const Meta* m = g && key ? g->index.meta(key) : nullptr;
  if (!m || !out || (m->type != frz::gguf::kF32 && m->type != frz::gguf::kF64))
    return fail(FRZ_ERR_ARGUMENT, std::string("no float value for ") + (key ? key : ""));
  *out = (float)m->f;
  return FRZ_OK;
}

int frz_gguf_get_string(const frz_gguf* g, const char* key, char* buf, uint64_t cap,
                        uint64_t* length) {
  const Meta* m = g && key ? g->index.meta(key) : nullptr;
  if (!m || m->type != frz::gguf::kString)
    return fail(FRZ_ERR_ARGUMENT, std::string("no string value for ") + (key ? key : ""));
  if (length) *length = m->s.size();
  if (buf && cap) {
    const uint64_t n = m->s.size() < cap - 1 ? m->s.size() : cap - 1;
    std::memcpy(buf, m->s.data(), n);
    buf[n] = '\0';
  }
  return FRZ_OK;
}

int frz_gguf_get_array(const frz_gguf* g, const char* key, uint32_t* element_type,
                       uint64_t* count) {
  const Meta* m = g && key ? g->index.meta(key) : nullptr;
  if (!m || m->type != frz::gguf::kArray)
    return fail(FRZ_ERR_ARGUMENT, std::string("no array for ") + (key ? key : ""));
  if (element_type) *element_type = m->array_type;
  if (count) *count = m->array_count;
  return FRZ_OK;
}

int frz_gemma3_config_from_gguf(const frz_gguf* g, int context, frz_model_config* out) {
  if (!g || !out) return fail(FRZ_ERR_ARGUMENT, "frz_gemma3_config_from_gguf: null argument");
  char arch[32];
  uint64_t n = 0;
  if (frz_gguf_get_string(g, "general.architecture", arch, sizeof arch, &n) != FRZ_OK ||
      std::string(arch, n < sizeof arch ? n : sizeof arch - 1) != "gemma3") {
    return fail(FRZ_ERR_ARGUMENT, "general.architecture is not gemma3");
  }
  frz_model_config c{};
  uint32_t v = 0;
  struct Required {
    const char* key;
    int* field;
  } required[] = {
      {"gemma3.block_count", &c.layers},
      {"gemma3.embedding_length", &c.hidden},
      {"gemma3.feed_forward_length", &c.ffn},
      {"gemma3.attention.head_count", &c.query_heads},
      {"gemma3.attention.head_count_kv", &c.kv_heads},
      {"gemma3.attention.sliding_window", &c.window},
  };
  for (const Required& r : required) {
    if (int rc = frz_gguf_get_u32(g, r.key, &v)) return rc;
    if (v == 0 || v > 0x7FFFFFFF) return fail(FRZ_ERR_ARGUMENT, std::string(r.key) + " is 0 or too large");
    *r.field = (int)v;
  }
  if (c.query_heads % c.kv_heads != 0)
    return fail(FRZ_ERR_ARGUMENT, "gemma3.attention.head_count is not a multiple of head_count_kv");
  c.head_dim = c.hidden / c.query_heads;
  if (frz_gguf_get_u32(g, "gemma3.attention.key_length", &v) == FRZ_OK) c.head_dim = (int)v;
  c.pattern = 6;
  if (g->index.meta("gemma3.attention.sliding_window_pattern")) {
    if (frz_gguf_get_u32(g, "gemma3.attention.sliding_window_pattern", &v) != FRZ_OK || v == 0)
      return fail(FRZ_ERR_ARGUMENT, "gemma3.attention.sliding_window_pattern: one nonzero number");
    c.pattern = (int)v;
  }
  if (int rc = frz_gguf_get_f32(g, "gemma3.attention.layer_norm_rms_epsilon", &c.epsilon))
    return rc;
  if (int rc = frz_gguf_get_f32(g, "gemma3.rope.freq_base", &c.rope_global)) return rc;
  c.rope_local = 10000.0f;
  if (g->index.meta("gemma3.rope.freq_base_swa")) {
    if (int rc = frz_gguf_get_f32(g, "gemma3.rope.freq_base_swa", &c.rope_local)) return rc;
  }
  const Tensor* embd = g->index.tensor("token_embd.weight");
  if (!embd || embd->dims != 2 || embd->shape[0] != (uint64_t)c.hidden || embd->shape[1] == 0 ||
      embd->shape[1] > 0x7FFFFFFF) {
    return fail(FRZ_ERR_ARGUMENT, "token_embd.weight: missing or not [embedding_length, vocab]");
  }
  c.vocab = (int)embd->shape[1];
  c.context = context > 0 ? context : 8192;
  c.local_slots = c.window + 512 + 4096;  // as frz_gemma3_1b_config: window + block + reserve
  *out = c;
  return FRZ_OK;
}

int frz_model_load_gguf(frz_model* model, const char* path) {
  if (!model || !path) return fail(FRZ_ERR_ARGUMENT, "frz_model_load_gguf: null argument");
  frz_model_config c;
  if (int rc = frz_model_get_config(model, &c)) return rc;
  frz::gguf::File file;
  if (!file.open(path)) return fail(FRZ_ERR_ARGUMENT, std::string("cannot open ") + path);
  frz_gguf g;
  if (int e = frz::gguf::read_file(file, g.index)) {
    return fail(FRZ_ERR_ARGUMENT, std::string(path) + ": " +
                                      (e < 0 ? "read failed" : frz::gguf::error_text(e)));
  }
  frz_model_config fc;
  if (int rc = frz_gemma3_config_from_gguf(&g, c.context, &fc)) return rc;
  if (fc.hidden != c.hidden || fc.ffn != c.ffn || fc.head_dim != c.head_dim ||
      fc.query_heads != c.query_heads || fc.kv_heads != c.kv_heads || fc.layers != c.layers ||
      fc.vocab != c.vocab || fc.window != c.window || fc.pattern != c.pattern) {
    return fail(FRZ_ERR_ARGUMENT, "the file's shapes are not the model's");
  }
  if (g.index.tensor("output.weight")) {
    return fail(FRZ_ERR_ARGUMENT, "output.weight: an untied output head is not supported");
  }
  std::vector<uint8_t> buf;
  auto load = [&](int layer, int role, const std::string& name) -> int {
    const Tensor* t = g.index.tensor(name);
    if (!t) return fail(FRZ_ERR_ARGUMENT, "missing tensor " + name);
    // The formats the pinned file mixes (device_layout.h:64-66): Q4_0
    // matrices, Q4_1 in the first downs, a Q8_0 embedding; F32 gains.
    const uint32_t type = t->type;
    const bool format_ok =
        !is_matrix(role) ? type == FRZ_FORMAT_F32
        : role == FRZ_ROLE_DOWN
            ? type == FRZ_FORMAT_Q4_0 || type == FRZ_FORMAT_Q4_1 || type == FRZ_FORMAT_Q8_0
        : role == FRZ_ROLE_EMBEDDING ? type == FRZ_FORMAT_Q4_0 || type == FRZ_FORMAT_Q8_0
                                     : type == FRZ_FORMAT_Q4_0;
    if (!format_ok) {
      const frz::gguf::Layout* l = frz::gguf::layout_of(type);
      return fail(FRZ_ERR_ARGUMENT,
                  name + ": format " + (l ? l->name : "?") +
                      " is not run here (matrices Q4_0; downs also Q4_1 or Q8_0; the embedding"
                      " also Q8_0; norms F32)");
    }
    uint64_t ne0, ne1;
    expected_shape(c, role, &ne0, &ne1);
    const bool shape_ok = t->shape[0] == ne0 && t->shape[1] == ne1 && t->shape[2] == 1 &&
                          t->shape[3] == 1 && (ne1 == 1 ? t->dims >= 1 : t->dims >= 2);
    const uint64_t want_bytes =
        is_matrix(role) ? frz_tensor_bytes(&c, role) / 18 * frz::gguf::layout_of(type)->bytes
                        : frz_tensor_bytes(&c, role);
    if (!shape_ok || t->bytes != want_bytes) {
      return fail(FRZ_ERR_ARGUMENT, name + ": shape is not the model's");
    }
    buf.resize(t->bytes);
    if (!file.read(t->offset, buf.data(), t->bytes)) {
      return fail(FRZ_ERR_ARGUMENT, name + ": read failed");
    }
    return frz_model_set_tensor_format(model, layer, role, (int)type, buf.data(), t->bytes);
  };
  if (int rc = load(-1, FRZ_ROLE_EMBEDDING, "token_embd.weight")) return rc;
  if (int rc = load(-1, FRZ_ROLE_OUTPUT_NORM, "output_norm.weight")) return rc;
  for (int l = 0; l < c.layers; ++l) {
    for (const RoleName& r : kLayerNames) {
      if (int rc = load(l, r.role, "blk." + std::to_string(l) + "." + r.name)) return rc;
    }
  }
  return FRZ_OK;
}

}  // extern "C"
