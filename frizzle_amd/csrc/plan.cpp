// The residency plan (src/core/residency/plan.h:14-326, plan.cpp): where
// every weight, each layer's KV cache and every working buffer lies on the
// device, and the context offered, as a pure function of a Gemma 3 file's
// tensor index, the device's limits and the load policy. No device and no
// I/O. Host code only.
//
// The rules are the reference's, stated there and kept here:
//   - three pools (weights, cache, working buffers), never sharing a buffer;
//     every range aligned to the storage offset alignment, its length
//     rounded up to 4, at most min(binding, buffer) long;
//   - a weight cut into pieces of whole rows (every dimension but the last),
//     in file order, filling a buffer before opening the next;
//   - a layer's Q, K, V and its gate, up become a group when they share a
//     format and an input width and their span (first member to last, with
//     what the file holds between) fits one range in one buffer;
//   - each working buffer alone in a buffer of its own;
//   - a sliding layer's ring of window + 512 + the rollback reserve slots, a
//     full-attention layer's slots the context offered; the context offered
//     the largest from min(512, trained) to the trained context whose cache
//     fits beside the weights and working buffers within the budget, found
//     by bisection.
// Sizes are summed and multiplied with overflow checks.

#include <algorithm>
#include <array>
#include <cstdint>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/frizzle_hip.h"
#include "gguf.h"

namespace frz {
int fail(int status, const std::string& message);
}  // namespace frz

namespace {

using frz::gguf::Index;
using frz::gguf::Tensor;

constexpr uint64_t kGranule = 4;         // a binding's size is a multiple of 4
constexpr uint32_t kPrefillBlock = 512;  // plan.h: kPrefillBlock
constexpr uint32_t kChunkKeys = 64;      // plan.h: kChunkKeys
constexpr uint32_t kCandidates = 64;     // plan.h: kCandidates
constexpr uint32_t kSelectionTile = 1024;
constexpr uint64_t kEditWords = 5;       // edit.h: kEditWords
constexpr uint64_t kMaxEdits = 4096;     // edit.h: kMaxEdits
constexpr int kRoles = 13;               // a layer's roles (frz_role 0 .. 12)

bool add(uint64_t a, uint64_t b, uint64_t& out) { return !__builtin_add_overflow(a, b, &out); }
bool mul(uint64_t a, uint64_t b, uint64_t& out) { return !__builtin_mul_overflow(a, b, &out); }

// v rounded up to a multiple of `to`, a power of two; false on overflow.
bool round_up(uint64_t v, uint64_t to, uint64_t& out) {
  uint64_t s = 0;
  if (!add(v, to - 1, s)) return false;
  out = s & ~(to - 1);
  return true;
}

struct Buffer {
  int pool;
  uint64_t size;
};

// Ranges placed into one pool's buffers, each at an aligned offset, padded
// to the granule (plan.cpp's Packer).
class Packer {
 public:
  Packer(std::vector<Buffer>& buffers, int pool, const frz_plan_limits& limits)
      : buffers_(&buffers), pool_(pool), limits_(limits) {}

  // Closes the open buffer when `length` more bytes at its next aligned
  // offset would not fit it.
  bool reserve(uint64_t length) {
    if (!open_) return true;
    uint64_t offset = 0;
    if (!round_up(buffers_->back().size, limits_.storage_offset_alignment, offset)) return false;
    if (offset > limits_.max_buffer_size || length > limits_.max_buffer_size - offset)
      open_ = false;
    return true;
  }

  // Places `length` bytes; `alone` gives the range a buffer of its own.
  bool place(uint64_t length, bool alone, frz_range& out) {
    uint64_t padded = 0;
    if (!round_up(length, kGranule, padded)) return false;
    uint64_t offset = 0;
    if (open_ && !alone) {
      if (!round_up(buffers_->back().size, limits_.storage_offset_alignment, offset))
        return false;
      if (offset > limits_.max_buffer_size || padded > limits_.max_buffer_size - offset)
        open_ = false;
    }
    if (!open_ || alone) {
      buffers_->push_back({pool_, 0});
      offset = 0;
    }
    buffers_->back().size = offset + padded;
    out = {(uint32_t)(buffers_->size() - 1), offset, padded};
    open_ = !alone;
    return true;
  }

 private:
  std::vector<Buffer>* buffers_;
  int pool_;
  frz_plan_limits limits_;
  bool open_ = false;
};

uint64_t range_limit(const frz_plan_limits& l) {
  return std::min(l.max_storage_binding_size, l.max_buffer_size) & ~(kGranule - 1);
}

// A model as the planner sees it (the reference's ModelDescription, for
// Gemma 3): per layer its role tensors (index positions, -1 absent), heads,
// widths and the keys it attends to.
struct LayerDesc {
  std::array<int64_t, kRoles> roles;
  uint32_t query_heads, kv_heads, head_dim, ffn, window;
};
struct ModelDesc {
  std::vector<LayerDesc> layers;
  uint32_t hidden = 0, vocab = 0, trained_context = 0;
  int64_t embedding = -1, output_norm = -1;
  frz_model_config config{};
};

struct ScratchNeed {
  const char* purpose;
  uint64_t rows, width;
};

}  // namespace

struct frz_plan {
  std::vector<Buffer> buffers;
  std::vector<std::vector<frz_piece>> tensors;  // per tensor of the index, its pieces
  struct Group {
    uint64_t members[3];
    uint32_t count;
    frz_range span;
  };
  std::vector<Group> groups;
  struct CacheLayer {
    frz_range keys, values;
    uint32_t slots;
  };
  std::vector<CacheLayer> cache;
  std::vector<std::pair<std::string, frz_range>> scratch;
  uint32_t partial_rows = 0;
  uint32_t context_offered = 0;
  uint64_t weight_bytes = 0, cache_bytes = 0, scratch_bytes = 0, total_bytes = 0;
  ModelDesc model;
  std::vector<uint32_t> formats;  // each tensor's GGUF format, index order
};

namespace {

const char* const kRoleNames[kRoles] = {
    "attn_q.weight",      "attn_k.weight",       "attn_v.weight",
    "attn_output.weight", "ffn_gate.weight",     "ffn_up.weight",
    "ffn_down.weight",    "attn_norm.weight",    "attn_q_norm.weight",
    "attn_k_norm.weight", "post_attention_norm.weight", "ffn_norm.weight",
    "post_ffw_norm.weight"};

int64_t index_of(const Index& ix, const std::string& name) {
  auto it = ix.tensor_at.find(name);
  return it == ix.tensor_at.end() ? -1 : (int64_t)it->second;
}

// The model a Gemma 3 file describes (gemma3.cpp:44-95, describe.cpp:
// 205-380): shapes from its metadata, the trained context from
// gemma3.context_length, every layer attending to the trained context but
// the sliding ones (all but each pattern's last), which attend to the window.
int describe(const frz_gguf* g, ModelDesc& out, std::string& subject) {
  if (int rc = frz_gemma3_config_from_gguf(g, 0, &out.config)) {
    subject = frz_last_error();
    return rc;
  }
  uint32_t trained = 0;
  if (frz_gguf_get_u32(g, "gemma3.context_length", &trained) != FRZ_OK || trained == 0) {
    subject = "gemma3.context_length";
    return FRZ_ERR_ARGUMENT;
  }
  const frz_model_config& c = out.config;
  out.hidden = (uint32_t)c.hidden;
  out.vocab = (uint32_t)c.vocab;
  out.trained_context = trained;
  out.embedding = index_of(g->index, "token_embd.weight");
  out.output_norm = index_of(g->index, "output_norm.weight");
  if (out.output_norm < 0) {
    subject = "output_norm.weight";
    return FRZ_ERR_ARGUMENT;
  }
  out.layers.assign(c.layers, LayerDesc{});
  for (int l = 0; l < c.layers; ++l) {
    LayerDesc& L = out.layers[l];
    for (int r = 0; r < kRoles; ++r) {
      L.roles[r] = index_of(g->index, "blk." + std::to_string(l) + "." + kRoleNames[r]);
    }
    L.query_heads = (uint32_t)c.query_heads;
    L.kv_heads = (uint32_t)c.kv_heads;
    L.head_dim = (uint32_t)c.head_dim;
    L.ffn = (uint32_t)c.ffn;
    L.window = l % c.pattern == c.pattern - 1 ? trained : (uint32_t)c.window;
  }
  out.config.context = (int)trained;
  return FRZ_OK;
}

// The most range sums a layer's products need split along K
// (graph.cpp:117-130, matmul.cpp:235-256 with the split gate {2, 1, 64} and
// 64-output tiles of up to 32 tokens; gate and up never split).
uint64_t range_sum_floats(uint64_t rows, uint64_t columns) {
  const uint64_t groups = columns / 32;
  const uint64_t out_tiles = (rows + 63) / 64;
  const uint64_t by_ratio = groups * 2 / (1 * out_tiles);
  const uint64_t by_cap = 64 / out_tiles;
  const uint64_t token_tiles = std::min(by_ratio, by_cap);
  const uint64_t split = token_tiles == 0 ? 1 : std::min<uint64_t>(token_tiles * 32, kPrefillBlock);
  return split < 2 ? 0 : split * rows * 32;
}

uint32_t partial_rows_for(uint32_t trained) {
  const uint32_t chunks = trained / kChunkKeys + (trained % kChunkKeys != 0 ? 1 : 0);
  return chunks > kPrefillBlock ? chunks : kPrefillBlock;
}

// The working buffers a decoder step binds (graph.cpp:132-198, in its order).
std::vector<ScratchNeed> working_set(const ModelDesc& m, uint32_t& partial_rows) {
  uint64_t query = 0, kv = 0, ffn = 0, heads = 0, sums = 1;
  for (const LayerDesc& l : m.layers) {
    query = std::max<uint64_t>(query, (uint64_t)l.query_heads * l.head_dim);
    heads = std::max<uint64_t>(heads, l.query_heads);
    kv = std::max<uint64_t>(kv, (uint64_t)l.kv_heads * l.head_dim);
    ffn = std::max<uint64_t>(ffn, l.ffn);
    const uint64_t lq = (uint64_t)l.query_heads * l.head_dim, lkv = (uint64_t)l.kv_heads * l.head_dim;
    sums = std::max({sums, range_sum_floats(lq + 2 * lkv, m.hidden), range_sum_floats(m.hidden, lq),
                     range_sum_floats(m.hidden, l.ffn)});
  }
  const uint64_t first = (m.vocab + kSelectionTile - 1) / kSelectionTile;
  const uint64_t second = (kCandidates * first + kSelectionTile - 1) / kSelectionTile;
  partial_rows = partial_rows_for(m.trained_context);
  frz_model_config at_trained = m.config;
  at_trained.context = (int)m.trained_context;
  const uint64_t captures = frz_capture_words(&at_trained, nullptr);
  const uint64_t edit_table = 2ull * m.layers.size() + kEditWords * kMaxEdits;
  return {{"hidden", kPrefillBlock, m.hidden},
          {"normed", kPrefillBlock, m.hidden},
          {"query", kPrefillBlock, query},
          {"key", kPrefillBlock, kv},
          {"value", kPrefillBlock, kv},
          {"attention", kPrefillBlock, query},
          {"partials", partial_rows, query},
          {"partial_stats", partial_rows, 2 * heads},
          {"output", kPrefillBlock, m.hidden},
          {"activation", kPrefillBlock, ffn},
          {"logits", 1, m.vocab},
          {"partials_a", 1, 2ull * kCandidates * first},
          {"partials_b", 1, 2ull * kCandidates * second},
          {"candidates", 1, 2ull * kCandidates},
          {"sampled", 1, 4},
          {"range_sums", 1, sums},
          {"edit_table", 1, edit_table},
          {"captures", 1, captures}};
}

// A row is every dimension but the last (format.h): ne0 elements.
uint64_t row_elements(const Tensor& t) { return t.shape[0]; }

int place_weights(const Index& ix, const ModelDesc& m, const frz_plan_limits& limits,
                  frz_plan& out, std::string& subject) {
  Packer packer{out.buffers, FRZ_POOL_WEIGHTS, limits};
  const uint64_t limit = range_limit(limits);
  const auto& tensors = ix.tensors;
  // Candidate groups: Q, K, V and gate, up (members in output order).
  std::vector<frz_plan::Group> groups;
  for (const LayerDesc& l : m.layers) {
    if (l.roles[FRZ_ROLE_Q] >= 0 && l.roles[FRZ_ROLE_K] >= 0 && l.roles[FRZ_ROLE_V] >= 0) {
      groups.push_back({{(uint64_t)l.roles[FRZ_ROLE_Q], (uint64_t)l.roles[FRZ_ROLE_K],
                         (uint64_t)l.roles[FRZ_ROLE_V]},
                        3,
                        {}});
    }
    if (l.roles[FRZ_ROLE_GATE] >= 0 && l.roles[FRZ_ROLE_UP] >= 0) {
      groups.push_back(
          {{(uint64_t)l.roles[FRZ_ROLE_GATE], (uint64_t)l.roles[FRZ_ROLE_UP], 0}, 2, {}});
    }
  }
  // Keep those whose members agree in format and input width and whose
  // span, as the packer would lay it out, fits one range.
  std::vector<uint64_t> reserve_before(tensors.size(), 0);
  std::vector<frz_plan::Group> kept;
  for (const frz_plan::Group& g : groups) {
    const Tensor& head = tensors[g.members[0]];
    uint64_t first = tensors.size(), last = 0;
    bool ok = true;
    for (uint32_t i = 0; i < g.count; ++i) {
      const Tensor& t = tensors[g.members[i]];
      if (t.type != head.type || t.shape[0] != head.shape[0]) ok = false;
      first = std::min(first, g.members[i]);
      last = std::max(last, g.members[i]);
    }
    if (!ok) continue;
    uint64_t bytes = 0;
    for (uint64_t k = first; k <= last && ok; ++k) {
      uint64_t padded = 0, aligned = 0;
      ok = tensors[k].bytes <= limit && round_up(tensors[k].bytes, kGranule, padded) &&
           round_up(padded, limits.storage_offset_alignment, aligned) && add(bytes, aligned, bytes);
    }
    if (!ok || bytes > limit) continue;
    reserve_before[first] = std::max(reserve_before[first], bytes);
    kept.push_back(g);
  }
  out.tensors.assign(tensors.size(), {});
  for (size_t i = 0; i < tensors.size(); ++i) {
    if (reserve_before[i] != 0 && !packer.reserve(reserve_before[i])) {
      subject.clear();
      return FRZ_PLAN_OVERFLOW;
    }
    const Tensor& t = tensors[i];
    const uint64_t row = row_elements(t);
    const uint64_t rows = row == 0 ? 0 : t.elements / row;
    if (rows == 0) continue;
    const uint64_t row_bytes = t.bytes / rows;
    if (row_bytes > limit) {
      subject = t.name;
      return FRZ_PLAN_ROW_EXCEEDS_BINDING;
    }
    const uint64_t per_piece = limit / row_bytes;
    for (uint64_t first = 0; first < rows; first += per_piece) {
      const uint64_t count = std::min(per_piece, rows - first);
      frz_range r{};
      if (!packer.place(count * row_bytes, false, r)) {
        subject = t.name;
        return FRZ_PLAN_OVERFLOW;
      }
      out.tensors[i].push_back(frz_piece{r, first, count});
    }
  }
  // Each kept group's span, now its members are placed.
  for (frz_plan::Group& g : kept) {
    const frz_piece& head = out.tensors[g.members[0]].front();
    uint64_t begin = head.range.offset, end = head.range.offset + head.range.length;
    bool one_buffer = true;
    for (uint32_t i = 0; i < g.count; ++i) {
      const frz_piece& p = out.tensors[g.members[i]].front();
      one_buffer = one_buffer && p.range.buffer == head.range.buffer;
      begin = std::min(begin, p.range.offset);
      end = std::max(end, p.range.offset + p.range.length);
    }
    if (one_buffer && end - begin <= limit) {
      g.span = {head.range.buffer, begin, end - begin};
      out.groups.push_back(g);
    }
  }
  return FRZ_PLAN_OK;
}

int place_scratch(const ModelDesc& m, const frz_plan_limits& limits, frz_plan& out,
                  std::string& subject) {
  const std::vector<ScratchNeed> needs = working_set(m, out.partial_rows);
  Packer packer{out.buffers, FRZ_POOL_SCRATCH, limits};
  for (const ScratchNeed& n : needs) {
    uint64_t values = 0, bytes = 0;
    if (!mul(n.rows, n.width, values) || !mul(values, 4, bytes)) {
      subject = n.purpose;
      return FRZ_PLAN_OVERFLOW;
    }
    if (bytes > range_limit(limits)) {
      subject = n.purpose;
      return FRZ_PLAN_SCRATCH_EXCEEDS_BINDING;
    }
    frz_range r{};
    if (!packer.place(bytes, true, r)) {
      subject = n.purpose;
      return FRZ_PLAN_OVERFLOW;
    }
    out.scratch.emplace_back(n.purpose, r);
  }
  return FRZ_PLAN_OK;
}

uint64_t pool_bytes(const std::vector<Buffer>& buffers, int pool) {
  uint64_t total = 0;
  for (const Buffer& b : buffers) {
    if (b.pool == pool) total += b.size;
  }
  return total;
}

struct CacheCost {
  uint64_t slot_bytes, ring;
};

// The cache's bytes at `context` before alignment padding; false when a size
// overflows or a layer's keys outgrow a binding.
bool cache_bytes_at(const std::vector<CacheCost>& layers, uint64_t context, uint64_t binding,
                    uint64_t& out) {
  out = 0;
  for (const CacheCost& l : layers) {
    uint64_t length = 0;
    if (!mul(std::min(context, l.ring), l.slot_bytes, length) || length > binding) return false;
    if (!add(out, 2 * length, out)) return false;
  }
  return true;
}

int place_cache(const ModelDesc& m, const frz_plan_limits& limits, const frz_load_policy& policy,
                frz_plan& out) {
  const uint64_t limit = range_limit(limits);
  // F16: blocks of one value in 2 bytes.
  std::vector<CacheCost> layers;
  for (const LayerDesc& l : m.layers) {
    CacheCost c{0, (uint64_t)l.window + kPrefillBlock + policy.rollback_reserve};
    if (!mul((uint64_t)l.kv_heads * l.head_dim, 2, c.slot_bytes)) return FRZ_PLAN_OVERFLOW;
    layers.push_back(c);
  }
  const uint64_t shortest = std::min<uint64_t>(kPrefillBlock, m.trained_context);
  const uint64_t slack = 2 * m.layers.size() * ((uint64_t)limits.storage_offset_alignment + kGranule);
  const uint64_t fixed = out.weight_bytes + out.scratch_bytes + slack;
  auto fits = [&](uint64_t context) {
    uint64_t bytes = 0, total = 0;
    return cache_bytes_at(layers, context, limit, bytes) && add(fixed, bytes, total) &&
           total <= policy.memory_budget;
  };
  if (!fits(shortest)) {
    uint64_t bytes = 0;
    if (!cache_bytes_at(layers, shortest, limit, bytes) || !add(fixed, bytes, out.total_bytes))
      return FRZ_PLAN_OVERFLOW;
    return FRZ_PLAN_EXCEEDS_BUDGET;
  }
  uint64_t low = shortest, high = m.trained_context;
  while (low < high) {
    const uint64_t mid = low + (high - low + 1) / 2;
    if (fits(mid)) {
      low = mid;
    } else {
      high = mid - 1;
    }
  }
  out.context_offered = (uint32_t)low;
  Packer packer{out.buffers, FRZ_POOL_CACHE, limits};
  for (const CacheCost& l : layers) {
    frz_plan::CacheLayer c{};
    c.slots = (uint32_t)std::min<uint64_t>(l.ring, out.context_offered);
    const uint64_t length = (uint64_t)c.slots * l.slot_bytes;
    if (!packer.place(length, false, c.keys) || !packer.place(length, false, c.values))
      return FRZ_PLAN_OVERFLOW;
    out.cache.push_back(c);
  }
  return FRZ_PLAN_OK;
}

void copy_subject(const std::string& s, char* buf, size_t cap) {
  if (!buf || cap == 0) return;
  const size_t n = std::min(s.size(), cap - 1);
  std::memcpy(buf, s.data(), n);
  buf[n] = '\0';
}

void summarize(const frz_plan& p, frz_plan_summary* s) {
  if (!s) return;
  std::memset(s, 0, sizeof *s);
  s->buffers = (uint32_t)p.buffers.size();
  s->tensors = (uint32_t)p.tensors.size();
  for (const auto& t : p.tensors) s->pieces += (uint32_t)t.size();
  s->groups = (uint32_t)p.groups.size();
  s->layers = (uint32_t)p.cache.size();
  s->scratch = (uint32_t)p.scratch.size();
  s->partial_rows = p.partial_rows;
  s->context_offered = p.context_offered;
  s->trained_context = p.model.trained_context;
  s->weight_bytes = p.weight_bytes;
  s->cache_bytes = p.cache_bytes;
  s->scratch_bytes = p.scratch_bytes;
  s->total_bytes = p.total_bytes;
}

}  // namespace

extern "C" {

void frz_load_policy_default(frz_load_policy* out) {
  if (!out) return;
  out->memory_budget = 2ull << 30;  // policy.h: kDefaultMemoryBudget
  out->rollback_reserve = 4096;     // policy.h: kDefaultRollbackReserve
}

int frz_plan_gemma3(const frz_gguf* index, const frz_plan_limits* limits,
                    const frz_load_policy* policy, frz_plan** out, frz_plan_summary* summary,
                    char* subject, size_t subject_cap) {
  if (summary) std::memset(summary, 0, sizeof *summary);
  copy_subject("", subject, subject_cap);
  if (!index || !limits || !policy || !out || limits->max_buffer_size == 0 ||
      limits->max_storage_binding_size == 0 || limits->storage_offset_alignment == 0 ||
      (limits->storage_offset_alignment & (limits->storage_offset_alignment - 1)) != 0) {
    copy_subject("arguments: null, or a zero or non-power-of-two limit", subject, subject_cap);
    return FRZ_PLAN_NOT_DESCRIBED;
  }
  *out = nullptr;
  auto* p = new frz_plan();
  std::string subj;
  int rc = describe(index, p->model, subj) == FRZ_OK ? FRZ_PLAN_OK : FRZ_PLAN_NOT_DESCRIBED;
  if (rc == FRZ_PLAN_OK) rc = place_weights(index->index, p->model, *limits, *p, subj);
  for (const Tensor& t : index->index.tensors) p->formats.push_back(t.type);
  if (rc == FRZ_PLAN_OK) {
    p->weight_bytes = pool_bytes(p->buffers, FRZ_POOL_WEIGHTS);
    rc = place_scratch(p->model, *limits, *p, subj);
  }
  if (rc == FRZ_PLAN_OK) {
    p->scratch_bytes = pool_bytes(p->buffers, FRZ_POOL_SCRATCH);
    rc = place_cache(p->model, *limits, *policy, *p);
  }
  if (rc == FRZ_PLAN_OK) {
    p->cache_bytes = pool_bytes(p->buffers, FRZ_POOL_CACHE);
    p->total_bytes = p->weight_bytes + p->scratch_bytes + p->cache_bytes;
    p->model.config.context = (int)p->context_offered;
    // A sliding layer's ring as placed: window + 512 + reserve, or the whole
    // context when that is shorter.
    p->model.config.local_slots = (int)std::min<uint64_t>(
        (uint64_t)p->model.config.window + 512 + policy->rollback_reserve, p->context_offered);
  }
  summarize(*p, summary);
  copy_subject(subj, subject, subject_cap);
  if (rc != FRZ_PLAN_OK) {
    delete p;
    return rc;
  }
  *out = p;
  return FRZ_PLAN_OK;
}

void frz_plan_free(frz_plan* plan) { delete plan; }

int frz_plan_summarize(const frz_plan* p, frz_plan_summary* out) {
  if (!p || !out) return frz::fail(FRZ_ERR_ARGUMENT, "frz_plan_summarize: null argument");
  summarize(*p, out);
  return FRZ_OK;
}

int frz_plan_format(const frz_plan* p, uint64_t tensor, uint32_t* format) {
  if (!p || !format || tensor >= p->formats.size())
    return frz::fail(FRZ_ERR_ARGUMENT, "frz_plan_format: index");
  *format = p->formats[tensor];
  return FRZ_OK;
}

const char* frz_plan_error_text(int error) {
  switch (error) {
    case FRZ_PLAN_OK: return "ok";
    case FRZ_PLAN_EXCEEDS_BUDGET: return "the weights and working buffers leave too little of the "
                                         "budget for a 512-token cache";
    case FRZ_PLAN_ROW_EXCEEDS_BINDING: return "a weight's row is wider than a binding";
    case FRZ_PLAN_SCRATCH_EXCEEDS_BINDING: return "a working buffer is wider than a binding";
    case FRZ_PLAN_OVERFLOW: return "a size overflows 64 bits";
    case FRZ_PLAN_NOT_DESCRIBED: return "the file does not describe a Gemma 3 model";
    default: return "unknown plan error";
  }
}

int frz_plan_config(const frz_plan* p, frz_model_config* out) {
  if (!p || !out) return frz::fail(FRZ_ERR_ARGUMENT, "frz_plan_config: null argument");
  *out = p->model.config;
  return FRZ_OK;
}

int frz_plan_buffer(const frz_plan* p, uint32_t i, int* pool, uint64_t* size) {
  if (!p || i >= p->buffers.size()) return frz::fail(FRZ_ERR_ARGUMENT, "frz_plan_buffer: index");
  if (pool) *pool = p->buffers[i].pool;
  if (size) *size = p->buffers[i].size;
  return FRZ_OK;
}

int frz_plan_tensor(const frz_plan* p, uint64_t tensor, uint32_t piece, frz_piece* out,
                    uint32_t* pieces) {
  if (!p || tensor >= p->tensors.size()) return frz::fail(FRZ_ERR_ARGUMENT, "frz_plan_tensor: index");
  const auto& t = p->tensors[tensor];
  if (pieces) *pieces = (uint32_t)t.size();
  if (out) {
    if (piece >= t.size()) return frz::fail(FRZ_ERR_ARGUMENT, "frz_plan_tensor: piece");
    *out = t[piece];
  }
  return FRZ_OK;
}

int frz_plan_group(const frz_plan* p, uint32_t i, uint64_t members[3], uint32_t* count,
                   frz_range* span) {
  if (!p || i >= p->groups.size()) return frz::fail(FRZ_ERR_ARGUMENT, "frz_plan_group: index");
  const frz_plan::Group& g = p->groups[i];
  if (members) std::memcpy(members, g.members, sizeof g.members);
  if (count) *count = g.count;
  if (span) *span = g.span;
  return FRZ_OK;
}

int frz_plan_cache(const frz_plan* p, uint32_t layer, frz_range* keys, frz_range* values,
                   uint32_t* slots) {
  if (!p || layer >= p->cache.size()) return frz::fail(FRZ_ERR_ARGUMENT, "frz_plan_cache: layer");
  const frz_plan::CacheLayer& c = p->cache[layer];
  if (keys) *keys = c.keys;
  if (values) *values = c.values;
  if (slots) *slots = c.slots;
  return FRZ_OK;
}

int frz_plan_scratch(const frz_plan* p, const char* purpose, frz_range* out) {
  if (!p || !purpose) return frz::fail(FRZ_ERR_ARGUMENT, "frz_plan_scratch: null argument");
  for (const auto& [name, range] : p->scratch) {
    if (name == purpose) {
      if (out) *out = range;
      return FRZ_OK;
    }
  }
  return frz::fail(FRZ_ERR_ARGUMENT, std::string("frz_plan_scratch: no working buffer ") + purpose);
}

int frz_plan_role(const frz_plan* p, int layer, int role, uint64_t* tensor) {
  if (!p || !tensor) return frz::fail(FRZ_ERR_ARGUMENT, "frz_plan_role: null argument");
  int64_t t = -1;
  if (layer == -1 && role == FRZ_ROLE_EMBEDDING) t = p->model.embedding;
  else if (layer == -1 && role == FRZ_ROLE_OUTPUT_NORM) t = p->model.output_norm;
  else if (layer >= 0 && layer < (int)p->model.layers.size() && role >= 0 && role < kRoles)
    t = p->model.layers[layer].roles[role];
  if (t < 0) return frz::fail(FRZ_ERR_ARGUMENT, "frz_plan_role: no such tensor");
  *tensor = (uint64_t)t;
  return FRZ_OK;
}

}  // extern "C"
