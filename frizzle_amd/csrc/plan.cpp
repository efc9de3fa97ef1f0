// The residency plan (src/core/residency/plan.h:14-326): where every weight,
// each layer's KV cache and every working buffer lies on the device, and the
// context offered, as a pure function of a Gemma 3 file's tensor index, the
// device's limits and the load policy. No device and no I/O. Host code only.
//
// What the plan must give is fixed by the reference's contract (the ranges
// a reference-side shim passes through unchanged); how it is computed here:
//
//   1. Everything to place becomes a *claim*: a run of bytes in one pool,
//      with how much room must be free at its start (a group's span, so the
//      group lands in one buffer) and whether it takes a buffer of its own.
//      Weights claim one run per piece of whole rows, in file order;
//      working buffers claim one buffer each; the cache one run per layer's
//      keys and values.
//   2. One routine lays out a pool's claims in order: each goes after the
//      newest buffer's last range, at the next aligned offset, when its room
//      fits there, and opens a new buffer when not.
//   3. The context offered is solved in closed form: the cache's cost is
//      piecewise linear in the context (a ring stops growing at its length),
//      so the largest context within the budget lies on the first segment
//      whose end no longer fits, found by walking the rings' lengths.
//   4. The ranges are read back into the plan's tables: pieces, groups (a
//      group stands when its members' ranges share a buffer and span at most
//      one range), working buffers by purpose, caches by layer.
//
// Rules kept from the reference (plan.h:27-72): three pools never sharing a
// buffer; every range aligned to storage_offset_alignment, its length
// rounded up to 4 and at most min(binding, buffer); a row is every dimension
// but the last; a sliding layer's ring holds window + 512 + the rollback
// reserve; the context lies between min(512, trained) and the trained
// context. Sizes are summed and multiplied with overflow checks.

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

constexpr uint64_t kWordBytes = 4;       // a binding's size is whole 32-bit words
constexpr uint32_t kBlockTokens = 512;   // a prefill step's rows (plan.h kPrefillBlock)
constexpr uint32_t kKeysPerChunk = 64;   // an attention chunk's keys
constexpr uint32_t kTopCandidates = 64;  // the selection's candidates
constexpr uint32_t kSelectTile = 1024;   // logits a selection workgroup reduces
constexpr uint64_t kEditWordsEach = 5;   // edit.h: words an edit entry takes
constexpr uint64_t kEditCapacity = 4096; // edit.h: entries a table holds
constexpr int kLayerRoles = 13;          // a layer's roles (frz_role 0 .. 12)

// Checked 64-bit arithmetic: every operation folds into `ok`.
struct Checked {
  bool ok = true;
  uint64_t sum(uint64_t a, uint64_t b) {
    uint64_t r = 0;
    ok = ok && !__builtin_add_overflow(a, b, &r);
    return r;
  }
  uint64_t product(uint64_t a, uint64_t b) {
    uint64_t r = 0;
    ok = ok && !__builtin_mul_overflow(a, b, &r);
    return r;
  }
  // v raised to a multiple of `step`, a power of two.
  uint64_t up_to(uint64_t v, uint64_t step) { return sum(v, step - 1) & ~(step - 1); }
};

struct Buffer {
  int pool;
  uint64_t size;
};

// A run of bytes to place (step 1 above).
struct Claim {
  uint64_t bytes = 0;  // before rounding to whole words
  uint64_t room = 0;   // contiguous bytes that must fit from its start
  bool own = false;    // a buffer of its own
};

// Lays out one pool's claims in order (step 2). `where[i]` receives claim
// i's range; new buffers are appended to `buffers`. False on overflow.
bool lay_out(int pool, const std::vector<Claim>& claims, const frz_plan_limits& lim,
             std::vector<Buffer>& buffers, std::vector<frz_range>& where) {
  Checked c;
  const uint64_t cap = lim.max_buffer_size;
  bool shared = false;  // the newest buffer takes further claims
  where.clear();
  where.reserve(claims.size());
  for (const Claim& claim : claims) {
    const uint64_t length = c.up_to(claim.bytes, kWordBytes);
    uint64_t at = 0;
    bool fresh = claim.own || !shared;
    if (!fresh) {
      at = c.up_to(buffers.back().size, lim.storage_offset_alignment);
      const uint64_t need = std::max(length, claim.room);
      fresh = at > cap || need > cap - at;
    }
    if (!c.ok) return false;
    if (fresh) {
      buffers.push_back({pool, 0});
      at = 0;
    }
    buffers.back().size = at + length;
    where.push_back({(uint32_t)(buffers.size() - 1), at, length});
    shared = !claim.own;
  }
  return true;
}

// The longest range a binding may hold.
uint64_t binding_cap(const frz_plan_limits& l) {
  return std::min(l.max_storage_binding_size, l.max_buffer_size) & ~(kWordBytes - 1);
}

// The model as the plan needs it (the reference's ModelDescription, for
// Gemma 3): per layer its role tensors (index positions, -1 absent), widths
// and the keys it attends to.
struct LayerShape {
  std::array<int64_t, kLayerRoles> tensor;
  uint32_t query_heads, kv_heads, head_dim, ffn, window;
};
struct Described {
  std::vector<LayerShape> layers;
  uint32_t hidden = 0, vocab = 0, trained_context = 0;
  int64_t embedding = -1, output_norm = -1;
  frz_model_config config{};
};

struct Working {
  const char* purpose;
  uint64_t rows, width;  // f32 values
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
  Described model;
  std::vector<uint32_t> formats;  // each tensor's GGUF format, index order
};

namespace {

const char* const kLeafNames[kLayerRoles] = {
    "attn_q.weight",      "attn_k.weight",       "attn_v.weight",
    "attn_output.weight", "ffn_gate.weight",     "ffn_up.weight",
    "ffn_down.weight",    "attn_norm.weight",    "attn_q_norm.weight",
    "attn_k_norm.weight", "post_attention_norm.weight", "ffn_norm.weight",
    "post_ffw_norm.weight"};

int64_t find(const Index& ix, const std::string& name) {
  const auto it = ix.tensor_at.find(name);
  return it == ix.tensor_at.end() ? -1 : (int64_t)it->second;
}

// The model a Gemma 3 file describes (gemma3.cpp:44-95, describe.cpp:
// 205-380): shapes from its metadata, the trained context from
// gemma3.context_length; a layer attends to the whole trained context when it
// ends its pattern (l % pattern == pattern - 1), else to the window.
int describe(const frz_gguf* g, Described& d, std::string& subject) {
  if (int rc = frz_gemma3_config_from_gguf(g, 0, &d.config)) {
    subject = frz_last_error();
    return rc;
  }
  uint32_t trained = 0;
  if (frz_gguf_get_u32(g, "gemma3.context_length", &trained) != FRZ_OK || trained == 0) {
    subject = "gemma3.context_length";
    return FRZ_ERR_ARGUMENT;
  }
  const frz_model_config& c = d.config;
  d.hidden = (uint32_t)c.hidden;
  d.vocab = (uint32_t)c.vocab;
  d.trained_context = trained;
  d.embedding = find(g->index, "token_embd.weight");
  d.output_norm = find(g->index, "output_norm.weight");
  if (d.output_norm < 0) {
    subject = "output_norm.weight";
    return FRZ_ERR_ARGUMENT;
  }
  d.layers.resize(c.layers);
  for (int l = 0; l < c.layers; ++l) {
    LayerShape& s = d.layers[l];
    const std::string prefix = "blk." + std::to_string(l) + ".";
    for (int r = 0; r < kLayerRoles; ++r) s.tensor[r] = find(g->index, prefix + kLeafNames[r]);
    s.query_heads = (uint32_t)c.query_heads;
    s.kv_heads = (uint32_t)c.kv_heads;
    s.head_dim = (uint32_t)c.head_dim;
    s.ffn = (uint32_t)c.ffn;
    const bool global = l % c.pattern == c.pattern - 1;
    s.window = global ? trained : (uint32_t)c.window;
  }
  d.config.context = (int)trained;
  return FRZ_OK;
}

// Floats of range sums a product of `rows` outputs over `columns` inputs
// keeps when the prefill splits it along K (graph.cpp:117-130,
// matmul.cpp:235-256: split when the groups per 64-row output tile, doubled,
// allow it, at most 64 tiles of tokens overall, 32 tokens a tile, never past
// a prefill block).
uint64_t split_sum_floats(uint64_t rows, uint64_t columns) {
  const uint64_t tiles = (rows + 63) / 64;
  const uint64_t token_tiles = std::min(columns / 32 * 2 / tiles, 64 / tiles);
  if (token_tiles == 0) return 0;
  const uint64_t tokens = std::min<uint64_t>(token_tiles * 32, kBlockTokens);
  return tokens < 2 ? 0 : tokens * rows * 32;
}

// The working buffers a decoder step binds, in graph.cpp:132-198's order
// (their names are the interface: the graph binds them by purpose).
std::vector<Working> working_buffers(const Described& m, uint32_t& partial_rows) {
  uint64_t query = 0, kv = 0, ffn = 0, heads = 0, sums = 1;
  for (const LayerShape& l : m.layers) {
    const uint64_t q = (uint64_t)l.query_heads * l.head_dim;
    const uint64_t k = (uint64_t)l.kv_heads * l.head_dim;
    query = std::max(query, q);
    kv = std::max(kv, k);
    heads = std::max<uint64_t>(heads, l.query_heads);
    ffn = std::max<uint64_t>(ffn, l.ffn);
    sums = std::max({sums, split_sum_floats(q + 2 * k, m.hidden), split_sum_floats(m.hidden, q),
                     split_sum_floats(m.hidden, l.ffn)});
  }
  const uint64_t chunks = ((uint64_t)m.trained_context + kKeysPerChunk - 1) / kKeysPerChunk;
  partial_rows = (uint32_t)std::max<uint64_t>(chunks, kBlockTokens);
  const uint64_t first_pass = (m.vocab + kSelectTile - 1) / kSelectTile;
  const uint64_t second_pass = (kTopCandidates * first_pass + kSelectTile - 1) / kSelectTile;
  frz_model_config at_trained = m.config;
  at_trained.context = (int)m.trained_context;
  const uint64_t capture_words = frz_capture_words(&at_trained, nullptr);
  const uint64_t edit_words = 2ull * m.layers.size() + kEditWordsEach * kEditCapacity;
  const uint64_t B = kBlockTokens;
  return {{"hidden", B, m.hidden},
          {"normed", B, m.hidden},
          {"query", B, query},
          {"key", B, kv},
          {"value", B, kv},
          {"attention", B, query},
          {"partials", partial_rows, query},
          {"partial_stats", partial_rows, 2 * heads},
          {"output", B, m.hidden},
          {"activation", B, ffn},
          {"logits", 1, m.vocab},
          {"partials_a", 1, 2ull * kTopCandidates * first_pass},
          {"partials_b", 1, 2ull * kTopCandidates * second_pass},
          {"candidates", 1, 2ull * kTopCandidates},
          {"sampled", 1, 4},
          {"range_sums", 1, sums},
          {"edit_table", 1, edit_words},
          {"captures", 1, capture_words}};
}

// A layer's Q/K/V or gate/up, members in output order.
struct Candidate {
  std::array<uint64_t, 3> members;
  uint32_t count;
};

std::vector<Candidate> candidates(const Described& m) {
  std::vector<Candidate> out;
  auto have = [](const LayerShape& l, int role) { return l.tensor[role] >= 0; };
  for (const LayerShape& l : m.layers) {
    if (have(l, FRZ_ROLE_Q) && have(l, FRZ_ROLE_K) && have(l, FRZ_ROLE_V))
      out.push_back({{(uint64_t)l.tensor[FRZ_ROLE_Q], (uint64_t)l.tensor[FRZ_ROLE_K],
                      (uint64_t)l.tensor[FRZ_ROLE_V]}, 3});
    if (have(l, FRZ_ROLE_GATE) && have(l, FRZ_ROLE_UP))
      out.push_back({{(uint64_t)l.tensor[FRZ_ROLE_GATE], (uint64_t)l.tensor[FRZ_ROLE_UP], 0}, 2});
  }
  return out;
}

// The bytes a candidate's span takes when every tensor from its first member
// to its last is laid out back to back (whole words, aligned starts), or 0
// when the members differ in format or input width, one is empty, or some
// tensor of the span or the span itself is longer than a range.
uint64_t span_room(const std::vector<Tensor>& ts, const Candidate& g, const frz_plan_limits& lim) {
  const Tensor& lead = ts[g.members[0]];
  const uint64_t cap = binding_cap(lim);
  uint64_t lo = g.members[0], hi = g.members[0];
  for (uint32_t i = 0; i < g.count; ++i) {
    const Tensor& t = ts[g.members[i]];
    if (t.type != lead.type || t.shape[0] != lead.shape[0] || t.elements == 0 || t.shape[0] == 0)
      return 0;
    lo = std::min(lo, g.members[i]);
    hi = std::max(hi, g.members[i]);
  }
  Checked c;
  uint64_t total = 0;
  for (uint64_t k = lo; k <= hi; ++k) {
    if (ts[k].bytes > cap) return 0;
    total = c.sum(total, c.up_to(c.up_to(ts[k].bytes, kWordBytes), lim.storage_offset_alignment));
  }
  return c.ok && total <= cap ? total : 0;
}

// Step 1 and 2 for the weights: one claim per piece of whole rows, a kept
// candidate's span as room at its first tensor's first piece.
int place_weights(const Index& ix, const Described& m, const frz_plan_limits& lim,
                  frz_plan& p, std::string& subject) {
  const std::vector<Tensor>& ts = ix.tensors;
  const uint64_t cap = binding_cap(lim);
  std::vector<uint64_t> room(ts.size(), 0);
  std::vector<Candidate> kept;
  for (const Candidate& g : candidates(m)) {
    const uint64_t bytes = span_room(ts, g, lim);
    if (bytes == 0) continue;
    const uint64_t first = *std::min_element(g.members.begin(), g.members.begin() + g.count);
    room[first] = std::max(room[first], bytes);
    kept.push_back(g);
  }
  p.tensors.assign(ts.size(), {});
  struct Owner {
    uint64_t tensor, first_row, rows;
  };
  std::vector<Claim> claims;
  std::vector<Owner> owners;
  for (uint64_t i = 0; i < ts.size(); ++i) {
    const Tensor& t = ts[i];
    const uint64_t rows = t.shape[0] == 0 ? 0 : t.elements / t.shape[0];
    if (rows == 0) continue;
    const uint64_t row_bytes = t.bytes / rows;
    if (row_bytes > cap) {
      subject = t.name;
      return FRZ_PLAN_ROW_EXCEEDS_BINDING;
    }
    const uint64_t rows_each = cap / row_bytes;
    for (uint64_t r = 0; r < rows; r += rows_each) {
      const uint64_t n = std::min(rows_each, rows - r);
      claims.push_back({n * row_bytes, r == 0 ? room[i] : 0, false});
      owners.push_back({i, r, n});
    }
  }
  std::vector<frz_range> where;
  if (!lay_out(FRZ_POOL_WEIGHTS, claims, lim, p.buffers, where)) {
    subject.clear();
    return FRZ_PLAN_OVERFLOW;
  }
  for (size_t k = 0; k < claims.size(); ++k)
    p.tensors[owners[k].tensor].push_back({where[k], owners[k].first_row, owners[k].rows});
  // A kept candidate stands as a group when its members landed in one
  // buffer within one range (each member is one piece: it fits a range).
  for (const Candidate& g : kept) {
    const frz_range& lead = p.tensors[g.members[0]].front().range;
    uint64_t begin = lead.offset, end = lead.offset + lead.length;
    bool together = true;
    for (uint32_t i = 1; i < g.count; ++i) {
      const frz_range& r = p.tensors[g.members[i]].front().range;
      together = together && r.buffer == lead.buffer;
      begin = std::min(begin, r.offset);
      end = std::max(end, r.offset + r.length);
    }
    if (!together || end - begin > cap) continue;
    frz_plan::Group out{{g.members[0], g.members[1], g.members[2]}, g.count,
                        {lead.buffer, begin, end - begin}};
    p.groups.push_back(out);
  }
  return FRZ_PLAN_OK;
}

int place_working(const Described& m, const frz_plan_limits& lim, frz_plan& p,
                  std::string& subject) {
  const std::vector<Working> wants = working_buffers(m, p.partial_rows);
  std::vector<Claim> claims;
  for (const Working& w : wants) {
    Checked c;
    const uint64_t bytes = c.product(c.product(w.rows, w.width), 4);
    subject = w.purpose;
    if (!c.ok) return FRZ_PLAN_OVERFLOW;
    if (bytes > binding_cap(lim)) return FRZ_PLAN_SCRATCH_EXCEEDS_BINDING;
    claims.push_back({bytes, 0, true});
  }
  subject.clear();
  std::vector<frz_range> where;
  if (!lay_out(FRZ_POOL_SCRATCH, claims, lim, p.buffers, where)) return FRZ_PLAN_OVERFLOW;
  for (size_t k = 0; k < wants.size(); ++k) p.scratch.emplace_back(wants[k].purpose, where[k]);
  return FRZ_PLAN_OK;
}

uint64_t pool_total(const std::vector<Buffer>& buffers, int pool) {
  uint64_t total = 0;
  for (const Buffer& b : buffers) total += b.pool == pool ? b.size : 0;
  return total;
}

// A layer's cache as its cost: bytes a slot (keys or values) and the most
// slots its ring holds.
struct Ring {
  uint64_t slot_bytes, length;
};

// Keys plus values at context `ctx` over every layer; false on overflow.
bool cache_cost(const std::vector<Ring>& rings, uint64_t ctx, uint64_t& bytes) {
  Checked c;
  bytes = 0;
  for (const Ring& r : rings) bytes = c.sum(bytes, c.product(2 * std::min(ctx, r.length), r.slot_bytes));
  return c.ok;
}

// Step 3: the largest context in [lowest, highest] whose cost is at most
// `avail`, or 0 when `lowest` does not fit. The cost grows by 2 x the slot
// bytes of every ring still longer than the context for each token, so
// between consecutive ring lengths it is linear.
uint64_t solve_context(const std::vector<Ring>& rings, uint64_t lowest, uint64_t highest,
                       uint64_t avail) {
  uint64_t at = 0;
  if (!cache_cost(rings, lowest, at) || at > avail) return 0;
  std::vector<uint64_t> stops{highest};
  for (const Ring& r : rings) {
    if (r.length > lowest && r.length < highest) stops.push_back(r.length);
  }
  std::sort(stops.begin(), stops.end());
  uint64_t from = lowest;
  for (uint64_t stop : stops) {
    uint64_t cost = 0;
    if (cache_cost(rings, stop, cost) && cost <= avail) {
      from = stop;
      at = cost;
      continue;
    }
    // The answer lies in [from, stop): the slope there is constant.
    uint64_t slope = 0;
    for (const Ring& r : rings) slope += r.length > from ? 2 * r.slot_bytes : 0;
    return slope == 0 ? from : std::min(stop - 1, from + (avail - at) / slope);
  }
  return from;
}

int place_cache(const Described& m, const frz_plan_limits& lim, const frz_load_policy& policy,
                frz_plan& p) {
  const uint64_t cap = binding_cap(lim);
  std::vector<Ring> rings;
  // The context may not pass what lets every layer's keys fit a range.
  uint64_t highest = m.trained_context;
  for (const LayerShape& l : m.layers) {
    Checked c;
    Ring r{c.product((uint64_t)l.kv_heads * l.head_dim, 2),  // F16 values
           c.sum((uint64_t)l.window, c.sum(kBlockTokens, policy.rollback_reserve))};
    if (!c.ok) return FRZ_PLAN_OVERFLOW;
    const uint64_t whole = c.product(r.length, r.slot_bytes);
    if (r.slot_bytes != 0 && (!c.ok || whole > cap)) highest = std::min(highest, cap / r.slot_bytes);
    rings.push_back(r);
  }
  const uint64_t lowest = std::min<uint64_t>(kBlockTokens, m.trained_context);
  Checked c;
  const uint64_t padding =
      c.product(2 * m.layers.size(), c.sum(lim.storage_offset_alignment, kWordBytes));
  const uint64_t fixed = c.sum(c.sum(p.weight_bytes, p.scratch_bytes), padding);
  if (!c.ok) return FRZ_PLAN_OVERFLOW;
  const uint64_t avail = policy.memory_budget >= fixed ? policy.memory_budget - fixed : 0;
  const uint64_t ctx = highest < lowest ? 0 : solve_context(rings, lowest, highest, avail);
  if (ctx == 0 || policy.memory_budget < fixed) {
    // What the shortest context would need, as the refusal states it.
    uint64_t need = 0;
    if (highest < lowest || !cache_cost(rings, lowest, need)) return FRZ_PLAN_OVERFLOW;
    p.total_bytes = c.sum(fixed, need);
    return c.ok ? FRZ_PLAN_EXCEEDS_BUDGET : FRZ_PLAN_OVERFLOW;
  }
  p.context_offered = (uint32_t)ctx;
  std::vector<Claim> claims;
  for (const Ring& r : rings) {
    const uint64_t bytes = std::min(r.length, ctx) * r.slot_bytes;
    claims.push_back({bytes, 0, false});  // keys
    claims.push_back({bytes, 0, false});  // values
  }
  std::vector<frz_range> where;
  if (!lay_out(FRZ_POOL_CACHE, claims, lim, p.buffers, where)) return FRZ_PLAN_OVERFLOW;
  for (size_t l = 0; l < rings.size(); ++l)
    p.cache.push_back({where[2 * l], where[2 * l + 1],
                       (uint32_t)std::min(rings[l].length, ctx)});
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

int plan_into(const frz_gguf* index, const frz_plan_limits& lim, const frz_load_policy& policy,
              frz_plan& p, std::string& subject) {
  for (const Tensor& t : index->index.tensors) p.formats.push_back(t.type);
  if (describe(index, p.model, subject) != FRZ_OK) return FRZ_PLAN_NOT_DESCRIBED;
  if (int rc = place_weights(index->index, p.model, lim, p, subject)) return rc;
  p.weight_bytes = pool_total(p.buffers, FRZ_POOL_WEIGHTS);
  if (int rc = place_working(p.model, lim, p, subject)) return rc;
  p.scratch_bytes = pool_total(p.buffers, FRZ_POOL_SCRATCH);
  if (int rc = place_cache(p.model, lim, policy, p)) return rc;
  p.cache_bytes = pool_total(p.buffers, FRZ_POOL_CACHE);
  p.total_bytes = p.weight_bytes + p.scratch_bytes + p.cache_bytes;
  p.model.config.context = (int)p.context_offered;
  // A sliding layer's ring as placed: window + 512 + reserve, or the whole
  // context when that is shorter.
  p.model.config.local_slots = (int)std::min<uint64_t>(
      (uint64_t)p.model.config.window + kBlockTokens + policy.rollback_reserve,
      p.context_offered);
  return FRZ_PLAN_OK;
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
  std::string why;
  const int rc = plan_into(index, *limits, *policy, *p, why);
  summarize(*p, summary);
  copy_subject(why, subject, subject_cap);
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
  else if (layer >= 0 && layer < (int)p->model.layers.size() && role >= 0 && role < kLayerRoles)
    t = p->model.layers[layer].tensor[role];
  if (t < 0) return frz::fail(FRZ_ERR_ARGUMENT, "frz_plan_role: no such tensor");
  *tensor = (uint64_t)t;
  return FRZ_OK;
}

}  // extern "C"
