// The Gemma-3 model on the device and its steps: weights in the split Q4_0
// layout, F16 KV caches (a ring for sliding layers), the working buffers of a
// 512-token block, the graph of launches in the reference's order
// (src/core/graph/graph.cpp:290-470), one captured HIP graph for a fed decode
// step, and generation with prefix reuse.

#include <algorithm>
#include <cmath>
#include <cstring>
#include <map>
#include <tuple>
#include <vector>

#include "../../include/frizzle_hip.h"
#include "backend.h"
#include "kernels.h"
#include "numerics.h"

using namespace frz;

namespace {

constexpr uint32_t kToTheEnd = 0xFFFFFFFFu;  // edit/edit.h: kToTheEnd
constexpr int kMaxEdits = 4096;              // edit/edit.h: kMaxEdits
constexpr int kMaxVariants = 64;             // rows of a variants step

// ---- the synthetic weights -------------------------------------------------
// SplitMix64 (Steele, Lea, Flood 2014), one stream per (seed, layer, role).
struct SplitMix64 {
  uint64_t state;
  uint64_t next() {
    uint64_t z = (state += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
  }
  // Uniform in (0, 1): 53 bits, offset by half a unit.
  double uniform() { return ((double)(next() >> 11) + 0.5) * (1.0 / 9007199254740992.0); }
  // N(0, 1) by Box-Muller in f64, one value per two uniforms.
  double normal() {
    const double u1 = uniform(), u2 = uniform();
    return std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2);
  }
};

SplitMix64 stream_of(uint64_t seed, int layer, int role) {
  SplitMix64 s{seed ^ (0x6A09E667F3BCC909ull * (uint64_t)(layer + 2)) ^
               (0xBB67AE8584CAA73Bull * (uint64_t)(role + 1))};
  s.next();
  return s;
}

bool is_matrix(int role) { return role <= FRZ_ROLE_DOWN || role == FRZ_ROLE_EMBEDDING; }

// A matrix role's rows and columns (N rows of K, matmul.h:19-22).
void matrix_shape(const frz_model_config& c, int role, int* rows, int* cols) {
  const int q = c.query_heads * c.head_dim, kv = c.kv_heads * c.head_dim;
  switch (role) {
    case FRZ_ROLE_Q: *rows = q; *cols = c.hidden; break;
    case FRZ_ROLE_K:
    case FRZ_ROLE_V: *rows = kv; *cols = c.hidden; break;
    case FRZ_ROLE_O: *rows = c.hidden; *cols = q; break;
    case FRZ_ROLE_GATE:
    case FRZ_ROLE_UP: *rows = c.ffn; *cols = c.hidden; break;
    case FRZ_ROLE_DOWN: *rows = c.hidden; *cols = c.ffn; break;
    case FRZ_ROLE_EMBEDDING: *rows = c.vocab; *cols = c.hidden; break;
    default: *rows = 0; *cols = 0; break;
  }
}

int gain_width(const frz_model_config& c, int role) {
  return (role == FRZ_ROLE_Q_NORM || role == FRZ_ROLE_K_NORM) ? c.head_dim : c.hidden;
}

bool is_global(const frz_model_config& c, int layer) {
  return layer % c.pattern == c.pattern - 1;
}

struct Layer {
  QMatrix qkv;  // Q rows, then K, then V (one product, matmul.h:27-33)
  QMatrix o, gate, up, down;
  float* gains[6];  // attn, q, k, post_attn, ffn, post_ffn
  uint16_t* kcache;
  uint16_t* vcache;
  float* turns;
  int slots;
  int window;
  int max_chunks;
};

}  // namespace

struct frz_model {
  frz_device* dev = nullptr;
  frz_model_config c{};
  std::vector<void*> owned;
  std::vector<Layer> layers;
  QMatrix embedding{};
  float* output_norm = nullptr;
  // working buffers, a prefill block of rows each
  float *hidden = nullptr, *hidden_b = nullptr, *normed = nullptr, *qkv = nullptr, *attn = nullptr,
        *output = nullptr, *act = nullptr, *logits = nullptr, *partials = nullptr,
        *stats = nullptr;
  // A split down product's later range sums (kSplitParts x 16 rows x hidden),
  // added by the norm that reads its output.
  float* split_parts = nullptr;
  uint32_t *topk_scratch = nullptr, *candidates = nullptr, *sampled = nullptr,
           *token_log = nullptr, *edits = nullptr;
  uint32_t token_log_capacity = 0;
  size_t partial_floats = 0;
  DevStep* step = nullptr;       // device
  DevStep* step_host = nullptr;  // pinned
  hipGraphExec_t decode_exec = nullptr;
  hipGraph_t decode_graph = nullptr;
  bool use_graphs = true;  // false: decode steps launch their kernels one by one
  // The fast prefill mode (frz_model_set_prefill): steps of several rows run
  // their products on the bf16 matrix cores, their activations as pair
  // planes (widest row x 512 rows each) and K-split partial sums in `parts`.
  int prefill_mode = FRZ_PREFILL_EXACT;
  uint16_t *planes_hi = nullptr, *planes_lo = nullptr;
  // Each layer's weights as bf16 fragment planes (Q/K/V, O, gate and up,
  // down), made when the mode is set and again before the next fast step
  // after a tensor changes.
  struct WeightPlanes {
    uint4 *qkv, *o, *gate_up, *down;
  };
  std::vector<WeightPlanes> weight_planes;
  bool planes_stale = true;
  // While a profiled step is enqueued: its launches' events and names.
  StepProfile* profile = nullptr;
  StepProfile own_profile;  // frz_model_profile_step's
  float* parts = nullptr;
  size_t parts_stride = 0;  // floats a split's partial sums take
  // generation state: the tokens whose keys and values the caches hold, and
  // the placed edit table they were computed under
  std::vector<uint32_t> cached;
  std::vector<uint32_t> cached_edits;
  uint64_t written_end = 0;  // one past the last position any step wrote
  uint32_t reused = 0;       // prompt tokens the last generation took from the caches
  std::vector<uint32_t> edit_words;
  // Buffers of a variants step (frz_generate_variants), grown on demand:
  // each layer's caches once per variant, `rows` rows of logits and
  // selection, the edit tables edit_stride words apart, the token log and
  // the residual capture of `steps` steps.
  struct Variants {
    int rows = 0;
    uint32_t steps = 0, edit_stride = 0;
    bool capture = false;  // this run writes the residual capture
    uint32_t position = 0;  // the step being enqueued: every row's position
    std::vector<uint16_t*> kcache, vcache;
    float* logits = nullptr;
    float* residuals = nullptr;
    uint32_t *scratch = nullptr, *candidates = nullptr, *sampled = nullptr, *token_log = nullptr,
             *edits = nullptr;
  } variants;
  // The capture store (frz_model_set_capture): written by the step that ends
  // a prompt while capture_on; the readouts' own norm, logits and selection.
  bool capture_on = false;
  float* store = nullptr;
  uint64_t store_words = 0;
  std::vector<frz_capture_slots> slots;
  float *ro_normed = nullptr, *ro_logits = nullptr;
  uint32_t* ro_scratch = nullptr;
  // A model created from a plan: its planned buffers (each one allocation,
  // also listed in `owned`), whether the capture store is the plan's.
  bool is_planned = false;
  bool planned_store = false;
  std::vector<void*> planned;
  std::vector<uint64_t> planned_bytes;
};

namespace {

template <typename T>
int alloc(frz_model* m, T** p, size_t bytes) {
  void* v = nullptr;
  if (int rc = check_hip(hipMalloc(&v, bytes ? bytes : 1), "hipMalloc")) return rc;
  m->owned.push_back(v);
  *p = static_cast<T*>(v);
  return FRZ_OK;
}

int alloc_q4(frz_model* m, QMatrix* w, int rows, int cols, int format = kQ4_0) {
  const size_t blocks = (size_t)rows * cols / 32;
  uint8_t* codes;
  uint16_t* scales;
  if (int rc = alloc(m, &codes, blocks * code_bytes(format))) return rc;
  if (int rc = alloc(m, &scales, blocks * 2 * scale_halves(format))) return rc;
  *w = QMatrix{codes, scales, rows, cols, format};
  return FRZ_OK;
}

// Frees one of the model's allocations.
void release(frz_model* m, const void* p) {
  auto it = std::find(m->owned.begin(), m->owned.end(), const_cast<void*>(p));
  if (it == m->owned.end()) return;
  hipFree(*it);
  m->owned.erase(it);
}

// Before a launch of a profiled step: an event on the stream, and the
// launch's roles and layer (role null: the event after the last launch).
// Nothing while no profiled step is being enqueued.
void mark(frz_model* m, const char* role, uint32_t layer = FRZ_NO_LAYER) {
  StepProfile* p = m->profile;
  if (!p) return;
  if (p->failed) return;
  if (p->used == p->events.size()) {
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) {
      p->failed = true;
      return;
    }
    p->events.push_back(e);
    p->roles.push_back(nullptr);
    p->layers.push_back(FRZ_NO_LAYER);
  }
  if (hipEventRecord(p->events[p->used], m->dev->stream) != hipSuccess) {
    p->failed = true;
    return;
  }
  p->roles[p->used] = role;
  p->layers[p->used] = layer;
  ++p->used;
}

// The caches no longer hold what the prompt-reuse record says: weights
// changed, or a step the record does not track wrote them.
void forget_prefix(frz_model* m) {
  m->cached.clear();
  m->cached_edits.clear();
}

// Each layer's weights as the fast prefill mode's fragment planes
// (prefill_bf16.hip): 107 MB a Gemma-3-1B layer, allocated the first time.
int unpack_weight_planes(frz_model* m) {
  if (m->weight_planes.empty()) {
    std::vector<frz_model::WeightPlanes> planes;
    for (const Layer& L : m->layers) {
      frz_model::WeightPlanes p{};
      if (int rc = alloc(m, &p.qkv, bf16_planes_bytes(L.qkv.rows, L.qkv.cols, false))) return rc;
      if (int rc = alloc(m, &p.o, bf16_planes_bytes(L.o.rows, L.o.cols, false))) return rc;
      if (int rc = alloc(m, &p.gate_up, bf16_planes_bytes(L.gate.rows, L.gate.cols, true)))
        return rc;
      if (int rc = alloc(m, &p.down, bf16_planes_bytes(L.down.rows, L.down.cols, false)))
        return rc;
      planes.push_back(p);
    }
    m->weight_planes = std::move(planes);
  }
  hipStream_t s = m->dev->stream;
  hipError_t e = hipSuccess;
  for (size_t l = 0; l < m->layers.size() && e == hipSuccess; ++l) {
    const Layer& L = m->layers[l];
    const frz_model::WeightPlanes& p = m->weight_planes[l];
    e = launch_unpack_planes(s, L.qkv, nullptr, p.qkv);
    if (e == hipSuccess) e = launch_unpack_planes(s, L.o, nullptr, p.o);
    if (e == hipSuccess) e = launch_unpack_planes(s, L.gate, &L.up, p.gate_up);
    if (e == hipSuccess) e = launch_unpack_planes(s, L.down, nullptr, p.down);
  }
  if (int rc = check_hip(e, "unpacking the weight planes")) return rc;
  m->planes_stale = false;
  return FRZ_OK;
}

// A matrix in `format`: the same one when it already is, else new buffers
// (the old ones freed once the new exist, so a failure leaves the matrix as
// it was; a captured decode graph holds the old addresses, so it is dropped
// and captured again at the next decode).
int reformat(frz_model* m, QMatrix* w, int format) {
  if (w->format == format) return FRZ_OK;
  if (m->is_planned) {
    return fail(FRZ_ERR_ARGUMENT, "frz_model_set_tensor: the plan placed this tensor in format " +
                                      std::to_string(w->format) + ", not " +
                                      std::to_string(format));
  }
  if (int rc = check_hip(hipDeviceSynchronize(), "reformat sync")) return rc;
  QMatrix fresh;
  if (int rc = alloc_q4(m, &fresh, w->rows, w->cols, format)) return rc;
  release(m, w->codes);
  release(m, w->scales);
  *w = fresh;
  if (m->decode_exec) {
    hipGraphExecDestroy(m->decode_exec);
    m->decode_exec = nullptr;
  }
  if (m->decode_graph) {
    hipGraphDestroy(m->decode_graph);
    m->decode_graph = nullptr;
  }
  return FRZ_OK;
}

// Writes GGUF blocks of the matrix's format into rows [row0, row0 + rows):
// each block's scale halves to the scale stream, its codes to the code
// stream.
int upload_q4(frz_model* m, const QMatrix& w, int row0, int rows, const void* data) {
  const size_t blocks = (size_t)rows * w.cols / 32;
  const size_t first = (size_t)row0 * w.cols / 32;
  const int cb = code_bytes(w.format), sh = scale_halves(w.format);
  std::vector<uint8_t> codes(blocks * cb), scales(blocks * 2 * sh);
  if (int rc = frz_block_split(w.format, data, blocks, codes.data(), scales.data())) return rc;
  hipStream_t s = m->dev->stream;
  if (int rc = check_hip(hipMemcpyAsync(const_cast<uint8_t*>(w.codes) + first * cb, codes.data(),
                                        codes.size(), hipMemcpyHostToDevice, s),
                         "upload codes"))
    return rc;
  if (int rc = check_hip(hipMemcpyAsync(const_cast<uint16_t*>(w.scales) + first * sh,
                                        scales.data(), scales.size(), hipMemcpyHostToDevice, s),
                         "upload scales"))
    return rc;
  return check_hip(hipStreamSynchronize(s), "upload sync");
}

// The head, the selection and the draw, after the final norm wrote the step's
// last row into `normed`.
// A fed decode step also advances the step parameters at its end.
hipError_t enqueue_output(frz_model* m, int max_tokens, bool advance) {
  hipStream_t s = m->dev->stream;
  mark(m, "output.head");
  hipError_t e = launch_gemv(s, m->step, m->embedding, m->normed, m->c.hidden, m->logits,
                             m->c.vocab, max_tokens, true);
  if (e == hipSuccess) {
    mark(m, "output.select+output.draw");
    e = launch_select(s, m->step, m->logits, m->c.vocab, m->topk_scratch, m->candidates,
                      m->sampled, m->token_log, advance);
  }
  return e;
}

float scale_log2e_of(const frz_model_config& c) {
  return (float)((double)(1.0f / std::sqrt((float)c.head_dim)) * 1.4426950408889634);
}

// The capture store's readouts (capture.h:28-34): the last layer's is the
// step's own candidates; layer l's (l below it) is the residual entering
// layer l + 1, already in the store, through the final norm, the head and
// the selection. Run after the step's own output, into buffers of their own.
hipError_t enqueue_readouts(frz_model* m) {
  const frz_model_config& c = m->c;
  hipStream_t s = m->dev->stream;
  auto slot = [m](int l, frz_capture_slot frz_capture_slots::*field) {
    return m->store + (m->slots[l].*field).first;
  };
  mark(m, "output.readout");
  hipError_t e = launch_capture_copy(s, m->step, m->candidates, 0, 2 * kCandidates,
                                     slot(c.layers - 1, &frz_capture_slots::readout));
  for (int l = 0; l + 1 < c.layers && e == hipSuccess; ++l) {
    mark(m, "readout", l);
    NormArgs n{m->output_norm, nullptr, nullptr, slot(l + 1, &frz_capture_slots::residual),
               m->ro_normed, c.epsilon, c.hidden, false};
    e = launch_norm(s, m->step, n, 1);
    if (e == hipSuccess)
      e = launch_gemv(s, m->step, m->embedding, m->ro_normed, c.hidden, m->ro_logits, c.vocab,
                      1, false);
    if (e == hipSuccess)
      e = launch_topk(s, m->ro_logits, c.vocab, m->ro_scratch,
                      reinterpret_cast<uint32_t*>(slot(l, &frz_capture_slots::readout)));
  }
  return e;
}

// The first and last positions of a rows step's rows (-1: not known).
struct RowSpan {
  int64_t first = -1, last = -1;
};

// A step of several rows, in the graph's order (graph.cpp:290-470): the
// embedding; per layer the attention norm (adding the last block's
// post-normed output), Q/K/V, rope and the cache append, attention, O; the
// feed-forward norm, gate-up with GELU and the pins, down; then the final
// norm and, with logits, the output block. The rows are one sequence's
// positions (the final norm and head on the last row only), or with `v` a
// variants step: each row its own sequence over its own caches and edit
// table, every row's logits drawn from, the residual entering each layer
// captured. `span`: the positions of the step's rows, when the host knows
// them; the attention grids then cover only the chunks those rows read.
int enqueue_rows(frz_model* m, int max_tokens, bool logits, const frz_model::Variants* v,
                 RowSpan span = {}) {
  const frz_model_config& c = m->c;
  hipStream_t s = m->dev->stream;
  const int H = c.hidden, qw = c.query_heads * c.head_dim, kvw = c.kv_heads * c.head_dim;
  const int qkv_stride = qw + 2 * kvw;
  const float scale_log2e = scale_log2e_of(c);
  mark(m, "embed");
  hipError_t e = launch_gather(s, m->step, m->embedding, v ? v->sampled : m->sampled, m->hidden,
                               std::sqrt((float)H), max_tokens);
  // The step that ends a prompt fills the capture store, when it is on.
  const bool cap = !v && logits && m->capture_on;
  auto slot = [m](int l, frz_capture_slot frz_capture_slots::*field) {
    return m->store + (m->slots[l].*field).first;
  };
  const float* pending = nullptr;
  // Where the last down product left its later range sums, when it split.
  const float* pending_parts = nullptr;
  size_t parts_stride = (size_t)kSplitRows * H;
  int pending_count = kSplitParts;
  // The fast prefill mode: the products on bf16 pair operands, each K-split
  // product's partial sums in m->parts, added by the norm that reads them.
  const bool fast = !v && m->prefill_mode == FRZ_PREFILL_BF16;
  const float* block_out = m->output;  // where the last block's output lies
  if (fast && m->planes_stale) {
    if (int rc = unpack_weight_planes(m)) return rc;
  }
  auto fast_product = [&](const uint4* planes, const QMatrix& w, int ldx, float* y, int ldy,
                          int* splits) {
    Bf16Gemm g;
    g.w = planes;
    g.rows = w.rows;
    g.cols = w.cols;
    g.x_hi = m->planes_hi;
    g.x_lo = m->planes_lo;
    g.ldx = ldx;
    g.y = y;
    g.ldy = ldy;
    g.part_stride = m->parts_stride;
    *splits = y == m->parts ? bf16_splits_for(w.rows, w.cols, max_tokens, false) : 1;
    return launch_gemm_bf16(s, m->step, g, max_tokens, *splits);
  };
  if (fast) parts_stride = m->parts_stride;
  for (int l = 0; l < c.layers && e == hipSuccess; ++l) {
    const Layer& L = m->layers[l];
    NormArgs attn_norm{L.gains[0], pending, block_out, m->hidden, m->normed,
                       c.epsilon, H, false};
    attn_norm.parts = pending_parts;
    attn_norm.parts_stride = parts_stride;
    attn_norm.part_count = pending_count;
    if (fast) {
      attn_norm.normed_hi = m->planes_hi;
      attn_norm.normed_lo = m->planes_lo;
    }
    if (cap) {
      attn_norm.store_x = slot(l, &frz_capture_slots::residual);
      if (l > 0) attn_norm.store_added = slot(l - 1, &frz_capture_slots::mlp_added);
    }
    if (v && v->capture) {
      // [step][layer][row][hidden] for this step's rows
      attn_norm.capture = v->residuals + (size_t)l * max_tokens * H;
      attn_norm.capture_step = (size_t)c.layers * max_tokens * H;
    }
    uint16_t* kcache = v ? v->kcache[l] : L.kcache;
    uint16_t* vcache = v ? v->vcache[l] : L.vcache;
    const size_t cache_stride = v ? (size_t)L.slots * kvw : 0;
    mark(m, "attention.norm", l);
    e = launch_norm(s, m->step, attn_norm, max_tokens);
    int qkv_splits = 1;
    if (e == hipSuccess) {
      mark(m, "attention.qkv", l);
      e = fast ? fast_product(m->weight_planes[l].qkv, L.qkv, H, m->parts, qkv_stride,
                              &qkv_splits)
               : launch_gemv(s, m->step, L.qkv, m->normed, H, m->qkv, qkv_stride, max_tokens,
                             false);
    }
    if (v) {
      // Each variant's row is one decode token: the fused rope and attention
      // a (chunk, head, row), then each row's fold.
      if (e == hipSuccess) {
        DecodeAttentionArgs d{m->qkv,      L.turns,  L.gains[1],  L.gains[2], kcache,
                              vcache,      m->partials, m->partials + m->partial_floats,
                              L.slots,     L.window, c.head_dim, c.query_heads, c.kv_heads,
                              L.max_chunks, c.epsilon, scale_log2e, qkv_stride, cache_stride};
        // The rows' position is known here: only its live chunks launch.
        d.grid_chunks = std::min(L.max_chunks, live_chunks(v->position, L.window));
        mark(m, "attention.rope+attention.scores", l);
        e = launch_attention_decode(s, m->step, d, max_tokens);
      }
      if (e == hipSuccess) {
        mark(m, "attention.combine", l);
        e = launch_attention_fold(
            s, m->step,
            FoldArgs{m->partials, m->partials + m->partial_floats, m->attn, L.window,
                     L.max_chunks},
            max_tokens);
      }
    } else {
      if (e == hipSuccess) {
        // The fast mode's Q/K/V are the product's partial sums, the rope
        // adding them (its queries then go to m->qkv).
        const float* src = fast ? m->parts : m->qkv;
        RopeArgs r{L.turns,     L.gains[1],  L.gains[2],   m->qkv,     src + qw,
                   src + qw + kvw, qkv_stride, qkv_stride, kcache, vcache,
                   L.slots,     c.head_dim,  c.query_heads, c.kv_heads, c.epsilon, cache_stride};
        if (fast) {
          r.query_in = m->parts;
          r.part_stride = m->parts_stride;
          r.part_count = qkv_splits;
        }
        mark(m, "attention.rope", l);
        e = launch_rope(s, m->step, r, max_tokens);
      }
      if (cap && e == hipSuccess) {
        mark(m, "attention.capture", l);
        e = launch_capture_copy(s, m->step, m->qkv, qkv_stride, qw,
                                slot(l, &frz_capture_slots::query));
      }
      // The fast mode's chunk states on the matrix cores, folded as the
      // exact path folds them (the capture store's scores come from the
      // exact path: a step that captures runs it).
      const bool fast_attention = fast && !cap && span.first >= 0;
      if (fast_attention && e == hipSuccess) {
        FastAttentionArgs fa{m->qkv,      qkv_stride,  kcache,        vcache,
                             m->partials, m->partials + m->partial_floats, L.slots, L.window,
                             c.head_dim,  c.query_heads, c.kv_heads,  L.max_chunks,
                             scale_log2e};
        mark(m, "attention.scores", l);
        e = launch_attention_fast(
            s, m->step, fa, max_tokens,
            fast_attention_chunks((uint32_t)span.first, (uint32_t)span.last, L.window));
        if (e == hipSuccess) {
          FoldArgs f{m->partials, m->partials + m->partial_floats, m->attn, L.window,
                     L.max_chunks};
          f.out_hi = m->planes_hi;
          f.out_lo = m->planes_lo;
          mark(m, "attention.combine", l);
          e = launch_attention_fold(s, m->step, f, max_tokens);
        }
      } else if (e == hipSuccess) {
        AttentionArgs a{m->qkv,     qkv_stride, kcache,       vcache,         m->attn,
                        m->partials, m->partials + m->partial_floats, L.slots, L.window,
                        c.head_dim, c.query_heads, c.kv_heads, L.max_chunks, scale_log2e,
                        cache_stride};
        if (span.first >= 0) {
          a.grid_chunks = std::min(
              L.max_chunks,
              live_chunks_over((uint32_t)span.first, (uint32_t)span.last, L.window));
        }
        if (cap) {
          a.store_scores = slot(l, &frz_capture_slots::weights);
          a.store_stats = slot(l, &frz_capture_slots::stats);
          a.keys = (int)m->slots[l].keys;
        }
        mark(m, "attention.scores+attention.combine", l);
        e = launch_attention(s, m->step, a, max_tokens);
        if (cap && e == hipSuccess) {
          mark(m, "attention.weights", l);
          e = launch_capture_weights(s, m->step, a.store_scores, a.store_stats, a.keys,
                                     c.query_heads);
        }
      }
    }
    int o_splits = 1;
    if (fast && e == hipSuccess) {
      // The fast attention's fold wrote the pair planes; the exact one's
      // output (a step that captures) is split here.
      if (cap || span.first < 0) {
        mark(m, "attention.output", l);
        e = launch_split_rows(s, m->step, m->attn, qw, qw, m->planes_hi, m->planes_lo,
                              max_tokens);
      }
      if (e == hipSuccess) {
        mark(m, "attention.output", l);
        e = fast_product(m->weight_planes[l].o, L.o, qw, m->parts, H, &o_splits);
      }
    } else if (e == hipSuccess) {
      mark(m, "attention.output", l);
      e = launch_gemv(s, m->step, L.o, m->attn, qw, m->output, H, max_tokens, false);
    }
    if (e == hipSuccess) {
      NormArgs ffn_norm{L.gains[4], L.gains[3], fast ? m->parts : m->output, m->hidden,
                        m->normed, c.epsilon, H, false};
      if (fast && o_splits > 1) {
        ffn_norm.parts = m->parts + m->parts_stride;
        ffn_norm.parts_stride = m->parts_stride;
        ffn_norm.part_count = o_splits - 1;
      }
      if (fast) {
        ffn_norm.normed_hi = m->planes_hi;
        ffn_norm.normed_lo = m->planes_lo;
      }
      if (cap) ffn_norm.store_added = slot(l, &frz_capture_slots::attention_added);
      mark(m, "ffn.norm", l);
      e = launch_norm(s, m->step, ffn_norm, max_tokens);
    }
    if (fast && e == hipSuccess) {
      Bf16Gemm g;
      g.w = m->weight_planes[l].gate_up;
      g.rows = L.gate.rows;
      g.cols = L.gate.cols;
      g.gated = true;
      g.x_hi = m->planes_hi;
      g.x_lo = m->planes_lo;
      g.ldx = H;
      g.y = cap ? m->act : nullptr;  // the down product reads the planes
      g.ldy = c.ffn;
      g.edits = m->edits;
      g.layer = l;
      // The planes hold the normed rows this product reads: the activation
      // planes go after them.
      g.y_hi = m->planes_hi + (size_t)kPrefillBlock * H;
      g.y_lo = m->planes_lo + (size_t)kPrefillBlock * H;
      mark(m, "ffn.gate_up+ffn.edit", l);
      e = launch_gemm_bf16(s, m->step, g, max_tokens, 1);
    } else if (e == hipSuccess) {
      mark(m, "ffn.gate_up+ffn.edit", l);
      e = launch_gated(s, m->step, L.gate, L.up, m->normed, m->act, max_tokens,
                       v ? v->edits : m->edits, l, v ? v->edit_stride : 0);
    }
    if (cap && e == hipSuccess) {
      mark(m, "ffn.capture", l);
      e = launch_capture_copy(s, m->step, m->act, c.ffn, c.ffn,
                              slot(l, &frz_capture_slots::neurons));
    }
    if (fast) {
      int splits = 1;
      if (e == hipSuccess) {
        Bf16Gemm g;
        g.w = m->weight_planes[l].down;
        g.rows = L.down.rows;
        g.cols = L.down.cols;
        g.x_hi = m->planes_hi + (size_t)kPrefillBlock * H;
        g.x_lo = m->planes_lo + (size_t)kPrefillBlock * H;
        g.ldx = c.ffn;
        g.y = m->parts;
        g.ldy = H;
        g.part_stride = m->parts_stride;
        splits = bf16_splits_for(L.down.rows, L.down.cols, max_tokens, false);
        mark(m, "ffn.down", l);
        e = launch_gemm_bf16(s, m->step, g, max_tokens, splits);
      }
      pending = L.gains[5];
      block_out = m->parts;
      pending_parts = splits > 1 ? m->parts + m->parts_stride : nullptr;
      pending_count = splits - 1;
      continue;
    }
    // Down over a step of few rows splits its tiles' ranges in halves; the
    // next norm adds the later half's sums.
    const bool split = max_tokens <= kSplitRows && gemv_splits(L.down, max_tokens);
    if (e == hipSuccess) {
      mark(m, "ffn.down", l);
      e = split ? launch_gemv_split(s, m->step, L.down, m->act, c.ffn, m->output, H, max_tokens,
                                    m->split_parts, parts_stride)
                : launch_gemv(s, m->step, L.down, m->act, c.ffn, m->output, H, max_tokens, false);
    }
    pending = L.gains[5];
    pending_parts = split ? m->split_parts : nullptr;
  }
  if (e == hipSuccess) {
    NormArgs final_norm{m->output_norm, pending, block_out, m->hidden, m->normed,
                        c.epsilon, H, v == nullptr};
    final_norm.parts = pending_parts;
    final_norm.parts_stride = parts_stride;
    final_norm.part_count = pending_count;
    if (cap) final_norm.store_added = slot(c.layers - 1, &frz_capture_slots::mlp_added);
    mark(m, "output.norm");
    e = launch_norm(s, m->step, final_norm, max_tokens);
  }
  if (logits && e == hipSuccess) {
    if (!v) {
      e = enqueue_output(m, max_tokens, false);
      if (cap && e == hipSuccess) e = enqueue_readouts(m);
    } else {
      e = launch_gemv(s, m->step, m->embedding, m->normed, H, v->logits, c.vocab, max_tokens,
                      false);
      if (e == hipSuccess) {
        e = launch_select_rows(s, m->step, v->logits, c.vocab, max_tokens, v->scratch,
                               v->candidates, v->sampled, v->token_log);
      }
    }
  }
  return check_hip(e, "enqueue_rows");
}

// One layer of a one-token step: Q/K/V with the attention norm in its
// prologue (layer 0 gathering the embedding there), the fused rope and
// attention, O (with the fold in its prologue for sliding layers), gate-up
// with the feed-forward norm and the pins, down. `pending` is the last
// layer's post-feed-forward gain (null at layer 0).
hipError_t enqueue_decode_layer(frz_model* m, int l, const float* pending) {
  const frz_model_config& c = m->c;
  hipStream_t s = m->dev->stream;
  const int H = c.hidden;
  const Layer& L = m->layers[l];
  GemvInput in{};
  in.hidden = m->hidden_b;
  in.output = m->output;
  in.post_gain = pending;
  in.gain = L.gains[0];
  in.hidden_out = m->hidden;
  in.table = m->embedding;
  in.sampled = m->sampled;
  in.scale = std::sqrt((float)H);
  in.epsilon = c.epsilon;
  mark(m, l == 0 ? "embed+attention.norm+attention.qkv" : "attention.norm+attention.qkv", l);
  hipError_t e = launch_gemv_decode(s, m->step, L.qkv, in, l == 0 ? 2 : 1, m->qkv);
  if (e == hipSuccess) {
    DecodeAttentionArgs d{m->qkv,      L.turns,  L.gains[1],  L.gains[2], L.kcache,
                          L.vcache,    m->partials, m->partials + m->partial_floats, L.slots,
                          L.window,    c.head_dim, c.query_heads, c.kv_heads, L.max_chunks,
                          c.epsilon,   scale_log2e_of(c)};
    mark(m, "attention.rope+attention.scores", l);
    e = launch_attention_decode(s, m->step, d);
  }
  // O: local layers fold their few chunks in the product's prologue.
  if (e == hipSuccess) {
    GemvInput x{};
    if (L.max_chunks <= kFoldPrologueChunks) {
      x.partials = m->partials;
      x.stats = m->partials + m->partial_floats;
      x.window = L.window;
      mark(m, "attention.combine+attention.output", l);
      e = launch_gemv_decode(s, m->step, L.o, x, 3, m->output);
    } else {
      mark(m, "attention.combine", l);
      e = launch_attention_fold(
          s, m->step,
          FoldArgs{m->partials, m->partials + m->partial_floats, m->attn, L.window, L.max_chunks},
          1);
      x.x = m->attn;
      if (e == hipSuccess) {
        mark(m, "attention.output", l);
        e = launch_gemv_decode(s, m->step, L.o, x, 0, m->output);
      }
    }
  }
  if (e == hipSuccess) {
    GemvInput g{};
    g.hidden = m->hidden;
    g.output = m->output;
    g.post_gain = L.gains[3];
    g.gain = L.gains[4];
    g.hidden_out = m->hidden_b;
    g.epsilon = c.epsilon;
    mark(m, "ffn.norm+ffn.gate_up+ffn.edit", l);
    e = launch_gated_decode(s, m->step, L.gate, L.up, g, 1, m->act, m->edits, l);
  }
  if (e == hipSuccess) {
    GemvInput x{};
    x.x = m->act;
    mark(m, "ffn.down", l);
    e = launch_gemv_decode(s, m->step, L.down, x, 0, m->output);
  }
  return e;
}

// A step of one token: five launches a layer, each norm inside the product
// that reads it. The hidden row alternates between two buffers: Q/K/V's
// prologue reads hidden_b (layer 0: the embedding) and writes hidden;
// gate-up's reads hidden and writes hidden_b.
int enqueue_decode(frz_model* m, bool logits, bool advance) {
  const frz_model_config& c = m->c;
  hipStream_t s = m->dev->stream;
  hipError_t e = hipSuccess;
  const float* pending = nullptr;
  for (int l = 0; l < c.layers && e == hipSuccess; ++l) {
    e = enqueue_decode_layer(m, l, pending);
    pending = m->layers[l].gains[5];
  }
  if (e == hipSuccess && logits && m->embedding.format == kQ4_0) {
    // A Q4_0 head takes the final norm in its prologue (every workgroup
    // makes the normed row; the first also writes it to `normed`).
    GemvInput h{};
    h.hidden = m->hidden_b;
    h.output = m->output;
    h.post_gain = pending;
    h.gain = m->output_norm;
    h.normed_out = m->normed;
    h.epsilon = c.epsilon;
    mark(m, "output.norm+output.head");
    e = launch_gemv_decode(s, m->step, m->embedding, h, 1, m->logits);
    if (e == hipSuccess) {
      mark(m, "output.select+output.draw");
      e = launch_select(s, m->step, m->logits, c.vocab, m->topk_scratch, m->candidates,
                        m->sampled, m->token_log, advance);
    }
    return check_hip(e, "enqueue_decode");
  }
  if (e == hipSuccess) {
    NormArgs final_norm{m->output_norm, pending, m->output, m->hidden_b, m->normed,
                        c.epsilon, c.hidden, true};
    mark(m, "output.norm");
    e = launch_norm(s, m->step, final_norm, 1);
  }
  if (logits && e == hipSuccess) e = enqueue_output(m, 1, advance);
  return check_hip(e, "enqueue_decode");
}

// `advance`: a fed decode step (logits drawn), whose last kernel advances
// the step parameters for the next.
int enqueue_step(frz_model* m, int max_tokens, bool logits, bool advance = false,
                 RowSpan span = {}) {
  // A one-token step that ends a prompt (logits, not a fed decode step that
  // advances) takes the rows path when the capture store is on: its kernels
  // write the store, and the bits are the same either way.
  const bool ends_prompt = logits && !advance;
  return max_tokens == 1 && !(ends_prompt && m->capture_on)
             ? enqueue_decode(m, logits, advance)
             : enqueue_rows(m, max_tokens, logits, nullptr, span);
}

int build_decode_graph(frz_model* m) {
  if (m->decode_exec) return FRZ_OK;
  hipStream_t s = m->dev->stream;
  if (int rc = check_hip(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal),
                         "hipStreamBeginCapture"))
    return rc;
  int rc = enqueue_step(m, 1, true, true);
  hipGraph_t graph = nullptr;
  const int end_rc = check_hip(hipStreamEndCapture(s, &graph), "hipStreamEndCapture");
  if (rc == FRZ_OK) rc = end_rc;
  hipGraphExec_t exec = nullptr;
  if (rc == FRZ_OK) {
    rc = check_hip(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0), "hipGraphInstantiate");
  }
  if (rc != FRZ_OK) {
    // Nothing is kept from a failed capture, so the next call captures anew.
    if (graph) (void)hipGraphDestroy(graph);
    return rc;
  }
  m->decode_graph = graph;
  m->decode_exec = exec;
  return FRZ_OK;
}

// One fed decode step: the captured graph, or its launches one by one.
int launch_decode_step(frz_model* m) {
  if (m->use_graphs) {
    return check_hip(hipGraphLaunch(m->decode_exec, m->dev->stream), "hipGraphLaunch");
  }
  return enqueue_step(m, 1, true, true);
}

int put_step(frz_model* m) {
  hipStream_t s = m->dev->stream;
  if (int rc = check_hip(hipMemcpyAsync(m->step, m->step_host, sizeof(DevStep),
                                        hipMemcpyHostToDevice, s),
                         "step copy"))
    return rc;
  // The pinned record may be rewritten by the next call only once copied.
  return check_hip(hipStreamSynchronize(s), "step copy sync");
}

// The placed edit table (edit.cpp:136-161 with place(), edit.cpp:35-38):
// step-relative ranges moved to positions origin + step, saturating.
std::vector<uint32_t> place_table(const frz_model_config& c, const uint32_t* table,
                                  uint32_t words, uint32_t origin) {
  std::vector<uint32_t> out(table, table + words);
  if (words < (uint32_t)(2 * c.layers)) out.assign(2 * c.layers, 0);
  auto place = [origin](uint32_t step) -> uint32_t {
    if (step == kToTheEnd || step > kToTheEnd - origin) return kToTheEnd;
    return step + origin;
  };
  for (int l = 0; l < c.layers; ++l) {
    const uint32_t first = out[2 * l], count = out[2 * l + 1];
    for (uint32_t i = 0; i < count; ++i) {
      const size_t at = first + 5 * (size_t)i;
      if (at + 4 >= out.size()) break;
      out[at + 3] = place(out[at + 3]);
      out[at + 4] = place(out[at + 4]);
    }
  }
  return out;
}

// The first position at which two placed tables can act differently: the
// least first position among edits one holds and the other does not
// (cache/prefix.h:87-94, first_edit_difference).
uint32_t first_edit_difference(const frz_model_config& c, const std::vector<uint32_t>& a,
                               const std::vector<uint32_t>& b) {
  using Key = std::tuple<uint32_t, uint32_t, uint32_t, uint32_t, uint32_t, uint32_t>;
  auto edits_of = [&c](const std::vector<uint32_t>& t) {
    std::map<Key, int> out;
    for (int l = 0; l < c.layers && (size_t)(2 * l + 1) < t.size(); ++l) {
      const uint32_t first = t[2 * l], count = t[2 * l + 1];
      for (uint32_t i = 0; i < count; ++i) {
        const size_t at = first + 5 * (size_t)i;
        if (at + 4 >= t.size()) break;
        out[Key{(uint32_t)l, t[at], t[at + 1], t[at + 2], t[at + 3], t[at + 4]}] += 1;
      }
    }
    return out;
  };
  const auto ea = edits_of(a), eb = edits_of(b);
  uint32_t least = kToTheEnd;
  for (const auto& [k, n] : ea) {
    if (eb.find(k) == eb.end()) least = std::min(least, std::get<4>(k));
  }
  for (const auto& [k, n] : eb) {
    if (ea.find(k) == ea.end()) least = std::min(least, std::get<4>(k));
  }
  return least;
}

// A planned range's device address.
template <typename T>
T* planned_at(frz_model* m, const frz_range& r) {
  return reinterpret_cast<T*>(static_cast<uint8_t*>(m->planned[r.buffer]) + r.offset);
}

// A weight tensor of the plan as one piece: its address and GGUF format.
int planned_tensor(frz_model* m, const frz_plan* plan, int layer, int role, uint8_t** at,
                   uint32_t* format, uint64_t want_bytes) {
  uint64_t tensor = 0;
  uint32_t pieces = 0;
  if (frz_plan_role(plan, layer, role, &tensor) != FRZ_OK ||
      frz_plan_tensor(plan, tensor, 0, nullptr, &pieces) != FRZ_OK) {
    return fail(FRZ_ERR_ARGUMENT, "frz_model_create_planned: the plan has no tensor for layer " +
                                      std::to_string(layer) + " role " + std::to_string(role));
  }
  frz_piece piece;
  if (pieces != 1 || frz_plan_tensor(plan, tensor, 0, &piece, nullptr) != FRZ_OK) {
    return fail(FRZ_ERR_ARGUMENT, "frz_model_create_planned: tensor " + std::to_string(tensor) +
                                      " is in " + std::to_string(pieces) +
                                      " pieces; this backend runs each weight as one");
  }
  (void)frz_plan_format(plan, tensor, format);
  if (piece.range.length < want_bytes) {
    return fail(FRZ_ERR_ARGUMENT, "frz_model_create_planned: tensor " + std::to_string(tensor) +
                                      "'s range is shorter than its role needs");
  }
  *at = planned_at<uint8_t>(m, piece.range);
  return FRZ_OK;
}

// A working buffer: the plan's of that purpose when it is at least as large,
// else the backend's own.
template <typename T>
int working_buffer(frz_model* m, const frz_plan* plan, T** p, const char* purpose, size_t bytes) {
  frz_range r;
  if (plan && frz_plan_scratch(plan, purpose, &r) == FRZ_OK && r.length >= bytes) {
    *p = planned_at<T>(m, r);
    return FRZ_OK;
  }
  return alloc(m, p, bytes);
}

// A matrix in the device layout at `at`: its codes, then its scales.
QMatrix matrix_at(uint8_t* at, int rows, int cols, int format) {
  const size_t blocks = (size_t)rows * cols / 32;
  return QMatrix{at, reinterpret_cast<const uint16_t*>(at + blocks * code_bytes(format)), rows,
                 cols, format};
}

// Builds a model: from a plan (its buffers, weights, caches and the working
// buffers it names), or with every buffer its own allocation.
int create_model(frz_device* dev, const frz_model_config& c, const frz_plan* plan,
                 frz_model** out) {
  // The kernels are built for Gemma-3's attention shape (d = 256, four query
  // heads on one key-value head), rows the norm prologues take (hidden at most
  // 2,048) and contexts up to the trained 32,768 tokens. A sliding ring holds
  // a window and a prefill block, or every position the context has.
  const int least_ring = std::min(c.window + kPrefillBlock, c.context);
  if (c.head_dim != 256 || c.query_heads != 4 || c.kv_heads != 1 || c.hidden % 32 != 0 ||
      c.ffn % 32 != 0 || c.vocab < kCandidates || c.layers <= 0 || c.pattern <= 0 ||
      c.window <= 0 || c.context < kPrefillBlock || c.local_slots < least_ring ||
      c.hidden > 2048 || attention_max_chunks(c.context, c.context) > kMaxContextChunks) {
    return fail(FRZ_ERR_ARGUMENT, "frz_model_create: unsupported shape");
  }
  if (plan && c.hidden != 1152) {
    return fail(FRZ_ERR_ARGUMENT,
                "frz_model_create_planned: the grouped Q/K/V product runs at K = 1,152 only");
  }
  (void)hipSetDevice(dev->ordinal);
  frz_model* m = new frz_model();
  m->dev = dev;
  m->c = c;
  auto bail = [m](int rc) {
    frz_model_destroy(m);
    return rc;
  };
  if (plan) {
    frz_plan_summary sum;
    if (int rc = frz_plan_summarize(plan, &sum)) return bail(rc);
    m->planned.assign(sum.buffers, nullptr);
    m->planned_bytes.assign(sum.buffers, 0);
    for (uint32_t i = 0; i < sum.buffers; ++i) {
      int pool = 0;
      if (int rc = frz_plan_buffer(plan, i, &pool, &m->planned_bytes[i])) return bail(rc);
      if (int rc = alloc(m, &m->planned[i], m->planned_bytes[i])) return bail(rc);
    }
  }
  const int qw = c.query_heads * c.head_dim, kvw = c.kv_heads * c.head_dim;
  size_t max_partials = 0;
  m->layers.resize(c.layers);
  for (int l = 0; l < c.layers; ++l) {
    Layer& L = m->layers[l];
    if (plan) {
      uint8_t *q, *k, *v, *o, *gate, *up, *down;
      uint32_t fq, fk, fv, fo, fg, fu, fd;
      const uint64_t qb = (uint64_t)qw * c.hidden / 32 * 18, kb = (uint64_t)kvw * c.hidden / 32 * 18;
      const uint64_t ob = (uint64_t)c.hidden * qw / 32 * 18, fb = (uint64_t)c.ffn * c.hidden / 32 * 18;
      int rc = planned_tensor(m, plan, l, FRZ_ROLE_Q, &q, &fq, qb);
      if (!rc) rc = planned_tensor(m, plan, l, FRZ_ROLE_K, &k, &fk, kb);
      if (!rc) rc = planned_tensor(m, plan, l, FRZ_ROLE_V, &v, &fv, kb);
      if (!rc) rc = planned_tensor(m, plan, l, FRZ_ROLE_O, &o, &fo, ob);
      if (!rc) rc = planned_tensor(m, plan, l, FRZ_ROLE_GATE, &gate, &fg, fb);
      if (!rc) rc = planned_tensor(m, plan, l, FRZ_ROLE_UP, &up, &fu, fb);
      if (!rc) rc = planned_tensor(m, plan, l, FRZ_ROLE_DOWN, &down, &fd, fb);
      if (rc) return bail(rc);
      if (fq != kQ4_0 || fk != kQ4_0 || fv != kQ4_0 || fo != kQ4_0 || fg != kQ4_0 ||
          fu != kQ4_0 || (fd != kQ4_0 && fd != kQ4_1 && fd != kQ8_0)) {
        return bail(fail(FRZ_ERR_ARGUMENT,
                         "frz_model_create_planned: layer " + std::to_string(l) +
                             ": matrices Q4_0 (downs also Q4_1 or Q8_0)"));
      }
      // Q, K and V: one product over the members the plan placed apart.
      L.qkv = matrix_at(q, qw, c.hidden, kQ4_0);
      L.qkv.rows = qw + 2 * kvw;
      const QMatrix km = matrix_at(k, kvw, c.hidden, kQ4_0), vm = matrix_at(v, kvw, c.hidden, kQ4_0);
      L.qkv.split[0] = qw;
      L.qkv.split[1] = qw + kvw;
      L.qkv.member_codes[0] = km.codes;
      L.qkv.member_scales[0] = km.scales;
      L.qkv.member_codes[1] = vm.codes;
      L.qkv.member_scales[1] = vm.scales;
      L.o = matrix_at(o, c.hidden, qw, kQ4_0);
      L.gate = matrix_at(gate, c.ffn, c.hidden, kQ4_0);
      L.up = matrix_at(up, c.ffn, c.hidden, kQ4_0);
      L.down = matrix_at(down, c.hidden, c.ffn, (int)fd);
      for (int g = 0; g < 6; ++g) {
        uint8_t* at;
        uint32_t f;
        const int role = FRZ_ROLE_ATTN_NORM + g;
        if (int rc2 = planned_tensor(m, plan, l, role, &at, &f, (uint64_t)gain_width(c, role) * 4))
          return bail(rc2);
        L.gains[g] = reinterpret_cast<float*>(at);
      }
    } else {
      if (int rc = alloc_q4(m, &L.qkv, qw + 2 * kvw, c.hidden)) return bail(rc);
      if (int rc = alloc_q4(m, &L.o, c.hidden, qw)) return bail(rc);
      if (int rc = alloc_q4(m, &L.gate, c.ffn, c.hidden)) return bail(rc);
      if (int rc = alloc_q4(m, &L.up, c.ffn, c.hidden)) return bail(rc);
      if (int rc = alloc_q4(m, &L.down, c.hidden, c.ffn)) return bail(rc);
      for (int g = 0; g < 6; ++g) {
        const int role = FRZ_ROLE_ATTN_NORM + g;
        if (int rc = alloc(m, &L.gains[g], (size_t)gain_width(c, role) * 4)) return bail(rc);
      }
    }
    const bool global = is_global(c, l);
    L.window = global ? c.context : c.window;
    size_t cache = 0;
    if (plan) {
      frz_range keys, values;
      uint32_t slots = 0;
      if (int rc = frz_plan_cache(plan, (uint32_t)l, &keys, &values, &slots)) return bail(rc);
      L.slots = (int)slots;
      cache = (size_t)L.slots * kvw * 2;
      if (keys.length < cache || values.length < cache || L.slots < std::min(L.window + kPrefillBlock, c.context))
        return bail(fail(FRZ_ERR_ARGUMENT, "frz_model_create_planned: layer " +
                                               std::to_string(l) + "'s cache is too small"));
      L.kcache = planned_at<uint16_t>(m, keys);
      L.vcache = planned_at<uint16_t>(m, values);
    } else {
      L.slots = global ? c.context : c.local_slots;
      cache = (size_t)L.slots * kvw * 2;
      if (int rc = alloc(m, &L.kcache, cache)) return bail(rc);
      if (int rc = alloc(m, &L.vcache, cache)) return bail(rc);
    }
    L.max_chunks = attention_max_chunks(L.window, L.slots);
    max_partials = std::max(max_partials, (size_t)kPrefillBlock * L.max_chunks * qw);
    (void)hipMemsetAsync(L.kcache, 0, cache, dev->stream);
    (void)hipMemsetAsync(L.vcache, 0, cache, dev->stream);
    std::vector<float> turns(c.head_dim / 2);
    frz_rope_turns(global ? c.rope_global : c.rope_local, c.head_dim, turns.data());
    if (int rc = alloc(m, &L.turns, turns.size() * 4)) return bail(rc);
    (void)hipMemcpy(L.turns, turns.data(), turns.size() * 4, hipMemcpyHostToDevice);
  }
  if (plan) {
    uint8_t *emb, *norm;
    uint32_t fe, fn;
    if (int rc = planned_tensor(m, plan, -1, FRZ_ROLE_EMBEDDING, &emb, &fe,
                                (uint64_t)c.vocab * c.hidden / 32 * 18))
      return bail(rc);
    if (int rc = planned_tensor(m, plan, -1, FRZ_ROLE_OUTPUT_NORM, &norm, &fn, (uint64_t)c.hidden * 4))
      return bail(rc);
    if (fe != kQ4_0 && fe != kQ8_0)
      return bail(fail(FRZ_ERR_ARGUMENT, "frz_model_create_planned: the embedding is Q4_0 or Q8_0"));
    m->embedding = matrix_at(emb, c.vocab, c.hidden, (int)fe);
    m->output_norm = reinterpret_cast<float*>(norm);
  } else {
    if (int rc = alloc_q4(m, &m->embedding, c.vocab, c.hidden)) return bail(rc);
    if (int rc = alloc(m, &m->output_norm, (size_t)c.hidden * 4)) return bail(rc);
  }
  const size_t B = kPrefillBlock;
  // The O product's fold prologue reads the states of kFoldPrologueChunks
  // chunks whatever a step's count (a prefill block's states are larger).
  max_partials = std::max(max_partials, (size_t)64 * kFoldPrologueChunks * qw);
  m->partial_floats = max_partials;
  auto working = [&](auto** p, const char* purpose, size_t bytes) {
    return working_buffer(m, plan, p, purpose, bytes);
  };
  if (int rc = working(&m->hidden, "hidden", B * c.hidden * 4)) return bail(rc);
  if (int rc = alloc(m, &m->hidden_b, (size_t)c.hidden * 4)) return bail(rc);
  if (int rc = working(&m->normed, "normed", B * c.hidden * 4)) return bail(rc);
  if (int rc = alloc(m, &m->qkv, B * (qw + 2 * kvw) * 4)) return bail(rc);
  if (int rc = working(&m->attn, "attention", B * qw * 4)) return bail(rc);
  if (int rc = working(&m->output, "output", B * c.hidden * 4)) return bail(rc);
  if (int rc = working(&m->act, "activation", B * c.ffn * 4)) return bail(rc);
  if (int rc = working(&m->logits, "logits", (size_t)c.vocab * 4)) return bail(rc);
  if (int rc = alloc(m, &m->partials, (max_partials + max_partials / 64) * 4)) return bail(rc);
  if (int rc = alloc(m, &m->split_parts, (size_t)kSplitParts * kSplitRows * c.hidden * 4))
    return bail(rc);
  if (int rc = alloc(m, &m->topk_scratch, topk_scratch_words(c.vocab) * 4)) return bail(rc);
  if (int rc = working(&m->candidates, "candidates", 2 * kCandidates * 4)) return bail(rc);
  if (int rc = working(&m->sampled, "sampled", 4 * 4)) return bail(rc);
  m->token_log_capacity = 1u << 16;
  if (int rc = alloc(m, &m->token_log, (size_t)2 * m->token_log_capacity * 4)) return bail(rc);
  const size_t edit_words = 2 * (size_t)c.layers + 5 * (size_t)kMaxEdits;
  if (int rc = working(&m->edits, "edit_table", edit_words * 4)) return bail(rc);
  (void)hipMemsetAsync(m->edits, 0, edit_words * 4, dev->stream);
  (void)hipMemsetAsync(m->sampled, 0, 16, dev->stream);
  (void)hipMemsetAsync(m->output, 0, B * c.hidden * 4, dev->stream);
  if (plan) {
    // The capture store is the plan's "captures" buffer when it holds it.
    frz_range r;
    const uint64_t words = frz_capture_words(&c, nullptr);
    if (frz_plan_scratch(plan, "captures", &r) == FRZ_OK && words != 0 && r.length >= words * 4) {
      m->store = planned_at<float>(m, r);
      m->planned_store = true;
    }
  }
  if (int rc = alloc(m, &m->step, sizeof(DevStep))) return bail(rc);
  if (int rc = check_hip(hipHostMalloc((void**)&m->step_host, sizeof(DevStep)), "hipHostMalloc"))
    return bail(rc);
  std::memset(m->step_host, 0, sizeof(DevStep));
  m->edit_words.assign(2 * c.layers, 0);
  m->is_planned = plan != nullptr;
  if (int rc = check_hip(hipStreamSynchronize(dev->stream), "create sync")) return bail(rc);
  *out = m;
  return FRZ_OK;
}

}  // namespace

extern "C" {

void frz_gemma3_1b_config(frz_model_config* out, int context) {
  frz_model_config c{};
  c.hidden = 1152;
  c.ffn = 6912;
  c.head_dim = 256;
  c.query_heads = 4;
  c.kv_heads = 1;
  c.layers = 26;
  c.vocab = 262144;
  c.window = 512;
  c.pattern = 6;
  c.context = context > 0 ? context : 8192;
  c.local_slots = 512 + 512 + 4096;  // plan.h:50-55: window + block + reserve
  c.rope_local = 10000.0f;
  c.rope_global = 1000000.0f;
  c.epsilon = 1e-6f;
  *out = c;
}

uint64_t frz_tensor_bytes(const frz_model_config* config, int role) {
  if (is_matrix(role)) {
    int rows, cols;
    matrix_shape(*config, role, &rows, &cols);
    return (uint64_t)rows * cols / 32 * 18;
  }
  if (role == FRZ_ROLE_OUTPUT_NORM) return (uint64_t)config->hidden * 4;
  if (role >= FRZ_ROLE_ATTN_NORM && role <= FRZ_ROLE_POST_FFN_NORM)
    return (uint64_t)gain_width(*config, role) * 4;
  return 0;
}

int frz_synth_tensor(const frz_model_config* config, uint64_t seed, int layer, int role,
                     void* out, uint64_t bytes) {
  if (!config || !out) return fail(FRZ_ERR_ARGUMENT, "frz_synth_tensor: null argument");
  if (bytes != frz_tensor_bytes(config, role) || bytes == 0) {
    return fail(FRZ_ERR_ARGUMENT, "frz_synth_tensor: wrong size for the role");
  }
  SplitMix64 rng = stream_of(seed, layer, role);
  if (is_matrix(role)) {
    uint8_t* p = static_cast<uint8_t*>(out);
    const uint64_t blocks = bytes / 18;
    for (uint64_t b = 0; b < blocks; ++b) {
      const uint16_t d = f16_pack((float)std::fabs(0.02 * rng.normal()));
      p[18 * b] = (uint8_t)(d & 0xFF);
      p[18 * b + 1] = (uint8_t)(d >> 8);
      const uint64_t c0 = rng.next(), c1 = rng.next();
      for (int i = 0; i < 8; ++i) {
        p[18 * b + 2 + i] = (uint8_t)(c0 >> (8 * i));
        p[18 * b + 10 + i] = (uint8_t)(c1 >> (8 * i));
      }
    }
  } else {
    float* g = static_cast<float*>(out);
    for (uint64_t i = 0; i < bytes / 4; ++i) g[i] = (float)(1.0 + 0.1 * rng.normal());
  }
  return FRZ_OK;
}

int frz_model_create(frz_device* dev, const frz_model_config* config, frz_model** out) {
  if (!dev || !config || !out) return fail(FRZ_ERR_ARGUMENT, "frz_model_create: null argument");
  return create_model(dev, *config, nullptr, out);
}

int frz_model_create_planned(frz_device* dev, const frz_plan* plan, frz_model** out) {
  if (!dev || !plan || !out) return fail(FRZ_ERR_ARGUMENT, "frz_model_create_planned: null argument");
  frz_model_config c;
  if (int rc = frz_plan_config(plan, &c)) return rc;
  return create_model(dev, c, plan, out);
}

int frz_model_planned_buffer(const frz_model* m, uint32_t index, void** dev_ptr, uint64_t* size) {
  if (!m || index >= m->planned.size())
    return fail(FRZ_ERR_ARGUMENT, "frz_model_planned_buffer: no such planned buffer");
  if (dev_ptr) *dev_ptr = m->planned[index];
  if (size) *size = m->planned_bytes[index];
  return FRZ_OK;
}

int frz_device_plan_limits(frz_device* dev, frz_plan_limits* out) {
  if (!dev || !out) return fail(FRZ_ERR_ARGUMENT, "frz_device_plan_limits: null argument");
  out->max_buffer_size = dev->props.totalGlobalMem;
  out->max_storage_binding_size = dev->props.totalGlobalMem;
  out->storage_offset_alignment = 256;
  return FRZ_OK;
}

void frz_model_destroy(frz_model* m) {
  if (!m) return;
  (void)hipSetDevice(m->dev->ordinal);
  (void)hipStreamSynchronize(m->dev->stream);
  if (m->decode_exec) hipGraphExecDestroy(m->decode_exec);
  if (m->decode_graph) hipGraphDestroy(m->decode_graph);
  for (void* p : m->owned) hipFree(p);
  if (m->step_host) hipHostFree(m->step_host);
  delete m;
}

int frz_model_set_tensor(frz_model* m, int layer, int role, const void* data, uint64_t bytes) {
  return frz_model_set_tensor_format(m, layer, role, is_matrix(role) ? kQ4_0 : 0, data, bytes);
}

int frz_model_set_tensor_format(frz_model* m, int layer, int role, int format, const void* data,
                                uint64_t bytes) {
  if (!m || !data) return fail(FRZ_ERR_ARGUMENT, "frz_model_set_tensor: null argument");
  forget_prefix(m);
  m->planes_stale = true;
  const frz_model_config& c = m->c;
  if (role < 0 || role > FRZ_ROLE_OUTPUT_NORM) return fail(FRZ_ERR_ARGUMENT, "frz_model_set_tensor: role");
  const bool ok_format = !is_matrix(role)          ? format == 0
                         : role == FRZ_ROLE_DOWN   ? (format == kQ4_0 || format == kQ4_1 || format == kQ8_0)
                         : role == FRZ_ROLE_EMBEDDING ? (format == kQ4_0 || format == kQ8_0)
                                                      : format == kQ4_0;
  if (!ok_format) {
    return fail(FRZ_ERR_ARGUMENT, "frz_model_set_tensor: format " + std::to_string(format) +
                                      " is not run for this role (matrices Q4_0 (2); down also "
                                      "Q4_1 (3) or Q8_0 (8); the embedding also Q8_0)");
  }
  const uint64_t want = is_matrix(role) ? frz_tensor_bytes(&c, role) / 18 * gguf_block_bytes(format)
                                        : frz_tensor_bytes(&c, role);
  if (bytes != want || bytes == 0) {
    return fail(FRZ_ERR_ARGUMENT, "frz_model_set_tensor: wrong size for the role");
  }
  if (role == FRZ_ROLE_EMBEDDING || role == FRZ_ROLE_OUTPUT_NORM) {
    if (layer != -1) return fail(FRZ_ERR_ARGUMENT, "frz_model_set_tensor: global tensor, layer -1");
    if (role == FRZ_ROLE_EMBEDDING) {
      if (int rc = reformat(m, &m->embedding, format)) return rc;
      return upload_q4(m, m->embedding, 0, c.vocab, data);
    }
    return check_hip(hipMemcpy(m->output_norm, data, bytes, hipMemcpyHostToDevice), "upload");
  }
  if (layer < 0 || layer >= c.layers) return fail(FRZ_ERR_ARGUMENT, "frz_model_set_tensor: layer");
  Layer& L = m->layers[layer];
  if (role == FRZ_ROLE_DOWN) {
    if (int rc = reformat(m, &L.down, format)) return rc;
  }
  const int qw = c.query_heads * c.head_dim, kvw = c.kv_heads * c.head_dim;
  if (has_members(L.qkv) && (role == FRZ_ROLE_Q || role == FRZ_ROLE_K || role == FRZ_ROLE_V)) {
    // Each member in its own planned range.
    const int member = role - FRZ_ROLE_Q;
    QMatrix w{member == 0 ? L.qkv.codes : L.qkv.member_codes[member - 1],
              member == 0 ? L.qkv.scales : L.qkv.member_scales[member - 1],
              member == 0 ? qw : kvw, c.hidden, kQ4_0};
    return upload_q4(m, w, 0, w.rows, data);
  }
  switch (role) {
    case FRZ_ROLE_Q: return upload_q4(m, L.qkv, 0, qw, data);
    case FRZ_ROLE_K: return upload_q4(m, L.qkv, qw, kvw, data);
    case FRZ_ROLE_V: return upload_q4(m, L.qkv, qw + kvw, kvw, data);
    case FRZ_ROLE_O: return upload_q4(m, L.o, 0, c.hidden, data);
    case FRZ_ROLE_GATE: return upload_q4(m, L.gate, 0, c.ffn, data);
    case FRZ_ROLE_UP: return upload_q4(m, L.up, 0, c.ffn, data);
    case FRZ_ROLE_DOWN: return upload_q4(m, L.down, 0, c.hidden, data);
    default:
      return check_hip(hipMemcpy(L.gains[role - FRZ_ROLE_ATTN_NORM], data, bytes,
                                 hipMemcpyHostToDevice),
                       "upload gain");
  }
}

int frz_model_get_config(const frz_model* m, frz_model_config* out) {
  if (!m || !out) return fail(FRZ_ERR_ARGUMENT, "frz_model_get_config: null argument");
  *out = m->c;
  return FRZ_OK;
}

int frz_model_synthesize(frz_model* m, uint64_t seed) {
  if (!m) return fail(FRZ_ERR_ARGUMENT, "frz_model_synthesize: null model");
  std::vector<uint8_t> buf;
  auto one = [&](int layer, int role) {
    const uint64_t bytes = frz_tensor_bytes(&m->c, role);
    buf.resize(bytes);
    if (int rc = frz_synth_tensor(&m->c, seed, layer, role, buf.data(), bytes)) return rc;
    return frz_model_set_tensor(m, layer, role, buf.data(), bytes);
  };
  for (int l = 0; l < m->c.layers; ++l) {
    for (int role = FRZ_ROLE_Q; role <= FRZ_ROLE_POST_FFN_NORM; ++role) {
      if (int rc = one(l, role)) return rc;
    }
  }
  if (int rc = one(-1, FRZ_ROLE_EMBEDDING)) return rc;
  return one(-1, FRZ_ROLE_OUTPUT_NORM);
}

int frz_model_set_capture(frz_model* m, int enabled) {
  if (!m) return fail(FRZ_ERR_ARGUMENT, "frz_model_set_capture: null model");
  const frz_model_config& c = m->c;
  if (enabled && m->slots.empty()) {
    const uint64_t words = frz_capture_words(&c, nullptr);
    if (words == 0) return fail(FRZ_ERR_ARGUMENT, "frz_model_set_capture: store too large");
    std::vector<frz_capture_slots> slots(c.layers);
    for (int l = 0; l < c.layers; ++l) {
      if (int rc = frz_capture_layer(&c, l, &slots[l])) return rc;
    }
    // A planned model's store is the plan's "captures" buffer.
    if (!m->store) {
      if (int rc = alloc(m, &m->store, words * 4)) return rc;
    }
    if (int rc = alloc(m, &m->ro_normed, (size_t)c.hidden * 4)) return rc;
    if (int rc = alloc(m, &m->ro_logits, (size_t)c.vocab * 4)) return rc;
    if (int rc = alloc(m, &m->ro_scratch, topk_scratch_words(c.vocab) * 4)) return rc;
    if (int rc = check_hip(hipMemsetAsync(m->store, 0, words * 4, m->dev->stream), "store"))
      return rc;
    m->store_words = words;
    m->slots = std::move(slots);
  }
  m->capture_on = enabled != 0;
  return check_hip(hipStreamSynchronize(m->dev->stream), "capture sync");
}

int frz_model_read_capture(frz_model* m, uint32_t* out, uint64_t words) {
  if (!m || !out) return fail(FRZ_ERR_ARGUMENT, "frz_model_read_capture: null argument");
  if (!m->store || words > m->store_words) {
    return fail(FRZ_ERR_ARGUMENT, "frz_model_read_capture: no store, or more words than it has");
  }
  if (int rc = check_hip(hipMemcpyAsync(out, m->store, words * 4, hipMemcpyDeviceToHost,
                                        m->dev->stream),
                         "read capture"))
    return rc;
  return check_hip(hipStreamSynchronize(m->dev->stream), "read capture sync");
}

uint32_t frz_model_reused(const frz_model* m) { return m ? m->reused : 0; }

int frz_model_set_prefill(frz_model* m, int mode) {
  if (!m) return fail(FRZ_ERR_ARGUMENT, "frz_model_set_prefill: null model");
  if (mode != FRZ_PREFILL_EXACT && mode != FRZ_PREFILL_BF16)
    return fail(FRZ_ERR_ARGUMENT, "frz_model_set_prefill: mode " + std::to_string(mode));
  const frz_model_config& c = m->c;
  if (mode == FRZ_PREFILL_BF16 && !m->planes_hi) {
    const int qw = c.query_heads * c.head_dim, qkv = qw + 2 * c.kv_heads * c.head_dim;
    for (const Layer& L : m->layers) {
      if (!bf16_gemm_shape_ok(L.qkv, c.hidden, qkv) || !bf16_gemm_shape_ok(L.o, qw, c.hidden) ||
          !bf16_gemm_shape_ok(L.gate, c.hidden, c.ffn) ||
          !bf16_gemm_shape_ok(L.down, c.ffn, c.hidden))
        return fail(FRZ_ERR_ARGUMENT, "frz_model_set_prefill: a shape the bf16 products refuse");
    }
    // Planes: the normed rows (hidden wide) then the activation rows (ffn
    // wide), which the gated product writes while reading the first.
    const size_t plane = (size_t)kPrefillBlock * (c.hidden + std::max(c.ffn, qw));
    m->parts_stride = (size_t)kPrefillBlock * std::max(c.hidden, qkv);
    if (int rc = alloc(m, &m->planes_hi, plane * 2)) return rc;
    if (int rc = alloc(m, &m->planes_lo, plane * 2)) return rc;
    if (int rc = alloc(m, &m->parts, m->parts_stride * kMaxBf16Splits * sizeof(float))) return rc;
  }
  // The weight planes are made afresh: a caller may have written the
  // weights through the planned buffers.
  if (mode == FRZ_PREFILL_BF16) {
    if (int rc = unpack_weight_planes(m)) return rc;
  }
  if (mode != m->prefill_mode) forget_prefix(m);
  m->prefill_mode = mode;
  return FRZ_OK;
}

int frz_model_set_graphs(frz_model* m, int enabled) {
  if (!m) return fail(FRZ_ERR_ARGUMENT, "frz_model_set_graphs: null model");
  m->use_graphs = enabled != 0;
  return FRZ_OK;
}

// An edit table as the kernels read it (edit.h:50-60), padded to the
// per-layer words; refused when an edit's words run past it, a neuron or
// kind is out of range, or a layer's edits are not sorted by neuron.
static int check_table(const frz_model_config& c, std::vector<uint32_t>& t, const char* what) {
  const size_t cap = 2 * (size_t)c.layers + 5 * (size_t)kMaxEdits;
  if (t.size() < (size_t)(2 * c.layers)) t.resize(2 * c.layers, 0);
  if (t.size() > cap) return fail(FRZ_ERR_ARGUMENT, std::string(what) + ": more than 4096 edits");
  for (int l = 0; l < c.layers; ++l) {
    const uint64_t first = t[2 * l], count = t[2 * l + 1];
    if (count && first + 5 * count > t.size()) {
      return fail(FRZ_ERR_ARGUMENT, std::string(what) + ": a layer's edits run past the table");
    }
    for (uint64_t i = 0; i < count; ++i) {
      const uint32_t* e = t.data() + first + 5 * i;
      if (e[0] >= (uint32_t)c.ffn || e[1] > 2u) {
        return fail(FRZ_ERR_ARGUMENT, std::string(what) + ": neuron or kind out of range");
      }
      if (i > 0 && e[0] < e[-5]) {
        return fail(FRZ_ERR_ARGUMENT, std::string(what) + ": a layer's edits are not by neuron");
      }
    }
  }
  return FRZ_OK;
}

int frz_model_set_edits(frz_model* m, const uint32_t* table, uint32_t words) {
  if (!m) return fail(FRZ_ERR_ARGUMENT, "frz_model_set_edits: null model");
  std::vector<uint32_t> t;
  if (table && words) t.assign(table, table + words);
  if (int rc = check_table(m->c, t, "frz_model_set_edits")) return rc;
  m->edit_words = t;
  if (int rc = check_hip(hipMemcpyAsync(m->edits, t.data(), t.size() * 4, hipMemcpyHostToDevice,
                                        m->dev->stream),
                         "edit table"))
    return rc;
  return check_hip(hipStreamSynchronize(m->dev->stream), "edit table sync");
}

static int model_step(frz_model* m, uint32_t position, uint32_t tokens, const uint32_t* ids,
               int logits, const frz_sampling* sampling);
static int model_decode(frz_model* m, uint32_t position, uint32_t steps, const frz_sampling* sampling,
                 uint32_t* tokens_out, uint32_t* failed_out);

int frz_model_step(frz_model* m, uint32_t position, uint32_t tokens, const uint32_t* ids,
                   int logits, const frz_sampling* sampling) {
  if (m) forget_prefix(m);
  return model_step(m, position, tokens, ids, logits, sampling);
}

int frz_model_decode(frz_model* m, uint32_t position, uint32_t steps,
                     const frz_sampling* sampling, uint32_t* tokens_out, uint32_t* failed_out) {
  if (m) forget_prefix(m);
  return model_decode(m, position, steps, sampling, tokens_out, failed_out);
}

static int model_step(frz_model* m, uint32_t position, uint32_t tokens, const uint32_t* ids,
               int logits, const frz_sampling* sampling) {
  if (!m || !ids || tokens == 0 || tokens > (uint32_t)kPrefillBlock) {
    return fail(FRZ_ERR_ARGUMENT, "frz_model_step: 1 to 512 tokens");
  }
  if ((uint64_t)position + tokens > (uint64_t)m->c.context) {
    return fail(FRZ_ERR_ARGUMENT, "frz_model_step: past the context");
  }
  for (uint32_t i = 0; i < tokens; ++i) {
    if (ids[i] >= (uint32_t)m->c.vocab) return fail(FRZ_ERR_ARGUMENT, "frz_model_step: token id");
  }
  if (sampling && (sampling->top_k < 1 || sampling->top_k > (uint32_t)kCandidates)) {
    return fail(FRZ_ERR_ARGUMENT, "frz_model_step: top_k outside 1..64");
  }
  DevStep& s = *m->step_host;
  std::memset(&s, 0, sizeof s);
  s.position = position;
  s.tokens = tokens;
  s.logits = logits ? 1 : 0;
  s.fed = 0;
  s.drawn = 0;
  fill_sampling(s, sampling);
  std::memcpy(s.ids, ids, tokens * 4);
  if (int rc = put_step(m)) return rc;
  return enqueue_step(m, (int)tokens, logits != 0, false,
                      RowSpan{(int64_t)position, (int64_t)position + tokens - 1});
}

static int model_decode(frz_model* m, uint32_t position, uint32_t steps, const frz_sampling* sampling,
                 uint32_t* tokens_out, uint32_t* failed_out) {
  if (!m || !tokens_out) return fail(FRZ_ERR_ARGUMENT, "frz_model_decode: null argument");
  if (steps == 0) return FRZ_OK;
  if (steps > m->token_log_capacity || (uint64_t)position + steps > (uint64_t)m->c.context) {
    return fail(FRZ_ERR_ARGUMENT, "frz_model_decode: too many steps for the context");
  }
  if (m->use_graphs) {
    if (int rc = build_decode_graph(m)) return rc;
  }
  DevStep& s = *m->step_host;
  std::memset(&s, 0, sizeof s);
  s.position = position;
  s.tokens = 1;
  s.logits = 1;
  s.fed = 1;
  s.drawn = 0;
  fill_sampling(s, sampling);
  if (int rc = put_step(m)) return rc;
  for (uint32_t i = 0; i < steps; ++i) {
    if (int rc = launch_decode_step(m)) return rc;
  }
  std::vector<uint32_t> log(2 * (size_t)steps);
  if (int rc = check_hip(hipMemcpyAsync(log.data(), m->token_log, log.size() * 4,
                                        hipMemcpyDeviceToHost, m->dev->stream),
                         "token log"))
    return rc;
  if (int rc = check_hip(hipStreamSynchronize(m->dev->stream), "decode sync")) return rc;
  for (uint32_t i = 0; i < steps; ++i) {
    tokens_out[i] = log[2 * i];
    if (failed_out) failed_out[i] = log[2 * i + 1];
  }
  return FRZ_OK;
}

int frz_model_time_decode(frz_model* m, uint32_t position, uint32_t steps,
                          const frz_sampling* sampling, double* us_per_step) {
  if (!m || !us_per_step || steps == 0) return fail(FRZ_ERR_ARGUMENT, "frz_model_time_decode");
  if (steps > m->token_log_capacity || (uint64_t)position + steps > (uint64_t)m->c.context) {
    return fail(FRZ_ERR_ARGUMENT, "frz_model_time_decode: too many steps for the context");
  }
  // The timed steps rewrite the caches from `position` on.
  forget_prefix(m);
  if (m->use_graphs) {
    if (int rc = build_decode_graph(m)) return rc;
  }
  DevStep& s = *m->step_host;
  std::memset(&s, 0, sizeof s);
  s.position = position;
  s.tokens = 1;
  s.logits = 1;
  s.fed = 1;
  fill_sampling(s, sampling);
  if (int rc = put_step(m)) return rc;
  hipEvent_t a, b;
  (void)hipEventCreate(&a);
  (void)hipEventCreate(&b);
  (void)hipEventRecord(a, m->dev->stream);
  int rc = FRZ_OK;
  for (uint32_t i = 0; i < steps && rc == FRZ_OK; ++i) {
    rc = launch_decode_step(m);
  }
  (void)hipEventRecord(b, m->dev->stream);
  if (rc == FRZ_OK) rc = check_hip(hipEventSynchronize(b), "hipEventSynchronize");
  float ms = 0.0f;
  if (rc == FRZ_OK) (void)hipEventElapsedTime(&ms, a, b);
  (void)hipEventDestroy(a);
  (void)hipEventDestroy(b);
  *us_per_step = (double)ms * 1000.0 / steps;
  return rc;
}

int frz_model_time_layer(frz_model* m, int layer, uint32_t position, uint32_t iters,
                         double* us_per_layer) {
  if (!m || !us_per_layer || iters == 0 || layer < 0 || layer >= m->c.layers ||
      position >= (uint32_t)m->c.context) {
    return fail(FRZ_ERR_ARGUMENT, "frz_model_time_layer: bad argument");
  }
  DevStep& st = *m->step_host;
  std::memset(&st, 0, sizeof st);
  st.position = position;
  st.tokens = 1;
  st.fed = 1;
  if (int rc = put_step(m)) return rc;
  hipStream_t s = m->dev->stream;
  // The layer's launches as one graph, replayed: each replay rewrites the
  // same cache slot with the same key and value.
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  if (int rc = check_hip(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal), "capture"))
    return rc;
  const hipError_t e =
      enqueue_decode_layer(m, layer, layer > 0 ? m->layers[layer - 1].gains[5] : nullptr);
  const hipError_t end = hipStreamEndCapture(s, &graph);
  int rc = check_hip(e != hipSuccess ? e : end, "frz_model_time_layer capture");
  if (rc == FRZ_OK) rc = check_hip(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0), "instantiate");
  hipEvent_t a = nullptr, b = nullptr;
  if (rc == FRZ_OK) {
    (void)hipEventCreate(&a);
    (void)hipEventCreate(&b);
    rc = check_hip(hipGraphLaunch(exec, s), "warm-up");
    if (rc == FRZ_OK) (void)hipEventRecord(a, s);
    for (uint32_t i = 0; i < iters && rc == FRZ_OK; ++i) rc = check_hip(hipGraphLaunch(exec, s), "replay");
    if (rc == FRZ_OK) (void)hipEventRecord(b, s);
    if (rc == FRZ_OK) rc = check_hip(hipEventSynchronize(b), "hipEventSynchronize");
    float ms = 0.0f;
    if (rc == FRZ_OK) (void)hipEventElapsedTime(&ms, a, b);
    *us_per_layer = (double)ms * 1000.0 / iters;
  }
  if (a) (void)hipEventDestroy(a);
  if (b) (void)hipEventDestroy(b);
  if (exec) (void)hipGraphExecDestroy(exec);
  if (graph) (void)hipGraphDestroy(graph);
  forget_prefix(m);  // its caches' slot at `position` was rewritten
  return rc;
}

static int read_back(frz_model* m, void* out, const void* src, size_t bytes) {
  if (int rc = check_hip(hipMemcpyAsync(out, src, bytes, hipMemcpyDeviceToHost, m->dev->stream),
                         "read back"))
    return rc;
  return check_hip(hipStreamSynchronize(m->dev->stream), "read back sync");
}

int frz_model_read_logits(frz_model* m, float* out, uint32_t count) {
  if (!m || !out || count > (uint32_t)m->c.vocab) return fail(FRZ_ERR_ARGUMENT, "read_logits");
  return read_back(m, out, m->logits, (size_t)count * 4);
}

int frz_model_read_record(frz_model* m, uint32_t record[4]) {
  if (!m || !record) return fail(FRZ_ERR_ARGUMENT, "read_record");
  return read_back(m, record, m->sampled, 16);
}

int frz_model_read_candidates(frz_model* m, uint32_t out[128]) {
  if (!m || !out) return fail(FRZ_ERR_ARGUMENT, "read_candidates");
  return read_back(m, out, m->candidates, 128 * 4);
}

int frz_model_read_hidden(frz_model* m, float* out, uint32_t rows) {
  if (!m || !out || rows > (uint32_t)kPrefillBlock) return fail(FRZ_ERR_ARGUMENT, "read_hidden");
  return read_back(m, out, m->normed, (size_t)rows * m->c.hidden * 4);
}

int frz_model_read_cache(frz_model* m, int layer, int values, uint16_t* out, uint64_t count) {
  if (!m || !out || layer < 0 || layer >= m->c.layers) return fail(FRZ_ERR_ARGUMENT, "read_cache");
  const Layer& L = m->layers[layer];
  const uint64_t cap = (uint64_t)L.slots * m->c.kv_heads * m->c.head_dim;
  if (count > cap) return fail(FRZ_ERR_ARGUMENT, "read_cache: more than the cache holds");
  return read_back(m, out, values ? L.vcache : L.kcache, count * 2);
}

}  // extern "C"

namespace frz {

// One step of a program's run (program.hip): the step record, already in
// pinned memory, is copied to the device in stream order; a fed decode step
// of one token with logits replays the decode graph (its launches one by
// one when graphs are off), any other step runs the rows path; a step with
// logits then copies the draw's 16-byte record to `readback` (pinned). The
// caches are rewritten, so generation's prompt-reuse record is forgotten.
int program_step(frz_model* m, const DevStep* pinned_step, uint32_t* readback,
                 StepProfile* profile) {
  hipStream_t s = m->dev->stream;
  forget_prefix(m);
  const DevStep& st = *pinned_step;
  const bool decode = st.tokens == 1 && st.fed != 0 && st.logits != 0 && !st.variants;
  // A profiled step runs its launches one by one (no captured graph).
  const bool graph = decode && m->use_graphs && !profile;
  if (graph) {
    if (int rc = build_decode_graph(m)) return rc;
  }
  if (int rc = check_hip(hipMemcpyAsync(m->step, pinned_step, sizeof(DevStep),
                                        hipMemcpyHostToDevice, s),
                         "program step record"))
    return rc;
  if (profile) profile->start();
  m->profile = profile;
  int rc = FRZ_OK;
  if (graph) {
    rc = launch_decode_step(m);
  } else if (decode) {
    rc = enqueue_step(m, 1, true, true);
  } else {
    // The record is host memory, written before this call: its positions
    // are known here.
    const int64_t last = (int64_t)st.position + (st.variants ? 0 : (int64_t)st.tokens - 1);
    rc = enqueue_step(m, (int)st.tokens, st.logits != 0, false,
                      RowSpan{(int64_t)st.position, last});
  }
  if (rc == FRZ_OK) mark(m, nullptr);
  m->profile = nullptr;
  if (rc != FRZ_OK) return rc;
  if (st.logits != 0 && readback) {
    return check_hip(hipMemcpyAsync(readback, m->sampled, 16, hipMemcpyDeviceToHost, s),
                     "program readback");
  }
  return FRZ_OK;
}

hipStream_t model_stream(const frz_model* m) { return m->dev->stream; }

int read_profile(const StepProfile& p, frz_launch_time* out, uint32_t cap, uint32_t* count) {
  if (p.failed) return fail(FRZ_ERR_DEVICE, "profiled step: a launch's event could not be recorded");
  const uint32_t n = p.used > 0 ? (uint32_t)p.used - 1 : 0;
  if (count) *count = n;
  if (n > 0) {
    if (int rc = check_hip(hipEventSynchronize(p.events[n]), "profiled step")) return rc;
  }
  for (uint32_t i = 0; i < n && i < cap && out; ++i) {
    float ms = 0.0f;
    if (int rc = check_hip(hipEventElapsedTime(&ms, p.events[i], p.events[i + 1]), "profile"))
      return rc;
    frz_launch_time& t = out[i];
    std::memset(t.role, 0, sizeof t.role);
    std::strncpy(t.role, p.roles[i] ? p.roles[i] : "", sizeof t.role - 1);
    t.layer = p.layers[i];
    t.graph_index = ~0u;
    t.microseconds = (double)ms * 1000.0;
  }
  return FRZ_OK;
}

}  // namespace frz

extern "C" {

int frz_model_profile_step(frz_model* m, uint32_t position, uint32_t tokens,
                           const uint32_t* ids, int logits, const frz_sampling* sampling,
                           frz_launch_time* out, uint32_t cap, uint32_t* count) {
  if (!m || !count) return fail(FRZ_ERR_ARGUMENT, "frz_model_profile_step: null argument");
  forget_prefix(m);
  m->own_profile.start();
  m->profile = &m->own_profile;
  int rc = model_step(m, position, tokens, ids, logits, sampling);
  if (rc == FRZ_OK) mark(m, nullptr);
  m->profile = nullptr;
  if (rc != FRZ_OK) return rc;
  return read_profile(m->own_profile, out, cap, count);
}

int frz_model_profile_decode(frz_model* m, uint32_t position, const frz_sampling* sampling,
                             frz_launch_time* out, uint32_t cap, uint32_t* count,
                             uint32_t* token) {
  if (!m || !count) return fail(FRZ_ERR_ARGUMENT, "frz_model_profile_decode: null argument");
  if ((uint64_t)position + 1 > (uint64_t)m->c.context)
    return fail(FRZ_ERR_ARGUMENT, "frz_model_profile_decode: past the context");
  forget_prefix(m);
  DevStep& s = *m->step_host;
  std::memset(&s, 0, sizeof s);
  s.position = position;
  s.tokens = 1;
  s.logits = 1;
  s.fed = 1;
  s.drawn = 0;
  fill_sampling(s, sampling);
  if (int rc = put_step(m)) return rc;
  m->own_profile.start();
  m->profile = &m->own_profile;
  int rc = enqueue_step(m, 1, true, true);
  if (rc == FRZ_OK) mark(m, nullptr);
  m->profile = nullptr;
  if (rc != FRZ_OK) return rc;
  if (int rc2 = read_profile(m->own_profile, out, cap, count)) return rc2;
  uint32_t log[2] = {0, 0};
  if (int rc2 = check_hip(hipMemcpyAsync(log, m->token_log, 8, hipMemcpyDeviceToHost,
                                         m->dev->stream),
                          "token log"))
    return rc2;
  if (int rc2 = check_hip(hipStreamSynchronize(m->dev->stream), "profile decode sync"))
    return rc2;
  if (token) *token = log[0];
  return FRZ_OK;
}

int frz_generate(frz_model* m, const uint32_t* prompt, uint32_t prompt_len,
                 const uint32_t* edit_table, uint32_t edit_words, const frz_sampling* sampling,
                 uint32_t max_tokens, const uint32_t* stop_ids, uint32_t stops,
                 uint32_t* tokens_out, uint32_t* drawn) {
  if (!m || !prompt || prompt_len == 0 || !tokens_out || !drawn) {
    return fail(FRZ_ERR_ARGUMENT, "frz_generate: null argument or empty prompt");
  }
  *drawn = 0;
  const frz_model_config& c = m->c;
  if ((uint64_t)prompt_len + max_tokens > (uint64_t)c.context) {
    return fail(FRZ_ERR_ARGUMENT, "frz_generate: prompt and reply exceed the context");
  }
  // A token past the vocabulary is refused before anything runs, by its
  // index (runtime.h: TurnFailure::Kept).
  for (uint32_t i = 0; i < prompt_len; ++i) {
    if (prompt[i] >= (uint32_t)c.vocab) {
      return fail(FRZ_ERR_ARGUMENT, "frz_generate: prompt token " + std::to_string(i) +
                                        " (id " + std::to_string(prompt[i]) +
                                        ") is past the vocabulary");
    }
  }
  const uint32_t origin = prompt_len - 1;
  std::vector<uint32_t> placed =
      place_table(c, edit_table ? edit_table : nullptr, edit_table ? edit_words : 0, origin);
  if (int rc = frz_model_set_edits(m, placed.data(), (uint32_t)placed.size())) return rc;
  // Reuse: the longest prefix of cached tokens the prompt repeats, cut at the
  // first position the edits act differently, and never past the prompt's
  // last token, whose row draws the first reply token.
  uint32_t common = 0;
  while (common < m->cached.size() && common < prompt_len && m->cached[common] == prompt[common])
    ++common;
  common = std::min(common, first_edit_difference(c, m->cached_edits, placed));
  common = std::min(common, prompt_len - 1);
  // A sliding layer's ring must still hold the window before the resume.
  if (m->written_end > (uint64_t)common + c.local_slots - c.window) common = 0;
  m->reused = common;
  // From here the caches are rewritten: the record is forgotten until the
  // run succeeds (a failed step leaves them partly rewritten, and the next
  // run starts over, as the reference empties the cache on a step failure,
  // runtime.h:51-54). The high-water mark is the most any run wrote since
  // the caches were last refilled from position 0 (cache/kv.h:30-35), here
  // counted before the steps so that a failure cannot understate it.
  forget_prefix(m);
  const uint64_t run_end = (uint64_t)prompt_len + (max_tokens > 1 ? max_tokens - 1 : 0);
  m->written_end = common == 0 ? run_end : std::max(m->written_end, run_end);
  uint32_t pos = common;
  while (pos < prompt_len) {
    const uint32_t n = std::min<uint32_t>(kPrefillBlock, prompt_len - pos);
    const bool last = pos + n == prompt_len;
    if (int rc = model_step(m, pos, n, prompt + pos, last ? 1 : 0, sampling)) return rc;
    pos += n;
  }
  if (max_tokens == 0) {
    if (int rc = check_hip(hipStreamSynchronize(m->dev->stream), "generate sync")) return rc;
    m->cached.assign(prompt, prompt + prompt_len);
    m->cached_edits = placed;
    return FRZ_OK;
  }
  uint32_t record[4];
  if (int rc = frz_model_read_record(m, record)) return rc;
  m->cached.assign(prompt, prompt + prompt_len);
  m->cached_edits = placed;
  std::vector<uint32_t> out{record[0]};
  bool stopped = record[1] != 0 || std::find(stop_ids, stop_ids + stops, record[0]) != stop_ids + stops;
  if (!stopped && max_tokens > 1) {
    std::vector<uint32_t> more(max_tokens - 1), failed(max_tokens - 1);
    if (int rc = model_decode(m, prompt_len, max_tokens - 1, sampling, more.data(),
                              failed.data())) {
      forget_prefix(m);
      return rc;
    }
    for (uint32_t i = 0; i + 1 < max_tokens; ++i) {
      out.push_back(more[i]);
      if (failed[i] || std::find(stop_ids, stop_ids + stops, more[i]) != stop_ids + stops) break;
    }
    // The caches now hold every fed token; the last drawn is not yet fed.
    for (uint32_t i = 0; i + 1 < out.size(); ++i) m->cached.push_back(out[i]);
    // Decode ran past a stop: those positions hold tokens the reply does not
    // keep, so the cached prefix ends at the reply's last fed token.
  }
  std::copy(out.begin(), out.end(), tokens_out);
  *drawn = (uint32_t)out.size();
  return FRZ_OK;
}

// Grows the variants buffers to `rows` rows, `steps` steps, tables of
// `stride` words and, when `residuals`, the capture; what is already large
// enough is kept.
static int ensure_variants(frz_model* m, int rows, uint32_t steps, uint32_t stride,
                           bool residuals) {
  frz_model::Variants& v = m->variants;
  const frz_model_config& c = m->c;
  const size_t kvw = (size_t)c.kv_heads * c.head_dim;
  if (rows > v.rows) {
    for (uint16_t* p : v.kcache) release(m, p);
    for (uint16_t* p : v.vcache) release(m, p);
    v.kcache.assign(c.layers, nullptr);
    v.vcache.assign(c.layers, nullptr);
    for (void* p : {(void*)v.logits, (void*)v.scratch, (void*)v.candidates, (void*)v.sampled})
      release(m, p);
    v.logits = nullptr;
    v.scratch = v.candidates = v.sampled = nullptr;
    v.rows = 0;
    for (int l = 0; l < c.layers; ++l) {
      const size_t bytes = (size_t)rows * m->layers[l].slots * kvw * 2;
      if (int rc = alloc(m, &v.kcache[l], bytes)) return rc;
      if (int rc = alloc(m, &v.vcache[l], bytes)) return rc;
    }
    if (int rc = alloc(m, &v.logits, (size_t)rows * c.vocab * 4)) return rc;
    if (int rc = alloc(m, &v.scratch, (size_t)rows * topk_scratch_words(c.vocab) * 4)) return rc;
    if (int rc = alloc(m, &v.candidates, (size_t)rows * 2 * kCandidates * 4)) return rc;
    if (int rc = alloc(m, &v.sampled, (size_t)rows * 16)) return rc;
    v.rows = rows;
    v.steps = 0;  // the token log and capture are sized by rows too
    v.edit_stride = 0;
  }
  if (steps > v.steps || (residuals && !v.residuals)) {
    release(m, v.token_log);
    release(m, v.residuals);
    v.token_log = nullptr;
    v.residuals = nullptr;
    v.steps = 0;
    const uint32_t n = std::max(steps, v.steps);
    if (int rc = alloc(m, &v.token_log, (size_t)n * v.rows * 2 * 4)) return rc;
    if (residuals) {
      if (int rc = alloc(m, &v.residuals, (size_t)n * c.layers * v.rows * c.hidden * 4))
        return rc;
    }
    v.steps = n;
  }
  if (stride > v.edit_stride) {
    release(m, v.edits);
    v.edits = nullptr;
    v.edit_stride = 0;
    if (int rc = alloc(m, &v.edits, (size_t)v.rows * stride * 4)) return rc;
    v.edit_stride = stride;
  }
  return FRZ_OK;
}

int frz_generate_variants(frz_model* m, const uint32_t* prompt, uint32_t prompt_len,
                          uint32_t variants, const uint32_t* edit_tables, uint32_t table_words,
                          const frz_sampling* sampling, uint32_t max_tokens,
                          const uint32_t* stop_ids, uint32_t stops, uint32_t* tokens_out,
                          uint32_t* drawn_out, float* residuals_out) {
  if (!m || !prompt || prompt_len == 0 || !tokens_out || !drawn_out) {
    return fail(FRZ_ERR_ARGUMENT, "frz_generate_variants: null argument or empty prompt");
  }
  const frz_model_config& c = m->c;
  if (variants < 1 || variants > (uint32_t)kMaxVariants) {
    return fail(FRZ_ERR_ARGUMENT, "frz_generate_variants: 1 to 64 variants");
  }
  if (max_tokens == 0 || (uint64_t)prompt_len + max_tokens > (uint64_t)c.context) {
    return fail(FRZ_ERR_ARGUMENT,
                "frz_generate_variants: at least one token, and prompt and reply within the "
                "context");
  }
  for (uint32_t i = 0; i < prompt_len; ++i) {
    if (prompt[i] >= (uint32_t)c.vocab)
      return fail(FRZ_ERR_ARGUMENT, "frz_generate_variants: token id");
  }
  if (sampling && (sampling->top_k < 1 || sampling->top_k > (uint32_t)kCandidates)) {
    return fail(FRZ_ERR_ARGUMENT, "frz_generate_variants: top_k outside 1..64");
  }
  // Each variant's table placed at the prompt's last position, as
  // frz_generate places one; none acts before it, so the prompt but its
  // last token is one prefix for all.
  const uint32_t origin = prompt_len - 1;
  std::vector<std::vector<uint32_t>> placed(variants);
  uint32_t stride = 2 * c.layers;
  for (uint32_t v = 0; v < variants; ++v) {
    placed[v] = place_table(c, edit_tables ? edit_tables + (size_t)v * table_words : nullptr,
                            edit_tables ? table_words : 0, origin);
    if (int rc = check_table(c, placed[v], "frz_generate_variants")) return rc;
    stride = std::max<uint32_t>(stride, (uint32_t)placed[v].size());
  }
  // The shared prefix through the model's own caches, reusing what they hold.
  const std::vector<uint32_t> none = place_table(c, nullptr, 0, origin);
  if (int rc = frz_model_set_edits(m, none.data(), (uint32_t)none.size())) return rc;
  uint32_t common = 0;
  while (common < m->cached.size() && common < origin && m->cached[common] == prompt[common])
    ++common;
  common = std::min(common, first_edit_difference(c, m->cached_edits, none));
  if (m->written_end > (uint64_t)common + c.local_slots - c.window) common = 0;
  m->reused = common;
  // As in frz_generate: the record forgotten while the caches are rewritten,
  // the high-water mark kept. The variants decode in caches of their own, so
  // the model's own caches receive positions up to the prompt's last but one.
  forget_prefix(m);
  m->written_end = common == 0 ? origin : std::max<uint64_t>(m->written_end, origin);
  for (uint32_t pos = common; pos < origin;) {
    const uint32_t n = std::min<uint32_t>(kPrefillBlock, origin - pos);
    if (int rc = model_step(m, pos, n, prompt + pos, 0, sampling)) return rc;
    pos += n;
  }
  m->cached.assign(prompt, prompt + origin);
  m->cached_edits = none;
  if (int rc = ensure_variants(m, (int)variants, max_tokens, stride, residuals_out != nullptr))
    return rc;
  frz_model::Variants& V = m->variants;
  V.capture = residuals_out != nullptr;
  hipStream_t s = m->dev->stream;
  // Every variant's caches start as the prefix's.
  const size_t kvw = (size_t)c.kv_heads * c.head_dim;
  for (int l = 0; l < c.layers; ++l) {
    const Layer& L = m->layers[l];
    const size_t bytes = (size_t)L.slots * kvw * 2, elems = (size_t)L.slots * kvw;
    for (uint32_t v = 0; v < variants; ++v) {
      if (int rc = check_hip(hipMemcpyAsync(V.kcache[l] + v * elems, L.kcache, bytes,
                                            hipMemcpyDeviceToDevice, s),
                             "variant keys"))
        return rc;
      if (int rc = check_hip(hipMemcpyAsync(V.vcache[l] + v * elems, L.vcache, bytes,
                                            hipMemcpyDeviceToDevice, s),
                             "variant values"))
        return rc;
    }
  }
  std::vector<uint32_t> tables((size_t)variants * V.edit_stride, 0);
  for (uint32_t v = 0; v < variants; ++v)
    std::copy(placed[v].begin(), placed[v].end(), tables.begin() + (size_t)v * V.edit_stride);
  if (int rc = check_hip(hipMemcpyAsync(V.edits, tables.data(), tables.size() * 4,
                                        hipMemcpyHostToDevice, s),
                         "variant tables"))
    return rc;
  // Step 0: every variant's row of the prompt's last token; its draw is each
  // variant's first token. The selection advances the step, so each later
  // step feeds every row its own draw.
  DevStep& st = *m->step_host;
  std::memset(&st, 0, sizeof st);
  st.position = origin;
  st.tokens = variants;
  st.logits = 1;
  st.variants = 1;
  fill_sampling(st, sampling);
  for (uint32_t v = 0; v < variants; ++v) st.ids[v] = prompt[origin];
  if (int rc = put_step(m)) return rc;
  for (uint32_t t = 0; t < max_tokens; ++t) {
    V.position = origin + t;
    if (int rc = enqueue_rows(m, (int)variants, true, &V)) return rc;
  }
  std::vector<uint32_t> log((size_t)max_tokens * variants * 2);
  if (int rc = check_hip(hipMemcpyAsync(log.data(), V.token_log, log.size() * 4,
                                        hipMemcpyDeviceToHost, s),
                         "variant tokens"))
    return rc;
  if (residuals_out) {
    const size_t n = (size_t)max_tokens * c.layers * variants * c.hidden;
    if (int rc = check_hip(hipMemcpyAsync(residuals_out, V.residuals, n * 4,
                                          hipMemcpyDeviceToHost, s),
                           "variant residuals"))
      return rc;
  }
  if (int rc = check_hip(hipStreamSynchronize(s), "variants sync")) return rc;
  // Each variant's reply as frz_generate ends one: at a failed draw or a
  // stop token, which it keeps.
  for (uint32_t v = 0; v < variants; ++v) {
    uint32_t n = 0;
    for (uint32_t t = 0; t < max_tokens; ++t) {
      const uint32_t token = log[2 * ((size_t)t * variants + v)];
      const uint32_t failed = log[2 * ((size_t)t * variants + v) + 1];
      tokens_out[(size_t)v * max_tokens + n++] = token;
      if (failed || std::find(stop_ids, stop_ids + stops, token) != stop_ids + stops) break;
    }
    drawn_out[v] = n;
  }
  return FRZ_OK;
}

}  // extern "C"
