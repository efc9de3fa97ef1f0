// The program: a Gemma 3 graph's launches (kernels::Launch, interface.h:
// 320-363, as graph::Builder emits them, graph.cpp:290-470) built into this
// backend's fused schedule, and its steps run at most two deep and reported
// in the order they were run (program.h:264-402, order.h:68-104).
//
// Build checks each launch as Program::build does (program.h:29-41), then
// recognises the graph: its stages in the graph's order, each named by the
// role and layer graph.h gives it and of the kernel the role needs, and each
// bound to the plan's ranges that role reads (a layer's weights, gains and
// caches, the working buffers the draw uses). The launches are descriptions:
// what runs is the model's fused schedule, which computes the same graph.
// Run writes the step record and inputs in stream order, enqueues the step
// (a fed decode step replays the model's decode graph) and records an
// event; poll reports settled steps in run order on the caller's thread.

#include <algorithm>
#include <cstddef>
#include <cstring>
#include <type_traits>
#include <string>
#include <vector>

#include "../../include/frizzle_hip.h"
#include "backend.h"
#include "kernels.h"

namespace frz {
int program_step(frz_model* m, const DevStep* pinned_step, uint32_t* readback,
                 StepProfile* profile = nullptr);
hipStream_t model_stream(const frz_model* m);
}  // namespace frz

using namespace frz;

namespace {

constexpr uint32_t kMaxLaunchConstants = 768;  // interface.h: kMaxLaunchConstants
constexpr uint64_t kMaxReadback = 16;          // program.h: kMaxReadback
constexpr uint64_t kMaxPositions = 1ull << 24; // interface.h: kMaxPositions
constexpr int kOutstanding = 2;                // order.h: kOutstanding

// A stage the graph holds: its role and layer (graph.h's names), the
// kernels its launches may be, the plan ranges its launches must bind.
struct Stage {
  std::string role;
  uint32_t layer;
  std::vector<int> kernels;
  std::vector<frz_range> binds;
  bool optional;
};

std::string layer_text(uint32_t layer) {
  return layer == FRZ_NO_LAYER ? std::string() : " of layer " + std::to_string(layer);
}

// A tensor's whole range (its one piece, or its pieces' first to last).
bool tensor_range(const frz_plan* plan, int layer, int role, std::vector<frz_range>& out,
                  std::string& why) {
  uint64_t t = 0;
  uint32_t n = 0;
  if (frz_plan_role(plan, layer, role, &t) != FRZ_OK ||
      frz_plan_tensor(plan, t, 0, nullptr, &n) != FRZ_OK || n == 0) {
    why = "the plan has no tensor for role " + std::to_string(role) + layer_text((uint32_t)layer);
    return false;
  }
  for (uint32_t i = 0; i < n; ++i) {
    frz_piece p;
    (void)frz_plan_tensor(plan, t, i, &p, nullptr);
    out.push_back(p.range);
  }
  return true;
}

// A layer's group span for (Q, K, V) or (gate, up).
bool group_range(const frz_plan* plan, int layer, const int* roles, uint32_t count,
                 frz_range& out, std::string& why) {
  uint64_t want[3] = {0, 0, 0};
  for (uint32_t i = 0; i < count; ++i) {
    if (frz_plan_role(plan, layer, roles[i], &want[i]) != FRZ_OK) {
      why = "the plan has no tensor for role " + std::to_string(roles[i]) +
            layer_text((uint32_t)layer);
      return false;
    }
  }
  frz_plan_summary s;
  (void)frz_plan_summarize(plan, &s);
  for (uint32_t g = 0; g < s.groups; ++g) {
    uint64_t members[3];
    uint32_t n = 0;
    frz_range span;
    (void)frz_plan_group(plan, g, members, &n, &span);
    if (n == count && std::equal(members, members + n, want)) {
      out = span;
      return true;
    }
  }
  why = std::string("the plan did not group ") + (count == 3 ? "Q, K and V" : "gate and up") +
        layer_text((uint32_t)layer) + " (graph.cpp: Ungrouped" +
        (count == 3 ? "QueryKeyValue)" : "FeedForward)");
  return false;
}

bool scratch_range(const frz_plan* plan, const char* purpose, frz_range& out, std::string& why) {
  if (frz_plan_scratch(plan, purpose, &out) != FRZ_OK) {
    why = std::string("the plan has no working buffer ") + purpose;
    return false;
  }
  return true;
}

// The stages of the Gemma 3 graph over `plan`, in order.
bool gemma3_stages(const frz_plan* plan, std::vector<Stage>& out, std::string& why) {
  frz_model_config c;
  if (frz_plan_config(plan, &c) != FRZ_OK) {
    why = "no plan";
    return false;
  }
  std::vector<frz_range> r;
  auto tensors = [&](std::initializer_list<std::pair<int, int>> roles) {
    std::vector<frz_range> v;
    for (auto [layer, role] : roles) {
      if (!tensor_range(plan, layer, role, v, why)) return std::vector<frz_range>{};
    }
    return v;
  };
  frz_range edit, logits, candidates, sampled;
  if (!scratch_range(plan, "edit_table", edit, why) || !scratch_range(plan, "logits", logits, why) ||
      !scratch_range(plan, "candidates", candidates, why) ||
      !scratch_range(plan, "sampled", sampled, why))
    return false;
  const std::vector<frz_range> embedding = tensors({{-1, FRZ_ROLE_EMBEDDING}});
  const std::vector<frz_range> output_norm = tensors({{-1, FRZ_ROLE_OUTPUT_NORM}});
  if (embedding.empty() || output_norm.empty()) return false;
  out.push_back({"embed", FRZ_NO_LAYER, {FRZ_KERNEL_GATHER}, embedding, false});
  for (int l = 0; l < c.layers; ++l) {
    const uint32_t L = (uint32_t)l;
    std::vector<frz_range> norm = tensors({{l, FRZ_ROLE_ATTN_NORM}});
    if (norm.empty()) return false;
    if (l > 0) {
      const std::vector<frz_range> pending = tensors({{l - 1, FRZ_ROLE_POST_FFN_NORM}});
      if (pending.empty()) return false;
      norm.insert(norm.end(), pending.begin(), pending.end());
    }
    out.push_back({"attention.norm", L, {FRZ_KERNEL_NORM}, norm, false});
    const int qkv_roles[3] = {FRZ_ROLE_Q, FRZ_ROLE_K, FRZ_ROLE_V};
    frz_range qkv, gate_up;
    if (!group_range(plan, l, qkv_roles, 3, qkv, why)) return false;
    out.push_back({"attention.qkv", L, {FRZ_KERNEL_MATMUL}, {qkv}, false});
    if (l > 0) {
      out.push_back({"readout", L - 1,
                     {FRZ_KERNEL_NORM, FRZ_KERNEL_MATMUL, FRZ_KERNEL_TOPK, FRZ_KERNEL_CAPTURE},
                     output_norm, false});
    }
    frz_range keys, values;
    uint32_t slots = 0;
    if (frz_plan_cache(plan, L, &keys, &values, &slots) != FRZ_OK) {
      why = "the plan has no cache" + layer_text(L);
      return false;
    }
    std::vector<frz_range> rope = tensors({{l, FRZ_ROLE_Q_NORM}, {l, FRZ_ROLE_K_NORM}});
    if (rope.empty()) return false;
    rope.push_back(keys);
    rope.push_back(values);
    out.push_back({"attention.rope", L, {FRZ_KERNEL_ROPE}, rope, false});
    out.push_back({"attention.capture", L, {FRZ_KERNEL_CAPTURE}, {}, false});
    out.push_back({"attention.scores", L, {FRZ_KERNEL_ATTENTION}, {keys, values}, false});
    out.push_back({"attention.combine", L, {FRZ_KERNEL_ATTENTION_COMBINE}, {}, true});
    out.push_back({"attention.weights", L, {FRZ_KERNEL_CAPTURE_WEIGHTS}, {}, false});
    const std::vector<frz_range> o = tensors({{l, FRZ_ROLE_O}});
    if (o.empty()) return false;
    out.push_back({"attention.output", L, {FRZ_KERNEL_MATMUL}, o, false});
    const std::vector<frz_range> fnorm =
        tensors({{l, FRZ_ROLE_FFN_NORM}, {l, FRZ_ROLE_POST_ATTN_NORM}});
    if (fnorm.empty()) return false;
    out.push_back({"ffn.norm", L, {FRZ_KERNEL_NORM}, fnorm, false});
    const int gu_roles[2] = {FRZ_ROLE_GATE, FRZ_ROLE_UP};
    if (!group_range(plan, l, gu_roles, 2, gate_up, why)) return false;
    out.push_back({"ffn.gate_up", L, {FRZ_KERNEL_MATMUL}, {gate_up}, false});
    out.push_back({"ffn.edit", L, {FRZ_KERNEL_EDIT}, {edit}, false});
    out.push_back({"ffn.capture", L, {FRZ_KERNEL_CAPTURE}, {}, false});
    const std::vector<frz_range> down = tensors({{l, FRZ_ROLE_DOWN}});
    if (down.empty()) return false;
    out.push_back({"ffn.down", L, {FRZ_KERNEL_MATMUL}, down, false});
  }
  std::vector<frz_range> onorm = output_norm;
  const std::vector<frz_range> last = tensors({{c.layers - 1, FRZ_ROLE_POST_FFN_NORM}});
  if (last.empty()) return false;
  onorm.insert(onorm.end(), last.begin(), last.end());
  out.push_back({"output.norm", FRZ_NO_LAYER, {FRZ_KERNEL_NORM}, onorm, false});
  out.push_back({"output.head", FRZ_NO_LAYER, {FRZ_KERNEL_MATMUL}, embedding, false});
  out.push_back({"output.select", FRZ_NO_LAYER, {FRZ_KERNEL_TOPK}, {logits}, false});
  out.push_back({"output.readout", FRZ_NO_LAYER, {FRZ_KERNEL_CAPTURE}, {}, false});
  out.push_back({"output.draw", FRZ_NO_LAYER, {FRZ_KERNEL_DRAW}, {candidates, sampled}, false});
  return true;
}

bool covers(const frz_binding& b, const frz_range& r) {
  return b.buffer == r.buffer && b.offset <= r.offset && r.offset + r.length <= b.offset + b.size;
}

std::string role_of(const frz_launch& l) { return l.role ? std::string(l.role) : std::string(); }

// Program::build's checks of one launch (program.h:29-41), given the plan's
// buffers.
bool launch_ok(const frz_launch& l, uint32_t i, const std::vector<uint64_t>& sizes,
               std::string& why) {
  const std::string at = "launch " + std::to_string(i);
  if (l.constants_bytes > kMaxLaunchConstants) {
    why = at + ": constants over 768 bytes";
    return false;
  }
  if (l.constants_bytes > 0 && !l.constants) {
    why = at + ": constants missing";
    return false;
  }
  if (l.workgroup_size == 0 || l.invocations_per_row == 0) {
    why = at + ": no invocations";
    return false;
  }
  if (l.rows_per_tile != 0 && l.rows == FRZ_ROWS_LAST_TOKEN) {
    why = at + ": a tiled launch over the last token";
    return false;
  }
  if (l.rows_per_tile != 0 &&
      ((uint64_t)l.rows_per_tile * l.invocations_per_row) % l.workgroup_size != 0) {
    why = at + ": a tile that is not a whole number of workgroups";
    return false;
  }
  if (l.key_split != FRZ_KEY_SPLIT_NONE && l.window == 0) {
    why = at + ": a key split with no window";
    return false;
  }
  if (l.rows < FRZ_ROWS_EVERY_TOKEN || l.rows > FRZ_ROWS_PROMPT_END || l.key_split < 0 ||
      l.key_split > FRZ_KEY_SPLIT_WHEN_SPLIT || l.kernel < FRZ_KERNEL_GATHER ||
      l.kernel > FRZ_KERNEL_CAPTURE_WEIGHTS) {
    why = at + ": an unknown kernel, rows or key split";
    return false;
  }
  if (l.binding_count > 0 && !l.bindings) {
    why = at + ": bindings missing";
    return false;
  }
  if (l.override_count > 0 && !l.overrides) {
    why = at + ": overrides missing";
    return false;
  }
  for (uint32_t o = 0; o < l.override_count; ++o) {
    const char* name = l.overrides[o].name;
    if (!name) {
      why = at + ": override " + std::to_string(o) + " has no name";
      return false;
    }
    bool twice = false;
    for (uint32_t e = 0; e < o && !twice; ++e)
      twice = l.overrides[e].name && std::strcmp(l.overrides[e].name, name) == 0;
    if (twice || std::strcmp(name, "workgroup_size") == 0 || std::strcmp(name, "last_token") == 0) {
      why = at + ": override " + name + (twice ? " given twice" : " is the program's to set");
      return false;
    }
  }
  for (uint32_t b = 0; b < l.binding_count; ++b) {
    const frz_binding& x = l.bindings[b];
    if (x.buffer >= sizes.size() || x.offset > sizes[x.buffer] ||
        x.size > sizes[x.buffer] - x.offset) {
      why = at + ": binding " + std::to_string(b) + " is not within a buffer the upload created";
      return false;
    }
  }
  return true;
}

int check(const frz_plan* plan, const frz_launch* launches, uint32_t count,
          const frz_binding* readback, std::string& why) {
  if (!plan || (count > 0 && !launches)) {
    why = "null plan or launches";
    return FRZ_ERR_BUILD;
  }
  frz_plan_summary s;
  if (frz_plan_summarize(plan, &s) != FRZ_OK) {
    why = "no plan";
    return FRZ_ERR_BUILD;
  }
  std::vector<uint64_t> sizes(s.buffers);
  for (uint32_t i = 0; i < s.buffers; ++i) (void)frz_plan_buffer(plan, i, nullptr, &sizes[i]);
  for (uint32_t i = 0; i < count; ++i) {
    if (!launch_ok(launches[i], i, sizes, why)) return FRZ_ERR_BUILD;
  }
  // The readback range: a buffer the upload created, whole words, 4 to 16
  // bytes; for Gemma 3's graph, the draw's record.
  frz_range sampled;
  if (!readback) {
    why = "no readback range (the draw's record)";
    return FRZ_ERR_BUILD;
  }
  if (readback->buffer >= sizes.size() || readback->offset > sizes[readback->buffer] ||
      readback->size > sizes[readback->buffer] - readback->offset || readback->size < 4 ||
      readback->size > kMaxReadback || readback->size % 4 != 0 || readback->offset % 4 != 0) {
    why = "the readback range is not 4 to 16 bytes of whole words within a buffer";
    return FRZ_ERR_BUILD;
  }
  std::vector<Stage> stages;
  if (!gemma3_stages(plan, stages, why)) return FRZ_ERR_BUILD;
  if (!scratch_range(plan, "sampled", sampled, why)) return FRZ_ERR_BUILD;
  if (readback->buffer != sampled.buffer || readback->offset != sampled.offset ||
      readback->size != 16) {
    why = "the readback range is not the draw's 16-byte record (\"sampled\")";
    return FRZ_ERR_BUILD;
  }
  // Walk the stages: each a run of launches of its role and layer.
  uint32_t i = 0;
  for (const Stage& st : stages) {
    const uint32_t first = i;
    while (i < count && role_of(launches[i]) == st.role && launches[i].layer == st.layer) {
      const frz_launch& l = launches[i];
      if (std::find(st.kernels.begin(), st.kernels.end(), l.kernel) == st.kernels.end()) {
        why = "launch " + std::to_string(i) + " (" + st.role + layer_text(st.layer) +
              "): kernel " + std::to_string(l.kernel) + " is not one this stage runs";
        return FRZ_ERR_BUILD;
      }
      ++i;
    }
    if (i == first) {
      if (st.optional) continue;
      why = "launch " + std::to_string(i) + ": expected " + st.role + layer_text(st.layer) +
            ", found " +
            (i < count ? (role_of(launches[i]).empty() ? std::string("an unnamed launch")
                                                        : role_of(launches[i])) +
                             layer_text(launches[i].layer)
                       : std::string("the end of the launches"));
      return FRZ_ERR_BUILD;
    }
    // Every launch of the stage's first kernel (the one that reads its
    // weights, gains and caches: each form of a product binds them) binds
    // each range the role reads.
    const int reader = st.kernels.front();
    for (const frz_range& r : st.binds) {
      uint32_t readers = 0;
      for (uint32_t k = first; k < i; ++k) {
        if (launches[k].kernel != reader) continue;
        ++readers;
        bool found = false;
        for (uint32_t b = 0; b < launches[k].binding_count && !found; ++b)
          found = covers(launches[k].bindings[b], r);
        if (!found) {
          why = "launch " + std::to_string(k) + " (" + st.role + layer_text(st.layer) +
                "): binds none of buffer " + std::to_string(r.buffer) + " bytes " +
                std::to_string(r.offset) + ".." + std::to_string(r.offset + r.length) +
                ", which this role reads in the plan";
          return FRZ_ERR_BUILD;
        }
      }
      if (readers == 0) {
        why = "launch " + std::to_string(first) + " (" + st.role + layer_text(st.layer) +
              "): no launch of kernel " + std::to_string(reader) + " reads its ranges";
        return FRZ_ERR_BUILD;
      }
    }
  }
  if (i != count) {
    why = "launch " + std::to_string(i) + " (" + role_of(launches[i]) + layer_text(launches[i].layer) +
          "): after the graph's last stage";
    return FRZ_ERR_BUILD;
  }
  return FRZ_OK;
}

void put_message(const std::string& m, char* buf, size_t cap) {
  if (!buf || cap == 0) return;
  const size_t n = std::min(m.size(), cap - 1);
  std::memcpy(buf, m.data(), n);
  buf[n] = '\0';
}

// A HIP error that leaves the device unusable, as opposed to a refused call.
bool is_loss(hipError_t e) {
  return e == hipErrorIllegalAddress || e == hipErrorLaunchFailure ||
         e == hipErrorECCNotCorrectable || e == hipErrorNoDevice ||
         e == hipErrorLaunchTimeOut || e == hipErrorAssert || e == hipErrorUnknown;
}

}  // namespace

struct frz_program {
  frz_model* model = nullptr;
  hipStream_t stream = nullptr;
  uint32_t context = 0;
  std::vector<uint8_t*> buffers;   // the upload's buffers, by the plan's index
  std::vector<uint64_t> sizes;
  DevStep* step[kOutstanding] = {};     // pinned step records, slot n mod 2
  uint32_t* readback[kOutstanding] = {};  // pinned 16-byte records
  uint8_t* staging[kOutstanding] = {};  // pinned input bytes
  size_t staging_bytes[kOutstanding] = {};
  hipEvent_t done_event[kOutstanding] = {};
  // The graph's launches' names (role, layer), for a profiled step's report.
  std::vector<std::pair<std::string, uint32_t>> names;
  StepProfile profiles[kOutstanding];  // a profiled step's events, by slot
  struct Slot {
    frz_step_callback done = nullptr;
    frz_profile_callback profiled = nullptr;  // a profiled step's callback
    void* userdata = nullptr;
    int status = FRZ_OK;      // a failure found before it ran
    std::string message;
    bool ran = false;         // work was enqueued (its event recorded)
    bool logits = false;
  } slot[kOutstanding];
  uint64_t next_run = 0, next_report = 0;  // order.h: run order, report order
  bool lost = false;
};

namespace {

uint32_t outstanding(const frz_program* p) { return (uint32_t)(p->next_run - p->next_report); }

// The index in the graph of the last of its launches that a launch of this
// backend runs: one of the launch's roles ("+" between them) in its layer.
uint32_t graph_index_of(const std::vector<std::pair<std::string, uint32_t>>& names,
                        const char* roles, uint32_t layer) {
  uint32_t found = ~0u;
  std::string all(roles ? roles : "");
  for (size_t at = 0; at <= all.size();) {
    size_t end = all.find('+', at);
    if (end == std::string::npos) end = all.size();
    const std::string one = all.substr(at, end - at);
    for (uint32_t i = 0; i < names.size(); ++i) {
      if (names[i].second == layer && names[i].first == one && (found == ~0u || i > found))
        found = i;
    }
    at = end + 1;
  }
  return found;
}

// Reports the oldest outstanding step (its work, if any, waited for when
// `wait`); false when it has not settled.
bool report_oldest(frz_program* p, bool wait, bool cancelled) {
  frz_program::Slot& s = p->slot[p->next_report % kOutstanding];
  const int k = (int)(p->next_report % kOutstanding);
  int status = s.status;
  std::string message = s.message;
  if (s.ran) {
    const hipError_t e = wait ? hipEventSynchronize(p->done_event[k]) : hipEventQuery(p->done_event[k]);
    if (e == hipErrorNotReady) return false;
    if (e != hipSuccess) {
      status = FRZ_ERR_STEP;
      message = std::string("the step failed on the device: ") + hipGetErrorString(e);
      if (is_loss(e)) p->lost = true;
    }
  }
  if (cancelled) {
    status = FRZ_ERR_CANCELLED;
    message = "cancelled";
  } else if (p->lost) {
    status = FRZ_ERR_DEVICE_LOST;
    message = "the device is lost";
  }
  uint32_t record[4] = {0, 0, 0, 0};
  const bool with = status == FRZ_OK && s.logits;
  if (with) std::memcpy(record, p->readback[k], 16);
  const frz_step_callback done = s.done;
  const frz_profile_callback profiled = s.profiled;
  void* ud = s.userdata;
  // A profiled step's times: each launch's from its events, its end as the
  // sum of those before it, and the graph's last launch it runs.
  std::vector<frz_launch_time> launches;
  std::vector<uint32_t> index;
  std::vector<uint64_t> end_ns;
  frz_profile_times times{};
  if (profiled && status == FRZ_OK) {
    // A profile that cannot be read fails the report (the step's own work
    // is done; its times are not known).
    uint32_t n = 0;
    int rc = read_profile(p->profiles[k], nullptr, 0, &n);
    if (rc == FRZ_OK) {
      launches.resize(n);
      rc = read_profile(p->profiles[k], launches.data(), n, &n);
    }
    if (rc != FRZ_OK) {
      launches.clear();
      status = rc;
      message = frz_last_error();
    }
    double at = 0.0;
    for (frz_launch_time& t : launches) {
      t.graph_index = graph_index_of(p->names, t.role, t.layer);
      at += t.microseconds;
      index.push_back(t.graph_index);
      end_ns.push_back((uint64_t)(at * 1000.0 + 0.5));
    }
    times.end_ns = end_ns.empty() ? 0 : end_ns.back();
    times.launch_index = index.data();
    times.launch_end_ns = end_ns.data();
    times.launches = launches.data();
    times.launch_count = (uint32_t)launches.size();
  }
  s = frz_program::Slot{};
  ++p->next_report;  // reported before the callback, which may run the next step
  if (profiled) {
    profiled(status, message.c_str(), with ? record : nullptr, with ? 16u : 0u, &times, ud);
  } else if (done) {
    done(status, message.c_str(), with ? record : nullptr, with ? 16u : 0u, ud);
  }
  return true;
}

}  // namespace

extern "C" {

int frz_program_check(const frz_plan* plan, const frz_launch* launches, uint32_t count,
                      const frz_binding* readback, char* message, size_t message_cap) {
  std::string why;
  const int rc = check(plan, launches, count, readback, why);
  put_message(why, message, message_cap);
  if (rc != FRZ_OK) return fail(rc, "frz_program_build: " + why);
  return FRZ_OK;
}

int frz_program_build(frz_model* upload, const frz_plan* plan, const frz_launch* launches,
                      uint32_t count, const frz_binding* readback, frz_program** out,
                      char* message, size_t message_cap) {
  put_message("", message, message_cap);
  if (!upload || !plan || !out) {
    put_message("null argument", message, message_cap);
    return fail(FRZ_ERR_BUILD, "frz_program_build: null argument");
  }
  *out = nullptr;
  if (int rc = frz_program_check(plan, launches, count, readback, message, message_cap)) return rc;
  frz_plan_summary s;
  (void)frz_plan_summarize(plan, &s);
  frz_model_config c;
  (void)frz_model_get_config(upload, &c);
  frz_model_config pc;
  (void)frz_plan_config(plan, &pc);
  auto* p = new frz_program();
  for (uint32_t i = 0; i < count; ++i)
    p->names.emplace_back(launches[i].role ? launches[i].role : "", launches[i].layer);
  p->model = upload;
  p->stream = model_stream(upload);
  p->context = (uint32_t)c.context;
  std::string why;
  for (uint32_t i = 0; i < s.buffers && why.empty(); ++i) {
    void* ptr = nullptr;
    uint64_t size = 0, planned = 0;
    (void)frz_plan_buffer(plan, i, nullptr, &planned);
    if (frz_model_planned_buffer(upload, i, &ptr, &size) != FRZ_OK || size != planned) {
      why = "the model was not created from this plan (buffer " + std::to_string(i) + ")";
    }
    p->buffers.push_back(static_cast<uint8_t*>(ptr));
    p->sizes.push_back(size);
  }
  if (why.empty() && (c.layers != pc.layers || c.context != pc.context))
    why = "the model was not created from this plan";
  for (int k = 0; k < kOutstanding && why.empty(); ++k) {
    if (hipHostMalloc((void**)&p->step[k], sizeof(DevStep)) != hipSuccess ||
        hipHostMalloc((void**)&p->readback[k], 16) != hipSuccess ||
        hipEventCreateWithFlags(&p->done_event[k], hipEventDisableTiming) != hipSuccess)
      why = "pinned step records or events could not be made";
  }
  // The graph's capture launches write the store at each prompt's end.
  if (why.empty() && frz_model_set_capture(upload, 1) != FRZ_OK) why = frz_last_error();
  if (!why.empty()) {
    frz_program_destroy(p);
    put_message(why, message, message_cap);
    return fail(FRZ_ERR_BUILD, "frz_program_build: " + why);
  }
  *out = p;
  return FRZ_OK;
}

// The step record's 64-byte head (interface.h:163-188) is copied whole into
// DevStep's first 64 bytes: the fields must lie alike, with the ids at 64.
#define FRZ_SAME_FIELD(f)                                                        \
  static_assert(offsetof(DevStep, f) == offsetof(frz_step_record, f) &&         \
                    sizeof(DevStep::f) == sizeof(frz_step_record::f),            \
                "DevStep and frz_step_record differ at " #f)
FRZ_SAME_FIELD(position);
FRZ_SAME_FIELD(tokens);
FRZ_SAME_FIELD(logits);
FRZ_SAME_FIELD(fed);
FRZ_SAME_FIELD(seed);
FRZ_SAME_FIELD(top_k);
FRZ_SAME_FIELD(temperature);
FRZ_SAME_FIELD(top_p);
FRZ_SAME_FIELD(min_p);
FRZ_SAME_FIELD(log_min_p);
FRZ_SAME_FIELD(ids);
#undef FRZ_SAME_FIELD
static_assert(offsetof(DevStep, log_min_p) == 40 && offsetof(DevStep, ids) == 64,
              "the step head is 64 bytes, log_min_p its eleventh word");
static_assert(std::is_same<decltype(DevStep::temperature), decltype(frz_step_record::temperature)>::value &&
                  std::is_same<decltype(DevStep::log_min_p), decltype(frz_step_record::log_min_p)>::value &&
                  std::is_same<decltype(DevStep::top_k), decltype(frz_step_record::top_k)>::value,
              "the step head's fields have the record's types");

}  // extern "C"

namespace {

// frz_program_run and frz_program_run_profiled (`profiled` not null, with
// `launches` the count asked for).
int run_step(frz_program* p, const frz_step_record* step, const frz_run_input* inputs,
             uint32_t input_count, frz_step_callback done, frz_profile_callback profiled,
             uint32_t launches, void* userdata) {
  const char* name = profiled ? "frz_program_run_profiled: " : "frz_program_run: ";
  if (!p || !step) return fail(FRZ_ERR_ARGUMENT, std::string(name) + "null argument");
  // Refused at once, unrun and unnumbered.
  auto refuse = [&](int status, const std::string& why) {
    if (profiled) {
      const frz_profile_times none{};
      profiled(status, why.c_str(), nullptr, 0, &none, userdata);
    } else if (done) {
      done(status, why.c_str(), nullptr, 0, userdata);
    }
    return fail(status, name + why);
  };
  if (p->lost) return refuse(FRZ_ERR_DEVICE_LOST, "the device is lost");
  if (outstanding(p) >= (uint32_t)kOutstanding) return refuse(FRZ_ERR_STEP, "two steps are outstanding");
  if (profiled) {
    if (launches != (uint32_t)p->names.size())
      return refuse(FRZ_ERR_STEP, "a prefix of " + std::to_string(launches) + " of the graph's " +
                                      std::to_string(p->names.size()) +
                                      " launches (this backend's launches each run several of "
                                      "the graph's, so it runs whole steps)");
    for (uint64_t n = p->next_report; n < p->next_run; ++n) {
      if (!p->slot[n % kOutstanding].profiled)
        return refuse(FRZ_ERR_STEP, "an unprofiled step is outstanding");
    }
  }
  if (step->tokens == 0 || step->tokens > (uint32_t)kPrefillBlock)
    return refuse(FRZ_ERR_STEP, "a step of " + std::to_string(step->tokens) + " tokens");
  const int k = (int)(p->next_run % kOutstanding);
  frz_program::Slot& s = p->slot[k];
  s = frz_program::Slot{};
  s.done = done;
  s.profiled = profiled;
  s.userdata = userdata;
  s.logits = step->logits != 0;
  ++p->next_run;
  // Failed with nothing run, reported in order.
  if ((uint64_t)step->position + step->tokens > kMaxPositions ||
      (uint64_t)step->position + step->tokens > p->context) {
    s.status = FRZ_ERR_STEP;
    s.message = "a step past the context";
    return FRZ_OK;
  }
  if (step->fed && step->tokens != 1) {
    s.status = FRZ_ERR_STEP;
    s.message = "a fed step of " + std::to_string(step->tokens) +
                " tokens (a fed step is one token, the last step's draw)";
    return FRZ_OK;
  }
  size_t input_bytes = 0;
  for (uint32_t i = 0; i < input_count; ++i) {
    const frz_run_input& in = inputs[i];
    if (!in.bytes || in.to.buffer >= p->buffers.size() || in.to.size % 4 != 0 ||
        in.to.offset % 4 != 0 || in.to.offset > p->sizes[in.to.buffer] ||
        in.to.size > p->sizes[in.to.buffer] - in.to.offset) {
      s.status = FRZ_ERR_STEP;
      s.message = "input " + std::to_string(i) + " is outside its buffer or not of whole words";
      return FRZ_OK;
    }
    input_bytes += in.to.size;
  }
  // The step record and the inputs, through pinned memory in stream order.
  DevStep& d = *p->step[k];
  std::memset(&d, 0, sizeof d);
  std::memcpy(&d, step, 64);  // the reference's 64-byte head: the same fields in order
  d.drawn = 0;
  d.variants = 0;
  d.pad[0] = d.pad[1] = d.pad[2] = 0;
  if (!step->fed) std::memcpy(d.ids, step->ids, (size_t)step->tokens * 4);
  hipError_t e = hipSuccess;
  if (input_bytes > p->staging_bytes[k]) {
    if (p->staging[k]) (void)hipHostFree(p->staging[k]);
    p->staging[k] = nullptr;
    p->staging_bytes[k] = 0;
    e = hipHostMalloc((void**)&p->staging[k], input_bytes);
    if (e == hipSuccess) p->staging_bytes[k] = input_bytes;
  }
  size_t at = 0;
  for (uint32_t i = 0; i < input_count && e == hipSuccess; ++i) {
    const frz_run_input& in = inputs[i];
    std::memcpy(p->staging[k] + at, in.bytes, in.to.size);
    e = hipMemcpyAsync(p->buffers[in.to.buffer] + in.to.offset, p->staging[k] + at, in.to.size,
                       hipMemcpyHostToDevice, p->stream);
    at += in.to.size;
  }
  int rc = e == hipSuccess ? program_step(p->model, p->step[k], p->readback[k],
                                          profiled ? &p->profiles[k] : nullptr)
                           : FRZ_ERR_DEVICE;
  if (rc == FRZ_OK) e = hipEventRecord(p->done_event[k], p->stream);
  if (rc != FRZ_OK || e != hipSuccess) {
    const hipError_t last = e != hipSuccess ? e : hipGetLastError();
    if (is_loss(last)) p->lost = true;
    s.status = FRZ_ERR_STEP;
    s.message = std::string("the step could not be enqueued: ") + frz_last_error();
    // Whatever was enqueued finishes before the slot is reused.
    (void)hipStreamSynchronize(p->stream);
    return FRZ_OK;
  }
  s.ran = true;
  return FRZ_OK;
}

}  // namespace

extern "C" {

int frz_program_run(frz_program* p, const frz_step_record* step, const frz_run_input* inputs,
                    uint32_t input_count, frz_step_callback done, void* userdata) {
  return run_step(p, step, inputs, input_count, done, nullptr, 0, userdata);
}

int frz_program_run_profiled(frz_program* p, const frz_step_record* step,
                             const frz_run_input* inputs, uint32_t input_count,
                             uint32_t launches, frz_profile_callback done, void* userdata) {
  if (!done) return fail(FRZ_ERR_ARGUMENT, "frz_program_run_profiled: null callback");
  return run_step(p, step, inputs, input_count, nullptr, done, launches, userdata);
}

uint32_t frz_program_launch_count(const frz_program* p) {
  return p ? (uint32_t)p->names.size() : 0;
}

int frz_program_can_profile(const frz_program* p) { return p ? 1 : 0; }

int frz_poll(frz_program* p, int wait) {
  if (!p) return 0;
  int n = 0;
  bool first = true;
  while (outstanding(p) > 0 && report_oldest(p, wait && first, false)) {
    ++n;
    first = false;
  }
  return n;
}

uint32_t frz_program_outstanding(const frz_program* p) { return p ? outstanding(p) : 0; }

int frz_program_cancel(frz_program* p) {
  if (!p) return fail(FRZ_ERR_ARGUMENT, "frz_program_cancel: null program");
  while (outstanding(p) > 0) report_oldest(p, true, true);
  return FRZ_OK;
}

void frz_program_destroy(frz_program* p) {
  if (!p) return;
  (void)frz_program_cancel(p);
  for (int k = 0; k < kOutstanding; ++k) {
    if (p->step[k]) (void)hipHostFree(p->step[k]);
    if (p->readback[k]) (void)hipHostFree(p->readback[k]);
    if (p->staging[k]) (void)hipHostFree(p->staging[k]);
    if (p->done_event[k]) (void)hipEventDestroy(p->done_event[k]);
  }
  delete p;
}

int frz_program_mark_lost(frz_program* p) {
  if (!p) return fail(FRZ_ERR_ARGUMENT, "frz_program_mark_lost: null program");
  p->lost = true;
  return FRZ_OK;
}

}  // extern "C"
