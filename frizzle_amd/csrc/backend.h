// Internal declarations shared by the C ABI's translation units.
#pragma once

#include <hip/hip_runtime.h>

#include <string>
#include <vector>

#include "../../include/frizzle_hip.h"
#include "kernels.h"

struct frz_device {
  int ordinal = 0;
  hipDeviceProp_t props{};
  hipStream_t stream = nullptr;
  frz::DevStep* step = nullptr;  // the one-kernel ops' step record
  // This device's copy of the static decode-attention workspace (the
  // address hipGetSymbolAddress gave at frz_open, with this device current).
  float* static_workspace = nullptr;
};

namespace frz {

// Sets the calling thread's message and returns `status`.
int fail(int status, const std::string& message);
// FRZ_OK, or FRZ_ERR_DEVICE with the HIP error's text.
int check_hip(hipError_t e, const char* what);
// Copies a step record to the device and waits.
int device_put_step(frz_device* dev, const DevStep& s);
// Reports a launch's error, else waits for the stream.
int device_finish(frz_device* dev, hipError_t launched, const char* what);
// The sampling settings into a step record (sampler::apply,
// src/core/sampler/sampler.cpp:51-62).
void fill_sampling(DevStep& s, const frz_sampling* sampling);
// The most chunks a row reaches for a window over a cache of `slots`.
int attention_max_chunks(int window, int slots);

// A profiled step (frz_model_profile_step, frz_program_run_profiled): an
// event recorded on the stream before each launch, with the roles the
// launch runs (the graph's names, graph.h:99-106, "+" between the roles a
// fused launch runs) and its layer, and one more after the last.
struct StepProfile {
  std::vector<hipEvent_t> events;
  std::vector<const char*> roles;  // null for the closing event
  std::vector<uint32_t> layers;
  size_t used = 0;
  bool failed = false;  // an event could not be made or recorded: the times are not reported
  void start() {
    used = 0;
    failed = false;
  }
  StepProfile() = default;
  StepProfile(const StepProfile&) = delete;
  StepProfile& operator=(const StepProfile&) = delete;
  ~StepProfile() {
    for (hipEvent_t e : events) (void)hipEventDestroy(e);
  }
};
// Each launch's time, from the event before it to the one after it, with its
// names; `count` is the launches the step made (at most `cap` are written).
// The step's events must have completed.
int read_profile(const StepProfile& p, frz_launch_time* out, uint32_t cap, uint32_t* count);

}  // namespace frz
