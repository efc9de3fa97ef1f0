// Internal declarations shared by the C ABI's translation units.
#pragma once

#include <hip/hip_runtime.h>

#include <string>

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

}  // namespace frz
