// The C ABI's device, buffer and one-kernel entry points (include/
// frizzle_hip.h). Each op call fills a device-side step record on the
// device's stream and launches one kernel family there; ops wait for their
// work so their host arguments need not outlive the call.

#include <algorithm>
#include <cmath>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/frizzle_hip.h"
#include "backend.h"
#include "kernels.h"
#include "numerics.h"

namespace frz {

thread_local std::string g_last_error;

int fail(int status, const std::string& message) {
  g_last_error = message;
  return status;
}

int check_hip(hipError_t e, const char* what) {
  if (e == hipSuccess) return FRZ_OK;
  return fail(FRZ_ERR_DEVICE, std::string(what) + ": " + hipGetErrorString(e));
}

namespace {

// The shared numerics run on the device, one value a lane.
__global__ void numerics_kernel(int which, const float* in, float* out, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float x = in[i];
  float r = 0.0f;
  switch (which) {
    case 0: r = exp2f_fixed(x); break;
    case 1: { float s, c; sincos_fixed(x, &s, &c); r = c; break; }
    case 2: { float s, c; sincos_fixed(x, &s, &c); r = s; break; }
    case 3: r = inverse_sqrt(x); break;
    case 4: r = gelu_tanh(x); break;
    case 5: r = exp_nonpositive(x); break;
    case 6: r = bits_to_float((uint32_t)f16_pack_device(x)); break;
    case 7: r = __builtin_sqrtf(x); break;
    case 8: r = in[2 * (i / 2)] / in[2 * (i / 2) + 1]; break;
    default: break;
  }
  out[i] = r;
}

DevStep host_step(uint32_t position, uint32_t tokens) {
  DevStep s;
  std::memset(&s, 0, sizeof s);
  s.position = position;
  s.tokens = tokens;
  s.top_k = 1;
  s.top_p = 1.0f;
  return s;
}

// The floor a launch costs: a kernel that does nothing.
__global__ void empty_kernel() {}

// The floor a product's bytes cost: every uint4 of a buffer read once, 4 in
// flight a thread, xor-folded into one word a workgroup (written so the
// reads stay). kStreamBlocks workgroups fill the chip.
constexpr int kStreamBlocks = 1024;
constexpr int kFloorCopies = 64;
__global__ __launch_bounds__(256) void stream_kernel(const uint4* __restrict__ src, size_t n4,
                                                     uint32_t* __restrict__ sink) {
  __shared__ uint32_t fold[4];
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  uint32_t x = 0;
  for (; i + 3 * stride < n4; i += 4 * stride) {
    const uint4 a = src[i], b = src[i + stride], c = src[i + 2 * stride], d = src[i + 3 * stride];
    x ^= a.x ^ a.y ^ a.z ^ a.w ^ b.x ^ b.y ^ b.z ^ b.w ^ c.x ^ c.y ^ c.z ^ c.w ^ d.x ^ d.y ^ d.z ^ d.w;
  }
  for (; i < n4; i += stride) {
    const uint4 a = src[i];
    x ^= a.x ^ a.y ^ a.z ^ a.w;
  }
  for (int o = 32; o > 0; o >>= 1) x ^= __shfl_xor(x, o);
  if ((threadIdx.x & 63) == 0) fold[threadIdx.x >> 6] = x;
  __syncthreads();
  if (threadIdx.x == 0) sink[blockIdx.x] = fold[0] ^ fold[1] ^ fold[2] ^ fold[3];
}

// The workspace of frz_op_rope_attention_noalloc: one row's chunk states
// (kStaticChunks x 4 heads x 256 outputs, then 4 statistics a chunk and
// head), 931,840 bytes. Every device the library opens holds its own copy
// until the process ends; host code reaches it only through the address
// frz_open takes for each device (frz_device::static_workspace).
constexpr int kStaticChunks = kMaxFoldChunks;
constexpr size_t kStaticPartialFloats = (size_t)kStaticChunks * 4 * 256;
static __device__ __align__(256) float scratch[kStaticPartialFloats + kStaticPartialFloats / 64];

}  // namespace

int device_put_step(frz_device* dev, const DevStep& s) {
  int rc = check_hip(hipMemcpyAsync(dev->step, &s, sizeof s, hipMemcpyHostToDevice, dev->stream),
                     "hipMemcpyAsync(step)");
  if (rc) return rc;
  return check_hip(hipStreamSynchronize(dev->stream), "hipStreamSynchronize");
}

int device_finish(frz_device* dev, hipError_t launched, const char* what) {
  if (launched != hipSuccess) return check_hip(launched, what);
  return check_hip(hipStreamSynchronize(dev->stream), what);
}

int attention_max_chunks(int window, int slots) {
  const int by_window = (window + kChunkKeys - 1) / kChunkKeys + 1;
  const int by_slots = (slots + kChunkKeys - 1) / kChunkKeys + 1;
  return by_window < by_slots ? by_window : by_slots;
}

void fill_sampling(DevStep& s, const frz_sampling* sampling) {
  s.top_k = sampling ? sampling->top_k : 1;
  s.temperature = sampling ? sampling->temperature : 0.0f;
  s.top_p = sampling ? sampling->top_p : 1.0f;
  s.min_p = sampling ? sampling->min_p : 0.0f;
  s.log_min_p = s.min_p > 0.0f ? std::log(s.min_p) : 0.0f;
  const uint64_t seed = sampling ? sampling->seed : 0;
  s.seed[0] = (uint32_t)seed;
  s.seed[1] = (uint32_t)(seed >> 32);
}

}  // namespace frz

using namespace frz;

extern "C" {

const char* frz_last_error(void) { return g_last_error.c_str(); }

int frz_open(int ordinal, frz_device** out, frz_limits* limits) {
  if (!out) return fail(FRZ_ERR_ARGUMENT, "frz_open: null out");
  *out = nullptr;
  int count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess || count == 0) {
    return fail(FRZ_ERR_DEVICE, "frz_open: no HIP device");
  }
  if (ordinal < 0 || ordinal >= count) return fail(FRZ_ERR_ARGUMENT, "frz_open: no such device");
  if (int rc = check_hip(hipSetDevice(ordinal), "hipSetDevice")) return rc;
  hipDeviceProp_t prop;
  if (int rc = check_hip(hipGetDeviceProperties(&prop, ordinal), "hipGetDeviceProperties")) return rc;
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
    return fail(FRZ_ERR_DEVICE, std::string("frz_open: built for gfx950, device is ") +
                                    prop.gcnArchName);
  }
  frz_device* dev = new frz_device();
  dev->ordinal = ordinal;
  dev->props = prop;
  if (int rc = check_hip(hipStreamCreateWithFlags(&dev->stream, hipStreamNonBlocking),
                         "hipStreamCreate")) {
    delete dev;
    return rc;
  }
  if (int rc = check_hip(hipMalloc(&dev->step, sizeof(DevStep)), "hipMalloc(step)")) {
    (void)hipStreamDestroy(dev->stream);
    delete dev;
    return rc;
  }
  // This device's address of the static workspace (each device holds its own
  // copy of the array; the name itself is no device address on the host).
  void* workspace = nullptr;
  if (int rc = check_hip(hipGetSymbolAddress(&workspace, HIP_SYMBOL(scratch)),
                         "hipGetSymbolAddress(scratch)")) {
    (void)hipFree(dev->step);
    (void)hipStreamDestroy(dev->stream);
    delete dev;
    return rc;
  }
  dev->static_workspace = static_cast<float*>(workspace);
  if (limits) {
    std::memset(limits, 0, sizeof *limits);
    std::strncpy(limits->name, prop.gcnArchName, sizeof(limits->name) - 1);
    limits->memory_bytes = prop.totalGlobalMem;
    limits->compute_units = prop.multiProcessorCount;
    limits->lds_bytes_per_block = (int)prop.sharedMemPerBlock;
  }
  *out = dev;
  return FRZ_OK;
}

void frz_close(frz_device* dev) {
  if (!dev) return;
  (void)hipSetDevice(dev->ordinal);
  (void)hipStreamSynchronize(dev->stream);
  (void)hipFree(dev->step);
  (void)hipStreamDestroy(dev->stream);
  delete dev;
}

int frz_sync(frz_device* dev) {
  return check_hip(hipStreamSynchronize(dev->stream), "hipStreamSynchronize");
}

int frz_alloc(frz_device* dev, uint64_t bytes, void** dev_ptr) {
  if (!dev || !dev_ptr) return fail(FRZ_ERR_ARGUMENT, "frz_alloc: null argument");
  (void)hipSetDevice(dev->ordinal);
  return check_hip(hipMalloc(dev_ptr, bytes ? bytes : 1), "hipMalloc");
}

int frz_free(frz_device* dev, void* dev_ptr) {
  if (!dev) return fail(FRZ_ERR_ARGUMENT, "frz_free: null device");
  return check_hip(hipFree(dev_ptr), "hipFree");
}

int frz_write(frz_device* dev, void* dev_dst, const void* host_src, uint64_t bytes) {
  if (int rc = check_hip(hipMemcpyAsync(dev_dst, host_src, bytes, hipMemcpyHostToDevice,
                                        dev->stream),
                         "hipMemcpyAsync(H2D)"))
    return rc;
  return frz_sync(dev);
}

int frz_read(frz_device* dev, void* host_dst, const void* dev_src, uint64_t bytes) {
  if (int rc = check_hip(hipMemcpyAsync(host_dst, dev_src, bytes, hipMemcpyDeviceToHost,
                                        dev->stream),
                         "hipMemcpyAsync(D2H)"))
    return rc;
  return frz_sync(dev);
}

int frz_fill_zero(frz_device* dev, void* dev_dst, uint64_t bytes) {
  if (int rc = check_hip(hipMemsetAsync(dev_dst, 0, bytes, dev->stream), "hipMemsetAsync"))
    return rc;
  return frz_sync(dev);
}

int frz_q4_0_split(const void* gguf_blocks, uint64_t blocks, void* codes_out,
                   void* scales_out) {
  return frz_block_split(kQ4_0, gguf_blocks, blocks, codes_out, scales_out);
}

int frz_block_split(int format, const void* gguf_blocks, uint64_t blocks, void* codes_out,
                    void* scales_out) {
  if (!gguf_blocks || !codes_out || !scales_out) {
    return fail(FRZ_ERR_ARGUMENT, "frz_block_split: null argument");
  }
  if (format != kQ4_0 && format != kQ4_1 && format != kQ8_0) {
    return fail(FRZ_ERR_ARGUMENT, "frz_block_split: format " + std::to_string(format) +
                                      " (Q4_0 2, Q4_1 3 or Q8_0 8)");
  }
  // A block is its scale halves (d; Q4_1: d, m) then its code bytes.
  const size_t cb = code_bytes(format), sb = 2 * scale_halves(format);
  const size_t bb = gguf_block_bytes(format);
  const uint8_t* in = static_cast<const uint8_t*>(gguf_blocks);
  uint8_t* codes = static_cast<uint8_t*>(codes_out);
  uint8_t* scales = static_cast<uint8_t*>(scales_out);
  for (uint64_t b = 0; b < blocks; ++b) {
    std::memcpy(codes + cb * b, in + bb * b + sb, cb);
    std::memcpy(scales + sb * b, in + bb * b, sb);
  }
  return FRZ_OK;
}

static QMatrix q4(const void* codes, const void* scales, int rows, int cols,
                  int format = kQ4_0) {
  return QMatrix{static_cast<const uint8_t*>(codes), static_cast<const uint16_t*>(scales), rows,
                 cols, format};
}

static bool shape_ok(int rows, int cols) { return rows > 0 && cols > 0 && cols % 32 == 0; }

int frz_op_gemv(frz_device* dev, const void* codes, const void* scales, int rows, int cols,
                const float* x, int x_stride, float* y, int y_stride, uint32_t tokens,
                int last_token) {
  return frz_op_gemv_format(dev, kQ4_0, codes, scales, rows, cols, x, x_stride, y, y_stride,
                            tokens, last_token);
}

int frz_op_gemv_format(frz_device* dev, int format, const void* codes, const void* scales,
                       int rows, int cols, const float* x, int x_stride, float* y, int y_stride,
                       uint32_t tokens, int last_token) {
  if (!shape_ok(rows, cols) || tokens == 0 || tokens > (uint32_t)kPrefillBlock) {
    return fail(FRZ_ERR_ARGUMENT, "frz_op_gemv: bad shape or tokens");
  }
  if (format != kQ4_0 && format != kQ4_1 && format != kQ8_0) {
    return fail(FRZ_ERR_ARGUMENT, "frz_op_gemv: format " + std::to_string(format));
  }
  if (int rc = device_put_step(dev, host_step(0, tokens))) return rc;
  return device_finish(dev,
                       launch_gemv(dev->stream, dev->step, q4(codes, scales, rows, cols, format),
                                   x, x_stride, y, y_stride, (int)tokens, last_token != 0),
                       "frz_op_gemv");
}

int frz_op_gated(frz_device* dev, const void* gate_codes, const void* gate_scales,
                 const void* up_codes, const void* up_scales, int rows, int cols, const float* x,
                 float* act, uint32_t tokens, uint32_t position, const uint32_t* edits_dev,
                 int layer) {
  if (!shape_ok(rows, cols) || tokens == 0 || tokens > (uint32_t)kPrefillBlock) {
    return fail(FRZ_ERR_ARGUMENT, "frz_op_gated: bad shape or tokens");
  }
  if (int rc = device_put_step(dev, host_step(position, tokens))) return rc;
  return device_finish(
      dev,
      launch_gated(dev->stream, dev->step, q4(gate_codes, gate_scales, rows, cols),
                   q4(up_codes, up_scales, rows, cols), x, act, (int)tokens, edits_dev, layer),
      "frz_op_gated");
}

// The fast prefill mode's products through the ABI: the weights unpacked
// into fragment planes, x split into bf16 pair planes, then the product (K
// split as the model splits it).
int frz_op_gemm_bf16(frz_device* dev, int format, const void* codes, const void* scales,
                     int rows, int cols, const float* x, int x_stride, float* y, int y_stride,
                     uint32_t tokens, int splits) {
  if (!shape_ok(rows, cols) || tokens == 0 || tokens > (uint32_t)kPrefillBlock || splits < 0 ||
      splits > kMaxBf16Splits || x_stride < cols || y_stride < rows || x_stride % 4 ||
      y_stride % 4) {
    return fail(FRZ_ERR_ARGUMENT, "frz_op_gemm_bf16: bad shape, tokens or splits");
  }
  const QMatrix w = q4(codes, scales, rows, cols, format);
  if (!bf16_gemm_shape_ok(w, cols, y_stride)) {
    return fail(FRZ_ERR_ARGUMENT, "frz_op_gemm_bf16: format or shape");
  }
  if (int rc = device_put_step(dev, host_step(0, tokens))) return rc;
  if (splits == 0) splits = bf16_splits_for(rows, cols, (int)tokens, false);
  uint16_t *hi = nullptr, *lo = nullptr;
  float* parts = nullptr;
  uint4* planes = nullptr;
  const size_t blocks_rows = (tokens + 31) / 32 * 32;  // the planes' whole token blocks
  const size_t plane = blocks_rows * cols, stride = (size_t)tokens * y_stride;
  hipError_t e = hipMalloc(&hi, plane * 2);
  if (e == hipSuccess) e = hipMalloc(&lo, plane * 2);
  if (e == hipSuccess) e = hipMalloc(&parts, stride * splits * sizeof(float));
  if (e == hipSuccess) e = hipMalloc(&planes, bf16_planes_bytes(rows, cols, false));
  if (e == hipSuccess) e = launch_unpack_planes(dev->stream, w, nullptr, planes);
  if (e == hipSuccess)
    e = launch_split_rows(dev->stream, dev->step, x, x_stride, cols, hi, lo, (int)tokens);
  if (e == hipSuccess) {
    Bf16Gemm g;
    g.w = planes;
    g.rows = rows;
    g.cols = cols;
    g.x_hi = hi;
    g.x_lo = lo;
    g.ldx = cols;
    g.y = parts;
    g.ldy = y_stride;
    g.part_stride = stride;
    e = launch_gemm_bf16(dev->stream, dev->step, g, (int)tokens, splits);
  }
  if (e == hipSuccess)
    e = launch_sum_parts(dev->stream, dev->step, parts, stride, splits, rows, y_stride, y,
                         (int)tokens);
  if (e == hipSuccess) e = hipStreamSynchronize(dev->stream);
  if (hi) (void)hipFree(hi);
  if (lo) (void)hipFree(lo);
  if (parts) (void)hipFree(parts);
  if (planes) (void)hipFree(planes);
  return check_hip(e, "frz_op_gemm_bf16");
}

int frz_op_gated_bf16(frz_device* dev, const void* gate_codes, const void* gate_scales,
                      const void* up_codes, const void* up_scales, int rows, int cols,
                      const float* x, float* act, uint32_t tokens, uint32_t position,
                      const uint32_t* edits_dev, int layer) {
  if (!shape_ok(rows, cols) || rows % 16 || tokens == 0 || tokens > (uint32_t)kPrefillBlock) {
    return fail(FRZ_ERR_ARGUMENT, "frz_op_gated_bf16: bad shape or tokens");
  }
  if (int rc = device_put_step(dev, host_step(position, tokens))) return rc;
  const QMatrix gate = q4(gate_codes, gate_scales, rows, cols);
  const QMatrix up = q4(up_codes, up_scales, rows, cols);
  uint16_t *hi = nullptr, *lo = nullptr;
  uint4* planes = nullptr;
  const size_t blocks_rows = (tokens + 31) / 32 * 32;  // the planes' whole token blocks
  const size_t in = blocks_rows * cols, out = blocks_rows * rows;
  hipError_t e = hipMalloc(&hi, (in + out) * 2);
  if (e == hipSuccess) e = hipMalloc(&lo, (in + out) * 2);
  if (e == hipSuccess) e = hipMalloc(&planes, bf16_planes_bytes(rows, cols, true));
  if (e == hipSuccess) e = launch_unpack_planes(dev->stream, gate, &up, planes);
  if (e == hipSuccess)
    e = launch_split_rows(dev->stream, dev->step, x, cols, cols, hi, lo, (int)tokens);
  if (e == hipSuccess) {
    Bf16Gemm g;
    g.w = planes;
    g.rows = rows;
    g.cols = cols;
    g.gated = true;
    g.x_hi = hi;
    g.x_lo = lo;
    g.ldx = cols;
    g.y = act;
    g.ldy = rows;
    g.y_hi = hi + in;
    g.y_lo = lo + in;
    g.edits = edits_dev;
    g.layer = layer;
    e = launch_gemm_bf16(dev->stream, dev->step, g, (int)tokens, 1);
  }
  if (e == hipSuccess) e = hipStreamSynchronize(dev->stream);
  if (hi) (void)hipFree(hi);
  if (lo) (void)hipFree(lo);
  if (planes) (void)hipFree(planes);
  return check_hip(e, "frz_op_gated_bf16");
}

int frz_op_norm(frz_device* dev, const float* gain, const float* post_gain, const float* output,
                float* hidden, float* normed, int width, float epsilon, uint32_t tokens,
                int last_token) {
  if (width <= 0 || width % 4 != 0 || tokens == 0 || tokens > (uint32_t)kPrefillBlock) {
    return fail(FRZ_ERR_ARGUMENT, "frz_op_norm: bad width or tokens");
  }
  if (int rc = device_put_step(dev, host_step(0, tokens))) return rc;
  NormArgs a{gain, post_gain, output, hidden, normed, epsilon, width, last_token != 0};
  return device_finish(dev, launch_norm(dev->stream, dev->step, a, (int)tokens), "frz_op_norm");
}

int frz_op_rope(frz_device* dev, const float* turns, const float* query_gain,
                const float* key_gain, float* query, const float* key, const float* value,
                int q_stride, int kv_stride, uint16_t* key_cache, uint16_t* value_cache,
                int slots, int head_dim, int query_heads, int kv_heads, float epsilon,
                uint32_t position, uint32_t tokens) {
  if (tokens == 0 || tokens > (uint32_t)kPrefillBlock || slots < (int)tokens) {
    return fail(FRZ_ERR_ARGUMENT, "frz_op_rope: bad tokens or slots");
  }
  if (int rc = device_put_step(dev, host_step(position, tokens))) return rc;
  RopeArgs a{turns, query_gain, key_gain, query, key, value, q_stride, kv_stride,
             key_cache, value_cache, slots, head_dim, query_heads, kv_heads, epsilon};
  return device_finish(dev, launch_rope(dev->stream, dev->step, a, (int)tokens), "frz_op_rope");
}

int frz_op_attention(frz_device* dev, const float* query, int q_stride,
                     const uint16_t* key_cache, const uint16_t* value_cache, float* out,
                     int slots, int window, int head_dim, int query_heads, int kv_heads,
                     float scale, uint32_t position, uint32_t tokens) {
  if (tokens == 0 || tokens > (uint32_t)kPrefillBlock || head_dim != 256 ||
      query_heads != 4 * kv_heads || window <= 0 || slots <= 0) {
    return fail(FRZ_ERR_ARGUMENT, "frz_op_attention: unsupported shape");
  }
  const int max_chunks = attention_max_chunks(window, slots);
  const size_t part_floats = (size_t)tokens * max_chunks * query_heads * head_dim;
  const size_t stat_floats = (size_t)tokens * max_chunks * query_heads * 4;
  float* partials = nullptr;
  if (int rc = check_hip(hipMalloc(&partials, (part_floats + stat_floats) * sizeof(float)),
                         "hipMalloc(partials)"))
    return rc;
  int rc = device_put_step(dev, host_step(position, tokens));
  if (rc == FRZ_OK) {
    const float scale_log2e = (float)((double)scale * 1.4426950408889634);
    AttentionArgs a{query,    q_stride, key_cache,  value_cache, out,       partials,
                    partials + part_floats, slots, window, head_dim, query_heads,
                    kv_heads, max_chunks, scale_log2e};
    rc = device_finish(dev, launch_attention(dev->stream, dev->step, a, (int)tokens),
                       "frz_op_attention");
  }
  (void)hipFree(partials);
  return rc;
}

int frz_op_rope_attention(frz_device* dev, const float* qkv, const float* turns,
                          const float* query_gain, const float* key_gain, uint16_t* key_cache,
                          uint16_t* value_cache, float* out, int slots, int window,
                          float epsilon, float scale, uint32_t position) {
  if (window <= 0 || slots <= 0 || slots > (1 << 21) || position >= (1u << 24)) {
    return fail(FRZ_ERR_ARGUMENT, "frz_op_rope_attention: bad window or slots (at most 2,097,152 slots,"
                                  " positions under 2^24)");
  }
  if ((uint64_t)slots < std::min<uint64_t>((uint64_t)window, (uint64_t)position + 1) ||
      (slots < kChunkKeys && position >= (uint32_t)slots)) {
    // The window's keys need slots of their own (the step's key is appended
    // while the others are read), and a chunk's rows may wrap the ring once.
    return fail(FRZ_ERR_ARGUMENT, "frz_op_rope_attention: the ring holds fewer slots than the window's keys"
                                  " (or, under 64 slots, than the positions)");
  }
  const int max_chunks = attention_max_chunks(window, slots);
  const size_t part_floats = (size_t)max_chunks * 4 * 256;
  float* partials = nullptr;
  if (int rc = check_hip(hipMalloc(&partials, (part_floats + part_floats / 64) * sizeof(float)),
                         "hipMalloc(partials)"))
    return rc;
  int rc = device_put_step(dev, host_step(position, 1));
  if (rc == FRZ_OK) {
    const float scale_log2e = (float)((double)scale * 1.4426950408889634);
    DecodeAttentionArgs a{qkv,        turns,    query_gain,            key_gain, key_cache,
                          value_cache, partials, partials + part_floats, slots,   window,
                          256,        4,        1,                     max_chunks, epsilon,
                          scale_log2e};
    hipError_t e = launch_attention_decode(dev->stream, dev->step, a);
    if (e == hipSuccess) {
      e = launch_attention_fold(dev->stream, dev->step,
                                FoldArgs{partials, partials + part_floats, out, window, max_chunks},
                                1);
    }
    rc = device_finish(dev, e, "frz_op_rope_attention");
  }
  (void)hipFree(partials);
  return rc;
}

int frz_op_rope_attention_noalloc(frz_device* dev, const float* qkv, const float* turns,
                                  const float* query_gain, const float* key_gain,
                                  uint16_t* key_cache, uint16_t* value_cache, float* out,
                                  int slots, int window, float epsilon, float scale,
                                  uint32_t position) {
  if (!dev || !dev->static_workspace) {
    return fail(FRZ_ERR_ARGUMENT, "frz_op_rope_attention_noalloc: no device");
  }
  if (window <= 0 || slots <= 0 || slots > (1 << 21) || position >= (1u << 24)) {
    return fail(FRZ_ERR_ARGUMENT, "frz_op_rope_attention_noalloc: bad window or slots (at most 2,097,152 slots,"
                                  " positions under 2^24)");
  }
  if ((uint64_t)slots < std::min<uint64_t>((uint64_t)window, (uint64_t)position + 1) ||
      (slots < kChunkKeys && position >= (uint32_t)slots)) {
    // The window's keys need slots of their own (the step's key is appended
    // while the others are read), and a chunk's rows may wrap the ring once.
    return fail(FRZ_ERR_ARGUMENT, "frz_op_rope_attention_noalloc: the ring holds fewer slots than the window's keys"
                                  " (or, under 64 slots, than the positions)");
  }
  const int max_chunks = attention_max_chunks(window, slots);
  if (max_chunks > kStaticChunks) {
    return fail(FRZ_ERR_ARGUMENT,
                "frz_op_rope_attention_noalloc: window and slots reach " +
                    std::to_string(max_chunks) + " chunks; the static workspace holds " +
                    std::to_string(kStaticChunks) + " (at most 14,272 keys)");
  }
  // Chunk states at the same offsets the allocating entry point gives them:
  // every state the fold reads is written first by this call's attention
  // launch, so nothing needs clearing between calls.
  float* partials = dev->static_workspace;
  const size_t part_floats = (size_t)max_chunks * 4 * 256;
  if (int rc = device_put_step(dev, host_step(position, 1))) return rc;
  const float scale_log2e = (float)((double)scale * 1.4426950408889634);
  DecodeAttentionArgs a{qkv,        turns,    query_gain,            key_gain, key_cache,
                        value_cache, partials, partials + part_floats, slots,   window,
                        256,        4,        1,                     max_chunks, epsilon,
                        scale_log2e};
  hipError_t e = launch_attention_decode(dev->stream, dev->step, a);
  if (e == hipSuccess) {
    e = launch_attention_fold(dev->stream, dev->step,
                              FoldArgs{partials, partials + part_floats, out, window, max_chunks},
                              1);
  }
  return device_finish(dev, e, "frz_op_rope_attention_noalloc");
}

int frz_op_gather(frz_device* dev, const void* codes, const void* scales, int rows, int cols,
                  const uint32_t* ids, uint32_t tokens, float scale, float* hidden) {
  return frz_op_gather_format(dev, kQ4_0, codes, scales, rows, cols, ids, tokens, scale, hidden);
}

int frz_op_gather_format(frz_device* dev, int format, const void* codes, const void* scales,
                         int rows, int cols, const uint32_t* ids, uint32_t tokens, float scale,
                         float* hidden) {
  if (!shape_ok(rows, cols) || tokens == 0 || tokens > (uint32_t)kPrefillBlock) {
    return fail(FRZ_ERR_ARGUMENT, "frz_op_gather: bad shape or tokens");
  }
  if (format != kQ4_0 && format != kQ8_0) {
    return fail(FRZ_ERR_ARGUMENT, "frz_op_gather: format " + std::to_string(format) +
                                      " (Q4_0 2 or Q8_0 8)");
  }
  DevStep s = host_step(0, tokens);
  std::memcpy(s.ids, ids, tokens * sizeof(uint32_t));
  if (int rc = device_put_step(dev, s)) return rc;
  return device_finish(
      dev,
      launch_gather(dev->stream, dev->step, q4(codes, scales, rows, cols, format), nullptr,
                    hidden, scale, (int)tokens),
      "frz_op_gather");
}

int frz_op_edit(frz_device* dev, const uint32_t* edits_dev, int layer, float* act, int width,
                uint32_t position, uint32_t tokens) {
  if (tokens == 0 || tokens > (uint32_t)kPrefillBlock) {
    return fail(FRZ_ERR_ARGUMENT, "frz_op_edit: bad tokens");
  }
  if (int rc = device_put_step(dev, host_step(position, tokens))) return rc;
  return device_finish(
      dev, launch_edit(dev->stream, dev->step, edits_dev, layer, act, width, (int)tokens),
      "frz_op_edit");
}

int frz_op_topk(frz_device* dev, const float* logits, int count, uint32_t* candidates_dev) {
  if (count < kCandidates) return fail(FRZ_ERR_ARGUMENT, "frz_op_topk: fewer than 64 logits");
  uint32_t* scratch = nullptr;
  if (int rc = check_hip(hipMalloc(&scratch, topk_scratch_words(count) * 4), "hipMalloc(topk)"))
    return rc;
  const int rc =
      device_finish(dev, launch_topk(dev->stream, logits, count, scratch, candidates_dev),
                    "frz_op_topk");
  (void)hipFree(scratch);
  return rc;
}

int frz_op_draw(frz_device* dev, const uint32_t* candidates_dev, const frz_sampling* sampling,
                uint32_t position, uint32_t tokens, uint32_t* record_dev) {
  if (sampling && (sampling->top_k < 1 || sampling->top_k > (uint32_t)kCandidates)) {
    return fail(FRZ_ERR_ARGUMENT, "frz_op_draw: top_k outside 1..64");
  }
  DevStep s = host_step(position, tokens);
  fill_sampling(s, sampling);
  if (int rc = device_put_step(dev, s)) return rc;
  return device_finish(
      dev, launch_draw(dev->stream, dev->step, candidates_dev, record_dev, nullptr),
      "frz_op_draw");
}

int frz_op_numerics(frz_device* dev, int which, const float* in_dev, float* out_dev, int n) {
  if (n <= 0) return fail(FRZ_ERR_ARGUMENT, "frz_op_numerics: n <= 0");
  hipLaunchKernelGGL(numerics_kernel, dim3((n + 255) / 256), dim3(256), 0, dev->stream, which,
                     in_dev, out_dev, n);
  return device_finish(dev, hipGetLastError(), "frz_op_numerics");
}

}  // extern "C"

namespace frz {
// Times launches replayed from a graph of one launch per weight copy: the
// captured launches run back to back, so the figure is the kernels' own
// rate, with the weights streaming from HBM as the copies rotate.
// Without `graph` the launches go to the stream one by one (for profilers
// that do not follow graph launches).
template <typename Launch>
static int bench_graph(frz_device* dev, int copies, int iters, int graph_mode, Launch launch,
                       const char* what, double* us_per_launch) {
  hipStream_t s = dev->stream;
  for (int i = 0; i < copies; ++i) {  // warm: every copy once
    if (int rc = check_hip(launch(i), what)) return rc;
  }
  if (int rc = check_hip(hipStreamSynchronize(s), what)) return rc;
  if (!graph_mode) {
    hipEvent_t start = nullptr, stop = nullptr;
    int rc = check_hip(hipEventCreate(&start), what);
    if (rc == FRZ_OK) rc = check_hip(hipEventCreate(&stop), what);
    if (rc == FRZ_OK) rc = check_hip(hipEventRecord(start, s), what);
    for (int i = 0; i < iters && rc == FRZ_OK; ++i) rc = check_hip(launch(i % copies), what);
    if (rc == FRZ_OK) rc = check_hip(hipEventRecord(stop, s), what);
    if (rc == FRZ_OK) rc = check_hip(hipEventSynchronize(stop), what);
    float ms = 0.0f;
    if (rc == FRZ_OK) rc = check_hip(hipEventElapsedTime(&ms, start, stop), what);
    if (start) (void)hipEventDestroy(start);
    if (stop) (void)hipEventDestroy(stop);
    *us_per_launch = (double)ms * 1000.0 / iters;
    return rc;
  }
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  int rc = check_hip(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal), what);
  if (rc == FRZ_OK) {
    hipError_t e = hipSuccess;
    for (int i = 0; i < copies && e == hipSuccess; ++i) e = launch(i);
    const hipError_t end = hipStreamEndCapture(s, &graph);
    rc = check_hip(e != hipSuccess ? e : end, what);
  }
  if (rc == FRZ_OK) rc = check_hip(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0), what);
  const int replays = (iters + copies - 1) / copies;
  hipEvent_t start = nullptr, stop = nullptr;
  if (rc == FRZ_OK) rc = check_hip(hipGraphLaunch(exec, s), what);  // warm the graph
  if (rc == FRZ_OK) rc = check_hip(hipEventCreate(&start), what);
  if (rc == FRZ_OK) rc = check_hip(hipEventCreate(&stop), what);
  if (rc == FRZ_OK) rc = check_hip(hipEventRecord(start, s), what);
  for (int i = 0; i < replays && rc == FRZ_OK; ++i) rc = check_hip(hipGraphLaunch(exec, s), what);
  if (rc == FRZ_OK) rc = check_hip(hipEventRecord(stop, s), what);
  if (rc == FRZ_OK) rc = check_hip(hipEventSynchronize(stop), what);
  float ms = 0.0f;
  if (rc == FRZ_OK) rc = check_hip(hipEventElapsedTime(&ms, start, stop), what);
  if (start) (void)hipEventDestroy(start);
  if (stop) (void)hipEventDestroy(stop);
  if (exec) (void)hipGraphExecDestroy(exec);
  if (graph) (void)hipGraphDestroy(graph);
  *us_per_launch = (double)ms * 1000.0 / ((double)replays * copies);
  return rc;
}
}  // namespace frz

extern "C" {

int frz_bench_gemv(frz_device* dev, const void* const* codes, const void* const* scales,
                   int copies, int rows, int cols, const float* x, float* y, int iters,
                   int graph, double* us_per_launch) {
  if (!shape_ok(rows, cols) || copies <= 0 || iters <= 0 || !us_per_launch) {
    return fail(FRZ_ERR_ARGUMENT, "frz_bench_gemv: bad argument");
  }
  if (int rc = device_put_step(dev, host_step(0, 1))) return rc;
  return bench_graph(dev, copies, iters, graph, [&](int c) {
    return launch_gemv(dev->stream, dev->step, q4(codes[c], scales[c], rows, cols), x, cols, y,
                       rows, 1, false);
  }, "frz_bench_gemv", us_per_launch);
}

int frz_bench_gated(frz_device* dev, const void* const* gate_codes,
                    const void* const* gate_scales, const void* const* up_codes,
                    const void* const* up_scales, int copies, int rows, int cols,
                    const float* x, float* act, int iters, int graph, double* us_per_launch) {
  if (!shape_ok(rows, cols) || copies <= 0 || iters <= 0 || !us_per_launch) {
    return fail(FRZ_ERR_ARGUMENT, "frz_bench_gated: bad argument");
  }
  if (int rc = device_put_step(dev, host_step(0, 1))) return rc;
  return bench_graph(dev, copies, iters, graph, [&](int c) {
    return launch_gated(dev->stream, dev->step, q4(gate_codes[c], gate_scales[c], rows, cols),
                        q4(up_codes[c], up_scales[c], rows, cols), x, act, 1, nullptr, 0);
  }, "frz_bench_gated", us_per_launch);
}

int frz_bench_launch_floor(frz_device* dev, int iters, int graph, double* us_per_launch) {
  if (!dev || iters <= 0 || !us_per_launch) {
    return fail(FRZ_ERR_ARGUMENT, "frz_bench_launch_floor: bad argument");
  }
  return bench_graph(dev, kFloorCopies, iters, graph, [&](int) {
    hipLaunchKernelGGL(empty_kernel, dim3(1), dim3(64), 0, dev->stream);
    return hipGetLastError();
  }, "frz_bench_launch_floor", us_per_launch);
}

int frz_bench_stream(frz_device* dev, const void* const* buffers, int copies, uint64_t bytes,
                     uint32_t* sink, int iters, int graph, double* us_per_launch) {
  if (!dev || !buffers || copies <= 0 || bytes < 16 || bytes % 16 || !sink || iters <= 0 ||
      !us_per_launch) {
    return fail(FRZ_ERR_ARGUMENT, "frz_bench_stream: bad argument");
  }
  for (int c = 0; c < copies; ++c) {
    if (!buffers[c]) return fail(FRZ_ERR_ARGUMENT, "frz_bench_stream: null buffer");
  }
  return bench_graph(dev, copies, iters, graph, [&](int c) {
    hipLaunchKernelGGL(stream_kernel, dim3(kStreamBlocks), dim3(256), 0, dev->stream,
                       static_cast<const uint4*>(buffers[c]), (size_t)(bytes / 16), sink);
    return hipGetLastError();
  }, "frz_bench_stream", us_per_launch);
}

int frz_copy(frz_device* dev, void* dev_dst, const void* dev_src, uint64_t bytes) {
  if (!dev || (bytes && (!dev_dst || !dev_src))) return fail(FRZ_ERR_ARGUMENT, "frz_copy: null");
  return device_finish(
      dev, hipMemcpyAsync(dev_dst, dev_src, bytes, hipMemcpyDeviceToDevice, dev->stream),
      "frz_copy");
}

void frz_rope_turns(float base, int head_dim, float* turns) {
  const double pi = 3.14159265358979323846;
  for (int k = 0; k < head_dim / 2; ++k) {
    const double theta = std::pow((double)base, -2.0 * k / head_dim);
    turns[k] = (float)(theta / (2 * pi));
  }
}

}  // extern "C"
