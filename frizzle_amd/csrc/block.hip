// The per-row kernels of a decoder layer: RMSNorm with the residual add and
// post-norm fused in, QK-norm + rope + KV-cache append, attention over 64-key
// chunks with its in-order fold, the embedding gather and the pin kernel.
// Each keeps the reference's reductions and rounding points (cited per
// kernel), so a token's rows are the same bits in any step.

#include "kernels.h"
#include "numerics.h"
#include "rope_common.h"

namespace frz {
namespace {

__device__ __forceinline__ float4 ld4(const float* p) {
  return *reinterpret_cast<const float4*>(p);
}
__device__ __forceinline__ void st4(float* p, float4 v) {
  *reinterpret_cast<float4*>(p) = v;
}
__device__ __forceinline__ float dot4v(float4 a, float4 b) {
  return dot4(a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w);
}

__device__ __forceinline__ float4 add4(float4 a, float4 b) {
  return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
}

// a and b plus `count` rows of partial sums each (rows `stride` floats
// apart from pa and pb), added in row order. Eight rows are requested
// before any is added, so a split product's later sums cost a memory round
// trip for every eight, not for every one.
__device__ __forceinline__ void add_parts(float4& a, float4& b, const float* pa, const float* pb,
                                          size_t stride, int count) {
  for (int j0 = 0; j0 < count; j0 += 8) {
    float4 sa[8], sb[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if (j0 + j < count) {
        sa[j] = ld4(pa + (size_t)(j0 + j) * stride);
        if (pb) sb[j] = ld4(pb + (size_t)(j0 + j) * stride);
      }
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if (j0 + j < count) {
        a = add4(a, sa[j]);
        if (pb) b = add4(b, sb[j]);
      }
    }
  }
}

// ---- RMSNorm (norm.wgsl:96-198) -----------------------------------------
constexpr int kNormThreads = 256;
constexpr int kNormMaxVec4 = 4;  // rows up to 4,096 wide

// The workgroup's sum in the reference's tree (norm.wgsl:75-85), halving
// the 256 partial sums at each level: levels 128 and 64 in registers from
// LDS, the last six across the wave, so every wave has the total after one
// barrier. `partial` is 256 floats the call owns.
__device__ __forceinline__ float norm_reduce(float* partial, float v) {
  const int i = threadIdx.x, lane = i & 63;
  partial[i] = v;
  __syncthreads();
  return wave_tree((partial[lane] + partial[lane + 128]) +
                   (partial[lane + 64] + partial[lane + 192]));
}

__global__ __launch_bounds__(kNormThreads) void norm_kernel(
    const DevStep* __restrict__ step, NormArgs a) {
  __shared__ float partial[2][kNormThreads];
  // Every load is issued first: rows of the launch past the step's are
  // still inside the buffers (the grid is the step's most rows) and leave
  // once their loads are out.
  const int row = a.last_token ? (int)step->tokens - 1 : (int)blockIdx.x;
  const int vec4s = a.width / 4;
  const size_t base = (size_t)row * a.width;
  const float n = (float)a.width;
  const int i = threadIdx.x;
  float4 x[kNormMaxVec4], y[kNormMaxVec4], pg[kNormMaxVec4], g[kNormMaxVec4];
  const int per = (vec4s + kNormThreads - 1) / kNormThreads;
#pragma unroll
  for (int k = 0; k < kNormMaxVec4; ++k) {
    const int q = i + k * kNormThreads;
    if (k < per && q < vec4s) {
      x[k] = ld4(a.hidden + base + 4 * q);
      g[k] = ld4(a.gain + 4 * q);
      if (a.post_gain) {
        y[k] = ld4(a.output + base + 4 * q);
        pg[k] = ld4(a.post_gain + 4 * q);
        // A split product's output: the prefix of its first ranges, then
        // the later range sums added in range order.
        if (a.parts) {
          float4 unused;
          add_parts(y[k], unused, a.parts + base + 4 * q, nullptr, a.parts_stride,
                    a.part_count);
        }
      }
    }
  }
  const int tokens = (int)step->tokens;
  if (row >= tokens) return;
  if (a.post_gain) {
    float squares = 0.0f;
#pragma unroll
    for (int k = 0; k < kNormMaxVec4; ++k) {
      if (k < per && i + k * kNormThreads < vec4s) squares = squares + dot4v(y[k], y[k]);
    }
    const float r = inverse_sqrt(norm_reduce(partial[0], squares) / n + a.epsilon);
#pragma unroll
    for (int k = 0; k < kNormMaxVec4; ++k) {
      const int q = i + k * kNormThreads;
      if (k < per && q < vec4s) {
        // ((y * r) * post_gain) * post_scale, post_scale 1 (norm.wgsl:149).
        y[k].x = ((y[k].x * r) * pg[k].x) * 1.0f;
        y[k].y = ((y[k].y * r) * pg[k].y) * 1.0f;
        y[k].z = ((y[k].z * r) * pg[k].z) * 1.0f;
        y[k].w = ((y[k].w * r) * pg[k].w) * 1.0f;
        x[k].x = x[k].x + y[k].x;
        x[k].y = x[k].y + y[k].y;
        x[k].z = x[k].z + y[k].z;
        x[k].w = x[k].w + y[k].w;
        st4(a.hidden + base + 4 * q, x[k]);
      }
    }
  }
  if (a.capture) {
    float* cap = a.capture + (size_t)step->drawn * a.capture_step + base;
#pragma unroll
    for (int k = 0; k < kNormMaxVec4; ++k) {
      const int q = i + k * kNormThreads;
      if (k < per && q < vec4s) st4(cap + 4 * q, x[k]);
    }
  }
  if (row == tokens - 1 && (a.store_x || a.store_added)) {
#pragma unroll
    for (int k = 0; k < kNormMaxVec4; ++k) {
      const int q = i + k * kNormThreads;
      if (k < per && q < vec4s) {
        if (a.store_x) st4(a.store_x + 4 * q, x[k]);
        if (a.store_added && a.post_gain) st4(a.store_added + 4 * q, y[k]);
      }
    }
  }
  float squares = 0.0f;
#pragma unroll
  for (int k = 0; k < kNormMaxVec4; ++k) {
    if (k < per && i + k * kNormThreads < vec4s) squares = squares + dot4v(x[k], x[k]);
  }
  const float r = inverse_sqrt(norm_reduce(partial[1], squares) / n + a.epsilon);
#pragma unroll
  for (int k = 0; k < kNormMaxVec4; ++k) {
    const int q = i + k * kNormThreads;
    if (k < per && q < vec4s) {
      float4 o;
      o.x = (x[k].x * r) * g[k].x;
      o.y = (x[k].y * r) * g[k].y;
      o.z = (x[k].z * r) * g[k].z;
      o.w = (x[k].w * r) * g[k].w;
      st4(a.normed + base + 4 * q, o);
      if (a.normed_hi) {
        const float v[4] = {o.x, o.y, o.z, o.w};
        store_pairs4(a.normed_hi, a.normed_lo, row, 4 * q, a.width, v);
      }
    }
  }
}

// ---- QK-norm, rope, KV append (rope.wgsl:51-138, rope_cache.wgsl) ----------
// One workgroup a token: head h's lane l holds dimensions 4l..4l+3 and
// d/2 + 4l..d/2 + 4l + 3; query and key heads reduce their squares over
// their d/8 lanes in a halving tree, normalize, and rotate pairs (k, k+d/2).
__global__ __launch_bounds__(256) void rope_kernel(const DevStep* __restrict__ step,
                                                   RopeArgs a) {
  __shared__ float cosines[kMaxHeadDim / 2], sines[kMaxHeadDim / 2];
  __shared__ float partial[256];
  const int row = blockIdx.x;
  if (row >= (int)step->tokens) return;
  const uint32_t p = step->position + (step->variants ? 0u : (uint32_t)row);
  const size_t cache_at = step->variants ? (size_t)row * a.cache_stride : 0;
  const int lanes = a.head_dim / 8, half = a.head_dim / 2;
  const int heads = a.query_heads + 2 * a.kv_heads;
  const int t = threadIdx.x;
  rope_angles(a.turns, p, half, cosines, sines, t, blockDim.x);
  const int h = t / lanes, lane = t % lanes;
  const bool active = h < heads;
  const bool is_query = h < a.query_heads;
  const bool is_value = h >= a.query_heads + a.kv_heads;
  const int kv = is_value ? h - a.query_heads - a.kv_heads : h - a.query_heads;
  const float* src;
  if (is_query) {
    src = (a.query_in ? a.query_in : a.query) + (size_t)row * a.q_stride +
          (size_t)h * a.head_dim;
  } else if (is_value) {
    src = a.value + (size_t)row * a.kv_stride + (size_t)kv * a.head_dim;
  } else {
    src = a.key + (size_t)row * a.kv_stride + (size_t)kv * a.head_dim;
  }
  float4 va = make_float4(0.f, 0.f, 0.f, 0.f), vb = va;
  if (active) {
    va = ld4(src + 4 * lane);
    vb = ld4(src + half + 4 * lane);
    // A K-split product's later partial sums, added in split order.
    add_parts(va, vb, src + a.part_stride + 4 * lane, src + a.part_stride + half + 4 * lane,
              a.part_stride, a.part_count - 1);
  }
  partial[t] = rope_lane_squares(va, vb);
  __syncthreads();
  for (int stride = lanes / 2; stride > 0; stride >>= 1) {
    if (active && lane < stride) partial[t] = partial[t] + partial[t + stride];
    __syncthreads();
  }
  if (!active) return;
  if (!is_value) {
    rope_norm_rotate(va, vb, partial[t - lane], a.head_dim, a.epsilon,
                     is_query ? a.query_gain : a.key_gain, lane, cosines, sines);
  }
  if (is_query) {
    float* dst = a.query + (size_t)row * a.q_stride + (size_t)h * a.head_dim;
    st4(dst + 4 * lane, va);
    st4(dst + half + 4 * lane, vb);
  } else {
    const uint32_t slot = p % (uint32_t)a.slots;
    uint16_t* cache = (is_value ? a.value_cache : a.key_cache) + cache_at +
                      ((size_t)slot * a.kv_heads + kv) * a.head_dim;
    *reinterpret_cast<ushort4*>(cache + 4 * lane) = pack4_f16(va);
    *reinterpret_cast<ushort4*>(cache + half + 4 * lane) = pack4_f16(vb);
  }
}

// ---- gather (gather.wgsl:25-48) ---------------------------------------------
__global__ __launch_bounds__(256) void gather_kernel(const DevStep* __restrict__ step,
                                                     QMatrix table,
                                                     const uint32_t* __restrict__ sampled,
                                                     float* __restrict__ hidden, float scale) {
  const int row = blockIdx.x;
  if (row >= (int)step->tokens) return;
  const uint32_t token = step->fed ? sampled[step->variants ? 4 * row : 0] : step->ids[row];
  if (token >= (uint32_t)table.rows) return;
  const int groups = table.cols / 32;
  // A Q8_0 table (the file's embedding) holds weight j of a block as the
  // signed byte j times d (q8_0.wgsl:10-21); a Q4_0 one as nibble (q - 8) d.
  // Either product is exact, so the one rounding is that of the scale.
  const bool bytes = table.format == kQ8_0;
  for (int i = threadIdx.x; i < table.cols; i += blockDim.x) {
    const size_t blk = (size_t)token * groups + i / 32;
    const int j = i % 32;
    const float d = (float)__builtin_bit_cast(_Float16, table.scales[blk]);
    float wv;
    if (bytes) {
      wv = (float)(int8_t)table.codes[blk * 32 + j] * d;
    } else {
      const uint8_t byte = table.codes[blk * 16 + (j & 15)];
      const uint32_t q = j < 16 ? (byte & 0xFu) : (uint32_t)(byte >> 4);
      wv = fmaf_((float)q, d, -8.0f * d);
    }
    hidden[(size_t)row * table.cols + i] = wv * scale;
  }
}

// ---- the capture store's copy (capture.wgsl) ----------------------------------
__global__ __launch_bounds__(256) void capture_copy_kernel(const DevStep* __restrict__ step,
                                                           const uint32_t* __restrict__ src,
                                                           size_t row_stride, int width,
                                                           uint32_t* __restrict__ dst) {
  const uint32_t* row = src + (size_t)(step->tokens - 1) * row_stride;
  for (int i = threadIdx.x; i < width; i += blockDim.x) dst[i] = row[i];
}

// The last row's scores into attention weights (weights.wgsl), a workgroup
// a query head: weight i = exp2(s_i - m) / l for the keys p read, earliest
// + i; zero past them.
__global__ __launch_bounds__(256) void capture_weights_kernel(const DevStep* __restrict__ step,
                                                              float* __restrict__ weights,
                                                              const float* __restrict__ stats,
                                                              int keys) {
  const int h = blockIdx.x;
  const uint32_t p = step->position + step->tokens - 1;
  const uint32_t read = min(p + 1, (uint32_t)keys);  // keys p's query read
  const float m = stats[2 * h], l = stats[2 * h + 1];
  float* w = weights + (size_t)h * keys;
  for (int i = threadIdx.x; i < keys; i += blockDim.x)
    w[i] = (uint32_t)i < read ? exp2f_fixed(w[i] - m) / l : 0.0f;
}

// ---- pins (edit.wgsl:55-76) ----------------------------------------------------
__global__ __launch_bounds__(64) void edit_kernel(const DevStep* __restrict__ step,
                                                  const uint32_t* __restrict__ table,
                                                  int layer, float* __restrict__ act,
                                                  int width) {
  const int row = blockIdx.x;
  if (row >= (int)step->tokens) return;
  const uint32_t first = table[2 * layer];
  const uint32_t count = table[2 * layer + 1];
  const uint32_t position = step->position + (step->variants ? 0u : (uint32_t)row);
  for (uint32_t i = threadIdx.x; i < count; i += 64) {
    const uint32_t* e = table + first + 5 * i;
    if (position < e[3] || position >= e[4]) continue;
    const float value = bits_to_float(e[2]);
    float* n = act + (size_t)row * width + e[0];
    float edited = value;
    if (e[1] == 1u) edited = value == 1.0f ? *n : *n * value;
    *n = edited;
  }
}

}  // namespace

hipError_t launch_norm(hipStream_t s, const DevStep* step, const NormArgs& a,
                       int max_tokens) {
  if (a.width % 4 != 0 || a.width > 4 * kNormThreads * kNormMaxVec4) return hipErrorInvalidValue;
  hipLaunchKernelGGL(norm_kernel, dim3(a.last_token ? 1 : max_tokens), dim3(kNormThreads), 0, s,
                     step, a);
  return hipGetLastError();
}

hipError_t launch_rope(hipStream_t s, const DevStep* step, const RopeArgs& a,
                       int max_tokens) {
  const int threads = (a.query_heads + 2 * a.kv_heads) * (a.head_dim / 8);
  if (a.head_dim > kMaxHeadDim || a.head_dim % 8 != 0 || threads > 256) return hipErrorInvalidValue;
  const int block = threads <= 64 ? 64 : (threads <= 128 ? 128 : 256);
  hipLaunchKernelGGL(rope_kernel, dim3(max_tokens), dim3(block), 0, s, step, a);
  return hipGetLastError();
}

hipError_t launch_gather(hipStream_t s, const DevStep* step, QMatrix table,
                         const uint32_t* sampled, float* hidden, float scale,
                         int max_tokens) {
  if (table.format != kQ4_0 && table.format != kQ8_0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(gather_kernel, dim3(max_tokens), dim3(256), 0, s, step, table, sampled,
                     hidden, scale);
  return hipGetLastError();
}

hipError_t launch_capture_copy(hipStream_t s, const DevStep* step, const void* src,
                               size_t row_stride, int width, void* dst) {
  hipLaunchKernelGGL(capture_copy_kernel, dim3(1), dim3(256), 0, s, step,
                     static_cast<const uint32_t*>(src), row_stride, width,
                     static_cast<uint32_t*>(dst));
  return hipGetLastError();
}

hipError_t launch_capture_weights(hipStream_t s, const DevStep* step, float* weights,
                                  const float* stats, int keys, int query_heads) {
  if (keys <= 0 || query_heads <= 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(capture_weights_kernel, dim3(query_heads), dim3(256), 0, s, step, weights,
                     stats, keys);
  return hipGetLastError();
}

hipError_t launch_edit(hipStream_t s, const DevStep* step,
                       const uint32_t* edits, int layer, float* act,
                       int width, int max_tokens) {
  hipLaunchKernelGGL(edit_kernel, dim3(max_tokens), dim3(64), 0, s, step, edits, layer, act,
                     width);
  return hipGetLastError();
}

}  // namespace frz
