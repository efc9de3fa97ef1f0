// The per-row kernels of a decoder layer: RMSNorm with the residual add and
// post-norm fused in, QK-norm + rope + KV-cache append, attention over 64-key
// chunks with its in-order fold, the embedding gather and the pin kernel.
// Each keeps the reference's reductions and rounding points (cited per
// kernel), so a token's rows are the same bits in any step.

#include "kernels.h"
#include "numerics.h"

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

// ---- RMSNorm (norm.wgsl:96-198) -----------------------------------------
constexpr int kNormThreads = 256;
constexpr int kNormMaxVec4 = 4;  // rows up to 4,096 wide

// The workgroup's sum in the reference's tree (norm.wgsl:75-85): halving
// the 256 partial sums at each level.
__device__ __forceinline__ float norm_reduce(float* partial, float v) {
  const int i = threadIdx.x;
  partial[i] = v;
  __syncthreads();
  for (int stride = kNormThreads / 2; stride > 0; stride >>= 1) {
    if (i < stride) partial[i] = partial[i] + partial[i + stride];
    __syncthreads();
  }
  return partial[0];
}

__global__ __launch_bounds__(kNormThreads) void norm_kernel(
    const DevStep* __restrict__ step, NormArgs a) {
  __shared__ float partial[kNormThreads];
  const int tokens = (int)step->tokens;
  const int row = a.last_token ? tokens - 1 : (int)blockIdx.x;
  if (row >= tokens) return;
  const int vec4s = a.width / 4;
  const size_t base = (size_t)row * a.width;
  const float n = (float)a.width;
  const int i = threadIdx.x;
  float4 x[kNormMaxVec4], y[kNormMaxVec4];
  const int per = (vec4s + kNormThreads - 1) / kNormThreads;
#pragma unroll
  for (int k = 0; k < kNormMaxVec4; ++k) {
    const int q = i + k * kNormThreads;
    if (k < per && q < vec4s) x[k] = ld4(a.hidden + base + 4 * q);
  }
  if (a.post_gain) {
#pragma unroll
    for (int k = 0; k < kNormMaxVec4; ++k) {
      const int q = i + k * kNormThreads;
      if (k < per && q < vec4s) y[k] = ld4(a.output + base + 4 * q);
    }
    float squares = 0.0f;
#pragma unroll
    for (int k = 0; k < kNormMaxVec4; ++k) {
      if (k < per && i + k * kNormThreads < vec4s) squares = squares + dot4v(y[k], y[k]);
    }
    const float r = inverse_sqrt(norm_reduce(partial, squares) / n + a.epsilon);
    __syncthreads();
#pragma unroll
    for (int k = 0; k < kNormMaxVec4; ++k) {
      const int q = i + k * kNormThreads;
      if (k < per && q < vec4s) {
        const float4 g = ld4(a.post_gain + 4 * q);
        // ((y * r) * post_gain) * post_scale, post_scale 1 (norm.wgsl:149).
        y[k].x = ((y[k].x * r) * g.x) * 1.0f;
        y[k].y = ((y[k].y * r) * g.y) * 1.0f;
        y[k].z = ((y[k].z * r) * g.z) * 1.0f;
        y[k].w = ((y[k].w * r) * g.w) * 1.0f;
        x[k].x = x[k].x + y[k].x;
        x[k].y = x[k].y + y[k].y;
        x[k].z = x[k].z + y[k].z;
        x[k].w = x[k].w + y[k].w;
        st4(a.hidden + base + 4 * q, x[k]);
      }
    }
  }
  float squares = 0.0f;
#pragma unroll
  for (int k = 0; k < kNormMaxVec4; ++k) {
    if (k < per && i + k * kNormThreads < vec4s) squares = squares + dot4v(x[k], x[k]);
  }
  const float r = inverse_sqrt(norm_reduce(partial, squares) / n + a.epsilon);
#pragma unroll
  for (int k = 0; k < kNormMaxVec4; ++k) {
    const int q = i + k * kNormThreads;
    if (k < per && q < vec4s) {
      const float4 g = ld4(a.gain + 4 * q);
      float4 o;
      o.x = (x[k].x * r) * g.x;
      o.y = (x[k].y * r) * g.y;
      o.z = (x[k].z * r) * g.z;
      o.w = (x[k].w * r) * g.w;
      st4(a.normed + base + 4 * q, o);
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
  const uint32_t p = step->position + (uint32_t)row;
  const int lanes = a.head_dim / 8, half = a.head_dim / 2;
  const int heads = a.query_heads + 2 * a.kv_heads;
  const int t = threadIdx.x;
  for (int k = t; k < half; k += blockDim.x) {
    const float tt = (float)p * a.turns[k];
    const float angle = 6.283185307179586f * (tt - rint_(tt));
    sincos_fixed(angle, &sines[k], &cosines[k]);
  }
  const int h = t / lanes, lane = t % lanes;
  const bool active = h < heads;
  const bool is_query = h < a.query_heads;
  const bool is_value = h >= a.query_heads + a.kv_heads;
  const int kv = is_value ? h - a.query_heads - a.kv_heads : h - a.query_heads;
  const float* src;
  if (is_query) {
    src = a.query + (size_t)row * a.q_stride + (size_t)h * a.head_dim;
  } else if (is_value) {
    src = a.value + (size_t)row * a.kv_stride + (size_t)kv * a.head_dim;
  } else {
    src = a.key + (size_t)row * a.kv_stride + (size_t)kv * a.head_dim;
  }
  float4 va = make_float4(0.f, 0.f, 0.f, 0.f), vb = va;
  if (active) {
    va = ld4(src + 4 * lane);
    vb = ld4(src + half + 4 * lane);
  }
  partial[t] = dot4v(va, va) + dot4v(vb, vb);
  __syncthreads();
  for (int stride = lanes / 2; stride > 0; stride >>= 1) {
    if (active && lane < stride) partial[t] = partial[t] + partial[t + stride];
    __syncthreads();
  }
  if (!active) return;
  if (!is_value) {
    const float r = inverse_sqrt(partial[t - lane] / (float)a.head_dim + a.epsilon);
    const float* g = is_query ? a.query_gain : a.key_gain;
    const float4 ga = ld4(g + 4 * lane), gb = ld4(g + half + 4 * lane);
    va.x = (va.x * r) * ga.x; va.y = (va.y * r) * ga.y;
    va.z = (va.z * r) * ga.z; va.w = (va.w * r) * ga.w;
    vb.x = (vb.x * r) * gb.x; vb.y = (vb.y * r) * gb.y;
    vb.z = (vb.z * r) * gb.z; vb.w = (vb.w * r) * gb.w;
    const int k = 4 * lane;
    const float c0 = cosines[k], c1 = cosines[k + 1], c2 = cosines[k + 2], c3 = cosines[k + 3];
    const float s0 = sines[k], s1 = sines[k + 1], s2 = sines[k + 2], s3 = sines[k + 3];
    const float4 ra = make_float4(va.x * c0 - vb.x * s0, va.y * c1 - vb.y * s1,
                                  va.z * c2 - vb.z * s2, va.w * c3 - vb.w * s3);
    const float4 rb = make_float4(va.x * s0 + vb.x * c0, va.y * s1 + vb.y * c1,
                                  va.z * s2 + vb.z * c2, va.w * s3 + vb.w * c3);
    va = ra;
    vb = rb;
  }
  if (is_query) {
    float* dst = a.query + (size_t)row * a.q_stride + (size_t)h * a.head_dim;
    st4(dst + 4 * lane, va);
    st4(dst + half + 4 * lane, vb);
  } else {
    const uint32_t slot = p % (uint32_t)a.slots;
    uint16_t* cache = (is_value ? a.value_cache : a.key_cache) +
                      ((size_t)slot * a.kv_heads + kv) * a.head_dim;
    ushort4 pa, pb;
    pa.x = f16_pack(va.x); pa.y = f16_pack(va.y); pa.z = f16_pack(va.z); pa.w = f16_pack(va.w);
    pb.x = f16_pack(vb.x); pb.y = f16_pack(vb.y); pb.z = f16_pack(vb.z); pb.w = f16_pack(vb.w);
    *reinterpret_cast<ushort4*>(cache + 4 * lane) = pa;
    *reinterpret_cast<ushort4*>(cache + half + 4 * lane) = pb;
  }
}

// ---- attention (attention.wgsl:95-438) -------------------------------------
// Workgroup (chunk slot cs, row): the row's chunk earliest/64 + cs, from an
// empty state over 8-key tiles (the first from the tile holding the earliest
// key), every query head of one key-value head; the chunk's unnormalized
// output and its (m, l, live) go to the partial buffers. A second kernel
// folds each row's chunks in order and divides (attention.wgsl:403-438). The
// result is the reference's whether its step split or not.
constexpr int kAttnThreads = 256;
constexpr int kKStride = 264;  // halves a staged key row: 256 + 8 of padding

struct Fold {
  float a, b, m;
};
__device__ __forceinline__ Fold fold_factors(bool live, float m, bool chunk_live,
                                             float chunk_max) {
  if (!chunk_live) return {1.0f, 0.0f, m};
  if (!live) return {0.0f, 1.0f, chunk_max};
  if (m == chunk_max) return {1.0f, 1.0f, m};
  if (m > chunk_max) return {1.0f, exp2f_fixed(chunk_max - m), m};
  return {exp2f_fixed(m - chunk_max), 1.0f, chunk_max};
}

// Specialized for head_dim 256 with 4 query heads a key-value head: the
// launcher refuses other shapes.
__global__ __launch_bounds__(kAttnThreads) void attention_chunk_kernel(
    const DevStep* __restrict__ step, AttentionArgs a) {
  constexpr int D = 256, QH = 4;
  __shared__ float qs[QH * D];
  __shared__ uint16_t ks[kChunkKeys * kKStride];
  __shared__ uint16_t vs[kChunkKeys * D];
  __shared__ float sc[QH * kChunkKeys];
  __shared__ float tile_a[QH * (kChunkKeys / kTileKeys)];
  __shared__ float chunk_stats[QH * 3];
  const int row = blockIdx.y;
  if (row >= (int)step->tokens) return;
  const int kvh = blockIdx.z;
  const int p = (int)step->position + row;
  const int earliest = p + 1 > a.window ? p + 1 - a.window : 0;
  const int c = earliest / kChunkKeys + (int)blockIdx.x;
  if (c > p / kChunkKeys) return;
  const int k_begin = max(c * kChunkKeys, earliest / kTileKeys * kTileKeys);
  const int k_end = min((c + 1) * kChunkKeys, p + 1);
  const int n_tiles = (k_end - k_begin + kTileKeys - 1) / kTileKeys;
  const int span = n_tiles * kTileKeys;
  const int t = threadIdx.x;

  // Queries of this key-value head, scaled into log2 units.
  for (int i = t; i < QH * D; i += kAttnThreads) {
    const int h = kvh * QH + i / D;
    qs[i] = a.query[(size_t)row * a.q_stride + (size_t)h * D + (i % D)] * a.scale_log2e;
  }
  // The chunk's key and value rows as stored, 8 halves at a time; value
  // rows past k_end staged as zeros (attention.wgsl:253-274).
  for (int i = t; i < span * (D / 8); i += kAttnThreads) {
    const int jj = i / (D / 8), w8 = i % (D / 8);
    const int j = k_begin + jj;
    uint4 kw = make_uint4(0, 0, 0, 0), vw = kw;
    if (j < k_end) {
      const size_t at = ((size_t)(j % a.slots) * a.kv_heads + kvh) * D + 8 * w8;
      kw = *reinterpret_cast<const uint4*>(a.key_cache + at);
      vw = *reinterpret_cast<const uint4*>(a.value_cache + at);
    }
    *reinterpret_cast<uint4*>(ks + jj * kKStride + 8 * w8) = kw;
    *reinterpret_cast<uint4*>(vs + jj * D + 8 * w8) = vw;
  }
  __syncthreads();

  // Scores: lane (head h, key jj), a dot of d by vec4s in order from zero.
  {
    const int h = t / kChunkKeys, jj = t % kChunkKeys;
    const int j = k_begin + jj;
    const bool live = jj < span && j < k_end && j <= p && j + a.window > p;
    float s = 0.0f;
    if (live) {
      const float* q = qs + h * D;
      const uint16_t* kr = ks + jj * kKStride;
      for (int w = 0; w < D / 4; ++w) {
        const ushort4 k4 = *reinterpret_cast<const ushort4*>(kr + 4 * w);
        s += dot4(q[4 * w], q[4 * w + 1], q[4 * w + 2], q[4 * w + 3], f16_unpack(k4.x),
                  f16_unpack(k4.y), f16_unpack(k4.z), f16_unpack(k4.w));
      }
    }
    sc[h * kChunkKeys + jj] = s;
  }
  __syncthreads();

  // The online softmax over the tiles in order, one lane a head
  // (attention.wgsl:304-340): sc becomes the weights e.
  if (t < QH) {
    const int h = t;
    bool chunk_live = false;
    float cm = 0.0f, cl = 0.0f;
    for (int tile = 0; tile < n_tiles; ++tile) {
      float top_tile = 0.0f;
      bool seen = false;
      bool live[kTileKeys];
      for (int b = 0; b < kTileKeys; ++b) {
        const int j = k_begin + tile * kTileKeys + b;
        live[b] = j < k_end && j <= p && j + a.window > p;
        if (live[b]) {
          const float s = sc[h * kChunkKeys + tile * kTileKeys + b];
          top_tile = seen ? __builtin_fmaxf(top_tile, s) : s;
          seen = true;
        }
      }
      float alpha = 1.0f;
      if (seen) {
        const float old = chunk_live ? cm : top_tile;
        chunk_live = true;
        const float top = __builtin_fmaxf(old, top_tile);
        alpha = old == top ? 1.0f : exp2f_fixed(old - top);
        float sum = 0.0f;
        for (int b = 0; b < kTileKeys; ++b) {
          float e = 0.0f;
          if (live[b]) e = exp2f_fixed(sc[h * kChunkKeys + tile * kTileKeys + b] - top);
          sc[h * kChunkKeys + tile * kTileKeys + b] = e;
          sum += e;
        }
        cl = cl * alpha + sum;
        cm = top;
      } else {
        for (int b = 0; b < kTileKeys; ++b) sc[h * kChunkKeys + tile * kTileKeys + b] = 0.0f;
      }
      tile_a[h * (kChunkKeys / kTileKeys) + tile] = alpha;
    }
    chunk_stats[h * 3 + 0] = cm;
    chunk_stats[h * 3 + 1] = cl;
    chunk_stats[h * 3 + 2] = chunk_live ? 1.0f : 0.0f;
  }
  __syncthreads();

  // O = O * alpha + sum_b e_b v_b per tile, lane (head, 4 dimensions).
  {
    const int h = t / 64, e0 = (t % 64) * 4;
    float o0 = 0.f, o1 = 0.f, o2 = 0.f, o3 = 0.f;
    for (int tile = 0; tile < n_tiles; ++tile) {
      const float alpha = tile_a[h * (kChunkKeys / kTileKeys) + tile];
      o0 = o0 * alpha; o1 = o1 * alpha; o2 = o2 * alpha; o3 = o3 * alpha;
      for (int b = 0; b < kTileKeys; ++b) {
        const int jj = tile * kTileKeys + b;
        const float e = sc[h * kChunkKeys + jj];
        const ushort4 v4 = *reinterpret_cast<const ushort4*>(vs + jj * D + e0);
        o0 = o0 + e * f16_unpack(v4.x);
        o1 = o1 + e * f16_unpack(v4.y);
        o2 = o2 + e * f16_unpack(v4.z);
        o3 = o3 + e * f16_unpack(v4.w);
      }
    }
    const size_t slot = ((size_t)row * a.max_chunks + blockIdx.x) * a.query_heads + kvh * QH + h;
    st4(a.partials + slot * D + e0, make_float4(o0, o1, o2, o3));
    if ((t % 64) == 0) {
      st4(a.stats + slot * 4, make_float4(chunk_stats[h * 3], chunk_stats[h * 3 + 1],
                                          chunk_stats[h * 3 + 2], 0.0f));
    }
  }
}

// The fold of a row's chunks in order, then o / l (attention.wgsl:403-438).
__global__ __launch_bounds__(256) void attention_combine_kernel(
    const DevStep* __restrict__ step, AttentionArgs a) {
  constexpr int D = 256;
  const int row = blockIdx.x;
  if (row >= (int)step->tokens) return;
  const int h = blockIdx.y * 4 + threadIdx.x / 64;
  if (h >= a.query_heads) return;
  const int e0 = (threadIdx.x % 64) * 4;
  const int p = (int)step->position + row;
  const int earliest = p + 1 > a.window ? p + 1 - a.window : 0;
  const int count = p / kChunkKeys - earliest / kChunkKeys + 1;
  bool live = false;
  float m = 0.0f, l = 0.0f;
  float o0 = 0.f, o1 = 0.f, o2 = 0.f, o3 = 0.f;
  for (int cs = 0; cs < count; ++cs) {
    const size_t slot = ((size_t)row * a.max_chunks + cs) * a.query_heads + h;
    const float4 st = ld4(a.stats + slot * 4);
    const bool chunk_live = st.z != 0.0f;
    const Fold f = fold_factors(live, m, chunk_live, st.x);
    l = l * f.a + st.y * f.b;
    const float4 po = ld4(a.partials + slot * D + e0);
    o0 = o0 * f.a + po.x * f.b;
    o1 = o1 * f.a + po.y * f.b;
    o2 = o2 * f.a + po.z * f.b;
    o3 = o3 * f.a + po.w * f.b;
    m = f.m;
    live = live || chunk_live;
  }
  float4 out = make_float4(0.f, 0.f, 0.f, 0.f);
  if (live) out = make_float4(o0 / l, o1 / l, o2 / l, o3 / l);
  st4(a.out + ((size_t)row * a.query_heads + h) * D + e0, out);
}

// ---- gather (gather.wgsl:25-48) ---------------------------------------------
__global__ __launch_bounds__(256) void gather_kernel(const DevStep* __restrict__ step,
                                                     Q4Matrix table,
                                                     const uint32_t* __restrict__ sampled,
                                                     float* __restrict__ hidden, float scale) {
  const int row = blockIdx.x;
  if (row >= (int)step->tokens) return;
  const uint32_t token = step->fed ? sampled[0] : step->ids[row];
  if (token >= (uint32_t)table.rows) return;
  const int groups = table.cols / 32;
  for (int i = threadIdx.x; i < table.cols; i += blockDim.x) {
    const size_t blk = (size_t)token * groups + i / 32;
    const int j = i % 32;
    const uint8_t byte = table.codes[blk * 16 + (j & 15)];
    const uint32_t q = j < 16 ? (byte & 0xFu) : (uint32_t)(byte >> 4);
    const float d = (float)__builtin_bit_cast(_Float16, table.scales[blk]);
    hidden[(size_t)row * table.cols + i] = fmaf_((float)q, d, -8.0f * d) * scale;
  }
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
  const uint32_t position = step->position + (uint32_t)row;
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

hipError_t launch_attention(hipStream_t s, const DevStep* step,
                            const AttentionArgs& a, int max_tokens) {
  if (a.head_dim != 256 || a.query_heads != 4 * a.kv_heads) return hipErrorInvalidValue;
  hipLaunchKernelGGL(attention_chunk_kernel, dim3(a.max_chunks, max_tokens, a.kv_heads),
                     dim3(kAttnThreads), 0, s, step, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(attention_combine_kernel, dim3(max_tokens, (a.query_heads + 3) / 4),
                     dim3(256), 0, s, step, a);
  return hipGetLastError();
}

hipError_t launch_gather(hipStream_t s, const DevStep* step, Q4Matrix table,
                         const uint32_t* sampled, float* hidden, float scale,
                         int max_tokens) {
  hipLaunchKernelGGL(gather_kernel, dim3(max_tokens), dim3(256), 0, s, step, table, sampled,
                     hidden, scale);
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
