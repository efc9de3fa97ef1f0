// The decode attention kernel: one token's QK-norm, rope and KV append
// fused with its attention over the cache (the chunk arithmetic is in
// attention_common.h).

#include "attention_common.h"

namespace frz {
namespace {
using namespace attn;

// ---- decode: rope + append + chunk + fold ------------------------------------
__global__ __launch_bounds__(kThreads) void attention_decode_kernel(
    const DevStep* __restrict__ step, DecodeAttentionArgs a) {
  __shared__ ChunkShared S;
  __shared__ float cosines[D / 2], sines[D / 2];
  __shared__ float red[256];
  __shared__ __align__(16) uint16_t knew[D];
  __shared__ __align__(16) uint16_t vnew[D];
  __shared__ int is_last;
  const int p = (int)step->position;
  const ChunkRange r = chunk_range(p, a.window, blockIdx.x);
  if ((int)blockIdx.x >= r.count) return;
  const bool holds_p = r.c == p / kChunkKeys;
  const int own = holds_p ? p : -1;
  const int t = threadIdx.x;
  // Heads: 4 query heads, then the key head, then the value head; 32 lanes
  // each (rope.wgsl:97-118). Key and value only where this chunk holds p.
  // Their loads go first, the cached rows' after, so the rope waits only for
  // the former while the latter are in flight.
  const int h = t >> 5, lane = t & 31;
  const bool active = t < 192 && (h < QH || holds_p);
  float4 va = make_float4(0.f, 0.f, 0.f, 0.f), vb = va;
  if (active) {
    const float* src = a.qkv + h * D;  // q heads, then k at 4 D, v at 5 D
    va = ld4f(src + 4 * lane);
    vb = ld4f(src + D / 2 + 4 * lane);
  }
  StageRegs R;
  stage_load(R, a.key_cache, a.value_cache, a.slots, r, own);
  rope_angles(a.turns, (uint32_t)p, D / 2, cosines, sines, t, kThreads);
  if (t < 256) red[t] = rope_lane_squares(va, vb);
  __syncthreads();
  for (int stride = 16; stride > 0; stride >>= 1) {
    if (active && lane < stride) red[t] = red[t] + red[t + stride];
    __syncthreads();
  }
  stage_store(S, R, r, own);
  if (active) {
    if (h <= QH) {
      rope_norm_rotate(va, vb, red[t - lane], D, a.epsilon, h < QH ? a.query_gain : a.key_gain,
                       lane, cosines, sines);
    }
    if (h < QH) {
      float* q = S.q + h * D;
      const float sc = a.scale_log2e;
      q[4 * lane] = va.x * sc; q[4 * lane + 1] = va.y * sc;
      q[4 * lane + 2] = va.z * sc; q[4 * lane + 3] = va.w * sc;
      q[D / 2 + 4 * lane] = vb.x * sc; q[D / 2 + 4 * lane + 1] = vb.y * sc;
      q[D / 2 + 4 * lane + 2] = vb.z * sc; q[D / 2 + 4 * lane + 3] = vb.w * sc;
    } else {
      uint16_t* dst = h == QH ? knew : vnew;
      const ushort4 pa = pack4_f16(va), pb = pack4_f16(vb);
      *reinterpret_cast<ushort4*>(dst + 4 * lane) = pa;
      *reinterpret_cast<ushort4*>(dst + D / 2 + 4 * lane) = pb;
      uint16_t* cache = (h == QH ? a.key_cache : a.value_cache) + (size_t)(p % a.slots) * D;
      *reinterpret_cast<ushort4*>(cache + 4 * lane) = pa;
      *reinterpret_cast<ushort4*>(cache + D / 2 + 4 * lane) = pb;
    }
  }
  __syncthreads();
  if (holds_p && t < D / 8) stage_put(S, p - r.k_begin, t, *reinterpret_cast<const uint4*>(knew + 8 * t),
                                      *reinterpret_cast<const uint4*>(vnew + 8 * t));
  __syncthreads();
  chunk_state<true>(S, p, a.window, r, a.partials + (size_t)blockIdx.x * QH * D,
                    a.stats + (size_t)blockIdx.x * QH * 4);
  // Arrival: this thread's coherent stores complete, then one count.
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (t == 0) {
    const uint32_t before =
        __hip_atomic_fetch_add(a.counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    is_last = before == (uint32_t)(r.count - 1);
  }
  __syncthreads();
  if (!is_last) return;
  a.out[t] = fold_chunks<true>(a.partials, a.stats, r.count);
  if (t == 0) __hip_atomic_store(a.counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace

hipError_t launch_attention_decode(hipStream_t s, const DevStep* step,
                                   const DecodeAttentionArgs& a) {
  if (a.head_dim != D || a.query_heads != QH || a.kv_heads != 1) return hipErrorInvalidValue;
  hipLaunchKernelGGL(attention_decode_kernel, dim3(a.max_chunks), dim3(kThreads), 0, s, step, a);
  return hipGetLastError();
}

}  // namespace frz
