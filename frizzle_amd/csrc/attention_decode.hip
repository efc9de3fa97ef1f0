// The decode attention kernel: one token's QK-norm, rope and KV append
// (rope.wgsl:51-138) fused with its attention over the cache; a workgroup
// per (chunk, head). Only the chunk holding the token's own position needs
// its key and value: that chunk's workgroups compute them (all four heads
// redundantly, head 0 also appends them to the cache). The chunk states are
// folded by the next launch (the O product's prologue, or the fold kernel).

#include "attention_common.h"

namespace frz {
namespace {
using namespace attn;

__global__ __launch_bounds__(kThreads) void attention_decode_kernel(
    const DevStep* __restrict__ step, DecodeAttentionArgs a) {
  __shared__ ChunkShared S;
  __shared__ float cosines[D / 2], sines[D / 2];
  const int h = blockIdx.y, t = threadIdx.x, row = blockIdx.z;
  if (row > 0) {  // a variants step's row: its own token and caches
    a.qkv += (size_t)row * a.qkv_stride;
    a.key_cache += (size_t)row * a.cache_stride;
    a.value_cache += (size_t)row * a.cache_stride;
  }
  // Rope lanes, 32 a head: the query head h, then the key and the value.
  // Their loads and the turns go first (none depends on the position), the
  // cached rows' after, so the rope waits only for the former.
  const int role = t >> 5, lane = t & 31;
  const float turn = a.turns[t & (D / 2 - 1)];
  const float* src = a.qkv + (role == 0 || role > 2 ? h : QH + role - 1) * D;
  float4 va = ld4f(src + 4 * lane), vb = ld4f(src + D / 2 + 4 * lane);
  const float* gain = role == 1 ? a.key_gain : a.query_gain;
  const float4 ga = ld4f(gain + 4 * lane), gb = ld4f(gain + D / 2 + 4 * lane);
  __asm__ volatile("" ::: "memory");  // keep these loads ahead of the position's
  const int p = (int)step->position;
  const ChunkRange r = chunk_range(p, a.window, blockIdx.x);
  if ((int)blockIdx.x >= r.count) return;
  // Key and value are needed only where this chunk holds p.
  const bool holds_p = r.c == p / kChunkKeys;
  const int own = holds_p ? p : -1;
  const bool active = role == 0 || (holds_p && role <= 2);
  uint4 kr[kKeyLoads], vr[kValueLoads];
  key_load(kr, a.key_cache, a.slots, r, own);
  value_load(vr, a.value_cache, a.slots, r, own);
  if (t < D / 2) rope_angle(turn, (uint32_t)p, &sines[t], &cosines[t]);
  if (!active) va = vb = make_float4(0.f, 0.f, 0.f, 0.f);
  // The head's sum of squares: the halving tree over its 32 lanes.
  // Each 32-lane group's lane 0 ends with the total (level 16 by a swizzle
  // within the group, lane l ^ 16; levels 8 to 1 within a row by DPP), which
  // goes to the group's lanes.
  float sum = rope_lane_squares(va, vb);
  sum = sum + __builtin_bit_cast(float, other_row(__builtin_bit_cast(int, sum)));
  sum = sum + row_shl<8>(sum);
  sum = sum + row_shl<4>(sum);
  sum = sum + row_shl<2>(sum);
  sum = sum + row_shl<1>(sum);
  {
    const int b = __builtin_bit_cast(int, sum);
    const int lo = __builtin_amdgcn_readlane(b, 0), hi = __builtin_amdgcn_readlane(b, 32);
    sum = __builtin_bit_cast(float, (t & 32) ? hi : lo);
  }
  __syncthreads();
  if (active) {
    if (role <= 1) {
      rope_norm_rotate(va, vb, sum, D, a.epsilon, ga, gb, lane, cosines, sines);
    }
    if (role == 0) {
      const float sc = a.scale_log2e;
      *reinterpret_cast<float4*>(S.q + 4 * lane) =
          make_float4(va.x * sc, va.y * sc, va.z * sc, va.w * sc);
      *reinterpret_cast<float4*>(S.q + D / 2 + 4 * lane) =
          make_float4(vb.x * sc, vb.y * sc, vb.z * sc, vb.w * sc);
    } else {
      const ushort4 pa = pack4_f16(va), pb = pack4_f16(vb);
      uint16_t* row = role == 1 ? S.knew : S.v + (p - r.k_begin) * D;
      *reinterpret_cast<ushort4*>(row + 4 * lane) = pa;
      *reinterpret_cast<ushort4*>(row + D / 2 + 4 * lane) = pb;
      if (h == 0) {
        uint16_t* cache = (role == 1 ? a.key_cache : a.value_cache) + (size_t)(p % a.slots) * D;
        *reinterpret_cast<ushort4*>(cache + 4 * lane) = pa;
        *reinterpret_cast<ushort4*>(cache + D / 2 + 4 * lane) = pb;
      }
    }
  }
  value_store(S, vr, r, own);
  __syncthreads();
  if (r.k_begin + (t >> 2) == own) {
    const uint4* src = reinterpret_cast<const uint4*>(S.knew + 64 * (t & 3));
#pragma unroll
    for (int m = 0; m < kKeyLoads; ++m) kr[m] = src[m];
  }
  const size_t slot = ((size_t)row * a.max_chunks + blockIdx.x) * QH + h;
  chunk_state<true>(S, kr, p, a.window, r, a.partials + slot * D, a.stats + slot * 4);
}

}  // namespace

hipError_t launch_attention_decode(hipStream_t s, const DevStep* step,
                                   const DecodeAttentionArgs& a, int rows) {
  if (a.head_dim != D || a.query_heads != QH || a.kv_heads != 1 || rows < 1)
    return hipErrorInvalidValue;
  hipLaunchKernelGGL(attention_decode_kernel, dim3(a.max_chunks, QH, rows), dim3(kThreads), 0, s,
                     step, a);
  return hipGetLastError();
}

}  // namespace frz
