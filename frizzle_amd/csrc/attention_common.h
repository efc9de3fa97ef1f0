// Attention over the F16 KV cache in 64-key chunks fixed by position
// (attention.wgsl:95-438), for Gemma-3's shape: d = 256, 4 query heads on
// one key-value head. A chunk's state (m, l, O) is computed from empty over
// its 8-key tiles in order; a row's chunk states are folded in chunk order
// and O divided by l. The same bits come out whether a step's chunks run in
// one workgroup or many (the reference's split): every chunk starts empty and
// the fold is one sequential pass.
//
// The kernels keep the reference's tile recursion exactly but run its
// independent parts in parallel: each key's score is the chain s +=
// dot(q_w, k_w) over the head's 64 vec4s; a tile's maximum is a max
// (order-free); each tile's running maximum, rescale factor and every
// exponential follow from those maxima; only the tile sums (8 ordered adds
// each), the running sum l over the tiles, and each output dimension's chain
// over the chunk's keys stay sequential.

#pragma once

#include "kernels.h"
#include "numerics.h"
#include "rope_common.h"

namespace frz {
namespace attn {

constexpr int D = 256;
constexpr int QH = 4;
constexpr int kThreads = 256;                             // a workgroup: 4 waves
constexpr int kTiles = kChunkKeys / kTileKeys;            // 8
constexpr int kKeyLanes = kThreads / kChunkKeys;          // 4 lanes a key (one-head kernels)
constexpr int kKeyLoads = D / kKeyLanes / 8;              // uint4s of its key row a lane holds

typedef _Float16 half2v __attribute__((ext_vector_type(2)));

// -0 in a register the compiler does not see into. fma(x, h, -0) is the
// product x h rounded once, the sign of a zero product kept (x h + -0 is
// x h for every x h, zeros included), and with h a half it stays one mixed
// fma instead of a conversion and a multiply.
__device__ __forceinline__ float negative_zero() {
  float z;
  asm("v_mov_b32 %0, 0x80000000" : "=v"(z));
  return z;
}

// dot4 of q with the four halves of words w0 (low, high) and w1: each
// product rounded, added ((p0 + p1) + p2) + p3.
__device__ __forceinline__ float dot4_halves(float4 q, uint32_t w0, uint32_t w1, float nz) {
  const half2v a = __builtin_bit_cast(half2v, w0), b = __builtin_bit_cast(half2v, w1);
  const float p0 = __builtin_fmaf(q.x, (float)a.x, nz);
  const float p1 = __builtin_fmaf(q.y, (float)a.y, nz);
  const float p2 = __builtin_fmaf(q.z, (float)b.x, nz);
  const float p3 = __builtin_fmaf(q.w, (float)b.y, nz);
  return ((p0 + p1) + p2) + p3;
}

// Orders a wave's LDS accesses around it: a wave's LDS instructions execute
// in program order; this keeps the compiler from moving them.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

struct Fold {
  float a, b, m;
};
// attention.wgsl:135-151.
__device__ __forceinline__ Fold fold_factors(bool live, float m, bool chunk_live,
                                             float chunk_max) {
  if (!chunk_live) return {1.0f, 0.0f, m};
  if (!live) return {0.0f, 1.0f, chunk_max};
  if (m == chunk_max) return {1.0f, 1.0f, m};
  if (m > chunk_max) return {1.0f, exp2f_fixed(chunk_max - m), m};
  return {exp2f_fixed(m - chunk_max), 1.0f, chunk_max};
}

struct ChunkRange {
  int earliest, count, c, k_begin, k_end, n_tiles;
};
__device__ __forceinline__ ChunkRange chunk_range(int p, int window, int cs) {
  ChunkRange r;
  r.earliest = p + 1 > window ? p + 1 - window : 0;
  r.count = p / kChunkKeys - r.earliest / kChunkKeys + 1;
  r.c = r.earliest / kChunkKeys + cs;
  r.k_begin = max(r.c * kChunkKeys, r.earliest / kTileKeys * kTileKeys);
  r.k_end = min((r.c + 1) * kChunkKeys, p + 1);
  r.n_tiles = (r.k_end - r.k_begin + kTileKeys - 1) / kTileKeys;
  return r;
}

// Lane UU of the calling lane's quad.
template <int UU>
__device__ __forceinline__ float quad_lane(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), UU * 0x55,
                                                            0xF, 0xF, true));
}

}  // namespace attn
}  // namespace frz
