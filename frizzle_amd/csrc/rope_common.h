// QK-norm and rotation of one head's values, shared by the rope kernel and
// the decode attention kernel (rope.wgsl:51-138). A head of d values is d/8
// lanes; lane l holds dimensions 4l..4l+3 (a) and d/2+4l..d/2+4l+3 (b).
#pragma once

#include "numerics.h"

namespace frz {

// Each pair's cos and sin at position p into LDS tables (rope.wgsl:122-129):
// t = f32(p) * turns_k, angle = 2 pi (t - round(t)).
__device__ __forceinline__ void rope_angle(float turn, uint32_t p, float* sine, float* cosine) {
  const float tt = (float)p * turn;
  const float angle = 6.283185307179586f * (tt - rint_(tt));
  sincos_fixed(angle, sine, cosine);
}

__device__ __forceinline__ void rope_angles(const float* __restrict__ turns, uint32_t p,
                                            int half, float* cosines, float* sines,
                                            int t, int threads) {
  for (int k = t; k < half; k += threads) rope_angle(turns[k], p, &sines[k], &cosines[k]);
}

__device__ __forceinline__ float4 ld4f(const float* p) {
  return *reinterpret_cast<const float4*>(p);
}

__device__ __forceinline__ float dot4f(float4 a, float4 b) {
  return dot4(a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w);
}

// A lane's share of its head's sum of squares: dot(a, a) + dot(b, b).
__device__ __forceinline__ float rope_lane_squares(float4 a, float4 b) {
  return dot4f(a, a) + dot4f(b, b);
}

// The normalization: x r g for r = 1/sqrt(sum / d + eps), the gain's values
// for the lane ga at 4 lane, gb at d/2 + 4 lane.
__device__ __forceinline__ void rope_normalize(float4& a, float4& b, float sum, int head_dim,
                                               float epsilon, float4 ga, float4 gb) {
  const float r = inverse_sqrt(sum / (float)head_dim + epsilon);
  a.x = (a.x * r) * ga.x; a.y = (a.y * r) * ga.y;
  a.z = (a.z * r) * ga.z; a.w = (a.w * r) * ga.w;
  b.x = (b.x * r) * gb.x; b.y = (b.y * r) * gb.y;
  b.z = (b.z * r) * gb.z; b.w = (b.w * r) * gb.w;
}

// The turn of pairs (k, k + d/2), k = 4 lane .. 4 lane + 3, by their angles:
// x' = x c - y s, y' = x s + y c.
__device__ __forceinline__ void rope_rotate(float4& a, float4& b, int lane, const float* cosines,
                                            const float* sines) {
  const int k = 4 * lane;
  const float c0 = cosines[k], c1 = cosines[k + 1], c2 = cosines[k + 2], c3 = cosines[k + 3];
  const float s0 = sines[k], s1 = sines[k + 1], s2 = sines[k + 2], s3 = sines[k + 3];
  const float4 ra = make_float4(a.x * c0 - b.x * s0, a.y * c1 - b.y * s1,
                                a.z * c2 - b.z * s2, a.w * c3 - b.w * s3);
  const float4 rb = make_float4(a.x * s0 + b.x * c0, a.y * s1 + b.y * c1,
                                a.z * s2 + b.z * c2, a.w * s3 + b.w * c3);
  a = ra;
  b = rb;
}

// Normalize, then turn.
__device__ __forceinline__ void rope_norm_rotate(float4& a, float4& b, float sum, int head_dim,
                                                 float epsilon, float4 ga, float4 gb, int lane,
                                                 const float* cosines, const float* sines) {
  rope_normalize(a, b, sum, head_dim, epsilon, ga, gb);
  rope_rotate(a, b, lane, cosines, sines);
}

__device__ __forceinline__ void rope_norm_rotate(float4& a, float4& b, float sum, int head_dim,
                                                 float epsilon, const float* __restrict__ gain,
                                                 int lane, const float* cosines,
                                                 const float* sines) {
  const int half = head_dim / 2;
  rope_norm_rotate(a, b, sum, head_dim, epsilon, ld4f(gain + 4 * lane),
                   ld4f(gain + half + 4 * lane), lane, cosines, sines);
}

__device__ __forceinline__ ushort4 pack4_f16(float4 v) {
  ushort4 o;
  o.x = f16_pack_device(v.x);
  o.y = f16_pack_device(v.y);
  o.z = f16_pack_device(v.z);
  o.w = f16_pack_device(v.w);
  return o;
}

}  // namespace frz
