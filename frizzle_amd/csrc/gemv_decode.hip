// Decode (one token) Q4_0 products with their input row made in a prologue,
// so each layer runs its norms inside the products that read them:
//   the attention norm (and layer 0's embedding gather) before Q/K/V,
//   the attention fold (local layers) before O,
//   the feed-forward norm before gate/up (GELU and the pins after it).
//   the final norm before a Q4_0 head (the first workgroup also writes the
//     normed row).
// Every workgroup computes its input row itself, redundantly, with the
// reference's 256-invocation reduction tree (norm.wgsl:75-198), so every
// workgroup holds the same bits; the first also writes the new hidden row.
// Hidden rows ping-pong between two buffers, so no workgroup rewrites a row
// another is still reading.
//
// The products keep the reference's order of addition (matmul.h:88-97):
// range r of a row is groups floor(r G / 32) .. floor((r + 1) G / 32), its
// products chained by fma from zero; the 32 range sums add in order to a
// total from zero. Three lane layouts:
//   one row a half-wave, lane r range r: the total is a DPP chain across
//     the half-wave, with no LDS (the write products, K other than 1,152);
//   K = 1,152 (`pair`): 18 lanes a row, each exactly two groups, so no lane
//     idles through a second group; sums meet in LDS. Many rows (the
//     262,144-row head) take 8 tiles a workgroup (`gemv_pair_tiles_kernel`);
//   two rows a half-wave (the Q8_0 head, other K of the gated product): lane
//     r takes range (r + j) mod 32 of row j, which spreads each row's longer
//     ranges over different lanes; sums meet in LDS.
// A lane's plan (which groups, where each range sum goes) is fixed for the
// kernel; a tile only moves it by whole rows.
//
// Latency: a workgroup issues its input loads, then its weight loads, then
// makes the input row while the weights are in flight. Loads return in issue
// order, so every load is issued unconditionally (out-of-range indexes
// clamped, values unused) and the code stays straight-line: a wait for the
// input row is then a wait for its own loads only. Where the input of a
// lane's groups fits in registers it is read from LDS before the weights are
// waited for. Totals read all 32 sums before adding, so one LDS round trip
// precedes the serial adds.

#include "attention_common.h"
#include "kernels.h"
#include "numerics.h"

namespace frz {
namespace {

constexpr int kXStride = 36;     // a staged group of x: 32 floats + 4 of padding
constexpr int kPartStride = 33;  // a row's 32 range sums + 1 of padding
constexpr int kNormLanes = 256;  // the norm's reduction width
constexpr int kRedFloats = 512;  // two trees' 256 sums
constexpr int kNormMaxCols = 2 * 4 * kNormLanes;  // two vec4s a norm lane
constexpr int kFoldWidth = attn::QH * attn::D;    // the attention output a fold makes

// Chunks of 64 keys a position's window reaches (attention.wgsl:95-120).
__device__ __forceinline__ int window_chunks(const DevStep* __restrict__ step, int window) {
  return attn::chunk_range((int)step->position, window, 0).count;
}

__device__ __forceinline__ float half_to_float(uint16_t h) {
  return (float)__builtin_bit_cast(_Float16, h);
}

__device__ __forceinline__ float4 ld4(const float* p) {
  return *reinterpret_cast<const float4*>(p);
}

// Orders a wave's LDS accesses around it (a wave's LDS instructions execute
// in program order; this keeps the compiler from moving them).
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

typedef _Float16 half2v __attribute__((ext_vector_type(2)));

// One group's 32 products chained into acc, weights in order: the 16 low
// nibbles (code byte j's low nibble is weight j), then the 16 high nibbles.
// Weight j is (q_j - 8) d (q4_0.wgsl:71-83), formed exactly in one mixed
// fma whose half operand carries the nibble under the exponent of 1024:
//   a low nibble, masked in place, is the half 1024 + q, and
//     fma(1024 + q, d, -1032 d) = (q - 8) d;
//   a high nibble, masked in place, is 1024 + 16 q, and
//     fma(1024 + 16 q, d / 16, -72 d) = 64 d + q d - 72 d = (q - 8) d.
// Each is rounded once and exact, since (q - 8) d needs 15 bits; d / 16,
// -72 d and -1032 d are exact in single precision. One bitwise select makes
// two halves (bytes 0 and 2, or 1 and 3, of a word), so a word's 8 weights
// take 1 shift and 4 selects. `x(i)` is vec4 i of the group's input.
template <class X>
__device__ __forceinline__ float chain_q4_0(float acc, uint4 c, uint16_t dbits, X x) {
  const float d = (float)__builtin_bit_cast(_Float16, dbits);
  const float bias_lo = -1032.0f * d;
  const float d16 = d * 0.0625f;
  const float bias_hi = -72.0f * d;
  const uint32_t words[4] = {c.x, c.y, c.z, c.w};
  // The exponent bits come from a register the compiler cannot see into, so
  // that (s & mask) | (exp & ~mask) stays one bitfield insert.
  uint32_t kExp;
  asm("v_mov_b32 %0, 0x64006400" : "=v"(kExp));
  constexpr uint32_t kLo = 0x000F000Fu, kHi = 0x00F000F0u;
  half2v lo_a[4], lo_b[4], hi_a[4], hi_b[4];
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const uint32_t s = words[w], s8 = words[w] >> 8;
    lo_a[w] = __builtin_bit_cast(half2v, (s & kLo) | (kExp & ~kLo));    // weights 4w, 4w + 2
    lo_b[w] = __builtin_bit_cast(half2v, (s8 & kLo) | (kExp & ~kLo));   // 4w + 1, 4w + 3
    hi_a[w] = __builtin_bit_cast(half2v, (s & kHi) | (kExp & ~kHi));    // 4w + 16, 4w + 18
    hi_b[w] = __builtin_bit_cast(half2v, (s8 & kHi) | (kExp & ~kHi));   // 4w + 17, 4w + 19
  }
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const float4 v = x(w);
    acc = fmaf_(__builtin_fmaf((float)lo_a[w].x, d, bias_lo), v.x, acc);
    acc = fmaf_(__builtin_fmaf((float)lo_b[w].x, d, bias_lo), v.y, acc);
    acc = fmaf_(__builtin_fmaf((float)lo_a[w].y, d, bias_lo), v.z, acc);
    acc = fmaf_(__builtin_fmaf((float)lo_b[w].y, d, bias_lo), v.w, acc);
  }
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const float4 v = x(4 + w);
    acc = fmaf_(__builtin_fmaf((float)hi_a[w].x, d16, bias_hi), v.x, acc);
    acc = fmaf_(__builtin_fmaf((float)hi_b[w].x, d16, bias_hi), v.y, acc);
    acc = fmaf_(__builtin_fmaf((float)hi_a[w].y, d16, bias_hi), v.z, acc);
    acc = fmaf_(__builtin_fmaf((float)hi_b[w].y, d16, bias_hi), v.w, acc);
  }
  return acc;
}

// The group's input staged in LDS at xg.
__device__ __forceinline__ float chain_group(float acc, uint4 c, uint16_t dbits, const float* xg) {
  return chain_q4_0(acc, c, dbits, [xg](int i) { return ld4(xg + 4 * i); });
}

// The group's input held in registers.
__device__ __forceinline__ float chain_group(float acc, uint4 c, uint16_t dbits,
                                             const float4 (&xv)[8]) {
  return chain_q4_0(acc, c, dbits, [&xv](int i) { return xv[i]; });
}

// The in-order total of each half-wave's 32 lane values, ((0 + s0) + s1) ...
// + s31 (matmul.h:88-97), without LDS: step k moves every lane's running
// value one lane up (DPP wave_shr:1) and adds the lane's own, so after step
// k lane i holds ((0 + s[i-k]) + ...) + s[i]. Lanes 31 and 63 end with their
// half-waves' totals; the running value stays first operand, as in a serial
// sum.
__device__ __forceinline__ float half_wave_total(float s) {
  float t = 0.0f + s;
#pragma unroll
  for (int k = 1; k < 32; ++k) {
    const float prev = __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, t), 0x138, 0xF, 0xF, false));
    t = prev + s;
  }
  return t;
}

// Q8_0: weight k = qs[k] d (q8_0.wgsl:12-24), qs signed. A code flipped to
// u = qs + 128 sits under the exponent of f16 1024 as 1024 + u, and
// fma(1024 + u, d, -1152 d) = (u - 128) d = qs d, exact (19 bits at most).
__device__ __forceinline__ float chain_group_q8_0(float acc, uint4 c0, uint4 c1, uint16_t dbits,
                                                  const float* xg) {
  const _Float16 dh = __builtin_bit_cast(_Float16, dbits);
  const float bias = -1152.0f * (float)dh;
  const uint32_t words[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
  constexpr uint32_t kMask = 0x00FF00FFu;
  uint32_t kExp;
  asm("v_mov_b32 %0, 0x64006400" : "=v"(kExp));
#pragma unroll
  for (int w = 0; w < 8; ++w) {
    const float4 x = *reinterpret_cast<const float4*>(xg + 4 * w);
    const uint32_t s = words[w] ^ 0x80808080u;
    // a: bytes 0 and 2 of the word; b: bytes 1 and 3.
    const half2v a = __builtin_bit_cast(half2v, (s & kMask) | (kExp & ~kMask));
    const half2v b = __builtin_bit_cast(half2v, ((s >> 8) & kMask) | (kExp & ~kMask));
    acc = fmaf_(__builtin_fmaf((float)a.x, (float)dh, bias), x.x, acc);
    acc = fmaf_(__builtin_fmaf((float)b.x, (float)dh, bias), x.y, acc);
    acc = fmaf_(__builtin_fmaf((float)a.y, (float)dh, bias), x.z, acc);
    acc = fmaf_(__builtin_fmaf((float)b.y, (float)dh, bias), x.w, acc);
  }
  return acc;
}

// Q4_1: weight = q d + m (q4_1.wgsl:12-25). fma(1024 + q, d, -1024 d) = q d
// exactly; the one rounding is that of adding m, as in the reference.
__device__ __forceinline__ float chain_group_q4_1(float acc, uint4 c, uint32_t dm,
                                                  const float* xg) {
  const _Float16 dh = __builtin_bit_cast(_Float16, (uint16_t)(dm & 0xFFFFu));
  const float m = (float)__builtin_bit_cast(_Float16, (uint16_t)(dm >> 16));
  const float bias = -1024.0f * (float)dh;
  const uint32_t words[4] = {c.x, c.y, c.z, c.w};
  constexpr uint32_t kMask = 0x000F000Fu;
  uint32_t kExp;
  asm("v_mov_b32 %0, 0x64006400" : "=v"(kExp));
#pragma unroll
  for (int hi = 0; hi < 2; ++hi) {
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float4 x = *reinterpret_cast<const float4*>(xg + 16 * hi + 4 * w);
      const uint32_t s = words[w] >> (4 * hi);
      const half2v a = __builtin_bit_cast(half2v, (s & kMask) | (kExp & ~kMask));
      const half2v b = __builtin_bit_cast(half2v, ((s >> 8) & kMask) | (kExp & ~kMask));
      acc = fmaf_(__builtin_fmaf((float)a.x, (float)dh, bias) + m, x.x, acc);
      acc = fmaf_(__builtin_fmaf((float)b.x, (float)dh, bias) + m, x.y, acc);
      acc = fmaf_(__builtin_fmaf((float)a.y, (float)dh, bias) + m, x.z, acc);
      acc = fmaf_(__builtin_fmaf((float)b.y, (float)dh, bias) + m, x.w, acc);
    }
  }
  return acc;
}

// ---- the input row ------------------------------------------------------------
// T threads (128 to 1,024). With N = min(T, 256) norm threads, norm lane
// t + k N (k < 256 / N) belongs to thread t and holds vec4s lane and
// lane + 256, in slot 2 k + m. Threads past 256 hold no norm lane.
template <int T>
struct Shape {
  static_assert(T == 128 || T == 256 || T == 512 || T == 1024, "two to sixteen waves");
  static constexpr int kNormThreads = T < kNormLanes ? T : kNormLanes;
  static constexpr int kLanesPer = kNormLanes / kNormThreads;
  static constexpr int kFoldVec4s = T <= kNormLanes ? kFoldWidth / 4 / T : 1;
};

template <int T>
__device__ __forceinline__ int norm_vec4(int k, int m) {
  constexpr int N = Shape<T>::kNormThreads;
  return (int)threadIdx.x + k * N + m * kNormLanes;
}

template <int T>
__device__ __forceinline__ bool norm_thread() {
  return (int)threadIdx.x < Shape<T>::kNormThreads;
}

// The norm's halving tree over its 256 lane sums (norm.wgsl:75-85). The
// levels above T add in registers; after one barrier every wave takes the
// remaining levels itself from LDS (levels 128 and 64 in registers, the last
// six across the wave), so every thread gets the total with no second
// barrier. `red` is 256 floats the call owns: a second tree uses another.

template <int T>
__device__ __forceinline__ float tree_total(float* red, const float (&lanes)[Shape<T>::kLanesPer]) {
  constexpr int LP = Shape<T>::kLanesPer;
  const int t = threadIdx.x, lane = t & 63;
  float v[LP];
#pragma unroll
  for (int k = 0; k < LP; ++k) v[k] = lanes[k];
#pragma unroll
  for (int width = LP; width > 1; width >>= 1) {
#pragma unroll
    for (int k = 0; k < width / 2; ++k) v[k] = v[k] + v[k + width / 2];
  }
  if (norm_thread<T>()) red[t] = v[0];  // the sum at level min(T, 256)
  __syncthreads();
  float s;
  if (T >= 256) {
    s = (red[lane] + red[lane + 128]) + (red[lane + 64] + red[lane + 192]);
  } else {
    s = red[lane] + red[lane + 64];
  }
  return wave_tree(s);
}

__device__ __forceinline__ void stage4(float* xs, int q, float4 v) {
  *reinterpret_cast<float4*>(xs + (q >> 3) * kXStride + 4 * (q & 7)) = v;
}

template <int T, int X4>
struct Prologue {
  static constexpr int S = 2 * Shape<T>::kLanesPer;
  float4 plain[X4];  // MODE 0: vec4s t + j T of x
  float4 v[S];       // hidden (MODE 1) or the embedding row (MODE 2)
  float4 y[S];       // the block output (MODE 1)
  float4 pg[S];      // its post-norm gain
  float4 g[S];       // the norm gain
  uint32_t word[S];
  uint16_t d[S];
  float4 st;                                                // MODE 3: a chunk state
  float4 po[kFoldPrologueChunks][Shape<T>::kFoldVec4s];     // MODE 3: the chunks' outputs
};

// Issues the input row's loads: MODE 0 a plain row x; 1 hidden, output and
// the gains; 2 the embedding of the step's token (gather.wgsl:25-48); 3 the
// chunk states.
template <int MODE, int T, int X4>
__device__ __forceinline__ void prologue_load(Prologue<T, X4>& P, const GemvInput& in,
                                              const DevStep* __restrict__ step, int width) {
  const int vec4s = width >> 2;
  if (MODE == 0) {
    // A slot past the row for the wave's first lane is past it for the whole
    // wave and is not loaded (the branch is uniform over the wave).
    const int wave_first = (int)threadIdx.x & ~63;
#pragma unroll
    for (int j = 0; j < X4; ++j) {
      if (wave_first + j * T >= vec4s) continue;
      P.plain[j] = ld4(in.x + 4 * min((int)threadIdx.x + j * T, vec4s - 1));
    }
    return;
  }
  if (MODE == 3) {
    // Every chunk state the prologue can fold is loaded, whatever the
    // window's count (the buffers hold kFoldPrologueChunks chunks; states
    // past the count are never used), so no load waits for the step's
    // position. Wave 0 holds the (chunk, head) statistics.
    if (threadIdx.x < 64)
      P.st = ld4(in.stats + 4 * min((int)threadIdx.x, kFoldPrologueChunks * attn::QH - 1));
#pragma unroll
    for (int c = 0; c < kFoldPrologueChunks; ++c) {
#pragma unroll
      for (int j = 0; j < Shape<T>::kFoldVec4s; ++j) {
        P.po[c][j] = ld4(in.partials + c * kFoldWidth + 4 * ((int)threadIdx.x + j * T));
      }
    }
    return;
  }
  // Past 256 threads, whole waves hold no norm lane and load nothing: the
  // loads skipped come before every other load, so no later wait counts
  // them.
  if (!norm_thread<T>()) return;
  uint32_t token = 0;
  if (MODE == 2) token = step->fed ? in.sampled[0] : step->ids[0];
  const int groups = width >> 5;
  // A slot past the row for the wave's first lane is past it for the whole
  // wave and is not loaded (the branch is uniform over the wave; at K =
  // 1,152 it halves a workgroup's prologue loads). The loads skipped come
  // after the ones kept and before the weights', so no wait counts them.
  const int wave_first = (int)threadIdx.x & ~63;
#pragma unroll
  for (int s = 0; s < Prologue<T, X4>::S; ++s) {
    if (norm_vec4<T>(s >> 1, s & 1) - ((int)threadIdx.x - wave_first) >= vec4s) continue;
    const int q = min(norm_vec4<T>(s >> 1, s & 1), vec4s - 1);
    if (MODE == 1) {
      P.v[s] = ld4(in.hidden + 4 * q);
      P.y[s] = ld4(in.output + 4 * q);
      P.pg[s] = ld4(in.post_gain + 4 * q);
    } else {
      // vec4 q is weights 4 (q % 8) .. + 3 of group q / 8: in Q4_0 nibbles of
      // word (q % 4) of the block's codes, in Q8_0 bytes of word q % 8.
      const size_t blk = (size_t)token * groups + (q >> 3);
      const size_t word = in.table.format == kQ8_0 ? blk * 8 + (q & 7) : blk * 4 + (q & 3);
      P.word[s] = reinterpret_cast<const uint32_t*>(in.table.codes)[word];
      P.d[s] = in.table.scales[blk];
    }
    P.g[s] = ld4(in.gain + 4 * q);
  }
}

__device__ __forceinline__ float squares4(float4 a) {
  return dot4(a.x, a.y, a.z, a.w, a.x, a.y, a.z, a.w);
}

// The attention output from its chunk states (attention.wgsl:403-438): the
// factors of chunk c for head h follow from the running maximum and
// liveness before it, which thread (c, h) replays; each thread then folds
// its vec4s' chains o = o a + po b (and the head's l) in chunk order, and
// stages o / l.
template <int T, int X4>
__device__ __forceinline__ void fold_prologue(float* xs, float* red, const Prologue<T, X4>& P,
                                              int count) {
  constexpr int QH = attn::QH;
  static_assert(6 * kFoldPrologueChunks * QH <= kRedFloats, "fold tables exceed the tree's LDS");
  static_assert(T <= kNormLanes, "the fold takes up to four waves");
  float4* st = reinterpret_cast<float4*>(red);  // [count][QH]
  float* fa = red + 4 * kFoldPrologueChunks * QH;
  float* fb = fa + kFoldPrologueChunks * QH;
  const int t = threadIdx.x;
  if (t < count * QH) st[t] = P.st;
  __syncthreads();
  if (t < count * QH) {
    const int c = t / QH, h = t % QH;
    // The head's states read at once, then the replay in registers.
    float4 sv[kFoldPrologueChunks];
#pragma unroll
    for (int b = 0; b < kFoldPrologueChunks; ++b) sv[b] = st[min(b, count - 1) * QH + h];
    bool live = false;
    float m = 0.0f;
#pragma unroll
    for (int b = 0; b < kFoldPrologueChunks; ++b) {
      if (b < c) {
        m = attn::fold_factors(live, m, sv[b].z != 0.0f, sv[b].x).m;
        live = live || sv[b].z != 0.0f;
      }
    }
    const attn::Fold f = attn::fold_factors(live, m, P.st.z != 0.0f, P.st.x);
    fa[t] = f.a;
    fb[t] = f.b;
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < Shape<T>::kFoldVec4s; ++j) {
    const int q = t + j * T, h = q / (attn::D / 4);
    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
    float l = 0.0f;
    bool live = false;
#pragma unroll
    for (int c = 0; c < kFoldPrologueChunks; ++c) {
      if (c < count) {
        const float a = fa[c * QH + h], b = fb[c * QH + h];
        const float4 s = st[c * QH + h], po = P.po[c][j];
        l = l * a + s.y * b;
        o.x = o.x * a + po.x * b;
        o.y = o.y * a + po.y * b;
        o.z = o.z * a + po.z * b;
        o.w = o.w * a + po.w * b;
        live = live || s.z != 0.0f;
      }
    }
    stage4(xs, q, live ? make_float4(o.x / l, o.y / l, o.z / l, o.w / l)
                       : make_float4(0.f, 0.f, 0.f, 0.f));
  }
}

// Makes the input row from the loads and stages it into xs.
template <int MODE, int T, int X4>
__device__ __forceinline__ void prologue_finish(float* xs, float* red, Prologue<T, X4>& P,
                                                const GemvInput& in,
                                                const DevStep* __restrict__ step, int width) {
  constexpr int LP = Shape<T>::kLanesPer, S = Prologue<T, X4>::S;
  const int vec4s = width >> 2;
  if (MODE == 0) {
#pragma unroll
    for (int j = 0; j < X4; ++j) {
      const int q = (int)threadIdx.x + j * T;
      if (q < vec4s) stage4(xs, q, P.plain[j]);
    }
    return;
  }
  if constexpr (MODE == 3) {
    fold_prologue<T, X4>(xs, red, P, window_chunks(step, in.window));
    return;
  }
  const float n = (float)width;
  float lanes[LP];
  if (MODE == 1) {
    // hidden + post-normed block output (norm.wgsl:120-160)
#pragma unroll
    for (int k = 0; k < LP; ++k) {
      lanes[k] = 0.0f;
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        if (norm_vec4<T>(k, m) < vec4s) lanes[k] = lanes[k] + squares4(P.y[2 * k + m]);
      }
    }
    const float ry = inverse_sqrt(tree_total<T>(red + kNormLanes, lanes) / n + in.epsilon);
#pragma unroll
    for (int s = 0; s < S; ++s) {
      if (norm_vec4<T>(s >> 1, s & 1) < vec4s) {
        float4& x = P.v[s];
        const float4 y = P.y[s], g = P.pg[s];
        x.x = x.x + ((y.x * ry) * g.x) * 1.0f;
        x.y = x.y + ((y.y * ry) * g.y) * 1.0f;
        x.z = x.z + ((y.z * ry) * g.z) * 1.0f;
        x.w = x.w + ((y.w * ry) * g.w) * 1.0f;
      }
    }
  } else {
    // weight j of the token's group, times the scale
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const int q = norm_vec4<T>(s >> 1, s & 1);
      if (q < vec4s) {
        const int shift = ((4 * q) & 31) < 16 ? 0 : 4;
        const float d = half_to_float(P.d[s]);
        float e[4];
        if (in.table.format == kQ8_0) {
#pragma unroll
          for (int b = 0; b < 4; ++b) {
            const float code = (float)(int8_t)(P.word[s] >> (8 * b));
            e[b] = (code * d) * in.scale;
          }
        } else {
#pragma unroll
          for (int b = 0; b < 4; ++b) {
            const float code = (float)((P.word[s] >> (8 * b + shift)) & 0xFu);
            e[b] = fmaf_(code, d, -8.0f * d) * in.scale;
          }
        }
        P.v[s] = make_float4(e[0], e[1], e[2], e[3]);
      }
    }
  }
  if (blockIdx.x == 0 && in.hidden_out && norm_thread<T>()) {
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const int q = norm_vec4<T>(s >> 1, s & 1);
      if (q < vec4s) *reinterpret_cast<float4*>(in.hidden_out + 4 * q) = P.v[s];
    }
  }
#pragma unroll
  for (int k = 0; k < LP; ++k) {
    lanes[k] = 0.0f;
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      if (norm_vec4<T>(k, m) < vec4s) lanes[k] = lanes[k] + squares4(P.v[2 * k + m]);
    }
  }
  const float r = inverse_sqrt(tree_total<T>(red, lanes) / n + in.epsilon);
#pragma unroll
  for (int s = 0; s < S; ++s) {
    const int q = norm_vec4<T>(s >> 1, s & 1);
    if (q < vec4s && norm_thread<T>()) {
      const float4 x = P.v[s], g = P.g[s];
      const float4 o = make_float4((x.x * r) * g.x, (x.y * r) * g.y, (x.z * r) * g.z,
                                   (x.w * r) * g.w);
      stage4(xs, q, o);
      if (blockIdx.x == 0 && in.normed_out) *reinterpret_cast<float4*>(in.normed_out + 4 * q) = o;
    }
  }
}

// ---- a lane's plan and weights ------------------------------------------------
// Item it of lane r is group off[it] of the half-wave's row jrow[it] (ranges
// rotated); xoff its offset in xs (-1: no item); dest the parts index its
// range's sum goes to when the item closes the range (-1: it does not).
template <int RH, int MAXI>
struct LanePlan {
  int off[MAXI];
  int jrow[MAXI];
  int xoff[MAXI];
  int dest[MAXI];
  int empty_dest[RH];  // parts index of an empty range's zero (-1: none)
};

template <int RH, int MAXI>
__device__ __forceinline__ void lane_plan(LanePlan<RH, MAXI>& P, int groups, int slot0, int r) {
  int lo[RH], len[RH];
#pragma unroll
  for (int j = 0; j < RH; ++j) {
    const int rr = (r + j) & 31;
    lo[j] = rr * groups / kRanges;
    len[j] = (rr + 1) * groups / kRanges - lo[j];
    P.empty_dest[j] = len[j] == 0 ? (slot0 + j) * kPartStride + rr : -1;
  }
#pragma unroll
  for (int it = 0; it < MAXI; ++it) {
    // Item it is the k-th group of the first row j whose ranges it reaches.
    int k = it, g = -1, last = -1, jsel = 0, dest = -1;
#pragma unroll
    for (int j = 0; j < RH; ++j) {
      if (g < 0) {
        if (k < len[j]) {
          g = lo[j] + k;
          last = lo[j] + len[j] - 1;
          jsel = j;
          dest = (slot0 + j) * kPartStride + ((r + j) & 31);
        } else {
          k -= len[j];
        }
      }
    }
    P.off[it] = g;
    P.jrow[it] = jsel;
    P.xoff[it] = g < 0 ? -1 : g * kXStride;
    P.dest[it] = g >= 0 && g == last ? dest : -1;
  }
}

template <int MAXI, int F = kQ4_0>
struct LaneWeights {
  uint4 codes[MAXI];
  uint16_t scale[MAXI];
};
template <int MAXI>
struct LaneWeights<MAXI, kQ8_0> {
  uint4 codes[2 * MAXI];
  uint16_t scale[MAXI];
};
template <int MAXI>
struct LaneWeights<MAXI, kQ4_1> {
  uint4 codes[MAXI];
  uint32_t scale[MAXI];  // d, then m in the high half
};

// Item it's block: row row0 + jrow of m (write products). Loaded
// unconditionally (block 0 for no item or a row past the end, whose sums are
// never written).
template <int RH, int MAXI, int F = kQ4_0>
__device__ __forceinline__ void load_rows(LaneWeights<MAXI, F>& W, const LanePlan<RH, MAXI>& P,
                                          const QMatrix& m, int row0) {
  const int groups = m.cols >> 5;
#pragma unroll
  for (int it = 0; it < MAXI; ++it) {
    const int row = row0 + P.jrow[it];
    const int blk = P.off[it] >= 0 && row < m.rows ? row * groups + P.off[it] : 0;
    if constexpr (F == kQ8_0) {
      W.codes[2 * it] = reinterpret_cast<const uint4*>(m.codes)[2 * blk];
      W.codes[2 * it + 1] = reinterpret_cast<const uint4*>(m.codes)[2 * blk + 1];
      W.scale[it] = m.scales[blk];
    } else if constexpr (F == kQ4_1) {
      W.codes[it] = reinterpret_cast<const uint4*>(m.codes)[blk];
      W.scale[it] = reinterpret_cast<const uint32_t*>(m.scales)[blk];
    } else {
      W.codes[it] = reinterpret_cast<const uint4*>(m.codes)[blk];
      W.scale[it] = m.scales[blk];
    }
  }
}

// Item it's block: row n of gate (jrow 0) or up (jrow 1).
template <int MAXI>
__device__ __forceinline__ void load_neuron(LaneWeights<MAXI>& W, const LanePlan<2, MAXI>& P,
                                            const QMatrix& gate, const QMatrix& up, int n) {
  const int groups = gate.cols >> 5;
#pragma unroll
  for (int it = 0; it < MAXI; ++it) {
    const int blk = P.off[it] >= 0 && n < gate.rows ? n * groups + P.off[it] : 0;
    const uint4* codes = reinterpret_cast<const uint4*>(P.jrow[it] ? up.codes : gate.codes);
    const uint16_t* scales = P.jrow[it] ? up.scales : gate.scales;
    W.codes[it] = codes[blk];
    W.scale[it] = scales[blk];
  }
}

// Item it's group chained into acc, in the weights' format.
template <int MAXI, int F>
__device__ __forceinline__ float lane_chain_item(float acc, const LaneWeights<MAXI, F>& W, int it,
                                                 const float* xg) {
  if constexpr (F == kQ8_0) {
    return chain_group_q8_0(acc, W.codes[2 * it], W.codes[2 * it + 1], W.scale[it], xg);
  } else if constexpr (F == kQ4_1) {
    return chain_group_q4_1(acc, W.codes[it], W.scale[it], xg);
  } else {
    return chain_group(acc, W.codes[it], W.scale[it], xg);
  }
}

// The lane's chains; each range's sum goes to its parts entry.
template <int RH, int MAXI, int F = kQ4_0>
__device__ __forceinline__ void lane_chains(const LaneWeights<MAXI, F>& W,
                                            const LanePlan<RH, MAXI>& P, const float* xs,
                                            float* parts) {
#pragma unroll
  for (int j = 0; j < RH; ++j) {
    if (P.empty_dest[j] >= 0) parts[P.empty_dest[j]] = 0.0f;
  }
  float acc = 0.0f;
#pragma unroll
  for (int it = 0; it < MAXI; ++it) {
    if (P.xoff[it] >= 0) {
      acc = lane_chain_item<MAXI, F>(acc, W, it, xs + P.xoff[it]);
      if (P.dest[it] >= 0) {
        parts[P.dest[it]] = acc;
        acc = 0.0f;
      }
    }
  }
}

__device__ __forceinline__ float row_total(const float* parts) {
  float total = 0.0f;
#pragma unroll
  for (int r = 0; r < kRanges; ++r) total = total + parts[r];
  return total;
}

// The layer's pin words [first, count], loaded through a vector register:
// a scalar load would be waited for before the kernel's other scalar loads,
// its arguments, which everything after waits on; a vector load is waited
// for where its words are used, at the end. Without a table the words are
// read from `fallback` (any two readable words) and not used: no branch
// around the load, whose join would wait for it.
__device__ __forceinline__ uint2 request_pin_words(const uint32_t* __restrict__ edits, int layer,
                                                   const void* fallback) {
  int at = 2 * layer;
  asm volatile("" : "+v"(at));
  const uint32_t* src = edits ? edits + at : static_cast<const uint32_t*>(fallback);
  return make_uint2(src[0], src[1]);
}

// A layer's pins on neuron n at `position` (edit.wgsl:55-76): the layer's
// edits are sorted by neuron then first position (edit.cpp:20-31), so a
// binary search finds the neuron's; its ranges never overlap.
// `first` and `count` are the layer's [first, count] words, read ahead.
__device__ __forceinline__ float apply_pins(const uint32_t* __restrict__ t, uint32_t first,
                                            uint32_t count, uint32_t n, uint32_t position,
                                            float value) {
  uint32_t lo = 0, hi = count;
  while (lo < hi) {
    const uint32_t mid = (lo + hi) >> 1;
    if (t[first + 5 * mid] < n) lo = mid + 1; else hi = mid;
  }
  for (uint32_t i = lo; i < count; ++i) {
    const uint32_t* e = t + first + 5 * i;
    if (e[0] != n) break;
    if (position < e[3] || position >= e[4]) continue;
    const float v = bits_to_float(e[2]);
    if (e[1] == 1u) {
      if (v != 1.0f) value = value * v;
    } else {
      value = v;
    }
  }
  return value;
}

// A plain row's vec4s a thread loads: RH = 1 products take K up to 1,024
// MAXI; RH = 2 ones (items of two rows' ranges at most 3) K below 1,536.
template <int RH, int MAXI, int T>
constexpr int plain_vec4s() {
  return RH == 1 ? (1024 * MAXI / 4 + T - 1) / T : (1536 / 4 + T - 1) / T;
}

// ---- kernels ------------------------------------------------------------------
// Write products: a tile is 2 RH WAVES rows, each wave two half-waves of RH
// rows. A workgroup stages its input row once and takes TPW tiles,
// blockIdx.x + k gridDim.x (clamped to the last tile, which a workgroup past
// the end then recomputes with the same bits), loading each tile's weights
// before it computes the one before. The tiles are unrolled into
// straight-line code over two register buffers, so every wait is for the
// oldest loads only.
template <int RH, int MAXI, int MODE, int TPW, int WAVES, int F = kQ4_0>
__global__ __launch_bounds__(64 * WAVES) void gemv_write_kernel(const DevStep* __restrict__ step,
                                                                QMatrix w, GemvInput in,
                                                                float* __restrict__ y) {
  extern __shared__ __align__(16) float smem[];
  constexpr int T = 64 * WAVES;
  constexpr int kRows = 2 * RH * WAVES;
  constexpr int X4 = plain_vec4s<RH, MAXI, T>();
  float* parts = smem;
  float* red = parts + kRows * kPartStride;
  float* xs = red + kRedFloats;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 31;
  const int slot0 = (wave * 2 + (lane >> 5)) * RH;
  const int tiles = (w.rows + kRows - 1) / kRows;
  auto tile_of = [&](int k) { return min((int)blockIdx.x + k * (int)gridDim.x, tiles - 1); };
  LanePlan<RH, MAXI> plan;
  lane_plan<RH, MAXI>(plan, w.cols >> 5, slot0, r);
  Prologue<T, X4> pro;
  prologue_load<MODE, T, X4>(pro, in, step, w.cols);
  LaneWeights<MAXI, F> buf[2];
  load_rows<RH, MAXI, F>(buf[0], plan, w, tile_of(0) * kRows + slot0);
  prologue_finish<MODE, T, X4>(xs, red, pro, in, step, w.cols);
  __syncthreads();
  if constexpr (RH == 1) {
    // One row a half-wave, lane r its range r: the lane's chain is the range
    // sum (0 for an empty range, which leaves a total unchanged) and the
    // total is a DPP chain, with no LDS round trip. Up to two items take
    // their input into registers before the weights are waited for.
    static_assert(TPW == 1, "one tile a workgroup");
    float acc = 0.0f;
    if constexpr (F == kQ4_0 && MAXI <= 2) {
      float4 xv[MAXI][8];
#pragma unroll
      for (int it = 0; it < MAXI; ++it) {
        const int xo = max(plan.xoff[it], 0);
#pragma unroll
        for (int q = 0; q < 8; ++q) xv[it][q] = ld4(xs + xo + 4 * q);
      }
#pragma unroll
      for (int it = 0; it < MAXI; ++it) {
        if (plan.xoff[it] >= 0) acc = chain_group(acc, buf[0].codes[it], buf[0].scale[it], xv[it]);
      }
    } else if constexpr (F == kQ4_0) {
      // Longer chains (K = 6,912: 6 or 7 groups) run about one wave a SIMD,
      // which cannot hide LDS latency: the next group's input is read into
      // the other register buffer while this group's chain runs.
      float4 xa[8], xb[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) xa[q] = ld4(xs + max(plan.xoff[0], 0) + 4 * q);
#pragma unroll
      for (int it = 0; it < MAXI; ++it) {
        float4 (&cur)[8] = (it & 1) ? xb : xa;
        float4 (&nxt)[8] = (it & 1) ? xa : xb;
        if (it + 1 < MAXI) {
          const int xo = max(plan.xoff[it + 1 < MAXI ? it + 1 : it], 0);
#pragma unroll
          for (int q = 0; q < 8; ++q) nxt[q] = ld4(xs + xo + 4 * q);
        }
        if (plan.xoff[it] >= 0) acc = chain_group(acc, buf[0].codes[it], buf[0].scale[it], cur);
      }
    } else {
#pragma unroll
      for (int it = 0; it < MAXI; ++it) {
        if (plan.xoff[it] >= 0) acc = lane_chain_item<MAXI, F>(acc, buf[0], it, xs + plan.xoff[it]);
      }
    }
    const float total = half_wave_total(acc);
    if (r == 31) {
      const int row = tile_of(0) * kRows + slot0;
      if (row < w.rows) y[row] = total;
    }
    return;
  }
#pragma unroll
  for (int k = 0; k < TPW; ++k) {
    if (k + 1 < TPW) load_rows<RH, MAXI, F>(buf[(k + 1) & 1], plan, w, tile_of(k + 1) * kRows + slot0);
    lane_chains<RH, MAXI, F>(buf[k & 1], plan, xs, parts);
    wave_sync();
    if (r < RH) {
      const int row = tile_of(k) * kRows + slot0 + r;
      if (row < w.rows) y[row] = row_total(parts + (slot0 + r) * kPartStride);
    }
    wave_sync();
  }
}

// ---- K = 1,152: every lane two groups --------------------------------------
// At K = 1,152 a row's 36 groups make 32 ranges, of which ranges 8p + 7
// (p < 4) hold two groups (9p + 7, 9p + 8) and the other 28 one each (range
// r starts at group r + r / 8). With a lane a range, lanes of a two-group
// range set every wave's length and half the lanes idle through the second
// group. Here 18 lanes take a row, each exactly two groups:
//   position p < 4: two-group range 8p + 7, one chain over both groups;
//   position p >= 4: the one-group ranges i and i + 1 of the 28 in order,
//     i = 2 (p - 4), two chains from zero (range of the i-th: i + i / 7).
// The range sums meet in LDS, row-major, and one thread a row adds its 32 in
// order.
namespace pair {
constexpr int kCols = 1152;
constexpr int kGroups = kCols / 32;
constexpr int kLanes = 18;   // lanes a row
constexpr int kStride = 36;  // a row's range sums in LDS (16-byte rows)

struct Plan {
  int g0, g1;  // the lane's groups
  int r0, r1;  // their ranges (r0 = -1: one chain over both)
};

__device__ __forceinline__ Plan plan(int p) {
  Plan P;
  if (p < 4) {
    P.r0 = -1;
    P.r1 = 8 * p + 7;
    P.g0 = 9 * p + 7;
    P.g1 = P.g0 + 1;
  } else {
    const int i0 = 2 * (p - 4), i1 = i0 + 1;
    P.r0 = i0 + i0 / 7;
    P.r1 = i1 + i1 / 7;
    P.g0 = P.r0 + (P.r0 >> 3);
    P.g1 = P.r1 + (P.r1 >> 3);
  }
  return P;
}

template <int T>
constexpr int rows() { return T / kLanes; }

// Bytes of LDS a workgroup of T threads takes.
template <int T>
constexpr size_t lds_bytes() {
  return (size_t)(rows<T>() * kStride + kRedFloats + kGroups * kXStride) * 4;
}

// The lane's two chains from its groups and staged input: the range sums
// (s0 for r0, s1 for r1).
__device__ __forceinline__ void chains(const Plan& P, uint4 c0, uint16_t d0, uint4 c1, uint16_t d1,
                                       const float* xs, float& s0, float& s1) {
  float4 x0[8], x1[8];
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    x0[q] = ld4(xs + P.g0 * kXStride + 4 * q);
    x1[q] = ld4(xs + P.g1 * kXStride + 4 * q);
  }
  s0 = chain_group(0.0f, c0, d0, x0);
  s1 = chain_group(P.r0 < 0 ? s0 : 0.0f, c1, d1, x1);
}

// Row `local`'s total from its 32 range sums at sums[local * kStride].
__device__ __forceinline__ float row_total(const float* sums, int local) {
  float4 v[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) v[k] = ld4(sums + local * kStride + 4 * k);
  float t = 0.0f;
#pragma unroll
  for (int k = 0; k < 8; ++k) t = (((t + v[k].x) + v[k].y) + v[k].z) + v[k].w;
  return t;
}
}  // namespace pair

template <int MODE, int WAVES>
__global__ __launch_bounds__(64 * WAVES) void gemv_pair_kernel(const DevStep* __restrict__ step,
                                                               QMatrix w, GemvInput in,
                                                               float* __restrict__ y) {
  extern __shared__ __align__(16) float smem[];
  constexpr int T = 64 * WAVES;
  constexpr int kRows = pair::rows<T>();
  constexpr int X4 = plain_vec4s<1, 2, T>();
  float* sums = smem;
  float* red = sums + kRows * pair::kStride;
  float* xs = red + kRedFloats;
  const int t = threadIdx.x;
  const int local = t / pair::kLanes, p = t - local * pair::kLanes;
  const int row = blockIdx.x * kRows + local;
  const bool live = local < kRows && row < w.rows;
  const pair::Plan P = pair::plan(p);
  Prologue<T, X4> pro;
  prologue_load<MODE, T, X4>(pro, in, step, w.cols);
  // Lanes past the rows load row 0's blocks, unused. A fused product over
  // members reads each row from its member's streams.
  const MemberRow mr = member_row(w, live ? row : 0);
  const int base = mr.row * pair::kGroups;
  const uint4 c0 = reinterpret_cast<const uint4*>(mr.codes)[base + P.g0];
  const uint16_t d0 = mr.scales[base + P.g0];
  const uint4 c1 = reinterpret_cast<const uint4*>(mr.codes)[base + P.g1];
  const uint16_t d1 = mr.scales[base + P.g1];
  prologue_finish<MODE, T, X4>(xs, red, pro, in, step, w.cols);
  __syncthreads();
  float s0, s1;
  pair::chains(P, c0, d0, c1, d1, xs, s0, s1);
  if (live) {
    if (P.r0 >= 0) sums[local * pair::kStride + P.r0] = s0;
    sums[local * pair::kStride + P.r1] = s1;
  }
  __syncthreads();
  if (t < kRows && blockIdx.x * kRows + t < w.rows)
    y[blockIdx.x * kRows + t] = pair::row_total(sums, t);
}

// The pair layout over many rows: a workgroup takes TPW tiles of kRows rows,
// blockIdx.x + k gridDim.x (clamped to the last tile, which a workgroup past
// the end recomputes with the same bits). The lane's two groups are the same
// in every tile, so their input goes into registers once; the next tile's
// weights load under this tile's chains; the range sums alternate between
// two LDS areas, so one barrier a tile orders writers and readers.
template <int MODE, int WAVES, int TPW>
__global__ __launch_bounds__(64 * WAVES) void gemv_pair_tiles_kernel(
    const DevStep* __restrict__ step, QMatrix w, GemvInput in, float* __restrict__ y) {
  extern __shared__ __align__(16) float smem[];
  constexpr int T = 64 * WAVES;
  constexpr int kRows = pair::rows<T>();
  constexpr int X4 = plain_vec4s<1, 2, T>();
  float* sums = smem;  // [2][kRows][pair::kStride]
  float* red = sums + 2 * kRows * pair::kStride;
  float* xs = red + kRedFloats;
  const int t = threadIdx.x;
  const int local = t / pair::kLanes, p = t - local * pair::kLanes;
  const int tiles = (w.rows + kRows - 1) / kRows;
  auto tile_of = [&](int k) { return min((int)blockIdx.x + k * (int)gridDim.x, tiles - 1); };
  const pair::Plan P = pair::plan(p);
  Prologue<T, X4> pro;
  prologue_load<MODE, T, X4>(pro, in, step, w.cols);
  uint4 c[2][2];
  uint16_t d[2][2];
  auto load_tile = [&](int k, int b) {
    const int row = tile_of(k) * kRows + local;
    const int base = local < kRows && row < w.rows ? row * pair::kGroups : 0;
    c[b][0] = reinterpret_cast<const uint4*>(w.codes)[base + P.g0];
    d[b][0] = w.scales[base + P.g0];
    c[b][1] = reinterpret_cast<const uint4*>(w.codes)[base + P.g1];
    d[b][1] = w.scales[base + P.g1];
  };
  load_tile(0, 0);
  prologue_finish<MODE, T, X4>(xs, red, pro, in, step, w.cols);
  __syncthreads();
  float4 x0[8], x1[8];
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    x0[q] = ld4(xs + P.g0 * kXStride + 4 * q);
    x1[q] = ld4(xs + P.g1 * kXStride + 4 * q);
  }
#pragma unroll
  for (int k = 0; k < TPW; ++k) {
    if (k + 1 < TPW) load_tile(k + 1, (k + 1) & 1);
    const float s0 = chain_group(0.0f, c[k & 1][0], d[k & 1][0], x0);
    const float s1 = chain_group(P.r0 < 0 ? s0 : 0.0f, c[k & 1][1], d[k & 1][1], x1);
    float* area = sums + (k & 1) * kRows * pair::kStride;
    const int row = tile_of(k) * kRows + local;
    if (local < kRows && row < w.rows) {
      if (P.r0 >= 0) area[local * pair::kStride + P.r0] = s0;
      area[local * pair::kStride + P.r1] = s1;
    }
    __syncthreads();
    if (t < kRows && tile_of(k) * kRows + t < w.rows)
      y[tile_of(k) * kRows + t] = pair::row_total(area, t);
  }
}

// Gated product: each half-wave one neuron n, its gate row and its up row
// (rotated ranges), then gelu_tanh(gate) * up and the layer's pins.
template <int MAXI, int MODE, int WAVES>
__global__ __launch_bounds__(64 * WAVES) void gemv_gated_kernel(const DevStep* __restrict__ step,
                                                                QMatrix gate, QMatrix up,
                                                                GemvInput in, float* __restrict__ act,
                                                                const uint32_t* __restrict__ edits,
                                                                int layer) {
  extern __shared__ __align__(16) float smem[];
  constexpr int T = 64 * WAVES;
  constexpr int kNeurons = 2 * WAVES;
  constexpr int X4 = (kNormMaxCols / 4 + T - 1) / T;
  float* parts = smem;
  float* red = parts + 2 * kNeurons * kPartStride;
  float* xs = red + kRedFloats;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 31;
  const int local = wave * 2 + (lane >> 5);
  const int n = blockIdx.x * kNeurons + local;
  LanePlan<2, MAXI> plan;
  lane_plan<2, MAXI>(plan, gate.cols >> 5, 2 * local, r);
  Prologue<T, X4> pro;
  prologue_load<MODE, T, X4>(pro, in, step, gate.cols);
  LaneWeights<MAXI> W;
  load_neuron<MAXI>(W, plan, gate, up, n);
  const uint2 pins = request_pin_words(edits, layer, step);
  prologue_finish<MODE, T, X4>(xs, red, pro, in, step, gate.cols);
  __syncthreads();
  lane_chains<2, MAXI>(W, plan, xs, parts);
  wave_sync();
  // Lane 0 totals the gate row while lane 1 totals the up row.
  const float total = r < 2 ? row_total(parts + (2 * local + r) * kPartStride) : 0.0f;
  const float u = row_shl<1>(total);  // lane t + 1: even t stays in its row
  if (r == 0 && n < gate.rows) {
    float v = gelu_tanh(total) * u;
    if (edits && pins.y) v = apply_pins(edits, pins.x, pins.y, (uint32_t)n, step->position, v);
    act[n] = v;
  }
}

// Gated product at K = 1,152: a neuron takes 36 lanes, 18 for its gate row
// and 18 for its up row, each lane two groups as in the pair layout; then
// gelu_tanh(gate) * up and the layer's pins.
template <int MODE, int WAVES, int TPW>
__global__ __launch_bounds__(64 * WAVES) void gemv_gated_pair_kernel(
    const DevStep* __restrict__ step, QMatrix gate, QMatrix up, GemvInput in,
    float* __restrict__ act, const uint32_t* __restrict__ edits, int layer) {
  extern __shared__ __align__(16) float smem[];
  constexpr int T = 64 * WAVES;
  constexpr int kNeurons = T / (2 * pair::kLanes);
  static_assert(2 * kNeurons <= 64, "the totals sit in the first wave");
  constexpr int X4 = plain_vec4s<1, 2, T>();
  float* sums = smem;  // [2][neuron][gate, up][pair::kStride]
  float* red = sums + 2 * 2 * kNeurons * pair::kStride;
  float* xs = red + kRedFloats;
  const int t = threadIdx.x;
  const int local = t / (2 * pair::kLanes);
  const int q = t - local * 2 * pair::kLanes;
  const int which = q >= pair::kLanes ? 1 : 0;
  const int tiles = (gate.rows + kNeurons - 1) / kNeurons;
  auto tile_of = [&](int k) { return min((int)blockIdx.x * TPW + k, tiles - 1); };
  const pair::Plan P = pair::plan(q - which * pair::kLanes);
  // Every argument the loads use, read at once (a single wait, rather than
  // one for each block of code that first needs one).
  asm volatile("" ::"s"(gate.codes), "s"(gate.scales), "s"(up.codes), "s"(up.scales),
               "s"(in.x), "s"(in.hidden), "s"(in.output), "s"(in.post_gain), "s"(in.gain),
               "s"(in.epsilon), "s"(edits), "s"(layer));
  Prologue<T, X4> pro;
  prologue_load<MODE, T, X4>(pro, in, step, gate.cols);
  const QMatrix& m = which ? up : gate;
  uint4 c[2][2];
  uint16_t d[2][2];
  auto load_tile = [&](int k, int b) {
    const int n = tile_of(k) * kNeurons + local;
    const int base = local < kNeurons && n < gate.rows ? n * pair::kGroups : 0;
    c[b][0] = reinterpret_cast<const uint4*>(m.codes)[base + P.g0];
    d[b][0] = m.scales[base + P.g0];
    c[b][1] = reinterpret_cast<const uint4*>(m.codes)[base + P.g1];
    d[b][1] = m.scales[base + P.g1];
  };
  load_tile(0, 0);
  const uint2 pins = request_pin_words(edits, layer, step);
  prologue_finish<MODE, T, X4>(xs, red, pro, in, step, gate.cols);
  __syncthreads();
  float4 x0[8], x1[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    x0[i] = ld4(xs + P.g0 * kXStride + 4 * i);
    x1[i] = ld4(xs + P.g1 * kXStride + 4 * i);
  }
  const int slot = 2 * local + which;
#pragma unroll
  for (int k = 0; k < TPW; ++k) {
    if (k + 1 < TPW) load_tile(k + 1, (k + 1) & 1);
    const float s0 = chain_group(0.0f, c[k & 1][0], d[k & 1][0], x0);
    const float s1 = chain_group(P.r0 < 0 ? s0 : 0.0f, c[k & 1][1], d[k & 1][1], x1);
    float* area = sums + (k & 1) * 2 * kNeurons * pair::kStride;
    const int n = tile_of(k) * kNeurons + local;
    if (local < kNeurons && n < gate.rows) {
      if (P.r0 >= 0) area[slot * pair::kStride + P.r0] = s0;
      area[slot * pair::kStride + P.r1] = s1;
    }
    __syncthreads();
    if (t < 64) {
      // Thread 2k totals neuron k's gate row, thread 2k + 1 its up row.
      const float total = t < 2 * kNeurons ? pair::row_total(area, t) : 0.0f;
      const float u = row_shl<1>(total);  // lane t + 1: even t stays in its row
      const int nn = tile_of(k) * kNeurons + (t >> 1);
      if ((t & 1) == 0 && t < 2 * kNeurons && nn < gate.rows) {
        float v = gelu_tanh(total) * u;
        if (edits && pins.y) v = apply_pins(edits, pins.x, pins.y, (uint32_t)nn, step->position, v);
        act[nn] = v;
      }
    }
  }
}

int max_items(int cols, int rh) {
  const int groups = cols / 32;
  int most = 0;
  for (int r = 0; r < kRanges; ++r) {
    int n = 0;
    for (int j = 0; j < rh; ++j) {
      const int rr = (r + j) & 31;
      n += (rr + 1) * groups / kRanges - rr * groups / kRanges;
    }
    most = n > most ? n : most;
  }
  return most;
}

// Tiles a workgroup of the many-row product (the 262,144-row head) takes:
// its input row is staged once for all of them.
constexpr int kHeadTilesPerGroup = 8;

template <int RH, int MAXI, int MODE, int TPW, int WAVES, int F = kQ4_0>
hipError_t launch_write(hipStream_t s, const DevStep* step, const QMatrix& w, const GemvInput& in,
                        float* y) {
  constexpr int kRows = 2 * RH * WAVES;
  const size_t lds = (size_t)(kRows * kPartStride + kRedFloats + (w.cols / 32) * kXStride) * 4;
  const int tiles = (w.rows + kRows - 1) / kRows;
  hipLaunchKernelGGL((gemv_write_kernel<RH, MAXI, MODE, TPW, WAVES, F>),
                     dim3((tiles + TPW - 1) / TPW), dim3(64 * WAVES), lds, s, step, w, in, y);
  return hipGetLastError();
}

template <int MODE, int WAVES>
hipError_t launch_pair(hipStream_t s, const DevStep* step, const QMatrix& w, const GemvInput& in,
                       float* y) {
  constexpr int T = 64 * WAVES, kRows = pair::rows<T>();
  hipLaunchKernelGGL((gemv_pair_kernel<MODE, WAVES>), dim3((w.rows + kRows - 1) / kRows), dim3(T),
                     pair::lds_bytes<T>(), s, step, w, in, y);
  return hipGetLastError();
}

template <int MODE, int F = kQ4_0>
hipError_t dispatch_write(hipStream_t s, const DevStep* step, const QMatrix& w,
                          const GemvInput& in, float* y) {
  const int items1 = max_items(w.cols, 1);
  const int items2 = max_items(w.cols, 2);
  // Many rows: two rows a half-wave, ranges rotated, where that balances.
  if constexpr (F == kQ4_0 && MODE != 3) {
    if (w.rows >= 16384 && w.cols == pair::kCols) {
      constexpr int T = 256, kRows = pair::rows<T>(), TPW = kHeadTilesPerGroup;
      const int tiles = (w.rows + kRows - 1) / kRows;
      const size_t lds = (size_t)(2 * kRows * pair::kStride + kRedFloats + pair::kGroups * kXStride) * 4;
      hipLaunchKernelGGL((gemv_pair_tiles_kernel<MODE, 4, TPW>), dim3((tiles + TPW - 1) / TPW),
                         dim3(T), lds, s, step, w, in, y);
      return hipGetLastError();
    }
  }
  if (w.rows >= 16384 && items2 <= 3 && w.cols < 1536)
    return launch_write<2, 3, MODE, kHeadTilesPerGroup, 2, F>(s, step, w, in, y);
  // K = 1,152 in Q4_0: two groups every lane; four waves (14 rows) share an
  // input row where there are thousands of rows, two (7 rows) below.
  if constexpr (F == kQ4_0 && MODE != 3) {
    if (w.cols == pair::kCols) {
      return w.rows >= 4096 ? launch_pair<MODE, 4>(s, step, w, in, y)
                            : launch_pair<MODE, 2>(s, step, w, in, y);
    }
  }
  if (items1 <= 1) return launch_write<1, 1, MODE, 1, 2, F>(s, step, w, in, y);
  if (items1 <= 2) return launch_write<1, 2, MODE, 1, 2, F>(s, step, w, in, y);
  if (items1 <= 4) return launch_write<1, 4, MODE, 1, 2, F>(s, step, w, in, y);
  // Up to 8 items (K to 8,192): four waves, so half as many workgroups stage
  // the long input row. K = 6,912 (7 items) has its own form, which issues
  // no load for an eighth item.
  if (items1 <= 7) return launch_write<1, 7, MODE, 1, 4, F>(s, step, w, in, y);
  if (items1 <= 8) return launch_write<1, 8, MODE, 1, 4, F>(s, step, w, in, y);
  return hipErrorInvalidValue;
}

// Gated workgroups of kGatedWaves waves: the fewer workgroups, the less
// redundant input-row work and L2 traffic for it.
constexpr int kGatedWaves = 4;
// Tiles of 7 neurons a K = 1,152 gated workgroup: its input row is made once for them.
constexpr int kGatedTiles = 2;

template <int MAXI, int MODE, int kWaves = kGatedWaves>
hipError_t launch_gated(hipStream_t s, const DevStep* step, const QMatrix& gate,
                        const QMatrix& up, const GemvInput& in, float* act,
                        const uint32_t* edits, int layer) {
  constexpr int kNeurons = 2 * kWaves;
  const size_t lds =
      (size_t)(2 * kNeurons * kPartStride + kRedFloats + (gate.cols / 32) * kXStride) * 4;
  hipLaunchKernelGGL((gemv_gated_kernel<MAXI, MODE, kWaves>),
                     dim3((gate.rows + kNeurons - 1) / kNeurons), dim3(64 * kWaves), lds, s, step,
                     gate, up, in, act, edits, layer);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_gemv_decode(hipStream_t s, const DevStep* step, const QMatrix& w,
                              const GemvInput& in, int mode, float* y) {
  if (w.cols % 32 != 0 || w.rows <= 0 || w.cols > 8 * 1024 ||
      (long long)w.rows * (w.cols / 32) >= (1ll << 31)) {
    return hipErrorInvalidValue;
  }
  if (mode != 0 && w.cols > kNormMaxCols) return hipErrorInvalidValue;
  // Members are read by the K = 1,152 pair form of fewer than 16,384 rows.
  if (has_members(w) &&
      (w.format != kQ4_0 || w.cols != pair::kCols || w.rows >= 16384 || mode == 3))
    return hipErrorInvalidValue;
  if (mode == 2 && in.table.format != kQ4_0 && in.table.format != kQ8_0)
    return hipErrorInvalidValue;
  // Q4_1 and Q8_0 weights (a file's downs and tied head) take a plain row.
  if (w.format != kQ4_0) {
    if (mode != 0) return hipErrorInvalidValue;
    if (w.format == kQ8_0) return dispatch_write<0, kQ8_0>(s, step, w, in, y);
    if (w.format == kQ4_1) return dispatch_write<0, kQ4_1>(s, step, w, in, y);
    return hipErrorInvalidValue;
  }
  switch (mode) {
    case 0: return dispatch_write<0>(s, step, w, in, y);
    case 1: return dispatch_write<1>(s, step, w, in, y);
    case 2: return dispatch_write<2>(s, step, w, in, y);
    case 3:
      if (w.cols != kFoldWidth || max_items(w.cols, 1) != 1) return hipErrorInvalidValue;
      // Four waves: half as many workgroups folding the chunk states.
      return launch_write<1, 1, 3, 1, 4>(s, step, w, in, y);
    default: return hipErrorInvalidValue;
  }
}

template <int MODE, int WAVES, int TPW>
hipError_t launch_gated_pair(hipStream_t s, const DevStep* step, const QMatrix& gate,
                             const QMatrix& up, const GemvInput& in, float* act,
                             const uint32_t* edits, int layer) {
  constexpr int T = 64 * WAVES, kNeurons = T / (2 * pair::kLanes);
  const size_t lds = (size_t)(2 * 2 * kNeurons * pair::kStride + kRedFloats +
                              pair::kGroups * kXStride) * 4;
  const int tiles = (gate.rows + kNeurons - 1) / kNeurons;
  hipLaunchKernelGGL((gemv_gated_pair_kernel<MODE, WAVES, TPW>), dim3((tiles + TPW - 1) / TPW),
                     dim3(T), lds, s, step, gate, up, in, act, edits, layer);
  return hipGetLastError();
}

hipError_t launch_gated_decode(hipStream_t s, const DevStep* step, const QMatrix& gate,
                               const QMatrix& up, const GemvInput& in, int mode, float* act,
                               const uint32_t* edits, int layer) {
  // Gate and up rows together: two rows' ranges, at most 4 items to K = 2,048.
  if (gate.cols % 32 != 0 || gate.rows != up.rows || gate.cols != up.cols ||
      gate.cols > kNormMaxCols || (long long)gate.rows * (gate.cols / 32) >= (1ll << 31) ||
      (mode != 0 && mode != 1) || gate.format != kQ4_0 || up.format != kQ4_0) {
    return hipErrorInvalidValue;
  }
  // K = 1,152: two groups every lane, 7 neurons a 4-wave workgroup.
  if (gate.cols == pair::kCols) {
    return mode == 0 ? launch_gated_pair<0, 4, kGatedTiles>(s, step, gate, up, in, act, edits, layer)
                     : launch_gated_pair<1, 4, kGatedTiles>(s, step, gate, up, in, act, edits, layer);
  }
  const int items = max_items(gate.cols, 2);
  if (items <= 3) {
    return mode == 0 ? launch_gated<3, 0>(s, step, gate, up, in, act, edits, layer)
                     : launch_gated<3, 1>(s, step, gate, up, in, act, edits, layer);
  }
  if (items <= 4) {
    return mode == 0 ? launch_gated<4, 0>(s, step, gate, up, in, act, edits, layer)
                     : launch_gated<4, 1>(s, step, gate, up, in, act, edits, layer);
  }
  return hipErrorInvalidValue;
}

}  // namespace frz
