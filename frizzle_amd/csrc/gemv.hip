// Q4_0 matrix products of the forward path, in the reference's order of
// addition (matmul.h:88-97): each output's K weights are cut into 32 ranges
// of whole 32-weight groups at fixed boundaries (range r is groups
// floor(r G / 32) .. floor((r + 1) G / 32)); a range's products chain by fma
// from zero, k in order; the 32 range sums add in order to a total from
// zero. Every form below keeps that order, so a token's outputs are the same
// bits whether it is decoded alone or prefilled in a tile.
//
// Q4_0 weight j of a block is ((code_j) - 8) * d (q4_0.wgsl:71-83), made
// exactly in f32: the value needs at most 15 significant bits.
//
// Single-token steps go to the decode forms (gemv_decode.hip); steps of
// several tokens run here on the fp32 matrix cores.

#include <algorithm>

#include "kernels.h"
#include "numerics.h"

namespace frz {
namespace {

__device__ __forceinline__ float half_to_float(uint16_t h) {
  return (float)__builtin_bit_cast(_Float16, h);
}

// A layer's pins on neuron n at `position` (edit.wgsl:55-76): the layer's
// edits are sorted by neuron then first position (edit.cpp:20-31), so a
// binary search finds the neuron's; its ranges never overlap.
__device__ __forceinline__ float apply_edits(const uint32_t* __restrict__ t,
                                             int layer, uint32_t n,
                                             uint32_t position, float value) {
  const uint32_t first = t[2 * layer];
  const uint32_t count = t[2 * layer + 1];
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

// ---- prefill form: matrix cores ------------------------------------------
// The fp32 matrix-core instructions with one k per step,
// v_mfma_f32_32x32x1_2b_f32 and v_mfma_f32_16x16x1_4b_f32, update NB
// independent blocks of D x D accumulators (NB = 2, D = 32 or NB = 4,
// D = 16) with one fma per element: C = fma(a_i, b_j, C), one rounding, the
// fma of the reference's chain. A run of them in k order is that chain.
//
// A wave owns a tile of D rows x D tokens and gives each block its own
// K-range of that same tile: at pass p, block b chains range NB p + b. When
// the pass's ranges are done, their sums join the totals in range order
// (matmul.wgsl:320-405), and the blocks start the next NB ranges. Ranges of
// one pass may differ in length by a group; a block whose range is done
// meanwhile multiplies zero inputs, which adds a zero to a range sum whose
// sign can then differ only for a zero sum - and the totals, which start at
// +0 and so are never -0, are the same either way.
//
// Lane l is row l % D and token l % D of block l / D: it decodes its row's
// weights for its block's group, in-register and exactly, and reads its
// token's inputs for that group. So every lane does distinct work and a pass
// keeps NB chains in flight. The inputs of a step (NB groups x D tokens = 64
// lines of 32 floats) are loaded whole-line into LDS and read back one line
// per lane. A gated wave holds the gate and up tiles of the same neurons,
// sharing the inputs.
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v32f __attribute__((ext_vector_type(32)));

constexpr int kTileWaves = 4;  // waves per workgroup; each its own tokens

template <int NB>
struct Mfma;

// Element (i, j) of block b: lane j + 32 ((i / 4) % 2), register
// 16 b + 4 (i / 8) + i % 4. Output slot o of lane L (o < 16) is
// row 8 (o / 4) + 4 ((L / 32) % 2) + o % 4, token L % 32; block b's value
// is register 16 b + o.
template <>
struct Mfma<2> {
  static constexpr int kDim = 32;
  static constexpr int kSlots = 16;
  typedef v32f Acc;
  __device__ static Acc op(float a, float b, Acc c) {
    return __builtin_amdgcn_mfma_f32_32x32x1f32(a, b, c, 0, 0, 0);
  }
  __device__ static int slot_row(int lane, int o) {
    return 8 * (o >> 2) + 4 * ((lane >> 5) & 1) + (o & 3);
  }
};

// Element (i, j) of block b: lane j + 16 (i / 4), register i % 4 + 4 b.
// Output slot o of lane L (o < 4) is row 4 (L / 16) + o, token L % 16;
// block b's value is register 4 b + o.
template <>
struct Mfma<4> {
  static constexpr int kDim = 16;
  static constexpr int kSlots = 4;
  typedef v16f Acc;
  __device__ static Acc op(float a, float b, Acc c) {
    return __builtin_amdgcn_mfma_f32_16x16x1f32(a, b, c, 0, 0, 0);
  }
  __device__ static int slot_row(int lane, int o) { return 4 * (lane >> 4) + o; }
};

// A group's 32 weights in k order (q4_0.wgsl:71-83). Weight k < 16 is the
// low nibble of byte k, weight 16 + k its high nibble. A bitfield insert puts
// a low nibble q under the exponent of 1024 (f16 0x6400) to make 1024 + q,
// and a high nibble in place to make 1024 + 16 q; then
//   fma(1024 + q, d, -1032 d) = (q - 8) d  and
//   fma(1024 + 16 q, d / 16, -72 d) = (q - 8) d,
// both exact: every operand and the result fit in 24 bits.
// Half H of a group: weights 16 H .. 16 H + 15.
template <int H>
__device__ __forceinline__ void decode_half(uint4 c, uint16_t dbits, float (&wk)[16]) {
  const float d = half_to_float(dbits);
  const float scale = H == 0 ? d : 0.0625f * d;
  const float bias = H == 0 ? -1032.0f * d : -72.0f * d;
  const uint32_t words[4] = {c.x, c.y, c.z, c.w};
  // The exponent comes from a register the compiler cannot see into, so that
  // (s & mask) | (exp & ~mask) stays one bitfield insert.
  uint32_t kExp;
  asm("v_mov_b32 %0, 0x64006400" : "=v"(kExp));
  constexpr uint32_t kMask = H == 0 ? 0x000F000Fu : 0x00F000F0u;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    // even: bytes 0 and 2 of the word; odd: bytes 1 and 3.
    const half2v e = __builtin_bit_cast(half2v, (words[w] & kMask) | (kExp & ~kMask));
    const half2v o = __builtin_bit_cast(half2v, ((words[w] >> 8) & kMask) | (kExp & ~kMask));
    wk[4 * w + 0] = __builtin_fmaf((float)e.x, scale, bias);
    wk[4 * w + 1] = __builtin_fmaf((float)o.x, scale, bias);
    wk[4 * w + 2] = __builtin_fmaf((float)e.y, scale, bias);
    wk[4 * w + 3] = __builtin_fmaf((float)o.y, scale, bias);
  }
}

// Q4_1, half H: (q - 0) d + m (q4_1.wgsl:12-25); the nibble placed as for
// Q4_0 gives q d exactly, fma(1024 + q, d, -1024 d) or
// fma(1024 + 16 q, d / 16, -64 d), and adding m is the one rounding.
template <int H>
__device__ __forceinline__ void decode_half_q4_1(uint4 c, uint32_t dm, float (&wk)[16]) {
  const float d = half_to_float((uint16_t)(dm & 0xFFFFu));
  const float m = half_to_float((uint16_t)(dm >> 16));
  const float scale = H == 0 ? d : 0.0625f * d;
  const float bias = H == 0 ? -1024.0f * d : -64.0f * d;
  const uint32_t words[4] = {c.x, c.y, c.z, c.w};
  uint32_t kExp;
  asm("v_mov_b32 %0, 0x64006400" : "=v"(kExp));
  constexpr uint32_t kMask = H == 0 ? 0x000F000Fu : 0x00F000F0u;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const half2v e = __builtin_bit_cast(half2v, (words[w] & kMask) | (kExp & ~kMask));
    const half2v o = __builtin_bit_cast(half2v, ((words[w] >> 8) & kMask) | (kExp & ~kMask));
    wk[4 * w + 0] = __builtin_fmaf((float)e.x, scale, bias) + m;
    wk[4 * w + 1] = __builtin_fmaf((float)o.x, scale, bias) + m;
    wk[4 * w + 2] = __builtin_fmaf((float)e.y, scale, bias) + m;
    wk[4 * w + 3] = __builtin_fmaf((float)o.y, scale, bias) + m;
  }
}

// Q8_0, half H: weights 16 H .. 16 H + 15 are code bytes 16 H .. 16 H + 15
// (c holds them), each qs d (q8_0.wgsl:10-21). A code flipped to
// u = qs + 128 sits under the exponent of 1024 as 1024 + u, and
// fma(1024 + u, d, -1152 d) = qs d exactly.
__device__ __forceinline__ void decode_half_q8_0(uint4 c, uint16_t dbits, float (&wk)[16]) {
  const float d = half_to_float(dbits);
  const float bias = -1152.0f * d;
  const uint32_t words[4] = {c.x ^ 0x80808080u, c.y ^ 0x80808080u, c.z ^ 0x80808080u,
                             c.w ^ 0x80808080u};
  uint32_t kExp;
  asm("v_mov_b32 %0, 0x64006400" : "=v"(kExp));
  constexpr uint32_t kMask = 0x00FF00FFu;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const half2v e = __builtin_bit_cast(half2v, (words[w] & kMask) | (kExp & ~kMask));
    const half2v o = __builtin_bit_cast(half2v, ((words[w] >> 8) & kMask) | (kExp & ~kMask));
    wk[4 * w + 0] = __builtin_fmaf((float)e.x, d, bias);
    wk[4 * w + 1] = __builtin_fmaf((float)o.x, d, bias);
    wk[4 * w + 2] = __builtin_fmaf((float)e.y, d, bias);
    wk[4 * w + 3] = __builtin_fmaf((float)o.y, d, bias);
  }
}

// Orders a wave's LDS accesses around it (a wave's LDS instructions execute
// in program order; this keeps the compiler from moving them).
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// The order of a wave's steps, the same for every tile of a product: at step
// t, block b reads group g (16 bits: g, and bit 15 when b's range is
// already done and its inputs are zeros). Step flags: kOpens (first step of
// a pass: the blocks start from zero), kCloses (last step: the pass's sums
// join the totals), kPads (some block's inputs are zeros). Built on the host.
constexpr int kMaxSteps = 256;
constexpr uint32_t kOpens = 1, kCloses = 2, kPads = 4;

template <int NB>
struct Schedule {
  static constexpr int kWords = NB / 2;  // two blocks per word
  int steps;
  uint32_t flags[kMaxSteps / 8];  // 4 bits per step
  uint32_t word[kMaxSteps * kWords];
  int16_t pass_start[kRanges / NB + 1];  // first step of pass p; steps at the end
};

// One step's schedule words, read ahead into scalar registers.
template <int NB>
struct StepInfo {
  uint32_t word[Schedule<NB>::kWords];
  uint32_t flags;
  __device__ uint32_t entry(int b) const { return (word[b / 2] >> (16 * (b & 1))) & 0xFFFFu; }
};

template <int NB>
__device__ __forceinline__ StepInfo<NB> step_info(const Schedule<NB>& S, int t) {
  t = min(t, S.steps - 1);
  StepInfo<NB> I;
#pragma unroll
  for (int i = 0; i < Schedule<NB>::kWords; ++i) I.word[i] = S.word[t * Schedule<NB>::kWords + i];
  I.flags = (S.flags[t >> 3] >> (4 * (t & 7))) & 0xFu;
  return I;
}

// Loads through a buffer resource over [base, base + bytes), with the
// per-lane part of the offset in a VGPR and the uniform part in an SGPR, so
// that no per-lane address arithmetic is needed; loads past the end read 0.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_of(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
}

// A step's inputs pass through LDS, one buffer per wave: 64 lines (line L =
// block L / D, token L % D) of 32 floats, stored 9 float4s apart so that the
// lanes' line reads fall in distinct banks. Lane l loads float4 l % 8 of
// lines 8 i + l / 8.
constexpr int kXLine = 9;
constexpr int kXBuf = 64 * kXLine;

template <int NB, bool GATED>
struct Tile {
  static constexpr int D = Mfma<NB>::kDim;
  static constexpr int kTokenRows = 8 / NB;  // distinct tokens a lane loads
  static constexpr int kMats = GATED ? 2 : 1;
  __amdgpu_buffer_rsrc_t x, codes[kMats], scales[kMats];
  uint32_t x_off[kTokenRows];  // byte offset of float4 lane % 8 of each token it loads
  uint32_t row_group0;         // this lane's row times the row's groups
  float4* x_put;               // its load slots (+ 8 kXLine i)
  const float4* x_get;         // its own line
  int block;                   // lane / D
};

// Step t's inputs: instruction i is lines 8 i .. 8 i + 7, block
// i / (8 / NB). A finished block's lines are loaded (from a valid group)
// and zeroed when staged.
template <int NB, bool GATED>
__device__ __forceinline__ void load_inputs(const Tile<NB, GATED>& T, const StepInfo<NB>& I,
                                            float4 (&G)[8]) {
  constexpr int kPer = Tile<NB, GATED>::kTokenRows;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t g = I.entry(i / kPer) & 0x7FFFu;
    G[i] = __builtin_bit_cast(
        float4, __builtin_amdgcn_raw_buffer_load_b128(T.x, T.x_off[i % kPer], 128 * g, 0));
  }
}

template <int NB, bool GATED>
__device__ __forceinline__ void stage_inputs(const Tile<NB, GATED>& T, const StepInfo<NB>& I,
                                             float4 (&G)[8]) {
  constexpr int kPer = Tile<NB, GATED>::kTokenRows;
  if (I.flags & kPads) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if (I.entry(i / kPer) & 0x8000u) G[i] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) T.x_put[8 * kXLine * i] = G[i];
}

// A lane's weights for a step: one group of each matrix. A gated product's
// matrices are Q4_0; a plain one's may be Q4_1 or Q8_0 as well.
template <bool GATED, int F>
struct Weights {
  uint4 c[GATED ? 2 : 1];
  uint16_t d[GATED ? 2 : 1];
};
template <>
struct Weights<false, kQ8_0> {
  uint4 c[2];  // code bytes 0..15, 16..31
  uint16_t d[1];
};
template <>
struct Weights<false, kQ4_1> {
  uint4 c[1];
  uint32_t d[1];  // d, then m in the high half
};

template <int NB, bool GATED, int F>
__device__ __forceinline__ void load_weights(const Tile<NB, GATED>& T, const StepInfo<NB>& I,
                                             Weights<GATED, F>& W) {
  // this lane's block's group
  uint32_t g = I.entry(0);
#pragma unroll
  for (int b = 1; b < NB; ++b) g = T.block == b ? I.entry(b) : g;
  const uint32_t blk = T.row_group0 + (g & 0x7FFFu);
#pragma unroll
  for (int m = 0; m < Tile<NB, GATED>::kMats; ++m) {
    if constexpr (F == kQ8_0) {
      W.c[0] = __builtin_bit_cast(uint4,
                                  __builtin_amdgcn_raw_buffer_load_b128(T.codes[m], 32 * blk, 0, 0));
      W.c[1] = __builtin_bit_cast(
          uint4, __builtin_amdgcn_raw_buffer_load_b128(T.codes[m], 32 * blk + 16, 0, 0));
      W.d[0] = __builtin_amdgcn_raw_buffer_load_b16(T.scales[m], 2 * blk, 0, 0);
    } else if constexpr (F == kQ4_1) {
      W.c[0] = __builtin_bit_cast(uint4,
                                  __builtin_amdgcn_raw_buffer_load_b128(T.codes[m], 16 * blk, 0, 0));
      W.d[0] = __builtin_amdgcn_raw_buffer_load_b32(T.scales[m], 4 * blk, 0, 0);
    } else {
      W.c[m] = __builtin_bit_cast(uint4,
                                  __builtin_amdgcn_raw_buffer_load_b128(T.codes[m], 16 * blk, 0, 0));
      W.d[m] = __builtin_amdgcn_raw_buffer_load_b16(T.scales[m], 2 * blk, 0, 0);
    }
  }
}

// Products for k = 16 H .. 16 H + 15 of a step, per matrix: decode the
// weights, then the 16 products per block.
template <int NB, bool GATED, int F, int H>
__device__ __forceinline__ void chain_half(const float4 (&xv)[8], const Weights<GATED, F>& W,
                                           typename Mfma<NB>::Acc (&acc)[GATED ? 2 : 1]) {
#pragma unroll
  for (int m = 0; m < (GATED ? 2 : 1); ++m) {
    float wk[16];
    if constexpr (F == kQ8_0) {
      decode_half_q8_0(W.c[H], W.d[0], wk);
    } else if constexpr (F == kQ4_1) {
      decode_half_q4_1<H>(W.c[0], W.d[0], wk);
    } else {
      decode_half<H>(W.c[m], W.d[m], wk);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float4 x4 = xv[4 * H + i];
      acc[m] = Mfma<NB>::op(wk[4 * i + 0], x4.x, acc[m]);
      acc[m] = Mfma<NB>::op(wk[4 * i + 1], x4.y, acc[m]);
      acc[m] = Mfma<NB>::op(wk[4 * i + 2], x4.z, acc[m]);
      acc[m] = Mfma<NB>::op(wk[4 * i + 3], x4.w, acc[m]);
    }
    __builtin_amdgcn_sched_barrier(0);
  }
}

// One step: read this step's inputs from the wave's LDS buffer, then stage
// step t + 1's there (loaded a step ago; a wave's LDS accesses run in
// order), start the loads of step t + 2's inputs and t + 1's weights, and
// chain this step's 32 products per block, half a group at a time so that
// the decoded weights need few registers. Vector instructions do not run
// beside the fp32 matrix instructions, so each kind is kept in runs.
template <int NB, bool GATED, int F>
__device__ __forceinline__ void chain_step(const Tile<NB, GATED>& T, const StepInfo<NB>& I1,
                                           const StepInfo<NB>& I2, float4 (&G)[8],
                                           const Weights<GATED, F>& W, Weights<GATED, F>& W_next,
                                           typename Mfma<NB>::Acc (&acc)[GATED ? 2 : 1]) {
  float4 xv[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) xv[i] = T.x_get[i];
  __builtin_amdgcn_sched_barrier(0);
  stage_inputs(T, I1, G);
  load_inputs(T, I2, G);
  load_weights(T, I1, W_next);
  // The loads stay here, a step ahead of their use.
  __builtin_amdgcn_sched_barrier(0);
  chain_half<NB, GATED, F, 0>(xv, W, acc);
  chain_half<NB, GATED, F, 1>(xv, W, acc);
  wave_sync();
}

// A pass's range sums kept apart, when the passes of a tile are split over
// the workgroup's waves: range NB p + b's sum for output (row, token) at
// sums[(NB p + b) D^2 + row D + token].
template <int NB>
__device__ __forceinline__ void store_pass(typename Mfma<NB>::Acc& acc, float* sums, int pass) {
  using M = Mfma<NB>;
  constexpr int S = M::kSlots, D = M::kDim;
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int b = 0; b < NB; ++b) {
#pragma unroll
    for (int o = 0; o < S; ++o)
      sums[(NB * pass + b) * D * D + M::slot_row(lane, o) * D + lane % D] = acc[S * b + o];
  }
#pragma unroll
  for (int i = 0; i < NB * S; ++i) acc[i] = 0.0f;
}

// A pass's range sums join the totals in range order.
template <int NB>
__device__ __forceinline__ void close_pass(typename Mfma<NB>::Acc& acc,
                                           float (&total)[Mfma<NB>::kSlots]) {
  constexpr int S = Mfma<NB>::kSlots;
#pragma unroll
  for (int b = 0; b < NB; ++b) {
#pragma unroll
    for (int o = 0; o < S; ++o) total[o] = total[o] + acc[S * b + o];
  }
#pragma unroll
  for (int i = 0; i < NB * S; ++i) acc[i] = 0.0f;
}

// Step t, with the schedule of steps t .. t + 2 in hand; starts reading
// step t + 3's (first used a step later, so its wait costs nothing).
template <int NB, bool GATED, int F, bool SPLIT>
__device__ __forceinline__ void run_step(const Tile<NB, GATED>& T, const Schedule<NB>& S, int t,
                                         StepInfo<NB> (&I)[4], float4 (&G)[8],
                                         const Weights<GATED, F>& W, Weights<GATED, F>& W_next,
                                         typename Mfma<NB>::Acc (&acc)[GATED ? 2 : 1],
                                         float (&total)[GATED ? 2 : 1][Mfma<NB>::kSlots],
                                         float* sums, int& pass) {
  constexpr int D2 = Mfma<NB>::kDim * Mfma<NB>::kDim;
  I[3] = step_info(S, t + 3);
  chain_step<NB, GATED, F>(T, I[1], I[2], G, W, W_next, acc);
  if (I[0].flags & kCloses) {
#pragma unroll
    for (int m = 0; m < (GATED ? 2 : 1); ++m) {
      if constexpr (SPLIT) {
        store_pass<NB>(acc[m], sums + m * kRanges * D2, pass);
      } else {
        close_pass<NB>(acc[m], total[m]);
      }
    }
    ++pass;
  }
  I[0] = I[1];
  I[1] = I[2];
  I[2] = I[3];
}

// Waves of a workgroup that split a tile's passes: one pass (four ranges)
// a wave.
constexpr int kSplitWaves = 8;

// Grid: x = D-row tiles, y = groups of kTileWaves x D tokens, a wave's own
// D tokens. SPLIT (one token tile, of a step of D tokens at most): y = the
// token tile, and the workgroup's kSplitWaves waves share it, wave w taking
// the passes from w (kRanges / NB) / kSplitWaves on; their range sums meet
// in LDS and are added in range order, the same sums in the same order.
// Rows and tokens past the ends are read clamped and not stored.
template <int NB, bool GATED, int F = kQ4_0, bool SPLIT = false>
__global__ __launch_bounds__((SPLIT ? kSplitWaves : kTileWaves) * 64) void gemm_ranges(
    const DevStep* __restrict__ step, QMatrix w, QMatrix up,
    const float* __restrict__ x, int x_stride, uint32_t x_bytes, float* __restrict__ y,
    int y_stride, const uint32_t* __restrict__ edits, int layer, uint32_t edit_stride,
    const Schedule<NB> S) {
  using M = Mfma<NB>;
  constexpr int D = M::kDim;
  constexpr int SL = M::kSlots;
  constexpr int kMats = GATED ? 2 : 1;
  constexpr int kWaves = SPLIT ? kSplitWaves : kTileWaves;
  constexpr int kPassesPerWave = (kRanges / NB) / kSplitWaves;
  static_assert(!SPLIT || (NB == 4 && kPassesPerWave >= 1), "split tiles are 16 x 16");
  __shared__ float4 staged[kWaves][kXBuf];
  __shared__ float sums[SPLIT ? kMats * kRanges * D * D : 1];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int tokens = (int)step->tokens;
  const int token0 = SPLIT ? (int)blockIdx.y * D : (int)(blockIdx.y * kTileWaves + wave) * D;
  // Whole waves (whole workgroups when SPLIT) leave, before any barrier.
  if (token0 >= tokens) return;
  const int groups = w.cols >> 5;

  Tile<NB, GATED> T;
  T.block = lane / D;
  const int row = min((int)blockIdx.x * D + lane % D, w.rows - 1);
  // The tile's member (a fused product over members placed apart): members
  // split at multiples of 32 rows, so a tile lies in one.
  const MemberRow mr = member_row(w, (int)blockIdx.x * D);
  const int member_rows = w.split[1] != 0 && (int)blockIdx.x * D >= w.split[1] ? w.rows - w.split[1]
                          : w.split[0] != 0 && (int)blockIdx.x * D >= w.split[0]
                              ? (w.split[1] != 0 ? w.split[1] : w.rows) - w.split[0]
                          : w.split[0] != 0 ? w.split[0]
                                            : w.rows;
  const uint32_t blocks = (uint32_t)member_rows * (uint32_t)groups;
  T.row_group0 = (uint32_t)(row - ((int)blockIdx.x * D - mr.row)) * (uint32_t)groups;
  T.codes[0] = buffer_of(mr.codes, (uint32_t)code_bytes(F) * blocks);
  T.scales[0] = buffer_of(mr.scales, 2u * (uint32_t)scale_halves(F) * blocks);
  if (GATED) {
    T.codes[kMats - 1] = buffer_of(up.codes, 16 * blocks);
    T.scales[kMats - 1] = buffer_of(up.scales, 2 * blocks);
  }
  T.x = buffer_of(x, x_bytes);
#pragma unroll
  for (int i = 0; i < Tile<NB, GATED>::kTokenRows; ++i) {
    // line 8 i + lane / 8 is token (8 i + lane / 8) % D
    const int tok = min(token0 + (8 * i + (lane >> 3)) % D, tokens - 1);
    T.x_off[i] = 4u * ((uint32_t)tok * (uint32_t)x_stride + 4u * (uint32_t)(lane & 7));
  }
  T.x_put = staged[wave] + (lane >> 3) * kXLine + (lane & 7);
  T.x_get = staged[wave] + lane * kXLine;

  typename M::Acc acc[kMats];
  float total[kMats][SL];
#pragma unroll
  for (int m = 0; m < kMats; ++m) {
#pragma unroll
    for (int i = 0; i < NB * SL; ++i) acc[m][i] = 0.0f;
#pragma unroll
    for (int o = 0; o < SL; ++o) total[m][o] = 0.0f;
  }

  // This wave's steps: all of them, or its passes' when SPLIT.
  int pass = SPLIT ? wave * kPassesPerWave : 0;
  const int t0 = SPLIT ? S.pass_start[pass] : 0;
  const int t1 = SPLIT ? S.pass_start[pass + kPassesPerWave] : S.steps;
  // Step t0 staged; step t0 + 1's inputs and step t0's weights in registers.
  StepInfo<NB> I[4];
  I[0] = step_info(S, t0);
  I[1] = step_info(S, t0 + 1);
  I[2] = step_info(S, t0 + 2);
  float4 G[8];
  load_inputs(T, I[0], G);
  stage_inputs(T, I[0], G);
  load_inputs(T, I[1], G);
  Weights<GATED, F> W0, W1;
  load_weights(T, I[0], W0);
  wave_sync();
  for (int t = t0; t < t1; t += 2) {
    run_step<NB, GATED, F, SPLIT>(T, S, t, I, G, W0, W1, acc, total, sums, pass);
    if (t + 1 >= t1) break;
    run_step<NB, GATED, F, SPLIT>(T, S, t + 1, I, G, W1, W0, acc, total, sums, pass);
  }

  if constexpr (SPLIT) {
    // Output i of the tile (row i / D, token i % D): its 32 range sums in
    // range order from +0, as the unsplit close adds them.
    __syncthreads();
    if (threadIdx.x >= D * D) return;
    const int i = threadIdx.x;
    const int tk = token0 + i % D, n = (int)blockIdx.x * D + i / D;
    if (tk >= tokens || n >= w.rows) return;
    float tot[kMats];
#pragma unroll
    for (int m = 0; m < kMats; ++m) {
      tot[m] = 0.0f;
#pragma unroll
      for (int r = 0; r < kRanges; ++r) tot[m] = tot[m] + sums[(m * kRanges + r) * D * D + i];
    }
    float* yr = y + (size_t)tk * y_stride;
    if (!GATED) {
      yr[n] = tot[0];
    } else {
      const uint32_t position = step->position + (step->variants ? 0u : (uint32_t)tk);
      const uint32_t* table =
          edits && step->variants ? edits + (size_t)tk * edit_stride : edits;
      float v = gelu_tanh(tot[0]) * tot[kMats - 1];
      if (table) v = apply_edits(table, layer, (uint32_t)n, position, v);
      yr[n] = v;
    }
    return;
  }

  const int tok = token0 + lane % D;
  if (tok >= tokens) return;
  float* yrow = y + (size_t)tok * y_stride;
  const int row0 = blockIdx.x * D;
  // A variants step: every row at the step's position, under its own table.
  const uint32_t position = step->position + (step->variants ? 0u : (uint32_t)tok);
  if (edits && step->variants) edits += (size_t)tok * edit_stride;
#pragma unroll
  for (int o = 0; o < SL; ++o) {
    const int n = row0 + M::slot_row(lane, o);
    if (n >= w.rows) continue;
    if (!GATED) {
      yrow[n] = total[0][o];
    } else {
      float v = gelu_tanh(total[0][o]) * total[kMats - 1][o];
      if (edits) v = apply_edits(edits, layer, (uint32_t)n, position, v);
      yrow[n] = v;
    }
  }
}

// Pass p holds ranges NB p .. NB p + NB - 1 and runs for its longest range;
// passes of empty ranges are left out (their sums add zero). False when the
// product has more steps than a schedule holds.
template <int NB>
bool build_schedule(int groups, Schedule<NB>& S) {
  S = Schedule<NB>{};
  int t = 0;
  for (int p = 0; p < kRanges / NB; ++p) {
    S.pass_start[p] = (int16_t)t;
    int lo[NB], len[NB], steps = 0;
    for (int b = 0; b < NB; ++b) {
      const int r = NB * p + b;
      lo[b] = r * groups / kRanges;
      len[b] = (r + 1) * groups / kRanges - lo[b];
      steps = std::max(steps, len[b]);
    }
    for (int s = 0; s < steps; ++s, ++t) {
      if (t >= kMaxSteps) return false;
      uint32_t f = (s == 0 ? kOpens : 0u) | (s + 1 == steps ? kCloses : 0u);
      for (int b = 0; b < NB; ++b) {
        const bool done = s >= len[b];
        const uint32_t g = (uint32_t)std::min(lo[b] + s, groups - 1);
        const uint32_t e = g | (done ? 0x8000u : 0u);
        S.word[t * Schedule<NB>::kWords + b / 2] |= e << (16 * (b & 1));
        if (done) f |= kPads;
      }
      S.flags[t >> 3] |= f << (4 * (t & 7));
    }
  }
  S.steps = t;
  S.pass_start[kRanges / NB] = (int16_t)t;
  return t > 0;
}

template <int NB, bool GATED, int F = kQ4_0, bool SPLIT = false>
hipError_t launch_ranges(hipStream_t s, const DevStep* step, QMatrix w, QMatrix up,
                         const float* x, int x_stride, float* y, int y_stride, int max_tokens,
                         const uint32_t* edits, int layer, uint32_t edit_stride = 0) {
  constexpr int D = Mfma<NB>::kDim;
  const int groups = w.cols >> 5;
  const uint64_t x_bytes = 4ull * (uint64_t)x_stride * (uint64_t)max_tokens;
  const uint64_t codes = (uint64_t)code_bytes(F) * (uint64_t)w.rows * (uint64_t)groups;
  Schedule<NB> S;
  if (groups >= 0x8000 || x_bytes >= (1ull << 31) || codes >= (1ull << 31) ||
      !build_schedule<NB>(groups, S)) {
    return hipErrorInvalidValue;
  }
  // Split passes need every pass to hold work: a range of a group at least.
  if (SPLIT && groups < kRanges) return hipErrorInvalidValue;
  const int token_span = SPLIT ? D : kTileWaves * D;
  const dim3 grid((w.rows + D - 1) / D, (max_tokens + token_span - 1) / token_span);
  hipLaunchKernelGGL((gemm_ranges<NB, GATED, F, SPLIT>), grid,
                     dim3((SPLIT ? kSplitWaves : kTileWaves) * 64), 0, s, step, w, up, x,
                     x_stride, (uint32_t)x_bytes, y, y_stride, edits, layer, edit_stride, S);
  return hipGetLastError();
}

// A step of at most 16 rows over K of 32 groups or more (a batch of variants)
// fills few waves with one 16 x 16 tile each; such a step splits each tile's
// passes over a workgroup's waves, unless the product has tiles enough to
// fill the chip without (the 262,144-row head has 16,384).
bool split_passes(const QMatrix& w, int max_tokens) {
  return max_tokens <= Mfma<4>::kDim && (w.cols >> 5) >= kRanges &&
         w.rows <= 2048 * Mfma<4>::kDim;
}

}  // namespace

hipError_t launch_gemv(hipStream_t s, const DevStep* step, QMatrix w,
                       const float* x, int x_stride, float* y, int y_stride,
                       int max_tokens, bool last_token) {
  if (w.cols % 32 != 0 || w.rows <= 0) return hipErrorInvalidValue;
  if (has_members(w) && (w.split[0] % 32 != 0 || w.split[1] % 32 != 0 || w.format != kQ4_0))
    return hipErrorInvalidValue;
  if (max_tokens <= 1 || last_token) {
    GemvInput in{};
    in.x = x + (size_t)(last_token ? max_tokens - 1 : 0) * x_stride;
    return launch_gemv_decode(s, step, w, in, 0, y);
  }
  // Tiles of 32 x 32 (two ranges in flight) when they are enough to cover
  // most of the chip's 1,024 SIMDs; else 16 x 16 tiles (four ranges), four
  // times as many.
  // 32 x 32 tiles waste half their columns on 16 tokens or fewer.
  const bool wide = (size_t)w.rows * (size_t)max_tokens >= (size_t)768 * 1024 &&
                    max_tokens > Mfma<4>::kDim;
  if (split_passes(w, max_tokens)) {
    switch (w.format) {
      case kQ4_0:
        return launch_ranges<4, false, kQ4_0, true>(s, step, w, w, x, x_stride, y, y_stride,
                                                    max_tokens, nullptr, 0);
      case kQ4_1:
        return launch_ranges<4, false, kQ4_1, true>(s, step, w, w, x, x_stride, y, y_stride,
                                                    max_tokens, nullptr, 0);
      case kQ8_0:
        return launch_ranges<4, false, kQ8_0, true>(s, step, w, w, x, x_stride, y, y_stride,
                                                    max_tokens, nullptr, 0);
      default:
        return hipErrorInvalidValue;
    }
  }
  switch (w.format) {
    case kQ4_0:
      if (wide)
        return launch_ranges<2, false>(s, step, w, w, x, x_stride, y, y_stride, max_tokens,
                                       nullptr, 0);
      return launch_ranges<4, false>(s, step, w, w, x, x_stride, y, y_stride, max_tokens, nullptr,
                                     0);
    case kQ4_1:
      if (wide)
        return launch_ranges<2, false, kQ4_1>(s, step, w, w, x, x_stride, y, y_stride,
                                              max_tokens, nullptr, 0);
      return launch_ranges<4, false, kQ4_1>(s, step, w, w, x, x_stride, y, y_stride, max_tokens,
                                            nullptr, 0);
    case kQ8_0:
      if (wide)
        return launch_ranges<2, false, kQ8_0>(s, step, w, w, x, x_stride, y, y_stride,
                                              max_tokens, nullptr, 0);
      return launch_ranges<4, false, kQ8_0>(s, step, w, w, x, x_stride, y, y_stride, max_tokens,
                                            nullptr, 0);
    default:
      return hipErrorInvalidValue;
  }
}

hipError_t launch_gated(hipStream_t s, const DevStep* step, QMatrix gate,
                        QMatrix up, const float* x, float* act,
                        int max_tokens, const uint32_t* edits, int layer, uint32_t edit_stride) {
  if (gate.cols % 32 != 0 || gate.rows != up.rows || gate.cols != up.cols ||
      gate.format != kQ4_0 || up.format != kQ4_0)
    return hipErrorInvalidValue;
  if (max_tokens <= 1) {
    GemvInput in{};
    in.x = x;
    return launch_gated_decode(s, step, gate, up, in, 0, act, edits, layer);
  }
  if (split_passes(gate, max_tokens)) {
    return launch_ranges<4, true, kQ4_0, true>(s, step, gate, up, x, gate.cols, act, gate.rows,
                                               max_tokens, edits, layer, edit_stride);
  }
  return launch_ranges<2, true>(s, step, gate, up, x, gate.cols, act, gate.rows, max_tokens, edits,
                               layer, edit_stride);
}

}  // namespace frz
