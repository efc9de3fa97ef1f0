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

#include "edit_common.h"
#include "kernels.h"
#include "numerics.h"

namespace frz {
namespace {

__device__ __forceinline__ float half_to_float(uint16_t h) {
  return (float)__builtin_bit_cast(_Float16, h);
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
// Half H of a group: weights 16 H .. 16 H + 15; words W0 .. W0 + N - 1 of
// it (4 weights a word) into wk[0 .. 4 N - 1].
template <int H, int W0 = 0, int N = 4>
__device__ __forceinline__ void decode_half(uint4 c, uint16_t dbits, float (&wk)[4 * N]) {
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
  for (int j = 0; j < N; ++j) {
    const uint32_t word = words[W0 + j];
    // even: bytes 0 and 2 of the word; odd: bytes 1 and 3.
    const half2v e = __builtin_bit_cast(half2v, (word & kMask) | (kExp & ~kMask));
    const half2v o = __builtin_bit_cast(half2v, ((word >> 8) & kMask) | (kExp & ~kMask));
    wk[4 * j + 0] = __builtin_fmaf((float)e.x, scale, bias);
    wk[4 * j + 1] = __builtin_fmaf((float)o.x, scale, bias);
    wk[4 * j + 2] = __builtin_fmaf((float)e.y, scale, bias);
    wk[4 * j + 3] = __builtin_fmaf((float)o.y, scale, bias);
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

// Two Q4_0 chains on the same inputs (gate and up, or two tiles), quarter Q
// (8 k) of half H of a step: each chain's 8 weights decoded, then their
// products alternating, so that neither chain waits on its own last product.
template <int H, int Q>
__device__ __forceinline__ void chain_quarter_two(const float4 (&xv)[8],
                                                  const Weights<true, kQ4_0>& W,
                                                  typename Mfma<4>::Acc (&acc)[2]) {
  float wa[8], wb[8];
  decode_half<H, 2 * Q, 2>(W.c[0], W.d[0], wa);
  decode_half<H, 2 * Q, 2>(W.c[1], W.d[1], wb);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const float4 x4 = xv[4 * H + 2 * Q + i];
    const float xs[4] = {x4.x, x4.y, x4.z, x4.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      acc[0] = Mfma<4>::op(wa[4 * i + j], xs[j], acc[0]);
      acc[1] = Mfma<4>::op(wb[4 * i + j], xs[j], acc[1]);
    }
  }
  __builtin_amdgcn_sched_barrier(0);
}

template <int H>
__device__ __forceinline__ void chain_half_two(const float4 (&xv)[8], const Weights<true, kQ4_0>& W,
                                               typename Mfma<4>::Acc (&acc)[2]) {
  chain_quarter_two<H, 0>(xv, W, acc);
  chain_quarter_two<H, 1>(xv, W, acc);
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
template <int NB, bool GATED, int F>
__device__ __forceinline__ void run_step(const Tile<NB, GATED>& T, const Schedule<NB>& S, int t,
                                         StepInfo<NB> (&I)[4], float4 (&G)[8],
                                         const Weights<GATED, F>& W, Weights<GATED, F>& W_next,
                                         typename Mfma<NB>::Acc (&acc)[GATED ? 2 : 1],
                                         float (&total)[GATED ? 2 : 1][Mfma<NB>::kSlots]) {
  I[3] = step_info(S, t + 3);
  chain_step<NB, GATED, F>(T, I[1], I[2], G, W, W_next, acc);
  if (I[0].flags & kCloses) {
#pragma unroll
    for (int m = 0; m < (GATED ? 2 : 1); ++m) close_pass<NB>(acc[m], total[m]);
  }
  I[0] = I[1];
  I[1] = I[2];
  I[2] = I[3];
}

// Grid: x = D-row tiles, y = groups of kTileWaves x D tokens, a wave's own
// D tokens. Rows and tokens past the ends are read clamped and not stored.
template <int NB, bool GATED, int F = kQ4_0>
__global__ __launch_bounds__(kTileWaves * 64) void gemm_ranges(
    const DevStep* __restrict__ step, QMatrix w, QMatrix up,
    const float* __restrict__ x, int x_stride, uint32_t x_bytes, float* __restrict__ y,
    int y_stride, const uint32_t* __restrict__ edits, int layer, uint32_t edit_stride,
    const Schedule<NB> S) {
  using M = Mfma<NB>;
  constexpr int D = M::kDim;
  constexpr int SL = M::kSlots;
  constexpr int kMats = GATED ? 2 : 1;
  __shared__ float4 staged[kTileWaves][kXBuf];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int tokens = (int)step->tokens;
  const int token0 = (int)(blockIdx.y * kTileWaves + wave) * D;
  // Whole waves leave (there is no barrier).
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

  // Step 0 staged; step 1's inputs and step 0's weights in registers.
  StepInfo<NB> I[4];
  I[0] = step_info(S, 0);
  I[1] = step_info(S, 1);
  I[2] = step_info(S, 2);
  float4 G[8];
  load_inputs(T, I[0], G);
  stage_inputs(T, I[0], G);
  load_inputs(T, I[1], G);
  Weights<GATED, F> W0, W1;
  load_weights(T, I[0], W0);
  wave_sync();
  for (int t = 0; t < S.steps; t += 2) {
    run_step<NB, GATED, F>(T, S, t, I, G, W0, W1, acc, total);
    if (t + 1 >= S.steps) break;
    run_step<NB, GATED, F>(T, S, t + 1, I, G, W1, W0, acc, total);
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
  return t > 0;
}

// ---- steps of at most 16 rows: a pass a wave ------------------------------
// A step of at most 16 rows (a batch of variants, a prompt's last rows) makes
// one 16 x 16 tile per 16 output rows. A workgroup takes a tile and its eight
// waves a pass each. A pass is any four of the 32 ranges, chained in the four
// blocks of one v_mfma_f32_16x16x1_4b_f32 per k; the range sums meet in LDS
// by range index and are added in range order, so which ranges share a pass
// changes no bit, and the host puts ranges of one length together: a pass
// runs past a range's end only where the lengths mix. Each lane loads its
// own operands straight from memory - its row's block of its range's group
// and its token's 32 inputs of that group, which the matrix instruction reads
// from the lane that loaded them - and a wave keeps its loads DEPTH steps
// ahead of its products. Loads past a range's end read zeros through the
// buffer resources' bounds: a zero input times a zero weight adds a zero.
constexpr int kPassWaves = kRanges / 4;
constexpr uint32_t kPastEnd = 0x40000000u;  // an offset past every buffer here

struct PassOrder {
  uint32_t word[kPassWaves];  // byte b of word p: the range in block b of pass p
  // Where range r's sums lie in the workgroup's LDS, in floats from the
  // sums' base (matrix 0, output 0): pass p's block b, p within the tile's
  // half, its wave's slot-0 region. The host computes them, so that the
  // combine adds each range's offset to its output's.
  uint32_t sum_at[kRanges];
};

// Pass p's word, p wave-uniform (the selects stay scalar).
__device__ __forceinline__ uint32_t pass_word(const PassOrder& o, int p) {
  uint32_t v = o.word[0];
#pragma unroll
  for (int i = 1; i < kPassWaves; ++i) v = p == i ? o.word[i] : v;
  return v;
}

__device__ __forceinline__ int range_lo(int r, int groups) { return (r * groups) >> 5; }

template <bool GATED, int F>
struct PassLane {
  static constexpr int kMats = GATED ? 2 : 1;
  __amdgpu_buffer_rsrc_t x, codes[kMats], scales[kMats];
  uint32_t x_off[2];  // what lane l moves to LDS: tokens l / 8 and 8 + l / 8, its float4
  int lo[4], len[4];  // the pass's ranges, block by block (wave-uniform)
  uint32_t blk0[kMats];  // each matrix's block of the lane's row's range's first group
  int my_len;            // its range's groups
  uint32_t x_read;       // its own line in a wave's slot, XOR-swizzled by float4
};

// A step's inputs in a wave's LDS slot: line L (block L / 16, token L % 16,
// the 32 inputs of the block's group) at L * 128 bytes, its float4 f at
// 16 (f ^ (L % 8)) within, so that the lanes' reads of float4 f fall in
// distinct banks. The loads go straight to LDS: instruction i writes the
// slot's bytes 1024 i + 16 l from lane l, which is line 8 i + l / 8 (block
// i / 2, token 8 (i % 2) + l / 8), float4 (l % 8) ^ (l / 8).
constexpr int kSlotFloat4s = 64 * 8;
typedef __attribute__((address_space(3))) void* LdsPtr;

// 16 bytes a lane from r at voffset + soffset to lds + 16 lane.
__device__ __forceinline__ void load_to_lds(__amdgpu_buffer_rsrc_t r, float4* lds, uint32_t voffset,
                                            uint32_t soffset) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (LdsPtr)lds, 16, voffset, (int)soffset, 0, 0);
}

// Step s's inputs into the wave's slot; a block past its range's end reads
// zeros.
template <bool GATED, int F>
__device__ __forceinline__ void load_pass_inputs(const PassLane<GATED, F>& L, int s,
                                                 float4* slot) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int b = i >> 1;
    const uint32_t at = s < L.len[b] ? 128u * (uint32_t)(L.lo[b] + s) : kPastEnd;
    load_to_lds(L.x, slot + 64 * i, L.x_off[i & 1], at);
  }
}

// Step s's weights of a lane: past its range's end, zeros.
template <bool GATED, int F>
__device__ __forceinline__ void load_pass_weights(const PassLane<GATED, F>& L, int s,
                                                  Weights<GATED, F>& W) {
  const bool live = s < L.my_len;
#pragma unroll
  for (int m = 0; m < PassLane<GATED, F>::kMats; ++m) {
    const uint32_t blk = L.blk0[m] + (uint32_t)s;
    if constexpr (F == kQ8_0) {
      const uint32_t co = live ? 32u * blk : kPastEnd;
      W.c[0] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(L.codes[m], co, 0, 0));
      W.c[1] = __builtin_bit_cast(uint4,
                                  __builtin_amdgcn_raw_buffer_load_b128(L.codes[m], co + 16, 0, 0));
      W.d[0] = __builtin_amdgcn_raw_buffer_load_b16(L.scales[m], live ? 2u * blk : kPastEnd, 0, 0);
    } else if constexpr (F == kQ4_1) {
      W.c[0] = __builtin_bit_cast(
          uint4, __builtin_amdgcn_raw_buffer_load_b128(L.codes[m], live ? 16u * blk : kPastEnd, 0, 0));
      W.d[0] = __builtin_amdgcn_raw_buffer_load_b32(L.scales[m], live ? 4u * blk : kPastEnd, 0, 0);
    } else {
      W.c[m] = __builtin_bit_cast(
          uint4, __builtin_amdgcn_raw_buffer_load_b128(L.codes[m], live ? 16u * blk : kPastEnd, 0, 0));
      W.d[m] = __builtin_amdgcn_raw_buffer_load_b16(L.scales[m], live ? 2u * blk : kPastEnd, 0, 0);
    }
  }
}

// A step's 32 products per block and chain.
template <bool GATED, int F>
__device__ __forceinline__ void pass_products(const float4 (&xv)[8], const Weights<GATED, F>& W,
                                              typename Mfma<4>::Acc (&acc)[GATED ? 2 : 1]) {
  if constexpr (GATED && F == kQ4_0) {
    chain_half_two<0>(xv, W, acc);
    chain_half_two<1>(xv, W, acc);
  } else {
    chain_half<4, GATED, F, 0>(xv, W, acc);
    chain_half<4, GATED, F, 1>(xv, W, acc);
  }
}

// One step: the lane's line from the wave's slot, then the 32 products per
// block.
template <bool GATED, int F>
__device__ __forceinline__ void pass_step(const PassLane<GATED, F>& L, const float4* slot,
                                          const Weights<GATED, F>& W,
                                          typename Mfma<4>::Acc (&acc)[GATED ? 2 : 1]) {
  const char* line = reinterpret_cast<const char*>(slot);
  float4 xv[8];
#pragma unroll
  for (int f = 0; f < 8; ++f)
    xv[f] = *reinterpret_cast<const float4*>(line + (L.x_read ^ (16u * (uint32_t)f)));
  pass_products(xv, W, acc);
}

// Waits for the LDS reads in flight (lgkmcnt 0, every other count left
// free): a slot's reads are done before new loads are aimed at it.
__device__ __forceinline__ void lds_reads_done() { __builtin_amdgcn_s_waitcnt(0xC07F); }

// What a pass kernel's two chains a lane are, when it has two: the gate and
// up rows of one neuron (GELU and pins to close), or rows n and n + 16 of
// one matrix (a pair of tiles on the same inputs).
constexpr int kPlainKind = 0, kGatedKind = 1, kPairKind = 2;

// Grid: x = 16-row tiles (32-row pairs); y = the halves of a split tile
// (HALVES = 2: the workgroup of half h takes passes 4 h .. 4 h + 3, which
// hold ranges 16 h .. 16 h + 15; half 0 writes their prefix to y, half 1
// each range's sum to parts). Rows past the end are read clamped and not
// stored; tokens past the step's read clamped and not stored. STEPS: the
// longest range's groups (every pass is that long or one shorter), or 0 for
// a loop over any length.
template <int KIND, int F, int STEPS, int HALVES>
__global__ __launch_bounds__(kPassWaves / HALVES * 64, 4 / HALVES) void pass_tiles_kernel(
    const DevStep* __restrict__ step, QMatrix w, QMatrix up, const float* __restrict__ x,
    int x_stride, int max_tokens, float* __restrict__ y, int y_stride,
    const uint32_t* __restrict__ edits, int layer, uint32_t edit_stride, PassOrder order,
    float* __restrict__ parts, size_t parts_stride) {
  using M = Mfma<4>;
  constexpr bool GATED = KIND == kGatedKind, PAIR = KIND == kPairKind, TWO = KIND != kPlainKind;
  constexpr int D = M::kDim, SL = M::kSlots;
  constexpr int kMats = TWO ? 2 : 1;
  constexpr int kWaves = kPassWaves / HALVES, kHalfRanges = kRanges / HALVES;
  static_assert(!TWO || HALVES == 1, "two chains a lane combine in their workgroup");
  // Input slots, a wave's 8 KB each: one when a pass is at most two steps
  // (the second reuses it), else a ring of three for four waves or two for
  // eight (the CU's 160 KB). Separate arrays, so that a read of one waits
  // only for its own loads.
  constexpr int kSlots = STEPS >= 1 && STEPS <= 2 ? 1 : kWaves == 4 && STEPS > 0 ? 3 : 2;
  __shared__ __align__(16) float4 slot0[kWaves * kSlotFloat4s];
  __shared__ __align__(16) float4 slot1[kSlots > 1 ? kWaves * kSlotFloat4s : 1];
  __shared__ __align__(16) float4 slot2[kSlots > 2 ? kWaves * kSlotFloat4s : 1];
  // Once a wave's chains are done, its slot-0 region holds its range sums.
  static_assert(kMats * 4 * D * D <= 4 * kSlotFloat4s, "a wave's sums exceed its slot");
  float* sums = reinterpret_cast<float*>(slot0);
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int groups = w.cols >> 5;
  const int row0 = (int)blockIdx.x * D * (PAIR ? 2 : 1);
  float4* const slots[3] = {slot0 + wave * kSlotFloat4s, slot1 + (kSlots > 1 ? wave : 0) * kSlotFloat4s,
                            slot2 + (kSlots > 2 ? wave : 0) * kSlotFloat4s};

  // The combining thread's output (row i % D, token i / D) and, gated, its
  // table's pin words for the layer, read now and used at the end. Rows of
  // the buffers past the step's tokens are read, not stored.
  const int i_out = t & (D * D - 1);
  const int tk_out = min(i_out / D, max_tokens - 1);
  // The step's fields the combine uses, loaded now through vector
  // registers: scalar loads return out of order, so a scalar read of the
  // step would be waited for with the arguments', before the first weight
  // load; these land with the passes' loads, which the combine waits for.
  int zero = 0;
  asm volatile("" : "+v"(zero));
  const uint32_t* step_words = reinterpret_cast<const uint32_t*>(step) + zero;
  const uint2 step_pt = *reinterpret_cast<const uint2*>(step_words);  // position, tokens
  const uint32_t step_variants = GATED ? step_words[offsetof(DevStep, variants) / 4] : 0u;
  static_assert(offsetof(DevStep, position) == 0 && offsetof(DevStep, tokens) == 4,
                "position and tokens lead the step record");
  // A variants step's rows each have an edit table (edit_stride apart; the
  // stride is 0 for any other step).
  const uint32_t* table = edits ? edits + (size_t)tk_out * edit_stride : nullptr;
  uint2 pins = make_uint2(0u, 0u);
  if (GATED) {
    int at = 2 * layer;
    asm volatile("" : "+v"(at));
    const uint32_t* src = table ? table + at : reinterpret_cast<const uint32_t*>(step);
    pins = make_uint2(src[0], src[1]);
  }

  // The pass: its four ranges and its steps, the longest of them.
  const int half = HALVES == 1 ? 0 : (int)blockIdx.y;
  const uint32_t word = pass_word(order, wave + kWaves * half);
  PassLane<TWO, F> L;
  int steps = 0;
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    const int r = (word >> (8 * b)) & 0xFF;
    L.lo[b] = range_lo(r, groups);
    L.len[b] = range_lo(r + 1, groups) - L.lo[b];
    steps = max(steps, L.len[b]);
  }
  const int r = (word >> (8 * (lane >> 4))) & 0xFF;
  const int lo = range_lo(r, groups);
  L.my_len = range_lo(r + 1, groups) - lo;
  const int row = min(row0 + (lane & (D - 1)), w.rows - 1);
  // The tile's member (a product fused over members placed apart): members
  // split at multiples of 32 rows, so a tile lies in one. Every candidate is
  // read, then selected, so that the arguments' loads are one batch.
  const int s0 = w.split[0], s1 = w.split[1], rows = w.rows;
  const uint8_t* const codes_in[3] = {w.codes, w.member_codes[0], w.member_codes[1]};
  const uint16_t* const scales_in[3] = {w.scales, w.member_scales[0], w.member_scales[1]};
  const int member = s1 != 0 && row0 >= s1 ? 2 : s0 != 0 && row0 >= s0 ? 1 : 0;
  const int member_first = member == 2 ? s1 : member == 1 ? s0 : 0;
  const int member_end = member == 2 ? rows : member == 1 ? (s1 != 0 ? s1 : rows)
                                     : (s0 != 0 ? s0 : rows);
  const uint8_t* member_codes = member == 2 ? codes_in[2] : member == 1 ? codes_in[1] : codes_in[0];
  const uint16_t* member_scales =
      member == 2 ? scales_in[2] : member == 1 ? scales_in[1] : scales_in[0];
  const uint32_t blocks = (uint32_t)(member_end - member_first) * (uint32_t)groups;
  L.blk0[0] = (uint32_t)(row - member_first) * (uint32_t)groups + (uint32_t)lo;
  L.codes[0] = buffer_of(member_codes, (uint32_t)code_bytes(F) * blocks);
  L.scales[0] = buffer_of(member_scales, 2u * (uint32_t)scale_halves(F) * blocks);
  if (GATED) {
    L.codes[kMats - 1] = buffer_of(up.codes, 16 * blocks);
    L.scales[kMats - 1] = buffer_of(up.scales, 2 * blocks);
    L.blk0[kMats - 1] = L.blk0[0];
  } else if (PAIR) {
    // The second tile's row, in the same member (members split at multiples
    // of 32 rows).
    const int row_b = min(row0 + D + (lane & (D - 1)), w.rows - 1);
    L.codes[kMats - 1] = L.codes[0];
    L.scales[kMats - 1] = L.scales[0];
    L.blk0[kMats - 1] = (uint32_t)(row_b - member_first) * (uint32_t)groups + (uint32_t)lo;
  }
  L.x = buffer_of(x, 4u * (uint32_t)x_stride * (uint32_t)max_tokens);
  const uint32_t f_moved = (uint32_t)((lane & 7) ^ (lane >> 3));
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int tok = min(8 * h + (lane >> 3), max_tokens - 1);
    L.x_off[h] = 4u * (uint32_t)tok * (uint32_t)x_stride + 16u * f_moved;
  }
  L.x_read = 128u * (uint32_t)lane + 16u * (uint32_t)(lane & 7);

  typename M::Acc acc[kMats];
#pragma unroll
  for (int m = 0; m < kMats; ++m) {
#pragma unroll
    for (int i = 0; i < 4 * SL; ++i) acc[m][i] = 0.0f;
  }
  if constexpr (STEPS > 0) {
    // Straight-line steps; every load is issued unconditionally, so each
    // wait is for the oldest loads only. Weights ride a ring of STEPS sets
    // (three at most); inputs a ring of kSlots slots. A pass one step
    // shorter skips its last step's products.
    constexpr int kDepth = STEPS < 3 ? STEPS : 3;
    Weights<TWO, F> W[kDepth];
#pragma unroll
    for (int d = 0; d < kSlots; ++d) load_pass_inputs(L, d, slots[d]);
#pragma unroll
    for (int d = 0; d < kDepth; ++d) load_pass_weights(L, d, W[d]);
#pragma unroll
    for (int k = 0; k < STEPS; ++k) {
      const bool live = k + 1 < STEPS || k < steps;
      if constexpr (kSlots == 1) {
        // One slot: the next step's inputs are aimed at it once its line
        // is read (a wave's loads complete in order of issue).
        if (k + 1 < STEPS) {
          const char* line = reinterpret_cast<const char*>(slots[0]);
          float4 xv[8];
#pragma unroll
          for (int f = 0; f < 8; ++f)
            xv[f] = *reinterpret_cast<const float4*>(line + (L.x_read ^ (16u * (uint32_t)f)));
          lds_reads_done();
          load_pass_inputs(L, k + 1, slots[0]);
          if (live) pass_products(xv, W[k % kDepth], acc);
        } else if (live) {
          pass_step(L, slots[0], W[k % kDepth], acc);
        }
      } else {
        if (live) pass_step(L, slots[k % kSlots], W[k % kDepth], acc);
        if (k + kSlots < STEPS) {
          lds_reads_done();
          load_pass_inputs(L, k + kSlots, slots[k % kSlots]);
        }
      }
      if (k + kDepth < STEPS) load_pass_weights(L, k + kDepth, W[k % kDepth]);
    }
  } else {
    // Any length: two slots and two weight sets, one step ahead.
    Weights<TWO, F> W[2];
#pragma unroll
    for (int d = 0; d < 2; ++d) {
      load_pass_inputs(L, d, slots[d]);
      load_pass_weights(L, d, W[d]);
    }
    for (int k = 0; k < steps; k += 2) {
#pragma unroll
      for (int d = 0; d < 2; ++d) {
        if (k + d >= steps) break;
        pass_step(L, slots[d], W[d], acc);
        lds_reads_done();
        load_pass_inputs(L, k + d + 2, slots[d]);
        load_pass_weights(L, k + d + 2, W[d]);
      }
    }
  }

  // Each wave's range sums in its own slot-0 region (whose loads are all
  // spent), block b of matrix m at (m 4 + b) D^2, output (row o, token j)
  // at j D + o: a lane's four rows are one 16-byte write. Pending loads past
  // a pass's end (the loop form's) land first.
  __builtin_amdgcn_s_waitcnt(0x0F70);
  float* mine = sums + wave * 4 * kSlotFloat4s;
#pragma unroll
  for (int m = 0; m < kMats; ++m) {
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const float4 v = make_float4(acc[m][SL * b], acc[m][SL * b + 1], acc[m][SL * b + 2],
                                   acc[m][SL * b + 3]);
      *reinterpret_cast<float4*>(mine + (m * 4 + b) * D * D + (lane & (D - 1)) * D +
                                 M::slot_row(lane, 0)) = v;
    }
  }
  __syncthreads();
  if (t >= D * D) return;
  const int tk = i_out / D, n = row0 + i_out % D;
  if (tk >= (int)step_pt.y || n >= w.rows) return;
  float* yr = y + (size_t)tk * y_stride;
  // Range r's sum for the thread's output (token tk, row i_out % D: at
  // i_out in a block).
  auto range_sum = [&](int m, int r) { return sums[order.sum_at[r] + m * 4 * D * D + i_out]; };
  if (HALVES == 2 && half == 1) {
    float sum[kHalfRanges];
#pragma unroll
    for (int j = 0; j < kHalfRanges; ++j) sum[j] = range_sum(0, kHalfRanges + j);
#pragma unroll
    for (int j = 0; j < kHalfRanges; ++j) parts[j * parts_stride + (size_t)tk * y_stride + n] = sum[j];
    return;
  }
  // Every sum read before the first add: the reads overlap, the adds wait
  // once.
  float part[kMats][kHalfRanges];
#pragma unroll
  for (int m = 0; m < kMats; ++m) {
#pragma unroll
    for (int r2 = 0; r2 < kHalfRanges; ++r2) part[m][r2] = range_sum(m, r2);
  }
  __builtin_amdgcn_sched_barrier(0);
  float tot[kMats];
#pragma unroll
  for (int m = 0; m < kMats; ++m) {
    tot[m] = 0.0f;
#pragma unroll
    for (int r2 = 0; r2 < kHalfRanges; ++r2) tot[m] = tot[m] + part[m][r2];
  }
  if (PAIR) {
    yr[n] = tot[0];
    if (n + D < w.rows) yr[n + D] = tot[1];
  } else if (!GATED) {
    yr[n] = tot[0];
  } else {
    const uint32_t position = step_pt.x + (step_variants ? 0u : (uint32_t)tk);
    float v = gelu_tanh(tot[0]) * tot[kMats - 1];
    if (table && pins.y) v = apply_pin_words(table, pins.x, pins.y, (uint32_t)n, position, v);
    yr[n] = v;
  }
}

// The passes: ranges sorted by length, longest first, four a pass (each
// half's own ranges when a tile is split in halves).
PassOrder pass_order(int groups, int halves) {
  int idx[kRanges];
  for (int r = 0; r < kRanges; ++r) idx[r] = r;
  auto len = [groups](int r) { return ((r + 1) * groups >> 5) - (r * groups >> 5); };
  const int per = kRanges / halves;
  for (int h = 0; h < halves; ++h)
    std::stable_sort(idx + h * per, idx + (h + 1) * per,
                     [&](int a, int b) { return len(a) > len(b); });
  PassOrder o{};
  const int waves = kPassWaves / halves;  // a tile's workgroup: one half's passes
  for (int e = 0; e < kRanges; ++e) {
    o.word[e / 4] |= (uint32_t)idx[e] << (8 * (e % 4));
    // Pass e / 4 is wave (e / 4) % waves of its half's workgroup; each
    // wave's sums sit in its slot-0 region (4 kSlotFloat4s floats), block b
    // of matrix m at (m 4 + b) D x D.
    o.sum_at[idx[e]] =
        (uint32_t)(((e / 4) % waves) * 4 * kSlotFloat4s + (e % 4) * Mfma<4>::kDim * Mfma<4>::kDim);
  }
  return o;
}

template <int KIND, int F>
hipError_t launch_pass_tiles(hipStream_t s, const DevStep* step, QMatrix w, QMatrix up,
                             const float* x, int x_stride, float* y, int y_stride, int max_tokens,
                             const uint32_t* edits, int layer, uint32_t edit_stride = 0,
                             float* parts = nullptr, size_t parts_stride = 0) {
  const int groups = w.cols >> 5;
  const uint64_t x_bytes = 4ull * (uint64_t)x_stride * (uint64_t)max_tokens;
  const uint64_t codes = (uint64_t)code_bytes(F) * (uint64_t)w.rows * (uint64_t)groups;
  // Every range holds a group; offsets stay below the past-the-end one.
  if (groups < kRanges || groups >= 0x8000 || max_tokens > Mfma<4>::kDim ||
      x_bytes >= kPastEnd || codes >= kPastEnd) {
    return hipErrorInvalidValue;
  }
  const int halves = parts ? 2 : 1;
  const PassOrder order = pass_order(groups, halves);
  const int rows_a_block = Mfma<4>::kDim * (KIND == kPairKind ? 2 : 1);
  const dim3 grid((w.rows + rows_a_block - 1) / rows_a_block, halves);
  const int threads = kPassWaves / halves * 64;
  // Straight-line forms for the lengths of the model's products (K = 1,024,
  // 1,152 and 6,912); a loop for the others.
  const int longest = (groups + kRanges - 1) / kRanges;
  auto launch = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, grid, dim3(threads), 0, s, step, w, up, x, x_stride, max_tokens, y,
                       y_stride, edits, layer, edit_stride, order, parts, parts_stride);
  };
  if constexpr (KIND == kPlainKind) {
    if (parts) {
      if (F == kQ4_0 && longest == 7) {
        launch(pass_tiles_kernel<KIND, F, 7, 2>);
      } else {
        launch(pass_tiles_kernel<KIND, F, 0, 2>);
      }
      return hipGetLastError();
    }
  }
  if (longest == 1) {
    launch(pass_tiles_kernel<KIND, F, 1, 1>);
  } else if (longest == 2) {
    launch(pass_tiles_kernel<KIND, F, 2, 1>);
  } else {
    if constexpr (KIND == kPlainKind && F == kQ4_0) {
      if (longest == 7) {
        launch(pass_tiles_kernel<KIND, F, 7, 1>);
        return hipGetLastError();
      }
    }
    launch(pass_tiles_kernel<KIND, F, 0, 1>);
  }
  return hipGetLastError();
}

template <int NB, bool GATED, int F = kQ4_0>
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
  const int token_span = kTileWaves * D;
  const dim3 grid((w.rows + D - 1) / D, (max_tokens + token_span - 1) / token_span);
  hipLaunchKernelGGL((gemm_ranges<NB, GATED, F>), grid, dim3(kTileWaves * 64), 0, s, step, w, up,
                     x, x_stride, (uint32_t)x_bytes, y, y_stride, edits, layer, edit_stride, S);
  return hipGetLastError();
}

// A step of at most 16 rows over K of 32 groups or more (a batch of
// variants, a prompt's last rows) takes a pass a wave.
bool pass_tiles(const QMatrix& w, int max_tokens) {
  return max_tokens <= Mfma<4>::kDim && (w.cols >> 5) >= kRanges;
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
  if (pass_tiles(w, max_tokens)) {
    switch (w.format) {
      case kQ4_0:
        // Thousands of tiles (a vocabulary's head) go a pair to a wave: half
        // the input traffic, two chains in flight.
        if (w.rows >= 2048 * Mfma<4>::kDim)
          return launch_pass_tiles<kPairKind, kQ4_0>(s, step, w, w, x, x_stride, y, y_stride,
                                                     max_tokens, nullptr, 0);
        return launch_pass_tiles<kPlainKind, kQ4_0>(s, step, w, w, x, x_stride, y, y_stride,
                                                    max_tokens, nullptr, 0);
      case kQ4_1:
        return launch_pass_tiles<kPlainKind, kQ4_1>(s, step, w, w, x, x_stride, y, y_stride,
                                                    max_tokens, nullptr, 0);
      case kQ8_0:
        return launch_pass_tiles<kPlainKind, kQ8_0>(s, step, w, w, x, x_stride, y, y_stride,
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

// Splitting pays where a tile's chains are long and the tiles few: down's
// 72 tiles of 216 groups would keep one workgroup of 8 waves on each of 72
// CUs, two chains a SIMD; split, 144 workgroups of 4 waves take one a SIMD.
bool gemv_splits(const QMatrix& w, int max_tokens) {
  return max_tokens > 1 && pass_tiles(w, max_tokens) && (w.cols >> 5) >= 4 * kRanges &&
         w.rows <= 256 * Mfma<4>::kDim && !has_members(w);
}

hipError_t launch_gemv_split(hipStream_t s, const DevStep* step, QMatrix w, const float* x,
                             int x_stride, float* y, int y_stride, int max_tokens, float* parts,
                             size_t parts_stride) {
  if (!gemv_splits(w, max_tokens) || !parts)
    return launch_gemv(s, step, w, x, x_stride, y, y_stride, max_tokens, false);
  switch (w.format) {
    case kQ4_0:
      return launch_pass_tiles<kPlainKind, kQ4_0>(s, step, w, w, x, x_stride, y, y_stride, max_tokens,
                                             nullptr, 0, 0, parts, parts_stride);
    case kQ4_1:
      return launch_pass_tiles<kPlainKind, kQ4_1>(s, step, w, w, x, x_stride, y, y_stride, max_tokens,
                                             nullptr, 0, 0, parts, parts_stride);
    case kQ8_0:
      return launch_pass_tiles<kPlainKind, kQ8_0>(s, step, w, w, x, x_stride, y, y_stride, max_tokens,
                                             nullptr, 0, 0, parts, parts_stride);
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
  if (pass_tiles(gate, max_tokens)) {
    return launch_pass_tiles<kGatedKind, kQ4_0>(s, step, gate, up, x, gate.cols, act, gate.rows,
                                          max_tokens, edits, layer, edit_stride);
  }
  return launch_ranges<2, true>(s, step, gate, up, x, gate.cols, act, gate.rows, max_tokens, edits,
                               layer, edit_stride);
}

}  // namespace frz
