// Prefill products on the bf16 matrix cores (v_mfma_f32_32x32x16_bf16), the
// fast prefill mode: outputs within a stated tolerance of the reference's
// order of addition instead of bit for bit.
//
// A product y[t][o] = sum_k W[o][k] x[t][k] runs on split operands:
//   - a weight w = (q - 8) d (Q4_0) needs at most 15 significant bits, so it
//     is exactly w_hi + w_lo with w_hi = bf16(w) and w_lo = bf16(w - w_hi)
//     (16 bits of bf16 mantissa between them; Q8_0's 19-bit and Q4_1's
//     rounded weights are left with an error below 2^-17 of w);
//   - an activation x is x_hi + x_lo the same way, to 2^-17 of x;
//   - y accumulates w_hi x_hi + w_hi x_lo + w_lo x_hi in fp32 (the dropped
//     w_lo x_lo is below 2^-16 of |w x|).
// So each product is within about 2^-16 of the exact one, and the sum's
// fp32 accumulation adds the usual K 2^-24 (matmul.h:71-78 states the
// reference's own bound, gamma(2K)).
//
// Weights are decoded from their blocks to bf16 pairs in registers and
// staged in LDS; activations arrive as bf16 pair planes (hi and lo, each
// [tokens][K]), written by the kernel that produced them.
//
// Tiles: a workgroup of four waves owns 128 output rows x 128 tokens and
// steps K one 32-weight block at a time, double-buffered in LDS. Wave w
// takes row blocks {w / 2, w / 2 + 2} (32 rows each) and token blocks
// {2 (w % 2), 2 (w % 2) + 1}: for the gated product, row blocks 0 and 1 are
// 64 neurons' gate rows and 2 and 3 the same neurons' up rows, so a wave
// holds each neuron's gate and up sums in matching registers and applies
// GELU and the pins in registers. LDS holds each operand in the order the
// instruction reads it (16 bytes a lane, a wave's 64 lanes contiguous).
// K may be split over grid z: split z writes its partial sums at
// y + z * part_stride, added in split order by the consumer.

#include "edit_common.h"
#include "kernels.h"
#include "numerics.h"

namespace frz {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kTileRows = 128;
constexpr int kTileTokens = 128;
constexpr int kThreads = 256;

// One K block's operands: [row or token block][k half][hi, lo][slot]. The
// instruction's lane L (row L % 32, k sub-block L / 32) reads slot
// 32 sub + (row ^ 4 sub): eight lanes reading eight rows of one sub-block,
// and a pair of threads writing one row's two sub-blocks four rows at a
// time, each touch eight distinct 16-byte bank groups.
__device__ __forceinline__ int slot_of(int row, int sub) { return 32 * sub + (row ^ (sub << 2)); }

struct Stage {
  uint4 w[4][2][2][64];
  uint4 x[4][2][2][64];
};

__device__ __forceinline__ float half_bits_to_float(uint32_t h) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// Two floats as bf16 pairs, packed: hi = bf16(v), lo = bf16(v - hi), round
// to nearest even (one v_cvt_pk_bf16_f32 each).
__device__ __forceinline__ void split2(float a, float b, uint32_t& hi, uint32_t& lo) {
  const f32x2 v = {a, b};
  hi = __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
  const f32x2 back = {__builtin_bit_cast(float, hi << 16),
                      __builtin_bit_cast(float, hi & 0xFFFF0000u)};
  lo = __builtin_bit_cast(uint32_t, __builtin_convertvector(v - back, bf16x2));
}

// Eight floats as bf16 pairs.
__device__ __forceinline__ void split8(const float (&v)[8], uint4& hi, uint4& lo) {
  uint32_t h[4], l[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) split2(v[2 * j], v[2 * j + 1], h[j], l[j]);
  hi = make_uint4(h[0], h[1], h[2], h[3]);
  lo = make_uint4(l[0], l[1], l[2], l[3]);
}

// A thread's share of one K block of one weight row: Q4_0 and Q4_1 take
// half the block's code bytes (8: weights 8h..8h+7 and 16+8h..16+8h+7),
// Q8_0 half its 32 (weights 16h..16h+15).
template <int FORMAT>
struct WeightLoad {
  uint4 codes;
  uint32_t scale;  // d, and m in the high half for Q4_1
};

// A load from global memory, said so: a pointer chosen among a fused
// product's members would otherwise load through the flat path, whose
// waits also hold back LDS reads.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint4 load_global4(const void* p) {
  const u32x4 v = *(const __attribute__((address_space(1))) u32x4*)(p);
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint2 load_global2(const void* p) {
  const u32x2 v = *(const __attribute__((address_space(1))) u32x2*)(p);
  return make_uint2(v.x, v.y);
}
template <typename T>
__device__ __forceinline__ T load_global(const void* p) {
  return *(const __attribute__((address_space(1))) T*)(p);
}

template <int FORMAT>
__device__ __forceinline__ WeightLoad<FORMAT> load_weights(const MemberRow& m, int blocks, int kb,
                                                           int h) {
  WeightLoad<FORMAT> r;
  const size_t b = (size_t)m.row * blocks + kb;
  if (FORMAT == kQ8_0) {
    r.codes = load_global4(m.codes + b * 32 + 16 * h);
  } else {
    const uint2 c = load_global2(m.codes + b * 16 + 8 * h);
    r.codes = make_uint4(c.x, c.y, 0, 0);
  }
  if (FORMAT == kQ4_1) {
    r.scale = load_global<uint32_t>(m.scales + 2 * b);
  } else {
    r.scale = load_global<uint16_t>(m.scales + b);
  }
  return r;
}

// Decodes a thread's weights and writes them to the stage as bf16 pairs:
// rows r of the tile (row block r / 32, lane r % 32 + 32 sub).
template <int FORMAT>
__device__ __forceinline__ void stage_weights(Stage& st, const WeightLoad<FORMAT>& in, int r,
                                              int h) {
  const int rb = r >> 5, lane = r & 31;
  const float d = half_bits_to_float(in.scale & 0xFFFFu);
  float a[8], b[8];
  if (FORMAT == kQ8_0) {
    // weights 16h..16h+15: k half h, lanes lane (first 8) and lane + 32
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint32_t w0 = j < 4 ? in.codes.x : in.codes.y;
      const uint32_t w1 = j < 4 ? in.codes.z : in.codes.w;
      const int sh = 8 * (j & 3);
      a[j] = (float)(int)(int8_t)(w0 >> sh) * d;
      b[j] = (float)(int)(int8_t)(w1 >> sh) * d;
    }
    uint4 hi, lo;
    split8(a, hi, lo);
    st.w[rb][h][0][slot_of(lane, 0)] = hi;
    st.w[rb][h][1][slot_of(lane, 0)] = lo;
    split8(b, hi, lo);
    st.w[rb][h][0][slot_of(lane, 1)] = hi;
    st.w[rb][h][1][slot_of(lane, 1)] = lo;
    return;
  }
  // Q4_0, Q4_1: low nibbles are weights 8h + j (k half 0, sub h), high
  // nibbles 16 + 8h + j (k half 1, sub h). A nibble masked under the
  // exponent of f16 1024 is the half 1024 + q (two at once, from bits 0 and
  // 16 of a shifted code word). Q4_0: fma(1024 + q, d, -1032 d) = (q - 8) d,
  // exact; Q4_1: fma(q, d, m) = q d + m rounded once, as q4_1.wgsl:12-25
  // computes it (q = (1024 + q) - 1024 exactly).
  const float c = FORMAT == kQ4_1 ? 0.0f : -1032.0f * d;  // exact
  const uint32_t w2[2] = {in.codes.x, in.codes.y};
#pragma unroll
  for (int wd = 0; wd < 2; ++wd) {
#pragma unroll
    for (int sh = 0; sh < 4; ++sh) {
      // shift 0: weights j, j + 2 (low nibbles); 4: 16 + j, 16 + j + 2;
      // 8: j + 1, j + 3; 12: 16 + j + 1, 16 + j + 3 (j = 4 wd)
      const uint32_t bits = ((w2[wd] >> (4 * sh)) & 0x000F000Fu) | 0x64006400u;
      const half2v q = __builtin_bit_cast(half2v, bits);
      float v0, v1;
      if (FORMAT == kQ4_1) {
        const float mn = half_bits_to_float(in.scale >> 16);
        v0 = __builtin_fmaf((float)q.x - 1024.0f, d, mn);
        v1 = __builtin_fmaf((float)q.y - 1024.0f, d, mn);
      } else {
        v0 = __builtin_fmaf((float)q.x, d, c);
        v1 = __builtin_fmaf((float)q.y, d, c);
      }
      const int j = 4 * wd + (sh >> 1);
      float* dst = (sh & 1) ? b : a;
      dst[j] = v0;
      dst[j + 2] = v1;
    }
  }
  const int l = slot_of(lane, h);
  uint4 hi, lo;
  split8(a, hi, lo);
  st.w[rb][0][0][l] = hi;
  st.w[rb][0][1][l] = lo;
  split8(b, hi, lo);
  st.w[rb][1][0][l] = hi;
  st.w[rb][1][1][l] = lo;
}

// A thread's share of one K block of the activations: token tk of the
// tile, sub-block `sub` of each k half (k 16 s + 8 sub .. + 7, s = 0, 1),
// 8 values of each plane each.
struct InputLoad {
  uint4 hi[2], lo[2];
};

__device__ __forceinline__ InputLoad load_inputs(const uint16_t* __restrict__ x_hi,
                                                 const uint16_t* __restrict__ x_lo, size_t row,
                                                 int kb, int sub) {
  InputLoad r;
  const size_t at = row + (size_t)kb * 32 + 8 * sub;
  r.hi[0] = load_global4(x_hi + at);
  r.hi[1] = load_global4(x_hi + at + 16);
  r.lo[0] = load_global4(x_lo + at);
  r.lo[1] = load_global4(x_lo + at + 16);
  return r;
}

__device__ __forceinline__ void stage_inputs(Stage& st, const InputLoad& in, int tk, int sub) {
  const int cb = tk >> 5, l = slot_of(tk & 31, sub);
  st.x[cb][0][0][l] = in.hi[0];
  st.x[cb][0][1][l] = in.lo[0];
  st.x[cb][1][0][l] = in.hi[1];
  st.x[cb][1][1][l] = in.lo[1];
}

__device__ __forceinline__ bf16x8 as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8, v); }

// One neuron's pins, out of line: the epilogue calls it for its 32 values
// only when the layer has pins.
__device__ __noinline__ float pin_one(const uint32_t* __restrict__ t, uint32_t first,
                                      uint32_t count, int n, uint32_t position, float value) {
  return apply_pin_words(t, first, count, (uint32_t)n, position, value);
}

template <int FORMAT, bool GATED>
__global__ __launch_bounds__(kThreads, 2) void gemm_bf16_kernel(const DevStep* __restrict__ step,
                                                                Bf16Gemm g) {
  __shared__ Stage stage[2];
  const int tokens = (int)step->tokens;
  const int n0 = blockIdx.y * kTileTokens;
  if (n0 >= tokens) return;  // the whole workgroup: past the step's rows
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wr = wave >> 1, wc = wave & 1;
  const int my_slot = slot_of(lane & 31, lane >> 5);
  const int blocks = g.w.cols / 32;
  const int kb0 = blockIdx.z * g.k_blocks;
  const int kb1 = min(blocks, kb0 + g.k_blocks);

  // This thread's weight row (r of the tile) and half block h (a pair of
  // threads reads one row's 16 code bytes).
  const int r = tid >> 1, h = tid & 1;
  int out_rows, row;
  MemberRow src;
  if (GATED) {
    out_rows = g.w.rows;
    const int n = blockIdx.x * (kTileRows / 2) + (r & 63);
    row = min(n, out_rows - 1);
    src = member_row(r < 64 ? g.w : g.up, row);
  } else {
    out_rows = g.w.rows;
    row = min((int)blockIdx.x * kTileRows + r, out_rows - 1);
    src = member_row(g.w, row);
  }
  // This thread's input token and k sub-block (a pair reads 64 bytes of a
  // row).
  const int tk = tid >> 1, kh = tid & 1;
  const size_t x_row = (size_t)min(n0 + tk, tokens - 1) * g.ldx;

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  // A split past the last block (splits that do not divide the blocks)
  // writes zero partial sums.
  if (kb0 >= kb1) {
    if (!GATED) {
      float* y = g.y + (size_t)blockIdx.z * g.part_stride;
      for (int i = tid; i < kTileRows * kTileTokens; i += kThreads) {
        const int o = blockIdx.x * kTileRows + (i % kTileRows), t = n0 + i / kTileRows;
        if (o < out_rows && t < tokens) y[(size_t)t * g.ldy + o] = 0.0f;
      }
    }
    return;
  }
  // Loads run three blocks ahead, into three register sets a, b, c: while
  // block kb computes from one LDS buffer, block kb + 1 (loaded two blocks
  // ago) is decoded into the other, and block kb + 3 is requested into the
  // set block kb came from. Every load is issued whatever kb (past the last
  // block it reloads the last), so the waits count exactly the loads they
  // need.
  WeightLoad<FORMAT> wa = load_weights<FORMAT>(src, blocks, kb0, h);
  InputLoad xa = load_inputs(g.x_hi, g.x_lo, x_row, kb0, kh);
  WeightLoad<FORMAT> wb = load_weights<FORMAT>(src, blocks, min(kb0 + 1, kb1 - 1), h);
  InputLoad xb = load_inputs(g.x_hi, g.x_lo, x_row, min(kb0 + 1, kb1 - 1), kh);
  WeightLoad<FORMAT> wc_ = load_weights<FORMAT>(src, blocks, min(kb0 + 2, kb1 - 1), h);
  InputLoad xc = load_inputs(g.x_hi, g.x_lo, x_row, min(kb0 + 2, kb1 - 1), kh);
  stage_weights<FORMAT>(stage[0], wa, r, h);
  stage_inputs(stage[0], xa, tk, kh);
  __syncthreads();
  auto block_step = [&](int kb, const Stage& cur, Stage& next, WeightLoad<FORMAT>& w_free,
                        InputLoad& x_free, const WeightLoad<FORMAT>& w_next,
                        const InputLoad& x_next) {
    // The next block is staged into the other buffer first (it was last
    // read before the previous barrier), so its decode can run while this
    // block's products do.
    stage_weights<FORMAT>(next, w_next, r, h);
    stage_inputs(next, x_next, tk, kh);
    const int ahead = min(kb + 3, kb1 - 1);
    w_free = load_weights<FORMAT>(src, blocks, ahead, h);
    x_free = load_inputs(g.x_hi, g.x_lo, x_row, ahead, kh);
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      bf16x8 ah[2], al[2], bh[2], bl[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        ah[i] = as_bf16x8(cur.w[wr + 2 * i][ks][0][my_slot]);
        al[i] = as_bf16x8(cur.w[wr + 2 * i][ks][1][my_slot]);
        bh[i] = as_bf16x8(cur.x[2 * wc + i][ks][0][my_slot]);
        bl[i] = as_bf16x8(cur.x[2 * wc + i][ks][1][my_slot]);
      }
      // The three products of each pair, four independent accumulators
      // between two that update the same one.
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah[i], bh[j], acc[i][j], 0, 0, 0);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah[i], bl[j], acc[i][j], 0, 0, 0);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al[i], bh[j], acc[i][j], 0, 0, 0);
    }
    __syncthreads();
  };
  // LDS buffers alternate every block, register sets every third: six
  // blocks a turn.
  for (int kb = kb0; kb < kb1; kb += 6) {
    block_step(kb, stage[0], stage[1], wa, xa, wb, xb);
    if (kb + 1 >= kb1) break;
    block_step(kb + 1, stage[1], stage[0], wb, xb, wc_, xc);
    if (kb + 2 >= kb1) break;
    block_step(kb + 2, stage[0], stage[1], wc_, xc, wa, xa);
    if (kb + 3 >= kb1) break;
    block_step(kb + 3, stage[1], stage[0], wa, xa, wb, xb);
    if (kb + 4 >= kb1) break;
    block_step(kb + 4, stage[0], stage[1], wb, xb, wc_, xc);
    if (kb + 5 >= kb1) break;
    block_step(kb + 5, stage[1], stage[0], wc_, xc, wa, xa);
  }

  // Lane l's register e of a 32 x 32 block: row (e / 4) 8 + (l / 32) 4 +
  // e % 4, token l % 32.
  const int row_in = (lane >> 5) * 4;
  const int tok_in = lane & 31;
  if (GATED) {
    const uint32_t first = g.edits ? g.edits[2 * g.layer] : 0u;
    const uint32_t count = g.edits ? g.edits[2 * g.layer + 1] : 0u;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int t = n0 + (2 * wc + j) * 32 + tok_in;
      const uint32_t position = step->position + (uint32_t)t;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int nb = blockIdx.x * (kTileRows / 2) + wr * 32 + q * 8 + row_in;
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = gelu_tanh(acc[0][j][4 * q + e]) * acc[1][j][4 * q + e];
        if (count) {
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = pin_one(g.edits, first, count, nb + e, position, v[e]);
        }
        if (t >= tokens || nb >= out_rows) continue;
        const size_t at = (size_t)t * g.ldy + nb;
        if (g.y) *reinterpret_cast<float4*>(g.y + at) = make_float4(v[0], v[1], v[2], v[3]);
        uint32_t hw[2], lw[2];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const __bf16 a = (__bf16)v[2 * e], b = (__bf16)v[2 * e + 1];
          const __bf16 c = (__bf16)(v[2 * e] - (float)a), d = (__bf16)(v[2 * e + 1] - (float)b);
          hw[e] = (uint32_t)__builtin_bit_cast(uint16_t, a) |
                  ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
          lw[e] = (uint32_t)__builtin_bit_cast(uint16_t, c) |
                  ((uint32_t)__builtin_bit_cast(uint16_t, d) << 16);
        }
        *reinterpret_cast<uint2*>(g.y_hi + at) = make_uint2(hw[0], hw[1]);
        *reinterpret_cast<uint2*>(g.y_lo + at) = make_uint2(lw[0], lw[1]);
      }
    }
    return;
  }
  float* y = g.y + (size_t)blockIdx.z * g.part_stride;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int t = n0 + (2 * wc + j) * 32 + tok_in;
      if (t >= tokens) continue;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int o = blockIdx.x * kTileRows + (wr + 2 * i) * 32 + q * 8 + row_in;
        if (o >= out_rows) continue;
        *reinterpret_cast<float4*>(y + (size_t)t * g.ldy + o) =
            make_float4(acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2],
                        acc[i][j][4 * q + 3]);
      }
    }
}

// Rows of fp32 values into bf16 pair planes: hi[t][k] = bf16(x), lo[t][k] =
// bf16(x - hi). A workgroup a row, eight values a thread a step.
__global__ __launch_bounds__(256) void split_rows_kernel(const DevStep* __restrict__ step,
                                                         const float* __restrict__ x, int ldx,
                                                         int width, uint16_t* __restrict__ hi,
                                                         uint16_t* __restrict__ lo, int ldo) {
  const int t = blockIdx.x;
  if (t >= (int)step->tokens) return;
  const float* xr = x + (size_t)t * ldx;
  for (int k = 8 * threadIdx.x; k < width; k += 8 * 256) {
    const float4 a = *reinterpret_cast<const float4*>(xr + k);
    const float4 b = *reinterpret_cast<const float4*>(xr + k + 4);
    const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    uint4 h, l;
    split8(v, h, l);
    *reinterpret_cast<uint4*>(hi + (size_t)t * ldo + k) = h;
    *reinterpret_cast<uint4*>(lo + (size_t)t * ldo + k) = l;
  }
}

// y[t][o] = the splits' partial sums added in split order (rows of `width`
// at ld in both).
__global__ __launch_bounds__(256) void sum_parts_kernel(const DevStep* __restrict__ step,
                                                        const float* __restrict__ parts,
                                                        size_t stride, int count, int width,
                                                        int ld, float* __restrict__ y) {
  const int t = blockIdx.x;
  if (t >= (int)step->tokens) return;
  for (int o = threadIdx.x; o < width; o += 256) {
    const size_t at = (size_t)t * ld + o;
    float v = parts[at];
    for (int z = 1; z < count; ++z) v = v + parts[z * stride + at];
    y[at] = v;
  }
}

template <int FORMAT, bool GATED>
hipError_t launch_one(hipStream_t s, const DevStep* step, const Bf16Gemm& g, int max_tokens,
                      int splits) {
  const int m_tiles = GATED ? (g.w.rows + 63) / 64 : (g.w.rows + kTileRows - 1) / kTileRows;
  const dim3 grid(m_tiles, (max_tokens + kTileTokens - 1) / kTileTokens, splits);
  hipLaunchKernelGGL((gemm_bf16_kernel<FORMAT, GATED>), grid, dim3(kThreads), 0, s, step, g);
  return hipGetLastError();
}

}  // namespace

bool bf16_gemm_shape_ok(const QMatrix& w, int ldx, int ldy) {
  return w.cols % 32 == 0 && w.rows % 4 == 0 && ldx % 8 == 0 && ldy % 4 == 0 &&
         (w.format == kQ4_0 || w.format == kQ4_1 || w.format == kQ8_0);
}

int bf16_splits_for(const QMatrix& w, int max_tokens, bool gated) {
  // Enough workgroups to fill 256 CUs twice, in whole K blocks a split.
  const int tiles = (gated ? (w.rows + 63) / 64 : (w.rows + kTileRows - 1) / kTileRows) *
                    ((max_tokens + kTileTokens - 1) / kTileTokens);
  if (gated) return 1;
  int splits = 1;
  const int blocks = w.cols / 32;
  while (tiles * splits < 384 && splits < 8 && blocks / (2 * splits) >= 4) splits *= 2;
  return splits;
}

hipError_t launch_gemm_bf16(hipStream_t s, const DevStep* step, Bf16Gemm g, int max_tokens,
                            int splits) {
  const int blocks = g.w.cols / 32;
  const bool gated = g.up.codes != nullptr;
  if (gated || splits < 1) splits = 1;
  g.k_blocks = (blocks + splits - 1) / splits;
  switch (g.w.format) {
    case kQ4_1:
      return gated ? launch_one<kQ4_1, true>(s, step, g, max_tokens, 1)
                   : launch_one<kQ4_1, false>(s, step, g, max_tokens, splits);
    case kQ8_0:
      return gated ? launch_one<kQ8_0, true>(s, step, g, max_tokens, 1)
                   : launch_one<kQ8_0, false>(s, step, g, max_tokens, splits);
    default:
      return gated ? launch_one<kQ4_0, true>(s, step, g, max_tokens, 1)
                   : launch_one<kQ4_0, false>(s, step, g, max_tokens, splits);
  }
}

hipError_t launch_sum_parts(hipStream_t s, const DevStep* step, const float* parts,
                            size_t stride, int count, int width, int ld, float* y,
                            int max_tokens) {
  hipLaunchKernelGGL(sum_parts_kernel, dim3(max_tokens), dim3(256), 0, s, step, parts, stride,
                     count, width, ld, y);
  return hipGetLastError();
}

hipError_t launch_split_rows(hipStream_t s, const DevStep* step, const float* x, int ldx,
                             int width, uint16_t* hi, uint16_t* lo, int ldo, int max_tokens) {
  hipLaunchKernelGGL(split_rows_kernel, dim3(max_tokens), dim3(256), 0, s, step, x, ldx, width,
                     hi, lo, ldo);
  return hipGetLastError();
}

}  // namespace frz
