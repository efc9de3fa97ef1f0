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
// The weights' pairs are made once (unpack_planes_kernel) into "fragment
// planes": for each 128-row tile and each step of 16 k, four 32-row blocks
// x (hi, lo) x 64 lanes x 16 bytes, lane L holding row L % 32's eight
// weights from k 8 (L / 32), the order in which the instruction's lanes
// read their operand. The gated product's tile is 64 neurons: its blocks 0
// and 1 are their gate rows, 2 and 3 their up rows. Activations arrive as
// bf16 pair planes (hi and lo) in the same fragment order, written by the
// kernel that produced them (plane_index). Gemma-3-1B's weight planes take
// 107 MB a layer, 2.8 GB in all.
//
// Tiles: a workgroup of eight waves (two a SIMD, so that one wave's
// products run while the other waits) owns 128 output rows x 256 tokens and
// steps K one 32-weight block at a time. Wave w computes all 128 rows for
// tokens 32 w .. 32 w + 31 (four 32 x 32 accumulators): the weights, which
// all eight waves read, pass through LDS (double-buffered), moved there by
// waves 0-3; each wave's token fragments, which only it reads, go straight
// into its registers. Loads run ahead and are copied as they are (no VALU). The
// instruction takes the tokens as its A operand and the weights as B, so
// that each output register's lanes are 32 consecutive rows of one token.
// For the gated product, row blocks 0 and 1 are 64 neurons' gate rows and
// 2 and 3 their up rows, so a wave holds each neuron's gate and up sums in
// matching registers and applies GELU (fast form) and the pins in
// registers. K may be split: split z writes its partial sums at
// y + z * part_stride, added in split order by the consumer.

#include <algorithm>

#include "edit_common.h"
#include "kernels.h"
#include "numerics.h"

namespace frz {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kTileRows = 128;
constexpr int kTileTokens = 256;
constexpr int kGemmThreads = 512;  // the products' workgroups: eight waves
constexpr int kStepBytes = 8 * 1024;       // a tile's weights for one step: 4 blocks x 2 planes

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

template <int FORMAT>
__device__ __forceinline__ WeightLoad<FORMAT> load_weights(const MemberRow& m, int blocks, int kb,
                                                           int h) {
  WeightLoad<FORMAT> r;
  const size_t b = (size_t)m.row * blocks + kb;
  if (FORMAT == kQ8_0) {
    r.codes = *reinterpret_cast<const uint4*>(m.codes + b * 32 + 16 * h);
  } else {
    const uint2 c = *reinterpret_cast<const uint2*>(m.codes + b * 16 + 8 * h);
    r.codes = make_uint4(c.x, c.y, 0, 0);
  }
  if (FORMAT == kQ4_1) {
    r.scale = *reinterpret_cast<const uint32_t*>(m.scales + 2 * b);
  } else {
    r.scale = m.scales[b];
  }
  return r;
}

// A thread's weights as bf16 pairs: out[0], out[1] are (hi, lo) of its
// first eight weights, out[2], out[3] of its second eight (Q4: k 8h + j and
// 16 + 8h + j; Q8_0: k 16h + j and 16h + 8 + j).
template <int FORMAT>
__device__ __forceinline__ void decode_pairs(const WeightLoad<FORMAT>& in, uint4 (&out)[4]) {
  const float d = half_bits_to_float(in.scale & 0xFFFFu);
  float a[8], b[8];
  if (FORMAT == kQ8_0) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint32_t w0 = j < 4 ? in.codes.x : in.codes.y;
      const uint32_t w1 = j < 4 ? in.codes.z : in.codes.w;
      const int sh = 8 * (j & 3);
      a[j] = (float)(int)(int8_t)(w0 >> sh) * d;
      b[j] = (float)(int)(int8_t)(w1 >> sh) * d;
    }
  } else {
    // A nibble masked under the exponent of f16 1024 is the half 1024 + q
    // (two at once, from bits 0 and 16 of a shifted code word). Q4_0:
    // fma(1024 + q, d, -1032 d) = (q - 8) d, exact; Q4_1: fma(q, d, m) =
    // q d + m rounded once, as q4_1.wgsl:12-25 computes it (q = (1024 + q)
    // - 1024 exactly).
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
  }
  split8(a, out[0], out[1]);
  split8(b, out[2], out[3]);
}

// The first uint4 of fragment (tile n, step s, block b, plane p).
__host__ __device__ inline size_t fragment_at(int n, int steps, int s, int b, int p) {
  return ((((size_t)n * steps + s) * 4 + b) * 2 + p) * 64;
}

// A thread a (tile, K block, block, half h, row of the block): the row's
// half block as pairs into the fragment planes; rows past the matrix are
// zeros. Consecutive threads write consecutive lanes.
template <int FORMAT, bool GATED>
__global__ __launch_bounds__(256) void unpack_planes_kernel(QMatrix w, QMatrix up, int tiles,
                                                            uint4* __restrict__ out) {
  const int blocks = w.cols / 32, steps = w.cols / 16;
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (size_t)tiles * blocks * 256) return;
  const int r = (int)(i & 31), h = (int)((i >> 5) & 1), b = (int)((i >> 6) & 3);
  const size_t rest = i >> 8;
  const int kb = (int)(rest % (size_t)blocks), n = (int)(rest / (size_t)blocks);
  const int row = GATED ? n * 64 + 32 * (b & 1) + r : n * kTileRows + 32 * b + r;
  uint4 q[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) q[j] = make_uint4(0, 0, 0, 0);
  if (row < w.rows) {
    const MemberRow src = GATED && b >= 2 ? member_row(up, row) : member_row(w, row);
    decode_pairs<FORMAT>(load_weights<FORMAT>(src, blocks, kb, h), q);
  }
  if (FORMAT == kQ8_0) {
    const size_t f = fragment_at(n, steps, 2 * kb + h, b, 0);
    out[f + r] = q[0];
    out[f + 64 + r] = q[1];
    out[f + 32 + r] = q[2];
    out[f + 96 + r] = q[3];
  } else {
    const size_t f0 = fragment_at(n, steps, 2 * kb, b, 0) + 32 * h + r;
    const size_t f1 = fragment_at(n, steps, 2 * kb + 1, b, 0) + 32 * h + r;
    out[f0] = q[0];
    out[f0 + 64] = q[1];
    out[f1] = q[2];
    out[f1 + 64] = q[3];
  }
}

__device__ __forceinline__ bf16x8 as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8, v); }

// One neuron's pins, out of line: the epilogue calls it for its 32 values
// only when the layer has pins.
__device__ __noinline__ float pin_one(const uint32_t* __restrict__ t, uint32_t first,
                                      uint32_t count, int n, uint32_t position, float value) {
  return apply_pin_words(t, first, count, (uint32_t)n, position, value);
}

// A load from global memory, said so: through a flat pointer the
// compiler's waits for it would also hold back LDS reads.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 load_global4(const void* p) {
  const u32x4 v = *(const __attribute__((address_space(1))) u32x4*)(p);
  return make_uint4(v.x, v.y, v.z, v.w);
}

// GELU, tanh form, from the hardware's exp2 and reciprocal: 0.5 g (1 +
// tanh z) = g / (1 + e^-2z). Within 2^-20 relative of the exact form
// (matmul.wgsl:141-147) for the fast mode's tolerance, not its bits.
__device__ __forceinline__ float gelu_fast(float g) {
  const float z = 0.7978845608028654f * __builtin_fmaf(0.044715f * g * g, g, g);
  const float e = __builtin_amdgcn_exp2f(-2.8853900817779268f * z);  // -2 z log2(e)
  return g * __builtin_amdgcn_rcpf(1.0f + e);
}

// A wave's share of one K block (two steps of 16 k): its weight block's
// fragments [step][hi, lo] (waves 0-3), staged in LDS for the workgroup, and
// its token block's [step][hi, lo], which only it reads.
struct WeightLoad2 {
  uint4 w[2][2];
};
struct TokenLoad {
  uint4 x[2][2];
};

template <bool GATED>
__global__ __launch_bounds__(kGemmThreads, 2) void gemm_bf16_kernel(const DevStep* __restrict__ step,
                                                                Bf16Gemm g) {
  // The weights of one K block: [step][row block][hi, lo][lane].
  __shared__ uint4 stage[2][2][4][2][64];
  const int tokens = (int)step->tokens;
  // Workgroups go to the eight XCDs in turn (linear id mod 8); the tile
  // order gives each XCD a contiguous run of tiles, so that the token tiles
  // of one row tile (the same weights) share an L2.
  const int total = (int)gridDim.x, wid = (int)blockIdx.x;
  const int xcd = wid & 7, per = total >> 3, extra = total & 7;
  const int tile = xcd * per + min(xcd, extra) + (wid >> 3);
  const int tt = tile % g.token_tiles, rest = tile / g.token_tiles;
  const int z = rest % g.splits, rt = rest / g.splits;
  const int n0 = tt * kTileTokens;
  if (n0 >= tokens) return;  // the whole workgroup: past the step's rows
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int steps = g.cols / 16;
  const int kb0 = z * g.k_blocks;
  const int kb1 = min(g.cols / 32, kb0 + g.k_blocks);

  // acc[row block][token block of the wave], transposed: the instruction
  // takes the tokens as its A operand and the weights as B, so a lane holds
  // one output row (lane % 32) for 16 tokens.
  f32x16 acc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[i][e] = 0.0f;

  // A split past the last block (splits that do not divide the blocks)
  // writes zero partial sums.
  if (kb0 >= kb1) {
    if (!GATED) {
      float* y = g.y + (size_t)z * g.part_stride;
      for (int i = tid; i < kTileRows * kTileTokens; i += kGemmThreads) {
        const int o = rt * kTileRows + (i % kTileRows), t = n0 + i / kTileRows;
        if (o < g.rows && t < tokens) y[(size_t)t * g.ldy + o] = 0.0f;
      }
    }
    return;
  }
  // Wave w < 4 moves weight block w of the row tile into LDS; wave w reads
  // its token block w of the tile (the last block with rows, for blocks
  // past them) straight into registers. Every fragment is a 1 KB run of its
  // planes, 16 bytes a lane.
  const bool mover = wave < 4;  // uniform over the wave
  const uint4* wsrc = g.w + fragment_at(rt, steps, 0, wave & 3, 0) + lane;
  const int last_tb = (tokens - 1) >> 5;
  const size_t x_at = plane_index(32 * min(n0 / 32 + wave, last_tb), 0, g.ldx) + 8 * lane;
  auto load_w = [&](int kb) {
    WeightLoad2 r;
    if (mover) {
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const size_t s = 2 * (size_t)kb + u;
        r.w[u][0] = load_global4(wsrc + s * (kStepBytes / 16));
        r.w[u][1] = load_global4(wsrc + s * (kStepBytes / 16) + 64);
      }
    }
    return r;
  };
  auto load_x = [&](int kb) {
    TokenLoad r;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const size_t s = 2 * (size_t)kb + u;
      r.x[u][0] = load_global4(g.x_hi + x_at + 512 * s);
      r.x[u][1] = load_global4(g.x_lo + x_at + 512 * s);
    }
    return r;
  };
  auto put = [&](uint4 (&st)[2][4][2][64], const WeightLoad2& r) {
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        if (mover) st[u][wave][p][lane] = r.w[u][p];
      }
  };
  auto compute = [&](const uint4 (&st)[2][4][2][64], const TokenLoad& r) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      bf16x8 wh[4], wl[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        wh[i] = as_bf16x8(st[u][i][0][lane]);
        wl[i] = as_bf16x8(st[u][i][1][lane]);
      }
      const bf16x8 xh = as_bf16x8(r.x[u][0]), xl = as_bf16x8(r.x[u][1]);
      // The three products of each pair, four independent accumulators
      // between two that update the same one.
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xh, wh[i], acc[i], 0, 0, 0);
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xl, wh[i], acc[i], 0, 0, 0);
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xh, wl[i], acc[i], 0, 0, 0);
    }
  };
  // Weights run three blocks ahead in three register sets, tokens two
  // ahead in two. Block kb: the next block's weights (loaded two blocks
  // ago) go to the other LDS buffer and block kb + 3's are requested into
  // their set; this block's products run from this buffer and this block's
  // token fragments; then block kb + 2's tokens are requested into theirs.
  // Every load is issued whatever kb (past the last block it reloads the
  // last), so the waits count exactly the loads they need.
  WeightLoad2 wa = load_w(kb0);
  TokenLoad xa = load_x(kb0);
  WeightLoad2 wb = load_w(min(kb0 + 1, kb1 - 1));
  TokenLoad xb = load_x(min(kb0 + 1, kb1 - 1));
  WeightLoad2 wc = load_w(min(kb0 + 2, kb1 - 1));
  put(stage[0], wa);
  __syncthreads();
  auto block_step = [&](int kb, const uint4 (&cur)[2][4][2][64], uint4 (&next)[2][4][2][64],
                        WeightLoad2& w_free, const WeightLoad2& w_next, TokenLoad& x_cur) {
    put(next, w_next);  // read before the previous barrier
    w_free = load_w(min(kb + 3, kb1 - 1));
    compute(cur, x_cur);
    x_cur = load_x(min(kb + 2, kb1 - 1));
    __syncthreads();
  };
  // LDS buffers and token sets alternate every block, weight sets every
  // third: six blocks a turn.
  for (int kb = kb0; kb < kb1; kb += 6) {
    block_step(kb, stage[0], stage[1], wa, wb, xa);
    if (kb + 1 >= kb1) break;
    block_step(kb + 1, stage[1], stage[0], wb, wc, xb);
    if (kb + 2 >= kb1) break;
    block_step(kb + 2, stage[0], stage[1], wc, wa, xa);
    if (kb + 3 >= kb1) break;
    block_step(kb + 3, stage[1], stage[0], wa, wb, xb);
    if (kb + 4 >= kb1) break;
    block_step(kb + 4, stage[0], stage[1], wb, wc, xa);
    if (kb + 5 >= kb1) break;
    block_step(kb + 5, stage[1], stage[0], wc, wa, xb);
  }

  // Lane l's register e of a 32 x 32 block: token (e / 4) 8 + (l / 32) 4 +
  // e % 4 of the token block, row l % 32 of the row block. A register's
  // 32 lanes are 32 consecutive rows of one token: 128 bytes a store.
  const int row_in = lane & 31;
  const int tok_in = (lane >> 5) * 4;
  if (GATED) {
    // Row blocks 0 and 1 are the tile's 64 neurons' gate rows, 2 and 3
    // their up rows.
    const uint32_t first = g.edits ? g.edits[2 * g.layer] : 0u;
    const uint32_t count = g.edits ? g.edits[2 * g.layer + 1] : 0u;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int n = rt * (kTileRows / 2) + i * 32 + row_in;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int t = n0 + wave * 32 + (e >> 2) * 8 + tok_in + (e & 3);
        float v = gelu_fast(acc[i][e]) * acc[i + 2][e];
        if (count) v = pin_one(g.edits, first, count, n, step->position + (uint32_t)t, v);
        if (t >= tokens || n >= g.rows) continue;
        if (g.y) g.y[(size_t)t * g.ldy + n] = v;
        const __bf16 h = (__bf16)v, l = (__bf16)(v - (float)h);
        const size_t at = plane_index(t, n, g.ldy);
        g.y_hi[at] = __builtin_bit_cast(uint16_t, h);
        g.y_lo[at] = __builtin_bit_cast(uint16_t, l);
      }
    }
    return;
  }
  float* y = g.y + (size_t)z * g.part_stride;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int o = rt * kTileRows + i * 32 + row_in;
    if (o >= g.rows) continue;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int t = n0 + wave * 32 + (e >> 2) * 8 + tok_in + (e & 3);
      if (t < tokens) y[(size_t)t * g.ldy + o] = acc[i][e];
    }
  }
}

// Rows of fp32 values into bf16 pair planes (plane_index order): hi =
// bf16(x), lo = bf16(x - hi). A workgroup a row, four values a thread a
// step.
__global__ __launch_bounds__(256) void split_rows_kernel(const DevStep* __restrict__ step,
                                                         const float* __restrict__ x, int ldx,
                                                         int width, uint16_t* __restrict__ hi,
                                                         uint16_t* __restrict__ lo) {
  const int t = blockIdx.x;
  if (t >= (int)step->tokens) return;
  const float* xr = x + (size_t)t * ldx;
  for (int k = 4 * threadIdx.x; k < width; k += 4 * 256) {
    const float4 a = *reinterpret_cast<const float4*>(xr + k);
    const float v[4] = {a.x, a.y, a.z, a.w};
    store_pairs4(hi, lo, t, k, width, v);
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

int row_tiles_of(int rows, bool gated) {
  return gated ? (rows + kTileRows / 2 - 1) / (kTileRows / 2) : (rows + kTileRows - 1) / kTileRows;
}

template <int FORMAT, bool GATED>
hipError_t launch_unpack(hipStream_t s, const QMatrix& w, const QMatrix& up, uint4* out) {
  const int tiles = row_tiles_of(w.rows, GATED);
  const size_t threads = (size_t)tiles * (w.cols / 32) * 256;
  hipLaunchKernelGGL((unpack_planes_kernel<FORMAT, GATED>), dim3((unsigned)(threads / 256)),
                     dim3(256), 0, s, w, up, tiles, out);
  return hipGetLastError();
}

}  // namespace

bool bf16_gemm_shape_ok(const QMatrix& w, int ldx, int ldy) {
  return w.cols % 32 == 0 && w.rows % 4 == 0 && ldx % 8 == 0 && ldy % 4 == 0 &&
         (w.format == kQ4_0 || w.format == kQ4_1 || w.format == kQ8_0);
}

size_t bf16_planes_bytes(int rows, int cols, bool gated) {
  return (size_t)row_tiles_of(rows, gated) * (cols / 16) * kStepBytes;
}

hipError_t launch_unpack_planes(hipStream_t s, const QMatrix& w, const QMatrix* up, uint4* out) {
  const QMatrix none{};
  if (up) {
    if (up->format != w.format || up->rows != w.rows || up->cols != w.cols)
      return hipErrorInvalidValue;
    switch (w.format) {
      case kQ4_1: return launch_unpack<kQ4_1, true>(s, w, *up, out);
      case kQ8_0: return launch_unpack<kQ8_0, true>(s, w, *up, out);
      default: return launch_unpack<kQ4_0, true>(s, w, *up, out);
    }
  }
  switch (w.format) {
    case kQ4_1: return launch_unpack<kQ4_1, false>(s, w, none, out);
    case kQ8_0: return launch_unpack<kQ8_0, false>(s, w, none, out);
    default: return launch_unpack<kQ4_0, false>(s, w, none, out);
  }
}

int bf16_splits_for(int rows, int cols, int max_tokens, bool gated) {
  // As many workgroups as the 256 CUs hold (one each), at least two K
  // blocks a split, and no split left empty.
  if (gated) return 1;
  const int tiles = row_tiles_of(rows, false) * ((max_tokens + kTileTokens - 1) / kTileTokens);
  const int blocks = cols / 32;
  int splits = std::min({kMaxBf16Splits, std::max(1, 256 / tiles), std::max(1, blocks / 2)});
  const int per = (blocks + splits - 1) / splits;
  return (blocks + per - 1) / per;
}

hipError_t launch_gemm_bf16(hipStream_t s, const DevStep* step, Bf16Gemm g, int max_tokens,
                            int splits) {
  // The activation planes are as wide as K; the gated product's output
  // planes as wide as its rows.
  if (!g.w || g.cols % 32 || g.rows <= 0 || g.ldx != g.cols || max_tokens <= 0 ||
      max_tokens > kPrefillBlock || (g.gated && g.ldy % 16))
    return hipErrorInvalidValue;
  const int blocks = g.cols / 32;
  if (g.gated || splits < 1) splits = 1;
  g.splits = splits;
  g.k_blocks = (blocks + splits - 1) / splits;
  g.token_tiles = (max_tokens + kTileTokens - 1) / kTileTokens;
  const int tiles = row_tiles_of(g.rows, g.gated) * splits * g.token_tiles;
  if (g.gated) {
    hipLaunchKernelGGL(gemm_bf16_kernel<true>, dim3(tiles), dim3(kGemmThreads), 0, s, step, g);
  } else {
    hipLaunchKernelGGL(gemm_bf16_kernel<false>, dim3(tiles), dim3(kGemmThreads), 0, s, step, g);
  }
  return hipGetLastError();
}


hipError_t launch_sum_parts(hipStream_t s, const DevStep* step, const float* parts,
                            size_t stride, int count, int width, int ld, float* y,
                            int max_tokens) {
  hipLaunchKernelGGL(sum_parts_kernel, dim3(max_tokens), dim3(256), 0, s, step, parts, stride,
                     count, width, ld, y);
  return hipGetLastError();
}

hipError_t launch_split_rows(hipStream_t s, const DevStep* step, const float* x, int ldx,
                             int width, uint16_t* hi, uint16_t* lo, int max_tokens) {
  if (width % 16) return hipErrorInvalidValue;
  hipLaunchKernelGGL(split_rows_kernel, dim3(max_tokens), dim3(256), 0, s, step, x, ldx, width,
                     hi, lo);
  return hipGetLastError();
}

}  // namespace frz
