// The decode attention kernel: one token's QK-norm, rope and KV append
// (rope.wgsl:51-138) fused with its attention over the cache; a workgroup
// per (chunk, head), a wave per 16 of the chunk's keys. The chunk states are
// folded by the next launch (the O product's prologue, or the fold kernel).
//
// A launch is a few dozen workgroups, one a CU, so its time is the chain of
// dependent steps one wave takes, and each CU streams its chunk's 64 KB of
// key and value rows; the kernel is laid out to keep both short:
// - the chunk's rows are requested first; wave 0 alone ropes the query (and
//   the key, in the workgroup holding the step's position) while they are
//   in flight, and a barrier hands the query to the other waves;
// - each key's score is the chain s += dot(q_w, k_w) over the head's 64
//   vec4s, its dots formed by the key's four lanes and added in order by
//   each of them, reading the others' through DPP;
// - the scores and value rows go to LDS, a second barrier, then every wave
//   derives all 64 weights itself (a lane a key): the tile maxima and the
//   running maxima by DPP, the rescale factors from them, and the running
//   sum l from the tile sums;
// - each output dimension's chain o = o a + sum_b e_b v_b runs over the
//   chunk's keys in order (thread t is dimension t), over all 8 tiles: keys
//   past the chunk's end have zero weights and zero rows, as the reference
//   stages them, and tiles past it a = 1.
// Products of a float and a half are one mixed fma with -0 added, which is
// the product rounded once.

#include "attention_rows.h"

namespace frz {
namespace {
using namespace attn;

constexpr int kWaves = kThreads / 64;

__device__ __forceinline__ uint4 load_row_part(__amdgpu_buffer_rsrc_t r, int byte_offset) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, byte_offset, 0, 0));
}

// LDS of one workgroup: a (chunk, head) pair, or with kSplit > 1 the
// D / kSplit output dimensions q D / kSplit .. of one.
template <int kSplit>
struct DecodeShared {
  static constexpr int kDims = D / kSplit;
  alignas(16) uint16_t v[(kChunkKeys + 1) * kDims];  // value rows' dimensions; a spare row
  alignas(16) float q[D];                    // the roped query, times scale * log2(e)
  alignas(16) float cosine[D / 2];           // rope angles
  alignas(16) float sine[D / 2];
  alignas(16) uint16_t knew[D];              // the step's key row
  alignas(16) float s[kThreads];             // scores, as each of a key's 4 lanes has it
  alignas(16) float e[kWaves][kChunkKeys];   // each wave's weights
  alignas(16) float a[kWaves][kTiles];       // and tile factors
};

// The launch is a few workgroups a CU at most: registers are budgeted for
// one wave a SIMD. With kSplit > 1, kSplit workgroups share a (chunk, head):
// each scores all the chunk's keys but stages and sums only its D / kSplit
// output dimensions, so each CU streams the key rows and a kSplit-th of the
// value rows (the launch picks this for grids of a few dozen workgroups).
template <int kSplit>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 1))) void
attention_decode_kernel(const DevStep* __restrict__ step, DecodeAttentionArgs a) {
  constexpr int kDims = D / kSplit;            // output dimensions of this workgroup
  constexpr int kOutWaves = kDims / 64;        // waves that sum them, a lane each
  constexpr int kRowParts = kDims / 8;         // uint4s of a value row's dimensions
  constexpr int kRowStep = kThreads / kRowParts;
  constexpr int kValueParts = kChunkKeys / kRowStep;  // uint4s a thread stages
  __shared__ DecodeShared<kSplit> S;
  const int h = blockIdx.y / kSplit, q = blockIdx.y % kSplit;
  const int t = threadIdx.x, row = blockIdx.z;
  const int w = t >> 6, lane = t & 63;
  if (row > 0) {  // a variants step's row: its own token and caches
    a.qkv += (size_t)row * a.qkv_stride;
    a.key_cache += (size_t)row * a.cache_stride;
    a.value_cache += (size_t)row * a.cache_stride;
  }
  // Wave 0 ropes: lanes 0-31 take the query head h, lanes 32-63 the key;
  // lane l of a half holds dimensions 4l..4l+3 and D/2 + 4l..+3 (the value's
  // too, in the key lanes). Its loads go first (none depends on the
  // position), the cached rows' after.
  const bool key_lane = lane >= 32;
  const int l = lane & 31;
  float2 turn;
  float4 va, vb, xa, xb, ga, gb;
  if (w == 1) turn = ld2f(a.turns + 2 * lane);
  if (w == 0) {
    const float* src = a.qkv + (key_lane ? QH : h) * D;
    va = ld4f(src + 4 * l);
    vb = ld4f(src + D / 2 + 4 * l);
    xa = ld4f(a.qkv + (QH + 1) * D + 4 * l);
    xb = ld4f(a.qkv + (QH + 1) * D + D / 2 + 4 * l);
    const float* gain = key_lane ? a.key_gain : a.query_gain;
    ga = ld4f(gain + 4 * l);
    gb = ld4f(gain + D / 2 + 4 * l);
  }
  __asm__ volatile("" ::: "memory");  // keep these loads ahead of the position's
  const int p = (int)step->position;
  const ChunkRange r = chunk_range(p, a.window, blockIdx.x);
  if ((int)blockIdx.x >= r.count) return;
  const int valid = r.k_end - r.k_begin;  // the chunk's keys
  // The step's own key, the chunk's last, when the chunk holds p; it is
  // not read from the cache (head 0's workgroups write it there).
  const bool holds_p = r.c == (p >> 6);
  const int own = holds_p ? valid - 1 : -1;
  const int cached = holds_p ? valid - 1 : valid;  // rows read from the cache
  const int base = ring_slot(r.k_begin, a.slots);
  const int jj = t >> 2, u = t & 3;  // key jj of the chunk, quarter u of its row
  // Lane t's part of key row jj: the 8 halves 8 (4m + u) .. +7 for m = 0..7,
  // so that a key's 4 lanes read 64 contiguous bytes a load (a wave's load
  // touches 16 cache lines, where quarter rows a lane would touch 64).
  // Thread t's share of the value rows' dimensions: uint4 i = t + 256 n is
  // row i / kRowParts, halves q kDims + 8 (i % kRowParts) .. +7. (Registers
  // named by constant indices: an array indexed in a loop is placed in LDS
  // before the loop is unrolled, and its stores then wait for each load.)
  const int vrow = t / kRowParts, part = t % kRowParts;
  uint4 kr[kKeyLoads], vr[kValueParts];
  auto request_rows = [&]() {
    const __amdgpu_buffer_rsrc_t kres = cache_resource(a.key_cache, a.slots);
    int slot = base + jj;
    slot = slot >= a.slots ? slot - a.slots : slot;
    const int at = jj < cached ? slot * (D * 2) + 16 * u : kPastEnd;
#pragma unroll
    for (int m = 0; m < kKeyLoads; ++m) kr[m] = load_row_part(kres, at + 64 * m);
    const __amdgpu_buffer_rsrc_t vres = cache_resource(a.value_cache, a.slots);
    auto value_part = [&](int n) {
      const int rr = vrow + kRowStep * n;
      int vslot = base + rr;
      vslot = vslot >= a.slots ? vslot - a.slots : vslot;
      return load_row_part(vres,
                           rr < cached ? vslot * (D * 2) + 2 * (q * kDims + 8 * part) : kPastEnd);
    };
    vr[0] = value_part(0);
    vr[1] = value_part(1);
    if constexpr (kValueParts == 8) {
      vr[2] = value_part(2); vr[3] = value_part(3); vr[4] = value_part(4);
      vr[5] = value_part(5); vr[6] = value_part(6); vr[7] = value_part(7);
    } else {
      static_assert(kValueParts == 2, "8 or 2 value parts a thread");
    }
  };
  request_rows();
  // Nothing below moves above the loads: the rope's arithmetic waits for its
  // inputs, which would hold back loads issued after it.
  __builtin_amdgcn_sched_barrier(0);
  // Wave 1 turns the rope angles (lane L pairs 2L and 2L + 1) while wave 0
  // normalizes; a barrier hands the angles over.
  if (w == 1) {
    float s0, c0, s1, c1;
    rope_angle(turn.x, (uint32_t)p, &s0, &c0);
    rope_angle(turn.y, (uint32_t)p, &s1, &c1);
    *reinterpret_cast<float2*>(&S.sine[2 * lane]) = make_float2(s0, s1);
    *reinterpret_cast<float2*>(&S.cosine[2 * lane]) = make_float2(c0, c1);
  }
  if (w == 0) {
    // The head's sum of squares: the halving tree over its 32 lanes. Each
    // 32-lane group's lane 0 ends with the total (level 16 by a lane swap,
    // lane l + 16; levels 8 to 1 within a row by DPP), which goes to the
    // group's lanes.
    float sum = rope_lane_squares(va, vb);
    sum = sum + lane_plus16(sum);
    sum = sum + row_shl<8>(sum);
    sum = sum + row_shl<4>(sum);
    sum = sum + row_shl<2>(sum);
    sum = sum + row_shl<1>(sum);
    {
      const int b = __builtin_bit_cast(int, sum);
      const int lo = __builtin_amdgcn_readlane(b, 0), hi = __builtin_amdgcn_readlane(b, 32);
      sum = __builtin_bit_cast(float, key_lane ? hi : lo);
    }
    rope_normalize(va, vb, sum, D, a.epsilon, ga, gb);
  }
  __syncthreads();  // the angles
  if (w == 0) {
    rope_rotate(va, vb, l, S.cosine, S.sine);
    if (!key_lane) {
      const float sc = a.scale_log2e;
      *reinterpret_cast<float4*>(&S.q[4 * l]) =
          make_float4(va.x * sc, va.y * sc, va.z * sc, va.w * sc);
      *reinterpret_cast<float4*>(&S.q[D / 2 + 4 * l]) =
          make_float4(vb.x * sc, vb.y * sc, vb.z * sc, vb.w * sc);
    } else if (holds_p) {
      // The step's key row to LDS (for the key's lanes) and its value row's
      // dimensions to the staged rows; head 0 appends both rows to the
      // cache, at slot p.
      const ushort4 ka = pack4_f16(va), kb = pack4_f16(vb);
      const ushort4 pa = pack4_f16(xa), pb = pack4_f16(xb);
      *reinterpret_cast<ushort4*>(S.knew + 4 * l) = ka;
      *reinterpret_cast<ushort4*>(S.knew + D / 2 + 4 * l) = kb;
      const int da = 4 * l - q * kDims, db = D / 2 + 4 * l - q * kDims;
      if (da >= 0 && da < kDims) *reinterpret_cast<ushort4*>(S.v + own * kDims + da) = pa;
      if (db >= 0 && db < kDims) *reinterpret_cast<ushort4*>(S.v + own * kDims + db) = pb;
      if (h == 0 && q == 0) {
        const size_t at = (size_t)ring_slot(p, a.slots) * D;
        *reinterpret_cast<ushort4*>(a.key_cache + at + 4 * l) = ka;
        *reinterpret_cast<ushort4*>(a.key_cache + at + D / 2 + 4 * l) = kb;
        *reinterpret_cast<ushort4*>(a.value_cache + at + 4 * l) = pa;
        *reinterpret_cast<ushort4*>(a.value_cache + at + D / 2 + 4 * l) = pb;
      }
    }
  }
  __syncthreads();  // the query, and the step's key and value rows
  // The lane's 64 query values (dimensions 8 (4m + u) .. +7), then the
  // step's key part for its lanes.
  float4 qv[2 * kKeyLoads];
#pragma unroll
  for (int m = 0; m < kKeyLoads; ++m) {
    qv[2 * m] = ld4f(&S.q[32 * m + 8 * u]);
    qv[2 * m + 1] = ld4f(&S.q[32 * m + 8 * u + 4]);
  }
  if (jj == own) {
#pragma unroll
    for (int m = 0; m < kKeyLoads; ++m) {
      kr[m] = *reinterpret_cast<const uint4*>(S.knew + 32 * m + 8 * u);
    }
  }
  // Scores (attention.wgsl:277-297): vec4 w of the head is d[w % 2 + 2m] of
  // lane (w / 2) % 4, m = w / 8; the chain adds them in w's order.
  const float nz = negative_zero();
  float d[2 * kKeyLoads];
#pragma unroll
  for (int m = 0; m < kKeyLoads; ++m) {
    d[2 * m] = dot4_halves(qv[2 * m], kr[m].x, kr[m].y, nz);
    d[2 * m + 1] = dot4_halves(qv[2 * m + 1], kr[m].z, kr[m].w, nz);
  }
  float s = 0.0f;
#pragma unroll
  for (int m = 0; m < kKeyLoads; ++m) {
    s = s + quad_lane<0>(d[2 * m]);
    s = s + quad_lane<0>(d[2 * m + 1]);
    s = s + quad_lane<1>(d[2 * m]);
    s = s + quad_lane<1>(d[2 * m + 1]);
    s = s + quad_lane<2>(d[2 * m]);
    s = s + quad_lane<2>(d[2 * m + 1]);
    s = s + quad_lane<3>(d[2 * m]);
    s = s + quad_lane<3>(d[2 * m + 1]);
  }
  S.s[t] = s;
  // The value rows to LDS; the step's own row is already there, and what was
  // loaded for it goes to the spare row.
  auto stage = [&](int n, uint4 v) {
    const int rr = vrow + kRowStep * n;
    *reinterpret_cast<uint4*>(S.v + (rr == own ? kChunkKeys : rr) * kDims + 8 * part) = v;
  };
  stage(0, vr[0]);
  stage(1, vr[1]);
  if constexpr (kValueParts == 8) {
    stage(2, vr[2]); stage(3, vr[3]); stage(4, vr[4]);
    stage(5, vr[5]); stage(6, vr[6]); stage(7, vr[7]);
  }
  __syncthreads();
  // The waves that sum the output dimensions, and one that sums l (the last
  // of them, or wave 1 when one wave sums the outputs): lane L is key L.
  constexpr int kLWave = kOutWaves > 1 ? kOutWaves - 1 : 1;
  if (w > kLWave) return;
  const float sl = S.s[4 * lane];
  // (attention.wgsl:304-340) A key is live when the token sees it; a tile is
  // seen when any of its keys is. A tile's maximum is over its live scores,
  // and tile T's running maximum over the seen tiles' maxima up to T: max is
  // order-free, so both are taken by DPP, the second as a prefix scan over
  // the tiles, 8 lanes apart. A quiet NaN stands for "nothing": max(x, NaN)
  // is x for every x, so it leaves any maximum, NaN maxima included, as the
  // reference's ordered recursion has it. The maximum before tile T is the
  // scan at tile T - 1, or T's own maximum when no tile before it is seen.
  const bool live = lane < valid && r.k_begin + lane + a.window > p;
  const uint64_t live_bits = __ballot(live);
  const int tile = lane >> 3;
  // Bit T: tile T seen (each byte of the ballot or-ed into its low bit,
  // the 8 low bits gathered by one multiply).
  uint64_t any = live_bits | (live_bits >> 4);
  any |= any >> 2;
  any |= any >> 1;
  const uint32_t seen_tiles =
      (uint32_t)(((any & 0x0101010101010101ull) * 0x0102040810204080ull) >> 56);
  const bool tile_seen = (seen_tiles >> tile) & 1u;
  const bool seen_before = (seen_tiles & ((1u << tile) - 1u)) != 0;
  const float none = __builtin_bit_cast(float, 0x7FC00000u);
  const float top = max8(live ? sl : none);
  // Dimension t of every value row the chunk uses, read now to land under
  // the weights' arithmetic: after the score has landed (an LDS counter
  // holds 15 reads, so a wait for a read issued before 64 others would
  // wait for 49 of them too).
  __builtin_amdgcn_sched_barrier(0);
  const _Float16* vh = reinterpret_cast<const _Float16*>(S.v);
  _Float16 vt[kChunkKeys];
  if (w < kOutWaves) {
#pragma unroll
    for (int key = 0; key < kChunkKeys; ++key) vt[key] = vh[key * kDims + t];
  }
  float run = tile_seen ? top : none;
  run = __builtin_fmaxf(run, dpp_or<0x118, 0xF>(run, none));  // row_shr:8: the row's first tile
  run = __builtin_fmaxf(run, dpp_or<0x142, 0xA>(run, none));  // row_bcast:15: rows 1, 3
  run = __builtin_fmaxf(run, dpp_or<0x143, 0xC>(run, none));  // row_bcast:31: rows 2, 3
  // The scan at tile T - 1: 8 lanes back within a row, or the previous
  // row's last lane. Both are taken in every lane (the empty asm keeps the
  // compiler from moving either under the choice, where the lanes they
  // read would be switched off).
  const float back8 = dpp_or<0x118, 0xF>(run, none), back_row = dpp_or<0x142, 0xE>(run, none);
  __asm__ volatile("" ::"v"(back8), "v"(back_row));
  const float prev = (lane & 8) ? back8 : back_row;
  const float my_top = run;
  const float my_old = seen_before ? prev : top;
  const bool chunk_live = seen_tiles != 0;
  const float cm = chunk_live ? lane_value(run, 63) : 0.0f;  // the chunk's maximum
  // The weight by each key's lane, the tile factor by every lane of the tile.
  // (exp2 of -200 is 0, of 0 is 1: no branch around either.)
  const float e = exp2_select(live ? sl - my_top : -200.0f);
  const float fa = exp2_select(tile_seen && my_old != my_top ? my_old - my_top : 0.0f);
  S.e[w][lane] = e;
  if ((lane & 7) == 0) S.a[w][tile] = fa;
  // Each tile's weights summed in order at its first lane, then
  // l = l a + sum over the seen tiles in order.
  float tsum = 0.0f;
  tsum = tsum + e;
  tsum = tsum + row_shl<1>(e);
  tsum = tsum + row_shl<2>(e);
  tsum = tsum + row_shl<3>(e);
  tsum = tsum + row_shl<4>(e);
  tsum = tsum + row_shl<5>(e);
  tsum = tsum + row_shl<6>(e);
  tsum = tsum + row_shl<7>(e);
  wave_lds_sync();
  const size_t slot_at = ((size_t)row * a.max_chunks + blockIdx.x) * QH + h;
  if (w == kLWave) {
    float cl = 0.0f;
#pragma unroll
    for (int tt = 0; tt < kTiles; ++tt) {
      const float next = cl * lane_value(fa, 8 * tt) + lane_value(tsum, 8 * tt);
      cl = (seen_tiles >> tt) & 1u ? next : cl;
    }
    if (lane == 0 && q == 0) {
      *reinterpret_cast<float4*>(a.stats + slot_at * 4) =
          make_float4(cm, cl, chunk_live ? 1.0f : 0.0f, 0.0f);
    }
  }
  if (w >= kOutWaves) return;
  // O = O a + sum_b e_b v_b per tile, over all 8 tiles: a tile past the
  // chunk's has a = 1 and zero weights and rows, and leaves o as it is (o is
  // never -0, and 0 * 0 adds +0); so does every key past the chunk's end.
  float4 ev[kChunkKeys / 4], av[kTiles / 4];
#pragma unroll
  for (int i = 0; i < kChunkKeys / 4; ++i) ev[i] = ld4f(&S.e[w][4 * i]);
#pragma unroll
  for (int i = 0; i < kTiles / 4; ++i) av[i] = ld4f(&S.a[w][4 * i]);
  float o = 0.0f;
#pragma unroll
  for (int tt = 0; tt < kTiles; ++tt) {
    const float4 at = av[tt / 4];
    o = o * (tt % 4 == 0 ? at.x : tt % 4 == 1 ? at.y : tt % 4 == 2 ? at.z : at.w);
    const float4 ea = ev[2 * tt], eb = ev[2 * tt + 1];
    const float e8[kTileKeys] = {ea.x, ea.y, ea.z, ea.w, eb.x, eb.y, eb.z, eb.w};
#pragma unroll
    for (int b = 0; b < kTileKeys; ++b) {
      o = o + __builtin_fmaf(e8[b], (float)vt[tt * kTileKeys + b], nz);
    }
  }
  a.partials[slot_at * D + q * kDims + t] = o;
}

// ---- a variants step: a workgroup per (chunk, row), a wave per head --------
// Each row of a variants step has its own caches, and the four query heads
// share the one key/value head. A workgroup per (chunk, row) loads the
// chunk's key and value rows straight to LDS once; wave h ropes query head h
// (wave 0 also the step's key and value, appended to the cache by the
// workgroup holding p), then scores head h with a lane a key: the key's 64
// vec4 dots chained in order by its own lane, the one-token kernel's chain.
// Its weights, state and output chains follow the one-token kernel step for
// step, a lane four output dimensions. Rows past the chunk's end read as
// zeros; the step's own rows sit in a spare row 64.
struct RowsShared {
  alignas(16) float q[QH][D];  // roped queries, times scale * log2(e)
  alignas(16) float cosine[D / 2];
  alignas(16) float sine[D / 2];
};

__global__ __launch_bounds__(kThreads) void attention_rows_kernel(const DevStep* __restrict__ step,
                                                                  DecodeAttentionArgs a) {
  __shared__ RowsShared S;
  // The chunk's rows (rows::stage's layout); row 64 holds the step's own key
  // and value.
  __shared__ __align__(16) uint16_t keys[(kChunkKeys + 1) * D];
  __shared__ __align__(16) uint16_t values[(kChunkKeys + 1) * D];
  const int cs = blockIdx.x, row = blockIdx.y;
  const int t = threadIdx.x, w = t >> 6, lane = t & 63;
  a.qkv += (size_t)row * a.qkv_stride;
  a.key_cache += (size_t)row * a.cache_stride;
  a.value_cache += (size_t)row * a.cache_stride;
  const bool key_lane = lane >= 32;
  const int l = lane & 31;
  float2 turn;
  float4 va, vb, xa, xb, ga, gb;
  if (w == 1) turn = ld2f(a.turns + 2 * lane);
  {
    const float* src = a.qkv + (key_lane ? QH : w) * D;
    va = ld4f(src + 4 * l);
    vb = ld4f(src + D / 2 + 4 * l);
    const float* gain = key_lane ? a.key_gain : a.query_gain;
    ga = ld4f(gain + 4 * l);
    gb = ld4f(gain + D / 2 + 4 * l);
  }
  if (w == 0) {
    xa = ld4f(a.qkv + (QH + 1) * D + 4 * l);
    xb = ld4f(a.qkv + (QH + 1) * D + D / 2 + 4 * l);
  }
  __asm__ volatile("" ::: "memory");
  const int p = (int)step->position;
  const ChunkRange r = chunk_range(p, a.window, cs);
  if (cs >= r.count) return;
  const int valid = r.k_end - r.k_begin;
  const bool holds_p = r.c == (p >> 6);
  const int own = holds_p ? valid - 1 : -1;
  const int cached = holds_p ? valid - 1 : valid;
  rows::stage(a.key_cache, a.value_cache, a.slots, r.k_begin, cached, keys, values);
  __builtin_amdgcn_sched_barrier(0);
  if (w == 1) {
    float s0, c0, s1, c1;
    rope_angle(turn.x, (uint32_t)p, &s0, &c0);
    rope_angle(turn.y, (uint32_t)p, &s1, &c1);
    *reinterpret_cast<float2*>(&S.sine[2 * lane]) = make_float2(s0, s1);
    *reinterpret_cast<float2*>(&S.cosine[2 * lane]) = make_float2(c0, c1);
  }
  {
    float sum = rope_lane_squares(va, vb);
    sum = sum + lane_plus16(sum);
    sum = sum + row_shl<8>(sum);
    sum = sum + row_shl<4>(sum);
    sum = sum + row_shl<2>(sum);
    sum = sum + row_shl<1>(sum);
    const int b = __builtin_bit_cast(int, sum);
    const int lo = __builtin_amdgcn_readlane(b, 0), hi = __builtin_amdgcn_readlane(b, 32);
    sum = __builtin_bit_cast(float, key_lane ? hi : lo);
    rope_normalize(va, vb, sum, D, a.epsilon, ga, gb);
  }
  __syncthreads();  // the angles
  rope_rotate(va, vb, l, S.cosine, S.sine);
  if (!key_lane) {
    const float sc = a.scale_log2e;
    *reinterpret_cast<float4*>(&S.q[w][4 * l]) =
        make_float4(va.x * sc, va.y * sc, va.z * sc, va.w * sc);
    *reinterpret_cast<float4*>(&S.q[w][D / 2 + 4 * l]) =
        make_float4(vb.x * sc, vb.y * sc, vb.z * sc, vb.w * sc);
  } else if (w == 0 && holds_p) {
    // The step's key and value rows to the spare row (row 64: no swizzle),
    // and to the cache at slot p.
    const ushort4 ka = pack4_f16(va), kb = pack4_f16(vb);
    const ushort4 pa = pack4_f16(xa), pb = pack4_f16(xb);
    *reinterpret_cast<ushort4*>(keys + kChunkKeys * D + 4 * l) = ka;
    *reinterpret_cast<ushort4*>(keys + kChunkKeys * D + D / 2 + 4 * l) = kb;
    *reinterpret_cast<ushort4*>(values + kChunkKeys * D + 4 * l) = pa;
    *reinterpret_cast<ushort4*>(values + kChunkKeys * D + D / 2 + 4 * l) = pb;
    const size_t at = (size_t)ring_slot(p, a.slots) * D;
    *reinterpret_cast<ushort4*>(a.key_cache + at + 4 * l) = ka;
    *reinterpret_cast<ushort4*>(a.key_cache + at + D / 2 + 4 * l) = kb;
    *reinterpret_cast<ushort4*>(a.value_cache + at + 4 * l) = pa;
    *reinterpret_cast<ushort4*>(a.value_cache + at + D / 2 + 4 * l) = pb;
  }
  __builtin_amdgcn_s_waitcnt(0x0F70);  // this wave's rows landed (vmcnt 0)
  __syncthreads();  // every wave's rows, the queries and the step's rows
  const size_t slot_at = ((size_t)row * a.max_chunks + cs) * QH + w;
  rows::head_state(keys, values, S.q[w], own, valid, r.k_begin, p, a.window,
                   a.stats + slot_at * 4, a.partials + slot_at * D, nullptr);
}

}  // namespace

hipError_t launch_attention_decode(hipStream_t s, const DevStep* step,
                                   const DecodeAttentionArgs& a, int rows) {
  if (a.head_dim != D || a.query_heads != QH || a.kv_heads != 1 || rows < 1 ||
      a.grid_chunks < 0 || a.grid_chunks > a.max_chunks)
    return hipErrorInvalidValue;
  const int chunks = a.grid_chunks > 0 ? a.grid_chunks : a.max_chunks;
  // A grid of a few dozen workgroups (a sliding window, one row) is split
  // four ways by output dimension, to spread the value rows over more CUs;
  // a longer one already fills the chip.
  if (rows > 1 && a.qkv_stride > 0) {
    // A variants step: a workgroup per (chunk, row), the heads sharing its
    // rows.
    hipLaunchKernelGGL(attention_rows_kernel, dim3(chunks, rows), dim3(kThreads), 0, s, step, a);
  } else if (chunks * rows <= 16) {
    hipLaunchKernelGGL(attention_decode_kernel<4>, dim3(chunks, QH * 4, rows), dim3(kThreads), 0,
                       s, step, a);
  } else {
    hipLaunchKernelGGL(attention_decode_kernel<1>, dim3(chunks, QH, rows), dim3(kThreads), 0, s,
                       step, a);
  }
  return hipGetLastError();
}

}  // namespace frz
