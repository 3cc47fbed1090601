// Device-side building blocks shared by the gfx950 decode-attention kernels.
//
// Wave layout used throughout (wave64, lane = threadIdx.x & 63):
//   t = m = n = lane & 15   (MFMA row / column index inside a 16x16 block)
//   g = lane >> 4           (which quarter of the MFMA reduction dimension)
// A 32-token tile is consumed by v_mfma_f32_16x16x32_f16:
//   QK : S[16 tokens x 16 heads] = K_tile[16 x 128] . Q^T, four MFMAs per
//        16-token block; lane (t, g) feeds K row t, channels 32c+8g..+7.
//   PV : O^T[16 channels x 16 heads] += V^T[16 x 32 tokens] . P^T, one MFMA
//        per channel offset jj; lane (m, g) feeds channel 8m+jj of the tile's
//        tokens tau(g, j) = 16*(j/4) + 4g + j%4, which is exactly the set of
//        tokens whose probabilities the same lane holds after QK.
// The GQA group (<= 16 query heads sharing one KV head) fills the 16 MFMA
// columns, so every K/V byte is read from HBM once per KV head.
//
// Memory access: every cache read is a raw buffer load against a resource
// that covers exactly the bytes of one region of one KV head.  A load past
// the region (the rows of a partial last tile, or the dummy loads a wave
// issues once its work queue is empty) returns zeros without touching
// memory, so a stream issues the same instructions whatever its state and
// the compiler's memory-counter waits stay exact across the prefetch ring.
// Every instruction of an fp16 tile reads 4 whole 256-byte rows (K) or 4
// whole rows (V); K is transposed into MFMA operand order through the wave's
// LDS slot.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kvdec.h"

namespace kvdec {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4v __attribute__((ext_vector_type(4)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef float float2v __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kHeadDim = 128;               // D: fixed by the MFMA tiling below
constexpr int kRowBytes = kHeadDim * 2;     // one fp16 K or V row
constexpr int kTile = 32;                   // tokens per tile (one KIVI group)
constexpr int kMaxGroup = 16;               // query heads per KV head (MFMA columns)
constexpr int kSlotBytes = kTile * kRowBytes;   // per-wave LDS slot: one K tile
constexpr uint32_t kOOB = 0x80000000u;      // buffer offset past every region

// Cache policy of the streaming K/V/code loads: non-temporal (read once per
// step; keeps them from displacing the caches' dirty lines).
#ifndef KVDEC_STREAM_AUX
#define KVDEC_STREAM_AUX 2
#endif
constexpr int kStreamAux = KVDEC_STREAM_AUX;

typedef __amdgpu_buffer_rsrc_t rsrc_t;

// Raw (unstructured) buffer resource over `bytes` bytes at `base`.
__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
}
__device__ __forceinline__ u32x4 bload16(rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kStreamAux);
}
__device__ __forceinline__ uint32_t bload4(rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, kStreamAux);
}

// The same with a wave-uniform byte offset `soff` added (an SGPR operand,
// outside the range check, which applies to `off`: an `off` of kOOB still
// reads zeros without a memory access).
__device__ __forceinline__ u32x4 bload16(rsrc_t r, uint32_t off, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, off, soff, kStreamAux);
}
__device__ __forceinline__ uint32_t bload4(rsrc_t r, uint32_t off, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, off, soff, kStreamAux);
}

__device__ __forceinline__ half8 as_h8(u32x4 v) { return __builtin_bit_cast(half8, v); }
__device__ __forceinline__ u32x4 as_u4(half8 v) { return __builtin_bit_cast(u32x4, v); }

// Sum / max over the four lanes t, t + 16, t + 32, t + 48 (the lane groups g
// of one MFMA row), left in all four.  Each step swaps rows between two
// copies of x with a VALU lane swap (no LDS round trip): after
// v_permlane16_swap the copies hold rows (0, 0, 2, 2) and (1, 1, 3, 3), after
// v_permlane32_swap the halves (lo, lo) and (hi, hi), so combining the two
// copies combines lanes L and L ^ 16, then L and L ^ 32.
__device__ __forceinline__ float group_sum(float x) {
  const uint32_t a = __builtin_bit_cast(uint32_t, x);
  const auto s16 = __builtin_amdgcn_permlane16_swap(a, a, false, false);
  const float y = __builtin_bit_cast(float, (uint32_t)s16[0]) + __builtin_bit_cast(float, (uint32_t)s16[1]);
  const uint32_t b = __builtin_bit_cast(uint32_t, y);
  const auto s32 = __builtin_amdgcn_permlane32_swap(b, b, false, false);
  return __builtin_bit_cast(float, (uint32_t)s32[0]) + __builtin_bit_cast(float, (uint32_t)s32[1]);
}
__device__ __forceinline__ float group_max(float x) {
  const uint32_t a = __builtin_bit_cast(uint32_t, x);
  const auto s16 = __builtin_amdgcn_permlane16_swap(a, a, false, false);
  const float y = fmaxf(__builtin_bit_cast(float, (uint32_t)s16[0]), __builtin_bit_cast(float, (uint32_t)s16[1]));
  const uint32_t b = __builtin_bit_cast(uint32_t, y);
  const auto s32 = __builtin_amdgcn_permlane32_swap(b, b, false, false);
  return fmaxf(__builtin_bit_cast(float, (uint32_t)s32[0]), __builtin_bit_cast(float, (uint32_t)s32[1]));
}

__device__ __forceinline__ float4v mfma16x16x32(u32x4 a, half8 b, float4v c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(as_h8(a), b, c, 0, 0, 0);
}

// Packed KIVI layout, for query groups of at most kPackGroup heads: the MFMA
// columns (QK) and rows (PV) 8..15, padding otherwise, carry the fp16
// remainder half of each two-part operand, so one MFMA does the work of a
// head-and-remainder pair; lanes n and n + 8 of a row of 16 hold the same
// head n & 7.  pack_lanes is all ones in the lanes n >= 8.
constexpr int kPackGroup = 8;
__device__ __forceinline__ uint32_t pack_lanes(int lane) { return (lane & 8) ? ~0u : 0u; }

// x plus the x of lane n ^ 8 of the same row of 16 lanes (DPP row_ror:8).
__device__ __forceinline__ float add_half_row(float x) {
  const int y = __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x128, 0xf, 0xf, false);
  return x + __builtin_bit_cast(float, y);
}

// Token (0..31) of a tile held in slot j (0..7) by lane group g: the C-layout
// of two stacked 16x16 QK blocks, reused as the PV reduction order.
__device__ __forceinline__ int tau(int g, int j) { return 16 * (j >> 2) + 4 * g + (j & 3); }

// Per-wave online-softmax state.  Lane (n, g) owns head n; logits are kept
// in the log2 domain (scaled by sm_scale * log2(e)).
//   O[jj][r] : unnormalised output of head n, channel 8*(4g + r) + jj
//   m        : reference max of head n, identical in the four lanes of a head;
//              starts at a finite sentinel so exp2(-inf - m) is 0, never NaN
//   l        : this lane's share of the softmax denominator
//   fs       : pending factor of O: max refreshes made by quantized tiles
//              after the wave's last fp16 tile multiply fs, not the 32
//              values of O (applied when O is published)
struct WaveState {
  float4v O[8];
  float m;
  float l;
  float fs;
};

constexpr float kMaxSentinel = -1e30f;
// The reference max is refreshed only when a tile's max exceeds it by more
// than this (log2 units), so probabilities stay <= 2^8: exact range for the
// fp16 P operand, and most tiles skip the cross-lane max and the O rescale.
constexpr float kRescaleSlack = 8.0f;

__device__ __forceinline__ void wave_state_init(WaveState& st) {
#pragma unroll
  for (int jj = 0; jj < 8; ++jj) st.O[jj] = float4v{0.f, 0.f, 0.f, 0.f};
  st.m = kMaxSentinel;
  st.l = 0.f;
  st.fs = 1.f;
}

// Slot validity inside one KV head: s < va, or vb <= s < vc (slot numbers of
// one head fit in 31 bits).  Dense uses va = L; the sparse and KIVI caches
// use the StreamingLLM sink / window ranges.
struct SlotRanges {
  int va, vb, vc;
};

__device__ __forceinline__ bool slot_valid(const SlotRanges& R, int s) {
  return s < R.va || (s >= R.vb && s < R.vc);
}

// Validity ranges of the [sink + window] cache at this length (the
// _kv_indices rule for the linear layout), clamped into [0, sink + window].
__host__ __device__ inline SlotRanges sparse_ranges(int64_t seq_len, int32_t window, int32_t sink,
                                                   int32_t layout) {
  const int64_t S = sink, W = window, n = S + W;
  auto clamp = [n](int64_t v) { return (int)(v < 0 ? 0 : (v > n ? n : v)); };
  SlotRanges R;
  R.va = clamp(seq_len < S ? seq_len : S);
  if (layout == KVDEC_LAYOUT_LINEAR) {
    const int64_t lo = 2 * S + W - seq_len;
    R.vb = clamp(lo > S ? lo : S);
    R.vc = clamp(n);
  } else {
    int64_t nwin = seq_len - S;
    if (nwin < 0) nwin = 0;
    if (nwin > W) nwin = W;
    R.vb = clamp(S);
    R.vc = clamp(S + nwin);
  }
  return R;
}

// The slots of a 32-token tile: tile row r (0..31) is slot
// base + step * (r >> 2) + (r & 3).  step 4 is the contiguous tile
// base .. base + 31; step 4n interleaves the n tiles of a group four rows
// at a time, so that the group's waves, loading their tiles together, read
// contiguous rows (measured: the sparse fp16 loads take 15% less time than
// with each wave on its own 8 KB of rows).
struct TileRows {
  int base, step;
};

__device__ __forceinline__ int tile_slot(const TileRows& T, int r) {
  return T.base + T.step * (r >> 2) + (r & 3);
}

// True when every token of the tile is valid (wave-uniform: the slots and
// the ranges are the same in every lane); the span of slots is tested, which
// for an interleaved tile also covers the other tiles' rows in between.
__device__ __forceinline__ bool tile_fully_valid(const SlotRanges& R, const TileRows& T) {
  const int first = T.base, last = tile_slot(T, kTile - 1);
  return last < R.va || (first >= R.vb && last < R.vc);
}
__device__ __forceinline__ bool tile_fully_valid(const SlotRanges& R, int slot0) {
  return tile_fully_valid(R, TileRows{slot0, 4});
}

// True when some slot of the tile's span is valid.
__device__ __forceinline__ bool tile_any_valid(const SlotRanges& R, const TileRows& T) {
  const int first = T.base, end = tile_slot(T, kTile - 1) + 1;
  return first < R.va || (end > R.vb && first < R.vc);
}
__device__ __forceinline__ bool tile_any_valid(const SlotRanges& R, int slot0) {
  return tile_any_valid(R, TileRows{slot0, 4});
}

// Validity bits of the lane's 8 tokens tau(g, j) of the tile (tokens at or
// past xlim do not belong to the region).
__device__ __forceinline__ uint32_t tile_valid_bits(const SlotRanges& R, const TileRows& T, int xlim,
                                                    int lane) {
  const int g = lane >> 4;
  uint32_t bits = 0;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int tok = tau(g, j);
    bits |= (tok < xlim && slot_valid(R, tile_slot(T, tok))) ? (1u << j) : 0u;
  }
  return bits;
}
__device__ __forceinline__ uint32_t tile_valid_bits(const SlotRanges& R, int slot0, int xlim,
                                                    int lane) {
  return tile_valid_bits(R, TileRows{slot0, 4}, xlim, lane);
}

// Consume one tile: QK on MFMA, masking, online softmax, PV on MFMA.
//   kop(blk, c) -> u32x4 : K operand of block blk, channel chunk c
//                          (K[token 16*blk + t][channels 32c + 8g .. +7])
//   vop(w, j)   -> u32   : dword w of V row j, i.e. channels 8m+2w, 8m+2w+1
//                          of token tau(g, j)
// FULL: every token of the tile is valid.  Otherwise bit j of `valid` says
// whether the lane's token tau(g, j) is, and masked logits become -inf.
// resc(alpha) rescales any other accumulators that share st.m (alpha per
// head, in lane layout) when the reference max is refreshed.
// The probabilities of a tile's tokens in the lane layout of the PV operand:
// p = pB + pL, the fp16 head and the fp16 rounding of the remainder (the
// remainder is exact in fp32), so the PV product carries p to ~2^-22
// instead of fp16's 2^-11 (one dominant token would otherwise put that
// whole rounding error into the output).
struct TileProbs {
  half8 pB, pL;
};

// QK, masking and the online-softmax update of one tile (the first half of
// tile_body): returns the tile's probabilities against the updated st.m.
template <bool FULL, class KOp, class Resc>
__device__ __forceinline__ TileProbs tile_probs(KOp&& kop, uint32_t valid, const half8 (&qB)[4],
                                                float scale_log2, WaveState& st, Resc&& resc) {
  float4v s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    s0 = mfma16x16x32(kop(0, c), qB[c], s0);
    s1 = mfma16x16x32(kop(1, c), qB[c], s1);
  }

  float x[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    x[j] = (j < 4 ? s0[j & 3] : s1[j & 3]) * scale_log2;
    if (!FULL) x[j] = ((valid >> j) & 1u) ? x[j] : -INFINITY;
  }
  float lmax = x[0];
#pragma unroll
  for (int j = 1; j < 8; ++j) lmax = fmaxf(lmax, x[j]);

  // Refresh the reference max only if some lane's tile max exceeds it by
  // more than kRescaleSlack (wave-uniform branch).  While every head is at
  // the sentinel nothing has been accumulated (l and O are zero), so the
  // wave's first refresh skips the rescale.
  if (__ballot(lmax > st.m + kRescaleSlack)) {
    const float mt = group_max(lmax);
    const float mnew = fmaxf(st.m, mt);
    if (__ballot(st.m != kMaxSentinel)) {
      const float alpha = __builtin_amdgcn_exp2f(st.m - mnew);
      st.l *= alpha;
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) st.O[jj] = st.O[jj] * alpha;
      resc(alpha);
    }
    st.m = mnew;
  }

  TileProbs P;
  float ls = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float p = __builtin_amdgcn_exp2f(x[j] - st.m);
    ls += p;
    P.pB[j] = (_Float16)p;
    P.pL[j] = (_Float16)__builtin_fmaf(-1.0f, (float)P.pB[j], p);
  }
  st.l += ls;
  return P;
}

// PV of one tile (the second half of tile_body).
template <class VOp>
__device__ __forceinline__ void tile_pv(VOp&& vop, const TileProbs& P, WaveState& st) {
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    uint32_t d[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) d[j] = vop(w, j);
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const uint32_t sel = e ? 0x07060302u : 0x05040100u;
      u32x4 a;
      a[0] = __builtin_amdgcn_perm(d[1], d[0], sel);
      a[1] = __builtin_amdgcn_perm(d[3], d[2], sel);
      a[2] = __builtin_amdgcn_perm(d[5], d[4], sel);
      a[3] = __builtin_amdgcn_perm(d[7], d[6], sel);
      st.O[2 * w + e] = mfma16x16x32(a, P.pB, st.O[2 * w + e]);
      st.O[2 * w + e] = mfma16x16x32(a, P.pL, st.O[2 * w + e]);
    }
  }
}

template <bool FULL, class KOp, class VOp, class Resc>
__device__ __forceinline__ void tile_body(KOp&& kop, VOp&& vop, uint32_t valid,
                                          const half8 (&qB)[4], float scale_log2, WaveState& st,
                                          Resc&& resc) {
  const TileProbs P = tile_probs<FULL>(kop, valid, qB, scale_log2, st, resc);
  tile_pv(vop, P, st);
}

// ---------------------------------------------------------------------------
// fp16 tiles
// ---------------------------------------------------------------------------

// One 32-token fp16 tile as loaded:
//   k[i] : K[row 4i + g][channels 8t .. 8t+7]     (whole rows per instruction)
//   v[j] : V[row tau(g, j)][channels 8t .. 8t+7]  (V operand order after perm)
struct F16Raw {
  u32x4 k[8];
  u32x4 v[8];
};

// Issue the loads of the tile whose first row sits at byte `base` of the
// region (kOOB: no tile, every load returns zeros without a memory access).
__device__ __forceinline__ void load_f16(rsrc_t rk, rsrc_t rv, uint32_t base, int lane,
                                         F16Raw& X) {
  const uint32_t t = lane & 15, g = lane >> 4;
#pragma unroll
  for (int i = 0; i < 8; ++i) X.k[i] = bload16(rk, base + (4u * i + g) * kRowBytes + 16u * t);
#pragma unroll
  for (int j = 0; j < 8; ++j) X.v[j] = bload16(rv, base + (uint32_t)tau(g, j) * kRowBytes + 16u * t);
}

// The tile whose row r is region row tile_slot(T, r) (live == false: zeros,
// no access), against a resource whose region starts `soff` bytes in.
__device__ __forceinline__ void load_f16(rsrc_t rk, rsrc_t rv, const TileRows& T, bool live, uint32_t soff,
                                         int lane, F16Raw& X) {
  const uint32_t t = lane & 15, g = lane >> 4;
  const uint32_t base = live ? (uint32_t)T.base * kRowBytes + 16u * t : kOOB;
  const uint32_t step = (uint32_t)T.step * kRowBytes;
#pragma unroll
  for (int i = 0; i < 8; ++i) X.k[i] = bload16(rk, base + (uint32_t)i * step + g * kRowBytes, soff);
#pragma unroll
  for (int j = 0; j < 8; ++j)
    X.v[j] = bload16(rv, base + (4u * (j >> 2) + g) * step + (uint32_t)(j & 3) * kRowBytes, soff);
}

// load_f16 against a resource over a whole tensor, the KV head's region
// starting `soff` bytes in.
__device__ __forceinline__ void load_f16(rsrc_t rk, rsrc_t rv, uint32_t base, uint32_t soff, int lane,
                                         F16Raw& X) {
  const uint32_t t = lane & 15, g = lane >> 4;
#pragma unroll
  for (int i = 0; i < 8; ++i) X.k[i] = bload16(rk, base + (4u * i + g) * kRowBytes + 16u * t, soff);
#pragma unroll
  for (int j = 0; j < 8; ++j) X.v[j] = bload16(rv, base + (uint32_t)tau(g, j) * kRowBytes + 16u * t, soff);
}

// The same, reading only the rows whose slots (slot0 + row) are valid in R:
// the other rows' registers hold zeros and cost no memory access.
__device__ __forceinline__ void load_f16(rsrc_t rk, rsrc_t rv, uint32_t base, uint32_t soff,
                                         const SlotRanges& R, int slot0, int lane, F16Raw& X) {
  const uint32_t t = lane & 15, g = lane >> 4;
  auto off = [&](uint32_t row) {
    return slot_valid(R, slot0 + (int)row) ? base + row * kRowBytes + 16u * t : kOOB;
  };
#pragma unroll
  for (int i = 0; i < 8; ++i) X.k[i] = bload16(rk, off(4u * i + g), soff);
#pragma unroll
  for (int j = 0; j < 8; ++j) X.v[j] = bload16(rv, off((uint32_t)tau(g, j)), soff);
}

// LDS byte offset of 16-byte chunk `chunk` of K row `row` inside a wave slot:
// chunks are XOR-swizzled by the row so that both the row-wise stores and
// the column-wise MFMA operand reads hit 16 distinct bank groups.
__device__ __forceinline__ uint32_t kslot_off(uint32_t row, uint32_t chunk) {
  return row * kRowBytes + 16u * (chunk ^ (row & 15u));
}

struct NoRescale {
  __device__ __forceinline__ void operator()(float) const {}
};

// Consume an fp16 tile.  V rows of masked tokens are replaced by zeros at use
// time: unwritten cache slots may hold anything, including non-finite values.
template <class Resc = NoRescale>
__device__ __forceinline__ void f16_tile_step(const F16Raw& X, char* slot, const half8 (&qB)[4],
                                              const TileRows& T, const SlotRanges& R, float scale_log2,
                                              WaveState& st, int lane, Resc&& resc = Resc()) {
  const uint32_t t = lane & 15, g = lane >> 4;
#pragma unroll
  for (int i = 0; i < 8; ++i)
    *reinterpret_cast<u32x4*>(slot + kslot_off(4u * i + g, t)) = X.k[i];
  auto kop = [&](int blk, int c) {
    return *reinterpret_cast<const u32x4*>(slot + kslot_off(16u * blk + t, 4u * c + g));
  };
  if (tile_fully_valid(R, T)) {
    tile_body<true>(kop, [&](int w, int j) { return X.v[j][w]; }, 0u, qB, scale_log2, st, resc);
  } else {
    const uint32_t valid = tile_valid_bits(R, T, kTile, lane);
    tile_body<false>(kop, [&](int w, int j) { return ((valid >> j) & 1u) ? X.v[j][w] : 0u; },
                     valid, qB, scale_log2, st, resc);
  }
}

// An fp16 tile in two phases, for a wave that issues the tile's V loads
// only after its K data has arrived: the QK and softmax half runs while the
// V rows are still in flight, so only the PV half follows the last byte.
//   f16_tile_probs: stage K (X.k), QK, softmax; returns the probabilities
//   and the tile's validity bits (all ones for a fully valid tile)
//   f16_tile_pv:    PV from X.v (V rows of masked tokens read as zeros)
__device__ __forceinline__ TileProbs f16_tile_probs(const F16Raw& X, char* slot, const half8 (&qB)[4],
                                                    const TileRows& T, const SlotRanges& R, float scale_log2,
                                                    WaveState& st, int lane, uint32_t& valid) {
  const uint32_t t = lane & 15, g = lane >> 4;
#pragma unroll
  for (int i = 0; i < 8; ++i)
    *reinterpret_cast<u32x4*>(slot + kslot_off(4u * i + g, t)) = X.k[i];
  auto kop = [&](int blk, int c) {
    return *reinterpret_cast<const u32x4*>(slot + kslot_off(16u * blk + t, 4u * c + g));
  };
  if (tile_fully_valid(R, T)) {
    valid = 0xffu;
    return tile_probs<true>(kop, 0u, qB, scale_log2, st, NoRescale());
  }
  valid = tile_valid_bits(R, T, kTile, lane);
  return tile_probs<false>(kop, valid, qB, scale_log2, st, NoRescale());
}
__device__ __forceinline__ void f16_tile_pv(const F16Raw& X, const TileProbs& P, uint32_t valid, WaveState& st) {
  tile_pv([&](int w, int j) { return ((valid >> j) & 1u) ? X.v[j][w] : 0u; }, P, st);
}

// A value the compiler must treat as depending on the tile's probabilities,
// so that loads addressed with it are issued only after them.
__device__ __forceinline__ bool after_probs(bool live, const TileProbs& P) {
  uint32_t x = live ? 1u : 0u;
  asm volatile("" : "+v"(x) : "v"(as_u4(P.pB)), "v"(as_u4(P.pL)));
  return x != 0u;
}

// K or V loads of a tile (the halves of load_f16 above).
__device__ __forceinline__ void load_f16_k(rsrc_t rk, const TileRows& T, bool live, uint32_t soff, int lane,
                                           F16Raw& X) {
  const uint32_t t = lane & 15, g = lane >> 4;
  const uint32_t base = live ? (uint32_t)T.base * kRowBytes + 16u * t : kOOB;
  const uint32_t step = (uint32_t)T.step * kRowBytes;
#pragma unroll
  for (int i = 0; i < 8; ++i) X.k[i] = bload16(rk, base + (uint32_t)i * step + g * kRowBytes, soff);
}
__device__ __forceinline__ void load_f16_v(rsrc_t rv, const TileRows& T, bool live, uint32_t soff, int lane,
                                           F16Raw& X) {
  const uint32_t t = lane & 15, g = lane >> 4;
  const uint32_t base = live ? (uint32_t)T.base * kRowBytes + 16u * t : kOOB;
  const uint32_t step = (uint32_t)T.step * kRowBytes;
#pragma unroll
  for (int j = 0; j < 8; ++j)
    X.v[j] = bload16(rv, base + (4u * (j >> 2) + g) * step + (uint32_t)(j & 3) * kRowBytes, soff);
}

// The contiguous tile of slots slot0 .. slot0 + 31.
template <class Resc = NoRescale>
__device__ __forceinline__ void f16_tile_step(const F16Raw& X, char* slot, const half8 (&qB)[4],
                                              int slot0, const SlotRanges& R, float scale_log2,
                                              WaveState& st, int lane, Resc&& resc = Resc()) {
  f16_tile_step(X, slot, qB, TileRows{slot0, 4}, R, scale_log2, st, lane, resc);
}

// ---------------------------------------------------------------------------
// KIVI 2-bit tiles
// ---------------------------------------------------------------------------

// Device pointers of one KIVI-quantized region of one KV head.  A 32-token
// tile tq is one quantization group: 1 KB of K codes (8 byte rows of 128
// channels), 128 K scales and zeros, 1 KB of V codes (32 tokens x 32 bytes),
// 32 x 4 V scales and zeros -- six contiguous pieces.
struct QRegion {
  const uint8_t* kp;     // [ntok/4][128]
  const _Float16* ks;    // [ntok/32][128]
  const _Float16* kz;
  const uint8_t* vp;     // [ntok][32]
  const _Float16* vs;    // [ntok][4]
  const _Float16* vz;
};

// A tile as loaded: every lane fetches a 1/64 slice of each piece with one
// coalesced load (12 VGPRs per tile, no duplication across lanes).
struct QTileRaw {
  u32x4 kc;            // K code bytes [16L, 16L+16)
  u32x4 vc;            // V code bytes [16L, 16L+16)
  uint32_t ks, kz;     // K scale / zero of channels 2L, 2L+1
  uint32_t vs, vz;     // V scale / zero of token L/2, groups 2(L%2), 2(L%2)+1
};

// Resources over the six whole tensors of a KIVI region (all KV heads):
// every 32-token group is 1024 bytes of K codes and of V codes and 256 bytes
// of each scale / zero piece, so group n starts at n * 1024 and n * 256.
struct QTensors {
  rsrc_t kc, vc, ks, kz, vs, vz;
};

__device__ __forceinline__ QTensors q_tensors(const QRegion& Q, uint32_t code_bytes, uint32_t meta_bytes) {
  return QTensors{make_rsrc(Q.kp, code_bytes), make_rsrc(Q.vp, code_bytes), make_rsrc(Q.ks, meta_bytes),
                  make_rsrc(Q.kz, meta_bytes), make_rsrc(Q.vs, meta_bytes), make_rsrc(Q.vz, meta_bytes)};
}

// Issue the loads of group n of the tensors (valid == false: zeros, no
// access); the group's offsets go in the scalar offset field.
__device__ __forceinline__ void load_q_group(const QTensors& T, uint32_t n, bool valid, int lane, QTileRaw& X) {
  const uint32_t oc = n * 1024u, om = n * 256u;
  const uint32_t l16 = valid ? 16u * lane : kOOB, l4 = valid ? 4u * lane : kOOB;
  X.kc = bload16(T.kc, l16, oc);
  X.vc = bload16(T.vc, l16, oc);
  X.ks = bload4(T.ks, l4, om);
  X.kz = bload4(T.kz, l4, om);
  X.vs = bload4(T.vs, l4, om);
  X.vz = bload4(T.vz, l4, om);
}

// Bytes of a group's pieces that hold its first `rows` tokens: K code byte
// rows of 4 tokens x 128 channels, V code rows of 32 bytes, V scale / zero
// rows of 4 fp16 (the K scales and zeros are per channel: all 256 bytes).
// A sink group holds `sink` real tokens padded to 32 with copies of token 0
// (quant_kernel.py:602-606); its padding is masked in the decode, so only
// these rows are read and the rest return zeros without a memory access.
__device__ __forceinline__ uint32_t q_kcode_bytes(int rows) { return 128u * (uint32_t)((rows + 3) / 4); }
__device__ __forceinline__ uint32_t q_vcode_bytes(int rows) { return 32u * (uint32_t)rows; }
__device__ __forceinline__ uint32_t q_vmeta_bytes(int rows) { return 8u * (uint32_t)rows; }

// Resources over the sink group of KV head `head` alone (group `head` of
// the sink tensors), sized to its `sink` real tokens; load it as group 0.
__device__ __forceinline__ QTensors q_sink_tensors(const QRegion& Q, uint32_t head, int sink) {
  return QTensors{make_rsrc(Q.kp + (size_t)head * 1024, q_kcode_bytes(sink)),
                  make_rsrc(Q.vp + (size_t)head * 1024, q_vcode_bytes(sink)),
                  make_rsrc(Q.ks + (size_t)head * kHeadDim, 256u),
                  make_rsrc(Q.kz + (size_t)head * kHeadDim, 256u),
                  make_rsrc(Q.vs + (size_t)head * 128, q_vmeta_bytes(sink)),
                  make_rsrc(Q.vz + (size_t)head * 128, q_vmeta_bytes(sink))};
}

// Issue the loads of tile tq of region Q (valid == false: zeros, no access),
// reading only the rows of its first `rows` tokens (32: the whole group).
__device__ __forceinline__ void load_q_raw(const QRegion& Q, int tq, bool valid, int lane,
                                           QTileRaw& X, int rows = kTile) {
  const size_t t = valid ? (size_t)tq : 0;
  const uint32_t nk = valid ? q_kcode_bytes(rows) : 0u, nv = valid ? q_vcode_bytes(rows) : 0u;
  const uint32_t nks = valid ? 256u : 0u, nvs = valid ? q_vmeta_bytes(rows) : 0u;
  X.kc = bload16(make_rsrc(Q.kp + t * 1024, nk), 16u * lane);
  X.vc = bload16(make_rsrc(Q.vp + t * 1024, nv), 16u * lane);
  X.ks = bload4(make_rsrc(Q.ks + t * kHeadDim, nks), 4u * lane);
  X.kz = bload4(make_rsrc(Q.kz + t * kHeadDim, nks), 4u * lane);
  X.vs = bload4(make_rsrc(Q.vs + t * 128, nvs), 4u * lane);
  X.vz = bload4(make_rsrc(Q.vz + t * 128, nvs), 4u * lane);
}

// Accumulators of the KIVI tiles, kept beside WaveState (whose m and l they
// share).  The PV product of a quantized tile is computed transposed,
// O[head][channel] = P'[head][token] . code[token][channel], with each MFMA
// covering 16 channels of one 32-channel V quantization group, so the
// per-token V scale folds into P' = p * scale.  The zero point is a
// separate product, sum_t P'[t] (code - zero) = sum_t P' code + sum_t P'
// (-zero), accumulated into the same block: both products are exact (codes
// 0..3 and the integer zeros are exact fp16 operands).
//   O[2 grp + m][r] : sum_t P'[t][head 4g + r] * (code - zero)[t][ch] for
//                     lane (t, g), channel ch = q_state_channel(grp, m, t)
struct QState {
  float4v O[8];
};

__device__ __forceinline__ void q_state_init(QState& qs) {
#pragma unroll
  for (int b = 0; b < 8; ++b) qs.O[b] = float4v{0.f, 0.f, 0.f, 0.f};
}

// Output channel of accumulator column t of QState::O[2 grp + m]: the two
// accumulators of a group hold adjacent channels.
__device__ __forceinline__ int q_state_channel(int grp, int m, int t) {
  return 32 * grp + 4 * (t & 7) + 2 * (t >> 3) + m;
}

// Rescale by alpha, given per head in lane layout (head = lane & 15); the
// rows of qs.O are heads 4g + r.
__device__ __forceinline__ void q_state_rescale(QState& qs, float alpha, int lane) {
  const int g = lane >> 4;
  float4v ar;
#pragma unroll
  for (int r = 0; r < 4; ++r) ar[r] = __shfl(alpha, 4 * g + r);
#pragma unroll
  for (int b = 0; b < 8; ++b) qs.O[b] = qs.O[b] * ar;
}

// Layout of a staged KIVI tile inside a wave slot (bytes):
//   [0, 1280)     K codes, 8 byte rows x 128 channels (as stored), rows
//                 kQsKRow = 160 bytes apart: QK reads rows 4 blk + 0..3 at
//                 once, which 128-byte rows would put in the same LDS banks
//   [1280, 1536)  K scales [128], [1536, 1792) negated K zeros [128]
//   [1792, 2816)  V codes, 32 token rows x 32 bytes (as stored; read back
//                 transposed by ds_read_b64_tr_b8)
//   [2816, 3072)  V scales transposed [4 groups][32 tokens],
//   [3072, 3328)  negated V zeros transposed
//   [3328, 4608)  the K code rows again, each 32-bit word shifted right by
//                 4 bits (fields 2 and 3 of a byte at its bits 0..3)
constexpr int kQsKRow = 160;
constexpr int kQsK = 0, kQsKS = 1280, kQsKZ = 1536, kQsV = 1792, kQsVS = 2816, kQsVZ = 3072;
constexpr int kQsK4 = 3328;
constexpr int kQsBytes = 4608;
static_assert(kQsBytes <= kSlotBytes, "a staged KIVI tile fits a wave slot");
constexpr uint32_t kNegPk = 0x80008000u;   // sign bits of an fp16 pair
constexpr uint32_t kOnePk = 0x3C003C00u;   // fp16 pair (1, 1)

__device__ __forceinline__ void stage_q_raw(const QTileRaw& X, char* slot, int lane) {
  *reinterpret_cast<u32x4*>(slot + kQsK + kQsKRow * (lane >> 3) + 16 * (lane & 7)) = X.kc;
  *reinterpret_cast<u32x4*>(slot + kQsK4 + kQsKRow * (lane >> 3) + 16 * (lane & 7)) =
      u32x4{X.kc[0] >> 4, X.kc[1] >> 4, X.kc[2] >> 4, X.kc[3] >> 4};
  *reinterpret_cast<uint32_t*>(slot + kQsKS + 4 * lane) = X.ks;
  *reinterpret_cast<uint32_t*>(slot + kQsKZ + 4 * lane) = X.kz ^ kNegPk;
  *reinterpret_cast<u32x4*>(slot + kQsV + 16 * lane) = X.vc;
  // lane L holds the scale / zero of token L/2, groups 2(L%2) and 2(L%2)+1
  const int tok = lane >> 1, g0 = 2 * (lane & 1);
  const uint32_t nvz = X.vz ^ kNegPk;
  *reinterpret_cast<uint16_t*>(slot + kQsVS + g0 * 64 + 2 * tok) = (uint16_t)X.vs;
  *reinterpret_cast<uint16_t*>(slot + kQsVS + (g0 + 1) * 64 + 2 * tok) = (uint16_t)(X.vs >> 16);
  *reinterpret_cast<uint16_t*>(slot + kQsVZ + g0 * 64 + 2 * tok) = (uint16_t)nvz;
  *reinterpret_cast<uint16_t*>(slot + kQsVZ + (g0 + 1) * 64 + 2 * tok) = (uint16_t)(nvz >> 16);
}

// Transposed LDS read (gfx950 ds_read_b64_tr_b8).  In each group of 16
// lanes, lane 2j + h supplies the address of row j (8 bytes; h picks
// columns 8h .. 8h + 7 of a 16-byte row) and lane i receives byte i of every
// row: result byte j = row j, column i.
__device__ __forceinline__ u32x2 lds_read_tr8(const char* p) {
  typedef int v2i __attribute__((ext_vector_type(2)));
  const v2i r = __builtin_amdgcn_ds_read_tr8_b64_v2i32((__attribute__((address_space(3))) v2i*)(p));
  return u32x2{(uint32_t)r[0], (uint32_t)r[1]};
}

// fp16(a0 * b.lo - c.lo) in the low half and fp16(a1 * b.hi - c.hi) in the
// high half of the result, from the fp32 a0, a1 and the fp16 pairs b, c:
// v_fma_mixlo_f16 then v_fma_mixhi_f16 (each writes its half of the dword).
// The compiler's own form of this (two v_fma_mix_f32 and a
// v_cvt_pk_f16_f32, rounding twice) measured no faster in the kernels.
__device__ __forceinline__ uint32_t fma_mix_pk_f16(float a0, float a1, uint32_t b, uint32_t c) {
  uint32_t d;
  asm("v_fma_mixlo_f16 %0, %1, %2, -%3 op_sel_hi:[0,1,1]" : "=v"(d) : "v"(a0), "v"(b), "v"(c));
  asm("v_fma_mixhi_f16 %0, %1, %2, -%3 op_sel:[0,1,1] op_sel_hi:[0,1,1]" : "+v"(d) : "v"(a1), "v"(b), "v"(c));
  return d;
}

// Four 2-bit codes, one in bits 0..1 of each byte of `c` (the other bits
// zero), as four exact fp16 values: such a byte is the OCP fp8 e4m3
// subnormal code * 2^-9, which v_cvt_scalef32_pk_f16_fp8 widens and scales
// by `scale` in one step per pair of bytes.
__device__ __forceinline__ u32x2 codes_f16(uint32_t c, float scale) {
  return u32x2{__builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(c, scale, false)),
               __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(c, scale, true))};
}
constexpr float kCodeScale = 512.0f;   // code * 2^-9 * 2^9 = code
// A code at bits 2..3 of a byte whose other bits are zero reads, as an OCP
// e4m3 byte, as code * 2^-7 (code 1 the subnormal 2^-7, codes 2 and 3 the
// least normal binade's 2^-6 and 1.5 * 2^-6): such fields need no shift.
constexpr float kCodeScale2 = 128.0f;
constexpr uint32_t kField0 = 0x03030303u, kField1 = 0x0C0C0C0Cu;

// |x| <= 2^(E - 15) (1 + m / 1024) for the fp16 bits x of exponent E and
// mantissa m: the least el with |x| <= 2^el (for normal x).
__device__ __forceinline__ int absmax_exp_raw(uint32_t x) {
  return (int)(x >> 10) - 15 + ((x & 0x3FFu) != 0u ? 1 : 0);
}
// Power-of-two prescale of the Q operand for quantized tiles.  Their QK
// forms the fp16 product q * scale of a query channel and a K channel's
// scale, finite for every fp16 scale only while |q| <= 1 (|q| = 64 with a
// K channel whose 32-token range is above ~3072 would give inf, and the
// MFMA against code 0 NaN).  The products are taken as (q * 2^-e) * scale
// with 2^e the least power of two at or above the KV head's largest |q|
// (e = 0, no change, when that is at most 1), and the quantized tiles'
// logit factor takes 2^e back.  The scaling is exact unless a scaled value
// falls below the fp16 normal range (|q| < 2^(e - 14)).  e is the wave's
// (every wave holds the KV head's whole Q), so it stays uniform.
__device__ __forceinline__ int q_prescale_exp(const half8 (&qB)[4]) {
  typedef uint16_t u16x2 __attribute__((ext_vector_type(2)));
  // |q| bits (unsigned order = the order of non-negative fp16), reduced
  // pairwise in a tree (a serial chain would be 32 dependent steps)
  u16x2 v[16];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const u32x4 u = as_u4(qB[c]);
#pragma unroll
    for (int i = 0; i < 4; ++i) v[4 * c + i] = __builtin_bit_cast(u16x2, u[i] & 0x7FFF7FFFu);
  }
#pragma unroll
  for (int w = 8; w >= 1; w >>= 1)
#pragma unroll
    for (int i = 0; i < w; ++i) v[i] = __builtin_elementwise_max(v[i], v[i + w]);
  const int el = absmax_exp_raw(max(v[0][0], v[0][1]));
  int e = 0;   // the wave's largest el (at most 16), by a search over ballots
#pragma unroll
  for (int b = 16; b >= 1; b >>= 1)
    if (__ballot(el >= e + b)) e += b;
  return min(e, 16);
}
// The fp16 pair (2^-e, 2^-e), 0 <= e <= 16.
__device__ __forceinline__ uint32_t pow2_neg_pk(int e) {
  const uint32_t h = e <= 14 ? (uint32_t)(15 - e) << 10 : 0x0200u >> (e - 15);
  return h | h << 16;
}
// scale_log2 * 2^e, kept uniform.
__device__ __forceinline__ float scale_pow2(float scale_log2, int e) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(
                                       __builtin_bit_cast(int, __builtin_ldexpf(scale_log2, e))));
}
// The Q operand scaled in place by 2^-e; returns the logit factor of every
// quantized tile stepped with it (fp16 tiles, whose products are fp32 and
// cannot overflow, keep the unscaled operand).  The empty asm statements
// keep the multiplies where they are written: called while the wave's tile
// loads are in flight, they would otherwise sink past the loads' wait onto
// the step's critical path.
__device__ __forceinline__ float q_prescale_by(half8 (&qB)[4], int e, float scale_log2) {
  const uint32_t h = pow2_neg_pk(e);
  const half8 p = as_h8(u32x4{h, h, h, h});
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    qB[c] = qB[c] * p;
    asm volatile("" : "+v"(qB[c]));
  }
  return scale_pow2(scale_log2, e);
}
// The same with e found from the operand itself (every wave holds the KV
// head's whole Q).
__device__ __forceinline__ float q_prescale(half8 (&qB)[4], float scale_log2) {
  return q_prescale_by(qB, q_prescale_exp(qB), scale_log2);
}

// Consume one KIVI tile staged in the wave's LDS slot.
//   QK: the codes are exact fp16 integers (A operand); the per-channel K
//       scale goes to the Q side as q * scale = head + remainder, both fp16
//       (the remainder of an fp16 x fp16 product is exact in fp16), so the
//       logits carry the dequantized K exactly instead of fp16 roundings of
//       scale * (code - zero).  The zero point adds -sum_ch zero[ch] *
//       q[ch] * scale[ch] to every token of a head: one extra 16x16 block
//       (the negated zeros, the same in every row, against the same head
//       and remainder of q * scale), so all its rows hold that term and it
//       enters the logits in the fused multiply-add that scales them.
//   softmax: the reference max is refreshed when the tile's max exceeds it
//       by more than `slack`: kRescaleSlack when every V scale of the tile
//       is at most kSlackVScale (then p <= 2^8 and P' = p * vscale < 2^15
//       stays within the fp16 range), otherwise 0 (p <= 1).
// MIXED: the wave also holds fp16-tile accumulators in `st`; a max refresh
// defers their rescale into st.fs (no fp16 tile may follow a MIXED step).
// Without MIXED, st.O must be zero.  HALF: only tokens 0..15 can be valid (the sink
// group), so the second 16-token block is skipped in QK and fed as zeros to
// PV.  Masked tokens get p = 0; their codes are finite.
constexpr float kSlackVScale = 128.0f;

// PACK (query groups of at most kPackGroup heads): QK's B operand holds the
// fp16 product q * scale in columns 0..7 and its exact remainder in columns
// 8..15, so one MFMA per block covers both and lanes n, n + 8 add their
// logits (zero term included); PV's A operand holds P' rounded to fp16 in
// rows 0..7 and the remainder in rows 8..15, which the accumulators keep
// apart until they are published.  The remainder is fp16(pr * scale + e), where
// pB + pr is p (pr = fp16(p - pB)) and e = pB * scale - fp16(pB * scale) is
// exact: ~2^-21 of P' instead of ~2^-22.  Lanes of both halves take each
// operand from one instruction sequence: the lane mask zeroes the
// subtrahend below row 8 and the remainder term's factor.  Subtrahends are
// negated as bits with the mask (one v_bitop3 per dword), not as fp16: the
// compiler turns some fp16 negations of packed operands into three-step
// integer sequences.
template <bool MIXED, bool HALF, bool PACK>
__device__ __forceinline__ void q_tile_body(const char* slot, const half8 (&qB)[4], int slot0,
                                            int xlim, const SlotRanges& R, float scale_log2,
                                            float slack, WaveState& st, QState& qs, int lane,
                                            uint32_t kmul = kOnePk) {
  const int t = lane & 15, g = lane >> 4;
  const uint32_t pm = PACK ? pack_lanes(lane) : 0u;
  // scale and negated zero of the lane's K channels 32c + 8g .. +7; kmul
  // (2^-e, for a Q operand not prescaled itself) joins the scale
  half8 ks[4], nz[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    ks[c] = *reinterpret_cast<const half8*>(slot + kQsKS + 2 * (32 * c + 8 * g));
    if (kmul != kOnePk) ks[c] = ks[c] * as_h8(u32x4{kmul, kmul, kmul, kmul});
    nz[c] = *reinterpret_cast<const half8*>(slot + kQsKZ + 2 * (32 * c + 8 * g));
  }

  // S[token][head] on MFMA: lane (t, g) feeds token 16 blk + t, channels
  // 32c + 8g .. +7 (code byte row (16 blk + t) / 4, bits 2 (t % 4)).
  // Fields 2 and 3 come from the rows shifted by 4 bits, so the lane's
  // field sits at bits 0..1 (t even) or 2..3 (t odd) of each byte and is
  // masked in place.
  const uint32_t kmask = (t & 1) ? kField1 : kField0;
  const float kcs = (t & 1) ? kCodeScale2 : kCodeScale;
  const char* krow = slot + ((t & 2) ? kQsK4 : kQsK) + (t >> 2) * kQsKRow + 8 * g;
  float4v s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
  float4v sz = {0.f, 0.f, 0.f, 0.f};   // the zero term of every token row
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const half8 qh = qB[c] * ks[c];
    // PACK: qh in columns 0..7, the remainder q * scale - qh in 8..15
    const half8 qx =
        PACK ? __builtin_elementwise_fma(qB[c], ks[c], as_h8((as_u4(qh) ^ kNegPk) & pm)) : qh;
    const half8 ql = PACK ? qx : __builtin_elementwise_fma(qB[c], ks[c], -qh);
    sz = mfma16x16x32(as_u4(nz[c]), qx, sz);
    if (!PACK) sz = mfma16x16x32(as_u4(nz[c]), ql, sz);
#pragma unroll
    for (int blk = 0; blk < (HALF ? 1 : 2); ++blk) {
      const u32x2 w = *reinterpret_cast<const u32x2*>(krow + 4 * blk * kQsKRow + 32 * c);
      const u32x2 d0 = codes_f16(w[0] & kmask, kcs), d1 = codes_f16(w[1] & kmask, kcs);
      const u32x4 d = {d0[0], d0[1], d1[0], d1[1]};
      float4v& sb = blk == 0 ? s0 : s1;
      sb = mfma16x16x32(d, qx, sb);
      if (!PACK) sb = mfma16x16x32(d, ql, sb);
    }
  }
  const float xz = sz[0] * scale_log2;
  float x[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    x[j] = fmaf(j < 4 ? s0[j & 3] : s1[j & 3], scale_log2, xz);
    if (PACK) x[j] = add_half_row(x[j]);
  }
  if (!(xlim == kTile && tile_fully_valid(R, slot0))) {
    const uint32_t valid = tile_valid_bits(R, slot0, xlim, lane);
#pragma unroll
    for (int j = 0; j < 8; ++j) x[j] = ((valid >> j) & 1u) ? x[j] : -INFINITY;
  }
  float lmax = x[0];
#pragma unroll
  for (int j = 1; j < 8; ++j) lmax = fmaxf(lmax, x[j]);
  if (__ballot(lmax > st.m + slack)) {
    const float mt = group_max(lmax);
    const float mnew = fmaxf(st.m, mt);
    if (__ballot(st.m != kMaxSentinel)) {   // else nothing accumulated yet
      const float alpha = __builtin_amdgcn_exp2f(st.m - mnew);   // head n (lane layout)
      st.l *= alpha;
      if (MIXED) st.fs *= alpha;
      q_state_rescale(qs, alpha, lane);
    }
    st.m = mnew;
  }
  float pf[8];
  half8 pB;
  float ls = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    pf[j] = __builtin_amdgcn_exp2f(x[j] - st.m);
    ls += pf[j];
    pB[j] = (_Float16)pf[j];
  }
  st.l += ls;
  // PACK: the lane-masked -pB and pr = fp16(p - pB) (zero in rows 0..7)
  u32x4 nBm = {0u, 0u, 0u, 0u}, prm = {0u, 0u, 0u, 0u};
  if (PACK) {
    const u32x4 pBu = as_u4(pB);
    const u32x4 pr = {fma_mix_pk_f16(pf[0], pf[1], kOnePk, pBu[0]), fma_mix_pk_f16(pf[2], pf[3], kOnePk, pBu[1]),
                      fma_mix_pk_f16(pf[4], pf[5], kOnePk, pBu[2]), fma_mix_pk_f16(pf[6], pf[7], kOnePk, pBu[3])};
    nBm = (pBu ^ kNegPk) & pm;
    prm = pr & pm;
  }

  // PV, one V group (32 channels, code byte columns 8 grp .. 8 grp + 7) at
  // a time.  One transposed LDS read gives lane (t, g) byte column
  // 8 grp + (t & 7) of the tokens tau(g, 0..7) (lane t of each lane group
  // supplies the row of token tau(g, t / 2)); MFMA m takes field
  // f = 2 (t >> 3) + m of those bytes (channel 32 grp + 4 (t & 7) + f).
  // P' = p * scale (the per-token V scale of the group) is taken as an fp16
  // head pq and the fp16 remainder pl (as for fp16 tiles);
  // tau(g, 0..3) = 4g..4g+3 and tau(g, 4..7) = 16 + 4g .. +3 sit
  // contiguously in the transposed scale and zero rows.
  const char* vrow = slot + kQsV + 32 * tau(g, t >> 1);
  const uint32_t vsh = 4u * (uint32_t)(t >> 3);
#pragma unroll
  for (int grp = 0; grp < 4; ++grp) {
    const u32x2 s_lo = *reinterpret_cast<const u32x2*>(slot + kQsVS + grp * 64 + 8 * g);
    const u32x2 s_hi = *reinterpret_cast<const u32x2*>(slot + kQsVS + grp * 64 + 32 + 8 * g);
    const u32x2 z_lo = *reinterpret_cast<const u32x2*>(slot + kQsVZ + grp * 64 + 8 * g);
    const u32x2 z_hi = *reinterpret_cast<const u32x2*>(slot + kQsVZ + grp * 64 + 32 + 8 * g);
    const u32x2 vb = lds_read_tr8(vrow + 8 * grp);
    const u32x4 vsc = {s_lo[0], s_lo[1], s_hi[0], s_hi[1]};
    u32x4 pq, pl;
    if (PACK) {
      const half8 hn = as_h8(nBm) * as_h8(vsc);                          // rows >= 8: -fp16(pB s)
      const half8 e = __builtin_elementwise_fma(pB, as_h8(vsc), hn);     // rows < 8: fp16(pB s)
      pq = as_u4(__builtin_elementwise_fma(as_h8(prm), as_h8(vsc), e));  // rows >= 8: pr s + e
      pl = pq;
    } else {
      // head: fp16 product of the fp16 p and scale; remainder: p * scale -
      // head, rounded once (one mixed-precision fused multiply-add per value)
      pq = as_u4(pB * as_h8(vsc));
      pl = u32x4{fma_mix_pk_f16(pf[0], pf[1], vsc[0], pq[0]), fma_mix_pk_f16(pf[2], pf[3], vsc[1], pq[1]),
                 fma_mix_pk_f16(pf[4], pf[5], vsc[2], pq[2]), fma_mix_pk_f16(pf[6], pf[7], vsc[3], pq[3])};
    }
    const half8 nzv = as_h8(u32x4{z_lo[0], z_lo[1], z_hi[0], z_hi[1]});
    // fields vsh / 2 and vsh / 2 + 1 (m = 0, 1) from one shift, each masked
    // in place (bits that cross words land above bit 3 of byte 3)
    const uint64_t vx = ((uint64_t)vb[1] << 32 | vb[0]) >> vsh;
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      const uint32_t msk = m ? kField1 : kField0;
      const float csc = m ? kCodeScale2 : kCodeScale;
      const u32x2 c = {(uint32_t)vx & msk, HALF ? 0u : (uint32_t)(vx >> 32) & msk};
      const u32x2 b0 = codes_f16(c[0], csc);
      const u32x2 b1 = HALF ? u32x2{0u, 0u} : codes_f16(c[1], csc);
      const half8 b = as_h8(u32x4{b0[0], b0[1], b1[0], b1[1]});
      float4v& acc = qs.O[2 * grp + m];
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_h8(pq), b, acc, 0, 0, 0);
      if (!PACK) acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_h8(pl), b, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_h8(pq), nzv, acc, 0, 0, 0);
      if (!PACK) acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(as_h8(pl), nzv, acc, 0, 0, 0);
    }
  }
}

// Stage a loaded tile into the wave's slot and return its rescale slack;
// the registers of `raw` are free afterwards.
__device__ __forceinline__ float q_tile_stage(const QTileRaw& raw, char* slot, int lane) {
  stage_q_raw(raw, slot, lane);
  // every lane holds two of the tile's 128 V scales
  const half2v vs = __builtin_bit_cast(half2v, raw.vs);
  return __ballot(!(fmaxf((float)vs[0], (float)vs[1]) <= kSlackVScale)) ? 0.0f : kRescaleSlack;
}

// Consume the staged tile (xlim real tokens: the sink group has at most 16).
template <bool MIXED, bool PACK = false>
__device__ __forceinline__ void q_tile_consume(char* slot, const half8 (&qB)[4], int slot0, int xlim,
                                               const SlotRanges& R, float scale_log2, float slack,
                                               WaveState& st, QState& qs, int lane,
                                               uint32_t kmul = kOnePk) {
  if (xlim <= kTile / 2)
    q_tile_body<MIXED, true, PACK>(slot, qB, slot0, xlim, R, scale_log2, slack, st, qs, lane, kmul);
  else
    q_tile_body<MIXED, false, PACK>(slot, qB, slot0, xlim, R, scale_log2, slack, st, qs, lane, kmul);
}

template <bool MIXED, bool PACK = false>
__device__ __forceinline__ void q_tile_step(const QTileRaw& raw, char* slot,
                                            const half8 (&qB)[4], int slot0, int xlim,
                                            const SlotRanges& R, float scale_log2, WaveState& st,
                                            QState& qs, int lane, uint32_t kmul = kOnePk) {
  const float slack = q_tile_stage(raw, slot, lane);
  q_tile_consume<MIXED, PACK>(slot, qB, slot0, xlim, R, scale_log2, slack, st, qs, lane, kmul);
}

}  // namespace kvdec
