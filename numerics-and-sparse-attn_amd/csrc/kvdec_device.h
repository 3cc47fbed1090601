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
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace kvdec {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kHeadDim = 128;   // D: fixed by the MFMA tiling below
constexpr int kTile = 32;       // tokens per tile (one KIVI group)
constexpr int kMaxGroup = 16;   // query heads per KV head (MFMA columns)

__device__ __forceinline__ half8 as_h8(u32x4 v) { return __builtin_bit_cast(half8, v); }
__device__ __forceinline__ u32x4 as_u4(half8 v) { return __builtin_bit_cast(u32x4, v); }

__device__ __forceinline__ float4v mfma16x16x32(u32x4 a, half8 b, float4v c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(as_h8(a), b, c, 0, 0, 0);
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
struct WaveState {
  float4v O[8];
  float m;
  float l;
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

// True when every token of the 32-token tile starting at slot0 is valid
// (wave-uniform: slot0 and the ranges are the same in every lane).
__device__ __forceinline__ bool tile_fully_valid(const SlotRanges& R, int slot0) {
  const int last = slot0 + kTile - 1;
  return last < R.va || (slot0 >= R.vb && last < R.vc);
}

// Validity bits of the lane's 8 tokens tau(g, j) of the tile at slot0
// (tokens at or past xlim do not belong to the region).
__device__ __forceinline__ uint32_t tile_valid_bits(const SlotRanges& R, int slot0, int xlim,
                                                    int lane) {
  const int g = lane >> 4;
  uint32_t bits = 0;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int tok = tau(g, j);
    bits |= (tok < xlim && slot_valid(R, slot0 + tok)) ? (1u << j) : 0u;
  }
  return bits;
}

// Consume one tile: QK on MFMA, masking, online softmax, PV on MFMA.
//   kop(blk, c) -> u32x4 : K operand of block blk, channel chunk c
//                          (K[token 16*blk + t][channels 32c + 8g .. +7])
//   vop(w, j)   -> u32   : dword w of V row j, i.e. channels 8m+2w, 8m+2w+1
//                          of token tau(g, j)
// FULL: every token of the tile is valid.  Otherwise bit j of `valid` says
// whether the lane's token tau(g, j) is, and masked logits become -inf.
template <bool FULL, class KOp, class VOp>
__device__ __forceinline__ void tile_body(KOp&& kop, VOp&& vop, uint32_t valid,
                                          const half8 (&qB)[4], float scale_log2, WaveState& st) {
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
  // more than kRescaleSlack (wave-uniform branch).
  if (__ballot(lmax > st.m + kRescaleSlack)) {
    float mt = fmaxf(lmax, __shfl_xor(lmax, 16));
    mt = fmaxf(mt, __shfl_xor(mt, 32));
    const float mnew = fmaxf(st.m, mt);
    const float alpha = __builtin_amdgcn_exp2f(st.m - mnew);
    st.l *= alpha;
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) st.O[jj] = st.O[jj] * alpha;
    st.m = mnew;
  }

  half8 pB;
  float ls = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float p = __builtin_amdgcn_exp2f(x[j] - st.m);
    ls += p;
    pB[j] = (_Float16)p;
  }
  st.l += ls;

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
      st.O[2 * w + e] = mfma16x16x32(a, pB, st.O[2 * w + e]);
    }
  }
}

// ---------------------------------------------------------------------------
// fp16 tiles
// ---------------------------------------------------------------------------

// One 32-token fp16 tile in MFMA operand layout:
//   k[blk][c] : K[token 16*blk + t][channels 32c + 8g .. +7]
//   v[j]      : V[token tau(g, j)][channels 8m .. 8m+7]
struct Tile {
  u32x4 k[2][4];
  u32x4 v[8];
};

// Consume an fp16 tile.  V rows of masked tokens are replaced by zeros at use
// time: unwritten cache slots may hold anything, including non-finite values.
__device__ __forceinline__ void tile_step(const Tile& T, const half8 (&qB)[4], int slot0,
                                          const SlotRanges& R, float scale_log2, WaveState& st,
                                          int lane) {
  auto kop = [&](int blk, int c) { return T.k[blk][c]; };
  if (tile_fully_valid(R, slot0)) {
    tile_body<true>(kop, [&](int w, int j) { return T.v[j][w]; }, 0u, qB, scale_log2, st);
  } else {
    const uint32_t valid = tile_valid_bits(R, slot0, kTile, lane);
    tile_body<false>(kop, [&](int w, int j) { return ((valid >> j) & 1u) ? T.v[j][w] : 0u; },
                     valid, qB, scale_log2, st);
  }
}

// Load an fp16 tile from a [rows, 128] region (one KV head, base pointers
// uniform across the wave).  Rows past the end are clamped to the last row;
// their slots are invalid, so tile_step masks them.
__device__ __forceinline__ void load_f16_tile(const _Float16* __restrict__ kb,
                                              const _Float16* __restrict__ vb, int row0,
                                              int rows, int lane, Tile& T) {
  const int t = lane & 15, g = lane >> 4;
  const char* kc = reinterpret_cast<const char*>(kb);
  const char* vc = reinterpret_cast<const char*>(vb);
#pragma unroll
  for (int blk = 0; blk < 2; ++blk) {
    const int r = min(row0 + 16 * blk + t, rows - 1);
    const uint32_t off = (uint32_t)r * (kHeadDim * 2) + 16u * g;
#pragma unroll
    for (int c = 0; c < 4; ++c) T.k[blk][c] = *reinterpret_cast<const u32x4*>(kc + off + 64u * c);
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int r = min(row0 + tau(g, j), rows - 1);
    T.v[j] = *reinterpret_cast<const u32x4*>(vc + (uint32_t)r * (kHeadDim * 2) + 16u * t);
  }
}

// ---------------------------------------------------------------------------
// KIVI 2-bit tiles
// ---------------------------------------------------------------------------

// Device pointers of one KIVI-quantized region, bound to one KV head.  A
// 32-token tile tq is one quantization group: 1 KB of K codes (8 byte rows of
// 128 channels), 128 K scales and zeros, 1 KB of V codes (32 tokens x 32
// bytes), 32 x 4 V scales and zeros -- six contiguous pieces.
struct QRegion {
  const uint8_t* kp;     // [ntok/4][128]
  const _Float16* ks;    // [ntok/32][128]
  const _Float16* kz;
  const uint8_t* vp;     // [ntok][32]
  const _Float16* vs;    // [ntok][4]
  const _Float16* vz;
};

// A tile as loaded from HBM: every lane fetches a 1/64 slice of each piece
// with one coalesced load (12 VGPRs per tile, no duplication across lanes).
struct QTileRaw {
  u32x4 kc;            // K code bytes [16L, 16L+16)
  u32x4 vc;            // V code bytes [16L, 16L+16)
  uint32_t ks, kz;     // K scale / zero of channels 2L, 2L+1
  uint32_t vs, vz;     // V scale / zero of token L/2, groups 2(L%2), 2(L%2)+1
};

__device__ __forceinline__ void load_q_raw(const QRegion& Q, int tq, int lane, QTileRaw& X) {
  X.kc = *reinterpret_cast<const u32x4*>(Q.kp + (size_t)tq * 1024 + 16 * lane);
  X.vc = *reinterpret_cast<const u32x4*>(Q.vp + (size_t)tq * 1024 + 16 * lane);
  X.ks = *reinterpret_cast<const uint32_t*>(Q.ks + (size_t)tq * kHeadDim + 2 * lane);
  X.kz = *reinterpret_cast<const uint32_t*>(Q.kz + (size_t)tq * kHeadDim + 2 * lane);
  X.vs = *reinterpret_cast<const uint32_t*>(Q.vs + (size_t)tq * 128 + 2 * lane);
  X.vz = *reinterpret_cast<const uint32_t*>(Q.vz + (size_t)tq * 128 + 2 * lane);
}

// Per-wave LDS staging slot of one tile (bytes): K codes [0,1024), K scales
// [1024,1280), K zeros [1280,1536), V codes [1536,2560), V (scale, zero)
// pairs [2560,3072) at 2560 + 16*token + 4*group.
constexpr int kQSlotBytes = 3072;

__device__ __forceinline__ void stage_q_raw(const QTileRaw& X, char* slot, int lane) {
  *reinterpret_cast<u32x4*>(slot + 16 * lane) = X.kc;
  *reinterpret_cast<uint32_t*>(slot + 1024 + 4 * lane) = X.ks;
  *reinterpret_cast<uint32_t*>(slot + 1280 + 4 * lane) = X.kz;
  *reinterpret_cast<u32x4*>(slot + 1536 + 16 * lane) = X.vc;
  u32x2 sz;
  sz[0] = __builtin_amdgcn_perm(X.vz, X.vs, 0x05040100u);   // (scale, zero) of group 2(L%2)
  sz[1] = __builtin_amdgcn_perm(X.vz, X.vs, 0x07060302u);   // (scale, zero) of group 2(L%2)+1
  *reinterpret_cast<u32x2*>(slot + 2560 + 8 * lane) = sz;
}

// The V part of a staged tile in MFMA operand layout (read back from the LDS
// slot; the K operands are read from the slot on demand):
//   vc[i]  : V code bytes (2 x 8 bit) of tokens tau(g, 2i) (low 16 bits) and
//            tau(g, 2i+1) (high 16 bits), channels 8m..8m+7
//   vsz[j] : V scale (low half) and zero (high half) of token tau(g, j),
//            channel group m/4
struct QTileV {
  uint32_t vc[4];
  uint32_t vsz[8];
};

__device__ __forceinline__ void read_q_v(const char* slot, int lane, QTileV& X) {
  const int t = lane & 15, g = lane >> 4;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t lo = *reinterpret_cast<const uint16_t*>(slot + 1536 + tau(g, 2 * i) * 32 + 2 * t);
    const uint32_t hi =
        *reinterpret_cast<const uint16_t*>(slot + 1536 + tau(g, 2 * i + 1) * 32 + 2 * t);
    X.vc[i] = lo | (hi << 16);
  }
#pragma unroll
  for (int j = 0; j < 8; ++j)
    X.vsz[j] = *reinterpret_cast<const uint32_t*>(slot + 2560 + tau(g, j) * 16 + 4 * (t >> 2));
}

// fp16 bit patterns 0x6400 | c encode 1024 + c exactly for c in 0..3; one
// packed subtract of 1024 gives the code itself, a second subtract of the
// stored fp16 zero gives c - z exactly while |c - z| <= 2048 (a rounding of
// at most 2^-11 relative beyond), and the multiply by the fp16 scale is the
// one rounding of the dequantized value (to fp16, the MFMA input type).

// K operand of block blk, chunk c, read from the staged slot: the code bytes
// of byte row (16*blk + t)/4 and the scales / zeros of channels 32c+8g..+7.
__device__ __forceinline__ u32x4 decode_q_k(const char* slot, int blk, int c, int lane) {
  const int t = lane & 15, g = lane >> 4;
  const uint32_t sh = 2u * (uint32_t)(t & 3);   // token 16*blk + t sits at bits 2*(t%4)
  const u32x2 kc =
      *reinterpret_cast<const u32x2*>(slot + (4 * blk + (t >> 2)) * 128 + 32 * c + 8 * g);
  const u32x4 ks = *reinterpret_cast<const u32x4*>(slot + 1024 + 2 * (32 * c + 8 * g));
  const u32x4 kz = *reinterpret_cast<const u32x4*>(slot + 1280 + 2 * (32 * c + 8 * g));
  const uint32_t c0 = (kc[0] >> sh) & 0x03030303u;
  const uint32_t c1 = (kc[1] >> sh) & 0x03030303u;
  u32x4 mg;
  mg[0] = __builtin_amdgcn_perm(c0, 0x64646464u, 0x00050004u);
  mg[1] = __builtin_amdgcn_perm(c0, 0x64646464u, 0x00070006u);
  mg[2] = __builtin_amdgcn_perm(c1, 0x64646464u, 0x00050004u);
  mg[3] = __builtin_amdgcn_perm(c1, 0x64646464u, 0x00070006u);
  const half8 code = as_h8(mg) - (_Float16)1024.0f;
  return as_u4((code - as_h8(kz)) * as_h8(ks));
}

// Dword w of V row j: channels 8m+2w and 8m+2w+1 sit at bits 4w and 4w+2 of
// the row's 16 code bits; b | (b << 14) moves the second one to bit 16 + 4w.
__device__ __forceinline__ uint32_t decode_q_v(const QTileV& X, int w, int j) {
  const uint32_t b = (X.vc[j >> 1] >> (16 * (j & 1))) & 0xffffu;
  const uint32_t t0 = b | (b << 14);
  const uint32_t mg = ((t0 >> (4 * w)) & 0x00030003u) | 0x64006400u;
  // broadcast scale (low half) and zero (high half) to both halves
  const half2v s2 = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(X.vsz[j], X.vsz[j], 0x01000100u));
  const half2v z2 = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(X.vsz[j], X.vsz[j], 0x03020302u));
  const half2v k1024 = {(_Float16)1024.0f, (_Float16)1024.0f};
  const half2v code = __builtin_bit_cast(half2v, mg) - k1024;
  return __builtin_bit_cast(uint32_t, (code - z2) * s2);
}

// Consume one KIVI tile staged in the wave's LDS slot.  Masked tokens get
// probability exactly 0 and their dequantized values are finite, so no row is
// zeroed (the reference masks only its fp16 residual loads).
__device__ __forceinline__ void q_tile_step(const char* slot, const half8 (&qB)[4], int slot0,
                                            int xlim, const SlotRanges& R, float scale_log2,
                                            WaveState& st, int lane) {
  QTileV X;
  read_q_v(slot, lane, X);
  auto kop = [&](int blk, int c) { return decode_q_k(slot, blk, c, lane); };
  auto vop = [&](int w, int j) { return decode_q_v(X, w, j); };
  if (xlim == kTile && tile_fully_valid(R, slot0))
    tile_body<true>(kop, vop, 0u, qB, scale_log2, st);
  else
    tile_body<false>(kop, vop, tile_valid_bits(R, slot0, xlim, lane), qB, scale_log2, st);
}

}  // namespace kvdec
