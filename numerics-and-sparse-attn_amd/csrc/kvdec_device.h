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
constexpr int kTile = 32;       // tokens per tile
constexpr int kWaves = 4;       // waves per workgroup
constexpr int kBlock = 64 * kWaves;
constexpr int kMaxGroup = 16;   // query heads per KV head (MFMA columns)
constexpr float kLog2e = 1.4426950408889634f;

__device__ __forceinline__ half8 as_h8(u32x4 v) { return __builtin_bit_cast(half8, v); }
__device__ __forceinline__ u32x4 as_u4(half8 v) { return __builtin_bit_cast(u32x4, v); }

__device__ __forceinline__ float4v mfma16x16x32(u32x4 a, half8 b, float4v c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(as_h8(a), b, c, 0, 0, 0);
}

// Token (0..31) of a tile held in slot j (0..7) by lane group g: the C-layout
// of two stacked 16x16 QK blocks, reused as the PV reduction order.
__device__ __forceinline__ int tau(int g, int j) { return 16 * (j >> 2) + 4 * g + (j & 3); }

// One 32-token tile in MFMA operand layout (fp16):
//   k[blk][c] : K[token 16*blk + t][channels 32c + 8g .. +7]
//   v[j]      : V[token tau(g, j)][channels 8m .. 8m+7]
struct Tile {
  u32x4 k[2][4];
  u32x4 v[8];
};

// Per-wave online-softmax state.  Lane (n, g) owns head n; logits are kept
// in the log2 domain (scaled by sm_scale * log2(e)).
//   O[jj][r] : unnormalised output of head n, channel 8*(4g + r) + jj
//   m        : running max, identical in the four lanes of a head
//   l        : this lane's share of the softmax denominator
struct WaveState {
  float4v O[8];
  float m;
  float l;
};

__device__ __forceinline__ void wave_state_init(WaveState& st) {
#pragma unroll
  for (int jj = 0; jj < 8; ++jj) st.O[jj] = float4v{0.f, 0.f, 0.f, 0.f};
  st.m = -INFINITY;
  st.l = 0.f;
}

// Slot validity: s < va, or vb <= s < vc.  Dense uses va = L; the sparse and
// KIVI caches use the StreamingLLM sink / window ranges.
struct SlotRanges {
  int64_t va, vb, vc;
};

__device__ __forceinline__ bool slot_valid(const SlotRanges& R, int64_t s) {
  return s < R.va || (s >= R.vb && s < R.vc);
}

// Consume one tile: QK on MFMA, masking, online softmax, PV on MFMA.
// `slot0` is the cache slot of the tile's token 0, `xlim` the number of
// tokens of the tile that belong to the region (the rest are masked).
__device__ __forceinline__ void tile_step(Tile& T, const half8 (&qB)[4], int64_t slot0,
                                          int xlim, const SlotRanges& R, float scale_log2,
                                          WaveState& st, int lane) {
  const int g = lane >> 4;

  float4v s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    s0 = mfma16x16x32(T.k[0][c], qB[c], s0);
    s1 = mfma16x16x32(T.k[1][c], qB[c], s1);
  }

  float x[8];
  bool all_ok = true;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int tok = tau(g, j);
    const float raw = (j < 4 ? s0[j & 3] : s1[j & 3]) * scale_log2;
    const bool ok = tok < xlim && slot_valid(R, slot0 + tok);
    all_ok = all_ok && ok;
    x[j] = ok ? raw : -INFINITY;
    if (!ok) T.v[j] = u32x4{0u, 0u, 0u, 0u};   // masked rows contribute exact zeros
  }
  (void)all_ok;

  float mt = x[0];
#pragma unroll
  for (int j = 1; j < 8; ++j) mt = fmaxf(mt, x[j]);
  mt = fmaxf(mt, __shfl_xor(mt, 16));
  mt = fmaxf(mt, __shfl_xor(mt, 32));
  const float mnew = fmaxf(st.m, mt);
  const float mu = (mnew == -INFINITY) ? 0.f : mnew;
  const float alpha = __builtin_amdgcn_exp2f(st.m - mu);

  half8 pB;
  float ls = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float p = __builtin_amdgcn_exp2f(x[j] - mu);
    ls += p;
    pB[j] = (_Float16)p;
  }
  st.l = st.l * alpha + ls;
  st.m = mnew;

#pragma unroll
  for (int jj = 0; jj < 8; ++jj) {
    const int w = jj >> 1;
    const uint32_t sel = (jj & 1) ? 0x07060302u : 0x05040100u;
    u32x4 a;
    a[0] = __builtin_amdgcn_perm(T.v[1][w], T.v[0][w], sel);
    a[1] = __builtin_amdgcn_perm(T.v[3][w], T.v[2][w], sel);
    a[2] = __builtin_amdgcn_perm(T.v[5][w], T.v[4][w], sel);
    a[3] = __builtin_amdgcn_perm(T.v[7][w], T.v[6][w], sel);
    st.O[jj] = st.O[jj] * alpha;
    st.O[jj] = mfma16x16x32(a, pB, st.O[jj]);
  }
}

// Load an fp16 tile from a [rows, 128] region (rows of this KV head).  Rows
// past the end are clamped to the last row; tile_step masks them.
__device__ __forceinline__ void load_f16_tile(const _Float16* __restrict__ kb,
                                              const _Float16* __restrict__ vb, int row0,
                                              int rows, int lane, Tile& T) {
  const int t = lane & 15, g = lane >> 4;
#pragma unroll
  for (int blk = 0; blk < 2; ++blk) {
    int r = row0 + 16 * blk + t;
    r = r < rows ? r : rows - 1;
    const u32x4* p = reinterpret_cast<const u32x4*>(kb + (size_t)r * kHeadDim) + g;
#pragma unroll
    for (int c = 0; c < 4; ++c) T.k[blk][c] = p[4 * c];
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    int r = row0 + tau(g, j);
    r = r < rows ? r : rows - 1;
    T.v[j] = *(reinterpret_cast<const u32x4*>(vb + (size_t)r * kHeadDim) + t);
  }
}

// Raw (still packed) KIVI tile: 32 tokens of one quantized region, i.e.
// exactly one quantization group of K.
//   kc[blk][c] : K code bytes of token row (16*blk + t)/4, channels 32c+8g..+7
//   ks/kz[c]   : K scale / zero of channels 32c+8g..+7 (fp16 x 8)
//   vc[j]      : V code bytes (2) of token tau(g, j), channels 8m..8m+7
//   vs/vz[j]   : V scale / zero of that token, channel group m/4 (fp16)
struct RawQTile {
  u32x2 kc[2][4];
  u32x4 ks[4], kz[4];
  uint32_t vc[8], vs[8], vz[8];
};

// Device pointers of one KIVI-quantized region, bound to one KV head.
struct QRegion {
  const uint8_t* kp;     // [ntok/4][128]
  const _Float16* ks;    // [ntok/32][128]
  const _Float16* kz;
  const uint8_t* vp;     // [ntok][32]
  const _Float16* vs;    // [ntok][4]
  const _Float16* vz;
};

__device__ __forceinline__ void load_q_tile(const QRegion& Q, int tq, int lane, RawQTile& X) {
  const int t = lane & 15, g = lane >> 4;
#pragma unroll
  for (int blk = 0; blk < 2; ++blk) {
    const int brow = 8 * tq + 4 * blk + (t >> 2);
    const uint8_t* p = Q.kp + (size_t)brow * kHeadDim + 8 * g;
#pragma unroll
    for (int c = 0; c < 4; ++c) X.kc[blk][c] = *reinterpret_cast<const u32x2*>(p + 32 * c);
  }
  const _Float16* sp = Q.ks + (size_t)tq * kHeadDim + 8 * g;
  const _Float16* zp = Q.kz + (size_t)tq * kHeadDim + 8 * g;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    X.ks[c] = *reinterpret_cast<const u32x4*>(sp + 32 * c);
    X.kz[c] = *reinterpret_cast<const u32x4*>(zp + 32 * c);
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int tok = 32 * tq + tau(g, j);
    X.vc[j] = *reinterpret_cast<const uint16_t*>(Q.vp + (size_t)tok * 32 + 2 * t);
    X.vs[j] = *reinterpret_cast<const uint16_t*>(Q.vs + (size_t)tok * 4 + (t >> 2));
    X.vz[j] = *reinterpret_cast<const uint16_t*>(Q.vz + (size_t)tok * 4 + (t >> 2));
  }
}

// fp16 bit patterns 0x6400 | c encode 1024 + c exactly for c in 0..3, so
// (0x6400|c) - (1024 + z) == c - z exactly for integer |c - z| <= 2048; the
// product with the fp16 scale is then the only rounding (to fp16).
__device__ __forceinline__ void decode_q_tile(const RawQTile& X, int lane, Tile& T) {
  const int t = lane & 15;
  const uint32_t sh = 2u * (uint32_t)(t & 3);
  const _Float16 k1024 = (_Float16)1024.0f;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const half8 s8 = as_h8(X.ks[c]);
    const half8 zz = as_h8(X.kz[c]) + k1024;
#pragma unroll
    for (int blk = 0; blk < 2; ++blk) {
      const uint32_t c0 = (X.kc[blk][c][0] >> sh) & 0x03030303u;
      const uint32_t c1 = (X.kc[blk][c][1] >> sh) & 0x03030303u;
      u32x4 mg;
      mg[0] = __builtin_amdgcn_perm(c0, 0x64646464u, 0x00050004u);
      mg[1] = __builtin_amdgcn_perm(c0, 0x64646464u, 0x00070006u);
      mg[2] = __builtin_amdgcn_perm(c1, 0x64646464u, 0x00050004u);
      mg[3] = __builtin_amdgcn_perm(c1, 0x64646464u, 0x00070006u);
      T.k[blk][c] = as_u4((as_h8(mg) - zz) * s8);
    }
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const uint32_t b = X.vc[j];
    const uint32_t t0 = b | (b << 14);
    u32x4 mg;
    mg[0] = (t0 & 0x00030003u) | 0x64006400u;
    mg[1] = ((t0 >> 4) & 0x00030003u) | 0x64006400u;
    mg[2] = ((t0 >> 8) & 0x00030003u) | 0x64006400u;
    mg[3] = ((t0 >> 12) & 0x00030003u) | 0x64006400u;
    const _Float16 s = __builtin_bit_cast(_Float16, (uint16_t)X.vs[j]);
    const _Float16 zz = __builtin_bit_cast(_Float16, (uint16_t)X.vz[j]) + k1024;
    T.v[j] = as_u4((as_h8(mg) - zz) * s);
  }
}

}  // namespace kvdec
