// KIVI 2-bit quantizers (K per-channel, V per-token, groups of 32) and the
// isolated tile dequantizers, for gfx950, with their C-ABI entry points.
//
// Codes must be bit-exact to the IEEE-float32 closed form
//   s = (mx - mn) / 3;  s = (s == 0) ? 1 : s;  z = floor(-mn / s + 0.5)
//   code = clamp(floor(x / s + 0.5) + z, 0, 3)
// so this file is compiled with -ffp-contract=off and keeps the HIP default
// of correctly rounded fp32 division for the per-group quantities.
//
// The per-element quotient fl32(x / s) takes three fp32 operations
// (Markstein's division): with y = fl32(1 / s) correctly rounded and
// q0 = fl32(x * y), which is within one ulp of x / s, the residual
// r = x - q0 * s is exact in one FMA and fl32(q0 + r * y) is the correctly
// rounded quotient.  The theorem needs y normal and r exact: groups whose
// scale lies outside [2^-40, 2^100] (and groups with infinite inputs, whose
// scale is infinite) take the slow path below instead.  Inside that range
// every residual that matters is a normal number: r is a multiple of
// ulp(q0) * ulp(s) / 2, which stays >= 2^-115 while |x / s| >= 2^-28, and a
// quotient below 2^-28 cannot move floor(q + 0.5).
//
// Slow path: fl32(x / s) as RN32(RN64(x * RN64(1 / s))).  The fp64 product
// is within 2^-52 (relative) of x / s, while a quotient of two 24-bit
// significands that is not exactly a float32 rounding midpoint lies at
// least ~2^-48 (relative) away from one, so rounding it to float32 gives the
// correctly rounded quotient for any finite s.

#include <type_traits>

#include "kvdec_device.h"
#include "kvdec_stream.h"
#include "kvdec.h"

using namespace kvdec;

namespace {

constexpr int kGroup = 32;

// Input formats.  Raw data stays in the loaded dwords (two elements per
// dword for the 16-bit formats) until each element is needed as a float.
template <typename T>
struct Fmt;
// elem() returns an element in a type that converts exactly to float (the
// code computation converts it where it is used, so the fp16 conversions fold
// into mixed-precision FMAs).
template <>
struct Fmt<float> {
  static constexpr int kPerWord = 1;
  __device__ static float elem(uint32_t w, int) { return __builtin_bit_cast(float, w); }
  __device__ static float get(uint32_t w, int i) { return elem(w, i); }
};
template <>
struct Fmt<_Float16> {
  static constexpr int kPerWord = 2;
  __device__ static _Float16 elem(uint32_t w, int i) { return __builtin_bit_cast(half2v, w)[i]; }
  __device__ static float get(uint32_t w, int i) { return (float)elem(w, i); }
};
template <>
struct Fmt<uint16_t> {   // bfloat16
  static constexpr int kPerWord = 2;
  __device__ static float elem(uint32_t w, int i) {
    return __builtin_bit_cast(float, i ? (w & 0xffff0000u) : (w << 16));
  }
  __device__ static float get(uint32_t w, int i) { return elem(w, i); }
};

// Exact min / max of element i over n words (a min or max of fp16 values is
// one of them, so the packed fp16 reduction is exact).
template <typename T, int N, int STRIDE>
__device__ __forceinline__ void minmax(const uint32_t* w, int i, float& mn, float& mx) {
  mn = mx = Fmt<T>::get(w[0], i);
#pragma unroll
  for (int k = 1; k < N; ++k) {
    const float v = Fmt<T>::get(w[k * STRIDE], i);
    mn = fminf(mn, v);
    mx = fmaxf(mx, v);
  }
}
// Both halves of N packed fp16 words at once.
template <int N>
__device__ __forceinline__ void minmax_h2(const uint32_t* w, half2v& mn, half2v& mx) {
  mn = mx = __builtin_bit_cast(half2v, w[0]);
#pragma unroll
  for (int k = 1; k < N; ++k) {
    const half2v v = __builtin_bit_cast(half2v, w[k]);
    mn = __builtin_elementwise_min(mn, v);
    mx = __builtin_elementwise_max(mx, v);
  }
}

// K: one lane owns two adjacent channels of one 32-token group; a wave owns
// a 128-channel slice.  unit = pg * chunks + chunk with pg = pair * groups +
// grp, the group's index over all (b, kv) heads: its input rows start at row
// 32 pg, its packed rows at row 8 pg and its scales / zeros at row pg.
// Raw: one dword per token (16-bit inputs, both channels) or two (fp32).
template <typename T>
struct KRaw {
  static constexpr int kW = 2 / Fmt<T>::kPerWord;
  uint32_t w[kGroup * kW];
};

// Wave-uniform position of a unit (chunks == 1, the usual D <= 128, needs
// no division).
struct KUnit {
  int64_t pg;
  int chunk;
};
__device__ __forceinline__ int64_t uniform64(int64_t v) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)((uint64_t)v >> 32));
  return (int64_t)(((uint64_t)hi << 32) | lo);
}
// Buffer resource over a wave-uniform range.  Base and size pass through
// readfirstlane: otherwise the compiler may keep parts of the resource in
// VGPRs and wrap every buffer access in a loop over distinct values.
__device__ __forceinline__ rsrc_t make_rsrc_uniform(const void* base, uint32_t bytes) {
  const void* b = reinterpret_cast<const void*>(uniform64(reinterpret_cast<int64_t>(base)));
  return make_rsrc(b, __builtin_amdgcn_readfirstlane(bytes));
}
__device__ __forceinline__ KUnit k_unit(int64_t unit, int chunks) {
  if (chunks == 1) return KUnit{unit, 0};
  return KUnit{unit / chunks, (int)(unit % chunks)};
}

template <typename T>
__device__ __forceinline__ void k_load(const T* x, KUnit u, bool live, int D, int lane,
                                       KRaw<T>& r) {
  constexpr int kW = KRaw<T>::kW;
  if (!live) return;
  // the group's 32 rows as one buffer: per-lane offset in a VGPR, per-row
  // offset in an SGPR (no 64-bit address arithmetic per load).  Lanes past
  // D read out of range: zeros, no access, no divergent branch.
  const int ch = u.chunk * 128 + 2 * lane;
  const rsrc_t rs = make_rsrc_uniform(x + (size_t)u.pg * kGroup * D,
                                      (uint32_t)(kGroup * D * sizeof(T)));
  const uint32_t vo = ch < D ? (uint32_t)ch * sizeof(T) : kOOB, row = (uint32_t)D * sizeof(T);
#pragma unroll
  for (int t = 0; t < kGroup; ++t) {
    if (kW == 1) {
      r.w[t] = __builtin_amdgcn_raw_buffer_load_b32(rs, vo, t * row, kStreamAux);
    } else {
      const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(rs, vo, t * row, kStreamAux);
      r.w[2 * t] = v[0];
      r.w[2 * t + 1] = v[1];
    }
  }
}

template <typename T>
__device__ __forceinline__ auto k_elem(const KRaw<T>& r, int t, int c) {
  if (KRaw<T>::kW == 1) return Fmt<T>::elem(r.w[t], c);
  return Fmt<T>::elem(r.w[2 * t + c], 0);
}

template <typename T>
__device__ __forceinline__ void k_quantize(const KRaw<T>& r, KUnit u, int D, int lane,
                                           uint8_t* __restrict__ packed,
                                           _Float16* __restrict__ scale,
                                           _Float16* __restrict__ zero) {
  // lanes past D compute codes of zeros and store out of range (dropped)
  const int ch = u.chunk * 128 + 2 * lane;
  const uint32_t vo = ch < D ? (uint32_t)ch : kOOB;
  float amn, amx, bmn, bmx;
  if (std::is_same<T, _Float16>::value) {
    half2v mn, mx;
    minmax_h2<kGroup>(r.w, mn, mx);
    amn = (float)mn[0];
    bmn = (float)mn[1];
    amx = (float)mx[0];
    bmx = (float)mx[1];
  } else {
    constexpr int kW = KRaw<T>::kW;
    minmax<T, kGroup, kW>(r.w, 0, amn, amx);
    minmax<T, kGroup, kW>(r.w + (kW - 1), kW == 1 ? 1 : 0, bmn, bmx);
  }
  const QParams qa = make_params(amn, amx), qb = make_params(bmn, bmx);
  // byte p of each channel holds the codes of tokens 4p .. 4p + 3, LSB first
  uint32_t rows[kGroup / 4];
  auto codes = [&](auto fast) {
    constexpr bool F = decltype(fast)::value;
#pragma unroll
    for (int p = 0; p < kGroup / 4; ++p) {
      uint32_t w = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int t = 4 * p + j;
        const uint32_t c = put_code(quant_code<F>(k_elem(r, t, 1), qb), 1,
                                    put_code(quant_code<F>(k_elem(r, t, 0), qa), 0, 0u));
        w |= c << (2 * j);
      }
      rows[p] = w;
    }
  };
  // one path for the whole wave (the slow path is exact for every group)
  if (__all(qa.fast && qb.fast))
    codes(std::true_type());
  else
    codes(std::false_type());
  const rsrc_t rp = make_rsrc_uniform(packed + (size_t)u.pg * (kGroup / 4) * D,
                                      (uint32_t)(kGroup / 4 * D));
#pragma unroll
  for (int p = 0; p < kGroup / 4; ++p)
    __builtin_amdgcn_raw_buffer_store_b16((uint16_t)rows[p], rp, vo, p * D, kStreamAux);
  const uint32_t mbytes = (uint32_t)D * 2, mo = vo == kOOB ? kOOB : 2 * vo;
  const half2v sv = {(_Float16)qa.s, (_Float16)qb.s};
  const half2v zv = {(_Float16)qa.z, (_Float16)qb.z};
  __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, sv),
                                        make_rsrc_uniform(scale + (size_t)u.pg * D, mbytes), mo, 0,
                                        kStreamAux);
  __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, zv),
                                        make_rsrc_uniform(zero + (size_t)u.pg * D, mbytes), mo, 0,
                                        kStreamAux);
}

// Grid-stride loop over units, one wave per unit; the next unit's loads are
// issued before the current unit is quantized.
template <typename T>
__global__ __launch_bounds__(256) void quantize_k_kernel(const T* __restrict__ x,
                                                         uint8_t* __restrict__ packed,
                                                         _Float16* __restrict__ scale,
                                                         _Float16* __restrict__ zero,
                                                         int64_t n_units, int D, int chunks) {
  const int lane = threadIdx.x & 63;
  const int64_t stride = (int64_t)gridDim.x * (blockDim.x >> 6);
  // wave-uniform (the buffer resources are built from it)
  int64_t unit = (int64_t)blockIdx.x * (blockDim.x >> 6) +
                 __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (unit >= n_units) return;
  KRaw<T> cur;
  KUnit u = k_unit(unit, chunks);
  k_load(x, u, true, D, lane, cur);
  for (; unit < n_units; unit += stride) {
    KRaw<T> nxt;
    const KUnit un = k_unit(unit + stride, chunks);
    k_load(x, un, unit + stride < n_units, D, lane, nxt);
    k_quantize(cur, u, D, lane, packed, scale, zero);
    cur = nxt;
    u = un;
  }
}

// V: one thread owns one (token, 32-channel group); unit = (pair*N + t)*(D/32)
// + grp and the group's 32 inputs start at x + unit*32.
template <typename T>
struct VRaw {
  static constexpr int kW = kGroup / Fmt<T>::kPerWord;
  uint32_t w[kW];
};

template <typename T>
__device__ __forceinline__ void v_load(const T* x, int64_t u, int64_t n_units, VRaw<T>& r) {
  if (u >= n_units) return;
  const u32x4* p = reinterpret_cast<const u32x4*>(x + (size_t)u * kGroup);
#pragma unroll
  for (int i = 0; i < VRaw<T>::kW / 4; ++i) {
    const u32x4 v = p[i];
#pragma unroll
    for (int j = 0; j < 4; ++j) r.w[4 * i + j] = v[j];
  }
}

template <typename T>
__device__ __forceinline__ auto v_elem(const VRaw<T>& r, int c) {
  constexpr int k = Fmt<T>::kPerWord;
  return Fmt<T>::elem(r.w[c / k], c % k);
}

template <typename T>
__device__ __forceinline__ void v_quantize(const VRaw<T>& r, int64_t u, uint8_t* __restrict__ packed,
                                           _Float16* __restrict__ scale,
                                           _Float16* __restrict__ zero) {
  float mn, mx;
  if (std::is_same<T, _Float16>::value) {
    half2v hn, hx;
    minmax_h2<VRaw<T>::kW>(r.w, hn, hx);
    mn = fminf((float)hn[0], (float)hn[1]);
    mx = fmaxf((float)hx[0], (float)hx[1]);
  } else {
    mn = mx = (float)v_elem(r, 0);
#pragma unroll
    for (int c = 1; c < kGroup; ++c) {
      mn = fminf(mn, (float)v_elem(r, c));
      mx = fmaxf(mx, (float)v_elem(r, c));
    }
  }
  const QParams q = make_params(mn, mx);
  // byte b of the 8 holds the codes of channels 4b .. 4b + 3, LSB first
  u32x2 out;
  auto codes = [&](auto fast) {
    constexpr bool F = decltype(fast)::value;
#pragma unroll
    for (int w = 0; w < 2; ++w) {
      uint32_t word = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        uint32_t t = 0;
#pragma unroll
        for (int b = 0; b < 4; ++b) t = put_code(quant_code<F>(v_elem(r, 16 * w + 4 * b + j), q), b, t);
        word |= t << (2 * j);
      }
      out[w] = word;
    }
  };
  if (__all(q.fast))
    codes(std::true_type());
  else
    codes(std::false_type());
  // streaming (non-temporal) stores: outputs are not read again here
  __builtin_nontemporal_store(out, reinterpret_cast<u32x2*>(packed) + u);
  __builtin_nontemporal_store((_Float16)q.s, scale + u);
  __builtin_nontemporal_store((_Float16)q.z, zero + u);
}

template <typename T>
__global__ __launch_bounds__(256) void quantize_v_kernel(const T* __restrict__ x,
                                                         uint8_t* __restrict__ packed,
                                                         _Float16* __restrict__ scale,
                                                         _Float16* __restrict__ zero,
                                                         int64_t n_units) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  int64_t u = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (u >= n_units) return;
  VRaw<T> cur;
  v_load(x, u, n_units, cur);
  for (; u < n_units; u += stride) {
    VRaw<T> nxt;
    v_load(x, u + stride, n_units, nxt);
    v_quantize(cur, u, packed, scale, zero);
    cur = nxt;
  }
}

// Any code width and group size (quant_kernel.py:44-126 and :129-214 with
// BITS and GROUP_SIZE as parameters): QMAX = 2^bits - 1, 8 / bits codes per
// byte at bits j * bits, LSB first.  One thread per (group, channel) of K or
// (token, channel group) of V, reading its inputs twice (min / max, then the
// codes); the 2-bit, 32-group kernels above are the fast path.  The
// quotient is the HIP default fp32 division, correctly rounded like the
// reference's IEEE division.
template <typename T>
__device__ __forceinline__ float gen_elem(const T* x, size_t i) {
  if constexpr (std::is_same<T, uint16_t>::value) return __builtin_bit_cast(float, (uint32_t)x[i] << 16);
  else return (float)x[i];
}
__device__ __forceinline__ void gen_params(float mn, float mx, float qmax, float& s, float& z) {
#pragma clang fp contract(off)
  s = (mx - mn) / qmax;
  s = (s == 0.0f) ? 1.0f : s;
  z = floorf(-mn / s + 0.5f);
}
__device__ __forceinline__ uint32_t gen_code(float x, float s, float z, float qmax) {
#pragma clang fp contract(off)
  const float c = floorf(x / s + 0.5f) + z;
  return (uint32_t)fminf(fmaxf(c, 0.0f), qmax);
}

template <typename T>
__global__ __launch_bounds__(256) void quantize_k_generic_kernel(const T* __restrict__ x,
                                                                 uint8_t* __restrict__ packed,
                                                                 _Float16* __restrict__ scale,
                                                                 _Float16* __restrict__ zero,
                                                                 int64_t n_units, int D, int group,
                                                                 int bits) {
  const int pf = 8 / bits;
  const float qmax = (float)((1 << bits) - 1);
  for (int64_t u = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; u < n_units;
       u += (int64_t)gridDim.x * blockDim.x) {
    // u = pg * D + ch; the group's rows start at row pg * group (every
    // sequence is a whole number of groups), its packed rows at pg * group / pf
    const int64_t pg = u / D;
    const int ch = (int)(u - pg * D);
    const T* xg = x + (size_t)pg * group * D + ch;
    float mn = gen_elem(xg, 0), mx = mn;
    for (int t = 1; t < group; ++t) {
      const float v = gen_elem(xg, (size_t)t * D);
      mn = fminf(mn, v);
      mx = fmaxf(mx, v);
    }
    float s, z;
    gen_params(mn, mx, qmax, s, z);
    uint8_t* pk = packed + (size_t)pg * (group / pf) * D + ch;
    for (int b = 0; b < group / pf; ++b) {
      uint32_t byte = 0;
      for (int j = 0; j < pf; ++j)
        byte |= gen_code(gen_elem(xg, (size_t)(b * pf + j) * D), s, z, qmax) << (j * bits);
      pk[(size_t)b * D] = (uint8_t)byte;
    }
    scale[u] = (_Float16)s;
    zero[u] = (_Float16)z;
  }
}

template <typename T>
__global__ __launch_bounds__(256) void quantize_v_generic_kernel(const T* __restrict__ x,
                                                                 uint8_t* __restrict__ packed,
                                                                 _Float16* __restrict__ scale,
                                                                 _Float16* __restrict__ zero,
                                                                 int64_t n_units, int group, int bits) {
  const int pf = 8 / bits;
  const float qmax = (float)((1 << bits) - 1);
  for (int64_t u = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; u < n_units;
       u += (int64_t)gridDim.x * blockDim.x) {
    // u = row * (D / group) + channel group: its inputs are x[u * group ..],
    // its packed bytes packed[u * group / pf ..] (the row's groups in order)
    const T* xg = x + (size_t)u * group;
    float mn = gen_elem(xg, 0), mx = mn;
    for (int c = 1; c < group; ++c) {
      const float v = gen_elem(xg, c);
      mn = fminf(mn, v);
      mx = fmaxf(mx, v);
    }
    float s, z;
    gen_params(mn, mx, qmax, s, z);
    uint8_t* pk = packed + (size_t)u * (group / pf);
    for (int b = 0; b < group / pf; ++b) {
      uint32_t byte = 0;
      for (int j = 0; j < pf; ++j) byte |= gen_code(gen_elem(xg, b * pf + j), s, z, qmax) << (j * bits);
      pk[b] = (uint8_t)byte;
    }
    scale[u] = (_Float16)s;
    zero[u] = (_Float16)z;
  }
}

__global__ __launch_bounds__(256) void dequant_k_tile_kernel(
    const uint8_t* __restrict__ packed, const _Float16* __restrict__ scale,
    const _Float16* __restrict__ zero, float* __restrict__ out, int64_t tok_start,
    int64_t num_packed, int64_t num_groups, int64_t pairs, int D, int block_n) {
  const int64_t total = pairs * block_n * D;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int d = (int)(e % D);
    const int t = (int)((e / D) % block_n);
    const int64_t pair = e / ((int64_t)D * block_n);
    int64_t byte_idx = tok_start / 4 + t / 4;   // C division, as the reference
    byte_idx = byte_idx < num_packed - 1 ? byte_idx : num_packed - 1;
    byte_idx = byte_idx > 0 ? byte_idx : 0;
    const uint32_t byte = packed[((size_t)pair * num_packed + byte_idx) * D + d];
    const float code = (float)((byte >> (2 * (t % 4))) & 3u);
    int64_t grp = byte_idx / (kGroup / 4);
    grp = grp < num_groups - 1 ? grp : num_groups - 1;
    const size_t mo = ((size_t)pair * num_groups + grp) * D + d;
    out[e] = (float)scale[mo] * (code - (float)zero[mo]);
  }
}

__global__ __launch_bounds__(256) void dequant_v_tile_kernel(
    const uint8_t* __restrict__ packed, const _Float16* __restrict__ scale,
    const _Float16* __restrict__ zero, float* __restrict__ out, int64_t tok_start,
    int64_t seq_len, int64_t pairs, int D, int block_n) {
  const int64_t total = pairs * block_n * D;
  const int dp = D / 4, ng = D / kGroup;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int d = (int)(e % D);
    const int t = (int)((e / D) % block_n);
    const int64_t pair = e / ((int64_t)D * block_n);
    int64_t tok = tok_start + t;
    tok = tok < seq_len - 1 ? tok : seq_len - 1;
    tok = tok > 0 ? tok : 0;
    const uint32_t byte = packed[((size_t)pair * seq_len + tok) * dp + d / 4];
    const float code = (float)((byte >> (2 * (d % 4))) & 3u);
    const size_t mo = ((size_t)pair * seq_len + tok) * ng + d / kGroup;
    out[e] = (float)scale[mo] * (code - (float)zero[mo]);
  }
}

__global__ __launch_bounds__(256) void stream_append_kernel(StreamArgs a) {
  const int64_t pair = blockIdx.x;
  const int D = a.D;
  int row = a.row, blk = a.blk, slot = a.slot;
  const int64_t b = a.appended ? pair / a.KVH : 0;
  RingStep rs{};
  int n = 0;
  bool act = false;
  if (a.appended) {
    // this sequence's step, from its append count (read by every workgroup
    // of the sequence before any of them advances it, below)
    n = max(a.appended[b], 0);
    act = !a.active || a.active[b] != 0;
    rs = ring_step(n, act, a.residual, a.cap, a.nwg);
    row = rs.row;
    blk = a.nwg > 0 ? rs.blk : -1;
    slot = rs.slot;
  }
  if (a.k_new && row >= 0)
    for (int i = threadIdx.x; i < D; i += blockDim.x) {
      a.k_ring[((size_t)pair * a.cap + row) * D + i] = a.k_new[(size_t)pair * D + i];
      a.v_ring[((size_t)pair * a.cap + row) * D + i] = a.v_new[(size_t)pair * D + i];
    }
  if (blk >= 0) evict_block(a, pair, blk, slot, threadIdx.x, blockDim.x);
  if (a.appended) {
    // the last of the sequence's KVH workgroups to arrive records the step
    // and advances the count.  Every workgroup's threads have consumed their
    // load of the count before its barrier, so no fence is needed; the
    // writes reach the next launch at the kernel boundary.
    __syncthreads();
    if (threadIdx.x == 0 && atomicAdd(a.arrive + b, 1) == a.KVH - 1) {
      a.arrive[b] = 0;
      a.appended[b] = n + (act ? 1 : 0);
      a.plan[3 * b] = rs.row;
      a.plan[3 * b + 1] = rs.blk;
      a.plan[3 * b + 2] = rs.blk >= 0 ? rs.slot : -1;
      a.ring[2 * b] = rs.start;
      a.ring[2 * b + 1] = rs.count;
    }
  }
}

// ---------------------------------------------------------------------------
// The whole KIVI cache from a compacted [B, KVH, sink + window, D] cache in
// one launch (the reference's build_quantized_kv_cache, quant_kernel.py:584-
// 622): residual rows copied (input dtype, or fp16 for the decode), the sink
// group (sink real tokens, the rest token 0 again) and the window-old groups
// quantized.  Grid: x = (b, kv) head, y = slices of that head's work.
// ---------------------------------------------------------------------------
struct BuildArgs {
  const void* kc;
  const void* vc;
  int n, D, sink, res_rows, win_tok;
  void* kres;
  void* vres;
  uint8_t* kp[2];   // [0] sink, [1] window-old
  _Float16* ks[2];
  _Float16* kz[2];
  uint8_t* vp[2];
  _Float16* vs[2];
  _Float16* vz[2];
};

template <typename T>
__device__ __forceinline__ float elem(const void* p, size_t i) {
  if constexpr (std::is_same<T, uint16_t>::value)
    return __builtin_bit_cast(float, (uint32_t)static_cast<const uint16_t*>(p)[i] << 16);
  else
    return (float)static_cast<const T*>(p)[i];
}

template <typename T, typename RT>
__global__ __launch_bounds__(256) void build_kernel(BuildArgs a) {
  const int64_t pair = blockIdx.x;
  const int D = a.D, ng = D / kGroup, nwg = a.win_tok / kGroup;
  const int first = blockIdx.y * blockDim.x + threadIdx.x, stride = gridDim.y * blockDim.x;
  const size_t in0 = (size_t)pair * a.n * D;
  // residual: the last res_rows slots (same element type, or fp16)
  const size_t res0 = (size_t)(a.n - a.res_rows) * D;
  for (int i = first; i < a.res_rows * D; i += stride) {
    const size_t o = (size_t)pair * a.res_rows * D + i;
    if constexpr (std::is_same<T, RT>::value) {
      static_cast<T*>(a.kres)[o] = static_cast<const T*>(a.kc)[in0 + res0 + i];
      static_cast<T*>(a.vres)[o] = static_cast<const T*>(a.vc)[in0 + res0 + i];
    } else {
      static_cast<RT*>(a.kres)[o] = (RT)elem<T>(a.kc, in0 + res0 + i);
      static_cast<RT*>(a.vres)[o] = (RT)elem<T>(a.vc, in0 + res0 + i);
    }
  }
  // K groups: region 0 = the sink group (slot t, or slot 0 past the sink
  // tokens), region 1 = window-old group g (slots sink + 32 g + t)
  for (int task = first; task < (1 + nwg) * D; task += stride) {
    const int grp = task / D, d = task % D;   // grp 0: sink
    const int r = grp == 0 ? 0 : 1, g = grp - r;
    float x[kGroup];
#pragma unroll
    for (int t = 0; t < kGroup; ++t) {
      const int slot = r == 0 ? (t < a.sink ? t : 0) : a.sink + kGroup * g + t;
      x[t] = elem<T>(a.kc, in0 + (size_t)slot * D + d);
    }
    QParams q;
    const u32x2 c = quant_group(x, q);
    const size_t gi = (size_t)pair * (r == 0 ? 1 : nwg) + g;
#pragma unroll
    for (int p = 0; p < kGroup / 4; ++p)
      a.kp[r][(gi * (kGroup / 4) + p) * D + d] = (uint8_t)(c[p >> 2] >> (8 * (p & 3)));
    a.ks[r][gi * D + d] = (_Float16)q.s;
    a.kz[r][gi * D + d] = (_Float16)q.z;
  }
  // V: one task per (token, 32-channel group); tokens 0..31 of the sink
  // group, then the window-old tokens
  for (int task = first; task < (kGroup + a.win_tok) * ng; task += stride) {
    const int tk = task / ng, cg = task % ng;
    const int r = tk < kGroup ? 0 : 1, t = tk - (r ? kGroup : 0);
    const int slot = r == 0 ? (t < a.sink ? t : 0) : a.sink + t;
    float x[kGroup];
#pragma unroll
    for (int i = 0; i < kGroup; ++i) x[i] = elem<T>(a.vc, in0 + (size_t)slot * D + cg * kGroup + i);
    QParams q;
    const u32x2 c = quant_group(x, q);
    const size_t tok = (size_t)pair * (r == 0 ? kGroup : a.win_tok) + t;
    *reinterpret_cast<u32x2*>(a.vp[r] + tok * (D / 4) + cg * (kGroup / 4)) = c;
    a.vs[r][tok * ng + cg] = (_Float16)q.s;
    a.vz[r][tok * ng + cg] = (_Float16)q.z;
  }
}

int launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? KVDEC_OK : (int)e;
}

// One unit per thread (V) or wave (K) while the grid allows: the streaming
// quantizers are fastest with the whole problem in flight as separate
// workgroups rather than fewer, looping ones.
unsigned grid_for(int64_t threads_needed, int block) {
  int64_t g = (threads_needed + block - 1) / block;
  const int64_t cap = (int64_t)1 << 30;   // workgroups; grid-stride beyond
  if (g > cap) g = cap;
  if (g < 1) g = 1;
  return (unsigned)g;
}

int check_quant_args(const void* x, int in_dtype, const void* p, const void* s, const void* z,
                     int64_t B, int32_t KVH, int64_t N, int32_t D, int32_t group, int32_t bits) {
  if (!x || !p || !s || !z) return KVDEC_E_NULL;
  if (bits < 1 || bits > 8) return KVDEC_E_BITS;
  if (in_dtype != KVDEC_F32 && in_dtype != KVDEC_F16 && in_dtype != KVDEC_BF16) return KVDEC_E_DTYPE;
  if (B < 1 || KVH < 1 || N < 1 || D < 1) return KVDEC_E_SHAPE;
  if (group < 1) return KVDEC_E_SHAPE;
  return KVDEC_OK;
}

template <typename T>
void launch_quant_generic_t(bool k, const void* x, uint8_t* p, _Float16* s, _Float16* z, int64_t n_units,
                            int D, int group, int bits, hipStream_t st) {
  const unsigned grid = grid_for(n_units, 256);
  if (k)
    hipLaunchKernelGGL(quantize_k_generic_kernel<T>, dim3(grid), dim3(256), 0, st, static_cast<const T*>(x), p,
                       s, z, n_units, D, group, bits);
  else
    hipLaunchKernelGGL(quantize_v_generic_kernel<T>, dim3(grid), dim3(256), 0, st, static_cast<const T*>(x), p,
                       s, z, n_units, group, bits);
}

int launch_quant_generic(bool k, const void* x, int in_dtype, void* packed_u8, void* scale_f16,
                         void* zero_f16, int64_t n_units, int D, int group, int bits, void* stream) {
  auto* p = static_cast<uint8_t*>(packed_u8);
  auto* s = static_cast<_Float16*>(scale_f16);
  auto* z = static_cast<_Float16*>(zero_f16);
  const hipStream_t st = static_cast<hipStream_t>(stream);
  if (in_dtype == KVDEC_F32)
    launch_quant_generic_t<float>(k, x, p, s, z, n_units, D, group, bits, st);
  else if (in_dtype == KVDEC_F16)
    launch_quant_generic_t<_Float16>(k, x, p, s, z, n_units, D, group, bits, st);
  else
    launch_quant_generic_t<uint16_t>(k, x, p, s, z, n_units, D, group, bits, st);
  return launch_status();
}

}  // namespace

extern "C" {

int kvdec_quantize_k(const void* x, int in_dtype, void* packed_u8, void* scale_f16, void* zero_f16,
                     int64_t B, int32_t KVH, int64_t N, int32_t D, int32_t group, int32_t bits,
                     void* stream) {
  int rc = check_quant_args(x, in_dtype, packed_u8, scale_f16, zero_f16, B, KVH, N, D, group, bits);
  if (rc) return rc;
  if (N % group != 0) return KVDEC_E_GROUP;
  if (bits != 2 || group != kGroup) {
    // any width: whole bytes per group
    if (group % (8 / bits) != 0) return KVDEC_E_GROUP;
    const int64_t n_units = B * KVH * (N / group) * D;
    return launch_quant_generic(true, x, in_dtype, packed_u8, scale_f16, zero_f16, n_units, D, group,
                                bits, stream);
  }
  if (D % 2 != 0) return KVDEC_E_SHAPE;
  if ((int64_t)D * kGroup * 4 >= ((int64_t)1 << 31)) return KVDEC_E_SHAPE;   // 32-bit buffer offsets
  const int64_t pairs = B * KVH;
  const int64_t groups = N / kGroup;
  const int chunks = (D + 127) / 128;
  const int64_t n_units = pairs * groups * chunks;
  const unsigned grid = grid_for(n_units * 64, 256);
  hipStream_t st = static_cast<hipStream_t>(stream);
  auto* p = static_cast<uint8_t*>(packed_u8);
  auto* s = static_cast<_Float16*>(scale_f16);
  auto* z = static_cast<_Float16*>(zero_f16);
  if (in_dtype == KVDEC_F32)
    hipLaunchKernelGGL(quantize_k_kernel<float>, dim3(grid), dim3(256), 0, st,
                       static_cast<const float*>(x), p, s, z, n_units, D, chunks);
  else if (in_dtype == KVDEC_F16)
    hipLaunchKernelGGL(quantize_k_kernel<_Float16>, dim3(grid), dim3(256), 0, st,
                       static_cast<const _Float16*>(x), p, s, z, n_units, D, chunks);
  else
    hipLaunchKernelGGL(quantize_k_kernel<uint16_t>, dim3(grid), dim3(256), 0, st,
                       static_cast<const uint16_t*>(x), p, s, z, n_units, D, chunks);
  return launch_status();
}

int kvdec_quantize_v(const void* x, int in_dtype, void* packed_u8, void* scale_f16, void* zero_f16,
                     int64_t B, int32_t KVH, int64_t N, int32_t D, int32_t group, int32_t bits,
                     void* stream) {
  int rc = check_quant_args(x, in_dtype, packed_u8, scale_f16, zero_f16, B, KVH, N, D, group, bits);
  if (rc) return rc;
  if (D % group != 0) return KVDEC_E_DGROUP;
  if (bits != 2 || group != kGroup) {
    if (group % (8 / bits) != 0) return KVDEC_E_DGROUP;
    const int64_t n_units = B * KVH * N * (D / group);
    return launch_quant_generic(false, x, in_dtype, packed_u8, scale_f16, zero_f16, n_units, D, group,
                                bits, stream);
  }
  const int64_t n_units = B * KVH * N * (D / kGroup);
  const unsigned grid = grid_for(n_units, 256);
  hipStream_t st = static_cast<hipStream_t>(stream);
  auto* p = static_cast<uint8_t*>(packed_u8);
  auto* s = static_cast<_Float16*>(scale_f16);
  auto* z = static_cast<_Float16*>(zero_f16);
  if (in_dtype == KVDEC_F32)
    hipLaunchKernelGGL(quantize_v_kernel<float>, dim3(grid), dim3(256), 0, st,
                       static_cast<const float*>(x), p, s, z, n_units);
  else if (in_dtype == KVDEC_F16)
    hipLaunchKernelGGL(quantize_v_kernel<_Float16>, dim3(grid), dim3(256), 0, st,
                       static_cast<const _Float16*>(x), p, s, z, n_units);
  else
    hipLaunchKernelGGL(quantize_v_kernel<uint16_t>, dim3(grid), dim3(256), 0, st,
                       static_cast<const uint16_t*>(x), p, s, z, n_units);
  return launch_status();
}

int kvdec_kivi_stream_append(const void* k_new, const void* v_new, void* k_ring, void* v_ring,
                             void* const* win, int64_t B, int32_t KVH, int32_t D, int32_t ring_cap,
                             int32_t row, int32_t evict_block, int32_t evict_slot, int32_t n_groups,
                             int32_t group, int32_t bits, void* stream) {
  if (!k_ring || !v_ring || (!k_new) != (!v_new)) return KVDEC_E_NULL;
  if (bits != 2) return KVDEC_E_BITS;
  if (group != kGroup) return KVDEC_E_UNSUPPORTED;
  if (B < 1 || KVH < 1 || D < 1 || B * (int64_t)KVH > 0x7fffffffLL) return KVDEC_E_SHAPE;
  if (D % kGroup != 0) return KVDEC_E_DGROUP;
  if (ring_cap < 2 * kGroup || ring_cap % kGroup != 0) return KVDEC_E_WINDOW;
  if (row < 0 || row >= ring_cap || n_groups < 0) return KVDEC_E_SHAPE;
  if (evict_block >= 0) {
    if (evict_block >= ring_cap / kGroup || row / kGroup == evict_block) return KVDEC_E_SHAPE;
    if (n_groups > 0) {
      if (!win) return KVDEC_E_NULL;
      for (int i = 0; i < 6; ++i)
        if (!win[i]) return KVDEC_E_NULL;
      if (evict_slot < 0 || evict_slot >= n_groups) return KVDEC_E_SHAPE;
    }
  }
  StreamArgs a{};
  a.k_new = static_cast<const _Float16*>(k_new);
  a.v_new = static_cast<const _Float16*>(v_new);
  a.k_ring = static_cast<_Float16*>(k_ring);
  a.v_ring = static_cast<_Float16*>(v_ring);
  a.D = D;
  a.cap = ring_cap;
  a.KVH = KVH;
  a.row = row;
  // a window == residual cache has no window-old groups: the block is dropped
  a.blk = (evict_block >= 0 && n_groups > 0) ? evict_block : -1;
  if (!k_new && a.blk < 0) return KVDEC_OK;   // nothing to do
  a.slot = evict_slot;
  a.nwg = n_groups;
  if (a.blk >= 0) {
    a.kp = static_cast<uint8_t*>(win[0]);
    a.ks = static_cast<_Float16*>(win[1]);
    a.kz = static_cast<_Float16*>(win[2]);
    a.vp = static_cast<uint8_t*>(win[3]);
    a.vs = static_cast<_Float16*>(win[4]);
    a.vz = static_cast<_Float16*>(win[5]);
  }
  hipLaunchKernelGGL(stream_append_kernel, dim3((unsigned)(B * KVH)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), a);
  return launch_status();
}

int kvdec_kivi_stream_step(const void* k_new, const void* v_new, void* k_ring, void* v_ring,
                           void* const* win, int32_t* appended, const int32_t* active,
                           int32_t* arrive, int32_t* plan, int32_t* ring, int64_t B, int32_t KVH,
                           int32_t D, int32_t residual, int32_t ring_cap, int32_t n_groups,
                           int32_t group, int32_t bits, void* stream) {
  if (!k_ring || !v_ring || !appended || !arrive || !plan || !ring || (!k_new) != (!v_new))
    return KVDEC_E_NULL;
  if (bits != 2) return KVDEC_E_BITS;
  if (group != kGroup) return KVDEC_E_UNSUPPORTED;
  if (B < 1 || KVH < 1 || D < 1 || B * (int64_t)KVH > 0x7fffffffLL || n_groups < 0)
    return KVDEC_E_SHAPE;
  if (D % kGroup != 0) return KVDEC_E_DGROUP;
  if (residual < kGroup || residual % kGroup != 0 || ring_cap != residual + kGroup)
    return KVDEC_E_WINDOW;
  if (n_groups > 0) {
    if (!win) return KVDEC_E_NULL;
    for (int i = 0; i < 6; ++i)
      if (!win[i]) return KVDEC_E_NULL;
  }
  StreamArgs a{};
  a.k_new = static_cast<const _Float16*>(k_new);
  a.v_new = static_cast<const _Float16*>(v_new);
  a.k_ring = static_cast<_Float16*>(k_ring);
  a.v_ring = static_cast<_Float16*>(v_ring);
  a.appended = appended;
  a.active = active;
  a.arrive = arrive;
  a.plan = plan;
  a.ring = ring;
  a.D = D;
  a.cap = ring_cap;
  a.nwg = n_groups;
  a.KVH = KVH;
  a.residual = residual;
  if (n_groups > 0) {
    a.kp = static_cast<uint8_t*>(win[0]);
    a.ks = static_cast<_Float16*>(win[1]);
    a.kz = static_cast<_Float16*>(win[2]);
    a.vp = static_cast<uint8_t*>(win[3]);
    a.vs = static_cast<_Float16*>(win[4]);
    a.vz = static_cast<_Float16*>(win[5]);
  }
  hipLaunchKernelGGL(stream_append_kernel, dim3((unsigned)(B * KVH)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), a);
  return launch_status();
}

int kvdec_build_kivi_cache(const void* k_compacted, const void* v_compacted, int in_dtype,
                           int residual_dtype, int64_t B, int32_t KVH, int32_t n_slots, int32_t D, int32_t sink,
                           int32_t residual, int32_t group, int32_t bits, void* const* out,
                           void* stream) {
  if (!k_compacted || !v_compacted || !out) return KVDEC_E_NULL;
  if (bits != 2) return KVDEC_E_BITS;
  if (group != kGroup) return KVDEC_E_UNSUPPORTED;
  if (in_dtype != KVDEC_F32 && in_dtype != KVDEC_F16 && in_dtype != KVDEC_BF16) return KVDEC_E_DTYPE;
  if (residual_dtype != in_dtype && residual_dtype != KVDEC_F16) return KVDEC_E_DTYPE;
  if (B < 1 || KVH < 1 || D < 1 || B * (int64_t)KVH > 0x7fffffffLL) return KVDEC_E_SHAPE;
  if (D % kGroup != 0) return KVDEC_E_DGROUP;
  if (sink < 1 || sink > kGroup || residual < 1 || n_slots <= sink) return KVDEC_E_WINDOW;
  if ((int64_t)n_slots * D > 0x7fffffffLL) return KVDEC_E_SHAPE;
  const int window = n_slots - sink;
  const int res_rows = window < residual ? window : residual;
  const int win_tok = window - res_rows;
  if (win_tok % kGroup != 0) return KVDEC_E_GROUP;
  for (int i = 0; i < 8; ++i)
    if (!out[i]) return KVDEC_E_NULL;
  if (win_tok > 0)
    for (int i = 8; i < 14; ++i)
      if (!out[i]) return KVDEC_E_NULL;
  BuildArgs a{};
  a.kc = k_compacted;
  a.vc = v_compacted;
  a.n = n_slots;
  a.D = D;
  a.sink = sink;
  a.res_rows = res_rows;
  a.win_tok = win_tok;
  a.kres = out[0];
  a.vres = out[1];
  for (int r = 0; r < 2; ++r) {
    if (r == 1 && win_tok == 0) break;
    a.kp[r] = static_cast<uint8_t*>(out[2 + 6 * r]);
    a.ks[r] = static_cast<_Float16*>(out[3 + 6 * r]);
    a.kz[r] = static_cast<_Float16*>(out[4 + 6 * r]);
    a.vp[r] = static_cast<uint8_t*>(out[5 + 6 * r]);
    a.vs[r] = static_cast<_Float16*>(out[6 + 6 * r]);
    a.vz[r] = static_cast<_Float16*>(out[7 + 6 * r]);
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  // about 1024 work items per workgroup, at most 64 workgroups per head
  const int64_t items = std::max<int64_t>((int64_t)res_rows * D, (int64_t)(kGroup + win_tok) * (D / kGroup));
  const unsigned split = (unsigned)std::min<int64_t>(64, std::max<int64_t>(1, (items + 1023) / 1024));
  const dim3 grid((unsigned)(B * KVH), split);
  const bool same = residual_dtype == in_dtype;
  void (*kern)(BuildArgs) = build_kernel<_Float16, _Float16>;
  if (in_dtype == KVDEC_F32)
    kern = same ? build_kernel<float, float> : build_kernel<float, _Float16>;
  else if (in_dtype == KVDEC_BF16)
    kern = same ? build_kernel<uint16_t, uint16_t> : build_kernel<uint16_t, _Float16>;
  hipLaunchKernelGGL(kern, grid, dim3(256), 0, st, a);
  return launch_status();
}

int kvdec_dequant_k_tile(const void* packed, const void* scale, const void* zero, void* out_f32,
                         int64_t tok_start, int64_t num_packed, int64_t num_groups, int32_t B,
                         int32_t KVH, int32_t D, int32_t block_n, void* stream) {
  if (!packed || !scale || !zero || !out_f32) return KVDEC_E_NULL;
  if (B < 1 || KVH < 1 || D < 1 || block_n < 1 || num_packed < 1 || num_groups < 1)
    return KVDEC_E_SHAPE;
  const int64_t pairs = (int64_t)B * KVH;
  hipLaunchKernelGGL(dequant_k_tile_kernel, dim3(grid_for(pairs * block_n * D, 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint8_t*>(packed),
                     static_cast<const _Float16*>(scale), static_cast<const _Float16*>(zero),
                     static_cast<float*>(out_f32), tok_start, num_packed, num_groups, pairs, D,
                     block_n);
  return launch_status();
}

int kvdec_dequant_v_tile(const void* packed, const void* scale, const void* zero, void* out_f32,
                         int64_t tok_start, int64_t seq_len, int32_t B, int32_t KVH, int32_t D,
                         int32_t block_n, void* stream) {
  if (!packed || !scale || !zero || !out_f32) return KVDEC_E_NULL;
  if (B < 1 || KVH < 1 || D < 1 || block_n < 1 || seq_len < 1) return KVDEC_E_SHAPE;
  if (D % kGroup != 0) return KVDEC_E_DGROUP;
  const int64_t pairs = (int64_t)B * KVH;
  hipLaunchKernelGGL(dequant_v_tile_kernel, dim3(grid_for(pairs * block_n * D, 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint8_t*>(packed),
                     static_cast<const _Float16*>(scale), static_cast<const _Float16*>(zero),
                     static_cast<float*>(out_f32), tok_start, seq_len, pairs, D, block_n);
  return launch_status();
}

}  // extern "C"
