// KIVI 2-bit quantizers (K per-channel, V per-token, groups of 32) and the
// isolated tile dequantizers, for gfx950, with their C-ABI entry points.
//
// Codes must be bit-exact to the IEEE-float32 closed form
//   s = (mx - mn) / 3;  s = (s == 0) ? 1 : s;  z = floor(-mn / s + 0.5)
//   code = clamp(floor(x / s + 0.5) + z, 0, 3)
// so this file is compiled with -ffp-contract=off and keeps the HIP default
// of correctly rounded fp32 division.  The per-element quotient fl32(x / s)
// is computed as RN32(RN64(x * RN64(1 / s))): the fp64 product is within
// 2^-52 (relative) of x / s, while a quotient of two 24-bit significands
// that is not exactly a float32 rounding midpoint lies at least ~2^-48
// (relative) away from one, so rounding the fp64 product to float32 gives
// exactly the correctly rounded float32 quotient, for a multiply instead of
// a full division per element.

#include "kvdec_device.h"
#include "kvdec.h"

using namespace kvdec;

namespace {

constexpr int kGroup = 32;

// Two adjacent elements (one 4- or 8-byte load).
__device__ __forceinline__ void load2(const float* p, float& a, float& b) {
  const float2 v = *reinterpret_cast<const float2*>(p);
  a = v.x;
  b = v.y;
}
__device__ __forceinline__ void load2(const _Float16* p, float& a, float& b) {
  const half2v v = *reinterpret_cast<const half2v*>(p);
  a = (float)v[0];
  b = (float)v[1];
}
__device__ __forceinline__ void load2(const uint16_t* p, float& a, float& b) {
  const uint32_t v = *reinterpret_cast<const uint32_t*>(p);
  a = __builtin_bit_cast(float, v << 16);
  b = __builtin_bit_cast(float, v & 0xffff0000u);
}

// 32 contiguous elements (16-byte loads; the group start is 64-byte aligned
// for 16-bit inputs and 128-byte aligned for fp32).
__device__ __forceinline__ void load32(const float* p, float (&a)[32]) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float4 v = reinterpret_cast<const float4*>(p)[i];
    a[4 * i] = v.x;
    a[4 * i + 1] = v.y;
    a[4 * i + 2] = v.z;
    a[4 * i + 3] = v.w;
  }
}
__device__ __forceinline__ void load32(const _Float16* p, float (&a)[32]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const half8 v = as_h8(reinterpret_cast<const u32x4*>(p)[i]);
#pragma unroll
    for (int j = 0; j < 8; ++j) a[8 * i + j] = (float)v[j];
  }
}
__device__ __forceinline__ void load32(const uint16_t* p, float (&a)[32]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const u32x4 v = reinterpret_cast<const u32x4*>(p)[i];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      a[8 * i + 2 * j] = __builtin_bit_cast(float, v[j] << 16);
      a[8 * i + 2 * j + 1] = __builtin_bit_cast(float, v[j] & 0xffff0000u);
    }
  }
}

// Scale and zero-point of one group (float32, reference formula).
__device__ __forceinline__ void group_params(float mn, float mx, float& s, float& z) {
  s = (mx - mn) / 3.0f;
  s = (s == 0.0f) ? 1.0f : s;
  z = floorf(-mn / s + 0.5f);
}

// code = clamp(floor(fl32(x / s) + 0.5) + z, 0, 3) with fl32(x / s) from
// the fp64 reciprocal (see file header).
__device__ __forceinline__ uint32_t quant_code(float x, double rinv, float z) {
  const float qv = (float)((double)x * rinv);
  float c = floorf(qv + 0.5f) + z;
  c = fminf(fmaxf(c, 0.0f), 3.0f);
  return (uint32_t)c;
}

// K: one thread owns two adjacent channels of one 32-token group.
//   unit = ((pair * groups) + grp) * chunks + chunk,  chunk = 128-channel slice
template <typename T>
__global__ __launch_bounds__(256) void quantize_k_kernel(const T* __restrict__ x,
                                                         uint8_t* __restrict__ packed,
                                                         _Float16* __restrict__ scale,
                                                         _Float16* __restrict__ zero,
                                                         int64_t n_units, int64_t groups, int64_t N,
                                                         int D, int chunks) {
  const int lane = threadIdx.x & 63;
  const int64_t stride = (int64_t)gridDim.x * (blockDim.x >> 6);
  for (int64_t unit = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6); unit < n_units;
       unit += stride) {
    const int chunk = (int)(unit % chunks);
    const int64_t pg = unit / chunks;
    const int64_t grp = pg % groups;
    const int64_t pair = pg / groups;
    const int ch = chunk * 128 + 2 * lane;
    if (ch >= D) continue;
    const T* xp = x + ((size_t)pair * N + (size_t)grp * kGroup) * D + ch;
    float a[kGroup], b[kGroup];
#pragma unroll
    for (int t = 0; t < kGroup; ++t) load2(xp + (size_t)t * D, a[t], b[t]);
    float amn = a[0], amx = a[0], bmn = b[0], bmx = b[0];
#pragma unroll
    for (int t = 1; t < kGroup; ++t) {
      amn = fminf(amn, a[t]);
      amx = fmaxf(amx, a[t]);
      bmn = fminf(bmn, b[t]);
      bmx = fmaxf(bmx, b[t]);
    }
    float as, az, bs, bz;
    group_params(amn, amx, as, az);
    group_params(bmn, bmx, bs, bz);
    const double ar = 1.0 / (double)as, br = 1.0 / (double)bs;
    uint8_t* pp = packed + ((size_t)pair * (N / 4) + (size_t)grp * (kGroup / 4)) * D + ch;
#pragma unroll
    for (int p = 0; p < kGroup / 4; ++p) {
      uint32_t ba = 0, bb = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        ba |= quant_code(a[4 * p + j], ar, az) << (2 * j);
        bb |= quant_code(b[4 * p + j], br, bz) << (2 * j);
      }
      *reinterpret_cast<uint16_t*>(pp + (size_t)p * D) = (uint16_t)(ba | (bb << 8));
    }
    const size_t mo = ((size_t)pair * groups + grp) * D + ch;
    half2v sv = {(_Float16)as, (_Float16)bs};
    half2v zv = {(_Float16)az, (_Float16)bz};
    *reinterpret_cast<half2v*>(scale + mo) = sv;
    *reinterpret_cast<half2v*>(zero + mo) = zv;
  }
}

// V: one thread owns one (token, 32-channel group); unit = (pair*N + t)*(D/32) + grp
// and the group's 32 inputs start at x + unit*32.
template <typename T>
__global__ __launch_bounds__(256) void quantize_v_kernel(const T* __restrict__ x,
                                                         uint8_t* __restrict__ packed,
                                                         _Float16* __restrict__ scale,
                                                         _Float16* __restrict__ zero,
                                                         int64_t n_units) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t u = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; u < n_units; u += stride) {
    const T* xp = x + (size_t)u * kGroup;
    float a[kGroup];
    load32(xp, a);
    float mn = a[0], mx = a[0];
#pragma unroll
    for (int i = 1; i < kGroup; ++i) {
      mn = fminf(mn, a[i]);
      mx = fmaxf(mx, a[i]);
    }
    float s, z;
    group_params(mn, mx, s, z);
    const double r = 1.0 / (double)s;
    u32x2 out;
#pragma unroll
    for (int w = 0; w < 2; ++w) {
      uint32_t word = 0;
#pragma unroll
      for (int i = 0; i < 16; ++i) word |= quant_code(a[16 * w + i], r, z) << (2 * i);
      out[w] = word;
    }
    *reinterpret_cast<u32x2*>(packed + (size_t)u * 8) = out;
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

int launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? KVDEC_OK : (int)e;
}

unsigned grid_for(int64_t threads_needed, int block) {
  int64_t g = (threads_needed + block - 1) / block;
  const int64_t cap = 256 * 64;   // 64 workgroups per CU on a 256-CU part, grid-stride beyond
  if (g > cap) g = cap;
  if (g < 1) g = 1;
  return (unsigned)g;
}

int check_quant_args(const void* x, int in_dtype, const void* p, const void* s, const void* z,
                     int64_t B, int32_t KVH, int64_t N, int32_t D, int32_t group, int32_t bits) {
  if (!x || !p || !s || !z) return KVDEC_E_NULL;
  if (bits != 2) return KVDEC_E_BITS;
  if (in_dtype != KVDEC_F32 && in_dtype != KVDEC_F16 && in_dtype != KVDEC_BF16) return KVDEC_E_DTYPE;
  if (B < 1 || KVH < 1 || N < 1 || D < 1) return KVDEC_E_SHAPE;
  if (group < 1) return KVDEC_E_SHAPE;
  return KVDEC_OK;
}

}  // namespace

extern "C" {

int kvdec_quantize_k(const void* x, int in_dtype, void* packed_u8, void* scale_f16, void* zero_f16,
                     int64_t B, int32_t KVH, int64_t N, int32_t D, int32_t group, int32_t bits,
                     void* stream) {
  int rc = check_quant_args(x, in_dtype, packed_u8, scale_f16, zero_f16, B, KVH, N, D, group, bits);
  if (rc) return rc;
  if (N % group != 0) return KVDEC_E_GROUP;
  if (group != kGroup) return KVDEC_E_UNSUPPORTED;
  if (D % 2 != 0) return KVDEC_E_SHAPE;
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
                       static_cast<const float*>(x), p, s, z, n_units, groups, N, D, chunks);
  else if (in_dtype == KVDEC_F16)
    hipLaunchKernelGGL(quantize_k_kernel<_Float16>, dim3(grid), dim3(256), 0, st,
                       static_cast<const _Float16*>(x), p, s, z, n_units, groups, N, D, chunks);
  else
    hipLaunchKernelGGL(quantize_k_kernel<uint16_t>, dim3(grid), dim3(256), 0, st,
                       static_cast<const uint16_t*>(x), p, s, z, n_units, groups, N, D, chunks);
  return launch_status();
}

int kvdec_quantize_v(const void* x, int in_dtype, void* packed_u8, void* scale_f16, void* zero_f16,
                     int64_t B, int32_t KVH, int64_t N, int32_t D, int32_t group, int32_t bits,
                     void* stream) {
  int rc = check_quant_args(x, in_dtype, packed_u8, scale_f16, zero_f16, B, KVH, N, D, group, bits);
  if (rc) return rc;
  if (D % group != 0) return KVDEC_E_DGROUP;
  if (group != kGroup) return KVDEC_E_UNSUPPORTED;
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
