// Device code shared by the KIVI quantizers (quant.hip) and the decode
// kernels (attn.hip): the exact group quantizer, and the ring bookkeeping and
// block eviction of the decode-time KIVI cache.
//
// The group quantities must be bit-exact to the IEEE-float32 closed form
//   s = (mx - mn) / 3;  s = (s == 0) ? 1 : s;  z = floor(-mn / s + 0.5)
//   code = clamp(floor(x / s + 0.5) + z, 0, 3)
// so the functions that compute them forbid FP contraction locally
// (whatever the including file is compiled with) and keep the HIP default
// of correctly rounded fp32 division.  The per-element quotient is computed
// as described in quant.hip.
#pragma once

#include "kvdec_device.h"

namespace kvdec {

constexpr int kQGroup = 32;

// Scale and zero-point of one group (float32, the reference's formula,
// quant_kernel.py:77-81 for K and :166-170 for V).
__device__ __forceinline__ void group_params(float mn, float mx, float& s, float& z) {
#pragma clang fp contract(off)
  s = (mx - mn) / 3.0f;
  s = (s == 0.0f) ? 1.0f : s;
  z = floorf(-mn / s + 0.5f);
}

// Per-group constants of the code computation.
struct QParams {
  float s, y, z;   // scale, fl32(1 / s), zero
  double rinv;     // RN64(1 / s), slow path
  bool fast;
};

__device__ __forceinline__ QParams make_params(float mn, float mx) {
#pragma clang fp contract(off)
  QParams q;
  group_params(mn, mx, q.s, q.z);
  q.fast = q.s >= 0x1p-40f && q.s <= 0x1p100f;
  q.y = 1.0f / q.s;
  q.rinv = 1.0 / (double)q.s;
  return q;
}

// clamp(floor(fl32(x / s) + 0.5) + z, 0, 3) as a float (see file header).
// E is float or _Float16.  q0 is formed as fma(x, y, +0), equal to fl32(x * y)
// up to the sign of a zero (which cannot change a code), so that a 16-bit x
// enters both FMAs unconverted.  The slow path converts x to double
// directly, which keeps the two paths from sharing a converted copy of x.
template <bool FAST, typename E>
__device__ __forceinline__ float quant_code(E x, const QParams& q) {
#pragma clang fp contract(off)
  float qv;
  if (FAST) {
    const float q0 = __builtin_fmaf((float)x, q.y, 0.0f);
    const float r = __builtin_fmaf(-q0, q.s, (float)x);
    qv = __builtin_fmaf(r, q.y, q0);
  } else {
    qv = (float)((double)x * q.rinv);
  }
  const float c = floorf(qv + 0.5f) + q.z;
  return fminf(fmaxf(c, 0.0f), 3.0f);
}

// Replace byte `b` of `w` by the code c (an integer-valued float in [0, 3]).
__device__ __forceinline__ uint32_t put_code(float c, uint32_t b, uint32_t w) {
  return __builtin_amdgcn_cvt_pk_u8_f32(c, b, w);
}

// One 32-value group (x in group order) quantized by one thread: byte b of
// the result holds the codes of x[4b .. 4b+3], LSB first (the K and V
// packings differ only in where those 8 bytes go).
__device__ __forceinline__ u32x2 quant_group(const float (&x)[32], QParams& q) {
  float mn = x[0], mx = x[0];
#pragma unroll
  for (int i = 1; i < 32; ++i) {
    mn = fminf(mn, x[i]);
    mx = fmaxf(mx, x[i]);
  }
  q = make_params(mn, mx);
  u32x2 out;
#pragma unroll
  for (int w = 0; w < 2; ++w) {
    uint32_t word = 0;
#pragma unroll
    for (int b = 0; b < 4; ++b)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float c = q.fast ? quant_code<true>(x[16 * w + 4 * b + j], q)
                               : quant_code<false>(x[16 * w + 4 * b + j], q);
        word |= (uint32_t)c << (8 * b + 2 * j);
      }
    out[w] = word;
  }
  return out;
}


// ---------------------------------------------------------------------------
// Decode-time KIVI cache: append one token per (b, kv) head to the fp16
// residual ring and, when the ring holds a full group more than the
// residual, quantize its oldest 32-row block into a window-old group slot.
// One workgroup per (b, kv) head.
// ---------------------------------------------------------------------------
struct StreamArgs {
  const _Float16* k_new;   // [pairs][D]
  const _Float16* v_new;
  _Float16* k_ring;        // [pairs][cap][D]
  _Float16* v_ring;
  uint8_t* kp;             // [pairs][nwg * group / 4][D]
  _Float16* ks;            // [pairs][nwg][D]
  _Float16* kz;
  uint8_t* vp;             // [pairs][nwg * group][D / 4]
  _Float16* vs;            // [pairs][nwg * group][D / group]
  _Float16* vz;
  // per-sequence bookkeeping (all null for one shared ring state)
  int32_t* appended;       // [B] tokens appended since each sequence's prefill
  const int32_t* active;   // [B] or null (all)
  int32_t* arrive;         // [B] workgroups done this step (0 between launches)
  int32_t* plan;           // [B][3] {row, evict block, evict slot} taken this step
  int32_t* ring;           // [B][2] {start, count} after this step
  int D, cap, row, blk, slot, nwg, KVH, residual;
};

// Ring bookkeeping of one sequence of a decode-time KIVI cache.  The state
// after n appended tokens is fixed by n: n / 32 evictions, so the residual
// ring holds rows [start, start + count) mod cap with start = 32 (n / 32)
// mod cap and count = residual + n mod 32, and the oldest window-old group
// sits in slot (n / 32) mod n_groups.  An active step takes row (start +
// count) mod cap; when that fills the ring, its oldest 32-row block is
// quantized into the oldest group's slot.  Returns the step ({row, block,
// slot}, -1 = none) and the state after it.
struct RingStep {
  int row, blk, slot, start, count;
};

__device__ __forceinline__ RingStep ring_step(int n, bool act, int residual, int cap, int ngroups) {
  const int e = n / kQGroup;
  RingStep r{-1, -1, -1, (int)(((int64_t)kQGroup * e) % cap), residual + n % kQGroup};
  if (act) {
    r.row = (r.start + r.count) % cap;
    if (r.count + 1 == cap) {
      r.blk = r.start / kQGroup;
      r.slot = ngroups > 0 ? e % ngroups : -1;
      r.start = (r.start + kQGroup) % cap;
      r.count = residual;
    } else {
      r.count += 1;
    }
  }
  return r;
}

// Quantize ring rows [32 blk, +32) of one (b, kv) head into window-old slot
// `slot` (K per channel, V per token, the quantizers' exact formulas).
// Threads tid = 0, 1, .. (nthreads of them) share the D K groups (one
// channel's 32 tokens each) and the 32 * D / 32 V groups (one token's 32
// channels each).
__device__ __forceinline__ void evict_block(const StreamArgs& a, int64_t pair, int blk, int slot,
                                            int tid, int nthreads) {
  const int D = a.D, ng = D / kQGroup;
  const size_t blk0 = (size_t)pair * a.cap + (size_t)blk * kQGroup;   // first ring row of the block
  const size_t g = (size_t)pair * a.nwg + slot;
  for (int u = tid; u < D + kQGroup * ng; u += nthreads) {
    float x[kQGroup];
    QParams q;
    if (u < D) {   // K channel u
#pragma unroll
      for (int t = 0; t < kQGroup; ++t) x[t] = (float)a.k_ring[(blk0 + t) * D + u];
      const u32x2 c = quant_group(x, q);
#pragma unroll
      for (int p = 0; p < kQGroup / 4; ++p)
        a.kp[(g * (kQGroup / 4) + p) * D + u] = (uint8_t)(c[p >> 2] >> (8 * (p & 3)));
      a.ks[g * D + u] = (_Float16)q.s;
      a.kz[g * D + u] = (_Float16)q.z;
    } else {       // V token t, channel group cg
      const int t = (u - D) / ng, cg = (u - D) % ng;
      const _Float16* src = a.v_ring + (blk0 + t) * D + cg * kQGroup;
#pragma unroll
      for (int i = 0; i < kQGroup; ++i) x[i] = (float)src[i];
      const u32x2 c = quant_group(x, q);
      const size_t tok = g * kQGroup + t;
      *reinterpret_cast<u32x2*>(a.vp + tok * (D / 4) + cg * (kQGroup / 4)) = c;
      a.vs[tok * ng + cg] = (_Float16)q.s;
      a.vz[tok * ng + cg] = (_Float16)q.z;
    }
  }
}

}  // namespace kvdec
