// Reference-semantics decode attention for gfx950, for what the MFMA kernels
// of attn.hip do not take:
//   - bf16 and fp32 queries and caches (dense_kernel.py:21-67 and
//     sparse_kernel.py:67-102 load q, k, v in whatever dtype they are given,
//     compute in fp32 and store o in q's dtype);
//   - KIVI caches of any code width and group size (quant_kernel.py:436-548,
//     whose BITS and GROUP_SIZE are kernel parameters: QMAX = 2^BITS - 1,
//     8 / BITS codes per byte).
// Everything is fp32: every K and V element is loaded (or dequantized as
// scale * (code - zero), quant_kernel.py:263-266, 308-311) as a float, the
// logits are fp32 dot products, the softmax runs online in the log2 domain
// and the output is rounded once to q's dtype.
//
// One workgroup of 256 threads per (KV head, split): Q of the KV head's
// query heads in LDS as fp32; the slots in chunks of 64.  Per chunk, thread
// (slot j = tid / 4, quarter c = tid % 4) loads channels 32c .. 32c + 31 of
// slot j's K and V, writes the V part to LDS and forms the partial logits of
// every query head, summed over the four quarters by lane shuffles; then
// thread (head h = tid / 16, i = tid % 16) takes the chunk's max over slots
// i, i + 16, .. (reduced over the head's 16 lanes), rescales its state,
// turns the logits into probabilities and accumulates channels 8i .. 8i + 7
// of P.V.  Several splits per KV head leave (m, l, acc) partials in the
// workspace, combined by generic_merge_kernel.
//
// KIVI slot mapping (the regime composition of quant_kernel.py:358-401):
// slot s < sink is sink token s, slot s < sink + win_tok window-old token
// s - sink, later slots residual row s - sink - win_tok.  (The reference's
// tile dequantizer positions a tile's codes relative to the tile start,
// quant_kernel.py:238-245, which agrees with this mapping whenever the sink
// is a multiple of 8 / BITS, as the default sink of 4 is for BITS >= 2.)

#include "generic.h"

#include "kvdec.h"

namespace kvdec {
namespace {

constexpr int kGT = 256;   // threads per workgroup
constexpr int kGC = 64;    // slots per chunk
constexpr int kGMaxHeads = kMaxGroup;

// Element types of the rows, q and o.
template <int DT>
struct GElt;
template <>
struct GElt<KVDEC_F16> {
  typedef _Float16 T;
  __device__ static float ld(const T* p, size_t i) { return (float)p[i]; }
  __device__ static void st(T* p, size_t i, float v) { p[i] = (_Float16)v; }
};
template <>
struct GElt<KVDEC_BF16> {
  typedef uint16_t T;
  __device__ static float ld(const T* p, size_t i) { return __builtin_bit_cast(float, (uint32_t)p[i] << 16); }
  __device__ static void st(T* p, size_t i, float v) { p[i] = __builtin_bit_cast(uint16_t, (__bf16)v); }
};
template <>
struct GElt<KVDEC_F32> {
  typedef float T;
  __device__ static float ld(const T* p, size_t i) { return p[i]; }
  __device__ static void st(T* p, size_t i, float v) { p[i] = v; }
};

// Slot validity of sequence b.
struct GRange {
  SlotRanges R;
  const int32_t* lens;   // null: R for every sequence
  bool sparse;
  int32_t window, sink, layout;
  int64_t rows;
  __device__ SlotRanges at(int64_t b) const {
    if (!lens) return R;
    int64_t len = lens[b];
    len = len < 0 ? 0 : len;
    if (sparse) return sparse_ranges(len, window, sink, layout);
    return SlotRanges{(int)(len < rows ? len : rows), 0, 0};
  }
};

template <int DT>
struct GArgs {
  const typename GElt<DT>::T* q;
  typename GElt<DT>::T* o;
  float* ws;              // split partials: acc [units][128], then m [units], then l [units]
  int64_t pairs;
  int32_t H, KVH, G;
  int64_t n_slots;
  int64_t per_split;      // slots per split, a multiple of kGC
  int n_splits;
  float scale_log2;
  GRange range;
};

// Rows of element type DT: [pairs][rows][128].
template <int DT>
struct GRowsSrc {
  const typename GElt<DT>::T* k;
  const typename GElt<DT>::T* v;
  int64_t rows;
  __device__ void load(int64_t pair, int64_t s, int c0, float (&kk)[32], float (&vv)[32]) const {
    const size_t base = ((size_t)pair * rows + s) * kHeadDim + c0;
#pragma unroll
    for (int c = 0; c < 32; ++c) {
      kk[c] = GElt<DT>::ld(k, base + c);
      vv[c] = GElt<DT>::ld(v, base + c);
    }
  }
};

// A KIVI cache of any width: residual rows of element type RT and the
// quantized sink (one group) and window-old (win_tok tokens) regions.
template <int RT>
struct GKiviSrc {
  const typename GElt<RT>::T* kres;
  const typename GElt<RT>::T* vres;
  const uint8_t* kp[2];     // sink, window-old
  const _Float16* ks[2];
  const _Float16* kz[2];
  const uint8_t* vp[2];
  const _Float16* vs[2];
  const _Float16* vz[2];
  int32_t ntok[2];          // tokens of each region: group, win_tok
  int32_t sink, win_tok, res_rows, group, bits;

  __device__ void load(int64_t pair, int64_t s, int c0, float (&kk)[32], float (&vv)[32]) const {
    if (s >= sink + win_tok) {
      const size_t base = ((size_t)pair * res_rows + (s - sink - win_tok)) * kHeadDim + c0;
#pragma unroll
      for (int c = 0; c < 32; ++c) {
        kk[c] = GElt<RT>::ld(kres, base + c);
        vv[c] = GElt<RT>::ld(vres, base + c);
      }
      return;
    }
    const int r = s < sink ? 0 : 1;
    const int t = r == 0 ? (int)s : (int)(s - sink);
    const int pf = 8 / bits, n = ntok[r];
    const uint32_t qmax = (1u << bits) - 1u;
    // K, per channel: byte row t / pf of the region, code at bits (t % pf) * bits,
    // scale and zero of group t / group (quant_kernel.py:236-266)
    const uint8_t* kb = kp[r] + ((size_t)pair * (n / pf) + t / pf) * kHeadDim + c0;
    const size_t km = ((size_t)pair * (n / group) + t / group) * kHeadDim + c0;
    const uint32_t ksh = (uint32_t)((t % pf) * bits);
    // V, per token: byte (channel / pf) of row t, code at bits (channel % pf)
    // * bits, scale and zero of channel group channel / group
    // (quant_kernel.py:281-311)
    const uint8_t* vb = vp[r] + ((size_t)pair * n + t) * (kHeadDim / pf);
    const size_t vm = ((size_t)pair * n + t) * (kHeadDim / group);
#pragma unroll
    for (int c = 0; c < 32; ++c) {
      const int ch = c0 + c;
      const float kc = (float)((kb[c] >> ksh) & qmax);
      kk[c] = (float)ks[r][km + c] * (kc - (float)kz[r][km + c]);
      const float vc = (float)((vb[ch / pf] >> ((ch % pf) * bits)) & qmax);
      const size_t g = vm + ch / group;
      vv[c] = (float)vs[r][g] * (vc - (float)vz[r][g]);
    }
  }
};

template <int DT, class Src>
__global__ __launch_bounds__(kGT) void generic_attn_kernel(GArgs<DT> A, Src S) {
  __shared__ float sq[kGMaxHeads][kHeadDim];
  __shared__ __align__(16) float sv[kGC][kHeadDim];
  __shared__ float ss[kGMaxHeads][kGC + 1];
  const int tid = threadIdx.x;
  const int64_t pair = blockIdx.x;
  const int split = blockIdx.y;
  const int64_t b = pair / A.KVH;
  const int kvh = (int)(pair % A.KVH);
  const int G = A.G;
  for (int i = tid; i < G * kHeadDim; i += kGT)
    sq[i / kHeadDim][i % kHeadDim] =
        GElt<DT>::ld(A.q, ((size_t)b * A.H + (size_t)kvh * G + i / kHeadDim) * kHeadDim + i % kHeadDim);
  const SlotRanges R = A.range.at(b);
  const int64_t lo = (int64_t)split * A.per_split;
  const int64_t hi = lo + A.per_split < A.n_slots ? lo + A.per_split : A.n_slots;
  const int j = tid >> 2, quarter = tid & 3;     // loads and logits
  const int h = tid >> 4, cb = tid & 15;         // softmax and P.V
  float m = -INFINITY, l = 0.f;
  float acc[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) acc[k] = 0.f;
  __syncthreads();
  for (int64_t c0 = lo; c0 < hi; c0 += kGC) {
    const int64_t s = c0 + j;
    const bool ok = s < hi && slot_valid(R, (int)s);
    float kk[32], vv[32];
    if (ok) {
      S.load(pair, s, 32 * quarter, kk, vv);
    } else {
#pragma unroll
      for (int c = 0; c < 32; ++c) kk[c] = vv[c] = 0.f;
    }
#pragma unroll
    for (int c = 0; c < 32; c += 4)
      *reinterpret_cast<float4v*>(&sv[j][32 * quarter + c]) = float4v{vv[c], vv[c + 1], vv[c + 2], vv[c + 3]};
    float dot[kGMaxHeads];
#pragma unroll
    for (int hh = 0; hh < kGMaxHeads; ++hh) {
      float d = 0.f;
      if (hh < G) {
#pragma unroll
        for (int c = 0; c < 32; ++c) d = fmaf(sq[hh][32 * quarter + c], kk[c], d);
      }
      d += __shfl_xor(d, 1);
      d += __shfl_xor(d, 2);
      dot[hh] = d;
    }
    if (quarter == 0) {
#pragma unroll
      for (int hh = 0; hh < kGMaxHeads; ++hh)
        if (hh < G) ss[hh][j] = ok ? dot[hh] * A.scale_log2 : -INFINITY;
    }
    __syncthreads();
    float mnew = m;
    if (h < G) {
      float cm = -INFINITY;
#pragma unroll
      for (int u = 0; u < kGC / 16; ++u) cm = fmaxf(cm, ss[h][cb + 16 * u]);
#pragma unroll
      for (int off = 8; off >= 1; off >>= 1) cm = fmaxf(cm, __shfl_xor(cm, off));
      mnew = fmaxf(m, cm);
      float ps = 0.f;
#pragma unroll
      for (int u = 0; u < kGC / 16; ++u) {
        const int jj = cb + 16 * u;
        const float p = mnew == -INFINITY ? 0.f : exp2f(ss[h][jj] - mnew);
        ss[h][jj] = p;
        ps += p;
      }
#pragma unroll
      for (int off = 8; off >= 1; off >>= 1) ps += __shfl_xor(ps, off);
      const float alpha = m == -INFINITY ? 0.f : exp2f(m - mnew);
      l = l * alpha + ps;
#pragma unroll
      for (int k = 0; k < 8; ++k) acc[k] *= alpha;
    }
    __syncthreads();
    if (h < G) {
      for (int jj = 0; jj < kGC; ++jj) {
        const float p = ss[h][jj];
        const float4v v0 = *reinterpret_cast<const float4v*>(&sv[jj][8 * cb]);
        const float4v v1 = *reinterpret_cast<const float4v*>(&sv[jj][8 * cb + 4]);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          acc[k] = fmaf(p, v0[k], acc[k]);
          acc[4 + k] = fmaf(p, v1[k], acc[4 + k]);
        }
      }
    }
    m = mnew;
    __syncthreads();
  }
  if (h >= G) return;
  if (A.n_splits == 1) {
    const float inv = l > 0.f ? 1.0f / l : 0.f;   // no valid slot: zeros
    const size_t row = ((size_t)b * A.H + (size_t)kvh * G + h) * kHeadDim + 8 * cb;
#pragma unroll
    for (int k = 0; k < 8; ++k) GElt<DT>::st(A.o, row + k, acc[k] * inv);
  } else {
    const size_t units = (size_t)A.pairs * A.n_splits * G;
    const size_t u = ((size_t)pair * A.n_splits + split) * G + h;
#pragma unroll
    for (int k = 0; k < 8; ++k) A.ws[u * kHeadDim + 8 * cb + k] = acc[k];
    if (cb == 0) {
      A.ws[units * kHeadDim + u] = m;
      A.ws[units * kHeadDim + units + u] = l;
    }
  }
}

// One workgroup per (KV head, query head of its group), one thread per
// channel: the splits' partials combined in the log2 domain.
template <int DT>
__global__ __launch_bounds__(kHeadDim) void generic_merge_kernel(GArgs<DT> A) {
  const int64_t pair = blockIdx.x / A.G;
  const int h = (int)(blockIdx.x % A.G);
  const int ch = threadIdx.x;
  const size_t units = (size_t)A.pairs * A.n_splits * A.G;
  float M = -INFINITY;
  for (int sp = 0; sp < A.n_splits; ++sp)
    M = fmaxf(M, A.ws[units * kHeadDim + ((size_t)pair * A.n_splits + sp) * A.G + h]);
  float L = 0.f, acc = 0.f;
  if (M != -INFINITY) {
    for (int sp = 0; sp < A.n_splits; ++sp) {
      const size_t u = ((size_t)pair * A.n_splits + sp) * A.G + h;
      const float mu = A.ws[units * kHeadDim + u];
      const float f = mu == -INFINITY ? 0.f : exp2f(mu - M);
      L = fmaf(A.ws[units * kHeadDim + units + u], f, L);
      acc = fmaf(A.ws[u * kHeadDim + ch], f, acc);
    }
  }
  const int64_t b = pair / A.KVH;
  const int kvh = (int)(pair % A.KVH);
  GElt<DT>::st(A.o, ((size_t)b * A.H + (size_t)kvh * A.G + h) * kHeadDim + ch, L > 0.f ? acc / L : 0.f);
}

int gstatus() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? KVDEC_OK : (int)e;
}

template <int DT, class Src>
int launch_generic(GArgs<DT> A, const Src& S, hipStream_t st) {
  dim3 grid((unsigned)A.pairs, (unsigned)A.n_splits);
  hipLaunchKernelGGL((generic_attn_kernel<DT, Src>), grid, dim3(kGT), 0, st, A, S);
  if (A.n_splits > 1)
    hipLaunchKernelGGL(generic_merge_kernel<DT>, dim3((unsigned)(A.pairs * A.G)), dim3(kHeadDim), 0, st, A);
  return gstatus();
}

// Splits: enough workgroups to fill the chip (>= 2048 with >= 8 chunks per
// split), as many as the workspace holds.
void plan_splits(int64_t pairs, int G, int64_t n_slots, void* ws, size_t ws_bytes, int& n_splits,
                 int64_t& per_split) {
  const int64_t chunks = (n_slots + kGC - 1) / kGC;
  int64_t sp = (2048 + pairs - 1) / pairs;
  const int64_t by_len = (chunks + 7) / 8;
  if (sp > by_len) sp = by_len;
  const size_t per_unit = (size_t)pairs * G * (kHeadDim + 2) * sizeof(float);
  const int64_t by_ws = ws ? (int64_t)(ws_bytes / per_unit) : 1;
  if (sp > by_ws) sp = by_ws;
  if (sp < 1) sp = 1;
  if (sp > 65535) sp = 65535;
  per_split = ((chunks + sp - 1) / sp) * kGC;
  n_splits = (int)((n_slots + per_split - 1) / per_split);
  if (n_splits < 1) n_splits = 1;
}

template <int DT>
int rows_decode_t(const void* q, const void* k, const void* v, void* o, int64_t B, int32_t H, int32_t KVH,
                  int64_t rows, SlotRanges R, const int32_t* lens, bool sparse, int32_t window,
                  int32_t sink, int32_t layout, float sm_scale, void* ws, size_t ws_bytes,
                  hipStream_t st) {
  typedef typename GElt<DT>::T T;
  GArgs<DT> A{};
  A.q = static_cast<const T*>(q);
  A.o = static_cast<T*>(o);
  A.ws = static_cast<float*>(ws);
  A.pairs = B * KVH;
  A.H = H;
  A.KVH = KVH;
  A.G = H / KVH;
  A.n_slots = rows;
  A.scale_log2 = (float)((double)sm_scale * 1.4426950408889634);
  A.range = GRange{R, lens, sparse, window, sink, layout, rows};
  plan_splits(A.pairs, A.G, rows, ws, ws_bytes, A.n_splits, A.per_split);
  GRowsSrc<DT> S{static_cast<const T*>(k), static_cast<const T*>(v), rows};
  return launch_generic(A, S, st);
}

}  // namespace

int generic_rows_decode(const void* q, const void* k, const void* v, void* o, int dtype, int64_t B,
                        int32_t H, int32_t KVH, int64_t rows, SlotRanges R, const int32_t* lens,
                        bool sparse, int32_t window, int32_t sink, int32_t layout, float sm_scale,
                        void* ws, size_t ws_bytes, hipStream_t stream) {
  if (dtype == KVDEC_F32)
    return rows_decode_t<KVDEC_F32>(q, k, v, o, B, H, KVH, rows, R, lens, sparse, window, sink, layout,
                                    sm_scale, ws, ws_bytes, stream);
  if (dtype == KVDEC_BF16)
    return rows_decode_t<KVDEC_BF16>(q, k, v, o, B, H, KVH, rows, R, lens, sparse, window, sink, layout,
                                     sm_scale, ws, ws_bytes, stream);
  if (dtype == KVDEC_F16)
    return rows_decode_t<KVDEC_F16>(q, k, v, o, B, H, KVH, rows, R, lens, sparse, window, sink, layout,
                                    sm_scale, ws, ws_bytes, stream);
  return KVDEC_E_DTYPE;
}

template <int QT, int RT>
int kivi_decode_t2(const void* q, const void* k_res, const void* v_res, const void* const* kivi, void* o,
                   const int32_t* lens, int64_t B, int32_t H, int32_t KVH, int64_t seq_len, int32_t window,
                   int32_t sink, int32_t res_rows, int32_t win_tok, int32_t group, int32_t bits,
                   float sm_scale, hipStream_t stream) {
  GArgs<QT> A{};
  A.q = static_cast<const typename GElt<QT>::T*>(q);
  A.o = static_cast<typename GElt<QT>::T*>(o);
  A.ws = nullptr;
  A.pairs = B * KVH;
  A.H = H;
  A.KVH = KVH;
  A.G = H / KVH;
  A.n_slots = (int64_t)sink + window;
  A.scale_log2 = (float)((double)sm_scale * 1.4426950408889634);
  A.range = GRange{sparse_ranges(seq_len, window, sink, KVDEC_LAYOUT_LINEAR), lens, true, window, sink,
                   KVDEC_LAYOUT_LINEAR, A.n_slots};
  A.n_splits = 1;
  A.per_split = ((A.n_slots + kGC - 1) / kGC) * kGC;
  GKiviSrc<RT> S{};
  S.kres = static_cast<const typename GElt<RT>::T*>(k_res);
  S.vres = static_cast<const typename GElt<RT>::T*>(v_res);
  for (int r = 0; r < 2; ++r) {
    const int base = 6 * r;
    S.kp[r] = static_cast<const uint8_t*>(kivi[base]);
    S.ks[r] = static_cast<const _Float16*>(kivi[base + 1]);
    S.kz[r] = static_cast<const _Float16*>(kivi[base + 2]);
    S.vp[r] = static_cast<const uint8_t*>(kivi[base + 3]);
    S.vs[r] = static_cast<const _Float16*>(kivi[base + 4]);
    S.vz[r] = static_cast<const _Float16*>(kivi[base + 5]);
  }
  S.ntok[0] = group;
  S.ntok[1] = win_tok;
  S.sink = sink;
  S.win_tok = win_tok;
  S.res_rows = res_rows;
  S.group = group;
  S.bits = bits;
  return launch_generic(A, S, stream);
}

template <int QT>
int kivi_decode_q(int res_dtype, const void* q, const void* k_res, const void* v_res,
                  const void* const* kivi, void* o, const int32_t* lens, int64_t B, int32_t H, int32_t KVH,
                  int64_t seq_len, int32_t window, int32_t sink, int32_t res_rows, int32_t win_tok,
                  int32_t group, int32_t bits, float sm_scale, hipStream_t stream) {
  if (res_dtype == KVDEC_F16)
    return kivi_decode_t2<QT, KVDEC_F16>(q, k_res, v_res, kivi, o, lens, B, H, KVH, seq_len, window, sink,
                                         res_rows, win_tok, group, bits, sm_scale, stream);
  if (res_dtype == KVDEC_BF16)
    return kivi_decode_t2<QT, KVDEC_BF16>(q, k_res, v_res, kivi, o, lens, B, H, KVH, seq_len, window, sink,
                                          res_rows, win_tok, group, bits, sm_scale, stream);
  if (res_dtype == KVDEC_F32)
    return kivi_decode_t2<QT, KVDEC_F32>(q, k_res, v_res, kivi, o, lens, B, H, KVH, seq_len, window, sink,
                                         res_rows, win_tok, group, bits, sm_scale, stream);
  return KVDEC_E_DTYPE;
}

int generic_kivi_decode(const void* q, const void* k_res, const void* v_res, const void* const* kivi,
                        void* o, int q_dtype, int res_dtype, const int32_t* lens, int64_t B, int32_t H,
                        int32_t KVH, int64_t seq_len, int32_t window, int32_t sink, int32_t res_rows,
                        int32_t win_tok, int32_t group, int32_t bits, float sm_scale,
                        hipStream_t stream) {
  if (q_dtype == KVDEC_F16)
    return kivi_decode_q<KVDEC_F16>(res_dtype, q, k_res, v_res, kivi, o, lens, B, H, KVH, seq_len, window,
                                    sink, res_rows, win_tok, group, bits, sm_scale, stream);
  if (q_dtype == KVDEC_BF16)
    return kivi_decode_q<KVDEC_BF16>(res_dtype, q, k_res, v_res, kivi, o, lens, B, H, KVH, seq_len, window,
                                     sink, res_rows, win_tok, group, bits, sm_scale, stream);
  if (q_dtype == KVDEC_F32)
    return kivi_decode_q<KVDEC_F32>(res_dtype, q, k_res, v_res, kivi, o, lens, B, H, KVH, seq_len, window,
                                    sink, res_rows, win_tok, group, bits, sm_scale, stream);
  return KVDEC_E_DTYPE;
}

}  // namespace kvdec
