// Split-K flash-decode kernels for gfx950: dense GQA decode, StreamingLLM
// sink+window decode and the fused KIVI-2bit decode, plus their C-ABI entry
// points (declared in include/kvdec.h).
//
// One workgroup = one (KV head, split) work item of 4 or 8 waves.  Each wave
// streams a contiguous run of 32-token tiles of that KV head through MFMA
// (all GQA query heads of the KV head at once, so each K/V byte is read
// once), keeps an online softmax, and the waves merge through LDS.  With one
// split the workgroup writes the fp16 output directly; otherwise it writes an
// fp32 partial (m, l, acc) and merge_kernel combines the splits.  At the
// benchmark shapes (B*KVH = 256 KV heads) every path runs in one pass.

#include "kvdec_device.h"
#include "kvdec.h"

using namespace kvdec;

namespace {

struct AttnCommon {
  const _Float16* q;     // [B, H, 128]
  _Float16* o;           // [B, H, 128]
  float* ws;             // [pairs*splits*G*128] acc, then [..*G] m, then l
  int64_t pairs;
  int32_t H, KVH, G;
  int32_t n_tiles, tiles_per_split, n_splits;
  float scale_log2;
  SlotRanges R;
};

__device__ __forceinline__ void load_q_operand(const AttnCommon& P, int64_t b, int kvh, int lane,
                                               half8 (&qB)[4]) {
  const int n = lane & 15, g = lane >> 4;
  if (n < P.G) {
    const u32x4* qp = reinterpret_cast<const u32x4*>(
                          P.q + ((size_t)b * P.H + (size_t)kvh * P.G + n) * kHeadDim) + g;
#pragma unroll
    for (int c = 0; c < 4; ++c) qB[c] = as_h8(qp[4 * c]);
  } else {
#pragma unroll
    for (int c = 0; c < 4; ++c) qB[c] = as_h8(u32x4{0u, 0u, 0u, 0u});
  }
}

// LDS of a workgroup: the per-wave KIVI staging slots (quantized sources
// only), then the merge area -- per wave, the max and sum of 16 heads and the
// G x 128 partial outputs (rows padded by 4 floats).
constexpr int kORow = kHeadDim + 4;
__host__ __device__ constexpr size_t merge_lds_bytes(int nw, int G) {
  return (size_t)(2 * nw * kMaxGroup + nw * G * kORow) * sizeof(float);
}
__host__ __device__ constexpr size_t stage_lds_bytes(int nw, bool quant) {
  return quant ? (size_t)nw * kQSlotBytes : 0;
}

// Merge the NW waves of the workgroup and emit the output or a partial.
template <int NW>
__device__ __forceinline__ void finish_block(const AttnCommon& P, WaveState& st, float* smem,
                                             int64_t pair, int split, int lane, int wave) {
  float* sh_m = smem;                       // [NW][16]
  float* sh_l = smem + NW * kMaxGroup;      // [NW][16]
  float* sh_o = smem + 2 * NW * kMaxGroup;  // [NW][G][kORow]

  st.l += __shfl_xor(st.l, 16);
  st.l += __shfl_xor(st.l, 32);
  const int n = lane & 15, g = lane >> 4;
  if (n < P.G) {
    if (g == 0) {
      sh_m[wave * kMaxGroup + n] = st.m;
      sh_l[wave * kMaxGroup + n] = st.l;
    }
    float* orow = sh_o + ((size_t)wave * P.G + n) * kORow + 32 * g;
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) orow[8 * r + jj] = st.O[jj][r];
  }
  __syncthreads();

  const int64_t b = pair / P.KVH;
  const int kvh = (int)(pair % P.KVH);
  const size_t total = (size_t)P.pairs * P.n_splits * P.G;
  for (int e = threadIdx.x; e < P.G * kHeadDim; e += 64 * NW) {
    const int hn = e / kHeadDim, d = e % kHeadDim;
    float M = kMaxSentinel;
#pragma unroll
    for (int w = 0; w < NW; ++w) M = fmaxf(M, sh_m[w * kMaxGroup + hn]);
    float L = 0.f, acc = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float f = __builtin_amdgcn_exp2f(sh_m[w * kMaxGroup + hn] - M);
      L += sh_l[w * kMaxGroup + hn] * f;
      acc += sh_o[((size_t)w * P.G + hn) * kORow + d] * f;
    }
    if (P.n_splits == 1) {
      P.o[((size_t)b * P.H + (size_t)kvh * P.G + hn) * kHeadDim + d] = (_Float16)(acc / L);
    } else {
      const size_t idx = ((size_t)pair * P.n_splits + split) * P.G + hn;
      P.ws[idx * kHeadDim + d] = acc;
      if (d == 0) {
        P.ws[total * kHeadDim + idx] = M;
        P.ws[total * kHeadDim + total + idx] = L;
      }
    }
  }
}

// Stream fp16 tiles [tb, te) of one region through the wave, two tiles in
// flight (ping-pong register buffers).  Row r of the region is slot
// slot_base + r.
__device__ __forceinline__ void run_f16_tiles(const _Float16* __restrict__ kb,
                                              const _Float16* __restrict__ vb, int rows,
                                              int slot_base, int tb, int te,
                                              const half8 (&qB)[4], const AttnCommon& P,
                                              WaveState& st, int lane) {
  if (tb >= te) return;
  Tile A, B;
  load_f16_tile(kb, vb, kTile * tb, rows, lane, A);
  for (int ti = tb; ti < te; ti += 2) {
    if (ti + 1 < te) load_f16_tile(kb, vb, kTile * (ti + 1), rows, lane, B);
    tile_step(A, qB, slot_base + kTile * ti, P.R, P.scale_log2, st, lane);
    if (ti + 1 >= te) break;
    if (ti + 2 < te) load_f16_tile(kb, vb, kTile * (ti + 2), rows, lane, A);
    tile_step(B, qB, slot_base + kTile * (ti + 1), P.R, P.scale_log2, st, lane);
  }
}

// fp16 rows: the dense cache [B, KVH, L, 128] or the compacted sparse cache
// [B, KVH, sink+window, 128]; slot == row.
struct F16Src {
  static constexpr bool kQuant = false;
  const _Float16* k;
  const _Float16* v;
  int rows;
  __device__ __forceinline__ void run(int64_t pair, int wb, int we, const half8 (&qB)[4],
                                      const AttnCommon& P, WaveState& st, char*, int lane) const {
    const size_t off = (size_t)pair * rows * kHeadDim;
    run_f16_tiles(k + off, v + off, rows, 0, wb, we, qB, P, st, lane);
  }
};

// KIVI cache: tile 0 = the sink group (quantized, `sink` real tokens), tiles
// 1..nwt = window-old groups (quantized), then the fp16 residual tiles.
struct KiviSrc {
  static constexpr bool kQuant = true;
  static constexpr int kRing = 3;   // quantized tiles in flight per wave
  const _Float16* kres;
  const _Float16* vres;
  int res_rows;
  QRegion sinkq;   // base pointers (pair 0)
  QRegion winq;
  int sink;
  int win_tok;     // window - residual
  int nwt;         // win_tok / 32

  __device__ __forceinline__ void run(int64_t pair, int wb, int we, const half8 (&qB)[4],
                                      const AttnCommon& P, WaveState& st, char* slot,
                                      int lane) const {
    const int nq = 1 + nwt;
    const int qb = wb, qe = we < nq ? we : nq;
    if (qb < qe) {
      QRegion S = sinkq, W = winq;
      S.kp += (size_t)pair * 8 * kHeadDim;
      S.ks += (size_t)pair * kHeadDim;
      S.kz += (size_t)pair * kHeadDim;
      S.vp += (size_t)pair * 32 * 32;
      S.vs += (size_t)pair * 32 * 4;
      S.vz += (size_t)pair * 32 * 4;
      if (nwt > 0) {
        W.kp += (size_t)pair * (win_tok / 4) * kHeadDim;
        W.ks += (size_t)pair * (win_tok / 32) * kHeadDim;
        W.kz += (size_t)pair * (win_tok / 32) * kHeadDim;
        W.vp += (size_t)pair * win_tok * 32;
        W.vs += (size_t)pair * win_tok * 4;
        W.vz += (size_t)pair * win_tok * 4;
      }
      // tile ti: 0 = sink group (slots 0..sink-1), else window-old group ti-1
      auto load = [&](int ti, QTileRaw& X) {
        if (ti == 0)
          load_q_raw(S, 0, lane, X);
        else
          load_q_raw(W, ti - 1, lane, X);
      };
      // Ring of kRing raw tiles in flight; each is staged through the wave's
      // LDS slot into operand layout just before it is consumed.
      QTileRaw ring[kRing];
#pragma unroll
      for (int k = 0; k < kRing; ++k)
        if (qb + k < qe) load(qb + k, ring[k]);
      for (int base = qb; base < qe; base += kRing) {
#pragma unroll
        for (int k = 0; k < kRing; ++k) {
          const int ti = base + k;
          if (ti < qe) {
            stage_q_raw(ring[k], slot, lane);
            if (ti + kRing < qe) load(ti + kRing, ring[k]);
            q_tile_step(slot, qB, ti == 0 ? 0 : sink + kTile * (ti - 1), ti == 0 ? sink : kTile,
                        P.R, P.scale_log2, st, lane);
          }
        }
      }
    }
    const int fb = (wb > nq ? wb : nq) - nq, fe = we - nq;
    if (fb < fe) {
      const size_t off = (size_t)pair * res_rows * kHeadDim;
      run_f16_tiles(kres + off, vres + off, res_rows, sink + win_tok, fb, fe, qB, P, st, lane);
    }
  }
};

// NW waves per workgroup, two waves per SIMD.
template <class Src, int NW>
__global__ __launch_bounds__(64 * NW, 8 / NW) void attn_kernel(AttnCommon P, Src S) {
  extern __shared__ float smem[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int split = (int)(blockIdx.x % (unsigned)P.n_splits);
  const int64_t pair = blockIdx.x / (unsigned)P.n_splits;
  const int64_t b = pair / P.KVH;
  const int kvh = (int)(pair % P.KVH);

  half8 qB[4];
  load_q_operand(P, b, kvh, lane, qB);

  const int t0 = split * P.tiles_per_split;
  const int t1 = min(t0 + P.tiles_per_split, P.n_tiles);
  const int nt = t1 - t0;
  const int wb = t0 + (nt * wave) / NW;
  const int we = t0 + (nt * (wave + 1)) / NW;

  WaveState st;
  wave_state_init(st);
  char* slot = reinterpret_cast<char*>(smem) + (size_t)wave * kQSlotBytes;
  S.run(pair, wb, we, qB, P, st, slot, lane);
  finish_block<NW>(P, st, smem + stage_lds_bytes(NW, Src::kQuant) / sizeof(float), pair, split,
                   lane, wave);
}

// Log-sum-exp merge of the split partials: one thread per output element.
__global__ __launch_bounds__(256) void merge_kernel(AttnCommon P) {
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= P.pairs * P.G * kHeadDim) return;
  const int d = (int)(e % kHeadDim);
  const int hn = (int)((e / kHeadDim) % P.G);
  const int64_t pair = e / ((int64_t)kHeadDim * P.G);
  const int64_t b = pair / P.KVH;
  const int kvh = (int)(pair % P.KVH);
  const size_t total = (size_t)P.pairs * P.n_splits * P.G;
  const float* wo = P.ws;
  const float* wm = P.ws + total * kHeadDim;
  const float* wl = wm + total;
  const size_t base = (size_t)pair * P.n_splits * P.G + hn;
  float M = kMaxSentinel;
  for (int s = 0; s < P.n_splits; ++s) M = fmaxf(M, wm[base + (size_t)s * P.G]);
  float L = 0.f, acc = 0.f;
#pragma unroll 4
  for (int s = 0; s < P.n_splits; ++s) {
    const size_t idx = base + (size_t)s * P.G;
    const float f = __builtin_amdgcn_exp2f(wm[idx] - M);
    L += wl[idx] * f;
    acc += wo[idx * kHeadDim + d] * f;
  }
  P.o[((size_t)b * P.H + (size_t)kvh * P.G + hn) * kHeadDim + d] = (_Float16)(acc / L);
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------

// Launch plan.  Aim for kTargetWaves resident waves over the whole chip (256
// CUs x 2 waves per SIMD x 4 SIMDs), at least kMinTilesPerWave tiles each; a
// KV head gets up to 8 waves in one workgroup and more waves only through
// splits (which need the merge pass).
constexpr int64_t kTargetWaves = 2048;
constexpr int64_t kMinTilesPerWave = 2;

struct Plan {
  int nw, splits, tps;
};

Plan make_plan(int64_t pairs, int64_t n_tiles, int G, bool quant) {
  int64_t wpp = (kTargetWaves + pairs - 1) / pairs;
  const int64_t cap = (n_tiles + kMinTilesPerWave - 1) / kMinTilesPerWave;
  if (wpp > cap) wpp = cap;
  if (wpp < 1) wpp = 1;
  const bool fits8 = merge_lds_bytes(8, G) + stage_lds_bytes(8, quant) <= 65536;
  Plan p;
  p.nw = (wpp > 4 && fits8) ? 8 : 4;
  int64_t s = (wpp + p.nw - 1) / p.nw;
  int64_t t = (n_tiles + s - 1) / s;
  s = (n_tiles + t - 1) / t;
  p.splits = (int)s;
  p.tps = (int)t;
  return p;
}

int64_t tiles_for(int kind, int64_t n_slots) {
  if (kind == KVDEC_KIND_KIVI) return 1 + n_slots / kTile;
  return (n_slots + kTile - 1) / kTile;
}

size_t ws_bytes_for(int64_t pairs, int splits, int G) {
  if (splits <= 1) return 0;
  return (size_t)pairs * splits * G * (kHeadDim + 2) * sizeof(float);
}

int check_heads(int64_t B, int32_t H, int32_t KVH, int32_t D) {
  if (B < 1 || H < 1 || KVH < 1 || H % KVH != 0) return KVDEC_E_SHAPE;
  if (H / KVH > kMaxGroup) return KVDEC_E_SHAPE;
  if (D != kHeadDim) return KVDEC_E_SHAPE;
  if (B * (int64_t)KVH > (int64_t)1 << 30) return KVDEC_E_SHAPE;
  return KVDEC_OK;
}

int launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? KVDEC_OK : (int)e;
}

template <class Src>
int launch_attn(AttnCommon P, const Src& S, size_t ws_bytes, hipStream_t stream) {
  const Plan plan = make_plan(P.pairs, P.n_tiles, P.G, Src::kQuant);
  P.n_splits = plan.splits;
  P.tiles_per_split = plan.tps;
  if (plan.splits > 1) {
    if (P.ws == nullptr) return KVDEC_E_WORKSPACE;
    if (ws_bytes < ws_bytes_for(P.pairs, plan.splits, P.G)) return KVDEC_E_WORKSPACE;
  }
  const int64_t blocks = P.pairs * plan.splits;
  if (blocks > 0x7fffffffLL) return KVDEC_E_SHAPE;
  const size_t lds = stage_lds_bytes(plan.nw, Src::kQuant) + merge_lds_bytes(plan.nw, P.G);
  if (plan.nw == 8)
    hipLaunchKernelGGL((attn_kernel<Src, 8>), dim3((unsigned)blocks), dim3(64 * 8), lds, stream,
                       P, S);
  else
    hipLaunchKernelGGL((attn_kernel<Src, 4>), dim3((unsigned)blocks), dim3(64 * 4), lds, stream,
                       P, S);
  int rc = launch_status();
  if (rc != KVDEC_OK || plan.splits == 1) return rc;
  const int64_t outs = P.pairs * P.G * kHeadDim;
  hipLaunchKernelGGL(merge_kernel, dim3((unsigned)((outs + 255) / 256)), dim3(256), 0, stream, P);
  return launch_status();
}

// Validity ranges of the [sink + window] cache at this length (the
// _kv_indices rule for the linear layout), clamped into [0, sink + window].
SlotRanges sparse_ranges(int64_t seq_len, int32_t window, int32_t sink, int32_t layout) {
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

}  // namespace

extern "C" {

const char* kvdec_strerror(int code) {
  switch (code) {
    case KVDEC_OK: return "success";
    case KVDEC_E_NULL: return "a required pointer is NULL";
    case KVDEC_E_SHAPE: return "a dimension is out of range or inconsistent";
    case KVDEC_E_DTYPE: return "unsupported element type";
    case KVDEC_E_GROUP: return "this simple version assumes seq_len is a multiple of group_size";
    case KVDEC_E_DGROUP: return "this simple version assumes D_HEAD is a multiple of group_size";
    case KVDEC_E_WORKSPACE: return "workspace missing or smaller than kvdec_workspace_bytes()";
    case KVDEC_E_WINDOW: return "unsupported window / sink / residual combination";
    case KVDEC_E_SEQLEN: return "seq_len must be >= 1";
    case KVDEC_E_BITS: return "only 2-bit quantization is implemented";
    case KVDEC_E_UNSUPPORTED: return "valid arguments, but not implemented";
    default: break;
  }
  if (code > 0) return hipGetErrorString((hipError_t)code);
  return "unknown kvdec error";
}

const char* kvdec_version(void) { return "kvdec 0.2 gfx950"; }

int kvdec_num_splits(int kind, int64_t B, int32_t KVH, int64_t n_slots) {
  if (B < 1 || KVH < 1 || n_slots < 1) return 1;
  // The plan's split count does not depend on the group size, only the
  // waves-per-workgroup choice does.
  return make_plan(B * KVH, tiles_for(kind, n_slots), 8, kind == KVDEC_KIND_KIVI).splits;
}

size_t kvdec_workspace_bytes(int kind, int64_t B, int32_t H, int32_t KVH, int64_t n_slots,
                             int32_t D) {
  if (check_heads(B, H, KVH, D) != KVDEC_OK || n_slots < 1) return 0;
  const Plan p = make_plan(B * KVH, tiles_for(kind, n_slots), H / KVH, kind == KVDEC_KIND_KIVI);
  return ws_bytes_for(B * KVH, p.splits, H / KVH);
}

int kvdec_dense_decode(const void* q, const void* k, const void* v, void* o, int dtype, int64_t B,
                       int32_t H, int32_t KVH, int64_t L, int32_t D, float sm_scale, void* ws,
                       size_t ws_bytes, void* stream) {
  if (!q || !k || !v || !o) return KVDEC_E_NULL;
  if (dtype != KVDEC_F16) return KVDEC_E_DTYPE;
  int rc = check_heads(B, H, KVH, D);
  if (rc) return rc;
  if (L < 1) return KVDEC_E_SEQLEN;
  if (L * kHeadDim * 2 >= ((int64_t)1 << 31)) return KVDEC_E_SHAPE;   // 32-bit in-head offsets
  AttnCommon P{};
  P.q = static_cast<const _Float16*>(q);
  P.o = static_cast<_Float16*>(o);
  P.ws = static_cast<float*>(ws);
  P.pairs = B * KVH;
  P.H = H;
  P.KVH = KVH;
  P.G = H / KVH;
  P.n_tiles = (int)tiles_for(KVDEC_KIND_DENSE, L);
  P.scale_log2 = (float)((double)sm_scale * 1.4426950408889634);
  P.R = SlotRanges{(int)L, 0, 0};
  F16Src S{static_cast<const _Float16*>(k), static_cast<const _Float16*>(v), (int)L};
  return launch_attn(P, S, ws_bytes, static_cast<hipStream_t>(stream));
}

int kvdec_sparse_decode(const void* q, const void* k_cache, const void* v_cache, void* o,
                        int dtype, int64_t B, int32_t H, int32_t KVH, int64_t seq_len,
                        int32_t window, int32_t sink, int32_t layout, float sm_scale, void* ws,
                        size_t ws_bytes, void* stream) {
  if (!q || !k_cache || !v_cache || !o) return KVDEC_E_NULL;
  if (dtype != KVDEC_F16) return KVDEC_E_DTYPE;
  int rc = check_heads(B, H, KVH, kHeadDim);
  if (rc) return rc;
  if (seq_len < 1) return KVDEC_E_SEQLEN;
  if (window < 0 || sink < 0 || (int64_t)window + sink < 1) return KVDEC_E_WINDOW;
  if (layout != KVDEC_LAYOUT_LINEAR && layout != KVDEC_LAYOUT_RING) return KVDEC_E_UNSUPPORTED;
  if (layout == KVDEC_LAYOUT_RING && window < 1) return KVDEC_E_WINDOW;
  const int64_t n = (int64_t)window + sink;
  if (n * kHeadDim * 2 >= ((int64_t)1 << 31)) return KVDEC_E_SHAPE;
  AttnCommon P{};
  P.q = static_cast<const _Float16*>(q);
  P.o = static_cast<_Float16*>(o);
  P.ws = static_cast<float*>(ws);
  P.pairs = B * KVH;
  P.H = H;
  P.KVH = KVH;
  P.G = H / KVH;
  P.n_tiles = (int)tiles_for(KVDEC_KIND_SPARSE, n);
  P.scale_log2 = (float)((double)sm_scale * 1.4426950408889634);
  P.R = sparse_ranges(seq_len, window, sink, layout);
  F16Src S{static_cast<const _Float16*>(k_cache), static_cast<const _Float16*>(v_cache), (int)n};
  return launch_attn(P, S, ws_bytes, static_cast<hipStream_t>(stream));
}

int kvdec_sparse_decode_kivi(const void* q, const void* k_res, const void* v_res,
                             const void* const* kivi, void* o, int64_t B, int32_t H, int32_t KVH,
                             int64_t seq_len, int32_t window, int32_t sink, int32_t residual,
                             int32_t group, int32_t bits, float sm_scale, void* ws,
                             size_t ws_bytes, void* stream) {
  if (!q || !k_res || !v_res || !kivi || !o) return KVDEC_E_NULL;
  if (bits != 2) return KVDEC_E_BITS;
  if (group != 32) return KVDEC_E_UNSUPPORTED;
  int rc = check_heads(B, H, KVH, kHeadDim);
  if (rc) return rc;
  if (seq_len < 1) return KVDEC_E_SEQLEN;
  if (sink < 1 || sink > group || residual < kTile || residual % kTile != 0 || window < residual)
    return KVDEC_E_WINDOW;
  const int32_t win_tok = window - residual;
  if (win_tok % group != 0) return KVDEC_E_GROUP;
  for (int i = 0; i < 6; ++i)
    if (!kivi[i]) return KVDEC_E_NULL;
  if (win_tok > 0)
    for (int i = 6; i < 12; ++i)
      if (!kivi[i]) return KVDEC_E_NULL;
  if ((int64_t)residual * kHeadDim * 2 >= ((int64_t)1 << 31) ||
      (int64_t)win_tok * kHeadDim >= ((int64_t)1 << 31))
    return KVDEC_E_SHAPE;

  AttnCommon P{};
  P.q = static_cast<const _Float16*>(q);
  P.o = static_cast<_Float16*>(o);
  P.ws = static_cast<float*>(ws);
  P.pairs = B * KVH;
  P.H = H;
  P.KVH = KVH;
  P.G = H / KVH;
  P.n_tiles = (int)tiles_for(KVDEC_KIND_KIVI, window);
  P.scale_log2 = (float)((double)sm_scale * 1.4426950408889634);
  P.R = sparse_ranges(seq_len, window, sink, KVDEC_LAYOUT_LINEAR);

  auto u8 = [&](int i) { return static_cast<const uint8_t*>(kivi[i]); };
  auto f16 = [&](int i) { return static_cast<const _Float16*>(kivi[i]); };
  KiviSrc S{};
  S.kres = static_cast<const _Float16*>(k_res);
  S.vres = static_cast<const _Float16*>(v_res);
  S.res_rows = residual;
  S.sinkq = QRegion{u8(0), f16(1), f16(2), u8(3), f16(4), f16(5)};
  if (win_tok > 0)
    S.winq = QRegion{u8(6), f16(7), f16(8), u8(9), f16(10), f16(11)};
  else
    S.winq = S.sinkq;   // never dereferenced: there are no window-old tiles
  S.sink = sink;
  S.win_tok = win_tok;
  S.nwt = win_tok / kTile;
  return launch_attn(P, S, ws_bytes, static_cast<hipStream_t>(stream));
}

}  // extern "C"
