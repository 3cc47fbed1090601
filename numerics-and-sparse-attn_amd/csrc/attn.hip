// Split-K flash-decode kernels for gfx950: dense GQA decode, StreamingLLM
// sink+window decode and the fused KIVI-2bit decode, plus their C-ABI entry
// points (declared in include/kvdec.h).
//
// One workgroup = 4 waves = one (KV head, split) work item.  Each wave streams
// a contiguous run of 32-token tiles of that KV head through MFMA (all GQA
// query heads of the KV head at once, so each K/V byte is read once), keeps an
// online softmax, and the 4 waves merge through LDS.  With one split the
// workgroup writes the fp16 output directly; otherwise it writes an fp32
// partial (m, l, acc) and merge_kernel combines the splits.

#include "kvdec_device.h"
#include "kvdec.h"

#include <string.h>

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

// Merge the 4 waves of the workgroup and emit the output or a partial.
__device__ __forceinline__ void finish_block(const AttnCommon& P, WaveState& st, int64_t pair,
                                             int split, int lane, int wave) {
  __shared__ float sh_m[kWaves][kMaxGroup];
  __shared__ float sh_l[kWaves][kMaxGroup];
  __shared__ float sh_o[kWaves][kMaxGroup][kHeadDim + 4];

  st.l += __shfl_xor(st.l, 16);
  st.l += __shfl_xor(st.l, 32);
  const int n = lane & 15, g = lane >> 4;
  if (n < P.G) {
    if (g == 0) {
      sh_m[wave][n] = st.m;
      sh_l[wave][n] = st.l;
    }
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) sh_o[wave][n][32 * g + 8 * r + jj] = st.O[jj][r];
  }
  __syncthreads();

  const int64_t b = pair / P.KVH;
  const int kvh = (int)(pair % P.KVH);
  const size_t total = (size_t)P.pairs * P.n_splits * P.G;
  for (int e = threadIdx.x; e < P.G * kHeadDim; e += kBlock) {
    const int hn = e / kHeadDim, d = e % kHeadDim;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) M = fmaxf(M, sh_m[w][hn]);
    const float Mu = (M == -INFINITY) ? 0.f : M;
    float L = 0.f, acc = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float f = __builtin_amdgcn_exp2f(sh_m[w][hn] - Mu);
      L += sh_l[w][hn] * f;
      acc += sh_o[w][hn][d] * f;
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
// flight (ping-pong register buffers).
__device__ __forceinline__ void run_f16_tiles(const _Float16* __restrict__ kb,
                                              const _Float16* __restrict__ vb, int rows,
                                              int64_t slot_base, int tb, int te,
                                              const half8 (&qB)[4], const AttnCommon& P,
                                              WaveState& st, int lane) {
  if (tb >= te) return;
  Tile A, B;
  load_f16_tile(kb, vb, kTile * tb, rows, lane, A);
  for (int ti = tb; ti < te; ti += 2) {
    if (ti + 1 < te) load_f16_tile(kb, vb, kTile * (ti + 1), rows, lane, B);
    tile_step(A, qB, slot_base + (int64_t)kTile * ti, kTile, P.R, P.scale_log2, st, lane);
    if (ti + 1 >= te) break;
    if (ti + 2 < te) load_f16_tile(kb, vb, kTile * (ti + 2), rows, lane, A);
    tile_step(B, qB, slot_base + (int64_t)kTile * (ti + 1), kTile, P.R, P.scale_log2, st, lane);
  }
}

// fp16 rows: the dense cache [B, KVH, L, 128] or the compacted sparse cache
// [B, KVH, sink+window, 128]; slot == row.
struct F16Src {
  const _Float16* k;
  const _Float16* v;
  int rows;
  __device__ __forceinline__ void run(int64_t pair, int wb, int we, const half8 (&qB)[4],
                                      const AttnCommon& P, WaveState& st, int lane) const {
    const size_t off = (size_t)pair * rows * kHeadDim;
    run_f16_tiles(k + off, v + off, rows, 0, wb, we, qB, P, st, lane);
  }
};

// KIVI cache: tile 0 = the sink group (quantized, `sink` real tokens), tiles
// 1..nwt = window-old groups (quantized), then the fp16 residual tiles.
struct KiviSrc {
  const _Float16* kres;
  const _Float16* vres;
  int res_rows;
  QRegion sinkq;   // base pointers (pair 0)
  QRegion winq;
  int sink;
  int win_tok;     // window - residual
  int nwt;         // win_tok / 32

  __device__ __forceinline__ void run(int64_t pair, int wb, int we, const half8 (&qB)[4],
                                      const AttnCommon& P, WaveState& st, int lane) const {
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
      RawQTile A, B;
      Tile T;
      load_q_tile(qb == 0 ? S : W, qb == 0 ? 0 : qb - 1, lane, A);
      for (int ti = qb; ti < qe; ti += 2) {
        if (ti + 1 < qe) load_q_tile(W, ti, lane, B);   // tile ti+1 >= 1: window-old tq = ti
        decode_q_tile(A, lane, T);
        tile_step(T, qB, ti == 0 ? 0 : sink + (int64_t)kTile * (ti - 1), ti == 0 ? sink : kTile,
                  P.R, P.scale_log2, st, lane);
        if (ti + 1 >= qe) break;
        if (ti + 2 < qe) load_q_tile(W, ti + 1, lane, A);
        decode_q_tile(B, lane, T);
        tile_step(T, qB, sink + (int64_t)kTile * ti, kTile, P.R, P.scale_log2, st, lane);
      }
    }
    const int fb = (wb > nq ? wb : nq) - nq, fe = we - nq;
    if (fb < fe) {
      const size_t off = (size_t)pair * res_rows * kHeadDim;
      run_f16_tiles(kres + off, vres + off, res_rows, sink + (int64_t)win_tok, fb, fe, qB, P, st,
                    lane);
    }
  }
};

template <class Src>
__global__ __launch_bounds__(kBlock) void attn_kernel(AttnCommon P, Src S) {
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
  const int wb = t0 + (nt * wave) / kWaves;
  const int we = t0 + (nt * (wave + 1)) / kWaves;

  WaveState st;
  wave_state_init(st);
  S.run(pair, wb, we, qB, P, st, lane);
  finish_block(P, st, pair, split, lane, wave);
}

// Log-sum-exp merge of the split partials; one workgroup per KV head.
__global__ __launch_bounds__(256) void merge_kernel(AttnCommon P) {
  const int64_t pair = blockIdx.x;
  const int64_t b = pair / P.KVH;
  const int kvh = (int)(pair % P.KVH);
  const size_t total = (size_t)P.pairs * P.n_splits * P.G;
  const float* wo = P.ws;
  const float* wm = P.ws + total * kHeadDim;
  const float* wl = wm + total;
  for (int e = threadIdx.x; e < P.G * kHeadDim; e += 256) {
    const int hn = e / kHeadDim, d = e % kHeadDim;
    const size_t base = (size_t)pair * P.n_splits * P.G + hn;
    float M = -INFINITY;
    for (int s = 0; s < P.n_splits; ++s) M = fmaxf(M, wm[base + (size_t)s * P.G]);
    const float Mu = (M == -INFINITY) ? 0.f : M;
    float L = 0.f, acc = 0.f;
    for (int s = 0; s < P.n_splits; ++s) {
      const size_t idx = base + (size_t)s * P.G;
      const float f = __builtin_amdgcn_exp2f(wm[idx] - Mu);
      L += wl[idx] * f;
      acc += wo[idx * kHeadDim + d] * f;
    }
    P.o[((size_t)b * P.H + (size_t)kvh * P.G + hn) * kHeadDim + d] = (_Float16)(acc / L);
  }
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------

// Split-K plan: aim for >= kTargetBlocks workgroups over the whole grid while
// giving every wave at least kMinTilesPerWave tiles.
constexpr int64_t kTargetBlocks = 2048;
constexpr int64_t kMinTilesPerWave = 4;

void plan_splits(int64_t pairs, int64_t n_tiles, int* splits, int* tps) {
  int64_t max_splits = n_tiles / (kWaves * kMinTilesPerWave);
  if (max_splits < 1) max_splits = 1;
  int64_t want = (kTargetBlocks + pairs - 1) / pairs;
  int64_t s = want < max_splits ? want : max_splits;
  if (s < 1) s = 1;
  int64_t t = (n_tiles + s - 1) / s;
  s = (n_tiles + t - 1) / t;
  *splits = (int)s;
  *tps = (int)t;
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
  int splits = 0, tps = 0;
  plan_splits(P.pairs, P.n_tiles, &splits, &tps);
  P.n_splits = splits;
  P.tiles_per_split = tps;
  if (splits > 1) {
    if (P.ws == nullptr) return KVDEC_E_WORKSPACE;
    if (ws_bytes < ws_bytes_for(P.pairs, splits, P.G)) return KVDEC_E_WORKSPACE;
  }
  const int64_t blocks = P.pairs * splits;
  if (blocks > 0x7fffffffLL) return KVDEC_E_SHAPE;
  hipLaunchKernelGGL(attn_kernel<Src>, dim3((unsigned)blocks), dim3(kBlock), 0, stream, P, S);
  int rc = launch_status();
  if (rc != KVDEC_OK || splits == 1) return rc;
  hipLaunchKernelGGL(merge_kernel, dim3((unsigned)P.pairs), dim3(256), 0, stream, P);
  return launch_status();
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

const char* kvdec_version(void) { return "kvdec 0.1 gfx950"; }

int kvdec_num_splits(int kind, int64_t B, int32_t KVH, int64_t n_slots) {
  if (B < 1 || KVH < 1 || n_slots < 1) return 1;
  int splits = 1, tps = 1;
  plan_splits(B * KVH, tiles_for(kind, n_slots), &splits, &tps);
  return splits;
}

size_t kvdec_workspace_bytes(int kind, int64_t B, int32_t H, int32_t KVH, int64_t n_slots,
                             int32_t D) {
  if (check_heads(B, H, KVH, D) != KVDEC_OK || n_slots < 1) return 0;
  const int splits = kvdec_num_splits(kind, B, KVH, n_slots);
  return ws_bytes_for(B * KVH, splits, H / KVH);
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
  P.R = SlotRanges{L, 0, 0};
  F16Src S{static_cast<const _Float16*>(k), static_cast<const _Float16*>(v), (int)L};
  return launch_attn(P, S, ws_bytes, static_cast<hipStream_t>(stream));
}

namespace {
SlotRanges sparse_ranges(int64_t seq_len, int32_t window, int32_t sink, int32_t layout) {
  const int64_t S = sink, W = window;
  SlotRanges R;
  R.va = seq_len < S ? seq_len : S;
  if (layout == KVDEC_LAYOUT_LINEAR) {
    const int64_t lo = 2 * S + W - seq_len;
    R.vb = lo > S ? lo : S;
    R.vc = S + W;
  } else {
    int64_t nwin = seq_len - S;
    if (nwin < 0) nwin = 0;
    if (nwin > W) nwin = W;
    R.vb = S;
    R.vc = S + nwin;
  }
  return R;
}
}  // namespace

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
