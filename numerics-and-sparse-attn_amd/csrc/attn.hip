// Split-K flash-decode kernels for gfx950: dense GQA decode, StreamingLLM
// sink+window decode and the fused KIVI-2bit decode, plus their C-ABI entry
// points (declared in include/kvdec.h).
//
// One workgroup of 8 waves = one (KV head, split) work unit.  The unit's
// 32-token tiles form a work queue: wave w takes tiles w and w + 8 at launch
// (their loads are the first thing the wave issues) and then claims further
// tiles from a counter in LDS, so waves that the SIMD arbiter serves later
// simply end up with fewer tiles.  Each wave streams its tiles through MFMA
// (all GQA query heads of the KV head at once, so each K/V byte is read
// once), keeps an online softmax, and the waves merge through LDS.  With one
// split the workgroup writes the fp16 output directly; otherwise it writes an
// fp32 partial (m, l, acc) and merge_kernel combines the splits.  At the
// benchmark shapes (B*KVH = 256 KV heads) every path runs in one pass.
//
// KIVI units have two queues: the fp16 residual tiles go to the first waves
// (one each while there are enough waves), the quantized tiles (window-old
// groups, then the sink group) to the others; a wave that finishes its
// residual tiles joins the quantized queue.  When a few quantized tiles are
// left over for the residual waves, the waves that take them hand their
// fp16 tiles to other residual waves, balancing the SIMDs' VALU load.

#include "kvdec_device.h"
#include "generic.h"
#include "kvdec_stream.h"
#include "kvdec.h"

#include <mutex>

using namespace kvdec;

// Workspace of kvdec_dense_decode_noalloc: the split-K partials of one call
// (fp32 [units][G][128] outputs, then [units][G] maxima and sums), in a
// file-scope device array that every GPU the library runs on holds until
// the process ends.  The launch plan splits only while there are fewer than
// 256 work units, so one call has at most 2 * 255 units of at most 16 heads:
// 510 * 16 * 130 * 4 = 4,243,200 bytes.
constexpr size_t kScratchBytes = (size_t)4160 << 10;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {

constexpr int kWaves = 8;                        // waves per workgroup
constexpr int kThreads = 64 * kWaves;

// Kernel clock, compiled only into the timing build (libkvdec_clock.so,
// -DKVDEC_CLOCK; the product library has none of it).  Every launch of an
// attention kernel gets slot `id` of a log armed by kvdec_clock_arm, with
// one record per workgroup (the first kClockWgs): thread 0 stores the GPU's
// constant-rate realtime counter and its core-clock counter when the
// workgroup starts and after its output store, with plain vector stores (no
// atomics, no shared address).  The host reduces a slot to the launch's
// first start and last end, i.e. its own duration with no profiler in the
// process, and the gap to the next launch; the two counters' ratio is the
// shader clock the launch ran at.
#ifdef KVDEC_CLOCK
constexpr int kClockWgs = 1024;
struct ClockRef {
  unsigned long long* log;
  int id;
};
__device__ __forceinline__ void clock_stamp(const ClockRef& c, int end) {
  if (c.log != nullptr && threadIdx.x == 0 && blockIdx.x < (unsigned)kClockWgs) {
    const unsigned long long t = __builtin_amdgcn_s_memrealtime();
    const unsigned long long k = __builtin_amdgcn_s_memtime();
    unsigned long long* rec = c.log + ((size_t)c.id * kClockWgs + blockIdx.x) * 4;
    rec[end] = t;
    rec[2 + end] = k;
  }
}
#define KVDEC_CLOCK_FIELD ClockRef clk;
#define CLOCK_STAMP(args, end) clock_stamp((args).clk, end)
#else
#define KVDEC_CLOCK_FIELD
#define CLOCK_STAMP(args, end) ((void)0)
#endif

struct AttnCommon {
  const _Float16* q;     // [B, H, 128]
  _Float16* o;           // [B, H, 128]
  float* ws;             // [pairs*splits*G*128] acc, then [..*G] m, then l
  int64_t pairs;
  int32_t H, KVH, G;
  int32_t n_tiles, tiles_per_split, n_splits;
  float scale_log2;
  SlotRanges R;
  KVDEC_CLOCK_FIELD
};

// LDS of a workgroup (bytes): two work counters, the per-wave max / sum of
// 16 heads, then one 8 KB slot per wave (K tile staging, KIVI tile staging,
// and at the end that wave's partial output rows).
constexpr int kLdsCtr = 0;
constexpr int kLdsM = 16;
constexpr int kLdsL = kLdsM + kWaves * kMaxGroup * 4;
constexpr int kLdsSlots = (kLdsL + kWaves * kMaxGroup * 4 + 255) & ~255;
constexpr int kLdsBytes = kLdsSlots + kWaves * kSlotBytes;
static_assert(kMaxGroup * kHeadDim * 4 <= kSlotBytes, "partial output must fit a wave slot");

// Everything a tile step needs besides the tile itself.
struct StepCtx {
  half8 qB[4];
  float scale_log2;     // logit factor of fp16 tiles
  float q_scale_log2;   // and of quantized tiles, with their K-scale factor
  uint32_t kmul;        // (fp16 pair 2^-e: Q's prescale, q_prescale_exp)
  SlotRanges R;
  char* lds;    // workgroup LDS base
  char* slot;   // this wave's slot
  int lane;
};

// Claim the next item of a dynamic queue (wave-uniform result).
__device__ __forceinline__ int grab(int* ctr, int lane) {
  int v = 0;
  if (lane == 0) v = atomicAdd(ctr, 1);
  return __builtin_amdgcn_readfirstlane(v);
}

// fp16 tiles [tile0, tile0 + n) of one region of one KV head; region row r
// is slot slot_base + r.
struct F16Items {
  typedef F16Raw Raw;
  rsrc_t rk, rv;
  int tile0, n, slot_base;
  int rot;        // queue item i is tile (i + rot) mod n
  SlotRanges R;   // loads of tiles with no valid slot are skipped
  __device__ __forceinline__ int tile(int i) const {
    const int j = i + rot;
    return tile0 + (j >= n ? j - n : j);
  }
  __device__ __forceinline__ void load(int i, Raw& X, int lane) const {
    const bool live = i < n && tile_any_valid(R, slot_base + kTile * tile(i));
    load_f16(rk, rv, live ? (uint32_t)tile(i) * kSlotBytes : kOOB, lane, X);
  }
  typedef WaveState State;
  __device__ __forceinline__ void step(int i, const Raw& X, State& st, const StepCtx& c) const {
    f16_tile_step(X, c.slot, c.qB, slot_base + kTile * tile(i), c.R, c.scale_log2, st, c.lane);
  }
  // The same, in a wave whose quantized-tile accumulators qs share st.m.
  __device__ __forceinline__ void step(int i, const Raw& X, State& st, QState& qs,
                                       const StepCtx& c) const {
    const int lane = c.lane;
    f16_tile_step(X, c.slot, c.qB, slot_base + kTile * tile(i), c.R, c.scale_log2, st, lane,
                  [&](float alpha) { q_state_rescale(qs, alpha, lane); });
  }
};

// The accumulators a quantized tile updates.
struct QRef {
  WaveState& st;
  QState& qs;
};

// Quantized tiles of one KV head: item i < nwt is window-old group i (slots
// sink + 32 i ..), item nwt is the sink group (`sink` real tokens at slots
// 0..sink-1; the cheapest tile, so it comes last in the queue).  MIXED: the
// wave also holds fp16-tile accumulators (and steps no fp16 tile after).
// PACK: the packed layout (query groups of at most kPackGroup heads).
template <bool MIXED, bool PACK>
struct QItems {
  typedef QTileRaw Raw;
  typedef QRef State;
  QRegion sinkq, winq;   // this KV head's sink group and window-old groups
  int n, sink;           // n = nwt + 1
  __device__ __forceinline__ void load(int i, Raw& X, int lane) const {
    const bool s = i == n - 1;
    QRegion Q;
    Q.kp = s ? sinkq.kp : winq.kp;
    Q.ks = s ? sinkq.ks : winq.ks;
    Q.kz = s ? sinkq.kz : winq.kz;
    Q.vp = s ? sinkq.vp : winq.vp;
    Q.vs = s ? sinkq.vs : winq.vs;
    Q.vz = s ? sinkq.vz : winq.vz;
    load_q_raw(Q, s ? 0 : i, i < n, lane, X, s ? sink : kTile);
  }
  __device__ __forceinline__ void step(int i, const Raw& X, State& s, const StepCtx& c) const {
    const bool sk = i == n - 1;
    q_tile_step<MIXED, PACK>(X, c.slot, c.qB, sk ? 0 : sink + kTile * i, sk ? sink : kTile, c.R,
                             c.q_scale_log2, s.st, s.qs, c.lane, c.kmul);
  }
};

// Two-deep prefetch ring over one queue.  The loads of both entries are in
// flight before the first step; every refill is issued unconditionally
// (items past the queue load nothing), which keeps the memory-counter waits
// of the steps exact.
template <class Items>
struct Ring {
  typename Items::Raw A, B;
  int ia, ib;
};

template <class Items>
__device__ __forceinline__ void ring_begin(const Items& it, Ring<Items>& r, int s0, int s1,
                                           int lane) {
  r.ia = s0;
  r.ib = s1;
  it.load(r.ia, r.A, lane);
  it.load(r.ib, r.B, lane);
}

// Static queue: the two entries are all the wave gets.
template <class Items>
__device__ __forceinline__ void ring_run_static(const Items& it, Ring<Items>& r,
                                                typename Items::State& st, const StepCtx& c) {
  if (r.ia < it.n) it.step(r.ia, r.A, st, c);
  if (r.ib < it.n) it.step(r.ib, r.B, st, c);
}

// Dynamic queue: refill each entry from the counter as soon as it is used.
template <class Items>
__device__ __forceinline__ void ring_run_dynamic(const Items& it, Ring<Items>& r, int* ctr,
                                                 typename Items::State& st, const StepCtx& c) {
  for (;;) {
    if (r.ia >= it.n) break;
    int nx = grab(ctr, c.lane);
    it.step(r.ia, r.A, st, c);
    r.ia = nx;
    it.load(r.ia, r.A, c.lane);
    if (r.ib >= it.n) break;
    nx = grab(ctr, c.lane);
    it.step(r.ib, r.B, st, c);
    r.ib = nx;
    it.load(r.ib, r.B, c.lane);
  }
}

// Publishing a wave's partial result for the workgroup merge: its max and
// softmax sum per head, and its unnormalised output rows [head][128 fp32] in
// its own LDS slot (16-byte chunks XOR-swizzled by head), so no wave waits
// to overwrite another's staging data.
__device__ __forceinline__ uint32_t row_off(int head, int chunk) {
  return (uint32_t)head * 512u + 16u * (uint32_t)(chunk ^ head);
}

// The fp16 output of 4 channels, stored non-temporally (written once and
// not read in this kernel: no L2 line is left dirty for the end-of-kernel
// release; KIVI W=256 5.83 -> 5.79 us, W=32 4.24 -> 4.20, sparse W=256
// 7.51 -> 7.48).
__device__ __forceinline__ void store_out4(_Float16* p, half4v h) {
  __builtin_nontemporal_store(__builtin_bit_cast(u32x2, h), reinterpret_cast<u32x2*>(p));
}

__device__ __forceinline__ void publish_ml(const AttnCommon& P, WaveState& st, char* lds, int lane,
                                           int wave) {
  st.l = group_sum(st.l);
  const int n = lane & 15, g = lane >> 4;
  if (n < P.G && g == 0) {
    reinterpret_cast<float*>(lds + kLdsM)[wave * kMaxGroup + n] = st.m;
    reinterpret_cast<float*>(lds + kLdsL)[wave * kMaxGroup + n] = st.l;
  }
}

// fp16-tile accumulators: O[jj][r] is channel 8(4g + r) + jj of head n.
__device__ __forceinline__ void publish_f(const AttnCommon& P, const WaveState& st, char* slot,
                                          int lane) {
  const int n = lane & 15, g = lane >> 4;
  if (n < P.G) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int c0 = 2 * (4 * g + r);
      float4v lo = float4v{st.O[0][r], st.O[1][r], st.O[2][r], st.O[3][r]} * st.fs;
      float4v hi = float4v{st.O[4][r], st.O[5][r], st.O[6][r], st.O[7][r]} * st.fs;
      *reinterpret_cast<float4v*>(slot + row_off(n, c0)) = lo;
      *reinterpret_cast<float4v*>(slot + row_off(n, c0 + 1)) = hi;
    }
  }
}

// Packed layout, remainder rows folded on the way out with VALU lane swaps:
// for rows r = 2p, 2p + 1 of an accumulator, v_permlane32_swap leaves
// (row 2p of lanes 0..31, row 2p + 1 of lanes 0..31) in one register and
// the same rows of lanes 32..63 in the other, so their sum holds, in lane
// L < 32, head 4g + 2p plus its remainder (lane L + 32) and, in lane
// L + 32, head 4g + 2p + 1 plus its remainder, g = L >> 4.  Each lane
// then writes its head's adjacent channel pair of every (grp, p): 8
// eight-byte writes of heads 0..7 (rows 8..15 are not written; the merges
// read heads only).  ADD as in publish_q.  The elements are copied to
// scalars before their bit casts: ROCm 7.2 clang compiles
// `__builtin_bit_cast` of a vector element (`v[i]`) as a read of element 0.
template <bool ADD>
__device__ __forceinline__ void publish_q_folded(const QState& qs, char* slot, int lane) {
  const int t = lane & 15, g = lane >> 4;
  const int hb = g < 2 ? 4 * g : 4 * (g - 2) + 1;
  float2v v[4][2];
  uint32_t off[4][2];
#pragma unroll
  for (int grp = 0; grp < 4; ++grp) {
    const int ch = q_state_channel(grp, 0, t);
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      off[grp][p] = row_off(hb + 2 * p, ch >> 2) + 4 * (ch & 3);
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const float fx = qs.O[2 * grp + c][2 * p], fy = qs.O[2 * grp + c][2 * p + 1];
        const auto sw = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, fx),
                                                         __builtin_bit_cast(uint32_t, fy), false, false);
        v[grp][p][c] = __builtin_bit_cast(float, (uint32_t)sw[0]) + __builtin_bit_cast(float, (uint32_t)sw[1]);
      }
    }
  }
  if (ADD) {
    float2v prev[4][2];
#pragma unroll
    for (int grp = 0; grp < 4; ++grp)
#pragma unroll
      for (int p = 0; p < 2; ++p) prev[grp][p] = *reinterpret_cast<const float2v*>(slot + off[grp][p]);
#pragma unroll
    for (int grp = 0; grp < 4; ++grp)
#pragma unroll
      for (int p = 0; p < 2; ++p) v[grp][p] += prev[grp][p];
  }
#pragma unroll
  for (int grp = 0; grp < 4; ++grp)
#pragma unroll
    for (int p = 0; p < 2; ++p) *reinterpret_cast<float2v*>(slot + off[grp][p]) = v[grp][p];
}

// Quantized-tile accumulators: lane (t, g) holds head 4g + r of channels
// q_state_channel(grp, 0..1, t) (adjacent) in QState::O[2 grp + 0..1]; each
// pair goes out as one 8-byte write.  All 16 head rows are written (rows of
// heads >= G stay inside the wave's slot and the merge never reads them), so
// no write is predicated.  ADD: the slot already holds this wave's fp16-tile
// rows (all reads are issued before any write, so the adds wait on LDS
// once).  PACK: publish_q_folded.
template <bool ADD, bool PACK = false>
__device__ __forceinline__ void publish_q(const QState& qs, char* slot, int lane) {
  if (PACK) {
    publish_q_folded<ADD>(qs, slot, lane);
    return;
  }
  const int t = lane & 15, g = lane >> 4;
  float2v v[4][4];
  uint32_t off[4][4];
#pragma unroll
  for (int grp = 0; grp < 4; ++grp) {
    const int ch = q_state_channel(grp, 0, t);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      off[grp][r] = row_off(4 * g + r, ch >> 2) + 4 * (ch & 3);
      v[grp][r] = float2v{qs.O[2 * grp][r], qs.O[2 * grp + 1][r]};
    }
  }
  if (ADD) {
    float2v prev[4][4];
#pragma unroll
    for (int grp = 0; grp < 4; ++grp)
#pragma unroll
      for (int r = 0; r < 4; ++r) prev[grp][r] = *reinterpret_cast<const float2v*>(slot + off[grp][r]);
#pragma unroll
    for (int grp = 0; grp < 4; ++grp)
#pragma unroll
      for (int r = 0; r < 4; ++r) v[grp][r] += prev[grp][r];
  }
#pragma unroll
  for (int grp = 0; grp < 4; ++grp)
#pragma unroll
    for (int r = 0; r < 4; ++r) *reinterpret_cast<float2v*>(slot + off[grp][r]) = v[grp][r];
}

// Barrier, then combine the waves' published partials into the output (one
// split) or the split's fp32 partial.
__device__ __forceinline__ void merge_out(const AttnCommon& P, char* lds, int64_t pair, int split) {
  __syncthreads();
  const float* sh_m = reinterpret_cast<const float*>(lds + kLdsM);
  const float* sh_l = reinterpret_cast<const float*>(lds + kLdsL);
  const int64_t b = pair / P.KVH;
  const int kvh = (int)(pair % P.KVH);
  const size_t total = (size_t)P.pairs * P.n_splits * P.G;
  // One thread per (head, 4-channel chunk): G * 32 <= 512 = kThreads.  All
  // LDS reads are issued before the first use.
  const int e = threadIdx.x;
  if (e >= P.G * 32) return;
  const int hn = e >> 5, ch = e & 31;
  float mw[kWaves], lw[kWaves];
  float4v ow[kWaves];
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    mw[w] = sh_m[w * kMaxGroup + hn];
    lw[w] = sh_l[w * kMaxGroup + hn];
    ow[w] = *reinterpret_cast<const float4v*>(lds + kLdsSlots + w * kSlotBytes + row_off(hn, ch));
  }
  float M = mw[0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) M = fmaxf(M, mw[w]);
  float L = 0.f;
  float4v acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    const float f = __builtin_amdgcn_exp2f(mw[w] - M);
    L += lw[w] * f;
    acc += ow[w] * f;
  }
  if (P.n_splits == 1) {
    const float inv = L > 0.f ? 1.0f / L : 0.f;   // L == 0: a sequence of length 0
    half4v h = {(_Float16)(acc[0] * inv), (_Float16)(acc[1] * inv), (_Float16)(acc[2] * inv),
                (_Float16)(acc[3] * inv)};
    store_out4(P.o + ((size_t)b * P.H + (size_t)kvh * P.G + hn) * kHeadDim + 4 * ch, h);
  } else {
    const size_t idx = ((size_t)pair * P.n_splits + split) * P.G + hn;
    *reinterpret_cast<float4v*>(P.ws + idx * kHeadDim + 4 * ch) = acc;
    if (ch == 0) {
      P.ws[total * kHeadDim + idx] = M;
      P.ws[total * kHeadDim + total + idx] = L;
    }
  }
  CLOCK_STAMP(P, 1);
}

// The fp16 queue of one unit: wave w takes items w and w + kWaves at launch
// and, when the queue is longer than 2 kWaves, claims more from the counter.
// A wave with at most one item issues only that item's loads: while the
// CU's memory pipeline is full every load instruction costs issue time,
// dummies included.
template <class Items, class Sync>
__device__ __forceinline__ void f16_queue(const AttnCommon& P, const Items& it, const SlotRanges& R,
                                          int wave, int lane, int* ctr, Sync&& sync, WaveState& st) {
  StepCtx c;
  const bool dyn = it.n > 2 * kWaves;
  if (!dyn && wave + kWaves >= it.n) {
    typename Items::Raw X;
    const bool has = wave < it.n;
    if (has) it.load(wave, X, lane);
    sync(c, false);
    c.R = R;
    if (has) it.step(wave, X, st, c);
  } else {
    Ring<Items> ring;
    ring_begin(it, ring, wave, wave + kWaves, lane);
    sync(c, dyn);
    c.R = R;
    if (dyn)
      ring_run_dynamic(it, ring, ctr, st, c);
    else
      ring_run_static(it, ring, st, c);
  }
  publish_ml(P, st, c.lds, lane, wave);
  publish_f(P, st, c.slot, lane);
}

// fp16 rows: the dense cache [B, KVH, L, 128] or the compacted sparse cache
// [B, KVH, sink+window, 128]; slot == row.
struct F16Src {
  const _Float16* k;
  const _Float16* v;
  int rows;

  __device__ __forceinline__ void init_counters(int* ctr) const { ctr[0] = 2 * kWaves; }

  // Issue the wave's first loads, then `sync` (workgroup barrier when the
  // queue is dynamic; fills the step context), then stream the queue.
  template <class Sync>
  __device__ __forceinline__ void process(int64_t pair, int split, const AttnCommon& P, int wave,
                                          int lane, int* ctr, Sync&& sync, WaveState& st) const {
    F16Items it;
    const size_t off = (size_t)pair * rows * kHeadDim;
    const uint32_t bytes = (uint32_t)rows * kRowBytes;
    it.rk = make_rsrc(k + off, bytes);
    it.rv = make_rsrc(v + off, bytes);
    it.tile0 = split * P.tiles_per_split;
    it.n = min(P.tiles_per_split, P.n_tiles - it.tile0);
    it.slot_base = 0;
    it.rot = 0;
    // Unit u starts its stream u tiles into its region (wrapping), so that
    // the 256 concurrent streams, whose regions start at multiples of the
    // same large stride, do not sweep the same address offsets in lockstep
    // (1.8% at L = 163840).
    if (it.n > 0) it.rot = (int)((uint64_t)pair % (uint64_t)it.n);
    it.R = P.R;
    f16_queue(P, it, P.R, wave, lane, ctr, sync, st);
  }
};

// A token-indexed fp16 cache with its own strides, optionally paged.  Token
// t of sequence b, KV head h sits at
//   base + page(b, t) * page_bytes + h * head_bytes + (t mod page_size) * row_bytes
// with page(b, t) = block_table[b][t / page_size]; without a table the
// "page" is the sequence (page(b, t) = b, page_size unbounded) holding
// `rows` rows.  A 32-token tile is two 16-row halves; page sizes are powers
// of two >= 16, so a half never straddles two pages, and each half gets a
// buffer resource of its own that ends at the half's last row (page ids
// outside [0, num_pages), rows past `rows` and halves with no valid token
// load zeros without touching memory).
typedef __attribute__((address_space(4))) const int32_t cint32;

struct PagedItems {
  typedef F16Raw Raw;
  const char* kb;      // this KV head's origin (+ the sequence's when untabled)
  const char* vb;
  cint32* bt;          // this sequence's block-table row, or null
  int64_t page_bytes;
  uint32_t row_bytes;
  int ps_log2, max_blocks;
  int64_t num_pages;
  int rows;            // untabled: rows of the sequence's region
  int tile0, n;
  SlotRanges R;

  __device__ __forceinline__ void load(int i, Raw& X, int lane) const {
    const int tile = tile0 + i;
    const bool live = i < n;
    rsrc_t rk[2], rv[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int tok = kTile * tile + 16 * h;
      bool ok = live && (tok < R.va || (tok + 16 > R.vb && tok < R.vc));
      int64_t off;
      int nr = 16;         // rows of this half inside the page / region
      if (bt) {
        const int idx = min(tok >> ps_log2, max_blocks - 1);   // always inside the row
        const int64_t page = bt[idx];
        ok = ok && page >= 0 && page < num_pages;
        off = page * page_bytes + (int64_t)(tok & ((1 << ps_log2) - 1)) * row_bytes;
      } else {
        off = (int64_t)tok * row_bytes;
        nr = min(16, rows - tok);
      }
      const uint32_t bytes = ok && nr > 0 ? (uint32_t)(nr - 1) * row_bytes + kRowBytes : 0u;
      rk[h] = make_rsrc(kb + off, bytes);
      rv[h] = make_rsrc(vb + off, bytes);
    }
    // the rows of load_f16: K rows 4i + g (half i / 4), V rows tau(g, j)
    // (half j / 4), at (row mod 16) * row_bytes inside the half
    const uint32_t t = lane & 15, g = lane >> 4;
#pragma unroll
    for (int k = 0; k < 8; ++k)
      X.k[k] = bload16(rk[k >> 2], ((4u * k + g) & 15u) * row_bytes + 16u * t);
#pragma unroll
    for (int j = 0; j < 8; ++j)
      X.v[j] = bload16(rv[j >> 2], (4u * g + (j & 3)) * row_bytes + 16u * t);
  }
  typedef WaveState State;
  __device__ __forceinline__ void step(int i, const Raw& X, State& st, const StepCtx& c) const {
    f16_tile_step(X, c.slot, c.qB, kTile * (tile0 + i), c.R, c.scale_log2, st, c.lane);
  }
};

// Per-sequence lengths over a paged or strided cache: dense attention over
// the first len(b) tokens, or (sparse) the sink + window rule over a
// compacted [sink + window] cache at position len(b).
struct PagedSrc {
  const char* k;
  const char* v;
  const int32_t* bt;     // [B, max_blocks] or null
  const int32_t* lens;   // [B] or null (every sequence max_len long)
  int64_t page_bytes, head_bytes;
  uint32_t row_bytes;
  int ps_log2, max_blocks;
  int64_t num_pages;
  int max_len;           // dense: lengths are clamped into [0, max_len]
  int rows;              // untabled: rows per (sequence, head) region
  int window, sink, layout;
  bool sparse;

  __device__ __forceinline__ void init_counters(int* ctr) const { ctr[0] = 2 * kWaves; }

  template <class Sync>
  __device__ __forceinline__ void process(int64_t pair, int split, const AttnCommon& P, int wave,
                                          int lane, int* ctr, Sync&& sync, WaveState& st) const {
    const int64_t b = pair / P.KVH;
    const int kvh = (int)(pair % P.KVH);
    int len = max_len;
    if (lens) len = min(max((int)((cint32*)lens)[b], 0), max_len);
    const SlotRanges R = sparse ? sparse_ranges(len, window, sink, layout) : SlotRanges{len, 0, 0};
    const int n_slots = sparse ? sink + window : len;
    const int tiles = (n_slots + kTile - 1) / kTile;
    PagedItems it;
    it.kb = k + (int64_t)kvh * head_bytes + (bt ? 0 : b * page_bytes);
    it.vb = v + (int64_t)kvh * head_bytes + (bt ? 0 : b * page_bytes);
    it.bt = bt ? (cint32*)bt + b * max_blocks : nullptr;
    it.page_bytes = page_bytes;
    it.row_bytes = row_bytes;
    it.rows = rows;
    it.ps_log2 = ps_log2;
    it.max_blocks = max_blocks;
    it.num_pages = num_pages;
    it.tile0 = split * P.tiles_per_split;
    it.n = max(0, min(P.tiles_per_split, tiles - it.tile0));
    it.R = R;
    f16_queue(P, it, R, wave, lane, ctr, sync, st);
  }
};

// KIVI cache: the fp16 residual (slots sink + win_tok ..) and the quantized
// sink and window-old groups.  Slot validity per MODE (separate
// instantiations, so the one-length kernel carries nothing of the others):
//   kOneRange  P.R for every sequence
//   kSeqLens   the _kv_indices rule at each sequence's own length lens[b]
//   kSeqStep   the same ring, first advanced by one token step in the
//              kernel's prologue (see KiviStepSrc)
//   kSeqRings  the residual is a ring of res_rows rows whose valid rows are
//              [start, start + count) mod res_rows, ring[b] = {start, count}
//              (a decode-time cache; every sink and window-old slot valid)
enum { kOneRange = 0, kSeqLens = 1, kSeqRings = 2, kSeqStep = 3 };

// kSeqStep: the decode-time cache's step arguments (nothing in the others).
template <int MODE>
struct KiviStepArgs {};
template <>
struct KiviStepArgs<kSeqStep> {
  StreamArgs a;
};

template <int MODE, bool PACK>
struct KiviSrcBase : KiviStepArgs<MODE> {
  static constexpr bool kPackQ = PACK;   // Q operand in the packed layout
  const _Float16* kres;
  const _Float16* vres;
  int res_rows;
  QRegion sinkq;   // base pointers (pair 0)
  QRegion winq;
  int sink;
  int win_tok;     // window - residual
  int nwt;         // win_tok / 32
  const int32_t* lens;   // kSeqLens: per-sequence lengths [B]; kSeqRings: {start, count} [B][2]
  int window;

  // Work split.  While the residual has at most kWaves tiles, the first nrw
  // waves take one residual tile each and the other nqw waves are quantized
  // waves.  The quantized queue is served in this order: one tile per
  // quantized wave, one extra tile per residual wave, a second tile per
  // quantized wave (all three loaded at launch), then dynamically.  A longer
  // residual makes every wave a residual wave with a dynamic residual queue,
  // and all quantized tiles dynamic.
  __device__ __forceinline__ int n_res() const { return (res_rows + kTile - 1) / kTile; }

  // kSeqStep, after the decode: the last of the sequence's KVH workgroups
  // to arrive records the step (every workgroup read the count at its
  // start, before it arrives)
  __device__ __forceinline__ void arrive(int64_t pair, const AttnCommon& P) const {
    if constexpr (MODE == kSeqStep) {
      const StreamArgs& a = this->a;
      const int64_t b = pair / P.KVH;
      if (threadIdx.x == kThreads - 1 && atomicAdd(a.arrive + b, 1) == P.KVH - 1) {
        const int n = max((int)((cint32*)a.appended)[b], 0);
        const bool act = !a.active || ((cint32*)a.active)[b] != 0;
        const RingStep rs = ring_step(n, act, a.residual, a.cap, a.nwg);
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
  __device__ __forceinline__ int n_res_waves() const { return min(n_res(), kWaves); }
  __device__ __forceinline__ int n_static_q() const {
    const int nrw = n_res_waves(), nqw = kWaves - nrw;
    return nqw == 0 ? 0 : 2 * nqw + nrw;
  }

  __device__ __forceinline__ void init_counters(int* ctr) const {
    ctr[0] = 2 * n_res_waves();
    ctr[1] = n_static_q();
  }

  // Residual waves and quantized waves run separate straight-line programs
  // (each issues its first loads, then `sync`, then streams), so the two
  // prefetch rings are never live at the same time.
  template <class Sync>
  __device__ __forceinline__ void process(int64_t pair, int, const AttnCommon& P, int wave,
                                          int lane, int* ctr, Sync&& sync, WaveState& st) const {
    const int nrw = n_res_waves();
    SlotRanges R = P.R;
    if constexpr (MODE == kSeqLens) {
      R = sparse_ranges(max((int)((cint32*)lens)[pair / P.KVH], 0), window, sink, KVDEC_LAYOUT_LINEAR);
    } else if constexpr (MODE == kSeqRings) {
      const int64_t b = pair / P.KVH;
      const int start = min(max((int)((cint32*)lens)[2 * b], 0), res_rows - 1);
      const int count = min(max((int)((cint32*)lens)[2 * b + 1], 0), res_rows);
      const int base = sink + win_tok, end = start + count;
      R = end <= res_rows ? SlotRanges{base, base + start, base + end}
                          : SlotRanges{base + end - res_rows, base + start, base + res_rows};
    } else if constexpr (MODE == kSeqStep) {
      // One token step of this (b, kv) head before the decode reads
      // anything: the token's K/V row written, the ring's oldest block
      // quantized into the oldest window-old slot when the ring fills, then
      // a workgroup barrier (the decode below reads both).  Every wave has
      // the sequence's count before the barrier; after the decode and its
      // merge, the last of the sequence's KVH workgroups to arrive records
      // the step and advances the count (arrive(), at the kernel's end: the
      // arrival atomic's round trip no longer holds back the last wave's
      // tile loads; the writes reach the next launch at the kernel
      // boundary).
      const StreamArgs& a = this->a;
      const int64_t b = pair / P.KVH;
      // the token's K/V row is loaded alongside the count (only the ring
      // row it goes to depends on the count): one memory round trip less
      // before the barrier
      const bool row_thread = threadIdx.x < 2 * kRowBytes / 16;
      const int i = threadIdx.x % (kRowBytes / 16);
      const bool isv = threadIdx.x >= kRowBytes / 16;
      u32x4 x = {0u, 0u, 0u, 0u};
      if (row_thread)
        x = *reinterpret_cast<const u32x4*>((isv ? a.v_new : a.k_new) + (size_t)pair * kHeadDim + 8 * i);
      const int n = max((int)((cint32*)a.appended)[b], 0);
      const bool act = !a.active || ((cint32*)a.active)[b] != 0;
      asm volatile("" ::"s"(n), "s"((int)act));   // both loaded before the barrier
      const RingStep rs = ring_step(n, act, a.residual, a.cap, a.nwg);
      if (rs.row >= 0 && row_thread)
        *reinterpret_cast<u32x4*>((isv ? a.v_ring : a.k_ring) + ((size_t)pair * a.cap + rs.row) * kHeadDim + 8 * i) = x;
      if (a.nwg > 0 && rs.blk >= 0) evict_block(a, pair, rs.blk, rs.slot, threadIdx.x, kThreads);
      __syncthreads();
      const int base = sink + win_tok, end = rs.start + rs.count;
      R = end <= res_rows ? SlotRanges{base, base + rs.start, base + end}
                          : SlotRanges{base + end - res_rows, base + rs.start, base + res_rows};
    }
    QRegion S = sinkq, Wq = winq;
    S.kp += (size_t)pair * 8 * kHeadDim;
    S.ks += (size_t)pair * kHeadDim;
    S.kz += (size_t)pair * kHeadDim;
    S.vp += (size_t)pair * 32 * 32;
    S.vs += (size_t)pair * 32 * 4;
    S.vz += (size_t)pair * 32 * 4;
    if (nwt > 0) {
      Wq.kp += (size_t)pair * (win_tok / 4) * kHeadDim;
      Wq.ks += (size_t)pair * (win_tok / 32) * kHeadDim;
      Wq.kz += (size_t)pair * (win_tok / 32) * kHeadDim;
      Wq.vp += (size_t)pair * win_tok * 32;
      Wq.vs += (size_t)pair * win_tok * 4;
      Wq.vz += (size_t)pair * win_tok * 4;
    }
    QItems<true, PACK> qit;   // tiles of a wave that also holds fp16-tile accumulators
    qit.sinkq = S;
    qit.winq = Wq;
    qit.n = 1 + nwt;
    qit.sink = sink;
    QItems<false, PACK> qonly;
    qonly.sinkq = S;
    qonly.winq = Wq;
    qonly.n = 1 + nwt;
    qonly.sink = sink;
    QState qs;
    q_state_init(qs);
    QRef qref{st, qs};
    const int nqw = kWaves - nrw;
    const bool dyn_q = qit.n > n_static_q();
    const bool dyn = dyn_q || (nqw == 0 && n_res() > 2 * nrw);   // any dynamic queue
    // Waves w and w + 4 share a SIMD, whose VALU the quantized steps
    // saturate.  When only e <= nrw / 2 residual waves get an extra
    // quantized tile (static queue), residual wave rw < e steps that tile
    // alone and residual wave e + rw takes its fp16 tile: no SIMD then
    // carries a quantized and an fp16 step more than the others.
    const int extra = nqw > 0 && !dyn_q ? max(qit.n - nqw, 0) : 0;
    const bool hand = extra > 0 && 2 * extra <= nrw;
    const int rw = wave, qw = wave - nrw;   // residual waves first
    StepCtx c;
    if (rw >= 0 && rw < nrw) {
      F16Items rit;
      const size_t roff = (size_t)pair * res_rows * kHeadDim;
      const uint32_t rbytes = (uint32_t)res_rows * kRowBytes;
      rit.rk = make_rsrc(kres + roff, rbytes);
      rit.rv = make_rsrc(vres + roff, rbytes);
      rit.tile0 = 0;
      rit.n = n_res();
      rit.slot_base = sink + win_tok;
      rit.rot = 0;
      rit.R = R;
      bool has_q = false;
      if (hand && rw < extra) {
        QTileRaw E;
        qonly.load(nqw + rw, E, lane);
        sync(c, true);
        if constexpr (MODE != kOneRange) c.R = R;
        qonly.step(nqw + rw, E, qref, c);
        publish_ml(P, st, c.lds, lane, wave);
        publish_q<false, PACK>(qs, c.slot, lane);
        return;
      }
      if (hand) {
        // loads issued after the barrier, behind every quantized tile's.
        // Only real tiles are loaded: while the CU's memory pipeline is
        // full, every load instruction costs issue time, dummies included.
        sync(c, true);
        if constexpr (MODE != kOneRange) c.R = R;
        if (rw - extra < extra) {
          Ring<F16Items> rring;
          ring_begin(rit, rring, rw, rw - extra, lane);
          ring_run_static(rit, rring, st, c);
        } else {
          // A single-tile wave holds its loads back ~0.6 us (24 x 64
          // clocks) so that the two-tile wave's loads enter the throttled
          // pipeline first and its two steps start earlier (measured: 6.79
          // -> 6.60 us per step at window 256).
          F16Raw X;
          __builtin_amdgcn_s_sleep(24);
          rit.load(rw, X, lane);
          rit.step(rw, X, st, c);
        }
      } else if (nqw > 0) {
        // one extra quantized tile (if there is one) and one residual tile.
        // The residual tile's loads are issued after the workgroup barrier,
        // behind the loads of every quantized tile: a CU serves its loads
        // roughly in issue order, and the quantized steps are the long ones.
        // The quantized tile goes first; the fp16 accumulators are still
        // zero then, so it is stepped without them.
        QTileRaw E;
        const int qe = nqw + rw;
        qonly.load(qe, E, lane);
        sync(c, true);
        if constexpr (MODE != kOneRange) c.R = R;
        F16Raw X;
        rit.load(rw, X, lane);
        if (qe < qonly.n) {
          qonly.step(qe, E, qref, c);
          has_q = true;
        }
        rit.step(rw, X, st, qs, c);
      } else {
        Ring<F16Items> rring;
        ring_begin(rit, rring, rw, rw + nrw, lane);
        sync(c, dyn);
        if constexpr (MODE != kOneRange) c.R = R;
        if (rit.n > 2 * nrw)
          ring_run_dynamic(rit, rring, ctr, st, c);
        else
          ring_run_static(rit, rring, st, c);
      }
      if (dyn_q) {
        const int s0 = grab(ctr + 1, lane);
        const int s1 = grab(ctr + 1, lane);
        if (s0 < qit.n) {
          Ring<QItems<true, PACK>> qring;
          ring_begin(qit, qring, s0, s1, lane);
          ring_run_dynamic(qit, qring, ctr + 1, qref, c);
          has_q = true;
        }
      }
      publish_ml(P, st, c.lds, lane, wave);
      publish_f(P, st, c.slot, lane);
      if (has_q) publish_q<true, PACK>(qs, c.slot, lane);
    } else {
      // Both entries are loaded even when the second is past the queue:
      // those loads return nothing but hold the quantized waves a little
      // longer before the barrier, which keeps the residual tiles' loads
      // behind every quantized tile's (measured: skipping them costs about
      // 0.5 us per step at window 256..288).
      Ring<QItems<false, PACK>> qring;
      ring_begin(qonly, qring, qw, qw + nqw + nrw, lane);
      sync(c, dyn || nqw > 0);
      if constexpr (MODE != kOneRange) c.R = R;
      if (dyn_q)
        ring_run_dynamic(qonly, qring, ctr + 1, qref, c);
      else
        ring_run_static(qonly, qring, qref, c);
      publish_ml(P, st, c.lds, lane, wave);
      publish_q<false, PACK>(qs, c.slot, lane);
    }
  }
};

template <bool PACK>
struct KiviSrc : KiviSrcBase<kOneRange, PACK> {};
template <bool PACK>
struct KiviVarSrc : KiviSrcBase<kSeqLens, PACK> {};
template <bool PACK>
struct KiviRingSrc : KiviSrcBase<kSeqRings, PACK> {};
// The decode-time cache with one ring state per sequence, stepped by one
// token in the same launch (kvdec_kivi_stream_step_decode).
template <bool PACK>
struct KiviStepSrc : KiviSrcBase<kSeqStep, PACK> {};

// Whether a source's kernel takes the Q operand in the packed layout.
// sources with an end-of-kernel hook (the KIVI sources: the decode-time
// cache's step bookkeeping)
template <class Src, class = void>
struct has_arrive : std::false_type {};
template <class Src>
struct has_arrive<Src, decltype((void)&Src::arrive)> : std::true_type {};

template <class Src, class = void>
struct packs_q {
  static constexpr bool value = false;
};
template <class Src>
struct packs_q<Src, decltype((void)Src::kPackQ)> {
  static constexpr bool value = Src::kPackQ;
};
// Whether a source has quantized tiles (the KIVI sources declare their Q
// layout), whose steps take the prescaled Q operand (q_prescale).
template <class Src, class = void>
struct has_qtiles : std::false_type {};
template <class Src>
struct has_qtiles<Src, decltype((void)Src::kPackQ)> : std::true_type {};

template <class Src>
__global__ __launch_bounds__(kThreads, 1) void attn_kernel(AttnCommon P, Src S) {
  extern __shared__ __align__(16) char lds[];
  CLOCK_STAMP(P, 0);
  // Bring every 64-byte line of the kernel arguments into the scalar cache
  // in one round trip: the compiler fetches the fields where they are first
  // used, which would otherwise cost a cache miss per line in series.
  {
    constexpr int kArgLines = (int)(sizeof(AttnCommon) + sizeof(Src) + 63) / 64;
    static_assert(kArgLines <= 8, "kernel arguments span more lines than are touched");
    const cint32* ka = (const cint32*)__builtin_amdgcn_kernarg_segment_ptr();
    int32_t x[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] = i < kArgLines ? ka[16 * i] : 0;
    asm volatile("" ::"s"(x[0]), "s"(x[1]), "s"(x[2]), "s"(x[3]), "s"(x[4]), "s"(x[5]));
    if constexpr (kArgLines > 6) asm volatile("" ::"s"(x[6]), "s"(x[7]));
  }
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int split = (int)(blockIdx.x % (unsigned)P.n_splits);
  const int64_t pair = blockIdx.x / (unsigned)P.n_splits;
  const int64_t b = pair / P.KVH;
  const int kvh = (int)(pair % P.KVH);

  // Q operand of this KV head's G query heads, loaded by every wave straight
  // into MFMA B-operand order (lane (n, g): head n, channels 32c + 8g .. +7)
  // before any tile load, so no wave waits on another to start computing.
  // Lanes of heads >= G read past the resource: zeros, no memory access.
  // In the packed layout lanes n and n + 8 both take head n & 7.
  half8 qB[4];
  {
    const int n = packs_q<Src>::value ? lane & 7 : lane & 15, g = lane >> 4;
    const rsrc_t rq = make_rsrc(P.q + ((size_t)b * P.H + (size_t)kvh * P.G) * kHeadDim,
                                (uint32_t)P.G * kRowBytes);
    const uint32_t qoff = n < P.G ? (uint32_t)n * kRowBytes + 16u * (uint32_t)g : kOOB;
#pragma unroll
    for (int cc = 0; cc < 4; ++cc)
      qB[cc] = as_h8(__builtin_amdgcn_raw_buffer_load_b128(rq, qoff + 64u * cc, 0, 0));
  }

  int* ctr = reinterpret_cast<int*>(lds + kLdsCtr);
  // Called exactly once by every wave, after its first tile loads.  With a
  // dynamic work queue (`barrier`, the same for every wave of the
  // workgroup) the counters are set and the workgroup synchronises.
  auto sync = [&](StepCtx& c, bool barrier) {
    if (barrier) {
      if (threadIdx.x == 0) S.init_counters(ctr);
      __syncthreads();
    }
#pragma unroll
    for (int cc = 0; cc < 4; ++cc) c.qB[cc] = qB[cc];
    c.scale_log2 = P.scale_log2;
    // quantized tiles: Q's power-of-two prescale joins their K scales (a
    // prescaled copy of the operand would not fit the registers here)
    c.q_scale_log2 = P.scale_log2;
    c.kmul = kOnePk;
    if constexpr (has_qtiles<Src>::value) {
      const int e = q_prescale_exp(qB);
      c.q_scale_log2 = scale_pow2(P.scale_log2, e);
      c.kmul = pow2_neg_pk(e);
    }
    c.R = P.R;
    c.lds = lds;
    c.slot = lds + kLdsSlots + wave * kSlotBytes;
    c.lane = lane;
  };

  WaveState st;
  wave_state_init(st);
  S.process(pair, split, P, wave, lane, ctr, sync, st);
  merge_out(P, lds, pair, split);
  if constexpr (has_arrive<Src>::value) S.arrive(pair, P);
}

// ---------------------------------------------------------------------------
// Lean single-pass kernels.  When a problem needs no split and every wave's
// share is at most two tiles, one workgroup of 8 waves per KV head runs a
// fixed program per wave: the KV head is the workgroup index (no division:
// query row b * H + kvh * G of the head is head * G), every per-head address
// is one multiply by a host-computed stride, and each wave issues all of
// its tile loads before it waits on anything (no work queue; Q comes
// through LDS, see q_quarter_load).  The tile steps, the published partials
// and the LDS merge are those of attn_kernel.  (The 16-wave KIVI kernel
// shares the prologue and the tile steps, with a work queue.)
// ---------------------------------------------------------------------------

struct LeanCommon {
  const _Float16* q;     // [heads][G][128]
  _Float16* o;
  float scale_log2;
  int G;
  SlotRanges R;
  KVDEC_CLOCK_FIELD
};

// The first part of every lean kernel: kernel-argument lines fetched in one
// scalar-cache round trip (lean_kernargs), then (lean_prologue) the Q
// operand of this KV head's G query heads in MFMA B-operand order (heads
// >= G read zeros without an access).
template <class Args>
__device__ __forceinline__ void lean_kernargs() {
  constexpr int kArgLines = (int)(sizeof(Args) + 63) / 64;
  static_assert(kArgLines <= 4, "kernel arguments span more lines than are touched");
  const cint32* ka = (const cint32*)__builtin_amdgcn_kernarg_segment_ptr();
  int32_t x[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) x[i] = i < kArgLines ? ka[16 * i] : 0;
  asm volatile("" ::"s"(x[0]), "s"(x[1]), "s"(x[2]), "s"(x[3]));
}

template <class Args, bool PACK = false>
__device__ __forceinline__ void lean_prologue(const LeanCommon& C, uint32_t head, int lane, half8 (&qB)[4]) {
  lean_kernargs<Args>();
  const int n = PACK ? lane & 7 : lane & 15, g = lane >> 4;   // PACK: lanes n, n + 8 take head n & 7
  const rsrc_t rq = make_rsrc(C.q + (size_t)head * C.G * kHeadDim, (uint32_t)C.G * kRowBytes);
  const uint32_t qoff = n < C.G ? (uint32_t)n * kRowBytes + 16u * (uint32_t)g : kOOB;
#pragma unroll
  for (int cc = 0; cc < 4; ++cc)
    qB[cc] = as_h8(__builtin_amdgcn_raw_buffer_load_b128(rq, qoff + 64u * cc, 0, 0));
}

// Q through LDS.  Instead of every wave loading its whole B operand (four
// 1 KiB load instructions per wave, all issued ahead of the tile loads, and
// a CU issues its loads one instruction at a time), quarter w of the KV
// head's 16 query rows (rows 4w .. 4w + 3, zeros past G) is loaded by wave
// w with one 1 KiB instruction and stored into the Q area once it has
// arrived; every wave reads its operand from there once the four quarters
// are in (KIVI W=256 6.08 -> 5.83 us, W=128 5.57 -> 5.24).  Rows are 272
// bytes apart, so that the operand reads (16 rows at one column) spread
// over the LDS banks.  A workgroup barrier instead of the readiness count
// measured slower (7.07 us at W=256): the waves that issue the residual
// tiles' loads reach it only once the memory pipeline has taken them all.
// The sparse fp16 kernel takes the same path (W=256 7.85 -> 7.55 us); the
// 16-wave KIVI kernel does not (W=1024 / 4096 0.6-0.8% slower with it), nor
// does attn_kernel (through its `sync`: the decode-time cache's W=256 step
// 7.14 -> 7.36 us, W=384 8.41 -> 8.64).
constexpr int kQPitch = kRowBytes + 16;
constexpr int kQAreaBytes = kMaxGroup * kQPitch;
constexpr int kQLdsBytes = kQAreaBytes + 16;   // + the readiness count
__device__ __forceinline__ u32x4 q_quarter_load(const LeanCommon& C, uint32_t head, int quarter, int lane) {
  const rsrc_t rq = make_rsrc(C.q + (size_t)head * C.G * kHeadDim, (uint32_t)C.G * kRowBytes);
  return bload16(rq, (uint32_t)(quarter * 4 * kRowBytes + 16 * lane));
}
__device__ __forceinline__ void q_quarter_store(char* qarea, int quarter, int lane, u32x4 v) {
  *reinterpret_cast<u32x4*>(qarea + (4 * quarter + (lane >> 4)) * kQPitch + 16 * (lane & 15)) = v;
}
// The Q area's readiness count (quarters stored), in the word after it:
// zeroed before a workgroup barrier that precedes every increment,
// incremented (release, one lane) by each wave that stored its quarter,
// polled (acquire) before the operand is read.  The poll is bounded: 2^16
// reads with an s_sleep 1 (~64 cycles) after each, ~4 x 10^6 cycles or
// ~2 ms (the four storing waves run unconditionally and their quarters
// arrive within microseconds, so it ends long before that).
__device__ __forceinline__ void q_quarter_ready(char* qarea, int lane) {
  if (lane == 0)
    __hip_atomic_fetch_add(reinterpret_cast<int*>(qarea + kQAreaBytes), 1, __ATOMIC_RELEASE,
                           __HIP_MEMORY_SCOPE_WORKGROUP);
}
// The operand read once the count is 4; should the bound ever run out, the
// operand is NaN, so the outputs show it instead of using a partial Q.
template <bool PACK>
__device__ __forceinline__ void q_operand_read(const char* qarea, int lane, half8 (&qB)[4]) {
  bool ready = false;
  for (int it = 0; it < (1 << 16); ++it) {
    if (__hip_atomic_load(reinterpret_cast<const int*>(qarea + kQAreaBytes), __ATOMIC_ACQUIRE,
                          __HIP_MEMORY_SCOPE_WORKGROUP) >= 4) {
      ready = true;
      break;
    }
    __builtin_amdgcn_s_sleep(1);
  }
  const int n = PACK ? lane & 7 : lane & 15, g = lane >> 4;   // PACK: lanes n, n + 8 take head n & 7
#pragma unroll
  for (int cc = 0; cc < 4; ++cc) qB[cc] = *reinterpret_cast<const half8*>(qarea + n * kQPitch + 64 * cc + 16 * g);
  if (!ready) {
#pragma unroll
    for (int cc = 0; cc < 4; ++cc) qB[cc] = as_h8(u32x4{0x7E007E00u, 0x7E007E00u, 0x7E007E00u, 0x7E007E00u});
  }
}

// LDS of a lean kernel with NW waves: the maxima and sums of every wave's
// partial (16 heads each), then one 8 KB slot per wave; the Q area follows.
// NW = 8 is attn_kernel's layout (kLdsM, kLdsL, kLdsSlots, kLdsBytes).
template <int NW>
struct LeanLds {
  static constexpr int kM = kLdsM;
  static constexpr int kL = kM + NW * kMaxGroup * 4;
  static constexpr int kSlots = (kL + NW * kMaxGroup * 4 + 255) & ~255;
  static constexpr int kBytes = kSlots + NW * kSlotBytes;
};
static_assert(LeanLds<kWaves>::kL == kLdsL && LeanLds<kWaves>::kSlots == kLdsSlots &&
                  LeanLds<kWaves>::kBytes == kLdsBytes,
              "the 8-wave lean layout is attn_kernel's");

// Barrier, then one thread per (head, 4 channels) combines the NW waves'
// published partials into the fp16 output rows of this KV head.  The waves
// of bit mask SKIP (never wave 0) have had their partials combined into
// another's.
template <int NW = kWaves, unsigned SKIP = 0>
__device__ __forceinline__ void lean_merge(const LeanCommon& C, const char* lds, uint32_t head) {
  typedef LeanLds<NW> Lds;
  static_assert((SKIP & 1u) == 0, "wave 0's partial is always read");
  __syncthreads();
  const float* sh_m = reinterpret_cast<const float*>(lds + Lds::kM);
  const float* sh_l = reinterpret_cast<const float*>(lds + Lds::kL);
  const int e = threadIdx.x;
  if (e >= C.G * 32) return;
  const int hn = e >> 5, ch = e & 31;
  float mw[NW], lw[NW];
  float4v ow[NW];
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    if ((SKIP >> w) & 1u) continue;
    mw[w] = sh_m[w * kMaxGroup + hn];
    lw[w] = sh_l[w * kMaxGroup + hn];
    ow[w] = *reinterpret_cast<const float4v*>(lds + Lds::kSlots + w * kSlotBytes + row_off(hn, ch));
  }
  float M = mw[0];
#pragma unroll
  for (int w = 1; w < NW; ++w)
    if (!((SKIP >> w) & 1u)) M = fmaxf(M, mw[w]);
  float L = 0.f;
  float4v acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    if ((SKIP >> w) & 1u) continue;
    const float f = __builtin_amdgcn_exp2f(mw[w] - M);
    L += lw[w] * f;
    acc += ow[w] * f;
  }
  const float inv = L > 0.f ? 1.0f / L : 0.f;
  half4v h = {(_Float16)(acc[0] * inv), (_Float16)(acc[1] * inv), (_Float16)(acc[2] * inv),
              (_Float16)(acc[3] * inv)};
  store_out4(C.o + ((size_t)head * C.G + hn) * kHeadDim + 4 * ch, h);
  CLOCK_STAMP(C, 1);
}

template <int NW = kWaves>
__device__ __forceinline__ void lean_publish_ml(int G, WaveState& st, char* lds, int lane, int wave) {
  st.l = group_sum(st.l);
  const int n = lane & 15, g = lane >> 4;
  if (n < G && g == 0) {
    reinterpret_cast<float*>(lds + LeanLds<NW>::kM)[wave * kMaxGroup + n] = st.m;
    reinterpret_cast<float*>(lds + LeanLds<NW>::kL)[wave * kMaxGroup + n] = st.l;
  }
}

__device__ __forceinline__ void lean_publish_f(int G, const WaveState& st, char* slot, int lane) {
  AttnCommon P{};
  P.G = G;
  publish_f(P, st, slot, lane);
}

// Waves 0..3 of a lean kernel whose quantized steps end well before its
// fp16 steps combine their four published partials into wave 0's while the
// other waves still step, so that the merge, on the critical path, reads
// one partial for the four (lean_merge SKIP 0xE).  Each wave counts itself
// in (`count`, zeroed before the workgroup's first barrier), waits for the
// four (a bounded poll; should it run out, the output is NaN), then wave w
// combines heads 2w, 2w + 1 (and 2w + 8, 2w + 9 when G > 8): one thread
// per (head, 4 channels).  The threads of a head sit in one wave, whose
// reads of the four partials are issued before its writes into wave 0's.
template <int NW>
__device__ __forceinline__ void quad_premerge(int G, char* lds, int* count, int lane, int wave) {
  typedef LeanLds<NW> Lds;
  if (lane == 0) __hip_atomic_fetch_add(count, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
  bool ready = false;
  for (int it = 0; it < (1 << 16); ++it) {
    if (__hip_atomic_load(count, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) >= 4) {
      ready = true;
      break;
    }
    __builtin_amdgcn_s_sleep(1);
  }
  float* sh_m = reinterpret_cast<float*>(lds + Lds::kM);
  float* sh_l = reinterpret_cast<float*>(lds + Lds::kL);
  for (int e = wave * 64 + lane; e < G * 32; e += 256) {
    const int hn = e >> 5, ch = e & 31;
    float mw[4], lw[4];
    float4v ow[4];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      mw[w] = sh_m[w * kMaxGroup + hn];
      lw[w] = sh_l[w * kMaxGroup + hn];
      ow[w] = *reinterpret_cast<const float4v*>(lds + Lds::kSlots + w * kSlotBytes + row_off(hn, ch));
    }
    float M = fmaxf(fmaxf(mw[0], mw[1]), fmaxf(mw[2], mw[3]));
    float L = 0.f;
    float4v acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float f = __builtin_amdgcn_exp2f(mw[w] - M);
      L += lw[w] * f;
      acc += ow[w] * f;
    }
    if (!ready) M = __builtin_nanf("");
    *reinterpret_cast<float4v*>(lds + Lds::kSlots + row_off(hn, ch)) = acc;
    if (ch == 0) {
      sh_m[hn] = M;
      sh_l[hn] = L;
    }
  }
}

// fp16 rows [heads][rows][128] (the compacted sink + window cache, or a
// short dense cache): wave w steps tiles w and w + 8 (at most 16 tiles).
struct F16LeanArgs {
  LeanCommon c;
  const _Float16* k;
  const _Float16* v;
  int rows;
};

template <bool TAIL>
__global__ __launch_bounds__(kThreads, 1) void f16_lean_kernel(F16LeanArgs A) {
  extern __shared__ __align__(16) char lds[];
  CLOCK_STAMP(A.c, 0);
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t head = blockIdx.x;
  lean_kernargs<F16LeanArgs>();
  // Q through LDS (waves 0..3 load a quarter each, the readiness count
  // zeroed before a barrier that precedes every increment)
  char* qarea = lds + kLdsBytes;
  if (threadIdx.x == 0) *reinterpret_cast<int*>(qarea + kQAreaBytes) = 0;
  __syncthreads();
  u32x4 qv = {0u, 0u, 0u, 0u};
  if (wave < 4) qv = q_quarter_load(A.c, head, wave, lane);
  half8 qB[4];
  // after the wave's first loads: its quarter stored, then the operand read
  // once all four are in (the store waits only for the quarter)
  auto q_in = [&](bool read) {
    if (wave < 4) {
      q_quarter_store(qarea, wave, lane, qv);
      q_quarter_ready(qarea, lane);
    }
    if (read) {
      q_operand_read<false>(qarea, lane, qB);
    }
  };
  char* slot = lds + kLdsSlots + wave * kSlotBytes;
  const size_t off = (size_t)head * A.rows * kHeadDim;
  const uint32_t bytes = (uint32_t)A.rows * kRowBytes;
  const rsrc_t rk = make_rsrc(A.k + off, bytes), rv = make_rsrc(A.v + off, bytes);
  const int n_tiles = (A.rows + kTile - 1) / kTile;
  // Tile i belongs to group i / 8 of n = min(8, n_tiles - 8 (i / 8)) tiles,
  // whose rows it takes four at a time, interleaved with the group's other
  // tiles (slot == row).  A tile with no valid slot loads nothing.
  auto rows = [&](int i) {
    const int grp = i / kWaves, nw = min(kWaves, n_tiles - kWaves * grp);
    return TileRows{kWaves * kTile * grp + 4 * (i % kWaves), 4 * nw};
  };
  auto live = [&](int i) { return i < n_tiles && tile_any_valid(A.c.R, rows(i)); };
  WaveState st;
  wave_state_init(st);
  if (wave + kWaves < n_tiles) {
    // 17 tiles (the host's condition: the last one at most 4 rows, rows
    // 512..515): the last wave also takes the tail, whose rows are its
    // first loads and its first step (they arrive early, while the two
    // full tiles stream in); only the tail's rows occupy registers
    // (a separate instantiation: the tail's registers would cost the
    // kernel of at most 16 tiles ~0.15 us per step)
    const bool tail = TAIL && n_tiles > 2 * kWaves && wave == kWaves - 1;
    u32x4 tk = {0u, 0u, 0u, 0u}, tv[4] = {};
    if (tail) {
      const uint32_t t = lane & 15, g = lane >> 4;
      const TileRows T = rows(2 * kWaves);
      const uint32_t base = live(2 * kWaves) ? (uint32_t)T.base * kRowBytes + 16u * t : kOOB;
      // rows past the region read zeros without an access
      tk = bload16(rk, base + g * kRowBytes);
#pragma unroll
      for (int j = 0; j < 4; ++j) tv[j] = bload16(rv, base + (4u * g + (uint32_t)j) * kRowBytes);
    }
    F16Raw X0, X1;
    load_f16(rk, rv, rows(wave), live(wave), 0u, lane, X0);
    load_f16(rk, rv, rows(wave + kWaves), live(wave + kWaves), 0u, lane, X1);
    q_in(true);
    if (tail) {
      F16Raw XT;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        XT.k[i] = i == 0 ? tk : u32x4{0u, 0u, 0u, 0u};
        XT.v[i] = i < 4 ? tv[i] : u32x4{0u, 0u, 0u, 0u};
      }
      f16_tile_step(XT, slot, qB, rows(2 * kWaves), A.c.R, A.c.scale_log2, st, lane);
    }
    f16_tile_step(X0, slot, qB, rows(wave), A.c.R, A.c.scale_log2, st, lane);
    f16_tile_step(X1, slot, qB, rows(wave + kWaves), A.c.R, A.c.scale_log2, st, lane);
  } else if (wave < n_tiles) {
    // a single tile in two phases: its V loads are issued once QK and the
    // softmax are done, so only the PV follows the last bytes to arrive
    F16Raw X;
    const TileRows T = rows(wave);
    const bool lv = live(wave);
    load_f16_k(rk, T, lv, 0u, lane, X);
    q_in(true);
    uint32_t valid;
    const TileProbs P = f16_tile_probs(X, slot, qB, T, A.c.R, A.c.scale_log2, st, lane, valid);
    load_f16_v(rv, T, after_probs(lv, P), 0u, lane, X);
    f16_tile_pv(X, P, valid, st);
  } else {
    q_in(false);   // no tile, but waves 0..3 still provide their quarter
  }
  lean_publish_ml(A.c.G, st, lds, lane, wave);
  lean_publish_f(A.c.G, st, slot, lane);
  lean_merge(A.c, lds, head);
}

// The fused KIVI decode with an fp16 residual of at most 128 rows (4 tiles;
// fewer when the window is shorter than the residual size) and at most
// 7 window-old groups: the quantized items are window-old groups 0..nwt-1
// and the sink group (item nwt, 4 real tokens, the cheapest step); waves
// 0..3 step items w and w + 4, waves 4..7 residual tiles 0..3 (if any).  Wave w and
// w + 4 share a SIMD.  Every load goes through a resource over a whole
// tensor with the KV head's (and group's) offset in the scalar offset
// field, so no per-head pointer arithmetic precedes the first load.  The
// residual loads are issued only after a workgroup barrier that the
// quantized waves reach once their loads are issued: a CU serves its loads
// roughly in issue order, so the quantized groups' data (their steps are
// the long ones) arrives first and the fp16 tiles stream in behind it.
struct KiviLeanArgs {
  LeanCommon c;
  const _Float16* kres;  // [heads][res_rows][128]
  const _Float16* vres;
  QRegion sinkq;         // [heads] groups
  QRegion winq;          // [heads][nwt] groups
  uint32_t res_bytes;    // whole-tensor sizes, each < 2^31
  int res_rows;          // residual rows per KV head (<= 128)
  uint32_t win_code_bytes, win_meta_bytes;
  int nwt;               // window-old groups (<= 7)
  int sink;
};

template <bool PACK>
__global__ __launch_bounds__(kThreads, 1) void kivi_lean_kernel(KiviLeanArgs A) {
  extern __shared__ __align__(16) char lds[];
  CLOCK_STAMP(A.c, 0);
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t head = blockIdx.x;
  lean_kernargs<KiviLeanArgs>();
  char* qarea = lds + kLdsBytes;
  half8 qB[4];
  char* slot = lds + kLdsSlots + wave * kSlotBytes;
  const int nwt = A.nwt;
  WaveState st;
  wave_state_init(st);
  if (wave < 4) {
    // Q quarter w first, then the groups' loads: the wait for the quarter
    // (after the barrier, before its store) leaves them in flight
    const u32x4 qv = q_quarter_load(A.c, head, wave, lane);
    QState qs;
    q_state_init(qs);
    const int n_q = nwt + 1;
    // item i < nwt: window-old group i; item nwt: the sink group
    auto load = [&](int i, QTileRaw& X) {
      const bool sk = i == nwt;
      const QTensors T = sk ? q_sink_tensors(A.sinkq, head, A.sink)
                            : q_tensors(A.winq, A.win_code_bytes, A.win_meta_bytes);
      load_q_group(T, sk ? 0u : head * (uint32_t)nwt + (uint32_t)i, i < n_q, lane, X);
    };
    // A wave whose second item is the sink group loads and steps it first:
    // its few bytes arrive early, and the wave's last step is no longer the
    // sink's next to a residual wave's step on the same SIMD (W=256: 0.5 to
    // 1.8% faster over three A/B runs).
    const bool sink_first = wave + 4 == nwt;
    const int i0 = sink_first ? wave + 4 : wave, i1 = sink_first ? wave : wave + 4;
    QTileRaw X0, X1;
    load(i0, X0);
    load(i1, X1);
    __syncthreads();
    q_quarter_store(qarea, wave, lane, qv);
    q_quarter_ready(qarea, lane);
    q_operand_read<PACK>(qarea, lane, qB);
    const float sl2 = q_prescale(qB, A.c.scale_log2);
    auto step = [&](int i, const QTileRaw& X) {
      const bool sk = i == nwt;
      q_tile_step<false, PACK>(X, slot, qB, sk ? 0 : A.sink + kTile * i, sk ? A.sink : kTile, A.c.R,
                               sl2, st, qs, lane);
    };
    if (i0 < n_q) step(i0, X0);
    if (i1 < n_q) step(i1, X1);
    lean_publish_ml(A.c.G, st, lds, lane, wave);
    publish_q<false, PACK>(qs, slot, lane);
  } else {
    // residual tile w - 4: rows 32 (w - 4) .. + 31 (interleaving the four
    // tiles' rows, or issuing V after the softmax, measured slower here:
    // these tiles' data arrives last and their steps end the kernel)
    const int tile = wave - 4;
    const int slot0 = A.sink + kTile * nwt + kTile * tile;
    const rsrc_t rk = make_rsrc(A.kres, A.res_bytes), rv = make_rsrc(A.vres, A.res_bytes);
    const uint32_t soff = head * (uint32_t)(A.res_rows * kRowBytes);
    // residual rows past res_rows (the next KV head's, or past the tensor)
    // are slots past the window: masked, their V rows read as zeros
    const bool has = tile * kTile < A.res_rows;
    const uint32_t base = has && tile_any_valid(A.c.R, slot0) ? (uint32_t)tile * kSlotBytes : kOOB;
    F16Raw X;
    if (wave == 4 && lane == 0) *reinterpret_cast<int*>(qarea + kQAreaBytes) = 0;
    __syncthreads();
    if (has) load_f16(rk, rv, base, soff, lane, X);
    q_operand_read<PACK>(qarea, lane, qB);
    if (has) f16_tile_step(X, slot, qB, slot0, A.c.R, A.c.scale_log2, st, lane);
    lean_publish_ml(A.c.G, st, lds, lane, wave);
    lean_publish_f(A.c.G, st, slot, lane);
  }
  lean_merge(A.c, lds, head);
}

// The lean KIVI kernel for exactly 4 window-old groups (W = 256 with
// R = 128) with a ninth wave: waves 0..3 step window-old group w, wave 4 the
// sink group, waves 5..8 residual tiles 0..3.  In the 8-wave kernel the
// fifth quantized item (the sink group) falls to wave 0, whose two steps in
// series (each ~1.3 us for a single wave on its SIMD) end the kernel last;
// here the sink step runs in its own wave beside them (wave 4 shares SIMD 0
// with waves 0 and 8; 138 VGPRs fit three waves per SIMD).  Measured per
// step (interleaved A/B, two boxes): 5.78 -> 5.67 us and 5.79 -> 5.69 us.
// The sink wave is wave 4 rather than the last one: waves start in order,
// ~0.05 us apart, and the residual waves issue their loads only after the
// barrier anyway, while the sink's step, sharing its SIMD with a window-old
// group's, published last when it started last (5.63 -> 5.47 us, with the
// four window-old partials combined early by quad_premerge).
// With fewer window-old groups every quantized item already has a wave of
// its own and the extra wave only costs (W = 160: 5.22 -> 5.43 us).
constexpr int kLean9Waves = 9;
typedef LeanLds<kLean9Waves> Lean9Lds;

template <bool PACK>
__global__ __launch_bounds__(64 * kLean9Waves, 1) void kivi_lean9_kernel(KiviLeanArgs A) {
  extern __shared__ __align__(16) char lds[];
  CLOCK_STAMP(A.c, 0);
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t head = blockIdx.x;
  lean_kernargs<KiviLeanArgs>();
  char* qarea = lds + Lean9Lds::kBytes;
  int* premerge_count = reinterpret_cast<int*>(qarea + kQAreaBytes + 12);
  half8 qB[4];
  char* slot = lds + Lean9Lds::kSlots + wave * kSlotBytes;
  const int nwt = A.nwt;
  WaveState st;
  wave_state_init(st);
  if (wave <= 4) {
    // quantized: Q quarter w first (waves 0..3), then the group's loads
    u32x4 qv = {0u, 0u, 0u, 0u};
    if (wave < 4) qv = q_quarter_load(A.c, head, wave, lane);
    QState qs;
    q_state_init(qs);
    const bool sk = wave == 4;
    const bool has = sk || wave < nwt;
    const QTensors T = sk ? q_sink_tensors(A.sinkq, head, A.sink)
                          : q_tensors(A.winq, A.win_code_bytes, A.win_meta_bytes);
    QTileRaw X;
    load_q_group(T, sk ? 0u : head * (uint32_t)nwt + (uint32_t)wave, has, lane, X);
    __syncthreads();
    if (wave < 4) {
      q_quarter_store(qarea, wave, lane, qv);
      q_quarter_ready(qarea, lane);
    }
    q_operand_read<PACK>(qarea, lane, qB);
    const float sl2 = q_prescale(qB, A.c.scale_log2);
    if (has)
      q_tile_step<false, PACK>(X, slot, qB, sk ? 0 : A.sink + kTile * wave, sk ? A.sink : kTile, A.c.R,
                               sl2, st, qs, lane);
    lean_publish_ml<kLean9Waves>(A.c.G, st, lds, lane, wave);
    publish_q<false, PACK>(qs, slot, lane);
    if (wave < 4) quad_premerge<kLean9Waves>(A.c.G, lds, premerge_count, lane, wave);
  } else {
    // residual tile w - 5, its loads after the barrier (as in kivi_lean_kernel)
    const int tile = wave - 5;
    const int slot0 = A.sink + kTile * nwt + kTile * tile;
    const rsrc_t rk = make_rsrc(A.kres, A.res_bytes), rv = make_rsrc(A.vres, A.res_bytes);
    const uint32_t soff = head * (uint32_t)(A.res_rows * kRowBytes);
    const bool has = tile * kTile < A.res_rows;
    const uint32_t base = has && tile_any_valid(A.c.R, slot0) ? (uint32_t)tile * kSlotBytes : kOOB;
    F16Raw X;
    if (wave == 5 && lane == 0) {
      *reinterpret_cast<int*>(qarea + kQAreaBytes) = 0;
      *premerge_count = 0;
    }
    __syncthreads();
    if (has) load_f16(rk, rv, base, soff, lane, X);
    q_operand_read<PACK>(qarea, lane, qB);
    if (has) f16_tile_step(X, slot, qB, slot0, A.c.R, A.c.scale_log2, st, lane);
    lean_publish_ml<kLean9Waves>(A.c.G, st, lds, lane, wave);
    lean_publish_f(A.c.G, st, slot, lane);
  }
  // waves 0..3 are in wave 0's partial
  lean_merge<kLean9Waves, 0xEu>(A.c, lds, head);
}

// The decode-time KIVI cache's decode over rings of 5 tiles (residual 128)
// with at most 4 window-old groups, as a lean kernel of 10 waves: waves
// 0..3 window-old slots 0..3, wave 4 the sink group (as in
// kivi_lean9_kernel), waves 5..9 ring tiles 0..4.  MODE kRingOne: one ring state for every sequence (c.R);
// kRingSeqs: per-sequence states ring[b] = {start, count}; kRingStep: one
// token step per sequence first (kvdec_kivi_stream_step_decode), from the
// sequence's count.  The three share the work split and the merge, so
// step + decode and append followed by decode give bit-identical outputs.
// kRingOne reads only the ring rows its state makes valid.  In the other
// modes nothing waits on the state before the loads are issued: the ring
// waves load their whole tiles, the state (the sink wave reads the count
// after the first barrier and passes it on through LDS; kRingSeqs reads
// ring[b]) decides only what is masked.  The ring tiles' loads follow the
// workgroup barrier that the quantized waves reach once theirs are issued,
// so the quantized groups (the long steps) get their data first.  The
// step's memory operations are off the critical path:
//   * the token's K/V row: every ring wave loads it from k_new / v_new
//     before its tile, and the wave whose tile holds the row puts it in
//     place of the ring's old content at its uses in the step (the tile's
//     loads read the ring before the row is stored there) and, once its
//     step is done, stores it into the ring for the later steps;
//   * an eviction (every 32nd step of a sequence): the wave of the slot that
//     receives the ring's oldest block quantizes it itself (the quantizers'
//     exact group formulas), stores the group for the later steps and
//     steps it from its LDS slot;
//   * the bookkeeping: the sink wave takes the workgroup's arrival number
//     once it has published its group; the last of the sequence's KVH
//     workgroups to arrive records the step after the merge.
// The general kernel (attn_kernel<KiviStepSrc>) read the count first, then
// wrote the row and quantized an evicted block with every thread, then
// passed a barrier before its first decode load, and took its arrival
// number after its merge.
enum { kRingOne = 0, kRingSeqs = 1, kRingStep = 2 };
struct StepLeanArgs {
  LeanCommon c;
  const _Float16* k_new;   // [pairs][128]
  const _Float16* v_new;
  _Float16* k_ring;        // [pairs][cap][128]
  _Float16* v_ring;
  QRegion sinkq;           // [pairs] groups
  QRegion winq;            // [pairs][nwg] groups (written on eviction)
  int32_t* appended;       // [B] tokens appended since each sequence's prefill
  const int32_t* active;   // [B] or null (all)
  int32_t* arrive;         // [B] workgroups arrived this step (0 between launches)
  int32_t* plan;           // [B][3] {row, evict block, evict slot} of this step
  int32_t* ring;           // [B][2] kRingStep: {start, count} after this step; kRingSeqs: the states
  uint32_t ring_bytes;     // pairs * cap * 256 (< 2^31)
  uint32_t win_code_bytes, win_meta_bytes;
  int nwg, sink, residual, cap, KVH;
};
constexpr int kStepWaves = 10;
typedef LeanLds<kStepWaves> StepLds;

// Quantize ring rows [32 blk, +32) of KV head `pair` into window-old slot
// `slot` by one wave (the group formulas of evict_block, so the same
// codes): lane L takes K channels 2L, 2L + 1 and V token L / 2, groups
// 2 (L % 2) and 2 (L % 2) + 1.  The group is stored for the later steps;
// its scales, zeros and V codes come back in X in the lane layout of a
// loaded group, and its K code bytes go straight to the wave's LDS slot
// (`stage_k`, called after the rest of the tile is staged).
struct EvictK {
  uint32_t rows[8];   // K code bytes of channels 2L, 2L + 1 for code rows 0..7
};
__device__ __forceinline__ void evict_group(const StepLeanArgs& A, uint32_t pair, int blk, int slot, int lane,
                                            QTileRaw& X, EvictK& kb) {
  const size_t row0 = (size_t)pair * A.cap + (size_t)blk * kTile;
  const _Float16* kr = A.k_ring + row0 * kHeadDim;
  const _Float16* vr = A.v_ring + row0 * kHeadDim;
  const size_t g = (size_t)pair * A.nwg + slot;
  // K: channels 2L, 2L + 1 over the block's 32 tokens
  float x0[kTile], x1[kTile];
#pragma unroll
  for (int t = 0; t < kTile; ++t) {
    const half2v h = *reinterpret_cast<const half2v*>(kr + (size_t)t * kHeadDim + 2 * lane);
    x0[t] = (float)h[0];
    x1[t] = (float)h[1];
  }
  QParams q0, q1;
  const u32x2 c0 = quant_group(x0, q0), c1 = quant_group(x1, q1);
  uint8_t* kp = const_cast<uint8_t*>(A.winq.kp) + g * (kTile / 4) * kHeadDim;
#pragma unroll
  for (int p = 0; p < kTile / 4; ++p) {
    const uint32_t b0 = (c0[p >> 2] >> (8 * (p & 3))) & 0xffu, b1 = (c1[p >> 2] >> (8 * (p & 3))) & 0xffu;
    kb.rows[p] = b0 | (b1 << 8);
    *reinterpret_cast<uint16_t*>(kp + p * kHeadDim + 2 * lane) = (uint16_t)kb.rows[p];
  }
  const half2v ks = {(_Float16)q0.s, (_Float16)q1.s}, kz = {(_Float16)q0.z, (_Float16)q1.z};
  X.ks = __builtin_bit_cast(uint32_t, ks);
  X.kz = __builtin_bit_cast(uint32_t, kz);
  *reinterpret_cast<uint32_t*>(const_cast<_Float16*>(A.winq.ks) + g * kHeadDim + 2 * lane) = X.ks;
  *reinterpret_cast<uint32_t*>(const_cast<_Float16*>(A.winq.kz) + g * kHeadDim + 2 * lane) = X.kz;
  // V: token t, channel groups g0, g0 + 1
  const int t = lane >> 1, g0 = 2 * (lane & 1);
  float y0[kTile], y1[kTile];
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    const half8 h = as_h8(*reinterpret_cast<const u32x4*>(vr + (size_t)t * kHeadDim + kTile * g0 + 8 * c));
#pragma unroll
    for (int e = 0; e < 8; ++e) (c < 4 ? y0 : y1)[8 * (c & 3) + e] = (float)h[e];
  }
  QParams q2, q3;
  const u32x2 c2 = quant_group(y0, q2), c3 = quant_group(y1, q3);
  X.vc = u32x4{c2[0], c2[1], c3[0], c3[1]};
  const size_t tok = g * kTile + t;
  *reinterpret_cast<u32x4*>(const_cast<uint8_t*>(A.winq.vp) + tok * (kHeadDim / 4) + 8 * g0) = X.vc;
  const half2v vs = {(_Float16)q2.s, (_Float16)q3.s}, vz = {(_Float16)q2.z, (_Float16)q3.z};
  X.vs = __builtin_bit_cast(uint32_t, vs);
  X.vz = __builtin_bit_cast(uint32_t, vz);
  *reinterpret_cast<uint32_t*>(const_cast<_Float16*>(A.winq.vs) + tok * 4 + g0) = X.vs;
  *reinterpret_cast<uint32_t*>(const_cast<_Float16*>(A.winq.vz) + tok * 4 + g0) = X.vz;
}
__device__ __forceinline__ void evict_stage_k(const EvictK& kb, char* slot, int lane) {
#pragma unroll
  for (int p = 0; p < kTile / 4; ++p) {
    *reinterpret_cast<uint16_t*>(slot + kQsK + p * kQsKRow + 2 * lane) = (uint16_t)kb.rows[p];
    *reinterpret_cast<uint16_t*>(slot + kQsK4 + p * kQsKRow + 2 * lane) = (uint16_t)(kb.rows[p] >> 4);
  }
}

// f16_tile_step of a ring tile whose row rr (rr < 0: none) is replaced by
// the token's row, chunk t of K and V in kn, vn of lane (t, g).  The row is
// put in at its uses (K: written over the staged row in the wave's LDS slot;
// V: selected in the PV operand), so the step still waits for the tile's
// loads one at a time: replacing the registers up front would wait for all
// of them first.
__device__ __forceinline__ void ring_tile_step(const F16Raw& X, char* slot, const half8 (&qB)[4], int slot0,
                                               const SlotRanges& R, float scale_log2, WaveState& st, int lane,
                                               int rr, const u32x4& kn, const u32x4& vn) {
  const uint32_t t = lane & 15, g = lane >> 4;
#pragma unroll
  for (int i = 0; i < 8; ++i)
    *reinterpret_cast<u32x4*>(slot + kslot_off(4u * i + g, t)) = X.k[i];
  if (rr >= 0 && (int)g == (rr & 3)) *reinterpret_cast<u32x4*>(slot + kslot_off((uint32_t)rr, t)) = kn;
  auto kop = [&](int blk, int c) {
    return *reinterpret_cast<const u32x4*>(slot + kslot_off(16u * blk + t, 4u * c + g));
  };
  // V row rr is tau(gv, jv): X.v[jv] of the lanes g == gv
  const int jv = rr >= 0 ? 4 * (rr >> 4) + (rr & 3) : -1;
  const bool vl = rr >= 0 && (int)g == ((rr >> 2) & 3);
  auto vrow = [&](int w, int j) { return j == jv && vl ? vn[w] : X.v[j][w]; };
  const TileRows T{slot0, 4};
  if (tile_fully_valid(R, T)) {
    tile_body<true>(kop, vrow, 0u, qB, scale_log2, st, NoRescale());
  } else {
    const uint32_t valid = tile_valid_bits(R, T, kTile, lane);
    tile_body<false>(kop, [&](int w, int j) { return ((valid >> j) & 1u) ? vrow(w, j) : 0u; }, valid, qB,
                     scale_log2, st, NoRescale());
  }
}

template <bool PACK, int MODE>
__global__ __launch_bounds__(64 * kStepWaves, 1) void kivi_ring_kernel(StepLeanArgs A) {
  extern __shared__ __align__(16) char lds[];
  CLOCK_STAMP(A.c, 0);
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t pair = blockIdx.x;
  lean_kernargs<StepLeanArgs>();
  const uint32_t b = pair / (uint32_t)A.KVH;
  char* qarea = lds + StepLds::kBytes;
  // kRingStep: the sequence's count and activity, read from memory by the
  // sink wave alone once the barrier below has passed (a scalar load in
  // front of the barrier would hold every wave's loads back by its round
  // trip) and passed to the other waves through LDS: (n << 1 | active) and
  // a readiness flag, polled with a bound.  Since no other wave of the
  // workgroup reads the count from memory, the sink wave may take the
  // workgroup's arrival number at any point after it has it.
  int* cnt_word = reinterpret_cast<int*>(qarea + kQAreaBytes + 4);
  int* cnt_flag = reinterpret_cast<int*>(qarea + kQAreaBytes + 8);
  int* premerge_count = reinterpret_cast<int*>(qarea + kQAreaBytes + 12);
  auto count_from_lds = [&](int& n, bool& act) {
    bool ready = false;
    for (int it = 0; it < (1 << 16); ++it) {
      if (__hip_atomic_load(cnt_flag, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) != 0) {
        ready = true;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    const int v = ready ? *cnt_word : 0;   // (never runs out: the sink wave always publishes)
    n = v >> 1;
    act = (v & 1) != 0;
  };
  // kRingSeqs: the sequence's ring state, clamped (read after the barrier)
  auto seq_state = [&]() {
    const int s0 = min(max((int)((cint32*)A.ring)[2 * b], 0), A.cap - 1);
    const int c0 = min(max((int)((cint32*)A.ring)[2 * b + 1], 0), A.cap);
    return RingStep{-1, -1, -1, s0, c0};
  };
  half8 qB[4];
  char* slot = lds + StepLds::kSlots + wave * kSlotBytes;
  const int nwg = A.nwg;
  WaveState st;
  wave_state_init(st);
  auto ranges = [&](const RingStep& rs) {
    if constexpr (MODE == kRingOne) return A.c.R;
    const int base = A.sink + kTile * nwg, end = rs.start + rs.count;
    return end <= A.cap ? SlotRanges{base, base + rs.start, base + end}
                        : SlotRanges{base + end - A.cap, base + rs.start, base + A.cap};
  };
  // kRingStep, the sink wave: its arrival number, and the step it took
  int prev = 0, n = 0;
  bool act = false;
  RingStep rs = {};
  if (wave <= 4) {
    u32x4 qv = {0u, 0u, 0u, 0u};
    if (wave < 4) qv = q_quarter_load(A.c, pair, wave, lane);
    QState qs;
    q_state_init(qs);
    const bool sk = wave == 4;
    const bool has = sk || wave < nwg;
    const QTensors T = sk ? q_sink_tensors(A.sinkq, pair, A.sink)
                          : q_tensors(A.winq, A.win_code_bytes, A.win_meta_bytes);
    QTileRaw X;
    load_q_group(T, sk ? 0u : pair * (uint32_t)nwg + (uint32_t)wave, has, lane, X);
    __syncthreads();
    if (MODE == kRingStep && sk) {
      n = max((int)((cint32*)A.appended)[b], 0);
      act = !A.active || ((cint32*)A.active)[b] != 0;
      if (lane == 0) {
        *cnt_word = n << 1 | (act ? 1 : 0);
        __hip_atomic_store(cnt_flag, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
      }
    }
    if (wave < 4) {
      q_quarter_store(qarea, wave, lane, qv);
      q_quarter_ready(qarea, lane);
    }
    q_operand_read<PACK>(qarea, lane, qB);
    const float sl2 = q_prescale(qB, A.c.scale_log2);
    if constexpr (MODE == kRingStep) {
      if (!sk) count_from_lds(n, act);
      rs = ring_step(n, act, A.residual, A.cap, nwg);
    } else if constexpr (MODE == kRingSeqs) {
      rs = seq_state();
    }
    const SlotRanges R = ranges(rs);
    if (has) {
      if (MODE == kRingStep && !sk && rs.blk >= 0 && rs.slot == wave) {
        // this slot receives the ring's oldest block this step
        __builtin_amdgcn_s_waitcnt(0);   // the slot's old group has been read
        EvictK kb;
        evict_group(A, pair, rs.blk, rs.slot, lane, X, kb);
        const float slack = q_tile_stage(X, slot, lane);
        evict_stage_k(kb, slot, lane);
        q_tile_consume<false, PACK>(slot, qB, A.sink + kTile * wave, kTile, R, sl2, slack, st, qs,
                                    lane);
      } else {
        q_tile_step<false, PACK>(X, slot, qB, sk ? 0 : A.sink + kTile * wave, sk ? A.sink : kTile, R,
                                 sl2, st, qs, lane);
      }
    }
    lean_publish_ml<kStepWaves>(A.c.G, st, lds, lane, wave);
    publish_q<false, PACK>(qs, slot, lane);
    if (wave < 4) quad_premerge<kStepWaves>(A.c.G, lds, premerge_count, lane, wave);
    if (MODE == kRingStep && sk && lane == 0) {
      // the workgroup's arrival, once the sink wave has published: a wait
      // for the atomic's return waits for every memory operation the wave
      // issued before it (the compiler's waits in the publish count the
      // atomic too), and the return comes after the CU's loads in flight.
      // The offset is a zero the compiler cannot prove uniform, so the
      // atomic stays one lane's and its result is first needed at the end
      // (a uniform-address atomic is rewritten to broadcast its result at
      // once, waiting for the round trip there).
      int zero;
      asm volatile("v_mov_b32 %0, 0" : "=v"(zero));
      prev = atomicAdd(A.arrive + b + zero, 1);
    }
  } else {
    // ring tile r: rows 32 r .. 32 r + 31 of this head's ring, all of them
    // loaded (the count decides which are valid), with the token's row
    const int r = wave - 5;
    const rsrc_t rk = make_rsrc(A.k_ring, A.ring_bytes), rv = make_rsrc(A.v_ring, A.ring_bytes);
    const uint32_t soff = pair * (uint32_t)(A.cap * kRowBytes);
    F16Raw X;
    if (wave == 5 && lane == 0) {
      *reinterpret_cast<int*>(qarea + kQAreaBytes) = 0;
      *cnt_flag = 0;
      *premerge_count = 0;
    }
    const int t = lane & 15, g = lane >> 4;
    u32x4 kn = {0u, 0u, 0u, 0u}, vn = {0u, 0u, 0u, 0u};
    if (MODE == kRingStep) {
      kn = *reinterpret_cast<const u32x4*>(A.k_new + (size_t)pair * kHeadDim + 8 * t);
      vn = *reinterpret_cast<const u32x4*>(A.v_new + (size_t)pair * kHeadDim + 8 * t);
    }
    // the ring tile's loads follow the barrier that the quantized waves
    // reach once theirs are issued (as in kivi_lean_kernel: their long
    // steps get their data first).  kRingOne knows the ring state from its
    // arguments and reads only the valid rows; the other modes learn it
    // from memory and load the whole tile rather than wait for it.
    __syncthreads();
    if constexpr (MODE == kRingOne)
      load_f16(rk, rv, (uint32_t)r * kSlotBytes, soff, A.c.R, A.sink + kTile * nwg + kTile * r, lane, X);
    else
      load_f16(rk, rv, (uint32_t)r * kSlotBytes, soff, lane, X);
    q_operand_read<PACK>(qarea, lane, qB);
    if constexpr (MODE == kRingStep) {
      count_from_lds(n, act);
      rs = ring_step(n, act, A.residual, A.cap, nwg);
    } else if constexpr (MODE == kRingSeqs) {
      rs = seq_state();
    }
    const SlotRanges R = ranges(rs);
    // the token's row replaces the ring's old content of its tile row
    const bool owner = MODE == kRingStep && rs.row >= 0 && rs.row / kTile == r;
    if constexpr (MODE == kRingStep)
      ring_tile_step(X, slot, qB, A.sink + kTile * nwg + kTile * r, R, A.c.scale_log2, st, lane,
                     owner ? rs.row % kTile : -1, kn, vn);
    else
      f16_tile_step(X, slot, qB, A.sink + kTile * nwg + kTile * r, R, A.c.scale_log2, st, lane);
    lean_publish_ml<kStepWaves>(A.c.G, st, lds, lane, wave);
    lean_publish_f(A.c.G, st, slot, lane);
    if (owner && g < 2) {
      // and stored into the ring for the later steps (lanes g = 0 the K
      // chunks, g = 1 the V chunks; no wave of this launch reads the row
      // from memory: an evicted block never holds it).  After the step: a
      // store in flight among the tile's loads makes the compiler wait for
      // all of them, and the store, at the step's first use of the tile.
      _Float16* dst = (g == 0 ? A.k_ring : A.v_ring) + ((size_t)pair * A.cap + rs.row) * kHeadDim + 8 * t;
      *reinterpret_cast<u32x4*>(dst) = g == 0 ? kn : vn;
    }
  }
  // waves 0..3 are in wave 0's partial
  lean_merge<kStepWaves, 0xEu>(A.c, lds, pair);
  // the step's record, by the last of the sequence's workgroups to arrive
  // (after the merge: the arrival atomic's round trip does not hold the
  // merge's barrier back)
  if (MODE == kRingStep && wave == 4 && lane == 0 && prev == A.KVH - 1) {
    A.arrive[b] = 0;
    A.appended[b] = n + (act ? 1 : 0);
    A.plan[3 * b] = rs.row;
    A.plan[3 * b + 1] = rs.blk;
    A.plan[3 * b + 2] = rs.blk >= 0 ? rs.slot : -1;
    A.ring[2 * b] = rs.start;
    A.ring[2 * b + 1] = rs.count;
  }
}

// The fused KIVI decode past the lean kernel's windows (more than 7
// window-old groups), for query groups of at most kPackGroup heads (the
// packed layout) and a residual of at most 128 rows: 16 waves, four per
// SIMD, so that the VALU the quantized steps saturate always has another
// wave's instructions to issue (a tile-step microbenchmark: 2043 cycles
// per tile per SIMD at 4 waves per SIMD and one tile in flight per wave,
// 2270 at 2 waves and two in flight; 128 VGPRs leave room for one).  Waves
// 0..11 start on window-old groups 0..11, waves 12..15 on residual tiles
// 0..3; the rest of the quantized items (window-old groups, then the sink
// group) are claimed from an LDS counter, the claim and the next item's
// loads issued before the current item's step.  A residual wave publishes
// its fp16 partial to its own area before it joins the quantized queue, so
// the merge combines 20 partials.
// Below 12 window-old groups every quantized wave steps at most one group
// and the 8-wave kernel is faster (measured per step, W = 384 / 480 / 512:
// 8.11 / 8.96 / 9.89 us there, 8.45 / 9.42 / 9.22 us here).
constexpr int kWideMinGroups = 12;
constexpr int kWideWaves = 16;
constexpr int kWideThreads = 64 * kWideWaves;
constexpr int kWideQWaves = 12;                  // waves that start on quantized items
constexpr int kWideParts = kWideWaves + 4;       // + the residual waves' fp16 partials
constexpr int kWideLdsCtr = 0;
constexpr int kWideLdsM = 16;
constexpr int kWideLdsL = kWideLdsM + kWideParts * kMaxGroup * 4;
constexpr int kWideLdsSlots = (kWideLdsL + kWideParts * kMaxGroup * 4 + 255) & ~255;
constexpr int kWideF16Bytes = kPackGroup * kHeadDim * 4;   // an fp16 partial of <= 8 heads
constexpr int kWideLdsF16 = kWideLdsSlots + kWideWaves * kSlotBytes;
constexpr int kWideLdsBytes = kWideLdsF16 + 4 * kWideF16Bytes;
static_assert(kWideLdsBytes <= 160 * 1024, "wide kernel LDS");

__device__ __forceinline__ void wide_publish_ml(int G, WaveState& st, char* lds, int lane, int part) {
  st.l = group_sum(st.l);
  const int n = lane & 15, g = lane >> 4;
  if (n < G && g == 0) {
    reinterpret_cast<float*>(lds + kWideLdsM)[part * kMaxGroup + n] = st.m;
    reinterpret_cast<float*>(lds + kWideLdsL)[part * kMaxGroup + n] = st.l;
  }
}

template <bool PACK>
__global__ __launch_bounds__(kWideThreads, 1) void kivi_wide_kernel(KiviLeanArgs A) {
  extern __shared__ __align__(16) char lds[];
  CLOCK_STAMP(A.c, 0);
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t head = blockIdx.x;
  half8 qB[4];
  lean_prologue<KiviLeanArgs, PACK>(A.c, head, lane, qB);
  char* slot = lds + kWideLdsSlots + wave * kSlotBytes;
  int* ctr = reinterpret_cast<int*>(lds + kWideLdsCtr);
  const int nwt = A.nwt, n_q = nwt + 1;
  const QTensors Tw = q_tensors(A.winq, A.win_code_bytes, A.win_meta_bytes);
  const QTensors Ts = q_sink_tensors(A.sinkq, head, A.sink);
  // item i < nwt: window-old group i; item nwt: the sink group
  auto load = [&](int i, QTileRaw& X) {
    const bool sk = i == nwt;
    load_q_group(sk ? Ts : Tw, sk ? 0u : head * (uint32_t)nwt + (uint32_t)i, i < n_q, lane, X);
  };
  if (threadIdx.x == 0) *ctr = kWideQWaves;
  QTileRaw X;
  int i = n_q;
  if (wave < kWideQWaves) {
    i = wave;
    load(i, X);
  }
  __syncthreads();
  if (wave >= kWideQWaves) {
    // residual tile r: rows 32 r .. + 31; rows past res_rows are slots past
    // the window (masked, V read as zeros)
    const int r = wave - kWideQWaves;
    const int slot0 = A.sink + kTile * nwt + kTile * r;
    const rsrc_t rk = make_rsrc(A.kres, A.res_bytes), rv = make_rsrc(A.vres, A.res_bytes);
    const uint32_t soff = head * (uint32_t)(A.res_rows * kRowBytes);
    const bool has = r * kTile < A.res_rows;
    const uint32_t base = has && tile_any_valid(A.c.R, slot0) ? (uint32_t)r * kSlotBytes : kOOB;
    WaveState sf;
    wave_state_init(sf);
    if (has) {
      F16Raw F;
      load_f16(rk, rv, base, soff, lane, F);
      f16_tile_step(F, slot, qB, slot0, A.c.R, A.c.scale_log2, sf, lane);
    }
    wide_publish_ml(A.c.G, sf, lds, lane, kWideWaves + r);
    lean_publish_f(A.c.G, sf, lds + kWideLdsF16 + r * kWideF16Bytes, lane);
    i = grab(ctr, lane);
    load(i, X);
  }
  // the quantized items' Q operand, prescaled once the wave's first group
  // load is in flight (before it, the wait for Q would hold the load back)
  const float sl2 = q_prescale(qB, A.c.scale_log2);
  WaveState st;   // the quantized items' max and sum (st.O stays zero)
  wave_state_init(st);
  QState qs;
  q_state_init(qs);
  // window-old groups; the sink group (claimed last, at most 16 tokens: the
  // host's condition) is stepped after the loop, so that the loop holds one
  // tile body (with two, the registers of 4 waves per SIMD do not suffice)
  while (i < nwt) {
    const float slack = q_tile_stage(X, slot, lane);
    const int nx = grab(ctr, lane);
    load(nx, X);
    q_tile_body<false, false, PACK>(slot, qB, A.sink + kTile * i, kTile, A.c.R, sl2, slack, st, qs,
                                    lane);
    i = nx;
  }
  if (i == nwt) {
    const float slack = q_tile_stage(X, slot, lane);
    q_tile_body<false, true, PACK>(slot, qB, 0, A.sink, A.c.R, sl2, slack, st, qs, lane);
  }
  wide_publish_ml(A.c.G, st, lds, lane, wave);
  publish_q<false, PACK>(qs, slot, lane);

  // merge: one thread per (head, 4 channels) over the 16 quantized partials
  // (remainders already folded in) and the 4 fp16 partials
  __syncthreads();
  const int e = threadIdx.x;
  if (e >= A.c.G * 32) return;
  const float* sh_m = reinterpret_cast<const float*>(lds + kWideLdsM);
  const float* sh_l = reinterpret_cast<const float*>(lds + kWideLdsL);
  const int hn = e >> 5, ch = e & 31;
  float mw[kWideParts];
#pragma unroll
  for (int p = 0; p < kWideParts; ++p) mw[p] = sh_m[p * kMaxGroup + hn];
  float M = mw[0];
#pragma unroll
  for (int p = 1; p < kWideParts; ++p) M = fmaxf(M, mw[p]);
  float L = 0.f;
  float4v acc = {0.f, 0.f, 0.f, 0.f};
  // four partials at a time (their reads issued together)
#pragma unroll
  for (int p0 = 0; p0 < kWideParts; p0 += 4) {
    float lw[4];
    float4v ow[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int p = p0 + j;
      lw[j] = sh_l[p * kMaxGroup + hn];
      const char* part = p < kWideWaves ? lds + kWideLdsSlots + p * kSlotBytes
                                        : lds + kWideLdsF16 + (p - kWideWaves) * kWideF16Bytes;
      ow[j] = *reinterpret_cast<const float4v*>(part + row_off(hn, ch));
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int p = p0 + j;
      const float f = __builtin_amdgcn_exp2f(mw[p] - M);
      L += lw[j] * f;
      acc += ow[j] * f;
    }
  }
  const float inv = L > 0.f ? 1.0f / L : 0.f;
  half4v h = {(_Float16)(acc[0] * inv), (_Float16)(acc[1] * inv), (_Float16)(acc[2] * inv),
              (_Float16)(acc[3] * inv)};
  store_out4(A.c.o + ((size_t)head * A.c.G + hn) * kHeadDim + 4 * ch, h);
  CLOCK_STAMP(A.c, 1);
}

// Streaming read of `n16` 16-byte words, for the measurement of a decode
// step's floor at the same launch scale (a workgroup reads one contiguous
// share, 512 threads x 4 loads in flight, non-temporal as the decode's
// streams): every workgroup writes the XOR of its share, so the reads stay.
__global__ __launch_bounds__(kThreads) void read_probe_kernel(const u32x4* src, int64_t n16, uint32_t* sink) {
  const int64_t per = (n16 + gridDim.x - 1) / gridDim.x;
  const int64_t b = (int64_t)blockIdx.x * per;
  const int64_t e = b + per < n16 ? b + per : n16;
  u32x4 acc = {0u, 0u, 0u, 0u};
  for (int64_t i = b + threadIdx.x; i < e; i += 4 * kThreads) {
#pragma unroll
    for (int u = 0; u < 4; ++u)
      if (i + u * kThreads < e) acc ^= __builtin_nontemporal_load(src + i + u * kThreads);
  }
  uint32_t v = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
  __shared__ uint32_t red[kWaves];
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v ^= (uint32_t)__shfl_xor((int)v, off);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t r = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) r ^= red[w];
    sink[blockIdx.x] = r;
  }
}

// The read probe's sweep form: THREADS threads per workgroup, each
// workgroup one contiguous share; KIND 0 global non-temporal loads, 1 plain
// global loads, 2 buffer loads with the decode streams' non-temporal hint,
// 3 buffer loads without it; UPFRONT: each thread issues up to 16 loads
// before it uses any (else 4 in flight per loop turn).  The dynamic LDS the
// launch reserves is not touched: it only gives the launch a decode
// kernel's LDS footprint.
template <int KIND>
__device__ __forceinline__ u32x4 probe_load(const u32x4* src, rsrc_t r, int64_t i, int64_t b, int64_t e) {
  if constexpr (KIND == 0) return i < e ? __builtin_nontemporal_load(src + i) : u32x4{0u, 0u, 0u, 0u};
  if constexpr (KIND == 1) return i < e ? src[i] : u32x4{0u, 0u, 0u, 0u};
  const uint32_t off = i < e ? (uint32_t)(i - b) * 16u : kOOB;
  if constexpr (KIND == 2) return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 2);
  return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
}

template <int THREADS, int KIND, bool UPFRONT>
__global__ __launch_bounds__(THREADS) void read_probe2_kernel(const u32x4* src, int64_t n16, uint32_t* sink) {
  const int64_t per = (n16 + gridDim.x - 1) / gridDim.x;
  const int64_t b = (int64_t)blockIdx.x * per;
  const int64_t e = b + per < n16 ? b + per : n16;
  const rsrc_t r = make_rsrc(src + (b < n16 ? b : 0), e > b ? (uint32_t)((e - b) * 16) : 0u);
  u32x4 acc = {0u, 0u, 0u, 0u};
  constexpr int kIn = UPFRONT ? 16 : 4;
  for (int64_t i = b + threadIdx.x; i < e; i += kIn * THREADS) {
    u32x4 x[kIn];
#pragma unroll
    for (int u = 0; u < kIn; ++u) x[u] = probe_load<KIND>(src, r, i + u * THREADS, b, e);
#pragma unroll
    for (int u = 0; u < kIn; ++u) acc ^= x[u];
  }
  uint32_t v = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
  __shared__ uint32_t red[THREADS / 64];
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v ^= (uint32_t)__shfl_xor((int)v, off);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t q = 0;
#pragma unroll
    for (int w = 0; w < THREADS / 64; ++w) q ^= red[w];
    sink[blockIdx.x] = q;
  }
}

template <int THREADS, int KIND>
void launch_probe2(bool upfront, unsigned blocks, size_t lds, hipStream_t st, const u32x4* src, int64_t n16,
                   uint32_t* sink) {
  if (upfront)
    hipLaunchKernelGGL((read_probe2_kernel<THREADS, KIND, true>), dim3(blocks), dim3(THREADS), lds, st, src, n16,
                       sink);
  else
    hipLaunchKernelGGL((read_probe2_kernel<THREADS, KIND, false>), dim3(blocks), dim3(THREADS), lds, st, src, n16,
                       sink);
}

template <int THREADS>
void launch_probe2_kind(int kind, bool upfront, unsigned blocks, size_t lds, hipStream_t st, const u32x4* src,
                        int64_t n16, uint32_t* sink) {
  switch (kind) {
    case 0: launch_probe2<THREADS, 0>(upfront, blocks, lds, st, src, n16, sink); break;
    case 1: launch_probe2<THREADS, 1>(upfront, blocks, lds, st, src, n16, sink); break;
    case 2: launch_probe2<THREADS, 2>(upfront, blocks, lds, st, src, n16, sink); break;
    default: launch_probe2<THREADS, 3>(upfront, blocks, lds, st, src, n16, sink); break;
  }
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
  __builtin_nontemporal_store((_Float16)(L > 0.f ? acc / L : 0.f),
                              P.o + ((size_t)b * P.H + (size_t)kvh * P.G + hn) * kHeadDim + d);
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------

// Launch plan: one workgroup per (KV head, split).  Splits are added only
// while there are fewer work units than CUs (kTargetUnits), and only while
// every unit keeps at least one tile per wave.
constexpr int64_t kTargetUnits = 256;
constexpr int64_t kMinTilesPerUnit = kWaves;

struct Plan {
  int splits, tps;
};

Plan make_plan(int64_t pairs, int64_t n_tiles) {
  int64_t s = (kTargetUnits + pairs - 1) / pairs;
  const int64_t cap = n_tiles / kMinTilesPerUnit;
  if (s > cap) s = cap;
  if (s < 1) s = 1;
  int64_t t = (n_tiles + s - 1) / s;
  s = (n_tiles + t - 1) / t;
  Plan p;
  p.splits = (int)s;
  p.tps = (int)t;
  return p;
}

int64_t tiles_for(int kind, int64_t n_slots) {
  if (kind == KVDEC_KIND_KIVI) return 1 + (n_slots + kTile - 1) / kTile;
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

// The timing build's launch counter: each attention launch takes the next
// slot of the armed log (slots are reused cyclically), none while disarmed.
#ifdef KVDEC_CLOCK
std::mutex g_clock_mu;
unsigned long long* g_clock_log = nullptr;
int g_clock_slots = 0, g_clock_next = 0;
ClockRef next_clock() {
  std::lock_guard<std::mutex> lock(g_clock_mu);
  ClockRef c{g_clock_log, 0};
  if (g_clock_log != nullptr) {
    c.id = g_clock_next;
    g_clock_next = g_clock_next + 1 == g_clock_slots ? 0 : g_clock_next + 1;
  }
  return c;
}
#define SET_CLOCK(args) ((args).clk = next_clock())
#else
#define SET_CLOCK(args) ((void)0)
#endif

template <class Src>
int launch_attn(AttnCommon P, const Src& S, bool kivi, size_t ws_bytes, hipStream_t stream) {
  // The KIVI plan never splits: its quantized and residual regions are
  // addressed per KV head, and the windows it serves are short.
  const Plan plan = kivi ? Plan{1, P.n_tiles} : make_plan(P.pairs, P.n_tiles);
  P.n_splits = plan.splits;
  P.tiles_per_split = plan.tps;
  if (plan.splits > 1) {
    if (P.ws == nullptr) return KVDEC_E_WORKSPACE;
    if (ws_bytes < ws_bytes_for(P.pairs, plan.splits, P.G)) return KVDEC_E_WORKSPACE;
  }
  const int64_t blocks = P.pairs * plan.splits;
  if (blocks > 0x7fffffffLL) return KVDEC_E_SHAPE;
  SET_CLOCK(P);
  hipLaunchKernelGGL((attn_kernel<Src>), dim3((unsigned)blocks), dim3(kThreads), kLdsBytes, stream,
                     P, S);
  int rc = launch_status();
  if (rc != KVDEC_OK || plan.splits == 1) return rc;
  const int64_t outs = P.pairs * P.G * kHeadDim;
  hipLaunchKernelGGL(merge_kernel, dim3((unsigned)((outs + 255) / 256)), dim3(256), 0, stream, P);
  return launch_status();
}

// The lean kernels' launches (one workgroup per KV head).
LeanCommon lean_common(const AttnCommon& P) {
  LeanCommon C;
  C.q = P.q;
  C.o = P.o;
  C.scale_log2 = P.scale_log2;
  C.G = P.G;
  C.R = P.R;
  return C;
}

// A contiguous fp16 source qualifies when one pass suffices and no wave has
// more than two tiles.
// Up to 16 tiles, or 16 tiles and a tail of at most kLeanTailRows rows
// (the sink of the W = 512 cache: 516 slots).
constexpr int kLeanTailRows = 4;
bool f16_lean_fits(const AttnCommon& P, int64_t rows) {
  const bool tiles = P.n_tiles <= 2 * kWaves ||
                     (P.n_tiles == 2 * kWaves + 1 && rows <= 2 * kWaves * kTile + kLeanTailRows);
  return make_plan(P.pairs, P.n_tiles).splits == 1 && tiles && P.pairs <= 0x7fffffffLL;
}

int launch_f16_lean(const AttnCommon& P, const _Float16* k, const _Float16* v, int rows,
                    hipStream_t stream) {
  F16LeanArgs A;
  A.c = lean_common(P);
  A.k = k;
  A.v = v;
  A.rows = rows;
  SET_CLOCK(A.c);
  if (P.n_tiles > 2 * kWaves)
    hipLaunchKernelGGL(f16_lean_kernel<true>, dim3((unsigned)P.pairs), dim3(kThreads), kLdsBytes + kQLdsBytes,
                       stream, A);
  else
    hipLaunchKernelGGL(f16_lean_kernel<false>, dim3((unsigned)P.pairs), dim3(kThreads), kLdsBytes + kQLdsBytes,
                       stream, A);
  return launch_status();
}

// The fused KIVI decode at one length (lens null) or at per-sequence
// lengths lens[b] (seq_len unused).
// Device address of `scratch` on the current device, looked up once per
// device (in host code the array's name is only a stand-in for the symbol).
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];

int scratch_address(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= kMaxDevices) return KVDEC_E_UNSUPPORTED;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return (int)e;
    if (p == nullptr) return KVDEC_E_WORKSPACE;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return KVDEC_OK;
}

int check_dense(const void* q, const void* k, const void* v, void* o, int dtype, int64_t B,
                int32_t H, int32_t KVH, int64_t L, int32_t D) {
  if (!q || !k || !v || !o) return KVDEC_E_NULL;
  if (dtype != KVDEC_F16 && dtype != KVDEC_F32 && dtype != KVDEC_BF16) return KVDEC_E_DTYPE;
  int rc = check_heads(B, H, KVH, D);
  if (rc) return rc;
  if (L < 1) return KVDEC_E_SEQLEN;
  if (L * kRowBytes >= ((int64_t)1 << 31)) return KVDEC_E_SHAPE;   // 32-bit in-head offsets
  return KVDEC_OK;
}

template <bool PACK>
int kivi_decode_t(const void* q, const void* k_res, const void* v_res, const void* const* kivi,
                void* o, const int32_t* lens, int64_t B, int32_t H, int32_t KVH, int64_t seq_len,
                int32_t window, int32_t sink, int32_t residual, int32_t group, int32_t bits,
                float sm_scale, void* stream) {
  if (!q || !k_res || !v_res || !kivi || !o) return KVDEC_E_NULL;
  if (bits != 2) return KVDEC_E_BITS;
  if (group != 32) return KVDEC_E_UNSUPPORTED;
  int rc = check_heads(B, H, KVH, kHeadDim);
  if (rc) return rc;
  if (seq_len < 1) return KVDEC_E_SEQLEN;
  if (sink < 1 || sink > group || residual < kTile || residual % kTile != 0 || window < 1)
    return KVDEC_E_WINDOW;
  // A window shorter than the residual stays fp16 entirely (residual rows =
  // window, no window-old tokens).
  const int32_t res_rows = window < residual ? window : residual;
  const int32_t win_tok = window - res_rows;
  if (win_tok % group != 0) return KVDEC_E_GROUP;
  for (int i = 0; i < 6; ++i)
    if (!kivi[i]) return KVDEC_E_NULL;
  if (win_tok > 0)
    for (int i = 6; i < 12; ++i)
      if (!kivi[i]) return KVDEC_E_NULL;
  if ((int64_t)res_rows * kRowBytes >= ((int64_t)1 << 31) ||
      (int64_t)win_tok * kHeadDim >= ((int64_t)1 << 31))
    return KVDEC_E_SHAPE;

  AttnCommon P{};
  P.q = static_cast<const _Float16*>(q);
  P.o = static_cast<_Float16*>(o);
  P.ws = nullptr;
  P.pairs = B * KVH;
  P.H = H;
  P.KVH = KVH;
  P.G = H / KVH;
  P.n_tiles = (int)tiles_for(KVDEC_KIND_KIVI, window);
  P.scale_log2 = (float)((double)sm_scale * 1.4426950408889634);
  P.R = sparse_ranges(seq_len, window, sink, KVDEC_LAYOUT_LINEAR);

  auto u8 = [&](int i) { return static_cast<const uint8_t*>(kivi[i]); };
  auto f16 = [&](int i) { return static_cast<const _Float16*>(kivi[i]); };
  KiviVarSrc<PACK> S{};
  S.kres = static_cast<const _Float16*>(k_res);
  S.vres = static_cast<const _Float16*>(v_res);
  S.res_rows = res_rows;
  S.sinkq = QRegion{u8(0), f16(1), f16(2), u8(3), f16(4), f16(5)};
  if (win_tok > 0)
    S.winq = QRegion{u8(6), f16(7), f16(8), u8(9), f16(10), f16(11)};
  else
    S.winq = S.sinkq;   // never dereferenced: there are no window-old tiles
  S.sink = sink;
  S.win_tok = win_tok;
  S.nwt = win_tok / kTile;
  S.lens = lens;
  S.window = window;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  if (lens) return launch_attn(P, S, true, 0, st);
  // the lean kernel: at most 4 residual tiles, at most 7 window-old groups,
  // and every tensor small enough for 31-bit offsets
  const int64_t lean_bytes = P.pairs * (int64_t)res_rows * kRowBytes;
  const bool lean = S.nwt + 1 <= 2 * 4;
  // the wide kernel: packed query groups, at least kWideMinGroups
  // window-old groups, a sink of at most 16 tokens, and the window-old code
  // tensors small enough for 31-bit offsets too
  const bool wide = PACK && S.nwt >= kWideMinGroups && P.G <= kPackGroup && sink <= kTile / 2 &&
                    P.pairs * (int64_t)S.nwt * 1024 < ((int64_t)1 << 31);
  if (res_rows <= 4 * kTile && (lean || wide) && lean_bytes < ((int64_t)1 << 31)) {
    KiviLeanArgs A;
    A.c = lean_common(P);
    A.kres = S.kres;
    A.vres = S.vres;
    A.sinkq = S.sinkq;
    A.winq = S.winq;
    A.res_bytes = (uint32_t)lean_bytes;
    A.res_rows = res_rows;
    A.win_code_bytes = (uint32_t)(P.pairs * S.nwt * 1024);
    A.win_meta_bytes = (uint32_t)(P.pairs * S.nwt * 256);
    A.nwt = S.nwt;
    A.sink = sink;
    SET_CLOCK(A.c);
    if (lean && S.nwt == 4)
      hipLaunchKernelGGL(kivi_lean9_kernel<PACK>, dim3((unsigned)P.pairs), dim3(64 * kLean9Waves),
                         Lean9Lds::kBytes + kQLdsBytes, st, A);
    else if (lean)
      hipLaunchKernelGGL(kivi_lean_kernel<PACK>, dim3((unsigned)P.pairs), dim3(kThreads), kLdsBytes + kQLdsBytes, st, A);
    else if constexpr (PACK)
      hipLaunchKernelGGL(kivi_wide_kernel<true>, dim3((unsigned)P.pairs), dim3(kWideThreads), kWideLdsBytes, st, A);
    return launch_status();
  }
  KiviSrc<PACK> S1{};
  S1.kres = S.kres;
  S1.vres = S.vres;
  S1.res_rows = S.res_rows;
  S1.sinkq = S.sinkq;
  S1.winq = S.winq;
  S1.sink = S.sink;
  S1.win_tok = S.win_tok;
  S1.nwt = S.nwt;
  return launch_attn(P, S1, true, 0, st);
}

// Query groups of at most kPackGroup heads take the packed-layout kernels
// from kPackMinGroups window-old groups on.  The packed step issues fewer
// instructions but has longer dependency chains; it pays once waves step
// more than one quantized tile (the lean kernel's four quantized waves take
// a second tile from 4 window-old groups on).  Measured per step: W = 160,
// 5.58 -> 5.73 us packed; W = 256, 6.38 -> 6.17 us.
constexpr int kPackMinGroups = 4;
bool packed_group(int32_t H, int32_t KVH, int64_t window_old_groups) {
  return window_old_groups >= kPackMinGroups && KVH > 0 && H % KVH == 0 && H / KVH <= kPackGroup;
}

// The element types the attention entry points take (q, o and row caches).
bool valid_attn_dtype(int dtype) { return dtype == KVDEC_F16 || dtype == KVDEC_F32 || dtype == KVDEC_BF16; }

// Code widths and group sizes other than 2 / 32, and queries or residual
// rows other than fp16: the generic kernel, with the reference's layout
// assumptions (whole bytes per group, channel groups that divide the head
// dim).
int kivi_decode_generic(const void* q, const void* k_res, const void* v_res, const void* const* kivi,
                        void* o, const int32_t* lens, int64_t B, int32_t H, int32_t KVH,
                        int64_t seq_len, int32_t window, int32_t sink, int32_t residual, int32_t group,
                        int32_t bits, float sm_scale, void* stream, int q_dtype = KVDEC_F16,
                        int res_dtype = KVDEC_F16) {
  if (!q || !k_res || !v_res || !kivi || !o) return KVDEC_E_NULL;
  if (!valid_attn_dtype(q_dtype) || !valid_attn_dtype(res_dtype)) return KVDEC_E_DTYPE;
  if (bits < 1 || bits > 8) return KVDEC_E_BITS;
  if (group < 1 || kHeadDim % group != 0 || group % (8 / bits) != 0) return KVDEC_E_GROUP;
  int rc = check_heads(B, H, KVH, kHeadDim);
  if (rc) return rc;
  if (seq_len < 1) return KVDEC_E_SEQLEN;
  if (sink < 1 || sink > group || residual < 1 || window < 1) return KVDEC_E_WINDOW;
  const int32_t res_rows = window < residual ? window : residual;
  const int32_t win_tok = window - res_rows;
  if (win_tok % group != 0) return KVDEC_E_GROUP;
  for (int i = 0; i < 6; ++i)
    if (!kivi[i]) return KVDEC_E_NULL;
  if (win_tok > 0)
    for (int i = 6; i < 12; ++i)
      if (!kivi[i]) return KVDEC_E_NULL;
  return generic_kivi_decode(q, k_res, v_res, kivi, o, q_dtype, res_dtype, lens, B, H, KVH, seq_len, window,
                             sink, res_rows, win_tok, group, bits, sm_scale, static_cast<hipStream_t>(stream));
}

int kivi_decode(const void* q, const void* k_res, const void* v_res, const void* const* kivi,
                void* o, const int32_t* lens, int64_t B, int32_t H, int32_t KVH, int64_t seq_len,
                int32_t window, int32_t sink, int32_t residual, int32_t group, int32_t bits,
                float sm_scale, void* stream) {
  if (bits != 2 || group != kQGroup)
    return kivi_decode_generic(q, k_res, v_res, kivi, o, lens, B, H, KVH, seq_len, window, sink, residual,
                               group, bits, sm_scale, stream);
  const int64_t res_rows = window < residual ? window : residual;
  if (packed_group(H, KVH, group > 0 ? (window - res_rows) / group : 0))
    return kivi_decode_t<true>(
      q, k_res, v_res, kivi, o, lens, B, H, KVH, seq_len, window, sink, residual, group, bits,
      sm_scale, stream);
  return kivi_decode_t<false>(
      q, k_res, v_res, kivi, o, lens, B, H, KVH, seq_len, window, sink, residual, group, bits,
      sm_scale, stream);
}

// The fused decode over a decode-time KIVI cache: one ring state for every
// sequence (ring null: ring_start / ring_count) or one per sequence.
template <bool PACK>
int stream_decode_t(const void* q, const void* k_ring, const void* v_ring, const void* const* kivi,
                  void* o, const int32_t* ring, int64_t B, int32_t H, int32_t KVH, int32_t sink,
                  int32_t n_groups, int32_t ring_cap, int32_t ring_start, int32_t ring_count,
                  int32_t group, int32_t bits, float sm_scale, void* stream) {
  if (!q || !k_ring || !v_ring || !kivi || !o) return KVDEC_E_NULL;
  if (bits != 2) return KVDEC_E_BITS;
  if (group != 32) return KVDEC_E_UNSUPPORTED;
  int rc = check_heads(B, H, KVH, kHeadDim);
  if (rc) return rc;
  if (sink < 1 || sink > group || n_groups < 0) return KVDEC_E_WINDOW;
  if (ring_cap < 2 * kTile || ring_cap % kTile != 0) return KVDEC_E_WINDOW;
  for (int i = 0; i < 6; ++i)
    if (!kivi[i]) return KVDEC_E_NULL;
  if (n_groups > 0)
    for (int i = 6; i < 12; ++i)
      if (!kivi[i]) return KVDEC_E_NULL;
  const int64_t win_tok = (int64_t)n_groups * group;
  if ((int64_t)ring_cap * kRowBytes >= ((int64_t)1 << 31) || win_tok * kHeadDim >= ((int64_t)1 << 31))
    return KVDEC_E_SHAPE;

  AttnCommon P{};
  P.q = static_cast<const _Float16*>(q);
  P.o = static_cast<_Float16*>(o);
  P.ws = nullptr;
  P.pairs = B * KVH;
  P.H = H;
  P.KVH = KVH;
  P.G = H / KVH;
  P.n_tiles = (int)(1 + n_groups + ring_cap / kTile);
  P.scale_log2 = (float)((double)sm_scale * 1.4426950408889634);
  // every sink and window-old slot is valid; ring rows [start, start + count)
  // (mod cap) of the residual are, at slots base + row
  const int base = sink + (int)win_tok;
  const int end = ring_start + ring_count;
  if (end <= ring_cap)
    P.R = SlotRanges{base, base + ring_start, base + end};
  else
    P.R = SlotRanges{base + end - ring_cap, base + ring_start, base + ring_cap};

  auto u8 = [&](int i) { return static_cast<const uint8_t*>(kivi[i]); };
  auto f16 = [&](int i) { return static_cast<const _Float16*>(kivi[i]); };
  KiviRingSrc<PACK> S{};
  S.kres = static_cast<const _Float16*>(k_ring);
  S.vres = static_cast<const _Float16*>(v_ring);
  S.res_rows = ring_cap;
  S.sinkq = QRegion{u8(0), f16(1), f16(2), u8(3), f16(4), f16(5)};
  S.winq = n_groups > 0 ? QRegion{u8(6), f16(7), f16(8), u8(9), f16(10), f16(11)} : S.sinkq;
  S.sink = sink;
  S.win_tok = (int)win_tok;
  S.nwt = n_groups;
  S.lens = ring;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  // the 10-wave ring kernel: a ring of 5 tiles, at most 4 window-old
  // groups, every tensor small enough for 31-bit offsets
  if (ring_cap == 5 * kTile && n_groups <= 4 && P.pairs * ring_cap * kRowBytes < ((int64_t)1 << 31) &&
      P.pairs <= 0x7fffffffLL) {
    StepLeanArgs L{};
    L.c = lean_common(P);
    L.k_ring = const_cast<_Float16*>(S.kres);
    L.v_ring = const_cast<_Float16*>(S.vres);
    L.sinkq = S.sinkq;
    L.winq = S.winq;
    L.ring = const_cast<int32_t*>(ring);
    L.ring_bytes = (uint32_t)(P.pairs * ring_cap * kRowBytes);
    L.win_code_bytes = (uint32_t)(P.pairs * n_groups * 1024);
    L.win_meta_bytes = (uint32_t)(P.pairs * n_groups * 256);
    L.nwg = n_groups;
    L.sink = sink;
    L.cap = ring_cap;
    L.KVH = KVH;
    SET_CLOCK(L.c);
    if (ring)
      hipLaunchKernelGGL((kivi_ring_kernel<PACK, kRingSeqs>), dim3((unsigned)P.pairs), dim3(64 * kStepWaves),
                         StepLds::kBytes + kQLdsBytes, st, L);
    else
      hipLaunchKernelGGL((kivi_ring_kernel<PACK, kRingOne>), dim3((unsigned)P.pairs), dim3(64 * kStepWaves),
                         StepLds::kBytes + kQLdsBytes, st, L);
    return launch_status();
  }
  if (ring) return launch_attn(P, S, true, 0, st);
  KiviSrc<PACK> S1{};
  S1.kres = S.kres;
  S1.vres = S.vres;
  S1.res_rows = S.res_rows;
  S1.sinkq = S.sinkq;
  S1.winq = S.winq;
  S1.sink = S.sink;
  S1.win_tok = S.win_tok;
  S1.nwt = S.nwt;
  return launch_attn(P, S1, true, 0, st);
}

int stream_decode(const void* q, const void* k_ring, const void* v_ring, const void* const* kivi,
                  void* o, const int32_t* ring, int64_t B, int32_t H, int32_t KVH, int32_t sink,
                  int32_t n_groups, int32_t ring_cap, int32_t ring_start, int32_t ring_count,
                  int32_t group, int32_t bits, float sm_scale, void* stream) {
  if (packed_group(H, KVH, n_groups))
    return stream_decode_t<true>(
      q, k_ring, v_ring, kivi, o, ring, B, H, KVH, sink, n_groups, ring_cap, ring_start,
      ring_count, group, bits, sm_scale, stream);
  return stream_decode_t<false>(
      q, k_ring, v_ring, kivi, o, ring, B, H, KVH, sink, n_groups, ring_cap, ring_start,
      ring_count, group, bits, sm_scale, stream);
}

// One token step of the per-sequence decode-time cache and the decode over
// the stepped state, in one launch.
template <bool PACK>
int stream_step_decode_t(const void* q, const void* k_new, const void* v_new, void* k_ring, void* v_ring,
                       void* const* kivi, void* o, int32_t* appended, const int32_t* active,
                       int32_t* arrive, int32_t* plan, int32_t* ring, int64_t B, int32_t H,
                       int32_t KVH, int32_t sink, int32_t residual, int32_t n_groups,
                       int32_t ring_cap, int32_t group, int32_t bits, float sm_scale, void* stream) {
  if (!q || !k_new || !v_new || !k_ring || !v_ring || !kivi || !o || !appended || !arrive || !plan ||
      !ring)
    return KVDEC_E_NULL;
  if (bits != 2) return KVDEC_E_BITS;
  if (group != 32) return KVDEC_E_UNSUPPORTED;
  int rc = check_heads(B, H, KVH, kHeadDim);
  if (rc) return rc;
  if (sink < 1 || sink > group || n_groups < 0) return KVDEC_E_WINDOW;
  if (residual < group || residual % group != 0 || ring_cap != residual + group) return KVDEC_E_WINDOW;
  for (int i = 0; i < 6; ++i)
    if (!kivi[i]) return KVDEC_E_NULL;
  if (n_groups > 0)
    for (int i = 6; i < 12; ++i)
      if (!kivi[i]) return KVDEC_E_NULL;
  const int64_t win_tok = (int64_t)n_groups * group;
  if ((int64_t)ring_cap * kRowBytes >= ((int64_t)1 << 31) || win_tok * kHeadDim >= ((int64_t)1 << 31))
    return KVDEC_E_SHAPE;

  AttnCommon P{};
  P.q = static_cast<const _Float16*>(q);
  P.o = static_cast<_Float16*>(o);
  P.ws = nullptr;
  P.pairs = B * KVH;
  P.H = H;
  P.KVH = KVH;
  P.G = H / KVH;
  P.n_tiles = (int)(1 + n_groups + ring_cap / kTile);
  P.scale_log2 = (float)((double)sm_scale * 1.4426950408889634);

  auto u8 = [&](int i) { return static_cast<uint8_t*>(kivi[i]); };
  auto f16 = [&](int i) { return static_cast<_Float16*>(kivi[i]); };
  KiviStepSrc<PACK> S{};
  S.kres = static_cast<const _Float16*>(k_ring);
  S.vres = static_cast<const _Float16*>(v_ring);
  S.res_rows = ring_cap;
  S.sinkq = QRegion{u8(0), f16(1), f16(2), u8(3), f16(4), f16(5)};
  S.winq = n_groups > 0 ? QRegion{u8(6), f16(7), f16(8), u8(9), f16(10), f16(11)} : S.sinkq;
  S.sink = sink;
  S.win_tok = (int)win_tok;
  S.nwt = n_groups;
  StreamArgs& a = S.a;
  a.k_new = static_cast<const _Float16*>(k_new);
  a.v_new = static_cast<const _Float16*>(v_new);
  a.k_ring = static_cast<_Float16*>(k_ring);
  a.v_ring = static_cast<_Float16*>(v_ring);
  if (n_groups > 0) {
    a.kp = u8(6);
    a.ks = f16(7);
    a.kz = f16(8);
    a.vp = u8(9);
    a.vs = f16(10);
    a.vz = f16(11);
  }
  a.appended = appended;
  a.active = active;
  a.arrive = arrive;
  a.plan = plan;
  a.ring = ring;
  a.D = kHeadDim;
  a.cap = ring_cap;
  a.nwg = n_groups;
  a.KVH = KVH;
  a.residual = residual;
  // the 10-wave step kernel: a ring of 5 tiles, at most 4 window-old
  // groups, every tensor small enough for 31-bit offsets
  if (ring_cap == 5 * kTile && n_groups <= 4 && P.pairs * ring_cap * kRowBytes < ((int64_t)1 << 31) &&
      P.pairs <= 0x7fffffffLL) {
    StepLeanArgs L;
    L.c = lean_common(P);
    L.c.R = SlotRanges{0, 0, 0};
    L.k_new = a.k_new;
    L.v_new = a.v_new;
    L.k_ring = a.k_ring;
    L.v_ring = a.v_ring;
    L.sinkq = S.sinkq;
    L.winq = S.winq;
    L.appended = appended;
    L.active = active;
    L.arrive = arrive;
    L.plan = plan;
    L.ring = ring;
    L.ring_bytes = (uint32_t)(P.pairs * ring_cap * kRowBytes);
    L.win_code_bytes = (uint32_t)(P.pairs * n_groups * 1024);
    L.win_meta_bytes = (uint32_t)(P.pairs * n_groups * 256);
    L.nwg = n_groups;
    L.sink = sink;
    L.residual = residual;
    L.cap = ring_cap;
    L.KVH = KVH;
    SET_CLOCK(L.c);
    hipLaunchKernelGGL((kivi_ring_kernel<PACK, kRingStep>), dim3((unsigned)P.pairs), dim3(64 * kStepWaves),
                       StepLds::kBytes + kQLdsBytes, static_cast<hipStream_t>(stream), L);
    return launch_status();
  }
  return launch_attn(P, S, true, 0, static_cast<hipStream_t>(stream));
}

int stream_step_decode(const void* q, const void* k_new, const void* v_new, void* k_ring, void* v_ring,
                       void* const* kivi, void* o, int32_t* appended, const int32_t* active,
                       int32_t* arrive, int32_t* plan, int32_t* ring, int64_t B, int32_t H,
                       int32_t KVH, int32_t sink, int32_t residual, int32_t n_groups,
                       int32_t ring_cap, int32_t group, int32_t bits, float sm_scale, void* stream) {
  if (packed_group(H, KVH, n_groups))
    return stream_step_decode_t<true>(
      q, k_new, v_new, k_ring, v_ring, kivi, o, appended, active, arrive, plan, ring, B, H, KVH,
      sink, residual, n_groups, ring_cap, group, bits, sm_scale, stream);
  return stream_step_decode_t<false>(
      q, k_new, v_new, k_ring, v_ring, kivi, o, appended, active, arrive, plan, ring, B, H, KVH,
      sink, residual, n_groups, ring_cap, group, bits, sm_scale, stream);
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
    case KVDEC_E_BITS: return "code width outside 1..8 bits, or not 2 bits where only 2-bit codes are implemented";
    case KVDEC_E_UNSUPPORTED: return "valid arguments, but not implemented";
    default: break;
  }
  if (code > 0) return hipGetErrorString((hipError_t)code);
  return "unknown kvdec error";
}

const char* kvdec_version(void) { return "kvdec 0.3 gfx950"; }

int kvdec_clock_arm(void* log, int32_t slots) {
#ifdef KVDEC_CLOCK
  if (log != nullptr && slots < 1) return KVDEC_E_SHAPE;
  std::lock_guard<std::mutex> lock(g_clock_mu);
  g_clock_log = static_cast<unsigned long long*>(log);
  g_clock_slots = log != nullptr ? slots : 0;
  g_clock_next = 0;
  return KVDEC_OK;
#else
  (void)log;
  (void)slots;
  return KVDEC_E_UNSUPPORTED;   // the product library has no kernel clock
#endif
}

int kvdec_num_splits(int kind, int64_t B, int32_t KVH, int64_t n_slots) {
  if (B < 1 || KVH < 1 || n_slots < 1) return 1;
  if (kind == KVDEC_KIND_KIVI) return 1;
  return make_plan(B * KVH, tiles_for(kind, n_slots)).splits;
}

size_t kvdec_workspace_bytes(int kind, int64_t B, int32_t H, int32_t KVH, int64_t n_slots,
                             int32_t D) {
  if (check_heads(B, H, KVH, D) != KVDEC_OK || n_slots < 1) return 0;
  if (kind == KVDEC_KIND_KIVI) return 0;
  const Plan p = make_plan(B * KVH, tiles_for(kind, n_slots));
  return ws_bytes_for(B * KVH, p.splits, H / KVH);
}

int kvdec_dense_decode(const void* q, const void* k, const void* v, void* o, int dtype, int64_t B,
                       int32_t H, int32_t KVH, int64_t L, int32_t D, float sm_scale, void* ws,
                       size_t ws_bytes, void* stream) {
  int rc = check_dense(q, k, v, o, dtype, B, H, KVH, L, D);
  if (rc) return rc;
  if (dtype != KVDEC_F16)
    return generic_rows_decode(q, k, v, o, dtype, B, H, KVH, L, SlotRanges{(int)L, 0, 0}, nullptr, false,
                               0, 0, KVDEC_LAYOUT_LINEAR, sm_scale, ws, ws_bytes,
                               static_cast<hipStream_t>(stream));
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
  if (f16_lean_fits(P, L))
    return launch_f16_lean(P, static_cast<const _Float16*>(k), static_cast<const _Float16*>(v), (int)L,
                           static_cast<hipStream_t>(stream));
  F16Src S{static_cast<const _Float16*>(k), static_cast<const _Float16*>(v), (int)L};
  return launch_attn(P, S, false, ws_bytes, static_cast<hipStream_t>(stream));
}

int kvdec_read_probe(const void* src, int64_t bytes, void* sink, int32_t blocks, void* stream) {
  if (!sink || (bytes > 0 && !src)) return KVDEC_E_NULL;
  if (bytes < 0 || bytes % 16 != 0 || blocks < 1 || blocks > 65536) return KVDEC_E_SHAPE;
  hipLaunchKernelGGL(read_probe_kernel, dim3((unsigned)blocks), dim3(kThreads), 0, static_cast<hipStream_t>(stream),
                     static_cast<const u32x4*>(src), bytes / 16, static_cast<uint32_t*>(sink));
  return launch_status();
}

int kvdec_read_probe_sweep(const void* src, int64_t bytes, void* sink, int32_t blocks, int32_t threads,
                           int32_t mode, int32_t lds_bytes, void* stream) {
  if (!sink || (bytes > 0 && !src)) return KVDEC_E_NULL;
  if (bytes < 0 || bytes % 16 != 0 || blocks < 1 || blocks > 65536) return KVDEC_E_SHAPE;
  if (threads != 256 && threads != 512 && threads != 1024) return KVDEC_E_SHAPE;
  if (mode < 0 || mode > 7 || lds_bytes < 0 || lds_bytes > 160 * 1024) return KVDEC_E_SHAPE;
  const int kind = mode & 3;
  const bool upfront = (mode & 4) != 0;
  const int64_t n16 = bytes / 16, per = (n16 + blocks - 1) / blocks;
  if (kind >= 2 && per * 16 >= ((int64_t)1 << 31)) return KVDEC_E_SHAPE;   // 31-bit buffer offsets
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const u32x4* s = static_cast<const u32x4*>(src);
  uint32_t* k = static_cast<uint32_t*>(sink);
  const size_t lds = (size_t)lds_bytes;
  if (threads == 256)
    launch_probe2_kind<256>(kind, upfront, (unsigned)blocks, lds, st, s, n16, k);
  else if (threads == 512)
    launch_probe2_kind<512>(kind, upfront, (unsigned)blocks, lds, st, s, n16, k);
  else
    launch_probe2_kind<1024>(kind, upfront, (unsigned)blocks, lds, st, s, n16, k);
  return launch_status();
}

int kvdec_dense_decode_noalloc(const void* q, const void* k, const void* v, void* o, int dtype,
                               int64_t B, int32_t H, int32_t KVH, int64_t L, int32_t D,
                               float sm_scale, void* stream) {
  int rc = check_dense(q, k, v, o, dtype, B, H, KVH, L, D);
  if (rc) return rc;
  const size_t need = kvdec_workspace_bytes(KVDEC_KIND_DENSE, B, H, KVH, L, D);
  if (need > kScratchBytes) return KVDEC_E_WORKSPACE;
  void* ws = nullptr;
  if (need > 0) {
    rc = scratch_address(&ws);
    if (rc) return rc;
  }
  return kvdec_dense_decode(q, k, v, o, dtype, B, H, KVH, L, D, sm_scale, ws, need, stream);
}

int kvdec_sparse_decode(const void* q, const void* k_cache, const void* v_cache, void* o,
                        int dtype, int64_t B, int32_t H, int32_t KVH, int64_t seq_len,
                        int32_t window, int32_t sink, int32_t layout, float sm_scale, void* ws,
                        size_t ws_bytes, void* stream) {
  if (!q || !k_cache || !v_cache || !o) return KVDEC_E_NULL;
  if (dtype != KVDEC_F16 && dtype != KVDEC_F32 && dtype != KVDEC_BF16) return KVDEC_E_DTYPE;
  int rc = check_heads(B, H, KVH, kHeadDim);
  if (rc) return rc;
  if (seq_len < 1) return KVDEC_E_SEQLEN;
  if (window < 0 || sink < 0 || (int64_t)window + sink < 1) return KVDEC_E_WINDOW;
  if (layout != KVDEC_LAYOUT_LINEAR && layout != KVDEC_LAYOUT_RING) return KVDEC_E_UNSUPPORTED;
  if (layout == KVDEC_LAYOUT_RING && window < 1) return KVDEC_E_WINDOW;
  const int64_t n = (int64_t)window + sink;
  if (n * kRowBytes >= ((int64_t)1 << 31)) return KVDEC_E_SHAPE;
  if (dtype != KVDEC_F16)
    return generic_rows_decode(q, k_cache, v_cache, o, dtype, B, H, KVH, n,
                               sparse_ranges(seq_len, window, sink, layout), nullptr, true, window, sink,
                               layout, sm_scale, ws, ws_bytes, static_cast<hipStream_t>(stream));
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
  if (f16_lean_fits(P, n))
    return launch_f16_lean(P, static_cast<const _Float16*>(k_cache), static_cast<const _Float16*>(v_cache),
                           (int)n, static_cast<hipStream_t>(stream));
  F16Src S{static_cast<const _Float16*>(k_cache), static_cast<const _Float16*>(v_cache), (int)n};
  return launch_attn(P, S, false, ws_bytes, static_cast<hipStream_t>(stream));
}

int kvdec_paged_decode(const void* q, const void* k_pages, const void* v_pages,
                       const int32_t* block_table, const int32_t* seq_lens, void* o, int dtype,
                       int64_t B, int32_t H, int32_t KVH, int32_t D, int64_t max_seq_len,
                       int32_t page_size, int32_t max_blocks, int64_t num_pages,
                       int64_t page_stride, int64_t row_stride, int64_t head_stride,
                       float sm_scale, void* ws, size_t ws_bytes, void* stream) {
  if (!q || !k_pages || !v_pages || !o) return KVDEC_E_NULL;
  if (dtype != KVDEC_F16) return KVDEC_E_DTYPE;
  int rc = check_heads(B, H, KVH, D);
  if (rc) return rc;
  if (max_seq_len < 1) return KVDEC_E_SEQLEN;
  if (max_seq_len >= ((int64_t)1 << 30)) return KVDEC_E_SHAPE;
  if (page_stride < 0 || row_stride < 0 || head_stride < 0) return KVDEC_E_SHAPE;
  if (row_stride * 2 * 16 >= ((int64_t)1 << 31)) return KVDEC_E_SHAPE;   // 32-bit in-half offsets
  int ps_log2 = 0;
  if (block_table) {
    if (page_size < 16 || page_size > (1 << 20) || (page_size & (page_size - 1))) return KVDEC_E_UNSUPPORTED;
    while ((1 << ps_log2) < page_size) ++ps_log2;
    if (num_pages < 1 || max_blocks < 1) return KVDEC_E_SHAPE;
    if ((int64_t)max_blocks * page_size < max_seq_len) return KVDEC_E_SHAPE;
  }
  AttnCommon P{};
  P.q = static_cast<const _Float16*>(q);
  P.o = static_cast<_Float16*>(o);
  P.ws = static_cast<float*>(ws);
  P.pairs = B * KVH;
  P.H = H;
  P.KVH = KVH;
  P.G = H / KVH;
  P.n_tiles = (int)tiles_for(KVDEC_KIND_DENSE, max_seq_len);
  P.scale_log2 = (float)((double)sm_scale * 1.4426950408889634);
  PagedSrc S{};
  S.k = static_cast<const char*>(k_pages);
  S.v = static_cast<const char*>(v_pages);
  S.bt = block_table;
  S.lens = seq_lens;
  S.page_bytes = page_stride * 2;
  S.head_bytes = head_stride * 2;
  S.row_bytes = (uint32_t)(row_stride * 2);
  S.ps_log2 = ps_log2;
  S.max_blocks = max_blocks;
  S.num_pages = num_pages;
  S.max_len = (int)max_seq_len;
  S.rows = (int)max_seq_len;
  S.sparse = false;
  return launch_attn(P, S, false, ws_bytes, static_cast<hipStream_t>(stream));
}

int kvdec_sparse_decode_varlen(const void* q, const void* k_cache, const void* v_cache, void* o,
                               const int32_t* seq_lens, int dtype, int64_t B, int32_t H,
                               int32_t KVH, int32_t window, int32_t sink, int32_t layout,
                               float sm_scale, void* ws, size_t ws_bytes, void* stream) {
  if (!q || !k_cache || !v_cache || !o || !seq_lens) return KVDEC_E_NULL;
  if (dtype != KVDEC_F16 && dtype != KVDEC_F32 && dtype != KVDEC_BF16) return KVDEC_E_DTYPE;
  int rc = check_heads(B, H, KVH, kHeadDim);
  if (rc) return rc;
  if (window < 0 || sink < 0 || (int64_t)window + sink < 1) return KVDEC_E_WINDOW;
  if (layout != KVDEC_LAYOUT_LINEAR && layout != KVDEC_LAYOUT_RING) return KVDEC_E_UNSUPPORTED;
  if (layout == KVDEC_LAYOUT_RING && window < 1) return KVDEC_E_WINDOW;
  const int64_t n = (int64_t)window + sink;
  if (n >= ((int64_t)1 << 30)) return KVDEC_E_SHAPE;
  if (dtype != KVDEC_F16)
    return generic_rows_decode(q, k_cache, v_cache, o, dtype, B, H, KVH, n, SlotRanges{0, 0, 0}, seq_lens,
                               true, window, sink, layout, sm_scale, ws, ws_bytes,
                               static_cast<hipStream_t>(stream));
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
  PagedSrc S{};
  S.k = static_cast<const char*>(k_cache);
  S.v = static_cast<const char*>(v_cache);
  S.lens = seq_lens;
  S.page_bytes = (int64_t)KVH * n * kRowBytes;
  S.head_bytes = n * kRowBytes;
  S.row_bytes = kRowBytes;
  S.max_len = 0x3fffffff;
  S.rows = (int)n;
  S.window = window;
  S.sink = sink;
  S.layout = layout;
  S.sparse = true;
  return launch_attn(P, S, false, ws_bytes, static_cast<hipStream_t>(stream));
}

int kvdec_sparse_decode_kivi(const void* q, const void* k_res, const void* v_res,
                             const void* const* kivi, void* o, int64_t B, int32_t H, int32_t KVH,
                             int64_t seq_len, int32_t window, int32_t sink, int32_t residual,
                             int32_t group, int32_t bits, float sm_scale, void* ws,
                             size_t ws_bytes, void* stream) {
  (void)ws;         // one pass: no workspace
  (void)ws_bytes;
  return kivi_decode(q, k_res, v_res, kivi, o, nullptr, B, H, KVH, seq_len, window, sink, residual,
                     group, bits, sm_scale, stream);
}

int kvdec_sparse_decode_kivi_varlen(const void* q, const void* k_res, const void* v_res,
                                    const void* const* kivi, void* o, const int32_t* seq_lens,
                                    int64_t B, int32_t H, int32_t KVH, int32_t window,
                                    int32_t sink, int32_t residual, int32_t group, int32_t bits,
                                    float sm_scale, void* stream) {
  if (!seq_lens) return KVDEC_E_NULL;
  return kivi_decode(q, k_res, v_res, kivi, o, seq_lens, B, H, KVH, 1, window, sink, residual,
                     group, bits, sm_scale, stream);
}

int kvdec_sparse_decode_kivi_typed(const void* q, const void* k_res, const void* v_res,
                                   const void* const* kivi, void* o, int q_dtype, int res_dtype,
                                   const int32_t* seq_lens, int64_t B, int32_t H, int32_t KVH,
                                   int64_t seq_len, int32_t window, int32_t sink, int32_t residual,
                                   int32_t group, int32_t bits, float sm_scale, void* stream) {
  const int64_t L = seq_lens ? 1 : seq_len;
  if (q_dtype == KVDEC_F16 && res_dtype == KVDEC_F16)
    return kivi_decode(q, k_res, v_res, kivi, o, seq_lens, B, H, KVH, L, window, sink, residual, group,
                       bits, sm_scale, stream);
  return kivi_decode_generic(q, k_res, v_res, kivi, o, seq_lens, B, H, KVH, L, window, sink, residual,
                             group, bits, sm_scale, stream, q_dtype, res_dtype);
}

int kvdec_kivi_stream_decode(const void* q, const void* k_ring, const void* v_ring,
                             const void* const* kivi, void* o, int64_t B, int32_t H, int32_t KVH,
                             int32_t sink, int32_t n_groups, int32_t ring_cap, int32_t ring_start,
                             int32_t ring_count, int32_t group, int32_t bits, float sm_scale,
                             void* stream) {
  if (ring_start < 0 || ring_start >= ring_cap || ring_count < 1 || ring_count > ring_cap)
    return KVDEC_E_WINDOW;
  return stream_decode(q, k_ring, v_ring, kivi, o, nullptr, B, H, KVH, sink, n_groups, ring_cap,
                       ring_start, ring_count, group, bits, sm_scale, stream);
}

int kvdec_kivi_stream_decode_seqs(const void* q, const void* k_ring, const void* v_ring,
                                  const void* const* kivi, void* o, const int32_t* ring,
                                  int64_t B, int32_t H, int32_t KVH, int32_t sink,
                                  int32_t n_groups, int32_t ring_cap, int32_t group, int32_t bits,
                                  float sm_scale, void* stream) {
  if (!ring) return KVDEC_E_NULL;
  return stream_decode(q, k_ring, v_ring, kivi, o, ring, B, H, KVH, sink, n_groups, ring_cap, 0,
                       ring_cap, group, bits, sm_scale, stream);
}

int kvdec_kivi_stream_step_decode(const void* q, const void* k_new, const void* v_new,
                                  void* k_ring, void* v_ring, void* const* kivi, void* o,
                                  int32_t* appended, const int32_t* active, int32_t* arrive,
                                  int32_t* plan, int32_t* ring, int64_t B, int32_t H, int32_t KVH,
                                  int32_t sink, int32_t residual, int32_t n_groups,
                                  int32_t ring_cap, int32_t group, int32_t bits, float sm_scale,
                                  void* stream) {
  return stream_step_decode(q, k_new, v_new, k_ring, v_ring, kivi, o, appended, active, arrive, plan,
                            ring, B, H, KVH, sink, residual, n_groups, ring_cap, group, bits, sm_scale,
                            stream);
}

}  // extern "C"
