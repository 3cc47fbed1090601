/*
 * kvdec.h -- C ABI of the MI355X (gfx950) decode-attention library
 * (libkvdec.so).
 *
 * One entry point per operator of the reference's decode-attention path.  The
 * reference is Python + Triton, so its "interface" is the Python function each
 * entry point replaces; the citation next to each declaration names it
 * (paths relative to the reference repository root).
 *
 * Conventions (all entry points):
 *   - every data pointer is a device pointer; tensors are dense row-major
 *     (contiguous) in the shapes stated below;
 *   - `stream` is a hipStream_t (NULL = the null stream); work is enqueued
 *     asynchronously and nothing synchronises;
 *   - the library never allocates device memory: split-K partials live in a
 *     caller-supplied workspace of kvdec_workspace_bytes() bytes;
 *   - return 0 on success, a negative KVDEC_E* code when host-side argument
 *     validation fails (nothing is launched, no HIP call is made), or a
 *     positive hipError_t value when a launch fails;
 *   - stateless and reentrant: no global state besides what the HIP runtime
 *     keeps.
 */
#ifndef KVDEC_H_
#define KVDEC_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- error codes (negative: rejected before launch) -------------------- */
#define KVDEC_OK 0
#define KVDEC_E_NULL (-1)        /* a required pointer is NULL                 */
#define KVDEC_E_SHAPE (-2)       /* a dimension is out of range / inconsistent */
#define KVDEC_E_DTYPE (-3)       /* unsupported element type                   */
#define KVDEC_E_GROUP (-4)       /* token count not a multiple of the group    */
#define KVDEC_E_DGROUP (-5)      /* head dim not a multiple of the group       */
#define KVDEC_E_WORKSPACE (-6)   /* workspace missing or too small             */
#define KVDEC_E_WINDOW (-7)      /* window / sink / residual combination       */
#define KVDEC_E_SEQLEN (-8)      /* seq_len < 1                                */
#define KVDEC_E_BITS (-9)        /* only 2-bit codes are implemented           */
#define KVDEC_E_UNSUPPORTED (-10)/* valid but not implemented for this entry point */

/* ---- element types --------------------------------------------------- */
#define KVDEC_F16 0
#define KVDEC_F32 1
#define KVDEC_BF16 2

/* ---- sparse cache layouts -------------------------------------------- */
#define KVDEC_LAYOUT_LINEAR 0    /* reference: slot s >= sink holds position
                                    (seq_len - window) + (s - sink)          */
#define KVDEC_LAYOUT_RING 1      /* position p >= sink in slot
                                    sink + (p - sink) mod window              */

/* ---- workspace kinds ------------------------------------------------- */
#define KVDEC_KIND_DENSE 0       /* n_slots = seq_len                          */
#define KVDEC_KIND_SPARSE 1      /* n_slots = sink + window                    */
#define KVDEC_KIND_KIVI 2        /* n_slots = window                           */

/* Human-readable text for any return code (never NULL). */
const char* kvdec_strerror(int code);

/* Library version string, e.g. "kvdec 0.1 gfx950". */
const char* kvdec_version(void);

/* Number of split-K partitions the attention entry points use for this
 * problem (1 = single pass, no workspace).  Pure arithmetic, no HIP call. */
int kvdec_num_splits(int kind, int64_t B, int32_t KVH, int64_t n_slots);

/* Workspace bytes the attention entry point of `kind` needs (0 when a
 * single pass suffices).  Pure arithmetic, no HIP call. */
size_t kvdec_workspace_bytes(int kind, int64_t B, int32_t H, int32_t KVH,
                             int64_t n_slots, int32_t D);

/*
 * Dense causal GQA decode: one query token per (batch, head) against the
 * whole context.  Replaces dense_kernel.py:70-82 (dense_decode_attention)
 * and its kernel dense_kernel.py:21-67.
 *   q, o : [B, H, D] dtype        k, v : [B, KVH, L, D] dtype
 *   head h reads KV head h / (H / KVH); H / KVH <= 16; D == 128.
 *   o = softmax(q k^T * sm_scale) v, fp32 softmax and accumulation.
 *   dtype KVDEC_F16 runs the MFMA kernels; KVDEC_BF16 and KVDEC_F32 (which
 *   the reference kernel also loads, dense_kernel.py:37,48-49) a generic
 *   kernel in fp32 arithmetic, output rounded once to dtype.
 */
int kvdec_dense_decode(const void* q, const void* k, const void* v, void* o,
                       int dtype, int64_t B, int32_t H, int32_t KVH, int64_t L,
                       int32_t D, float sm_scale, void* ws, size_t ws_bytes,
                       void* stream);

/*
 * kvdec_dense_decode without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  No counterpart in the
 * reference.  The split-K partials go to a file-scope device array of
 * 4160 KiB that each GPU holds until the process ends (every shape the
 * split plan allows fits; a larger need returns KVDEC_E_WORKSPACE).  The
 * call allocates nothing.  All calls on one GPU share that array: calls
 * that overlap on one GPU (two streams) race.  Nothing in it needs to
 * start at zero (each call writes every partial it reads).  `stream` must
 * belong to the current device.  Results are those of kvdec_dense_decode.
 */
int kvdec_dense_decode_noalloc(const void* q, const void* k, const void* v, void* o,
                               int dtype, int64_t B, int32_t H, int32_t KVH,
                               int64_t L, int32_t D, float sm_scale, void* stream);

/*
 * StreamingLLM sink + window decode over a compacted [B, KVH, sink+window, D]
 * cache.  Replaces sparse_kernel.py:105-118 (sparse_decode_attention) and
 * sparse_kernel.py:67-102; slot validity follows _kv_indices
 * (sparse_kernel.py:15-46) for KVDEC_LAYOUT_LINEAR.  q, o and the caches
 * are all of dtype (KVDEC_F16: MFMA kernels; KVDEC_BF16 / KVDEC_F32: the
 * generic fp32 kernel, as for kvdec_dense_decode).
 */
int kvdec_sparse_decode(const void* q, const void* k_cache, const void* v_cache,
                        void* o, int dtype, int64_t B, int32_t H, int32_t KVH,
                        int64_t seq_len, int32_t window, int32_t sink,
                        int32_t layout, float sm_scale, void* ws,
                        size_t ws_bytes, void* stream);

/*
 * Dense decode over a paged or strided fp16 cache with per-sequence lengths
 * (no counterpart in the reference, which passes one scalar seq_len and a
 * contiguous cache: dense_kernel.py:70-82; this is the vLLM-style caller's
 * form of the same attention).  Token t of sequence b, KV head h is the row
 *   k_pages + page * page_stride + h * head_stride + (t % page_size) * row_stride
 * (strides in elements; the last dim, D = 128, contiguous) with page =
 * block_table[b * max_blocks + t / page_size].  block_table NULL: no paging,
 * page = b (page_stride is the per-sequence stride) -- e.g. a [B, L, KVH, D]
 * cache, or a [B, KVH, L_max, D] cache with per-sequence lengths.
 * seq_lens [B] int32 on the device (NULL: every sequence max_seq_len long);
 * lengths are clamped into [0, max_seq_len], a length of 0 gives zeros.
 * page_size is a power of two >= 16 and max_blocks * page_size >=
 * max_seq_len; page ids outside [0, num_pages) read as zeros.  ws /
 * ws_bytes as for kvdec_dense_decode with L = max_seq_len
 * (kvdec_workspace_bytes(KVDEC_KIND_DENSE, B, H, KVH, max_seq_len, D)).
 */
int kvdec_paged_decode(const void* q, const void* k_pages, const void* v_pages,
                       const int32_t* block_table, const int32_t* seq_lens, void* o,
                       int dtype, int64_t B, int32_t H, int32_t KVH, int32_t D,
                       int64_t max_seq_len, int32_t page_size, int32_t max_blocks,
                       int64_t num_pages, int64_t page_stride, int64_t row_stride,
                       int64_t head_stride, float sm_scale, void* ws, size_t ws_bytes,
                       void* stream);

/*
 * kvdec_sparse_decode with one seq_len per sequence (seq_lens [B] int32 on
 * the device, each >= 1; the reference passes one scalar,
 * sparse_kernel.py:105-118).  Same cache, dtypes, layouts, masking rule per
 * sequence and workspace (kvdec_workspace_bytes(KVDEC_KIND_SPARSE, ...)).
 */
int kvdec_sparse_decode_varlen(const void* q, const void* k_cache, const void* v_cache,
                               void* o, const int32_t* seq_lens, int dtype, int64_t B,
                               int32_t H, int32_t KVH, int32_t window, int32_t sink,
                               int32_t layout, float sm_scale, void* ws, size_t ws_bytes,
                               void* stream);

/*
 * KIVI per-channel quantization of K.  Replaces quant_kernel.py:106-126
 * (quantize_k_cache) and quant_kernel.py:44-103.
 *   x      : [B, KVH, N, D] of in_dtype (KVDEC_F32, KVDEC_F16 or KVDEC_BF16)
 *   packed : [B, KVH, N/pf, D] u8 with pf = 8 / bits codes per byte: code of
 *            token pf*p+j in bits j*bits .. j*bits + bits - 1
 *   scale, zero : [B, KVH, N/group, D] fp16
 *   1 <= bits <= 8, N % group == 0, group % pf == 0 (whole bytes per group).
 *   bits == 2 with group == 32 (D even) is the fast path, anything else a
 *   generic kernel.  QMAX = 2^bits - 1; codes are bit-exact to the
 *   IEEE-float32 closed form s = (mx - mn) / QMAX, ... (quant_kernel.py:77-99).
 */
int kvdec_quantize_k(const void* x, int in_dtype, void* packed_u8,
                     void* scale_f16, void* zero_f16, int64_t B, int32_t KVH,
                     int64_t N, int32_t D, int32_t group, int32_t bits,
                     void* stream);

/*
 * KIVI per-token quantization of V.  Replaces quant_kernel.py:193-214
 * (quantize_v_cache) and quant_kernel.py:129-190.
 *   packed : [B, KVH, N, D/pf] u8, code of channel pf*c+j in bits j*bits ..
 *   scale, zero : [B, KVH, N, D/group] fp16
 *   1 <= bits <= 8, D % group == 0, group % pf == 0; bits == 2 with group
 *   == 32 is the fast path.
 */
int kvdec_quantize_v(const void* x, int in_dtype, void* packed_u8,
                     void* scale_f16, void* zero_f16, int64_t B, int32_t KVH,
                     int64_t N, int32_t D, int32_t group, int32_t bits,
                     void* stream);

/*
 * Fused sink + window + KIVI-2bit decode.  Replaces quant_kernel.py:551-581
 * (sparse_decode_attention_quantized) and quant_kernel.py:436-548.
 *   k_res, v_res : [B, KVH, min(window, residual), D] fp16 (the most recent tokens)
 *   kivi[12] (host array of device pointers), in this order:
 *     k_sink_packed [B,KVH,group/4,D] u8, k_sink_scale, k_sink_zero [B,KVH,1,D],
 *     v_sink_packed [B,KVH,group,D/4] u8, v_sink_scale, v_sink_zero [B,KVH,group,D/group],
 *     k_win_packed  [B,KVH,(W-R)/4,D],   k_win_scale,  k_win_zero  [B,KVH,(W-R)/group,D],
 *     v_win_packed  [B,KVH,W-R,D/4],     v_win_scale,  v_win_zero  [B,KVH,W-R,D/group]
 *   (the k_win / v_win pointers may be NULL when window == residual).
 *   Slot s of the logical [sink + window] cache is sink token s (s < sink),
 *   window-old token s - sink, or residual row s - (sink + window - residual);
 *   slots are masked by _kv_indices validity.  (window - residual) % group
 *   == 0, residual % 32 == 0, sink <= group.  window < residual (left
 *   undefined by the reference, quant_kernel.py:589-590) means the whole
 *   window stays fp16: k_res / v_res hold the `window` window tokens and
 *   there are no window-old tokens.
 *   Runs in one pass (one workgroup per KV head): ws / ws_bytes are
 *   accepted for interface stability and ignored (kvdec_workspace_bytes
 *   returns 0 for KVDEC_KIND_KIVI).
 *   bits / group other than 2 / 32 (the tensors of kvdec_quantize_k / _v at
 *   that width, /4 above reading /pf) run a generic kernel in fp32
 *   arithmetic: 1 <= bits <= 8, D % group == 0, group % pf == 0,
 *   (window - residual) % group == 0, 1 <= sink <= group, residual >= 1.
 */
int kvdec_sparse_decode_kivi(const void* q, const void* k_res, const void* v_res,
                             const void* const* kivi, void* o, int64_t B,
                             int32_t H, int32_t KVH, int64_t seq_len,
                             int32_t window, int32_t sink, int32_t residual,
                             int32_t group, int32_t bits, float sm_scale,
                             void* ws, size_t ws_bytes, void* stream);

/*
 * kvdec_sparse_decode_kivi with one length per sequence (seq_lens [B] int32
 * on the device, each >= 1; the reference passes one scalar,
 * quant_kernel.py:551-581): each sequence's slots are masked by the
 * _kv_indices rule at its own length, so sequences in ramp-up and in steady
 * state share one launch.  Same cache tensors and limits; no workspace.
 */
int kvdec_sparse_decode_kivi_varlen(const void* q, const void* k_res, const void* v_res,
                                    const void* const* kivi, void* o,
                                    const int32_t* seq_lens, int64_t B, int32_t H,
                                    int32_t KVH, int32_t window, int32_t sink,
                                    int32_t residual, int32_t group, int32_t bits,
                                    float sm_scale, void* stream);

/*
 * kvdec_sparse_decode_kivi / _varlen with the element types of the query
 * and of the residual rows as arguments: quant_kernel.py:436-548 loads q and
 * the fp16 residual cache (K_cache_ptr, V_cache_ptr) in whatever dtype they
 * come in, computes in fp32 and stores o in q's dtype (:548), and
 * build_quantized_kv_cache keeps the residual in the compacted cache's dtype
 * (quant_kernel.py:592-593).
 *   q, o   : [B, H, D] of q_dtype (KVDEC_F16, KVDEC_BF16 or KVDEC_F32)
 *   k_res, v_res : residual rows of res_dtype (the same three)
 *   seq_lens : NULL -> every sequence at seq_len; else [B] int32 on the
 *              device (as kvdec_sparse_decode_kivi_varlen; seq_len ignored)
 *   Other arguments and limits as kvdec_sparse_decode_kivi.  Both dtypes
 *   KVDEC_F16 run exactly kvdec_sparse_decode_kivi / _varlen; any other
 *   pair runs the generic kernel in fp32 arithmetic (one rounding of the
 *   output to q_dtype).  No workspace.
 */
int kvdec_sparse_decode_kivi_typed(const void* q, const void* k_res, const void* v_res,
                                   const void* const* kivi, void* o, int q_dtype, int res_dtype,
                                   const int32_t* seq_lens, int64_t B, int32_t H, int32_t KVH,
                                   int64_t seq_len, int32_t window, int32_t sink, int32_t residual,
                                   int32_t group, int32_t bits, float sm_scale, void* stream);

/*
 * Decode-time KIVI cache, the write side of the fused decode (no counterpart
 * in the reference, which builds the cache once per call:
 * quant_kernel.py:584-622).  State per (b, kv) head: the quantized sink
 * group, a ring of n_groups window-old groups (the layouts of
 * kvdec_sparse_decode_kivi's k_win / v_win tensors with W - R = n_groups *
 * group), and an fp16 residual ring of ring_cap rows (a multiple of 32,
 * >= residual + 32).
 *
 * kvdec_kivi_stream_append: writes k_new / v_new [B, KVH, D] fp16 into row
 * `row` of k_ring / v_ring [B, KVH, ring_cap, D] (both NULL: no write, the
 * caller's producer writes the row itself); when evict_block >= 0 it
 * also quantizes ring rows [32 * evict_block, +32) (K per channel, V per
 * token, the quantizers' exact formulas) into window-old group slot
 * evict_slot of win[6] = {k_win_packed, k_win_scale, k_win_zero,
 * v_win_packed, v_win_scale, v_win_zero}.  With n_groups == 0 the block is
 * dropped.  The evicted block must not contain `row`.
 */
int kvdec_kivi_stream_append(const void* k_new, const void* v_new, void* k_ring,
                             void* v_ring, void* const* win, int64_t B,
                             int32_t KVH, int32_t D, int32_t ring_cap,
                             int32_t row, int32_t evict_block,
                             int32_t evict_slot, int32_t n_groups,
                             int32_t group, int32_t bits, void* stream);

/*
 * kvdec_kivi_stream_decode: the fused decode over that state.  kivi[12] as
 * for kvdec_sparse_decode_kivi (window-old tensors holding n_groups groups,
 * in any order: attention does not depend on it); every sink and
 * window-old token is attended, and residual ring rows
 * [ring_start, ring_start + ring_count) modulo ring_cap.  Same kernel as
 * kvdec_sparse_decode_kivi, one pass, no workspace.
 */
int kvdec_kivi_stream_decode(const void* q, const void* k_ring,
                             const void* v_ring, const void* const* kivi,
                             void* o, int64_t B, int32_t H, int32_t KVH,
                             int32_t sink, int32_t n_groups, int32_t ring_cap,
                             int32_t ring_start, int32_t ring_count,
                             int32_t group, int32_t bits, float sm_scale,
                             void* stream);

/*
 * The same cache with one ring state per sequence, for sequences that join
 * (a new prefill in their batch slot) and pause independently.  Both entry
 * points are asynchronous on `stream`; nothing is read back.
 *
 * kvdec_kivi_stream_step: one token step.  appended [B] int32 counts the
 * tokens appended to each sequence since its prefill (set it to 0 when a
 * prefill is written into the slot); active [B] int32 (NULL: all) selects
 * the sequences that take a token.  Each active sequence's next ring row
 * gets k_new / v_new [B, KVH, D] (both NULL: the producer writes the rows
 * itself, after this call), and a ring that fills has its oldest 32-row
 * block quantized into its oldest window-old slot.  Writes plan [B][3] =
 * {row, evict block, evict slot} taken (-1 = none), ring [B][2] = {start,
 * count} after the step, and advances `appended`.  arrive [B] int32 is
 * scratch the caller zeroes once (the kernel leaves it zero).
 * ring_cap == residual + group.
 */
int kvdec_kivi_stream_step(const void* k_new, const void* v_new, void* k_ring, void* v_ring,
                           void* const* win, int32_t* appended, const int32_t* active,
                           int32_t* arrive, int32_t* plan, int32_t* ring, int64_t B,
                           int32_t KVH, int32_t D, int32_t residual, int32_t ring_cap,
                           int32_t n_groups, int32_t group, int32_t bits, void* stream);

/*
 * kvdec_kivi_stream_decode_seqs: kvdec_kivi_stream_decode with each
 * sequence's valid residual rows from ring [B][2] = {start, count}.
 */
int kvdec_kivi_stream_decode_seqs(const void* q, const void* k_ring, const void* v_ring,
                                  const void* const* kivi, void* o, const int32_t* ring,
                                  int64_t B, int32_t H, int32_t KVH, int32_t sink,
                                  int32_t n_groups, int32_t ring_cap, int32_t group,
                                  int32_t bits, float sm_scale, void* stream);

/*
 * kvdec_kivi_stream_step_decode: kvdec_kivi_stream_step with k_new / v_new
 * (required here) followed by kvdec_kivi_stream_decode_seqs over the
 * stepped state, in one launch: each (b, kv) workgroup first writes its
 * token's row and quantizes its evicted block (if any), then attends.
 * kivi[12] as for kvdec_kivi_stream_decode (the window-old tensors are
 * written by evictions); appended, active, arrive, plan and ring as for
 * kvdec_kivi_stream_step, left as that call leaves them.  No counterpart
 * in the reference, which builds its caches once (quant_kernel.py:584-622).
 */
int kvdec_kivi_stream_step_decode(const void* q, const void* k_new, const void* v_new,
                                  void* k_ring, void* v_ring, void* const* kivi, void* o,
                                  int32_t* appended, const int32_t* active, int32_t* arrive,
                                  int32_t* plan, int32_t* ring, int64_t B, int32_t H,
                                  int32_t KVH, int32_t sink, int32_t residual,
                                  int32_t n_groups, int32_t ring_cap, int32_t group,
                                  int32_t bits, float sm_scale, void* stream);

/*
 * The whole KIVI cache from a compacted K/V cache in one launch.  Replaces
 * build_quantized_kv_cache (quant_kernel.py:584-622: slicing :592-593 and
 * :608-609, sink padding :602-606, four quantizer calls :611-614).
 *   k_compacted, v_compacted : [B, KVH, n_slots, D] of in_dtype (KVDEC_F32,
 *     KVDEC_F16 or KVDEC_BF16), n_slots = sink + window.
 *   out[14], in the reference dict's key order: k_residual, v_residual
 *     [B, KVH, min(window, residual), D] of residual_dtype (in_dtype, or
 *     KVDEC_F16 for kvdec_sparse_decode_kivi); then the twelve tensors of
 *     kvdec_sparse_decode_kivi's kivi[12] (sink group: the sink tokens, then
 *     token 0 repeated up to `group` tokens; window-old: slots
 *     [sink, sink + window - residual)).  The six window-old pointers may be
 *     NULL when window <= residual.
 *   Codes, scales and zeros equal kvdec_quantize_k / kvdec_quantize_v on the
 *   same slices.  (window - residual) % group == 0 when window > residual;
 *   1 <= sink <= group; D % group == 0; group == 32, bits == 2.
 */
int kvdec_build_kivi_cache(const void* k_compacted, const void* v_compacted,
                           int in_dtype, int residual_dtype, int64_t B,
                           int32_t KVH, int32_t n_slots, int32_t D,
                           int32_t sink, int32_t residual, int32_t group,
                           int32_t bits, void* const* out, void* stream);

/*
 * Dequantize one block_n-token tile of a K region, with the reference's
 * clamping: byte = clamp(tok_start/4 + t/4, 0, num_packed-1) (C division),
 * code = (byte >> 2*(t%4)) & 3, group = min(byte/(group/4), num_groups-1),
 * out = float(scale) * (code - float(zero)).  Replaces the debug wrapper
 * test_dequantize_tile_isolated.py:28-44 around quant_kernel.py:219-266.
 *   packed [B,KVH,num_packed,D] u8, scale/zero [B,KVH,num_groups,D] fp16,
 *   out [B,KVH,block_n,D] fp32.
 */
int kvdec_dequant_k_tile(const void* packed, const void* scale,
                         const void* zero, void* out_f32, int64_t tok_start,
                         int64_t num_packed, int64_t num_groups, int32_t B,
                         int32_t KVH, int32_t D, int32_t block_n,
                         void* stream);

/*
 * Dequantize one block_n-token tile of a V region: token =
 * clamp(tok_start + t, 0, seq_len-1), code from byte d/4 shifted 2*(d%4),
 * group d/32.  Replaces test_dequantize_tile_isolated.py:47-63 around
 * quant_kernel.py:269-311.
 *   packed [B,KVH,seq_len,D/4] u8, scale/zero [B,KVH,seq_len,D/32] fp16,
 *   out [B,KVH,block_n,D] fp32.
 */
int kvdec_dequant_v_tile(const void* packed, const void* scale,
                         const void* zero, void* out_f32, int64_t tok_start,
                         int64_t seq_len, int32_t B, int32_t KVH, int32_t D,
                         int32_t block_n, void* stream);

/*
 * Measurement probe, no counterpart in the reference: streams `bytes` bytes
 * (a multiple of 16) from `src` with `blocks` workgroups of 512 threads, each
 * reading one contiguous share with non-temporal 16-byte loads, and writes
 * the XOR of each workgroup's share (as 32-bit words) to sink[blockIdx]
 * (`blocks` uint32 words).  bytes = 0 launches the same grid with no reads:
 * the per-launch cost.  bench.py times both to state a decode step's floor
 * on the box it runs on.
 */
int kvdec_read_probe(const void* src, int64_t bytes, void* sink, int32_t blocks, void* stream);

/*
 * The read probe's sweep form, no counterpart in the reference: `threads`
 * (256, 512 or 1024) per workgroup, each workgroup one contiguous share;
 * mode bits 0..1 pick the load (0 global non-temporal, 1 global, 2 buffer
 * with the decode streams' non-temporal hint, 3 buffer without it), bit 2
 * issues up to 16 loads per thread before any is used (else 4 in flight);
 * `lds_bytes` (<= 160 KiB) of dynamic LDS are reserved and not touched, so
 * that bytes = 0 times an empty launch with a decode kernel's grid, block
 * and LDS footprint.  Buffer modes need each share below 2 GiB.
 */
int kvdec_read_probe_sweep(const void* src, int64_t bytes, void* sink, int32_t blocks,
                           int32_t threads, int32_t mode, int32_t lds_bytes, void* stream);

/*
 * Kernel clock, no counterpart in the reference.  In the timing build
 * (libkvdec_clock.so, the same sources compiled with -DKVDEC_CLOCK) every
 * attention-kernel launch after this call takes the next of `slots` slots
 * of `log` (cyclically): device memory of slots x 1024 x 4 uint64, zeroed
 * by the caller.  Workgroup w < 1024 of the launch stores the GPU realtime
 * counter (100 MHz) at its start into [slot][w][0] and after its output
 * store into [slot][w][1], and the core-clock counter (s_memtime) at the
 * same two points into [slot][w][2] and [slot][w][3].  log = NULL disarms.  The product library
 * returns KVDEC_E_UNSUPPORTED.
 */
int kvdec_clock_arm(void* log, int32_t slots);

#ifdef __cplusplus
}
#endif

#endif /* KVDEC_H_ */
