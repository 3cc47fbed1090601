// Internal interface of generic.hip: the reference-semantics decode kernels
// that the C-ABI entry points of attn.hip hand the cases their MFMA kernels
// do not take (bf16 / fp32 queries and caches; KIVI codes of any width and
// group size).  Argument validation is the entry points' job.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "kvdec_device.h"

namespace kvdec {

// Rows of `dtype` (KVDEC_F32 / KVDEC_BF16 / KVDEC_F16): q, o [B, H, 128];
// k, v [B, KVH, rows, 128].  Slot validity: `lens` null -> R for every
// sequence; else per sequence b at length lens[b] (clamped at 0): dense
// (sparse == false) the first min(len, rows) slots, sparse the sink +
// window rule of `layout` (sparse_ranges).  The split-K partials go to ws
// (ws_bytes; a single pass when they do not fit or ws is null).
int generic_rows_decode(const void* q, const void* k, const void* v, void* o, int dtype, int64_t B,
                        int32_t H, int32_t KVH, int64_t rows, SlotRanges R, const int32_t* lens,
                        bool sparse, int32_t window, int32_t sink, int32_t layout, float sm_scale,
                        void* ws, size_t ws_bytes, hipStream_t stream);

// The fused KIVI decode for any code width (1..8 bits) and group size: q, o
// [B, H, 128] of q_dtype; residual rows [B, KVH, res_rows, 128] of
// res_dtype (KVDEC_F16 / KVDEC_BF16 / KVDEC_F32 each); kivi[12] as
// kvdec_sparse_decode_kivi (sink tensors of one padded group, window-old
// tensors of win_tok tokens).  Slot validity: `lens` null -> the linear
// sink + window rule at seq_len, else at lens[b] per sequence.
int generic_kivi_decode(const void* q, const void* k_res, const void* v_res, const void* const* kivi,
                        void* o, int q_dtype, int res_dtype, const int32_t* lens, int64_t B, int32_t H,
                        int32_t KVH, int64_t seq_len, int32_t window, int32_t sink, int32_t res_rows,
                        int32_t win_tok, int32_t group, int32_t bits, float sm_scale,
                        hipStream_t stream);

}  // namespace kvdec
