"""Dense causal GQA decode attention on MI355X (gfx950).

Drop-in for the reference's dense_kernel.py: same function name, argument
order, defaults and result (o = softmax(q K^T * sm_scale) V per query head,
query head h reading KV head h // (N_HEADS // N_KV_HEADS), output in q's
dtype).  The work runs in libkvdec's split-K flash-decode kernel: one
workgroup per (KV head, split) serves all query heads of the group from one
pass over K/V, the splits are merged by a second kernel.
"""

import torch

from constants import D_HEAD
import _checks
import _kvdec as K


def dense_decode_attention(q, k, v, seq_len, sm_scale=None):
    """q: [BATCH, N_HEADS, D_HEAD]. k/v: [BATCH, N_KV_HEADS, seq_len, D_HEAD].

    Mirrors dense_kernel.py:70-82.  Shapes are read from the tensors and
    checked (the reference takes them from constants.py); D_HEAD must be 128
    and N_HEADS / N_KV_HEADS <= 16.  Asynchronous on torch's current stream.
    q, k, v share one dtype: fp16 runs the MFMA kernels; bf16 and fp32, which
    the reference's kernel also loads (dense_kernel.py:37,48-49), run the
    generic fp32 kernel (output in q's dtype).

    Beyond the reference: ``seq_len`` may be a [BATCH] int32 tensor on the
    GPU (per-sequence lengths; k / v are then [BATCH, N_KV_HEADS, L_max,
    D_HEAD] and sequence b attends over its first seq_len[b] rows, a length
    of 0 giving zeros), and k / v may be strided views (any strides with a
    contiguous head dim, e.g. a permuted [BATCH, L, N_KV_HEADS, D_HEAD]
    cache).  Both go through the strided kernel source; the contiguous,
    scalar-length call is the reference's.
    """
    _checks.require_gpu_tensor("q", q, dtypes=tuple(_checks.ATTN_DTYPES), ndim=3)
    _checks.require_gpu_tensor("k", k, dtypes=(q.dtype,), ndim=4, contiguous=False)
    _checks.require_gpu_tensor("v", v, dtypes=(q.dtype,), ndim=4, contiguous=False)
    _checks.require_same_device(("q", q), ("k", k), ("v", v))
    dtype = _checks.ATTN_DTYPES[q.dtype]
    B, H, D = q.shape
    KVH = k.shape[1]
    varlen = isinstance(seq_len, torch.Tensor)
    if varlen:
        _checks.seq_lens_tensor("seq_len", seq_len, B, q.device)
        L = k.shape[2]
    else:
        L = seq_len = int(seq_len)
    _checks.require_shape("k", k, (B, KVH, L, D))
    _checks.require_shape("v", v, (B, KVH, L, D))
    if not q.is_contiguous():
        raise ValueError("q must be contiguous")
    o = torch.empty_like(q)
    if sm_scale is None:
        sm_scale = D_HEAD**-0.5
    ws, nbytes = K.workspace(K.KIND_DENSE, B, H, KVH, L, D, q.device)
    if not varlen and k.is_contiguous() and v.is_contiguous():
        rc = K.lib.kvdec_dense_decode(K.ptr(q), K.ptr(k), K.ptr(v), K.ptr(o), dtype, B, H, KVH, L, D,
                                      float(sm_scale), K.ptr(ws), nbytes, K.stream_of(q))
        K.check(rc, "dense_decode_attention")
        return o
    if dtype != K.F16:
        raise ValueError("per-sequence lengths and strided caches take fp16 q / k / v")
    _checks.row_major_rows("k", k)
    _checks.row_major_rows("v", v)
    if k.stride() != v.stride():
        raise ValueError(f"k and v must share strides, got {k.stride()} and {v.stride()}")
    sb, sh, sl, _ = k.stride()
    rc = K.lib.kvdec_paged_decode(K.ptr(q), K.ptr(k), K.ptr(v), None,
                                  K.ptr(seq_len) if varlen else None, K.ptr(o), K.F16, B, H, KVH, D,
                                  L, 0, 0, 0, sb, sl, sh, float(sm_scale), K.ptr(ws), nbytes,
                                  K.stream_of(q))
    K.check(rc, "dense_decode_attention")
    return o
