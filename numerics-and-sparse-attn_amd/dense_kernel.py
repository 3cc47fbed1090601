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
    checked (the reference takes them from constants.py); q, k, v are fp16
    and contiguous; D_HEAD must be 128 and N_HEADS / N_KV_HEADS <= 16.
    Asynchronous on torch's current stream.
    """
    _checks.require_gpu_tensor("q", q, ndim=3)
    _checks.require_gpu_tensor("k", k, ndim=4)
    _checks.require_gpu_tensor("v", v, ndim=4)
    _checks.require_same_device(("q", q), ("k", k), ("v", v))
    B, H, D = q.shape
    KVH = k.shape[1]
    seq_len = int(seq_len)
    _checks.require_shape("k", k, (B, KVH, seq_len, D))
    _checks.require_shape("v", v, (B, KVH, seq_len, D))
    o = torch.empty_like(q)
    if sm_scale is None:
        sm_scale = D_HEAD**-0.5
    ws, nbytes = K.workspace(K.KIND_DENSE, B, H, KVH, seq_len, D, q.device)
    rc = K.lib.kvdec_dense_decode(K.ptr(q), K.ptr(k), K.ptr(v), K.ptr(o), K.F16, B, H, KVH, seq_len,
                                  D, float(sm_scale), K.ptr(ws), nbytes, K.stream_of(q))
    K.check(rc, "dense_decode_attention")
    return o
