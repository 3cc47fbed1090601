"""StreamingLLM sink + sliding-window decode attention on MI355X (gfx950).

Drop-in for the reference's sparse_kernel.py.  The compacted cache holds
``sink + window`` slots per (batch, KV head); in the reference's linear
layout slot s < sink holds position s and slot sink + i holds position
(seq_len - window) + i, and a slot is attended only while that position
exists (the _kv_indices rule, sparse_kernel.py:15-46).  layout="ring" selects
the ring-buffer layout (position p >= sink in slot sink + (p - sink) % window)
used by a streaming writer; both give the same result in steady state.
"""

import torch

from constants import D_HEAD, SINK_SIZE
import _checks
import _kvdec as K

_LAYOUTS = {"linear": K.LAYOUT_LINEAR, "ring": K.LAYOUT_RING}


def sparse_decode_attention(q, k_cache, v_cache, seq_len, window, sink=SINK_SIZE, sm_scale=None,
                            layout="linear"):
    """k_cache/v_cache must be [BATCH, N_KV_HEADS, SINK+WINDOW, D_HEAD].

    Mirrors sparse_kernel.py:105-118 (same arguments and defaults; ``layout``
    is an added keyword).  Contiguous, D_HEAD == 128; q and the caches share
    one dtype: fp16 runs the MFMA kernels, bf16 and fp32 the generic fp32
    kernel.  ``seq_len`` may also be a [BATCH] int32 tensor on the GPU: each
    sequence is masked at its own length (each >= 1).
    """
    _checks.require_gpu_tensor("q", q, dtypes=tuple(_checks.ATTN_DTYPES), ndim=3)
    _checks.require_gpu_tensor("k_cache", k_cache, dtypes=(q.dtype,), ndim=4)
    _checks.require_gpu_tensor("v_cache", v_cache, dtypes=(q.dtype,), ndim=4)
    dtype = _checks.ATTN_DTYPES[q.dtype]
    _checks.require_same_device(("q", q), ("k_cache", k_cache), ("v_cache", v_cache))
    if layout not in _LAYOUTS:
        raise ValueError(f"layout must be one of {sorted(_LAYOUTS)}, got {layout!r}")
    B, H, D = q.shape
    KVH = k_cache.shape[1]
    varlen = isinstance(seq_len, torch.Tensor)
    if varlen:
        _checks.seq_lens_tensor("seq_len", seq_len, B, q.device)
    else:
        seq_len = int(seq_len)
    window, sink = int(window), int(sink)
    if window < 0 or sink < 0:
        raise ValueError(f"window and sink must be >= 0 (window={window}, sink={sink})")
    _checks.require_shape("k_cache", k_cache, (B, KVH, sink + window, D))
    _checks.require_shape("v_cache", v_cache, (B, KVH, sink + window, D))
    o = torch.empty_like(q)
    if sm_scale is None:
        sm_scale = D_HEAD**-0.5
    ws, nbytes = K.workspace(K.KIND_SPARSE, B, H, KVH, sink + window, D, q.device)
    if varlen:
        rc = K.lib.kvdec_sparse_decode_varlen(K.ptr(q), K.ptr(k_cache), K.ptr(v_cache), K.ptr(o),
                                              K.ptr(seq_len), dtype, B, H, KVH, window, sink,
                                              _LAYOUTS[layout], float(sm_scale), K.ptr(ws), nbytes,
                                              K.stream_of(q))
        K.check(rc, "sparse_decode_attention")
        return o
    rc = K.lib.kvdec_sparse_decode(K.ptr(q), K.ptr(k_cache), K.ptr(v_cache), K.ptr(o), dtype, B, H,
                                   KVH, seq_len, window, sink, _LAYOUTS[layout], float(sm_scale),
                                   K.ptr(ws), nbytes, K.stream_of(q))
    K.check(rc, "sparse_decode_attention")
    return o
