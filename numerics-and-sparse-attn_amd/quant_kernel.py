"""KIVI 2-bit KV cache on top of the sink + window cache, on MI355X (gfx950).

Drop-in for the reference's quant_kernel.py: quantize_k_cache /
quantize_v_cache (K per-channel over 32-token groups, V per-token over
32-channel groups, asymmetric min/max, fp16 scale and zero, four 2-bit codes
per byte, LSB first), sparse_decode_attention_quantized (decode over the sink,
window-old and fp16-residual regimes with the 2-bit codes unpacked in
registers) and build_quantized_kv_cache.  dequantize_k_tile /
dequantize_v_tile expose the single-tile dequantizers that the reference tests
reach through Triton debug kernels.

Codes, scales and zeros are bit-exact to the IEEE-float32 closed form of the
reference's formulas (s = (mx - mn) / 3, s := 1 if 0, z = floor(-mn / s + 0.5),
code = clamp(floor(x / s + 0.5) + z, 0, 3)).  The quantizers and the fused
decode also take the reference's ``bits`` (1..8, QMAX = 2^bits - 1, 8 // bits
codes per byte) and ``group_size`` parameters; widths and groups other than
2 / 32 run generic kernels (the 2-bit, 32-group kernels are the fast path).
"""

import torch

from constants import (
    BLOCK_N, D_HEAD, GROUP_SIZE, QUANT_BITS, RESIDUAL_SIZE, SINK_SIZE,
)
import _checks
import _kvdec as K

_IN_DTYPES = {torch.float32: K.F32, torch.float16: K.F16, torch.bfloat16: K.BF16}


def _quant_input(name, x):
    _checks.require_gpu_tensor(name, x, dtypes=tuple(_IN_DTYPES), ndim=4)


def quantize_k_cache(k, group_size=GROUP_SIZE, bits=QUANT_BITS):
    """k: [BATCH, N_KV_HEADS, seq_len, D_HEAD], fp32. Returns (packed_codes,
    scale, zero_point). Assumes seq_len is a multiple of group_size.

    Mirrors quant_kernel.py:106-126.  Also accepts fp16 / bf16 input (the
    conversion to fp32 is exact, so the codes are the same).
    Shapes: packed [B, KVH, seq_len/4, D] u8; scale, zero [B, KVH, seq_len/group, D] fp16.
    """
    batch, n_kv_heads, seq_len, d_head = k.shape
    if seq_len % group_size != 0:
        raise AssertionError("this simple version assumes seq_len is a multiple of group_size")
    if not k.is_contiguous():
        k = k.contiguous()
    _quant_input("k", k)
    pack_factor = 8 // bits
    num_groups = seq_len // group_size
    num_packed = seq_len // pack_factor
    packed = torch.empty((batch, n_kv_heads, num_packed, d_head), dtype=torch.uint8, device=k.device)
    scale = torch.empty((batch, n_kv_heads, num_groups, d_head), dtype=torch.float16, device=k.device)
    zero_point = torch.empty((batch, n_kv_heads, num_groups, d_head), dtype=torch.float16, device=k.device)
    if seq_len == 0:
        return packed, scale, zero_point
    rc = K.lib.kvdec_quantize_k(K.ptr(k), _IN_DTYPES[k.dtype], K.ptr(packed), K.ptr(scale),
                                K.ptr(zero_point), batch, n_kv_heads, seq_len, d_head, group_size,
                                bits, K.stream_of(k))
    K.check(rc, "quantize_k_cache")
    return packed, scale, zero_point


def quantize_v_cache(v, group_size=GROUP_SIZE, bits=QUANT_BITS):
    """v: [BATCH, N_KV_HEADS, seq_len, D_HEAD], fp32. Returns (packed_codes,
    scale, zero_point) -- shapes mirror-flip vs. quantize_k_cache: seq_len
    stays full-size, D_HEAD shrinks (opposite of K).

    Mirrors quant_kernel.py:193-214.  Shapes: packed [B, KVH, seq_len, D/4] u8;
    scale, zero [B, KVH, seq_len, D/group] fp16.
    """
    batch, n_kv_heads, seq_len, d_head = v.shape
    if d_head % group_size != 0:
        raise AssertionError("this simple version assumes D_HEAD is a multiple of group_size")
    if not v.is_contiguous():
        v = v.contiguous()
    _quant_input("v", v)
    pack_factor = 8 // bits
    num_chan_groups = d_head // group_size
    d_packed = d_head // pack_factor
    packed = torch.empty((batch, n_kv_heads, seq_len, d_packed), dtype=torch.uint8, device=v.device)
    scale = torch.empty((batch, n_kv_heads, seq_len, num_chan_groups), dtype=torch.float16, device=v.device)
    zero_point = torch.empty((batch, n_kv_heads, seq_len, num_chan_groups), dtype=torch.float16,
                             device=v.device)
    if seq_len == 0:
        return packed, scale, zero_point
    rc = K.lib.kvdec_quantize_v(K.ptr(v), _IN_DTYPES[v.dtype], K.ptr(packed), K.ptr(scale),
                                K.ptr(zero_point), batch, n_kv_heads, seq_len, d_head, group_size,
                                bits, K.stream_of(v))
    K.check(rc, "quantize_v_cache")
    return packed, scale, zero_point


def dequantize_k_tile(packed, scale, zero_point, tok_start, num_packed=None, num_groups=None,
                      block_n=BLOCK_N):
    """One block_n-token tile of a per-channel-quantized K region, fp32
    [B, KVH, block_n, D], with the reference's clamping of the byte and group
    indices (quant_kernel.py:219-266; the Triton debug wrapper of
    test_dequantize_tile_isolated.py:28-44)."""
    _checks.require_gpu_tensor("packed", packed, dtypes=(torch.uint8,), ndim=4)
    _checks.require_gpu_tensor("scale", scale, ndim=4)
    _checks.require_gpu_tensor("zero_point", zero_point, ndim=4)
    B, KVH, np_, D = packed.shape
    num_packed = np_ if num_packed is None else int(num_packed)
    num_groups = scale.shape[2] if num_groups is None else int(num_groups)
    if num_packed != np_ or scale.shape[2] != num_groups:
        raise ValueError("num_packed / num_groups must match the tensors' token axes")
    _checks.require_shape("zero_point", zero_point, scale.shape)
    out = torch.empty((B, KVH, block_n, D), dtype=torch.float32, device=packed.device)
    rc = K.lib.kvdec_dequant_k_tile(K.ptr(packed), K.ptr(scale), K.ptr(zero_point), K.ptr(out),
                                    int(tok_start), num_packed, num_groups, B, KVH, D, block_n,
                                    K.stream_of(packed))
    K.check(rc, "dequantize_k_tile")
    return out


def dequantize_v_tile(packed, scale, zero_point, tok_start, seq_len=None, block_n=BLOCK_N):
    """One block_n-token tile of a per-token-quantized V region, fp32
    [B, KVH, block_n, D], token index clamped to [0, seq_len) as in
    quant_kernel.py:269-311 (the debug wrapper of
    test_dequantize_tile_isolated.py:47-63)."""
    _checks.require_gpu_tensor("packed", packed, dtypes=(torch.uint8,), ndim=4)
    _checks.require_gpu_tensor("scale", scale, ndim=4)
    _checks.require_gpu_tensor("zero_point", zero_point, ndim=4)
    B, KVH, n, dp = packed.shape
    seq_len = n if seq_len is None else int(seq_len)
    if seq_len != n:
        raise ValueError("seq_len must match the packed tensor's token axis")
    D = dp * 4
    _checks.require_shape("scale", scale, (B, KVH, n, D // GROUP_SIZE))
    _checks.require_shape("zero_point", zero_point, (B, KVH, n, D // GROUP_SIZE))
    out = torch.empty((B, KVH, block_n, D), dtype=torch.float32, device=packed.device)
    rc = K.lib.kvdec_dequant_v_tile(K.ptr(packed), K.ptr(scale), K.ptr(zero_point), K.ptr(out),
                                    int(tok_start), seq_len, B, KVH, D, block_n,
                                    K.stream_of(packed))
    K.check(rc, "dequantize_v_tile")
    return out


_KIVI_ORDER = (
    "k_sink_packed", "k_sink_scale", "k_sink_zero",
    "v_sink_packed", "v_sink_scale", "v_sink_zero",
    "k_win_packed", "k_win_scale", "k_win_zero",
    "v_win_packed", "v_win_scale", "v_win_zero",
)


def sparse_decode_attention_quantized(
    q, k_cache, v_cache,
    k_sink_packed, k_sink_scale, k_sink_zero,
    v_sink_packed, v_sink_scale, v_sink_zero,
    k_win_packed, k_win_scale, k_win_zero,
    v_win_packed, v_win_scale, v_win_zero,
    seq_len, window, sink=SINK_SIZE, residual_size=RESIDUAL_SIZE,
    group_size=GROUP_SIZE, bits=QUANT_BITS, sm_scale=None,
):
    """k_cache/v_cache here is the RESIDUAL cache specifically (own
    [.., RESIDUAL_SIZE, D_HEAD] shape) -- not the full compacted cache like
    sparse_decode_attention takes.

    Mirrors quant_kernel.py:551-581.  Slot s of the logical [sink + window]
    cache is the sink token s (s < sink), the window-old token s - sink, or
    the residual row s - (sink + window - residual_size); slots are attended
    under the _kv_indices validity rule.  window < residual_size, which the
    reference leaves undefined (quant_kernel.py:589-590), means the whole
    window stays fp16: k_cache / v_cache are [.., window, D_HEAD] (what
    build_quantized_kv_cache returns then) and there is no window-old part.
    ``seq_len`` may also be a [BATCH] int32 tensor on the GPU: each sequence
    is masked at its own length (ramp-up per sequence).
    ``bits`` / ``group_size`` other than 2 / 32 (caches from
    quantize_k_cache / quantize_v_cache with the same arguments, the sink
    padded to one group) take the generic fp32 kernel: 1..8-bit codes,
    8 // bits per byte, groups that divide D_HEAD and hold whole bytes.
    q and the residual may each be fp16, bf16 or fp32 (quant_kernel.py:
    436-548 loads them in their own dtype); o has q's dtype.  Anything but
    fp16 / fp16 takes the generic fp32 kernel.
    """
    tensors = dict(zip(_KIVI_ORDER, (k_sink_packed, k_sink_scale, k_sink_zero,
                                     v_sink_packed, v_sink_scale, v_sink_zero,
                                     k_win_packed, k_win_scale, k_win_zero,
                                     v_win_packed, v_win_scale, v_win_zero)))
    _checks.require_gpu_tensor("q", q, dtypes=tuple(_checks.ATTN_DTYPES), ndim=3)
    _checks.require_gpu_tensor("k_cache", k_cache, dtypes=tuple(_checks.ATTN_DTYPES), ndim=4)
    _checks.require_gpu_tensor("v_cache", v_cache, dtypes=(k_cache.dtype,), ndim=4)
    B, H, D = q.shape
    KVH = k_cache.shape[1]
    varlen = isinstance(seq_len, torch.Tensor)
    if varlen:
        _checks.seq_lens_tensor("seq_len", seq_len, B, q.device)
    else:
        seq_len = int(seq_len)
    window, sink, R = int(window), int(sink), int(residual_size)
    if window < 1:
        raise ValueError(f"window ({window}) must be >= 1")
    res_rows = min(window, R)
    win_tok = window - res_rows
    G, bits = int(group_size), int(bits)
    if not 1 <= bits <= 8:
        raise ValueError(f"bits must be in 1..8, got {bits}")
    if G < 1 or D % G or G % (8 // bits):
        raise ValueError(f"group_size {G} must divide D_HEAD ({D}) and hold whole bytes of {bits}-bit codes")
    pf = 8 // bits
    _checks.require_shape("k_cache", k_cache, (B, KVH, res_rows, D))
    _checks.require_shape("v_cache", v_cache, (B, KVH, res_rows, D))
    expect = {
        "k_sink_packed": (B, KVH, G // pf, D), "k_sink_scale": (B, KVH, 1, D), "k_sink_zero": (B, KVH, 1, D),
        "v_sink_packed": (B, KVH, G, D // pf), "v_sink_scale": (B, KVH, G, D // G),
        "v_sink_zero": (B, KVH, G, D // G),
        "k_win_packed": (B, KVH, win_tok // pf, D), "k_win_scale": (B, KVH, win_tok // G, D),
        "k_win_zero": (B, KVH, win_tok // G, D),
        "v_win_packed": (B, KVH, win_tok, D // pf), "v_win_scale": (B, KVH, win_tok, D // G),
        "v_win_zero": (B, KVH, win_tok, D // G),
    }
    for name, t in tensors.items():
        dt = (torch.uint8,) if name.endswith("packed") else (torch.float16,)
        _checks.require_gpu_tensor(name, t, dtypes=dt, ndim=4)
        _checks.require_shape(name, t, expect[name])
    _checks.require_same_device(("q", q), ("k_cache", k_cache), ("v_cache", v_cache),
                                *tensors.items())
    o = torch.empty_like(q)
    if sm_scale is None:
        sm_scale = D_HEAD**-0.5
    arr = (K._vp * 12)(*[K.ptr(tensors[n]) if tensors[n].numel() else None for n in _KIVI_ORDER])
    if q.dtype != torch.float16 or k_cache.dtype != torch.float16:
        # quant_kernel.py:436-548 loads q and the residual in their own dtype
        # and stores o in q's: the generic kernel (fp32 arithmetic)
        lens = K.ptr(seq_len) if varlen else None
        rc = K.lib.kvdec_sparse_decode_kivi_typed(K.ptr(q), K.ptr(k_cache), K.ptr(v_cache), arr, K.ptr(o),
                                                  _checks.ATTN_DTYPES[q.dtype],
                                                  _checks.ATTN_DTYPES[k_cache.dtype], lens, B, H, KVH,
                                                  1 if varlen else seq_len, window, sink, R, G, bits,
                                                  float(sm_scale), K.stream_of(q))
        K.check(rc, "sparse_decode_attention_quantized")
        return o
    if varlen:
        rc = K.lib.kvdec_sparse_decode_kivi_varlen(K.ptr(q), K.ptr(k_cache), K.ptr(v_cache), arr, K.ptr(o),
                                                   K.ptr(seq_len), B, H, KVH, window, sink, R, G, bits,
                                                   float(sm_scale), K.stream_of(q))
        K.check(rc, "sparse_decode_attention_quantized")
        return o
    ws, nbytes = K.workspace(K.KIND_KIVI, B, H, KVH, window, D, q.device)
    rc = K.lib.kvdec_sparse_decode_kivi(K.ptr(q), K.ptr(k_cache), K.ptr(v_cache), arr, K.ptr(o), B,
                                        H, KVH, seq_len, window, sink, R, G, bits, float(sm_scale),
                                        K.ptr(ws), nbytes, K.stream_of(q))
    K.check(rc, "sparse_decode_attention_quantized")
    return o


def build_quantized_kv_cache(k_compacted, v_compacted, residual_size=RESIDUAL_SIZE, sink=SINK_SIZE,
                             residual_dtype=None):
    """Slices a compacted [BATCH, N_KV_HEADS, SINK+WINDOW, D_HEAD] K/V cache
    into residual/sink/window-old and quantizes sink+window-old separately,
    producing the tensors sparse_decode_attention_quantized expects.

    Mirrors quant_kernel.py:584-622 (same slicing, sink padded to one group by
    repeating token 0, same 14 keys) in one kernel launch that reads the
    compacted cache once: no slice, pad or ``.float()`` copies (fp16 / bf16
    -> fp32 is exact, so the codes equal the quantizers' on those copies).
    The residual keeps the input dtype, as in the reference, unless
    residual_dtype says otherwise (torch.float16 turns an fp32 or bf16 cache
    into what the fp16 fused decode reads; a bf16 or fp32 residual takes the
    generic fp32 kernel).  A window shorter than residual_size
    (undefined in the reference, whose slicing would then put sink slots into
    the residual) keeps the whole window as the residual and has no
    window-old part.
    """
    _checks.require_gpu_tensor("k_compacted", k_compacted, dtypes=tuple(_IN_DTYPES), ndim=4,
                               contiguous=False)
    _checks.require_gpu_tensor("v_compacted", v_compacted, dtypes=tuple(_IN_DTYPES), ndim=4,
                               contiguous=False)
    B, KVH, n, D = k_compacted.shape
    _checks.require_same_device(("k_compacted", k_compacted), ("v_compacted", v_compacted))
    _checks.require_shape("v_compacted", v_compacted, (B, KVH, n, D))
    if v_compacted.dtype != k_compacted.dtype:
        raise TypeError(f"v_compacted dtype {v_compacted.dtype} != k_compacted dtype {k_compacted.dtype}")
    sink = int(sink)
    if not 1 <= sink <= GROUP_SIZE or n <= sink:
        raise ValueError(f"unsupported sink={sink} for a cache of {n} slots")
    res_dtype = k_compacted.dtype if residual_dtype is None else residual_dtype
    if res_dtype not in (k_compacted.dtype, torch.float16):
        raise TypeError(f"residual_dtype must be the input dtype or torch.float16, got {res_dtype}")
    res = min(int(residual_size), n - sink)
    win = n - sink - res
    if win % GROUP_SIZE != 0:
        raise AssertionError("this simple version assumes seq_len is a multiple of group_size")
    k_compacted = k_compacted.contiguous()
    v_compacted = v_compacted.contiguous()
    dev, G, P = k_compacted.device, GROUP_SIZE, 8 // QUANT_BITS

    def u8(*shape):
        return torch.empty(shape, dtype=torch.uint8, device=dev)

    def f16(*shape):
        return torch.empty(shape, dtype=torch.float16, device=dev)

    out = {
        "k_residual": torch.empty((B, KVH, res, D), dtype=res_dtype, device=dev),
        "v_residual": torch.empty((B, KVH, res, D), dtype=res_dtype, device=dev),
        "k_sink_packed": u8(B, KVH, G // P, D), "k_sink_scale": f16(B, KVH, 1, D),
        "k_sink_zero": f16(B, KVH, 1, D),
        "v_sink_packed": u8(B, KVH, G, D // P), "v_sink_scale": f16(B, KVH, G, D // G),
        "v_sink_zero": f16(B, KVH, G, D // G),
        "k_win_packed": u8(B, KVH, win // P, D), "k_win_scale": f16(B, KVH, win // G, D),
        "k_win_zero": f16(B, KVH, win // G, D),
        "v_win_packed": u8(B, KVH, win, D // P), "v_win_scale": f16(B, KVH, win, D // G),
        "v_win_zero": f16(B, KVH, win, D // G),
    }
    ptrs = (K._vp * 14)(*[K.ptr(t) if t.numel() else None for t in out.values()])
    rc = K.lib.kvdec_build_kivi_cache(K.ptr(k_compacted), K.ptr(v_compacted), _IN_DTYPES[k_compacted.dtype],
                                      _IN_DTYPES[res_dtype], B, KVH, n, D, sink, int(residual_size), G,
                                      QUANT_BITS, ptrs, K.stream_of(k_compacted))
    K.check(rc, "build_quantized_kv_cache")
    return out
