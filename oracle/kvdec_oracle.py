"""CPU oracle for the decode-attention path.  TEST INFRASTRUCTURE ONLY.

This module restates, in numpy, the reference's algorithms for dense GQA
decode, StreamingLLM sink+window decode, the KIVI quantizers (2-bit and any
other code width the reference's BITS parameter allows), the tile
dequantizers, the quantized-cache builder and the fused quantized decode.  It
is the checker the HIP path is compared against.  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it, and only to check or to time the CPU baseline; the product path in
the package never imports it and has no CPU fallback.

Every function cites the reference file:line it follows (paths relative to the
reference repository root).  How each function is pinned (closed forms,
invariants, brute force, library routines) is exercised by
``tests/test_oracle.py``; no function here is left parity-unpinned against the
closed-form contract.  What no artefact pins is the bit-level behaviour of the
reference's A100 Triton binaries (fp16 products in the logit reduction,
``tl.math.exp`` and the lowering of ``/``); the reference's own tests only
bound those to max-abs 1e-2.

Conventions
-----------
* Attention math runs in float64 by default (``dtype`` argument), on inputs
  already rounded to the dtype the kernel sees (fp16), so the only differences
  left against the GPU are the GPU's own rounding.
* Quantizer math is IEEE float32 with round-to-nearest-even, exactly as the
  reference writes it: ``s = (mx - mn) / QMAX``, ``s = 1 if s == 0``,
  ``z = floor(-mn / s + 0.5)``, ``code = clamp(floor(x / s + 0.5) + z, 0, QMAX)``
  with the float32 ``s, z`` and QMAX = 2^bits - 1 (3 for the default 2
  bits); scale and zero are stored as fp16 (RNE).
"""

from __future__ import annotations

import numpy as np

F32 = np.float32
F16 = np.float16

PACK_FACTOR = 4          # 2-bit codes, four per byte
QMAX = 3


# --------------------------------------------------------------------------
# Dense GQA decode
# --------------------------------------------------------------------------

def dense_attention(q, k, v, sm_scale, dtype=np.float64):
    """softmax(q . K[kv]^T * sm_scale) . V[kv] with kv = h // (H // KVH).

    Follows test_dense_correctness.py:13-30 (GQA by reshaping q into
    (KVH, group) and broadcasting against un-repeated K/V) and the kernel's
    head mapping dense_kernel.py:34.  q: [B, H, D]; k, v: [B, KVH, N, D].
    Returns [B, H, D] in ``dtype``.
    """
    q = np.asarray(q)
    B, H, D = q.shape
    _, KVH, N, _ = k.shape
    G = H // KVH
    qg = q.astype(dtype).reshape(B, KVH, G, D)
    kk = np.asarray(k).astype(dtype)
    vv = np.asarray(v).astype(dtype)
    s = np.matmul(qg, np.swapaxes(kk, -1, -2)) * dtype(sm_scale)      # [B,KVH,G,N]
    s = s - s.max(axis=-1, keepdims=True)
    p = np.exp(s)
    p = p / p.sum(axis=-1, keepdims=True)
    o = np.matmul(p, vv)                                             # [B,KVH,G,D]
    return o.reshape(B, H, D)


def masked_attention(q, k, v, valid, sm_scale, dtype=np.float64):
    """Dense GQA attention restricted to the positions where ``valid`` is True.

    ``valid`` is a bool vector over the N positions of k/v (shared by every
    batch row and head), the masked-softmax form of
    test_sparse_correctness.py:41-48.  Invalid positions never enter the
    softmax, whatever values they hold.
    """
    valid = np.asarray(valid, dtype=bool)
    idx = np.nonzero(valid)[0]
    if idx.size == 0:
        raise ValueError("masked_attention: no valid position")
    return dense_attention(q, np.asarray(k)[:, :, idx], np.asarray(v)[:, :, idx], sm_scale, dtype)


# --------------------------------------------------------------------------
# StreamingLLM sink + window
# --------------------------------------------------------------------------

def streaming_llm_mask(seq_len, window, sink):
    """Positions kept by StreamingLLM's StartRecentKVCache at this length.

    Restates test_sparse_correctness.py:35-39: no eviction until
    seq_len > sink + window, then sink prefix plus the last ``window``.
    """
    pos = np.arange(seq_len)
    if seq_len <= sink + window:
        return np.ones(seq_len, dtype=bool)
    return (pos < sink) | (pos >= seq_len - window)


def kv_indices(seq_len, slot_start, window, sink, block_n):
    """Physical slot numbers and validity for one tile of the compacted cache.

    Restates sparse_kernel.py:34-46 for slots slot_start .. slot_start+block_n-1:
    sink slot s is valid iff s < seq_len; window slot s holds logical position
    (seq_len - window) + (s - sink) and is valid iff that position >= sink.
    Returns (addr_slot, valid) as int64 / bool arrays.
    """
    slot = slot_start + np.arange(block_n, dtype=np.int64)
    in_bounds = slot < (sink + window)
    is_sink = slot < sink
    window_logical_pos = (seq_len - window) + (slot - sink)
    sink_valid = slot < seq_len
    window_valid = window_logical_pos >= sink
    valid = in_bounds & np.where(is_sink, sink_valid, window_valid)
    addr_slot = np.where(in_bounds, slot, 0)
    return addr_slot, valid


def slot_validity(seq_len, window, sink, layout=0):
    """Validity of every slot of a [sink + window] compacted cache.

    layout 0 is the reference's linear layout (kv_indices above over all
    slots).  layout 1 is the ring layout of the north-star config 3: logical
    position p >= sink lives in slot sink + (p - sink) mod window, so the
    valid window slots are the first min(window, seq_len - sink) ones.
    """
    n = sink + window
    if layout == 0:
        return kv_indices(seq_len, 0, window, sink, n)[1]
    valid = np.zeros(n, dtype=bool)
    valid[: min(sink, seq_len)] = True
    nwin = min(window, max(0, seq_len - sink))
    valid[sink: sink + nwin] = True
    return valid


def build_compacted_cache(k_full, v_full, seq_len, window, sink, garbage=1e4):
    """Reference-layout compacted cache with ``garbage`` in unwritten slots.

    Restates test_sparse_correctness.py:51-72: slot i < sink holds position i;
    slot sink + i holds position (seq_len - window) + i when that exists.
    """
    B, KVH, _, D = k_full.shape
    kc = np.full((B, KVH, sink + window, D), garbage, dtype=k_full.dtype)
    vc = np.full_like(kc, garbage)
    ns = min(sink, seq_len)
    kc[:, :, :ns] = k_full[:, :, :ns]
    vc[:, :, :ns] = v_full[:, :, :ns]
    start = seq_len - window
    for i in range(window):
        pos = start + i
        if 0 <= pos < seq_len:
            kc[:, :, sink + i] = k_full[:, :, pos]
            vc[:, :, sink + i] = v_full[:, :, pos]
    return kc, vc


def build_ring_cache(k_full, v_full, seq_len, window, sink, garbage=1e4):
    """Ring-layout compacted cache: position p >= sink in slot sink + (p-sink) % window.

    The write side of the north-star config 3 layout; only the positions the
    StreamingLLM mask keeps are written.
    """
    B, KVH, _, D = k_full.shape
    kc = np.full((B, KVH, sink + window, D), garbage, dtype=k_full.dtype)
    vc = np.full_like(kc, garbage)
    keep = streaming_llm_mask(seq_len, window, sink)
    for p in range(seq_len):
        if not keep[p]:
            continue
        s = p if p < sink else sink + (p - sink) % window
        kc[:, :, s] = k_full[:, :, p]
        vc[:, :, s] = v_full[:, :, p]
    return kc, vc


def sparse_attention_full(q, k_full, v_full, seq_len, window, sink, sm_scale, dtype=np.float64):
    """StreamingLLM attention over the full, un-evicted context.

    Restates test_sparse_correctness.py:22-48 (mask from streaming-llm, GQA).
    """
    mask = streaming_llm_mask(seq_len, window, sink)
    return masked_attention(q, k_full[:, :, :seq_len], v_full[:, :, :seq_len], mask, sm_scale, dtype)


def sparse_attention_compacted(q, k_cache, v_cache, seq_len, window, sink, sm_scale,
                               layout=0, dtype=np.float64):
    """What the sparse kernel computes: attention over the valid cache slots.

    Follows sparse_kernel.py:87-102 (tile loop over sink + window slots, masked
    by kv_indices) for layout 0; layout 1 uses the ring validity above.
    """
    valid = slot_validity(seq_len, window, sink, layout)
    return masked_attention(q, k_cache, v_cache, valid, sm_scale, dtype)


# --------------------------------------------------------------------------
# Per-sequence lengths and paged caches (no counterpart in the reference,
# which passes one scalar seq_len and a contiguous cache, dense_kernel.py:70-
# 82 and sparse_kernel.py:105-118; each sequence reduces to those calls)
# --------------------------------------------------------------------------

def dense_attention_varlen(q, k, v, seq_lens, sm_scale, dtype=np.float64):
    """Sequence b attends over rows [0, seq_lens[b]) of k[b], v[b]
    ([B, KVH, L_max, D]); a length of 0 gives zeros."""
    q = np.asarray(q)
    out = np.zeros(q.shape, dtype=dtype)
    for b, n in enumerate(np.asarray(seq_lens).tolist()):
        if n > 0:
            out[b] = dense_attention(q[b:b + 1], k[b:b + 1, :, :n], v[b:b + 1, :, :n], sm_scale, dtype)[0]
    return out


def sparse_attention_varlen(q, k_cache, v_cache, seq_lens, window, sink, sm_scale, layout=0,
                            dtype=np.float64):
    """sparse_attention_compacted per sequence, at that sequence's length."""
    q = np.asarray(q)
    out = np.zeros(q.shape, dtype=dtype)
    for b, n in enumerate(np.asarray(seq_lens).tolist()):
        out[b] = sparse_attention_compacted(q[b:b + 1], k_cache[b:b + 1], v_cache[b:b + 1], n, window,
                                            sink, sm_scale, layout, dtype)[0]
    return out


def gather_pages(pages, block_row, n, layout="NHD"):
    """Rows [0, n) of one sequence as [KVH, n, D]: token t is row t % P of
    page block_row[t // P] (pages [num_pages, P, KVH, D] for "NHD",
    [num_pages, KVH, P, D] for "HND")."""
    pages = np.asarray(pages)
    P = pages.shape[1] if layout == "NHD" else pages.shape[2]
    t = np.arange(n)
    page = np.asarray(block_row)[t // P]
    if layout == "NHD":
        rows = pages[page, t % P]                 # [n, KVH, D]
        return np.swapaxes(rows, 0, 1)
    return np.swapaxes(pages[page, :, t % P], 0, 1)   # [n, KVH, D] -> [KVH, n, D]


def paged_attention(q, k_pages, v_pages, block_table, seq_lens, sm_scale, layout="NHD",
                    dtype=np.float64):
    """Dense decode of each sequence over its pages."""
    q = np.asarray(q)
    out = np.zeros(q.shape, dtype=dtype)
    for b, n in enumerate(np.asarray(seq_lens).tolist()):
        if n > 0:
            kb = gather_pages(k_pages, block_table[b], n, layout)[None]
            vb = gather_pages(v_pages, block_table[b], n, layout)[None]
            out[b] = dense_attention(q[b:b + 1], kb, vb, sm_scale, dtype)[0]
    return out


# --------------------------------------------------------------------------
# KIVI 2-bit quantizers
# --------------------------------------------------------------------------

def _quant_params(mn, mx, qmax=QMAX):
    """float32 scale / zero-point of one group, quant_kernel.py:79-81 (:168-170)."""
    s = (mx - mn) / F32(qmax)
    s = np.where(s == F32(0), F32(1), s).astype(F32)
    z = np.floor(-mn / s + F32(0.5)).astype(F32)
    return s, z


def _codes(x, s, z, qmax=QMAX):
    """clamp(floor(x / s + 0.5) + z, 0, QMAX), quant_kernel.py:98-99 (:184-185)."""
    c = np.floor(x / s + F32(0.5)) + z
    return np.minimum(np.maximum(c, F32(0)), F32(qmax)).astype(np.uint8)


def _width(group_size, bits):
    """QMAX and codes per byte of a ``bits``-wide code (quant_kernel.py:58-59,
    :144-145), with the reference's layout assumption of whole bytes per group."""
    if not 1 <= bits <= 8:
        raise ValueError("bits must be in 1..8")
    pf = 8 // bits
    if group_size % pf:
        raise ValueError("group_size must be a multiple of 8 // bits")
    return (1 << bits) - 1, pf


def _pack(codes, axis, pf, bits):
    """packed[.., p, ..] = sum_j code[.., pf p + j, ..] << (j bits) along ``axis``
    (quant_kernel.py:92-103, :176-190)."""
    out = np.zeros(np.take(codes, np.arange(0, codes.shape[axis], pf), axis=axis).shape, dtype=np.int32)
    for j in range(pf):
        out |= np.take(codes, np.arange(j, codes.shape[axis], pf), axis=axis).astype(np.int32) << (j * bits)
    return out.astype(np.uint8)


def quantize_k(x, group_size=32, bits=2):
    """Per-channel KIVI quantization of K.

    Restates quant_kernel.py:58-103 / :106-126.  x: [B, KVH, N, D] (any float
    dtype; converted to float32 exactly as ``.float()`` does).  Each group of
    ``group_size`` consecutive tokens gets, per channel, a float32 scale and
    zero-point; codes are packed pf = 8 // bits per byte along tokens, LSB
    first: packed[b,h,p,d] = sum_j code[b,h,pf p+j,d] << (j bits).
    Returns (packed u8 [B,KVH,N/pf,D], scale f16 [B,KVH,N/G,D], zero f16).
    """
    qmax, pf = _width(group_size, bits)
    x = np.asarray(x).astype(F32)
    B, KVH, N, D = x.shape
    if N % group_size:
        raise ValueError("this simple version assumes seq_len is a multiple of group_size")
    xg = x.reshape(B, KVH, N // group_size, group_size, D)
    mn = xg.min(axis=3)
    mx = xg.max(axis=3)
    s, z = _quant_params(mn, mx, qmax)
    codes = _codes(xg, s[:, :, :, None, :], z[:, :, :, None, :], qmax).reshape(B, KVH, N, D)
    return _pack(codes, 2, pf, bits), s.astype(F16), z.astype(F16)


def quantize_v(x, group_size=32, bits=2):
    """Per-token KIVI quantization of V.

    Restates quant_kernel.py:144-190 / :193-214: groups of ``group_size``
    consecutive channels of one token; codes packed pf = 8 // bits per byte
    along channels, LSB first: packed[b,h,t,c] = sum_j code[b,h,t,pf c+j] << (j bits).
    Returns (packed u8 [B,KVH,N,D/pf], scale f16 [B,KVH,N,D/G], zero f16).
    """
    qmax, pf = _width(group_size, bits)
    x = np.asarray(x).astype(F32)
    B, KVH, N, D = x.shape
    if D % group_size:
        raise ValueError("this simple version assumes D_HEAD is a multiple of group_size")
    xg = x.reshape(B, KVH, N, D // group_size, group_size)
    mn = xg.min(axis=4)
    mx = xg.max(axis=4)
    s, z = _quant_params(mn, mx, qmax)
    codes = _codes(xg, s[..., None], z[..., None], qmax).reshape(B, KVH, N, D)
    return _pack(codes, 3, pf, bits), s.astype(F16), z.astype(F16)


def unpack_dequant(packed, scale, zero, full_axis_len, pack_axis, group_size=32, bits=2):
    """Unpack (shift + mask, strided slice j::4) and affine dequant in float32.

    Restates test_quantize_correctness.py:16-43: pack_axis 2 for K's layout,
    3 for V's.  Value = float32(scale) * (code - float32(zero)).
    """
    qmax = (1 << bits) - 1
    pf = 8 // bits
    packed = np.asarray(packed)
    shape = list(packed.shape)
    shape[pack_axis] = full_axis_len
    codes = np.zeros(shape, dtype=F32)
    pint = packed.astype(np.int32)
    for j in range(pf):
        idx = [slice(None)] * len(shape)
        idx[pack_axis] = slice(j, None, pf)
        codes[tuple(idx)] = ((pint >> (j * bits)) & qmax).astype(F32)
    gidx = np.arange(full_axis_len) // group_size
    se = np.take(np.asarray(scale), gidx, axis=pack_axis).astype(F32)
    ze = np.take(np.asarray(zero), gidx, axis=pack_axis).astype(F32)
    return (se * (codes - ze)).astype(F32)


def _trunc_div(a, b):
    """C / Triton integer division (truncates toward zero)."""
    q = abs(a) // abs(b)
    return q if (a >= 0) == (b >= 0) else -q


def dequant_k_tile(packed, scale, zero, tok_start, num_packed, num_groups, block_n=128, group_size=32):
    """One block_n-token tile of K dequantized, with the reference's clamps.

    Restates quant_kernel.py:236-266: byte = clamp(tok_start/4 + t/4, 0,
    num_packed-1) (C division), code = (byte >> 2*(t % 4)) & 3, group =
    min(byte / 8, num_groups - 1), value = s * (code - z) in float32.
    packed: [B, KVH, num_packed, D]; returns [B, KVH, block_n, D] float32.
    """
    t = np.arange(block_n, dtype=np.int64)
    byte_idx = _trunc_div(int(tok_start), PACK_FACTOR) + t // PACK_FACTOR
    byte_idx = np.clip(byte_idx, 0, num_packed - 1)
    sub = t % PACK_FACTOR
    bpg = group_size // PACK_FACTOR
    gidx = np.minimum(byte_idx // bpg, num_groups - 1)
    pb = np.asarray(packed)[:, :, byte_idx, :].astype(np.int32)          # [B,KVH,T,D]
    code = ((pb >> (2 * sub)[None, None, :, None]) & QMAX).astype(F32)
    s = np.asarray(scale)[:, :, gidx, :].astype(F32)
    z = np.asarray(zero)[:, :, gidx, :].astype(F32)
    return (s * (code - z)).astype(F32)


def dequant_v_tile(packed, scale, zero, tok_start, seq_len, block_n=128, group_size=32):
    """One block_n-token tile of V dequantized, with the reference's clamps.

    Restates quant_kernel.py:281-311: token = clamp(tok_start + t, 0,
    seq_len - 1), byte column d/4, shift 2*(d % 4), group d / group_size.
    packed: [B, KVH, seq_len, D/4]; returns [B, KVH, block_n, D] float32.
    """
    packed = np.asarray(packed)
    D = packed.shape[-1] * PACK_FACTOR
    tok = np.clip(int(tok_start) + np.arange(block_n), 0, seq_len - 1)
    d = np.arange(D)
    pb = packed[:, :, tok][:, :, :, d // PACK_FACTOR].astype(np.int32)  # [B,KVH,T,D]
    code = ((pb >> (2 * (d % PACK_FACTOR))[None, None, None, :]) & QMAX).astype(F32)
    s = np.asarray(scale)[:, :, tok][:, :, :, d // group_size].astype(F32)
    z = np.asarray(zero)[:, :, tok][:, :, :, d // group_size].astype(F32)
    return (s * (code - z)).astype(F32)


# --------------------------------------------------------------------------
# Quantized cache builder and fused quantized decode
# --------------------------------------------------------------------------

CACHE_KEYS = (
    "k_residual", "v_residual",
    "k_sink_packed", "k_sink_scale", "k_sink_zero",
    "v_sink_packed", "v_sink_scale", "v_sink_zero",
    "k_win_packed", "k_win_scale", "k_win_zero",
    "v_win_packed", "v_win_scale", "v_win_zero",
)


def build_quantized_kv_cache(k_compacted, v_compacted, residual_size=128, sink=4, group_size=32, bits=2):
    """Split a compacted [B, KVH, sink+W, D] cache into the KIVI regimes.

    Restates quant_kernel.py:592-622: residual = last ``residual_size`` slots
    (kept in the input dtype); sink = the ``sink`` real tokens padded to one
    group by repeating token 0, quantized; window-old = slots
    [sink, sink + W - residual), quantized.  Returns the 14-key dict.
    A window W < residual (undefined in the reference) keeps the whole
    window as the residual and has no window-old part (this build's rule).
    """
    k_compacted = np.asarray(k_compacted)
    v_compacted = np.asarray(v_compacted)
    n = k_compacted.shape[2]
    residual_size = min(residual_size, n - sink)
    kres = np.ascontiguousarray(k_compacted[:, :, n - residual_size:])
    vres = np.ascontiguousarray(v_compacted[:, :, n - residual_size:])
    pad = group_size - sink

    def padded(x):
        real = x[:, :, :sink]
        return np.concatenate([real, np.repeat(real[:, :, :1], pad, axis=2)], axis=2).astype(F32)

    kwin = k_compacted[:, :, sink:n - residual_size].astype(F32)
    vwin = v_compacted[:, :, sink:n - residual_size].astype(F32)
    out = {"k_residual": kres, "v_residual": vres}
    for name, arr, fn in (("k_sink", padded(k_compacted), quantize_k),
                          ("v_sink", padded(v_compacted), quantize_v),
                          ("k_win", kwin, quantize_k),
                          ("v_win", vwin, quantize_v)):
        p, s, z = fn(arr, group_size, bits)
        out[name + "_packed"], out[name + "_scale"], out[name + "_zero"] = p, s, z
    return out


def stream_cache(k_full, v_full, prefill_len, seq_len, window, sink=4, residual_size=128,
                 group_size=32):
    """Expected contents of the decode-time KIVI cache after a prefill of
    ``prefill_len`` tokens and ``seq_len - prefill_len`` single-token appends.

    The reference has no streaming cache; its builder (quant_kernel.py:584-622,
    ``build_quantized_kv_cache`` above) is this state right after an eviction.
    Semantics: after e = (seq_len - prefill_len) // group evictions the
    residual holds positions [prefill_len - residual_size + group * e,
    seq_len) (residual_size .. residual_size + group - 1 tokens), the
    window-old groups the (window - residual_size) positions before that, in
    group-aligned blocks, and the sink the first ``sink`` positions.  So the
    state is the builder's output on the compacted cache sink + [window-old
    start, seq_len) with the residual length extended by the pending tokens.
    Returns (14-key dict with window-old in position order, win_old_len).
    k_full, v_full: [B, KVH, >= seq_len, D] (positions 0..).
    """
    L0, L = int(prefill_len), int(seq_len)
    e = (L - L0) // group_size
    res_start = L0 - residual_size + group_size * e
    wo_start = res_start - (window - residual_size)
    comp_k = np.concatenate([k_full[:, :, :sink], k_full[:, :, wo_start:L]], axis=2)
    comp_v = np.concatenate([v_full[:, :, :sink], v_full[:, :, wo_start:L]], axis=2)
    cache = build_quantized_kv_cache(comp_k, comp_v, residual_size=L - res_start, sink=sink,
                                     group_size=group_size)
    return cache, window - residual_size


def dequantized_regimes(cache, win_old_len, sink=4, group_size=32, bits=2):
    """Dequantized K and V of the whole [sink + W] cache, in slot order.

    The composition of test_quantized_attention_correctness.py:40-50: sink
    (first ``sink`` of the padded group), window-old, then the fp16 residual
    (as float32).  Returns (k, v) float32 [B, KVH, sink + W, D].
    """
    D = cache["k_sink_packed"].shape[-1]
    ks = unpack_dequant(cache["k_sink_packed"], cache["k_sink_scale"], cache["k_sink_zero"],
                        group_size, 2, group_size, bits)[:, :, :sink]
    vs = unpack_dequant(cache["v_sink_packed"], cache["v_sink_scale"], cache["v_sink_zero"],
                        D, 3, group_size, bits)[:, :, :sink]
    parts_k, parts_v = [ks], [vs]
    if win_old_len > 0:
        parts_k.append(unpack_dequant(cache["k_win_packed"], cache["k_win_scale"], cache["k_win_zero"],
                                      win_old_len, 2, group_size, bits))
        parts_v.append(unpack_dequant(cache["v_win_packed"], cache["v_win_scale"], cache["v_win_zero"],
                                      D, 3, group_size, bits))
    parts_k.append(np.asarray(cache["k_residual"]).astype(F32))
    parts_v.append(np.asarray(cache["v_residual"]).astype(F32))
    return np.concatenate(parts_k, axis=2), np.concatenate(parts_v, axis=2)


def quantized_attention(q, win_old_len, cache, sm_scale, sink=4, group_size=32, dtype=np.float64, bits=2):
    """Dequantize-then-attend composition of the three regimes.

    Restates test_quantized_attention_correctness.py:32-61 (steady state: every
    slot attended).
    """
    k, v = dequantized_regimes(cache, win_old_len, sink, group_size, bits)
    return dense_attention(q, k, v, sm_scale, dtype)


def quantized_attention_masked(q, cache, seq_len, window, sm_scale, sink=4, residual_size=128,
                               group_size=32, dtype=np.float64, bits=2):
    """What the fused quantized kernel computes, ramp-up included.

    The regime composition of quant_kernel.py:358-401 (sink slot s -> sink
    token s; window-old slot s -> window-old token s - sink; residual slot s ->
    residual row s - (sink + window - residual)) attended over the slots that
    kv_indices marks valid (quant_kernel.py:485,496).  Equals
    ``quantized_attention`` in steady state.
    """
    k, v = dequantized_regimes(cache, max(window - residual_size, 0), sink, group_size, bits)
    valid = slot_validity(seq_len, window, sink, 0)
    return masked_attention(q, k, v, valid, sm_scale, dtype)


def quantized_attention_varlen(q, cache, seq_lens, window, sm_scale, sink=4, residual_size=128,
                               group_size=32, dtype=np.float64, bits=2):
    """quantized_attention_masked per sequence, at that sequence's length
    (the reference's call at one scalar length, quant_kernel.py:551-581,
    applied to each batch row)."""
    q = np.asarray(q)
    out = np.zeros(q.shape, dtype=dtype)
    for b, n in enumerate(np.asarray(seq_lens).tolist()):
        cb = {key: np.asarray(val)[b:b + 1] for key, val in cache.items()}
        out[b] = quantized_attention_masked(q[b:b + 1], cb, n, window, sm_scale, sink, residual_size,
                                            group_size, dtype, bits)[0]
    return out


# --------------------------------------------------------------------------
# Byte models (benchmark.py:30-31,56-57,121-129)
# --------------------------------------------------------------------------

def bytes_dense(B, H, KVH, L, D, elt=2):
    """Q + O + K + V bytes of one dense step: 1,048,576 + 131,072 * L at the constants."""
    return 2 * B * H * D * elt + 2 * B * KVH * L * D * elt
