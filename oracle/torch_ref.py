"""PyTorch (CPU) restatement of the reference's own test oracles.  TEST AND
BASELINE INFRASTRUCTURE ONLY.

The reference checks its Triton kernels against plain-PyTorch functions in
its test files; those functions are "the repo's PyTorch reference" that the
CPU baseline times.  This module restates them for torch CPU tensors so that
``bench.py``'s ``cpu_baseline`` leg can time the same computation on the
host cores.  ``tests/test_oracle.py`` pins every function here against the
numpy oracle (``oracle/kvdec_oracle.py``), itself pinned by closed forms and
brute force.  Nothing in the package imports this module.

  dense_attention      test_dense_correctness.py:13-30 (GQA by reshaping q
                       into KV-head groups, no repeated K/V copy)
  sparse_attention     test_sparse_correctness.py:22-48 (the streaming-llm
                       validity mask) applied to the compacted
                       [sink + window] cache the kernel reads
                       (sparse_kernel.py:15-46 slot rule)
  unpack_dequant       test_quantize_correctness.py:16-43
  quantized_attention  test_quantized_attention_correctness.py:32-61
"""

from __future__ import annotations

import torch


def _grouped(q, kv_heads):
    B, H, D = q.shape
    return q.reshape(B, kv_heads, H // kv_heads, D)


def dense_attention(q, k, v, sm_scale, valid=None):
    """softmax(q K^T * sm_scale) V per query head, query head h reading KV
    head h // (H / KVH).  q [B, H, D]; k, v [B, KVH, N, D]; valid: optional
    [N] bool mask of attended slots.  Computes in q's dtype."""
    B, H, D = q.shape
    KVH = k.shape[1]
    logits = torch.matmul(_grouped(q, KVH), k.transpose(-1, -2)) * sm_scale   # [B, KVH, G, N]
    if valid is not None:
        logits = logits.masked_fill(~valid, float("-inf"))
    return torch.matmul(torch.softmax(logits, dim=-1), v).reshape(B, H, D)


def slot_validity(seq_len, window, sink, n_slots):
    """Attended slots of the compacted linear-layout cache at ``seq_len``:
    the sink slots holding real tokens, and the window slots whose position
    seq_len - window + (slot - sink) is past the sink (ramp-up leaves the
    first ones unwritten)."""
    s = torch.arange(n_slots)
    return torch.where(s < sink, s < seq_len, seq_len - window + (s - sink) >= sink) & (s < sink + window)


def sparse_attention(q, k_cache, v_cache, seq_len, window, sink, sm_scale):
    """Sink + window decode over the compacted [B, KVH, sink + window, D] cache."""
    valid = slot_validity(int(seq_len), int(window), int(sink), k_cache.shape[2])
    return dense_attention(q, k_cache, v_cache, sm_scale, valid)


def unpack_dequant(packed, scale, zero, full_len, axis, group_size=32, bits=2):
    """scale * (code - zero) with the codes unpacked LSB-first along ``axis``
    (2: K's tokens, 3: V's channels) and scale / zero broadcast per group."""
    per_byte = 8 // bits
    mask = (1 << bits) - 1
    p = packed.to(torch.int32)
    # code j of every byte, then interleave: element per_byte * i + j
    codes = torch.stack([(p >> (bits * j)) & mask for j in range(per_byte)], dim=axis + 1)
    shape = list(packed.shape)
    shape[axis] = full_len
    codes = codes.reshape(shape).to(torch.float32)
    grp = torch.arange(full_len) // group_size
    s = scale.to(torch.float32).index_select(axis, grp)
    z = zero.to(torch.float32).index_select(axis, grp)
    return s * (codes - z)


def quantized_attention(q, win_old_len, cache, sm_scale, sink=4, group_size=32):
    """Dequantize the sink group (first ``sink`` tokens), the window-old
    groups and the fp16 residual, concatenate in slot order, attend (every
    slot valid: steady state).  Float32 throughout."""
    D = cache["k_sink_packed"].shape[-1]
    ks = unpack_dequant(cache["k_sink_packed"], cache["k_sink_scale"], cache["k_sink_zero"],
                        group_size, 2, group_size)[:, :, :sink]
    vs = unpack_dequant(cache["v_sink_packed"], cache["v_sink_scale"], cache["v_sink_zero"],
                        D, 3, group_size)[:, :, :sink]
    ks_, vs_ = [ks], [vs]
    if win_old_len > 0:
        ks_.append(unpack_dequant(cache["k_win_packed"], cache["k_win_scale"], cache["k_win_zero"],
                                  win_old_len, 2, group_size))
        vs_.append(unpack_dequant(cache["v_win_packed"], cache["v_win_scale"], cache["v_win_zero"],
                                  D, 3, group_size))
    ks_.append(cache["k_residual"].to(torch.float32))
    vs_.append(cache["v_residual"].to(torch.float32))
    return dense_attention(q.to(torch.float32), torch.cat(ks_, dim=2), torch.cat(vs_, dim=2), sm_scale)
