"""Dense decode attention over a paged KV cache on MI355X (gfx950).

The reference decodes one scalar seq_len over a contiguous [B, KVH, L, D]
cache (dense_kernel.py:70-82).  Serving engines keep K/V in fixed-size pages
shared by all sequences, with a block table per sequence and one length per
sequence; this module is that caller's form of the same attention, on the
same split-K kernel: each 32-token tile is fetched as two 16-row halves,
each from the page the block table names (page ids come through the scalar
cache, one per half).

Page layouts (kv_layout):
  "NHD"  k_pages [num_pages, page_size, N_KV_HEADS, D_HEAD]  (token-major)
  "HND"  k_pages [num_pages, N_KV_HEADS, page_size, D_HEAD]  (head-major)
page_size is a power of two >= 16; D_HEAD == 128; fp16.
"""

import torch

from constants import D_HEAD
import _checks
import _kvdec as K

_LAYOUTS = ("NHD", "HND")


def paged_decode_attention(q, k_pages, v_pages, block_table, seq_lens, max_seq_len=None,
                           sm_scale=None, kv_layout="NHD"):
    """q: [B, N_HEADS, D_HEAD] fp16; block_table: [B, max_blocks] int32
    (token t of sequence b is row t % page_size of page block_table[b,
    t // page_size]); seq_lens: [B] int32.  Returns o [B, N_HEADS, D_HEAD].

    max_seq_len bounds every length (the launch is planned for it); None
    reads seq_lens.max() back to the host, which synchronises.  Lengths are
    clamped into [0, max_seq_len] on the device; a length of 0 gives zeros;
    page ids outside [0, num_pages) read as zeros.
    """
    if kv_layout not in _LAYOUTS:
        raise ValueError(f"kv_layout must be one of {_LAYOUTS}, got {kv_layout!r}")
    _checks.require_gpu_tensor("q", q, ndim=3)
    _checks.require_gpu_tensor("k_pages", k_pages, ndim=4, contiguous=False)
    _checks.require_gpu_tensor("v_pages", v_pages, ndim=4, contiguous=False)
    _checks.require_gpu_tensor("block_table", block_table, dtypes=(torch.int32,), ndim=2)
    _checks.require_same_device(("q", q), ("k_pages", k_pages), ("v_pages", v_pages),
                                ("block_table", block_table))
    B, H, D = q.shape
    _checks.seq_lens_tensor("seq_lens", seq_lens, B, q.device)
    if kv_layout == "NHD":
        num_pages, page_size, KVH, Dk = k_pages.shape
        sp, sr, sh, _ = k_pages.stride()
    else:
        num_pages, KVH, page_size, Dk = k_pages.shape
        sp, sh, sr, _ = k_pages.stride()
    _checks.require_shape("k_pages", k_pages, tuple(k_pages.shape[:3]) + (D,))
    _checks.require_shape("v_pages", v_pages, tuple(k_pages.shape))
    _checks.row_major_rows("k_pages", k_pages)
    if k_pages.stride() != v_pages.stride():
        raise ValueError(f"k_pages and v_pages must share strides, got {k_pages.stride()} and "
                         f"{v_pages.stride()}")
    if block_table.shape[0] != B:
        raise ValueError(f"block_table must have {B} rows, got {tuple(block_table.shape)}")
    max_blocks = block_table.shape[1]
    if max_seq_len is None:
        max_seq_len = int(seq_lens.max().item()) if B else 0
    max_seq_len = max(int(max_seq_len), 1)
    o = torch.empty_like(q)
    if sm_scale is None:
        sm_scale = D_HEAD**-0.5
    ws, nbytes = K.workspace(K.KIND_DENSE, B, H, KVH, max_seq_len, D, q.device)
    rc = K.lib.kvdec_paged_decode(K.ptr(q), K.ptr(k_pages), K.ptr(v_pages), K.ptr(block_table),
                                  K.ptr(seq_lens), K.ptr(o), K.F16, B, H, KVH, D, max_seq_len,
                                  page_size, max_blocks, num_pages, sp, sr, sh, float(sm_scale),
                                  K.ptr(ws), nbytes, K.stream_of(q))
    K.check(rc, "paged_decode_attention")
    return o
