"""Per-sequence lengths, strided and paged caches on the GPU vs the CPU
oracle.  The reference passes one scalar seq_len and a contiguous cache
(dense_kernel.py:70-82, sparse_kernel.py:105-118); each sequence here must
give what that call gives at its own length over its own rows."""

import numpy as np
import pytest
import torch

from helpers import ATTN_TOL, SCALE, dev, host, max_abs, randn, say
from oracle import kvdec_oracle as O

pytestmark = pytest.mark.gpu

S = 4


def _lens(device, *vals):
    return torch.tensor(vals, dtype=torch.int32, device=device)


def test_dense_varlen(device):
    """Lengths around the tile (32) and half-tile (16) edges, 1, L_max and
    0; rows past each length hold garbage, NaN included."""
    from dense_kernel import dense_decode_attention
    lens = [1, 15, 16, 17, 31, 32, 33, 0, 1000, 2999, 3000]
    B, H, KVH, D, L = len(lens), 32, 8, 128, 3000
    q = randn((B, H, D), 1, np.float16)
    k = randn((B, KVH, L, D), 2, np.float16)
    v = randn((B, KVH, L, D), 3, np.float16)
    ref = O.dense_attention_varlen(q, k, v, lens, SCALE)
    for b, n in enumerate(lens):
        k[b, :, n:] = np.float16(1e4) if b % 2 else np.float16(np.nan)
        v[b, :, n:] = np.float16(np.nan) if b % 2 else np.float16(-1e4)
    say("dense varlen")
    o = dense_decode_attention(dev(q, device), dev(k, device), dev(v, device), _lens(device, *lens))
    torch.cuda.synchronize()
    o = host(o)
    assert np.all(o[lens.index(0)] == 0)
    assert max_abs(o, ref) < ATTN_TOL


@pytest.mark.parametrize("L", [4096, 163840])
def test_dense_varlen_split_path(L, device):
    """Long caches take the split-K path: per-sequence lengths across the
    splits (some sequences end inside the first split, some are empty)."""
    from dense_kernel import dense_decode_attention
    B, H, KVH, D = 4, 64, 8, 128
    gen = torch.Generator(device=device).manual_seed(L)
    q = torch.randn(B, H, D, generator=gen, device=device, dtype=torch.float16)
    k = torch.randn(B, KVH, L, D, generator=gen, device=device, dtype=torch.float16)
    v = torch.randn(B, KVH, L, D, generator=gen, device=device, dtype=torch.float16)
    lens = [L, L // 3 + 7, 0, 45]
    say(f"dense varlen split L={L}")
    o = dense_decode_attention(q, k, v, _lens(device, *lens))
    full = dense_decode_attention(q, k, v, L)
    torch.cuda.synchronize()
    assert torch.all(o[2] == 0)
    # sequence 0 is full length: same attention as the contiguous call
    assert float((o[0].float() - full[0].float()).abs().max()) < ATTN_TOL
    qh, kh, vh = host(q), host(k), host(v)
    for b in (1, 3):
        n = lens[b]
        ref = O.dense_attention(qh[b:b + 1], kh[b:b + 1, :, :n], vh[b:b + 1, :, :n], SCALE)
        assert max_abs(host(o[b:b + 1]), ref) < ATTN_TOL, b


def test_dense_strided_views(device):
    """A [B, L, KVH, D] cache seen as [B, KVH, L, D] (permuted view), and a
    slice of a longer cache, give the contiguous call's attention."""
    from dense_kernel import dense_decode_attention
    B, H, KVH, D, L = 3, 16, 4, 128, 1000
    q = randn((B, H, D), 5, np.float16)
    kb = randn((B, L + 77, KVH, D), 6, np.float16)
    vb = randn((B, L + 77, KVH, D), 7, np.float16)
    k = torch.from_numpy(kb).to(device).permute(0, 2, 1, 3)[:, :, :L]
    v = torch.from_numpy(vb).to(device).permute(0, 2, 1, 3)[:, :, :L]
    assert not k.is_contiguous()
    say("dense strided")
    o = dense_decode_attention(dev(q, device), k, v, L)
    torch.cuda.synchronize()
    ref = O.dense_attention(q, np.swapaxes(kb, 1, 2)[:, :, :L], np.swapaxes(vb, 1, 2)[:, :, :L], SCALE)
    assert max_abs(host(o), ref) < ATTN_TOL


def _paged(k, v, lens, page_size, layout, seed, extra_pages=5, bad_id=None):
    """Scatter [B, KVH, L, D] into pages in a random order: (k_pages,
    v_pages, block_table) with unused table entries -1."""
    B, KVH, L, D = k.shape
    nblk = [(n + page_size - 1) // page_size for n in lens]
    max_blocks = max(1, (L + page_size - 1) // page_size)
    num_pages = sum(nblk) + extra_pages
    rng = np.random.default_rng(seed)
    perm = rng.permutation(num_pages)
    shape = (num_pages, page_size, KVH, D) if layout == "NHD" else (num_pages, KVH, page_size, D)
    kp = rng.standard_normal(shape).astype(np.float16) * np.float16(100)   # garbage in free pages
    vp = rng.standard_normal(shape).astype(np.float16) * np.float16(100)
    table = np.full((B, max_blocks), -1, dtype=np.int32)
    nxt = 0
    for b in range(B):
        for j in range(nblk[b]):
            p = perm[nxt]
            nxt += 1
            table[b, j] = p
            rows = slice(j * page_size, min((j + 1) * page_size, L))
            n = rows.stop - rows.start
            if layout == "NHD":
                kp[p, :n] = np.swapaxes(k[b, :, rows], 0, 1)
                vp[p, :n] = np.swapaxes(v[b, :, rows], 0, 1)
            else:
                kp[p, :, :n] = k[b, :, rows]
                vp[p, :, :n] = v[b, :, rows]
    return kp, vp, table


@pytest.mark.parametrize("layout", ["NHD", "HND"])
@pytest.mark.parametrize("page_size", [16, 32, 64, 256])
def test_paged_matches_oracle(layout, page_size, device):
    from paged_kernel import paged_decode_attention
    lens = [1, 16, 17, 40, 511, 0, 700, 1024]
    B, H, KVH, D, L = len(lens), 64, 8, 128, 1024
    q = randn((B, H, D), 30 + page_size, np.float16)
    k = randn((B, KVH, L, D), 31 + page_size, np.float16)
    v = randn((B, KVH, L, D), 32 + page_size, np.float16)
    kp, vp, table = _paged(k, v, lens, page_size, layout, page_size)
    say(f"paged {layout} page_size={page_size}")
    o = paged_decode_attention(dev(q, device), dev(kp, device), dev(vp, device), dev(table, device),
                               _lens(device, *lens), max_seq_len=L, kv_layout=layout)
    torch.cuda.synchronize()
    o = host(o)
    ref = O.paged_attention(q, kp, vp, table, lens, SCALE, layout)
    assert max_abs(o, ref) < ATTN_TOL
    # the paged oracle is the varlen oracle over the original rows
    assert max_abs(ref, O.dense_attention_varlen(q, k, v, lens, SCALE)) < 1e-12


def test_paged_without_max_len_and_bad_page_ids(device):
    """max_seq_len read back from seq_lens; a page id past the pool reads as
    zero rows (attention over zero K and V rows for those tokens)."""
    from paged_kernel import paged_decode_attention
    lens = [300, 64]
    B, H, KVH, D, L = 2, 8, 2, 128, 300
    q = randn((B, H, D), 40, np.float16)
    k = randn((B, KVH, L, D), 41, np.float16)
    v = randn((B, KVH, L, D), 42, np.float16)
    kp, vp, table = _paged(k, v, lens, 32, "NHD", 3)
    table[0, 2] = kp.shape[0] + 1000     # tokens 64..95 of sequence 0
    say("paged bad page id")
    o = paged_decode_attention(dev(q, device), dev(kp, device), dev(vp, device), dev(table, device),
                               _lens(device, *lens))
    torch.cuda.synchronize()
    kz, vz = k.copy(), v.copy()
    kz[0, :, 64:96] = 0
    vz[0, :, 64:96] = 0
    assert max_abs(host(o), O.dense_attention_varlen(q, kz, vz, lens, SCALE)) < ATTN_TOL


@pytest.mark.parametrize("page_size", [16, 128])
def test_paged_bench_size_matches_contiguous(page_size, device):
    """B=32, H=64, KVH=8, L=163840 (the dense benchmark's shape) scattered
    over pages in a random order: the paged decode equals the contiguous
    dense decode of the same cache."""
    from dense_kernel import dense_decode_attention
    from paged_kernel import paged_decode_attention
    B, H, KVH, D, L = 32, 64, 8, 128, 163840
    gen = torch.Generator(device=device).manual_seed(page_size)
    q = torch.randn(B, H, D, generator=gen, device=device, dtype=torch.float16)
    k = torch.randn(B, KVH, L, D, generator=gen, device=device, dtype=torch.float16)
    v = torch.randn(B, KVH, L, D, generator=gen, device=device, dtype=torch.float16)
    say(f"paged bench size page_size={page_size}")
    full = dense_decode_attention(q, k, v, L)
    nb = L // page_size
    perm = torch.randperm(B * nb, generator=torch.Generator().manual_seed(7)).to(device)
    table = perm.view(B, nb).to(torch.int32)
    # page p = table[b, j] holds tokens [j * page_size, +page_size) of sequence b, NHD
    kp = torch.empty(B * nb, page_size, KVH, D, dtype=torch.float16, device=device)
    vp = torch.empty_like(kp)
    kp[table.view(-1).long()] = k.view(B, KVH, nb, page_size, D).permute(0, 2, 3, 1, 4).reshape(-1, page_size, KVH, D)
    vp[table.view(-1).long()] = v.view(B, KVH, nb, page_size, D).permute(0, 2, 3, 1, 4).reshape(-1, page_size, KVH, D)
    del k, v
    o = paged_decode_attention(q, kp, vp, table, _lens(device, *([L] * B)), max_seq_len=L)
    torch.cuda.synchronize()
    assert float((o.float() - full.float()).abs().max()) < 1e-3


@pytest.mark.parametrize("layout", ["linear", "ring"])
@pytest.mark.parametrize("W", [0, 60, 256])
def test_sparse_varlen(layout, W, device):
    """Each sequence at its own length (pre-sink, ramp-up, steady state),
    garbage in its unwritten slots."""
    from sparse_kernel import sparse_decode_attention
    if layout == "ring" and W == 0:
        pytest.skip("the ring layout needs a window")
    lens = [1, 3, 4, 5, S + W - 1, S + W, S + W + 1, 5000]
    B, H, KVH, D = len(lens), 16, 4, 128
    q = randn((B, H, D), 50 + W, np.float16)
    kf = randn((B, KVH, max(lens), D), 51 + W, np.float16)
    vf = randn((B, KVH, max(lens), D), 52 + W, np.float16)
    build = O.build_compacted_cache if layout == "linear" else O.build_ring_cache
    kc = np.zeros((B, KVH, S + W, D), np.float16)
    vc = np.zeros((B, KVH, S + W, D), np.float16)
    ref = np.zeros((B, H, D))
    for b, n in enumerate(lens):
        kb, vb = build(kf[b:b + 1], vf[b:b + 1], n, W, S)
        kc[b], vc[b] = kb[0], vb[0]
        ref[b] = O.sparse_attention_full(q[b:b + 1], kf[b:b + 1, :, :n], vf[b:b + 1, :, :n], n, W, S,
                                         SCALE)[0]
    say(f"sparse varlen {layout} W={W}")
    o = sparse_decode_attention(dev(q, device), dev(kc, device), dev(vc, device), _lens(device, *lens),
                                window=W, layout=layout)
    torch.cuda.synchronize()
    o = host(o)
    assert max_abs(o, ref) < ATTN_TOL
    lay = 0 if layout == "linear" else 1
    assert max_abs(o, O.sparse_attention_varlen(q, kc, vc, lens, W, S, SCALE, lay)) < ATTN_TOL
