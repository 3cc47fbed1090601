"""Sink + window sparse decode on the GPU vs the CPU oracle (restates the
reference's test_sparse_correctness.py: streaming-llm mask over the full
context, 1e4 garbage in not-yet-written slots)."""

import numpy as np
import pytest
import torch

from conftest import load_golden
from helpers import ATTN_TOL, REF_TOL, SCALE, dev, host, max_abs, randn, say
from oracle import kvdec_oracle as O

pytestmark = pytest.mark.gpu

S = 4


def _run(q16, kc16, vc16, L, W, device, layout="linear"):
    from sparse_kernel import sparse_decode_attention
    o = sparse_decode_attention(dev(q16, device), dev(kc16, device), dev(vc16, device), seq_len=L,
                                window=W, layout=layout)
    torch.cuda.synchronize()
    return host(o)


def test_sparse_golden(device):
    g = load_golden("sparse_golden.npz")
    W = int(g["window"])
    for tag in ("ramp", "steady"):
        say(f"sparse golden {tag}")
        o = _run(g[f"{tag}_q"], g[f"{tag}_k"], g[f"{tag}_v"], int(g[f"{tag}_seq_len"]), W, device)
        assert max_abs(o, g[f"{tag}_o"]) < ATTN_TOL


@pytest.mark.parametrize("L,W", [(2, 256), (100, 256), (5000, 256), (2, 0), (10000, 0)])
def test_sparse_reference_cases(L, W, device):
    """The reference's five cases: pre-sink, ramp-up, steady state, W=0."""
    B, H, KVH, D = 8, 64, 8, 128
    q = randn((B, H, D), 11 + L)
    kf = randn((B, KVH, L, D), 12 + L)
    vf = randn((B, KVH, L, D), 13 + L)
    kc, vc = O.build_compacted_cache(kf, vf, L, W, S)
    q16, kc16, vc16 = q.astype(np.float16), kc.astype(np.float16), vc.astype(np.float16)
    say(f"sparse L={L} W={W}")
    o = _run(q16, kc16, vc16, L, W, device)
    assert max_abs(o, O.sparse_attention_compacted(q16, kc16, vc16, L, W, S, SCALE)) < ATTN_TOL
    ref32 = O.sparse_attention_full(q, kf, vf, L, W, S, SCALE, dtype=np.float32)
    assert max_abs(o, ref32) < REF_TOL


@pytest.mark.parametrize("W", [0, 4, 32, 60])
def test_sparse_every_length_through_rampup(W, device):
    """Brute force over every seq_len from 1 to past the ramp-up, linear and
    ring layouts, garbage in unwritten slots."""
    B, H, KVH, D = 2, 16, 2, 128
    Lmax = S + W + 40
    q16 = randn((B, H, D), 21, np.float16)
    kf = randn((B, KVH, Lmax, D), 22, np.float16)
    vf = randn((B, KVH, Lmax, D), 23, np.float16)
    say(f"sparse sweep W={W}")
    for L in range(1, Lmax + 1):
        ref = O.sparse_attention_full(q16, kf, vf, L, W, S, SCALE)
        kc, vc = O.build_compacted_cache(kf, vf, L, W, S)
        assert max_abs(_run(q16, kc, vc, L, W, device), ref) < ATTN_TOL, ("linear", L)
        if W > 0:
            kr, vr = O.build_ring_cache(kf, vf, L, W, S)
            assert max_abs(_run(q16, kr, vr, L, W, device, "ring"), ref) < ATTN_TOL, ("ring", L)


@pytest.mark.parametrize("W", [256, 1024, 4096, 16384])
def test_sparse_steady_state_windows(W, device):
    """Config-3 shape (B=32, logical L=163840, every slot valid), incl. the
    split-K path at large W; ring layout gives the same result."""
    B, H, KVH, D, L = 32, 64, 8, 128, 163840
    gen = torch.Generator(device=device).manual_seed(W)
    say(f"sparse steady W={W}")
    q = torch.randn(B, H, D, generator=gen, device=device, dtype=torch.float16)
    kc = torch.randn(B, KVH, S + W, D, generator=gen, device=device, dtype=torch.float16)
    vc = torch.randn(B, KVH, S + W, D, generator=gen, device=device, dtype=torch.float16)
    from sparse_kernel import sparse_decode_attention
    o = host(sparse_decode_attention(q, kc, vc, seq_len=L, window=W))
    o_ring = host(sparse_decode_attention(q, kc, vc, seq_len=L, window=W, layout="ring"))
    torch.cuda.synchronize()
    for b in (0, 17, 31):
        ref = O.dense_attention(host(q[b:b + 1]), host(kc[b:b + 1]), host(vc[b:b + 1]), SCALE)
        assert max_abs(o[b:b + 1], ref) < ATTN_TOL, b
    assert max_abs(o, o_ring) < 1e-3


@pytest.mark.parametrize("G", [1, 4, 12, 16])
@pytest.mark.parametrize("W", [60, 256, 1024])
def test_sparse_query_group_sizes(G, W, device):
    """Query groups of 1..16 heads through both fp16 kernels (W <= 476: the
    single-pass lean kernel with interleaved tiles; W=1024: the work-queue
    kernel), steady state and ramp-up, each output correctly rounded."""
    from helpers import assert_nearly_rounded
    B, KVH, D = 3, 2, 128
    H = G * KVH
    for L in (S + W // 2, 100000):
        q16 = randn((B, H, D), 31 + G + L, np.float16)
        kf = randn((B, KVH, min(L, S + W + 8), D), 32 + W, np.float16)
        vf = randn((B, KVH, min(L, S + W + 8), D), 33 + W, np.float16)
        n = min(L, S + W)
        kc = np.zeros((B, KVH, S + W, D), np.float16)
        vc = np.zeros((B, KVH, S + W, D), np.float16)
        kc[:, :, :n] = kf[:, :, :n]
        vc[:, :, :n] = vf[:, :, :n]
        say(f"sparse G={G} W={W} L={L}")
        o = _run(q16, kc, vc, L, W, device)
        ref = O.sparse_attention_compacted(q16, kc, vc, L, W, S, SCALE)
        assert_nearly_rounded(o, ref)


def test_sparse_rejects_bad_cache_shape(device):
    from sparse_kernel import sparse_decode_attention
    q = torch.zeros(2, 64, 128, dtype=torch.float16, device=device)
    kc = torch.zeros(2, 8, 259, 128, dtype=torch.float16, device=device)
    with pytest.raises(ValueError):
        sparse_decode_attention(q, kc, kc, seq_len=1000, window=256)
    with pytest.raises(ValueError):
        sparse_decode_attention(q, kc, kc, seq_len=1000, window=255, layout="spiral")


@pytest.mark.parametrize("W", [508, 512])
def test_sparse_sixteen_tiles_and_a_tail(W, device):
    """W=508 fills the lean kernel's 16 tiles exactly; W=512 (516 slots)
    adds a tail of 4 rows that the lean kernel's last wave steps first.
    Steady state (both layouts), ramp-up through the tail, and 1e4 garbage
    in slots not yet written."""
    B, H, KVH, D = 4, 64, 8, 128
    q = randn((B, H, D), W).astype(np.float16)
    kc = randn((B, KVH, S + W, D), W + 1).astype(np.float16)
    vc = randn((B, KVH, S + W, D), W + 2).astype(np.float16)
    for L, layout in ((163840, "linear"), (163840, "ring"), (S + W - 2, "linear"), (S + W - 2, "ring"),
                      (300, "linear")):
        say(f"sparse W={W} L={L} {layout}")
        valid = O.slot_validity(L, W, S, 0 if layout == "linear" else 1)
        k = np.where(valid[None, None, :, None], kc, np.float16(1e4))
        v = np.where(valid[None, None, :, None], vc, np.float16(1e4))
        o = _run(q, k, v, L, W, device, layout=layout)
        ref = O.masked_attention(q, kc, vc, valid, SCALE)
        assert max_abs(o, ref) < ATTN_TOL, (L, layout)
