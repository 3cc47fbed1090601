"""Decode steps captured in a HIP graph (torch.cuda.CUDAGraph) and replayed:
every replay, with eager work and synchronisations in between, must give
the eager result.  Covers the paths a decode loop captures: the split-K
dense decode (workspace + merge kernel), the fused KIVI decode, the paged
decode and a step of the per-sequence streaming cache (bookkeeping,
evictions, decode), whose state advances on every replay."""

import numpy as np
import pytest
import torch

from helpers import ATTN_TOL, host, max_abs, say

pytestmark = pytest.mark.gpu

S = 4


def _capture(fn):
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()                                   # warm-up outside the graph
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = fn()
    return g, out


def _replays(g, out, want, scratch, n=4):
    for i in range(n):
        scratch.normal_()                      # unrelated eager work between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert max_abs(host(out), want) < ATTN_TOL, i


def test_graph_dense_split_path(device):
    """B=2 at L=20000 runs split-K (workspace written by the attention
    kernel, combined by the merge kernel)."""
    from dense_kernel import dense_decode_attention
    import _kvdec as K
    B, H, KVH, D, L = 2, 16, 2, 128, 20000
    assert K.lib.kvdec_num_splits(K.KIND_DENSE, B, KVH, L) > 1
    gen = torch.Generator(device=device).manual_seed(1)
    q = torch.randn(B, H, D, generator=gen, device=device, dtype=torch.float16)
    k = torch.randn(B, KVH, L, D, generator=gen, device=device, dtype=torch.float16)
    v = torch.randn(B, KVH, L, D, generator=gen, device=device, dtype=torch.float16)
    want = host(dense_decode_attention(q, k, v, L))
    say("graph dense split")
    g, out = _capture(lambda: dense_decode_attention(q, k, v, L))
    _replays(g, out, want, torch.empty(1 << 20, device=device))


def test_graph_kivi_and_paged(device):
    from paged_kernel import paged_decode_attention
    from quant_kernel import build_quantized_kv_cache, sparse_decode_attention_quantized
    B, H, KVH, D, W = 4, 32, 4, 128, 1024
    gen = torch.Generator(device=device).manual_seed(2)
    q = torch.randn(B, H, D, generator=gen, device=device, dtype=torch.float16)
    kc = torch.randn(B, KVH, S + W, D, generator=gen, device=device, dtype=torch.float16)
    vc = torch.randn(B, KVH, S + W, D, generator=gen, device=device, dtype=torch.float16)
    c = build_quantized_kv_cache(kc, vc)
    args = [c[n] for n in ("k_residual", "v_residual", "k_sink_packed", "k_sink_scale", "k_sink_zero",
                           "v_sink_packed", "v_sink_scale", "v_sink_zero", "k_win_packed", "k_win_scale",
                           "k_win_zero", "v_win_packed", "v_win_scale", "v_win_zero")]

    def kivi():
        return sparse_decode_attention_quantized(q, *args, seq_len=100000, window=W)

    want = host(kivi())
    say("graph kivi")
    g, out = _capture(kivi)
    scratch = torch.empty(1 << 20, device=device)
    _replays(g, out, want, scratch)

    # paged: the same fp16 window as 16-token pages in reverse order
    L, ps = S + W, 16
    nb = -(-L // ps)
    table = torch.arange(B * nb, device=device, dtype=torch.int32).flip(0).view(B, nb).contiguous()
    kp = torch.zeros(B * nb, ps, KVH, D, dtype=torch.float16, device=device)
    vp = torch.zeros_like(kp)
    pad = nb * ps - L
    kpad = torch.nn.functional.pad(kc, (0, 0, 0, pad)).view(B, KVH, nb, ps, D).permute(0, 2, 3, 1, 4)
    vpad = torch.nn.functional.pad(vc, (0, 0, 0, pad)).view(B, KVH, nb, ps, D).permute(0, 2, 3, 1, 4)
    kp[table.view(-1).long()] = kpad.reshape(-1, ps, KVH, D)
    vp[table.view(-1).long()] = vpad.reshape(-1, ps, KVH, D)
    lens = torch.full((B,), L, dtype=torch.int32, device=device)

    def paged():
        return paged_decode_attention(q, kp, vp, table, lens, max_seq_len=L)

    want = host(paged())
    say("graph paged")
    g, out = _capture(paged)
    _replays(g, out, want, scratch)


def test_graph_stream_batch_step(device):
    """A captured step of KiviStreamBatch (plan, evictions, decode) advances
    the on-GPU state on every replay: the outputs of N replays equal N
    eager steps on an identical cache."""
    from kivi_stream import KiviStreamBatch
    B, H, KVH, D, W = 3, 16, 2, 128, 256
    L0 = S + W + 11
    gen = torch.Generator(device=device).manual_seed(3)
    k = torch.randn(B, KVH, L0, D, generator=gen, device=device, dtype=torch.float16)
    v = torch.randn(B, KVH, L0, D, generator=gen, device=device, dtype=torch.float16)
    q = torch.randn(B, H, D, generator=gen, device=device, dtype=torch.float16)
    kn = torch.randn(B, KVH, D, generator=gen, device=device, dtype=torch.float16)
    vn = torch.randn(B, KVH, D, generator=gen, device=device, dtype=torch.float16)
    active = torch.tensor([1, 1, 0], dtype=torch.int32, device=device)
    eager = KiviStreamBatch.from_prefill(k, v, W)
    graphed = KiviStreamBatch.from_prefill(k, v, W)

    def step(c):
        c.append(kn, vn, active)
        return c.attend(q)

    say("graph stream batch")
    warm = KiviStreamBatch.from_prefill(k, v, W)   # warm-up on a cache of its own
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step(warm)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = step(graphed)                    # captured, not run
    for i in range(40):                        # crosses an eviction (every 32 appends)
        want = host(step(eager))
        g.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(host(out), want, err_msg=str(i))
    np.testing.assert_array_equal(host(graphed.appended), host(eager.appended))


def test_graph_stream_step_attend(device):
    """A captured step_attend (one launch: row write, eviction, bookkeeping,
    decode) advances the cache on every replay: 40 replays (crossing an
    eviction) equal 40 eager calls on an identical cache."""
    from kivi_stream import KiviStreamBatch
    B, H, KVH, D, W = 3, 16, 2, 128, 256
    L0 = S + W + 5
    gen = torch.Generator(device=device).manual_seed(4)
    k = torch.randn(B, KVH, L0, D, generator=gen, device=device, dtype=torch.float16)
    v = torch.randn(B, KVH, L0, D, generator=gen, device=device, dtype=torch.float16)
    q = torch.randn(B, H, D, generator=gen, device=device, dtype=torch.float16)
    kn = torch.randn(B, KVH, D, generator=gen, device=device, dtype=torch.float16)
    vn = torch.randn(B, KVH, D, generator=gen, device=device, dtype=torch.float16)
    active = torch.tensor([1, 0, 1], dtype=torch.int32, device=device)
    eager = KiviStreamBatch.from_prefill(k, v, W)
    graphed = KiviStreamBatch.from_prefill(k, v, W)
    warm = KiviStreamBatch.from_prefill(k, v, W)
    say("graph stream step_attend")
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        warm.step_attend(q, kn, vn, active)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = graphed.step_attend(q, kn, vn, active)   # captured, not run
    for i in range(40):
        want = host(eager.step_attend(q, kn, vn, active))
        g.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(host(out), want, err_msg=str(i))
    np.testing.assert_array_equal(host(graphed.ring), host(eager.ring))
    np.testing.assert_array_equal(host(graphed.appended), host(eager.appended))
    for name in eager.t:
        if name in ("k_ring", "v_ring"):   # free rows hold whatever the allocation held
            for b, (start, count) in enumerate(host(eager.ring)):
                rows = [(start + i) % eager.cap for i in range(count)]
                np.testing.assert_array_equal(host(graphed.t[name][b])[:, rows], host(eager.t[name][b])[:, rows])
        else:
            np.testing.assert_array_equal(host(graphed.t[name]), host(eager.t[name]), err_msg=name)
