"""kvdec_dense_decode_noalloc (the entry point that allocates nothing; its
split-K partials live in the library's own device array) against
kvdec_dense_decode with a torch workspace: two calls in a row, the second on
a smaller problem, each bit-identical to the workspace entry point (same
kernels, same split plan) and within the attention gate of the fp64 oracle."""

import ctypes

import numpy as np
import pytest
import torch

from helpers import ATTN_TOL, SCALE, host, max_abs, say
from oracle import kvdec_oracle as O

pytestmark = pytest.mark.gpu


def _inputs(B, H, KVH, L, seed, device):
    g = torch.Generator(device=device).manual_seed(seed)
    q = torch.randn(B, H, 128, generator=g, device=device, dtype=torch.float16)
    k = torch.randn(B, KVH, L, 128, generator=g, device=device, dtype=torch.float16)
    v = torch.randn(B, KVH, L, 128, generator=g, device=device, dtype=torch.float16)
    return q, k, v


def test_noalloc_first_call_under_graph_capture(device):
    """The entry point's first call in the process is made inside a HIP graph
    capture (no other test calls it, and this one runs first in this file):
    that call looks up the device array's address, and must neither fail
    the capture nor allocate.  The graph is replayed three times, with eager
    work between the replays and the output reset to NaN before each, and
    every replay is bit-identical to the workspace entry point."""
    import _kvdec as K
    torch.cuda.set_device(device)
    B, H, KVH, L = 2, 32, 2, 16384
    q, k, v = _inputs(B, H, KVH, L, 3, device)
    ws, nbytes = K.workspace(K.KIND_DENSE, B, H, KVH, L, 128, device)
    o_ws = torch.empty_like(q)

    def eager():
        rc = K.lib.kvdec_dense_decode(K.ptr(q), K.ptr(k), K.ptr(v), K.ptr(o_ws), K.F16, B, H, KVH, L, 128,
                                      SCALE, K.ptr(ws), nbytes, torch.cuda.current_stream(device).cuda_stream)
        assert rc == 0, K.strerror(rc)

    eager()
    torch.cuda.synchronize()
    o_na = torch.full_like(q, float("nan"))
    say(f"noalloc under capture B={B} H={H} KVH={KVH} L={L}")
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        rc = K.lib.kvdec_dense_decode_noalloc(K.ptr(q), K.ptr(k), K.ptr(v), K.ptr(o_na), K.F16, B, H, KVH, L,
                                              128, SCALE, torch.cuda.current_stream(device).cuda_stream)
    assert rc == 0, K.strerror(rc)
    for r in range(3):
        o_na.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(o_na, o_ws), f"replay {r}"
        eager()
        torch.cuda.synchronize()
    del g


def test_noalloc_equals_workspace_entry_point(device):
    import _kvdec as K
    torch.cuda.set_device(device)
    # first a problem with many splits (4 KV heads, 64 splits: 2 MiB of
    # partials), then a smaller one with fewer splits (its partials overwrite
    # the start of the same array)
    for (B, H, KVH, L, seed) in ((2, 32, 2, 16384, 1), (1, 8, 2, 3000, 2)):
        q, k, v = _inputs(B, H, KVH, L, seed, device)
        splits = K.lib.kvdec_num_splits(K.KIND_DENSE, B, KVH, L)
        assert splits > 1
        ws, nbytes = K.workspace(K.KIND_DENSE, B, H, KVH, L, 128, device)
        o_ws = torch.empty_like(q)
        o_na = torch.full_like(q, float("nan"))
        stream = torch.cuda.current_stream(device).cuda_stream
        say(f"noalloc dense B={B} H={H} KVH={KVH} L={L} splits={splits}")
        rc = K.lib.kvdec_dense_decode(K.ptr(q), K.ptr(k), K.ptr(v), K.ptr(o_ws), K.F16, B, H, KVH, L, 128,
                                      SCALE, K.ptr(ws), nbytes, stream)
        assert rc == 0, K.strerror(rc)
        rc = K.lib.kvdec_dense_decode_noalloc(K.ptr(q), K.ptr(k), K.ptr(v), K.ptr(o_na), K.F16, B, H, KVH, L,
                                              128, SCALE, stream)
        assert rc == 0, K.strerror(rc)
        torch.cuda.synchronize()
        assert torch.equal(o_ws, o_na)
        ref = O.dense_attention(host(q), host(k), host(v), SCALE)
        assert max_abs(host(o_na), ref) < ATTN_TOL


def test_noalloc_validates_before_launch(device):
    import _kvdec as K
    z = torch.zeros(1, 8, 128, dtype=torch.float16, device=device)
    assert K.lib.kvdec_dense_decode_noalloc(None, None, None, None, K.F16, 1, 8, 1, 16, 128, SCALE,
                                            None) == -1
    assert K.lib.kvdec_dense_decode_noalloc(K.ptr(z), K.ptr(z), K.ptr(z), K.ptr(z), K.F16, 1, 8, 1, 16, 64,
                                            SCALE, None) == -2
