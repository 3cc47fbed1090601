"""The bandwidth probe (kvdec_read_probe): every workgroup's XOR of its
contiguous share, against numpy, for ragged sizes and grid shapes."""
import numpy as np
import pytest
import torch

import _kvdec as K
from helpers import say

pytestmark = pytest.mark.gpu


def _expected(words, blocks):
    n16 = len(words) // 4
    per = -(-n16 // blocks) if n16 else 0
    out = np.zeros(blocks, dtype=np.uint32)
    w4 = words.reshape(n16, 4)
    for b in range(blocks):
        lo, hi = min(b * per, n16), min((b + 1) * per, n16)
        if hi > lo:
            out[b] = np.bitwise_xor.reduce(w4[lo:hi].reshape(-1))
    return out


@pytest.mark.parametrize("n16,blocks", [(0, 256), (1, 256), (4095, 7), (65536 + 13, 256), (262144, 1024)])
def test_read_probe_xor(n16, blocks):
    say(f"read probe n16={n16} blocks={blocks}")
    rng = np.random.default_rng(n16 + blocks)
    words = rng.integers(0, 2**32, size=4 * max(n16, 1), dtype=np.uint32)[: 4 * n16]
    gpu = torch.device("cuda:0")
    src = (torch.from_numpy(words.view(np.int32).copy()).to(gpu) if n16
           else torch.empty(4, dtype=torch.int32, device=gpu))
    sink = torch.full((blocks,), -1, dtype=torch.int32, device=gpu)
    K.check(K.lib.kvdec_read_probe(K.ptr(src), 16 * n16, K.ptr(sink), blocks, K.stream_of(sink)), "read_probe")
    got = sink.cpu().numpy().view(np.uint32)
    np.testing.assert_array_equal(got, _expected(words, blocks))


@pytest.mark.parametrize("threads", [256, 512, 1024])
@pytest.mark.parametrize("mode", range(8))
@pytest.mark.parametrize("n16,blocks", [(0, 256), (4095, 7), (65536 + 13, 256), (262144, 2048)])
def test_read_probe_sweep_xor(n16, blocks, threads, mode):
    """Every block size and load form of the sweep probe reads exactly its
    share (buffer forms: past the share, zeros without an access)."""
    say(f"read probe sweep n16={n16} blocks={blocks} threads={threads} mode={mode}")
    rng = np.random.default_rng(n16 + blocks + threads + mode)
    words = rng.integers(0, 2**32, size=4 * max(n16, 1), dtype=np.uint32)[: 4 * n16]
    gpu = torch.device("cuda:0")
    src = (torch.from_numpy(words.view(np.int32).copy()).to(gpu) if n16
           else torch.empty(4, dtype=torch.int32, device=gpu))
    sink = torch.full((blocks,), -1, dtype=torch.int32, device=gpu)
    K.check(K.lib.kvdec_read_probe_sweep(K.ptr(src), 16 * n16, K.ptr(sink), blocks, threads, mode, 4096,
                                         K.stream_of(sink)), "read_probe_sweep")
    got = sink.cpu().numpy().view(np.uint32)
    np.testing.assert_array_equal(got, _expected(words, blocks))
