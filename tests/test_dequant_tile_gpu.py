"""Isolated tile dequantizers on the GPU vs the oracle (restates the
reference's test_dequantize_tile_isolated.py, plus the clamped cases)."""

import numpy as np
import pytest
import torch

from helpers import dev, host, randn, say
from oracle import kvdec_oracle as O

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("tok_start", [0, 128, -4, 5, 200, 300])
def test_dequantize_k_tile(tok_start, device):
    import quant_kernel
    k = randn((2, 3, 256, 128), 4)
    pk, sk, zk = O.quantize_k(k)
    say(f"dequant k tile start={tok_start}")
    out = quant_kernel.dequantize_k_tile(dev(pk, device), dev(sk, device), dev(zk, device), tok_start)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host(out), O.dequant_k_tile(pk, sk, zk, tok_start, 64, 8))
    if tok_start in (0, 128):   # the reference's own comparison: the unpacked cache
        ref = O.unpack_dequant(pk, sk, zk, 256, pack_axis=2)[:, :, tok_start:tok_start + 128]
        assert np.abs(host(out) - ref).max() < 1e-2


@pytest.mark.parametrize("tok_start", [0, 100, -7, 250])
def test_dequantize_v_tile(tok_start, device):
    import quant_kernel
    v = randn((2, 3, 256, 128), 5)
    pv, sv, zv = O.quantize_v(v)
    say(f"dequant v tile start={tok_start}")
    out = quant_kernel.dequantize_v_tile(dev(pv, device), dev(sv, device), dev(zv, device), tok_start)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host(out), O.dequant_v_tile(pv, sv, zv, tok_start, 256))
