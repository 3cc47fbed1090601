"""The one-launch KIVI cache builder on the GPU: every one of the 14 tensors
bit-exact vs the CPU oracle's build (quant_kernel.py:584-622 restated) and vs
the quantizers run on the reference's own slices, for fp16 / bf16 / fp32
caches, every sink size, other head dims, W < R and W = R, and at the
benchmark's full size."""

import numpy as np
import pytest
import torch

from helpers import dev, host, say
from oracle import kvdec_oracle as O

pytestmark = pytest.mark.gpu

R = 128


def _cache(B, KVH, n, D, seed, device, dtype, scale=1.0):
    gen = torch.Generator(device=device).manual_seed(seed)
    kc = (torch.randn(B, KVH, n, D, generator=gen, device=device) * scale).to(dtype)
    vc = (torch.randn(B, KVH, n, D, generator=gen, device=device) * scale).to(dtype)
    return kc, vc


def _np32(t):
    return host(t.float())   # fp16 / bf16 -> fp32 is exact


def _assert_cache_equal(got, want):
    assert list(got) == list(O.CACHE_KEYS)
    for key in O.CACHE_KEYS:
        g = got[key]
        w = want[key]
        g = _np32(g) if g.dtype in (torch.bfloat16,) else host(g)
        assert g.shape == tuple(w.shape), key
        np.testing.assert_array_equal(np.asarray(g, dtype=w.dtype), w, err_msg=key)


def _oracle(kc, vc, residual=R, sink=4):
    if kc.dtype == torch.bfloat16:
        return O.build_quantized_kv_cache(_np32(kc), _np32(vc), residual, sink)
    return O.build_quantized_kv_cache(host(kc), host(vc), residual, sink)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("W", [32, 100, 128, 160, 256, 1024])
def test_build_matches_oracle(dtype, W, device):
    from quant_kernel import build_quantized_kv_cache
    B, KVH, D, sink = 2, 3, 128, 4
    kc, vc = _cache(B, KVH, sink + W, D, 11 + W, device, dtype)
    say(f"build dtype={dtype} W={W}")
    got = build_quantized_kv_cache(kc, vc)
    torch.cuda.synchronize()
    assert got["k_residual"].dtype == dtype
    assert got["k_residual"].shape == (B, KVH, min(W, R), D)
    _assert_cache_equal(got, _oracle(kc, vc))


@pytest.mark.parametrize("sink", [1, 2, 4, 17, 31, 32])
@pytest.mark.parametrize("D", [32, 64, 128, 256])
def test_build_sink_sizes_and_head_dims(sink, D, device):
    from quant_kernel import build_quantized_kv_cache
    B, KVH, W = 2, 2, 192
    kc, vc = _cache(B, KVH, sink + W, D, 100 * sink + D, device, torch.float16)
    say(f"build sink={sink} D={D}")
    got = build_quantized_kv_cache(kc, vc, sink=sink)
    torch.cuda.synchronize()
    _assert_cache_equal(got, _oracle(kc, vc, sink=sink))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_build_fp16_residual(dtype, device):
    """residual_dtype=float16 converts the residual (RN, as torch's .half())
    and leaves the codes unchanged."""
    from quant_kernel import build_quantized_kv_cache
    kc, vc = _cache(2, 2, 4 + 256, 128, 5, device, dtype, scale=3.0)
    say(f"build fp16 residual from {dtype}")
    got = build_quantized_kv_cache(kc, vc, residual_dtype=torch.float16)
    same = build_quantized_kv_cache(kc, vc)
    torch.cuda.synchronize()
    assert got["k_residual"].dtype == torch.float16
    assert torch.equal(got["k_residual"], same["k_residual"].half())
    assert torch.equal(got["v_residual"], same["v_residual"].half())
    for key in O.CACHE_KEYS[2:]:
        assert torch.equal(got[key], same[key]), key


def test_build_equals_quantizers_on_slices(device):
    """The reference's own recipe (slices, torch.cat padding, four quantizer
    calls) on the GPU quantizers gives the same 14 tensors."""
    from quant_kernel import build_quantized_kv_cache, quantize_k_cache, quantize_v_cache
    B, KVH, D, S, W = 4, 8, 128, 4, 512
    kc, vc = _cache(B, KVH, S + W, D, 77, device, torch.float16)
    n = S + W
    want = {"k_residual": kc[:, :, n - R:], "v_residual": vc[:, :, n - R:]}
    for x, nm in ((kc, "k"), (vc, "v")):
        real = x[:, :, :S]
        pad = torch.cat([real, real[:, :, :1].expand(-1, -1, 32 - S, -1)], dim=2).float().contiguous()
        win = x[:, :, S:n - R].float().contiguous()
        fn = quantize_k_cache if nm == "k" else quantize_v_cache
        want[nm + "_sink_packed"], want[nm + "_sink_scale"], want[nm + "_sink_zero"] = fn(pad)
        want[nm + "_win_packed"], want[nm + "_win_scale"], want[nm + "_win_zero"] = fn(win)
    say("build vs quantizers on slices")
    got = build_quantized_kv_cache(kc, vc)
    torch.cuda.synchronize()
    for key in O.CACHE_KEYS:
        assert torch.equal(got[key], want[key]), key


def test_build_non_contiguous_and_scales(device):
    """A strided view of a larger cache, and values spanning the quantizers'
    slow-division ranges (scales below 2^-40 and above 2^100 per group)."""
    from quant_kernel import build_quantized_kv_cache
    B, KVH, D, S, W = 2, 4, 128, 4, 256
    kc, vc = _cache(B, 2 * KVH, S + W, D, 9, device, torch.float32)
    mag = torch.tensor([1e-14, 1e-3, 1.0, 1e3, 1e32], device=device)
    kc = kc * mag[torch.arange(D, device=device) % 5]
    vc = vc * mag[(torch.arange(S + W, device=device) % 5)][:, None]
    kc, vc = kc[:, ::2], vc[:, ::2]
    assert not kc.is_contiguous()
    say("build strided + scales")
    got = build_quantized_kv_cache(kc, vc)
    torch.cuda.synchronize()
    _assert_cache_equal(got, _oracle(kc.contiguous(), vc.contiguous()))


@pytest.mark.parametrize("W", [256, 4096])
def test_build_bench_size(W, device):
    """The benchmark's cache (B=32, KVH=8, D=128): bit-exact vs the GPU
    quantizers on the slices (the oracle would take minutes here)."""
    from quant_kernel import build_quantized_kv_cache, quantize_k_cache, quantize_v_cache
    B, KVH, D, S = 32, 8, 128, 4
    kc, vc = _cache(B, KVH, S + W, D, W, device, torch.float16)
    say(f"build bench size W={W}")
    got = build_quantized_kv_cache(kc, vc)
    n = S + W
    assert torch.equal(got["k_residual"], kc[:, :, n - R:])
    assert torch.equal(got["v_residual"], vc[:, :, n - R:])
    for x, nm, fn in ((kc, "k", quantize_k_cache), (vc, "v", quantize_v_cache)):
        p, s, z = fn(x[:, :, S:n - R].contiguous())
        assert torch.equal(got[nm + "_win_packed"], p)
        assert torch.equal(got[nm + "_win_scale"], s)
        assert torch.equal(got[nm + "_win_zero"], z)
        real = x[:, :, :S]
        p, s, z = fn(torch.cat([real, real[:, :, :1].expand(-1, -1, 32 - S, -1)], dim=2).contiguous())
        assert torch.equal(got[nm + "_sink_packed"], p)
        assert torch.equal(got[nm + "_sink_scale"], s)
        assert torch.equal(got[nm + "_sink_zero"], z)
    torch.cuda.synchronize()


def test_build_rejects(device):
    from quant_kernel import build_quantized_kv_cache
    kc, vc = _cache(1, 1, 4 + 144, 128, 1, device, torch.float16)
    with pytest.raises(AssertionError):
        build_quantized_kv_cache(kc, vc)          # window-old of 16 tokens
    kc, vc = _cache(1, 1, 4 + 160, 128, 1, device, torch.float16)
    with pytest.raises(TypeError):
        build_quantized_kv_cache(kc, vc.float())
    with pytest.raises(ValueError):
        build_quantized_kv_cache(kc, vc, sink=33)
    with pytest.raises(ValueError):
        build_quantized_kv_cache(kc, vc, sink=0)
    with pytest.raises(TypeError):
        build_quantized_kv_cache(kc, vc, residual_dtype=torch.float32)
