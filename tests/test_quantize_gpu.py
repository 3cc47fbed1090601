"""KIVI quantizers on the GPU: codes, scales and zeros bit-exact vs the CPU
oracle (the reference's test_quantize_correctness.py only bounds the round
trip; this pins every byte)."""

import numpy as np
import pytest
import torch

from conftest import load_golden
from helpers import dev, host, randn, say
from oracle import kvdec_oracle as O

pytestmark = pytest.mark.gpu


def _quant(fn_name, x, device, torch_dtype=torch.float32):
    import quant_kernel
    t = dev(x, device).to(torch_dtype)
    out = getattr(quant_kernel, fn_name)(t)
    torch.cuda.synchronize()
    return tuple(host(a) for a in out)


def _assert_same(got, want):
    for g, w, name in zip(got, want, ("packed", "scale", "zero")):
        assert g.shape == w.shape, name
        assert g.dtype == w.dtype, name
        np.testing.assert_array_equal(g, w, err_msg=name)


def test_quant_golden(device):
    g = load_golden("quant_golden.npz")
    for name, fn in (("k", "quantize_k_cache"), ("v", "quantize_v_cache")):
        say(f"quant golden {name}")
        _assert_same(_quant(fn, g[name], device),
                     (g[name + "_packed"], g[name + "_scale"], g[name + "_zero"]))


@pytest.mark.parametrize("N", [32, 256, 8192])
def test_quantize_k_reference_lengths(N, device):
    x = randn((1, 1, N, 128), N)
    say(f"quantize_k N={N}")
    _assert_same(_quant("quantize_k_cache", x, device), O.quantize_k(x))


@pytest.mark.parametrize("N", [32, 256, 8192])
def test_quantize_v_reference_lengths(N, device):
    x = randn((1, 1, N, 128), N + 1)
    say(f"quantize_v N={N}")
    _assert_same(_quant("quantize_v_cache", x, device), O.quantize_v(x))


@pytest.mark.parametrize("tdt", [torch.float16, torch.bfloat16, torch.float32])
def test_quantize_input_dtypes_with_outliers(tdt, device):
    x = randn((2, 8, 512, 128), 3)
    x[..., [1, 40, 77, 120]] *= 10
    xt = torch.from_numpy(x).to(tdt)
    xr = xt.float().numpy()                      # the values the kernel actually sees
    say(f"quantize dtype={tdt}")
    _assert_same(_quant("quantize_k_cache", xr, device, tdt), O.quantize_k(xr))
    _assert_same(_quant("quantize_v_cache", xr, device, tdt), O.quantize_v(xr))


def test_quantize_coarse_grid_ties(device):
    """fp16 values on a coarse grid hit x/s + 0.5 == integer often: the
    round-half-up ties must match exactly."""
    r = np.random.default_rng(5)
    x = (r.integers(-6, 7, size=(1, 4, 1024, 128)) * 0.5).astype(np.float32)
    say("quantize ties")
    _assert_same(_quant("quantize_k_cache", x, device), O.quantize_k(x))
    _assert_same(_quant("quantize_v_cache", x, device), O.quantize_v(x))


def test_quantize_scale_magnitudes(device):
    """Groups whose scales span 1e-30 .. 1e30 (fp32 input): the kernels'
    three-FMA quotient covers scales in [2^-40, 2^100] and an fp64 path the
    rest; both must give the IEEE float32 codes.  Magnitudes vary per 32x32
    block, so K and V groups see both uniform and mixed magnitudes."""
    r = np.random.default_rng(11)
    B, KVH, N, D = 1, 2, 512, 128
    e = r.uniform(-30, 30, size=(B, KVH, N // 32, 1, D // 32, 1))
    mag = np.broadcast_to(10.0 ** e, (B, KVH, N // 32, 32, D // 32, 32)).reshape(B, KVH, N, D)
    x = (r.standard_normal((B, KVH, N, D)) * mag).astype(np.float32)
    x[0, 0, :32, :5] = 3.0                          # constant groups (scale 0 -> 1)
    x[0, 1, 64:96] += np.float32(1e4)               # large offsets: zero-points far from 0
    say("quantize scale magnitudes")
    with np.errstate(over="ignore"):                # scales above 65504 store as fp16 inf
        want_k, want_v = O.quantize_k(x), O.quantize_v(x)
    _assert_same(_quant("quantize_k_cache", x, device), want_k)
    _assert_same(_quant("quantize_v_cache", x, device), want_v)


@pytest.mark.parametrize("D", [64, 96, 192])
@pytest.mark.parametrize("tdt", [torch.float16, torch.float32])
def test_quantize_other_head_dims(D, tdt, device):
    """Head dims other than 128: K runs 128-channel slices (the second slice
    of D=192 is half empty), V any multiple of 32."""
    x = randn((2, 3, 96, D), D)
    xr = torch.from_numpy(x).to(tdt).float().numpy()
    say(f"quantize D={D} dtype={tdt}")
    _assert_same(_quant("quantize_k_cache", xr, device, tdt), O.quantize_k(xr))
    _assert_same(_quant("quantize_v_cache", xr, device, tdt), O.quantize_v(xr))


def test_quantize_config4_shape(device):
    """Config 4: [32, 8, 163840, 128] fp16, 4 outlier channels x10; the
    per-(b, kv) quantization is independent, so three heads spread over the
    tensor (largest offsets included) are checked bit-exact."""
    B, KVH, N, D = 32, 8, 163840, 128
    gen = torch.Generator(device=device).manual_seed(0)
    say("quantize config4 (generate)")
    k = torch.randn(B, KVH, N, D, generator=gen, device=device, dtype=torch.float16)
    outl = torch.randperm(D, generator=torch.Generator().manual_seed(0))[:4].tolist()
    k[..., outl] *= 10
    import quant_kernel
    say("quantize config4 K (run)")
    pk, sk, zk = quant_kernel.quantize_k_cache(k)
    say("quantize config4 V (run)")
    pv, sv, zv = quant_kernel.quantize_v_cache(k)
    torch.cuda.synchronize()
    for b, h in ((0, 0), (17, 3), (31, 7)):
        x = host(k[b:b + 1, h:h + 1])
        _assert_same((host(pk[b:b + 1, h:h + 1]), host(sk[b:b + 1, h:h + 1]), host(zk[b:b + 1, h:h + 1])),
                     O.quantize_k(x))
        _assert_same((host(pv[b:b + 1, h:h + 1]), host(sv[b:b + 1, h:h + 1]), host(zv[b:b + 1, h:h + 1])),
                     O.quantize_v(x))
    del k


def test_sink_padding_boundary(device):
    """The reference's sink-padding case (seed 2 analogue): 4 real tokens
    padded to 32 by repeating token 0, then the reference round-trip bound on
    the real tokens."""
    sink = randn((1, 1, 4, 128), 2)
    padded = np.concatenate([sink, np.repeat(sink[:, :, :1], 28, axis=2)], axis=2)
    say("sink padding")
    got = _quant("quantize_k_cache", padded, device)
    _assert_same(got, O.quantize_k(padded))
    rec = O.unpack_dequant(*got, 32, pack_axis=2)[:, :, :4]
    tol = (sink.max(axis=2) - sink.min(axis=2)).max() / 2 + 1e-3
    assert np.abs(rec - sink).max() < tol
