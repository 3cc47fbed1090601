"""The generic kernels on the GPU vs the CPU oracle: quantizers and the fused
decode at code widths and group sizes other than 2 / 32 (the reference's
BITS / GROUP_SIZE parameters, quant_kernel.py:44-214,436-581), and dense /
sparse decode with bf16 and fp32 q / k / v (dense_kernel.py:21-82 and
sparse_kernel.py:67-118 load whatever dtype they are given)."""

import numpy as np
import pytest
import torch

from helpers import ATTN_TOL, SCALE, assert_nearly_rounded, dev, host, max_abs, randn, say
from oracle import kvdec_oracle as O

pytestmark = pytest.mark.gpu

WIDTHS = [(1, 16), (3, 16), (4, 32), (4, 64), (8, 16), (2, 64), (2, 16), (5, 8)]
TORCH_DT = {"fp32": torch.float32, "fp16": torch.float16, "bf16": torch.bfloat16}


def _host_f32(t):
    return t.detach().float().cpu().numpy()


@pytest.mark.parametrize("bits,group", WIDTHS)
@pytest.mark.parametrize("dt", ["fp32", "fp16", "bf16"])
def test_quantize_any_width_bit_exact(bits, group, dt, device):
    from quant_kernel import quantize_k_cache, quantize_v_cache
    B, KVH, N, D = 2, 4, 4 * group, 128
    x = torch.from_numpy(randn((B, KVH, N, D), 70 + bits)).to(TORCH_DT[dt])
    x[..., 5] *= 10
    xh = x.float().numpy()
    xd = x.to(device)
    say(f"quantize any width bits={bits} group={group} {dt}")
    for fn, ofn in ((quantize_k_cache, O.quantize_k), (quantize_v_cache, O.quantize_v)):
        got = [host(t) for t in fn(xd, group_size=group, bits=bits)]
        torch.cuda.synchronize()
        want = ofn(xh, group, bits)
        for name, g, w in zip(("packed", "scale", "zero"), got, want):
            assert g.shape == w.shape, name
            np.testing.assert_array_equal(g, w, err_msg=f"{fn.__name__} {name}")


def _quantized_cache(kc, vc, S, R, group, bits, device):
    """The 14 tensors of a KIVI cache of this width: the oracle's builder
    (the sink padded to one group), uploaded."""
    c = O.build_quantized_kv_cache(kc, vc, residual_size=R, sink=S, group_size=group, bits=bits)
    return c, {k: dev(v, device) for k, v in c.items()}


def _attend(q, c, L, W, S, R, group, bits):
    from quant_kernel import sparse_decode_attention_quantized
    o = sparse_decode_attention_quantized(
        q, c["k_residual"], c["v_residual"],
        c["k_sink_packed"], c["k_sink_scale"], c["k_sink_zero"],
        c["v_sink_packed"], c["v_sink_scale"], c["v_sink_zero"],
        c["k_win_packed"], c["k_win_scale"], c["k_win_zero"],
        c["v_win_packed"], c["v_win_scale"], c["v_win_zero"],
        seq_len=L, window=W, sink=S, residual_size=R, group_size=group, bits=bits)
    torch.cuda.synchronize()
    return host(o) if o.dtype == torch.float16 else _host_f32(o)


@pytest.mark.parametrize("bits,group,W", [(4, 32, 256), (1, 16, 256), (8, 16, 512), (3, 64, 320),
                                          (2, 64, 256), (2, 16, 160), (4, 128, 384), (8, 32, 96)])
def test_quantized_attention_any_width(bits, group, W, device):
    """Steady state, ramp-up and per-sequence lengths against the oracle's
    dequantize-then-attend; outputs within half an fp16 ulp of it (the
    generic kernel's arithmetic is fp32)."""
    B, H, KVH, D, S, R = 3, 64, 8, 128, 4, 128
    kc = randn((B, KVH, S + W, D), 80 + bits).astype(np.float16)
    kc[..., 3] *= 10
    vc = randn((B, KVH, S + W, D), 81 + bits).astype(np.float16)
    q = randn((B, H, D), 82 + bits).astype(np.float16)
    say(f"kivi any width bits={bits} group={group} W={W}")
    hc, c = _quantized_cache(kc, vc, S, R, group, bits, device)
    qd = dev(q, device)
    for L in (163840, S + W - 37, 3):
        o = _attend(qd, c, L, W, S, R, group, bits)
        ref = O.quantized_attention_masked(q, hc, L, W, SCALE, sink=S, residual_size=R, group_size=group,
                                           bits=bits)
        assert max_abs(o, ref) < ATTN_TOL, L
        assert_nearly_rounded(o, ref)
    lens = np.array([163840, S + 40, 1], dtype=np.int32)
    o = _attend(qd, c, dev(lens, device), W, S, R, group, bits)
    ref = O.quantized_attention_varlen(q, hc, lens, W, SCALE, sink=S, residual_size=R, group_size=group,
                                       bits=bits)
    assert_nearly_rounded(o, ref)


def test_quantized_attention_any_width_from_gpu_quantizers(device):
    """The same cache made on the GPU (quantize_*_cache with the sink padded
    to one group by repeating token 0) gives the oracle's output."""
    from quant_kernel import quantize_k_cache, quantize_v_cache
    B, H, KVH, D, S, R, W, group, bits = 2, 64, 8, 128, 4, 128, 256, 16, 4
    kc = randn((B, KVH, S + W, D), 90).astype(np.float16)
    vc = randn((B, KVH, S + W, D), 91).astype(np.float16)
    q = randn((B, H, D), 92).astype(np.float16)
    kd, vd = dev(kc, device), dev(vc, device)
    pad = lambda x: torch.cat([x[:, :, :S], x[:, :, :1].expand(-1, -1, group - S, -1)], dim=2).float().contiguous()
    c = {"k_residual": kd[:, :, -R:].contiguous(), "v_residual": vd[:, :, -R:].contiguous()}
    say("kivi any width from the GPU quantizers")
    for name, fn, src in (("k_sink", quantize_k_cache, pad(kd)), ("v_sink", quantize_v_cache, pad(vd)),
                          ("k_win", quantize_k_cache, kd[:, :, S:-R].float().contiguous()),
                          ("v_win", quantize_v_cache, vd[:, :, S:-R].float().contiguous())):
        c[name + "_packed"], c[name + "_scale"], c[name + "_zero"] = fn(src, group_size=group, bits=bits)
    o = _attend(dev(q, device), c, 163840, W, S, R, group, bits)
    hc = O.build_quantized_kv_cache(kc, vc, residual_size=R, sink=S, group_size=group, bits=bits)
    for key in O.CACHE_KEYS:
        np.testing.assert_array_equal(host(c[key]), hc[key], err_msg=key)
    assert_nearly_rounded(o, O.quantized_attention(q, W - R, hc, SCALE, sink=S, group_size=group, bits=bits))


def _bf16_half_ulp(ref):
    a = np.abs(np.asarray(ref, dtype=np.float64))
    e = np.floor(np.log2(np.maximum(a, 2.0**-126)))
    return 2.0 ** (e - 8)


def _check_dtype_output(o, ref, dt):
    ref = np.asarray(ref, dtype=np.float64)
    if dt == "fp32":
        assert max_abs(o, ref) < 2e-6
    else:   # one rounding to bf16 of an fp32-accurate result
        assert (np.abs(o - ref) - _bf16_half_ulp(ref)).max() <= 2e-6


@pytest.mark.parametrize("dt", ["fp32", "bf16"])
@pytest.mark.parametrize("L", [1000, 70001])
def test_dense_other_dtypes(dt, L, device):
    from dense_kernel import dense_decode_attention
    B, H, KVH, D = 2, 64, 8, 128
    q = torch.from_numpy(randn((B, H, D), 100)).to(TORCH_DT[dt])
    k = torch.from_numpy(randn((B, KVH, L, D), 101)).to(TORCH_DT[dt])
    v = torch.from_numpy(randn((B, KVH, L, D), 102)).to(TORCH_DT[dt])
    say(f"dense {dt} L={L}")
    o = dense_decode_attention(q.to(device), k.to(device), v.to(device), seq_len=L)
    torch.cuda.synchronize()
    assert o.dtype == TORCH_DT[dt]
    ref = O.dense_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(), SCALE)
    _check_dtype_output(_host_f32(o), ref, dt)


@pytest.mark.parametrize("dt", ["fp32", "bf16"])
@pytest.mark.parametrize("layout", ["linear", "ring"])
def test_sparse_other_dtypes(dt, layout, device):
    from sparse_kernel import sparse_decode_attention
    B, H, KVH, D, S, W = 3, 64, 8, 128, 4, 256
    rng = np.random.default_rng(110)
    q = torch.from_numpy(randn((B, H, D), 111)).to(TORCH_DT[dt])
    kc = torch.from_numpy(randn((B, KVH, S + W, D), 112)).to(TORCH_DT[dt])
    vc = torch.from_numpy(randn((B, KVH, S + W, D), 113)).to(TORCH_DT[dt])
    qh, kh, vh = q.float().numpy(), kc.float().numpy(), vc.float().numpy()
    lay = 0 if layout == "linear" else 1
    say(f"sparse {dt} {layout}")
    for L in (163840, 150, 3):
        o = sparse_decode_attention(q.to(device), kc.to(device), vc.to(device), seq_len=L, window=W, sink=S,
                                    layout=layout)
        torch.cuda.synchronize()
        valid = O.slot_validity(L, W, S, lay)
        ref = O.masked_attention(qh, kh, vh, valid, SCALE)
        _check_dtype_output(_host_f32(o), ref, dt)
    lens = rng.integers(1, S + W + 50, B).astype(np.int32)
    o = sparse_decode_attention(q.to(device), kc.to(device), vc.to(device), seq_len=dev(lens, device),
                                window=W, sink=S, layout=layout)
    torch.cuda.synchronize()
    ref = O.sparse_attention_varlen(qh, kh, vh, lens, W, S, SCALE, layout=lay)
    _check_dtype_output(_host_f32(o), ref, dt)


def _check_typed_output(o, ref, dt):
    if dt == "fp16":
        assert_nearly_rounded(o, ref)
    elif dt == "fp32":
        # fp32 online softmax over logits up to ~10 in magnitude (the x10
        # channel): a few fp32 ulps per logit, 1e-5 on outputs of order 1
        assert max_abs(o, ref) < 1e-5
    else:
        _check_dtype_output(o, ref, dt)


@pytest.mark.parametrize("q_dt,res_dt", [("bf16", "bf16"), ("fp32", "fp32"), ("fp16", "bf16"),
                                         ("bf16", "fp16"), ("fp32", "fp16"), ("fp16", "fp32")])
def test_quantized_attention_other_dtypes(q_dt, res_dt, device):
    """q and the residual in bf16 / fp32 (quant_kernel.py:436-548 loads both
    in their own dtype and stores o in q's): the cache built on the GPU from
    a compacted cache of the residual's dtype equals the oracle's builder on
    the same values, and the decode over it (steady state, ramp-up,
    per-sequence lengths) is one rounding to q's dtype away from the oracle's
    fp64 attention."""
    from quant_kernel import build_quantized_kv_cache, sparse_decode_attention_quantized
    B, H, KVH, D, S, R, W = 3, 64, 8, 128, 4, 128, 256
    q = torch.from_numpy(randn((B, H, D), 120)).to(TORCH_DT[q_dt])
    kc = torch.from_numpy(randn((B, KVH, S + W, D), 121))
    kc[..., 3] *= 10
    kc = kc.to(TORCH_DT[res_dt])
    vc = torch.from_numpy(randn((B, KVH, S + W, D), 122)).to(TORCH_DT[res_dt])
    qh = q.float().numpy()
    hc = O.build_quantized_kv_cache(kc.float().numpy(), vc.float().numpy(), residual_size=R, sink=S)
    say(f"kivi q={q_dt} residual={res_dt}")
    c = build_quantized_kv_cache(kc.to(device), vc.to(device), residual_size=R, sink=S)
    assert c["k_residual"].dtype == TORCH_DT[res_dt]
    for key in O.CACHE_KEYS:
        np.testing.assert_array_equal(_host_f32(c[key]), np.asarray(hc[key], dtype=np.float32), err_msg=key)
    qd = q.to(device)

    def attend(L):
        o = sparse_decode_attention_quantized(
            qd, c["k_residual"], c["v_residual"],
            c["k_sink_packed"], c["k_sink_scale"], c["k_sink_zero"],
            c["v_sink_packed"], c["v_sink_scale"], c["v_sink_zero"],
            c["k_win_packed"], c["k_win_scale"], c["k_win_zero"],
            c["v_win_packed"], c["v_win_scale"], c["v_win_zero"],
            seq_len=L, window=W, sink=S, residual_size=R)
        torch.cuda.synchronize()
        assert o.dtype == TORCH_DT[q_dt]
        return _host_f32(o)

    for L in (163840, S + W - 37, 3):
        ref = O.quantized_attention_masked(qh, hc, L, W, SCALE, sink=S, residual_size=R)
        _check_typed_output(attend(L), ref, q_dt)
    lens = np.array([163840, S + 40, 1], dtype=np.int32)
    ref = O.quantized_attention_varlen(qh, hc, lens, W, SCALE, sink=S, residual_size=R)
    _check_typed_output(attend(dev(lens, device)), ref, q_dt)


@pytest.mark.parametrize("bits,group", [(4, 32), (3, 16)])
def test_quantized_attention_other_dtypes_any_width(bits, group, device):
    """bf16 q with an fp32 residual at code widths other than 2 bits."""
    B, H, KVH, D, S, R, W = 2, 64, 8, 128, 4, 128, 320
    kc = randn((B, KVH, S + W, D), 130 + bits).astype(np.float16)
    vc = randn((B, KVH, S + W, D), 131 + bits).astype(np.float16)
    q = torch.from_numpy(randn((B, H, D), 132 + bits)).to(torch.bfloat16)
    say(f"kivi bf16 q, fp32 residual, bits={bits} group={group}")
    hc, c = _quantized_cache(kc, vc, S, R, group, bits, device)
    c["k_residual"], c["v_residual"] = c["k_residual"].float(), c["v_residual"].float()
    qh = q.float().numpy()
    for L in (163840, S + W - 37):
        o = _attend(q.to(device), c, L, W, S, R, group, bits)
        ref = O.quantized_attention_masked(qh, hc, L, W, SCALE, sink=S, residual_size=R, group_size=group,
                                           bits=bits)
        _check_dtype_output(o, ref, "bf16")


def test_other_dtypes_rejected_where_fp16_only(device):
    from dense_kernel import dense_decode_attention
    q = torch.zeros(2, 64, 128, dtype=torch.float32, device=device)
    k = torch.zeros(2, 8, 64, 128, dtype=torch.float32, device=device)
    with pytest.raises(ValueError):   # per-sequence lengths take fp16
        dense_decode_attention(q, k, k, seq_len=torch.full((2,), 10, dtype=torch.int32, device=device))
    with pytest.raises(ValueError):   # mixed dtypes
        dense_decode_attention(q, k.half(), k.half(), seq_len=64)
