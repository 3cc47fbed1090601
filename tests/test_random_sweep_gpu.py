"""Seeded random shapes through every decode entry point, against the CPU
oracle: the fused KIVI decode (random batch, query/KV head grouping, residual
size, sink of 1..32 tokens, windows below and above the residual, scalar and
per-sequence lengths in ramp-up and steady state), the sparse decode (linear
and ring layouts), the dense decode, the paged decode (NHD / HND pages of
16..128 tokens, shuffled block tables, lengths 0..3000) and the generic
kernels (1..8-bit codes with every whole-byte group size, bf16 and fp32
dense inputs).  The reference's own tests fix a handful of shapes
(test_quantized_attention_correctness.py, test_sparse_attention_correctness.py);
this covers the combinations between them.

Outputs must be within the attention gate of the oracle's.  At 7 and 8 bits
a group whose range is tiny against its minimum has a zero point beyond the
fp16 range (the cache format stores it in fp16, as the reference's does):
the dequantized value is then NaN, and the decode must give NaN in exactly
the oracle's NaN elements."""

import numpy as np
import pytest
import torch

from helpers import ATTN_TOL, SCALE, dev, host, say
from oracle import kvdec_oracle as O

pytestmark = pytest.mark.gpu

GROUPINGS = [(16, 2), (8, 8), (32, 4), (64, 8), (24, 2), (32, 2), (12, 1)]   # (H, KVH)


def _rn(rng, shape):
    return rng.standard_normal(shape).astype(np.float16)


def _length(rng, n, extra):
    return int(rng.integers(1, n + 1)) if rng.random() < 0.5 else n + int(rng.integers(0, extra))


def _kivi(rng, q, B, KVH, device):
    from quant_kernel import build_quantized_kv_cache, sparse_decode_attention_quantized
    D = q.shape[2]
    R = int(rng.choice([128, 128, 64, 32]))
    S = int(rng.integers(1, 33))
    W = int(rng.integers(1, R)) if rng.random() < 0.25 else R + 32 * int(rng.integers(0, 40))
    n = S + W
    kc = _rn(rng, (B, KVH, n, D))
    kc[..., rng.integers(D, size=3)] *= 10
    vc = _rn(rng, (B, KVH, n, D))
    cache = build_quantized_kv_cache(dev(kc, device), dev(vc, device), residual_size=R, sink=S)
    hc = {k: host(v) for k, v in cache.items()}
    args = [cache[k] for k in O.CACHE_KEYS]
    if rng.random() < 0.3:
        lens = rng.integers(1, n + 3000, B).astype(np.int32)
        desc = f"kivi B={B} KVH={KVH} R={R} S={S} W={W} lens={lens.tolist()}"
        say(desc)
        o = sparse_decode_attention_quantized(dev(q, device), *args, seq_len=dev(lens, device), window=W,
                                              sink=S, residual_size=R)
        return desc, o, O.quantized_attention_varlen(q, hc, lens, W, SCALE, sink=S, residual_size=R)
    L = _length(rng, n, 5000)
    desc = f"kivi B={B} KVH={KVH} R={R} S={S} W={W} L={L}"
    say(desc)
    o = sparse_decode_attention_quantized(dev(q, device), *args, seq_len=L, window=W, sink=S, residual_size=R)
    return desc, o, O.quantized_attention_masked(q, hc, L, W, SCALE, sink=S, residual_size=R)


def _generic(rng, q, B, KVH, device):
    from quant_kernel import sparse_decode_attention_quantized
    D = q.shape[2]
    bits = int(rng.integers(1, 9))
    group = int(rng.choice([g for g in (8, 16, 32, 64, 128) if g % (8 // bits) == 0]))
    R = 128
    S = int(rng.integers(1, min(group, 32) + 1))
    W = R + group * int(rng.integers(0, 8)) if rng.random() < 0.8 else int(rng.integers(1, R))
    n = S + W
    hc = O.build_quantized_kv_cache(_rn(rng, (B, KVH, n, D)), _rn(rng, (B, KVH, n, D)), residual_size=R,
                                    sink=S, group_size=group, bits=bits)
    c = {k: dev(v, device) for k, v in hc.items()}
    L = _length(rng, n, 3000)
    desc = f"generic bits={bits} group={group} B={B} KVH={KVH} S={S} W={W} L={L}"
    say(desc)
    o = sparse_decode_attention_quantized(dev(q, device), *[c[k] for k in O.CACHE_KEYS], seq_len=L, window=W,
                                          sink=S, residual_size=R, group_size=group, bits=bits)
    return desc, o, O.quantized_attention_masked(q, hc, L, W, SCALE, sink=S, residual_size=R, group_size=group,
                                                 bits=bits)


def _sparse(rng, q, B, KVH, device):
    from sparse_kernel import sparse_decode_attention
    D = q.shape[2]
    S, W = int(rng.integers(1, 40)), int(rng.integers(1, 1200))
    n = S + W
    kc, vc = _rn(rng, (B, KVH, n, D)), _rn(rng, (B, KVH, n, D))
    layout = str(rng.choice(["linear", "ring"]))
    L = _length(rng, n, 5000)
    desc = f"sparse {layout} B={B} KVH={KVH} S={S} W={W} L={L}"
    say(desc)
    o = sparse_decode_attention(dev(q, device), dev(kc, device), dev(vc, device), seq_len=L, window=W, sink=S,
                                layout=layout)
    return desc, o, O.masked_attention(q, kc, vc, O.slot_validity(L, W, S, 0 if layout == "linear" else 1), SCALE)


def _dense(rng, q, B, KVH, device, dtype=torch.float16):
    from dense_kernel import dense_decode_attention
    D = q.shape[2]
    L = int(rng.integers(1, 6000))
    qt = torch.from_numpy(q).to(dtype)
    k = torch.from_numpy(_rn(rng, (B, KVH, L, D))).to(dtype)
    v = torch.from_numpy(_rn(rng, (B, KVH, L, D))).to(dtype)
    desc = f"dense {dtype} B={B} KVH={KVH} L={L}"
    say(desc)
    o = dense_decode_attention(qt.to(device), k.to(device), v.to(device), seq_len=L)
    return desc, o, O.dense_attention(qt.float().numpy(), k.float().numpy(), v.float().numpy(), SCALE)


def _paged(rng, q, B, KVH, device):
    from paged_kernel import paged_decode_attention
    D = q.shape[2]
    P = int(rng.choice([16, 32, 64, 128]))
    lens = rng.integers(0, 3000, B).astype(np.int32)
    nb = int(max(1, (int(lens.max()) + P - 1) // P))
    pages = B * nb + 3
    layout = str(rng.choice(["NHD", "HND"]))
    shape = (pages, P, KVH, D) if layout == "NHD" else (pages, KVH, P, D)
    kp, vp = _rn(rng, shape), _rn(rng, shape)
    table = rng.permutation(pages)[:B * nb].reshape(B, nb).astype(np.int32)
    desc = f"paged {layout} P={P} B={B} KVH={KVH} lens={lens.tolist()}"
    say(desc)
    o = paged_decode_attention(dev(q, device), dev(kp, device), dev(vp, device), dev(table, device),
                               dev(lens, device), kv_layout=layout)
    return desc, o, O.paged_attention(q, kp, vp, table, lens, SCALE, layout)


KINDS = {"kivi": _kivi, "generic": _generic, "sparse": _sparse, "dense": _dense, "paged": _paged,
         "dense_bf16": lambda *a: _dense(*a, dtype=torch.bfloat16),
         "dense_f32": lambda *a: _dense(*a, dtype=torch.float32)}
TOL = {"dense_bf16": 4e-3, "dense_f32": 2e-6}


@pytest.mark.parametrize("seed", [1, 2, 3])
def test_random_shapes_against_oracle(seed, device):
    rng = np.random.default_rng(1000 + seed)
    kinds = ["kivi"] * 4 + ["generic", "sparse", "dense", "paged", "dense_bf16", "dense_f32"]
    for case in range(80):
        kind = kinds[int(rng.integers(len(kinds)))]
        H, KVH = GROUPINGS[int(rng.integers(len(GROUPINGS)))]
        B = int(rng.integers(1, 4))
        q = _rn(rng, (B, H, 128))
        desc, o, ref = KINDS[kind](rng, q, B, KVH, device)
        torch.cuda.synchronize()
        o = o.float().cpu().numpy().astype(np.float64)
        ref = np.asarray(ref, dtype=np.float64)
        nan = np.isnan(ref)
        assert np.array_equal(np.isnan(o), nan), f"case {case}: {desc}: NaN elements differ from the oracle's"
        err = float(np.abs(o[~nan] - ref[~nan]).max()) if (~nan).any() else 0.0
        assert err < TOL.get(kind, ATTN_TOL), f"case {case}: {desc}: max error {err:.3e}"


def _values(rng, shape, dtype):
    """Inputs of a random character: plain normals, a huge or tiny overall
    scale, constant stretches (zero-range groups) and single outliers."""
    x = rng.standard_normal(shape).astype(np.float32)
    mode = int(rng.integers(5))
    if mode == 1:
        x *= np.float32(2.0 ** int(rng.integers(-20, 12)))
    elif mode == 2:
        x[..., ::3] = np.float32(rng.standard_normal())
    elif mode == 3:
        x.reshape(-1)[rng.integers(x.size, size=8)] *= 1000
    elif mode == 4:
        x = np.round(x * 4) / 4                      # many exact ties with the code grid
    t = torch.from_numpy(x).to(dtype)
    if dtype == torch.float16:
        t = torch.nan_to_num(t, posinf=65504.0, neginf=-65504.0)
    return t


@pytest.mark.parametrize("seed", [1, 2])
def test_random_quantizer_inputs_bit_exact(seed, device):
    """quantize_k_cache / quantize_v_cache on random shapes, input dtypes and
    value patterns (wide and tiny ranges, constant groups, outliers, values
    on the code grid): codes, scales and zeros bit-identical to the oracle's
    (IEEE float32 with correctly rounded division)."""
    from quant_kernel import quantize_k_cache, quantize_v_cache
    rng = np.random.default_rng(2000 + seed)
    for case in range(40):
        dtype = [torch.float16, torch.bfloat16, torch.float32][int(rng.integers(3))]
        B, KVH = int(rng.integers(1, 4)), int(rng.integers(1, 9))
        N = 32 * int(rng.integers(1, 12))
        x = _values(rng, (B, KVH, N, 128), dtype)
        xh = x.float().numpy()
        for fn, ofn in ((quantize_k_cache, O.quantize_k), (quantize_v_cache, O.quantize_v)):
            say(f"random quantizer case {case}: {fn.__name__} {dtype} B={B} KVH={KVH} N={N}")
            got = [host(t) for t in fn(x.to(device))]
            torch.cuda.synchronize()
            for name, g, w in zip(("packed", "scale", "zero"), got, ofn(xh)):
                np.testing.assert_array_equal(g, w, err_msg=f"case {case} {fn.__name__} {name}")


@pytest.mark.parametrize("seed", [1, 2])
def test_random_stream_sequences(seed, device):
    """The decode-time cache driven by a random mix of append, reserve (row
    written afterwards) and step_attend calls from a random prefill, attended
    at random points: the output matches the oracle's stream_cache state at
    that length (one ring state for all sequences, and one per sequence)."""
    from kivi_stream import KiviStreamBatch, KiviStreamCache
    rng = np.random.default_rng(3000 + seed)
    for case in range(6):
        H, KVH = GROUPINGS[int(rng.integers(len(GROUPINGS)))]
        B, D = int(rng.integers(1, 4)), 128
        W = int(rng.choice([128, 160, 224, 256, 288, 352, 384, 512]))
        L0 = 4 + W + int(rng.integers(0, 100))
        steps = int(rng.integers(20, 90))
        kf = _rn(rng, (B, KVH, L0 + steps, D))
        vf = _rn(rng, (B, KVH, L0 + steps, D))
        q = _rn(rng, (B, H, D))
        per_seq = bool(rng.random() < 0.5)
        cls = KiviStreamBatch if per_seq else KiviStreamCache
        kd, vd, qd = dev(kf, device), dev(vf, device), dev(q, device)
        cache = cls.from_prefill(kd[:, :, :L0], vd[:, :, :L0], W)
        L = L0
        for step in range(steps):
            op = int(rng.integers(3))
            if op == 0 or (op == 2 and not per_seq):
                cache.append(kd[:, :, L], vd[:, :, L])
                o = None
            elif op == 1:
                if per_seq:   # the ring row each sequence takes
                    rows = cache.reserve().cpu().tolist()
                    for b, r in enumerate(rows):
                        cache.t["k_ring"][b, :, r] = kd[b, :, L]
                        cache.t["v_ring"][b, :, r] = vd[b, :, L]
                else:
                    kv, vv = cache.reserve()
                    kv.copy_(kd[:, :, L])
                    vv.copy_(vd[:, :, L])
                o = None
            else:
                o = cache.step_attend(qd, kd[:, :, L], vd[:, :, L])
            L += 1
            if o is None and rng.random() < 0.2:
                o = cache.attend(qd)
            if o is not None:
                say(f"random stream case {case}: per_seq={per_seq} B={B} H={H} KVH={KVH} W={W} L0={L0} L={L}")
                torch.cuda.synchronize()
                sc, wlen = O.stream_cache(kf, vf, L0, L, W)
                ref = O.quantized_attention(q, wlen, sc, SCALE)
                err = float(np.abs(host(o).astype(np.float64) - ref).max())
                assert err < ATTN_TOL, f"case {case} L={L}: max error {err:.3e}"
