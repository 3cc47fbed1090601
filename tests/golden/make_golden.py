"""Write the committed golden fixtures under tests/golden/.

    python tests/golden/make_golden.py

Inputs come from fixed numpy seeds (CPU, reproducible everywhere); expected
outputs come from the CPU oracle (oracle/kvdec_oracle.py), which the oracle
tests pin independently.  The fixtures freeze those vectors so that a later
change to either the oracle or the kernels is caught against known bytes, and
so that the GPU box needs no regeneration.  The reference repository ships no
golden vectors of its own and is not run to make these.
"""

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import kvdec_oracle as O  # noqa: E402

F16, F32 = np.float16, np.float32
SCALE = 128**-0.5


def quant_inputs():
    """K and V inputs [1, 2, 64, 128] fp32 holding the quantizer edge cases."""
    r = np.random.default_rng(1234)
    k = r.standard_normal((1, 2, 64, 128)).astype(F32)
    k[..., 5] *= 10                          # outlier channels
    k[..., 77] *= 10
    k[0, 0, :32, 1] = 0.7                    # constant group -> scale 1
    k[0, 0, :32, 2] = np.linspace(5, 6, 32)  # all-positive group, negative zero-point
    col = np.array([0.0, 3.0, 0.5, 1.5, 2.5, 1.0, 2.0] + [0.0] * 25, dtype=F32)
    k[0, 1, 32:, 3] = col                    # exact round-half-up ties
    k[0, 1, :32, 4] = np.arange(32)          # linear ramp
    v = r.standard_normal((1, 2, 64, 128)).astype(F32)
    v[0, 0, 0, :32] = -1.25                  # constant group
    v[0, 0, 1, :32] = col                    # ties along channels
    v[0, 1, 2, 32:64] = np.linspace(100, 101, 32)
    v[0, 1, 3] *= 10
    return k, v


def make_quant():
    k, v = quant_inputs()
    out = {"k": k, "v": v}
    for name, fn, x in (("k", O.quantize_k, k), ("v", O.quantize_v, v)):
        p, s, z = fn(x)
        out[name + "_packed"], out[name + "_scale"], out[name + "_zero"] = p, s, z
    return out


def make_dense():
    r = np.random.default_rng(99)
    B, H, KVH, L, D = 2, 16, 2, 77, 128
    q = r.standard_normal((B, H, D)).astype(F16)
    k = r.standard_normal((B, KVH, L, D)).astype(F16)
    v = r.standard_normal((B, KVH, L, D)).astype(F16)
    return {"q": q, "k": k, "v": v, "o": O.dense_attention(q, k, v, SCALE)}


def make_sparse():
    r = np.random.default_rng(7)
    B, H, KVH, D, S, W = 2, 16, 2, 128, 4, 64
    out = {}
    for tag, L in (("ramp", 30), ("steady", 500)):
        q = r.standard_normal((B, H, D)).astype(F32)
        kf = r.standard_normal((B, KVH, L, D)).astype(F32)
        vf = r.standard_normal((B, KVH, L, D)).astype(F32)
        kc, vc = O.build_compacted_cache(kf, vf, L, W, S)
        q16, kc16, vc16 = q.astype(F16), kc.astype(F16), vc.astype(F16)
        out[f"{tag}_q"], out[f"{tag}_k"], out[f"{tag}_v"] = q16, kc16, vc16
        out[f"{tag}_seq_len"] = np.array(L)
        out[f"{tag}_o"] = O.sparse_attention_compacted(q16, kc16, vc16, L, W, S, SCALE)
    out["window"] = np.array(W)
    out["sink"] = np.array(S)
    return out


def make_kivi():
    r = np.random.default_rng(2024)
    B, H, KVH, D, S, W, R = 1, 16, 2, 128, 4, 192, 128
    q = r.standard_normal((B, H, D)).astype(F16)
    kc = r.standard_normal((B, KVH, S + W, D)).astype(F16)
    kc[..., 9] *= 10
    vc = r.standard_normal((B, KVH, S + W, D)).astype(F16)
    cache = O.build_quantized_kv_cache(kc, vc, R, S)
    out = {"q": q, "k_compacted": kc, "v_compacted": vc, "window": np.array(W),
           "sink": np.array(S), "residual": np.array(R)}
    out.update({"cache_" + key: val for key, val in cache.items()})
    out["o_steady"] = O.quantized_attention_masked(q, cache, S + W + 1000, W, SCALE, S, R)
    out["o_ramp"] = O.quantized_attention_masked(q, cache, 150, W, SCALE, S, R)
    return out


FIXTURES = {
    "quant_golden.npz": make_quant,
    "dense_golden.npz": make_dense,
    "sparse_golden.npz": make_sparse,
    "kivi_golden.npz": make_kivi,
}


def main():
    for name, fn in FIXTURES.items():
        path = os.path.join(HERE, name)
        np.savez_compressed(path, **fn())
        print(f"{path}: {os.path.getsize(path)} bytes")


if __name__ == "__main__":
    main()
