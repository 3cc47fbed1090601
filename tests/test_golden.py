"""The oracle reproduces the committed golden fixtures bit for bit (CPU).

The fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py)
freeze seeded inputs and the oracle's outputs; the GPU tests compare the HIP
kernels against the same files.
"""

import numpy as np

from conftest import load_golden
from oracle import kvdec_oracle as O

SCALE = 128**-0.5


def test_quant_golden():
    g = load_golden("quant_golden.npz")
    for name, fn in (("k", O.quantize_k), ("v", O.quantize_v)):
        p, s, z = fn(g[name])
        np.testing.assert_array_equal(p, g[name + "_packed"])
        np.testing.assert_array_equal(s, g[name + "_scale"])
        np.testing.assert_array_equal(z, g[name + "_zero"])
    # the edge cases are really in there
    assert float(g["k_scale"][0, 0, 0, 1]) == 1.0
    assert float(g["k_zero"][0, 0, 0, 2]) == -15.0


def test_dense_golden():
    g = load_golden("dense_golden.npz")
    np.testing.assert_array_equal(O.dense_attention(g["q"], g["k"], g["v"], SCALE), g["o"])


def test_sparse_golden():
    g = load_golden("sparse_golden.npz")
    W, S = int(g["window"]), int(g["sink"])
    for tag in ("ramp", "steady"):
        o = O.sparse_attention_compacted(g[f"{tag}_q"], g[f"{tag}_k"], g[f"{tag}_v"],
                                         int(g[f"{tag}_seq_len"]), W, S, SCALE)
        np.testing.assert_array_equal(o, g[f"{tag}_o"])


def test_kivi_golden():
    g = load_golden("kivi_golden.npz")
    W, S, R = int(g["window"]), int(g["sink"]), int(g["residual"])
    cache = O.build_quantized_kv_cache(g["k_compacted"], g["v_compacted"], R, S)
    for key in O.CACHE_KEYS:
        np.testing.assert_array_equal(cache[key], g["cache_" + key])
    o = O.quantized_attention_masked(g["q"], cache, S + W + 1000, W, SCALE, S, R)
    np.testing.assert_array_equal(o, g["o_steady"])
    o = O.quantized_attention_masked(g["q"], cache, 150, W, SCALE, S, R)
    np.testing.assert_array_equal(o, g["o_ramp"])
