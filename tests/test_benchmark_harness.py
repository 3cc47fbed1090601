"""The sweep harness (numerics-and-sparse-attn_amd/benchmark.py) without a
GPU: its byte models against the figures the reference's benchmark.py
produces, and its CSV writer's column order."""

import csv
import os

import benchmark as BM

# benchmark.py:30-31 (B_FIXED_FP16, C_FP16) and the bytes columns of the
# reference's results/benchmark_results_quantized.csv (W=256: 21,757,952;
# W=1024: 40,632,320; W=4096: 116,129,792; W=128: 18,612,224).
REF_QUANT_BYTES = {128: 18_612_224, 256: 21_757_952, 1024: 40_632_320, 4096: 116_129_792}
# real sink tokens only (the minimal bytes the fused kernel reads)
MIN_QUANT_BYTES = {256: 21_184_512, 1024: 40_058_880, 4096: 115_556_352}


def test_byte_models():
    assert BM.B_FIXED_FP16 + BM.C_FP16 * (256 + 4) == 35_127_296
    assert BM.B_FIXED_FP16 + BM.C_FP16 * 163_840 == 21_475_885_056
    for W, b in REF_QUANT_BYTES.items():
        assert BM.quantized_bytes(W)[0] == b, W
    for W, b in MIN_QUANT_BYTES.items():
        assert BM.quantized_bytes(W)[1] == b, W


def _point(L=163840, W=256):
    p = BM.Point(L, W, dense=(3.0, 2.9), sparse=(0.008, 0.0079), quant=(0.006, 0.0059),
                 quant_bytes=BM.quantized_bytes(W))
    p.cpu.update(dense=100.0, sparse=1.0, quantized=2.0)
    return p


def test_csv_columns_start_with_the_reference_columns(tmp_path):
    """Both tables lead with the reference's two CSV headers, in its order
    (benchmark.py:66-72, :140-149), and end with the host fields."""
    ref_dense = ["L", "W", "ms_sparse", "ms_dense", "measured_ratio", "predicted_ratio", "gap_pct"]
    ref_quant = ["L", "W", "ms_dense", "ms_sparse", "ms_quantized", "bytes_sparse_pred",
                 "bytes_quantized_pred", "predicted_marginal_multiplier",
                 "measured_marginal_multiplier", "gap_pct"]
    info = BM.HostInfo(16, "Test CPU")
    for ref, table in ((ref_dense, BM.SPARSE_TABLE), (ref_quant, BM.QUANT_TABLE)):
        path = os.path.join(tmp_path, "r.csv")
        assert BM.write_table(table, [_point(), _point(8192, 4096)], path, info) == 2
        rows = list(csv.reader(open(path)))
        assert rows[0][:len(ref)] == ref
        assert rows[0][-2:] == ["cpu_threads", "cpu_model"] and rows[1][-2:] == ["16", "Test CPU"]


def test_table_values_follow_the_reference_formulas():
    """ratios and gap as the reference computes them (benchmark.py:61-63,
    :133-135), on a hand-made point."""
    p = _point()
    row = {name: fn(p) for name, fn in BM.SPARSE_TABLE}
    pred = (1_048_576 + 131_072 * 163_840) / (1_048_576 + 131_072 * 260)
    assert abs(row["predicted_ratio"] - pred) < 1e-9
    assert abs(row["measured_ratio"] - 3.0 / 0.008) < 1e-9
    assert abs(row["gap_pct"] - 100 * (3.0 / 0.008 - pred) / pred) < 1e-9
    qrow = {name: fn(p) for name, fn in BM.QUANT_TABLE}
    pm = 35_127_296 / 21_757_952
    assert qrow["bytes_quantized_pred"] == 21_757_952 and qrow["bytes_quantized_min"] == 21_184_512
    assert abs(qrow["predicted_marginal_multiplier"] - pm) < 1e-12
    assert abs(qrow["gap_pct"] - 100 * (0.008 / 0.006 - pm) / pm) < 1e-9
    assert abs(qrow["pct_peak_quantized"] - 100 * 21_184_512 / 6e-6 / 8e12) < 1e-9


def test_host_baseline_unpack_matches_oracle():
    """The CPU baseline's dequantization (batch row 0 of a cache) equals the
    oracle's unpack_dequant for K (tokens packed) and V (channels packed)."""
    import numpy as np
    import torch
    from oracle import kvdec_oracle as O
    rng = np.random.default_rng(3)
    x = rng.standard_normal((1, 2, 96, 128)).astype(np.float32)
    for fn, axis, n in ((O.quantize_k, 1, 96), (O.quantize_v, 2, 128)):
        p, s, z = fn(x)
        got = BM._host_unpack(torch.from_numpy(p[0]), torch.from_numpy(s[0]), torch.from_numpy(z[0]), axis, n)
        want = O.unpack_dequant(p, s, z, n, axis + 1)[0]
        np.testing.assert_array_equal(got.numpy(), want)
