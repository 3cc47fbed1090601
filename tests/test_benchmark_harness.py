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


def test_csv_columns_start_with_the_reference_columns(tmp_path):
    # the reference's two CSV headers (benchmark.py:66-72, :140-149)
    ref_dense = ["L", "W", "ms_sparse", "ms_dense", "measured_ratio", "predicted_ratio", "gap_pct"]
    ref_quant = ["L", "W", "ms_dense", "ms_sparse", "ms_quantized", "bytes_sparse_pred",
                 "bytes_quantized_pred", "predicted_marginal_multiplier",
                 "measured_marginal_multiplier", "gap_pct"]
    for ref, extra in ((ref_dense, {"tbs_sparse": 1.0}), (ref_quant, {"tbs_quantized": 1.0})):
        row = {k: 1.0 for k in ref}
        row.update(extra)
        path = os.path.join(tmp_path, "r.csv")
        BM._print_and_save([row], path)
        header = next(csv.reader(open(path)))
        assert header[:len(ref)] == ref
