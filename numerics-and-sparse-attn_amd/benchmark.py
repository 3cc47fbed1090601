"""Context-length x window sweep of the decode paths on one MI355X.

Drop-in for the reference's benchmark.py (benchmark.py:34-169): the same two
sweeps, the same untimed setup (the KIVI cache is built outside the timed
region, benchmark.py:104-106), the same byte models (B_FIXED_FP16 +
C_FP16 * tokens, benchmark.py:30-31,56-57; quantized bytes = every cache
tensor's size + Q + O, benchmark.py:121-129) and the same CSV columns, in
the same order, followed by extra columns:

  *_median           median of the per-call times (the ms_* columns are means)
  tbs_* / pct_peak_* achieved TB/s of the path's predicted bytes, and that as
                     a percentage of MI355X's 8 TB/s
  cpu_ms_*_b1        the same step at batch 1 in float32 on the host CPU
                     (torch, all cores), a labelled baseline; 0 with --no-cpu

    python benchmark.py [--quick] [--no-cpu] [--out-dir results]

Timing follows triton.testing.do_bench (which the reference uses): estimate
the call time, warm up for ~25 ms, then time ~100 ms worth of calls, each
preceded by zeroing a flush buffer, with one pair of events per call; the
mean is reported.  The flush buffer here is 1 GiB (the reference's do_bench
uses 256 MB), more than this GPU's L2 plus its 256 MB Infinity Cache.
Inputs are fp16 N(0, 1) from torch.randn on the GPU, as in the reference.
"""

from __future__ import annotations

import argparse
import csv
import os
import time

import torch

from constants import (
    BATCH, CONTEXT_LENGTHS, D_HEAD, N_HEADS, N_KV_HEADS, RESIDUAL_SIZE, SINK_SIZE, WINDOW_SIZES,
)
from dense_kernel import dense_decode_attention
from quant_kernel import build_quantized_kv_cache, sparse_decode_attention_quantized
from sparse_kernel import sparse_decode_attention

B_FIXED_FP16 = 1_048_576     # Q + O bytes at B=32, H=64, D=128, fp16
C_FP16 = 131_072             # K + V bytes per token across the batch, fp16
PEAK_TBS = 8.0               # MI355X HBM3E
FLUSH_BYTES = 1 << 30

_flush = None


def do_bench(fn, warmup_ms: float = 25.0, rep_ms: float = 100.0):
    """Mean and median milliseconds per call of fn() with cold caches."""
    global _flush
    if _flush is None:
        _flush = torch.empty(FLUSH_BYTES, dtype=torch.int8, device="cuda")
    fn()
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(5):
        _flush.zero_()
        fn()
    t1.record()
    torch.cuda.synchronize()
    est = max(t0.elapsed_time(t1) / 5, 1e-3)
    n_warmup = max(1, int(warmup_ms / est))
    n_rep = max(1, int(rep_ms / est))
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(n_rep)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(n_rep)]
    for _ in range(n_warmup):
        fn()
    for i in range(n_rep):
        _flush.zero_()
        starts[i].record()
        fn()
        ends[i].record()
    torch.cuda.synchronize()
    times = sorted(s.elapsed_time(e) for s, e in zip(starts, ends))
    return sum(times) / len(times), times[len(times) // 2]


def _tbs(nbytes: int, ms: float) -> float:
    return nbytes / (ms * 1e-3) / 1e12


def quantized_bytes(W: int, group: int = 32):
    """(reference accounting, minimal) bytes of one quantized decode step.

    Reference accounting (benchmark.py:121-129): every tensor of the cache
    that build_quantized_kv_cache returns, at its allocated size (the sink
    group padded to `group` tokens), plus Q and O.  Minimal: only the `sink`
    real tokens of the sink group are read (their packed K row, their packed
    V rows and V scales / zeros)."""
    bk = BATCH * N_KV_HEADS
    win = W - RESIDUAL_SIZE
    residual = 2 * bk * RESIDUAL_SIZE * D_HEAD * 2
    sink = bk * (group // 4 * D_HEAD + 2 * D_HEAD * 2 + group * (D_HEAD // 4) + 2 * group * (D_HEAD // 32) * 2)
    window_old = bk * (win // 4 * D_HEAD + 2 * (win // group) * D_HEAD * 2 + win * (D_HEAD // 4)
                       + 2 * win * (D_HEAD // 32) * 2)
    qo = 2 * BATCH * N_HEADS * D_HEAD * 2
    ref = residual + sink + window_old + qo
    pad = group - SINK_SIZE
    unread = bk * (pad // 4 * D_HEAD + pad * (D_HEAD // 4) + 2 * pad * (D_HEAD // 32) * 2)
    return ref, ref - unread


# --------------------------------------------------------------------------
# Host CPU baselines (batch 1, float32, torch on all cores).  Restatements of
# the reference tests' PyTorch oracles (test_dense_correctness.py,
# test_sparse_correctness.py, test_quantized_attention_correctness.py) on the
# positions each path attends to; used only as a timing baseline.
# --------------------------------------------------------------------------

def _cpu_attend(q, k, v, scale):
    """q [H, D]; k, v [KVH, T, D] -> o [H, D] (GQA, float32)."""
    g = q.shape[0] // k.shape[0]
    qg = q.view(k.shape[0], g, -1)
    s = torch.matmul(qg, k.transpose(1, 2)) * scale
    p = torch.softmax(s, dim=-1)
    return torch.matmul(p, v).reshape(q.shape)


def _cpu_time(fn, reps: int = 5) -> float:
    fn()
    ts = []
    for _ in range(reps):
        t = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t)
    ts.sort()
    return ts[len(ts) // 2] * 1e3


def cpu_dense_ms(L: int) -> float:
    g = torch.Generator().manual_seed(0)
    q = torch.randn(N_HEADS, D_HEAD, generator=g)
    k = torch.randn(N_KV_HEADS, L, D_HEAD, generator=g)
    v = torch.randn(N_KV_HEADS, L, D_HEAD, generator=g)
    return _cpu_time(lambda: _cpu_attend(q, k, v, D_HEAD**-0.5), reps=3 if L > 65536 else 5)


def cpu_sparse_ms(W: int) -> float:
    # steady state: all sink + window slots are valid
    g = torch.Generator().manual_seed(0)
    n = SINK_SIZE + W
    q = torch.randn(N_HEADS, D_HEAD, generator=g)
    k = torch.randn(N_KV_HEADS, n, D_HEAD, generator=g)
    v = torch.randn(N_KV_HEADS, n, D_HEAD, generator=g)
    return _cpu_time(lambda: _cpu_attend(q, k, v, D_HEAD**-0.5))


def _cpu_dequant_k(packed, scale, zero, n):
    codes = torch.stack([(packed >> (2 * j)) & 3 for j in range(4)], dim=-2)   # [KVH, n/4, 4, D]
    codes = codes.reshape(packed.shape[0], -1, packed.shape[-1])[:, :n].float()
    s = scale.float().repeat_interleave(32, dim=1)[:, :n]
    z = zero.float().repeat_interleave(32, dim=1)[:, :n]
    return s * (codes - z)


def _cpu_dequant_v(packed, scale, zero):
    codes = torch.stack([(packed >> (2 * j)) & 3 for j in range(4)], dim=-1)   # [KVH, n, D/4, 4]
    codes = codes.reshape(packed.shape[0], packed.shape[1], -1).float()
    s = scale.float().repeat_interleave(32, dim=2)
    z = zero.float().repeat_interleave(32, dim=2)
    return s * (codes - z)


def cpu_quantized_ms(cache: dict, W: int) -> float:
    """Dequantize-then-attend over the 4 real sink tokens, the window-old
    tokens and the fp16 residual of batch row 0."""
    c = {k: t[0].cpu() for k, t in cache.items()}
    g = torch.Generator().manual_seed(0)
    q = torch.randn(N_HEADS, D_HEAD, generator=g)
    win = W - RESIDUAL_SIZE

    def step():
        ks = [_cpu_dequant_k(c["k_sink_packed"], c["k_sink_scale"], c["k_sink_zero"], SINK_SIZE)]
        vs = [_cpu_dequant_v(c["v_sink_packed"], c["v_sink_scale"], c["v_sink_zero"])[:, :SINK_SIZE]]
        if win > 0:
            ks.append(_cpu_dequant_k(c["k_win_packed"], c["k_win_scale"], c["k_win_zero"], win))
            vs.append(_cpu_dequant_v(c["v_win_packed"], c["v_win_scale"], c["v_win_zero"]))
        ks.append(c["k_residual"].float())
        vs.append(c["v_residual"].float())
        return _cpu_attend(q, torch.cat(ks, 1), torch.cat(vs, 1), D_HEAD**-0.5)

    return _cpu_time(step)


# --------------------------------------------------------------------------
# Sweeps
# --------------------------------------------------------------------------

def benchmark(contexts, windows, cpu: bool):
    """Native sparse vs. dense, both fp16, across the sweep
    (benchmark.py:34-73)."""
    sm_scale = D_HEAD**-0.5
    device = "cuda"
    results = []
    cpu_dense, cpu_sparse = {}, {}
    for L in contexts:
        k_dense = torch.randn(BATCH, N_KV_HEADS, L, D_HEAD, dtype=torch.float16, device=device)
        v_dense = torch.randn(BATCH, N_KV_HEADS, L, D_HEAD, dtype=torch.float16, device=device)
        if cpu and L not in cpu_dense:
            cpu_dense[L] = cpu_dense_ms(L)
        for W in windows:
            q = torch.randn(BATCH, N_HEADS, D_HEAD, dtype=torch.float16, device=device)
            k_cache = torch.randn(BATCH, N_KV_HEADS, SINK_SIZE + W, D_HEAD, dtype=torch.float16,
                                  device=device)
            v_cache = torch.randn(BATCH, N_KV_HEADS, SINK_SIZE + W, D_HEAD, dtype=torch.float16,
                                  device=device)
            ms_sparse, md_sparse = do_bench(
                lambda: sparse_decode_attention(q, k_cache, v_cache, seq_len=L, window=W))
            ms_dense, md_dense = do_bench(
                lambda: dense_decode_attention(q, k_dense, v_dense, seq_len=L, sm_scale=sm_scale))
            if cpu and W not in cpu_sparse:
                cpu_sparse[W] = cpu_sparse_ms(W)

            bytes_sparse_pred = B_FIXED_FP16 + C_FP16 * (W + SINK_SIZE)
            bytes_dense_pred = B_FIXED_FP16 + C_FP16 * L
            predicted_ratio = bytes_dense_pred / bytes_sparse_pred
            measured_ratio = ms_dense / ms_sparse
            gap_pct = 100 * (measured_ratio - predicted_ratio) / predicted_ratio
            results.append({
                "L": L, "W": W,
                "ms_sparse": ms_sparse, "ms_dense": ms_dense,
                "measured_ratio": measured_ratio,
                "predicted_ratio": predicted_ratio,
                "gap_pct": gap_pct,
                "ms_sparse_median": md_sparse, "ms_dense_median": md_dense,
                "tbs_sparse": _tbs(bytes_sparse_pred, ms_sparse),
                "pct_peak_sparse": 100 * _tbs(bytes_sparse_pred, ms_sparse) / PEAK_TBS,
                "tbs_dense": _tbs(bytes_dense_pred, ms_dense),
                "pct_peak_dense": 100 * _tbs(bytes_dense_pred, ms_dense) / PEAK_TBS,
                "cpu_ms_sparse_b1": cpu_sparse.get(W, 0.0),
                "cpu_ms_dense_b1": cpu_dense.get(L, 0.0),
            })
            _progress(results[-1])
        del k_dense, v_dense
    return results


def benchmark_quantized(contexts, windows, cpu: bool):
    """Quantized sparse vs. native sparse (and dense), windows >= the
    residual size (benchmark.py:76-153)."""
    sm_scale = D_HEAD**-0.5
    device = "cuda"
    results = []
    cpu_q = {}
    windows = [w for w in windows if w >= RESIDUAL_SIZE]
    for L in contexts:
        k_dense = torch.randn(BATCH, N_KV_HEADS, L, D_HEAD, dtype=torch.float16, device=device)
        v_dense = torch.randn(BATCH, N_KV_HEADS, L, D_HEAD, dtype=torch.float16, device=device)
        for W in windows:
            q = torch.randn(BATCH, N_HEADS, D_HEAD, dtype=torch.float16, device=device)
            k_compacted = torch.randn(BATCH, N_KV_HEADS, SINK_SIZE + W, D_HEAD, dtype=torch.float16,
                                      device=device)
            v_compacted = torch.randn(BATCH, N_KV_HEADS, SINK_SIZE + W, D_HEAD, dtype=torch.float16,
                                      device=device)
            ms_sparse, _ = do_bench(
                lambda: sparse_decode_attention(q, k_compacted, v_compacted, seq_len=L, window=W))
            ms_dense, _ = do_bench(
                lambda: dense_decode_attention(q, k_dense, v_dense, seq_len=L, sm_scale=sm_scale))

            # untimed setup: the cache is quantized once, outside the timed region
            cache = build_quantized_kv_cache(k_compacted, v_compacted)
            ms_quantized, md_quantized = do_bench(
                lambda: sparse_decode_attention_quantized(
                    q, cache["k_residual"], cache["v_residual"],
                    cache["k_sink_packed"], cache["k_sink_scale"], cache["k_sink_zero"],
                    cache["v_sink_packed"], cache["v_sink_scale"], cache["v_sink_zero"],
                    cache["k_win_packed"], cache["k_win_scale"], cache["k_win_zero"],
                    cache["v_win_packed"], cache["v_win_scale"], cache["v_win_zero"],
                    seq_len=L, window=W,
                ))
            if cpu and W not in cpu_q:
                cpu_q[W] = cpu_quantized_ms(cache, W)

            quant_tensors = [cache[k] for k in (
                "k_residual", "v_residual",
                "k_sink_packed", "k_sink_scale", "k_sink_zero",
                "v_sink_packed", "v_sink_scale", "v_sink_zero",
                "k_win_packed", "k_win_scale", "k_win_zero",
                "v_win_packed", "v_win_scale", "v_win_zero")]
            bytes_quantized_pred = sum(t.numel() * t.element_size() for t in quant_tensors) \
                + 2 * q.numel() * q.element_size()
            ref_bytes, bytes_quantized_min = quantized_bytes(W)
            assert bytes_quantized_pred == ref_bytes, (bytes_quantized_pred, ref_bytes)
            bytes_sparse_pred = B_FIXED_FP16 + C_FP16 * (W + SINK_SIZE)
            predicted = bytes_sparse_pred / bytes_quantized_pred
            measured = ms_sparse / ms_quantized
            gap_pct = 100 * (measured - predicted) / predicted
            results.append({
                "L": L, "W": W,
                "ms_dense": ms_dense, "ms_sparse": ms_sparse, "ms_quantized": ms_quantized,
                "bytes_sparse_pred": bytes_sparse_pred, "bytes_quantized_pred": bytes_quantized_pred,
                "predicted_marginal_multiplier": predicted,
                "measured_marginal_multiplier": measured,
                "gap_pct": gap_pct,
                "ms_quantized_median": md_quantized,
                "bytes_quantized_min": bytes_quantized_min,
                "tbs_quantized": _tbs(bytes_quantized_min, ms_quantized),
                "pct_peak_quantized": 100 * _tbs(bytes_quantized_min, ms_quantized) / PEAK_TBS,
                "dense_over_quantized": ms_dense / ms_quantized,
                "cpu_ms_quantized_b1": cpu_q.get(W, 0.0),
            })
            _progress(results[-1])
            del cache
        del k_dense, v_dense
    return results


def _progress(r):
    keys = [k for k in r if k.startswith("ms_") and not k.endswith("median")]
    print("  L=%-6d W=%-5d " % (r["L"], r["W"]) + " ".join(f"{k}={r[k]:.4f}" for k in keys), flush=True)


def _print_and_save(results, path):
    header = list(results[0].keys())
    print(" ".join(f"{h:>12}" for h in header))
    for r in results:
        print(" ".join(f"{v:>12.4f}" if isinstance(v, float) else f"{v:>12}" for v in r.values()))
    with open(path, "w", newline="") as f:
        writer = csv.DictWriter(f, fieldnames=header)
        writer.writeheader()
        writer.writerows(results)
    print(f"\nSaved {len(results)} rows to {path}", flush=True)


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--quick", action="store_true",
                    help="L in {8192, 163840}, W in {0, 32, 128, 256, 4096} only")
    ap.add_argument("--no-cpu", action="store_true", help="skip the host CPU baseline columns")
    ap.add_argument("--out-dir", default="results")
    a = ap.parse_args(argv)
    if not torch.cuda.is_available():
        raise SystemExit("benchmark.py needs a GPU (the kernels are HIP for gfx950)")
    contexts = [8192, 163840] if a.quick else CONTEXT_LENGTHS
    windows = [0, 32, 128, 256, 4096] if a.quick else WINDOW_SIZES
    if not a.no_cpu:
        torch.set_num_threads(os.cpu_count() or 1)
        print(f"CPU baseline: torch float32, batch 1, {torch.get_num_threads()} threads", flush=True)
    os.makedirs(a.out_dir, exist_ok=True)
    _print_and_save(benchmark(contexts, windows, not a.no_cpu),
                    os.path.join(a.out_dir, "benchmark_results.csv"))
    _print_and_save(benchmark_quantized(contexts, windows, not a.no_cpu),
                    os.path.join(a.out_dir, "benchmark_results_quantized.csv"))


if __name__ == "__main__":
    main()
