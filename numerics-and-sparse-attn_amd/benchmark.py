"""Context-length x window sweep of the decode paths on one MI355X.

Drop-in for the reference's benchmark.py (benchmark.py:34-169): the same two
result tables (dense vs. native sparse; quantized sparse vs. native sparse
and dense), the KIVI cache built outside the timed region
(benchmark.py:104-106), the reference's byte models (B_FIXED_FP16 +
C_FP16 * tokens, benchmark.py:30-31,56-57; quantized bytes = every cache
tensor's size + Q + O, benchmark.py:121-129) and its CSV columns, in its
order, followed by extra columns:

  *_median           median of the per-call times (the ms_* columns are means)
  tbs_* / pct_peak_* achieved TB/s of the path's predicted bytes, and that as
                     a percentage of MI355X's 8 TB/s
  cpu_ms_*_b1        the same step at batch 1 in float32 on the host CPU
                     (torch), a labelled baseline; 0 with --no-cpu
  cpu_threads, cpu_model
                     the host threads the CPU columns used and the CPU model

    python benchmark.py [--quick] [--no-cpu] [--out-dir results]

How it is organised: each context length's dense cache and each window's
sparse and KIVI caches are allocated once (fp16 N(0, 1) from torch.randn on
the GPU, as in the reference); every (L, W) point then times the three
decodes on them.  A table is a list of column specs (name, value of a
measured point); rows, the console table and the CSV all come from it.  The
dense decode is timed once per L and shared by both tables (the reference
re-times it in its second sweep).

Timing follows triton.testing.do_bench (which the reference uses): estimate
the call time, warm up for ~25 ms, then time ~100 ms worth of calls, each
preceded by zeroing a flush buffer, with one pair of events per call; the
mean is reported.  The flush buffer here is 1 GiB (the reference's do_bench
uses 256 MB), more than this GPU's L2 plus its 256 MB Infinity Cache.
"""

from __future__ import annotations

import argparse
import csv
import os
import platform
import time
from dataclasses import dataclass, field
from typing import Callable, Dict, List, Optional, Tuple

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
KIVI_KEYS = ("k_residual", "v_residual",
             "k_sink_packed", "k_sink_scale", "k_sink_zero",
             "v_sink_packed", "v_sink_scale", "v_sink_zero",
             "k_win_packed", "k_win_scale", "k_win_zero",
             "v_win_packed", "v_win_scale", "v_win_zero")

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
# Host CPU baseline: batch 1, float32, torch.  The decode's math (softmax of
# q K^T * scale, times V, GQA by grouping the query heads) on the positions
# each path attends to, after dequantizing for the quantized path; timing
# only, no result is used.
# --------------------------------------------------------------------------

@dataclass
class HostInfo:
    threads: int
    model: str

    @staticmethod
    def probe() -> "HostInfo":
        model = platform.processor() or "unknown"
        try:
            with open("/proc/cpuinfo") as f:
                for line in f:
                    if line.startswith("model name"):
                        model = line.split(":", 1)[1].strip()
                        break
        except OSError:
            pass
        return HostInfo(torch.get_num_threads(), model)


def _median_ms(fn, reps: int) -> float:
    fn()
    samples = []
    for _ in range(reps):
        t = time.perf_counter()
        fn()
        samples.append(time.perf_counter() - t)
    return sorted(samples)[len(samples) // 2] * 1e3


def _host_attend(q, k, v):
    """q [H, D]; k, v [KVH, T, D] -> [H, D]."""
    kvh = k.shape[0]
    p = torch.softmax(torch.matmul(q.view(kvh, -1, q.shape[-1]), k.transpose(1, 2)) * D_HEAD**-0.5, -1)
    return torch.matmul(p, v).reshape(q.shape)


def _host_unpack(packed, scale, zero, axis, n):
    """Codes of `packed` (LSB first along `axis`), dequantized per group of 32."""
    p = packed.to(torch.int32)
    codes = torch.stack([(p >> (2 * j)) & 3 for j in range(4)], dim=axis + 1).flatten(axis, axis + 1)
    codes = codes.narrow(axis, 0, n).float()
    grp = torch.arange(n) // 32
    return scale.float().index_select(axis, grp) * (codes - zero.float().index_select(axis, grp))


class HostBaseline:
    """Per-L and per-W batch-1 CPU times, each measured once and memoised."""

    def __init__(self, reps: int = 5):
        self.reps = reps
        self.memo: Dict[Tuple[str, int], float] = {}
        self.gen = torch.Generator().manual_seed(0)

    def _rand(self, *shape):
        return torch.randn(*shape, generator=self.gen)

    def dense(self, L: int) -> float:
        key = ("dense", L)
        if key not in self.memo:
            q, k, v = self._rand(N_HEADS, D_HEAD), self._rand(N_KV_HEADS, L, D_HEAD), self._rand(N_KV_HEADS, L, D_HEAD)
            self.memo[key] = _median_ms(lambda: _host_attend(q, k, v), 3 if L > 65536 else self.reps)
        return self.memo[key]

    def sparse(self, W: int) -> float:
        key = ("sparse", W)
        if key not in self.memo:
            n = SINK_SIZE + W
            q, k, v = self._rand(N_HEADS, D_HEAD), self._rand(N_KV_HEADS, n, D_HEAD), self._rand(N_KV_HEADS, n, D_HEAD)
            self.memo[key] = _median_ms(lambda: _host_attend(q, k, v), self.reps)
        return self.memo[key]

    def quantized(self, W: int, cache: dict) -> float:
        key = ("quantized", W)
        if key not in self.memo:
            c = {name: t[0].cpu() for name, t in cache.items()}
            q = self._rand(N_HEADS, D_HEAD)
            win = W - RESIDUAL_SIZE

            def step():
                ks = [_host_unpack(c["k_sink_packed"], c["k_sink_scale"], c["k_sink_zero"], 1, SINK_SIZE)]
                vs = [_host_unpack(c["v_sink_packed"], c["v_sink_scale"], c["v_sink_zero"], 2, D_HEAD)[:, :SINK_SIZE]]
                if win > 0:
                    ks.append(_host_unpack(c["k_win_packed"], c["k_win_scale"], c["k_win_zero"], 1, win))
                    vs.append(_host_unpack(c["v_win_packed"], c["v_win_scale"], c["v_win_zero"], 2, D_HEAD))
                ks.append(c["k_residual"].float())
                vs.append(c["v_residual"].float())
                return _host_attend(q, torch.cat(ks, 1), torch.cat(vs, 1))

            self.memo[key] = _median_ms(step, self.reps)
        return self.memo[key]


# --------------------------------------------------------------------------
# Measurement
# --------------------------------------------------------------------------

@dataclass
class Point:
    """Everything measured at one (L, W)."""
    L: int
    W: int
    dense: Tuple[float, float]                 # (mean, median) ms
    sparse: Tuple[float, float]
    quant: Optional[Tuple[float, float]] = None
    quant_bytes: Tuple[int, int] = (0, 0)      # (reference accounting, minimal)
    cpu: Dict[str, float] = field(default_factory=dict)


def _sparse_bytes(W: int) -> int:
    return B_FIXED_FP16 + C_FP16 * (W + SINK_SIZE)


def _dense_bytes(L: int) -> int:
    return B_FIXED_FP16 + C_FP16 * L


def _tbs(nbytes: float, ms: float) -> float:
    return nbytes / (ms * 1e-3) / 1e12


def _fp16_randn(*shape):
    return torch.randn(*shape, dtype=torch.float16, device="cuda")


def measure(contexts: List[int], windows: List[int], host: Optional[HostBaseline],
            report: Callable[[Point], None] = lambda p: None) -> List[Point]:
    """Time dense, sparse and (W >= residual) quantized decode at every (L, W)."""
    q = _fp16_randn(BATCH, N_HEADS, D_HEAD)
    sparse_cache, kivi_cache = {}, {}
    for W in windows:
        sparse_cache[W] = (_fp16_randn(BATCH, N_KV_HEADS, SINK_SIZE + W, D_HEAD),
                           _fp16_randn(BATCH, N_KV_HEADS, SINK_SIZE + W, D_HEAD))
        if W >= RESIDUAL_SIZE:
            # untimed setup, as in the reference: quantized once, outside every timed call
            built = build_quantized_kv_cache(*sparse_cache[W])
            kivi_cache[W] = [built[name] for name in KIVI_KEYS]
            allocated = sum(t.numel() * t.element_size() for t in kivi_cache[W]) + 2 * q.numel() * q.element_size()
            assert allocated == quantized_bytes(W)[0], (W, allocated)
    points = []
    for L in contexts:
        kd, vd = _fp16_randn(BATCH, N_KV_HEADS, L, D_HEAD), _fp16_randn(BATCH, N_KV_HEADS, L, D_HEAD)
        t_dense = do_bench(lambda: dense_decode_attention(q, kd, vd, seq_len=L, sm_scale=D_HEAD**-0.5))
        for W in windows:
            kc, vc = sparse_cache[W]
            pt = Point(L, W, t_dense, do_bench(lambda: sparse_decode_attention(q, kc, vc, seq_len=L, window=W)))
            if W in kivi_cache:
                parts = kivi_cache[W]
                pt.quant = do_bench(lambda: sparse_decode_attention_quantized(q, *parts, seq_len=L, window=W))
                pt.quant_bytes = quantized_bytes(W)
            if host is not None:
                pt.cpu["dense"] = host.dense(L)
                pt.cpu["sparse"] = host.sparse(W)
                if W in kivi_cache:
                    pt.cpu["quantized"] = host.quantized(W, dict(zip(KIVI_KEYS, kivi_cache[W])))
            points.append(pt)
            report(pt)
        del kd, vd
    return points


# --------------------------------------------------------------------------
# Tables: (column name, value of a Point); the first columns are the
# reference's, in its order.
# --------------------------------------------------------------------------

Column = Tuple[str, Callable[[Point], object]]


def _pct(tbs: float) -> float:
    return 100 * tbs / PEAK_TBS


SPARSE_TABLE: List[Column] = [
    ("L", lambda p: p.L),
    ("W", lambda p: p.W),
    ("ms_sparse", lambda p: p.sparse[0]),
    ("ms_dense", lambda p: p.dense[0]),
    ("measured_ratio", lambda p: p.dense[0] / p.sparse[0]),
    ("predicted_ratio", lambda p: _dense_bytes(p.L) / _sparse_bytes(p.W)),
    ("gap_pct", lambda p: 100 * (p.dense[0] / p.sparse[0]) / (_dense_bytes(p.L) / _sparse_bytes(p.W)) - 100),
    ("ms_sparse_median", lambda p: p.sparse[1]),
    ("ms_dense_median", lambda p: p.dense[1]),
    ("tbs_sparse", lambda p: _tbs(_sparse_bytes(p.W), p.sparse[0])),
    ("pct_peak_sparse", lambda p: _pct(_tbs(_sparse_bytes(p.W), p.sparse[0]))),
    ("tbs_dense", lambda p: _tbs(_dense_bytes(p.L), p.dense[0])),
    ("pct_peak_dense", lambda p: _pct(_tbs(_dense_bytes(p.L), p.dense[0]))),
    ("cpu_ms_sparse_b1", lambda p: p.cpu.get("sparse", 0.0)),
    ("cpu_ms_dense_b1", lambda p: p.cpu.get("dense", 0.0)),
]

QUANT_TABLE: List[Column] = [
    ("L", lambda p: p.L),
    ("W", lambda p: p.W),
    ("ms_dense", lambda p: p.dense[0]),
    ("ms_sparse", lambda p: p.sparse[0]),
    ("ms_quantized", lambda p: p.quant[0]),
    ("bytes_sparse_pred", lambda p: _sparse_bytes(p.W)),
    ("bytes_quantized_pred", lambda p: p.quant_bytes[0]),
    ("predicted_marginal_multiplier", lambda p: _sparse_bytes(p.W) / p.quant_bytes[0]),
    ("measured_marginal_multiplier", lambda p: p.sparse[0] / p.quant[0]),
    ("gap_pct", lambda p: 100 * (p.sparse[0] / p.quant[0]) / (_sparse_bytes(p.W) / p.quant_bytes[0]) - 100),
    ("ms_quantized_median", lambda p: p.quant[1]),
    ("bytes_quantized_min", lambda p: p.quant_bytes[1]),
    ("tbs_quantized", lambda p: _tbs(p.quant_bytes[1], p.quant[0])),
    ("pct_peak_quantized", lambda p: _pct(_tbs(p.quant_bytes[1], p.quant[0]))),
    ("dense_over_quantized", lambda p: p.dense[0] / p.quant[0]),
    ("cpu_ms_quantized_b1", lambda p: p.cpu.get("quantized", 0.0)),
]


def write_table(table: List[Column], points: List[Point], path: str, host: Optional[HostInfo]) -> int:
    """Evaluate `table` on every point, print it aligned, write it as CSV
    (with the host fields as trailing columns); returns the row count."""
    names = [name for name, _ in table] + ["cpu_threads", "cpu_model"]
    meta = [host.threads, host.model] if host else [0, ""]
    rows = [[fn(p) for _, fn in table] + meta for p in points]
    cell = lambda v: f"{v:>14.5g}" if isinstance(v, float) else f"{str(v)[:14]:>14}"
    print("".join(f"{n[:14]:>14}" for n in names[:len(table)]))
    for r in rows:
        print("".join(cell(v) for v in r[:len(table)]))
    with open(path, "w", newline="") as f:
        out = csv.writer(f)
        out.writerow(names)
        out.writerows(rows)
    print(f"{len(rows)} rows -> {path}", flush=True)
    return len(rows)


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
    host, info = None, None
    if not a.no_cpu:
        host, info = HostBaseline(), HostInfo.probe()
        print(f"CPU baseline: torch float32, batch 1, {info.threads} threads ({info.model}; "
              f"os.cpu_count() = {os.cpu_count()})", flush=True)
    os.makedirs(a.out_dir, exist_ok=True)

    def report(p: Point):
        q = f" quantized={p.quant[0]:.4f}" if p.quant else ""
        print(f"  L={p.L:<6d} W={p.W:<5d} dense={p.dense[0]:.4f} sparse={p.sparse[0]:.4f}{q} ms", flush=True)

    points = measure(contexts, windows, host, report)
    write_table(SPARSE_TABLE, points, os.path.join(a.out_dir, "benchmark_results.csv"), info)
    write_table(QUANT_TABLE, [p for p in points if p.quant], os.path.join(a.out_dir, "benchmark_results_quantized.csv"),
                info)


if __name__ == "__main__":
    main()
