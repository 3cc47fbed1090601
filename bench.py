"""Decode-attention benchmark on one MI355X: prints ONE JSON line.

    python bench.py [--gpus 1] [--steps K] [--warmup W]
                    [--paths kivi,sweep,dense,sparse,quantize,stream,paged,grid]
                    [--no-cpu] [--no-latency]

Workload (the headline metric's configuration): B=32, 64 query / 8 KV heads,
head_dim 128, logical context L=163840, sink S=4, window W=256, KIVI residual
R=128, fp16 inputs ~ N(0,1) from a fixed seed with 4 of the 128 K channels
scaled x10.  A "step" is one decode call of a path over the whole batch:

  kivi      fused sink+window(W=256)+KIVI-2bit decode (the headline ``value``)
  sweep     the fused decode at W = 32, 1024 and 4096 (config 5; W=32 < R,
            which the reference leaves undefined, keeps the window fp16)
  dense     dense GQA decode over all 163840 tokens (and L=32768, config 2)
  sparse    fp16 sink+window(W=256) decode (config 3)
  quantize  KIVI quantization of the [32, 8, 163840, 128] K and V caches (config 4)
  stream    a decode loop on the streaming KIVI cache (kivi_stream.py, W=256):
            reserve the next token's ring row (quantizing a block every 32
            steps), then attend; also the same loop with one ring state per
            sequence (KiviStreamBatch.step_attend: the token's row write,
            evictions, bookkeeping and decode in one launch)
  paged     the dense L=163840 cache scattered over 16-token pages in a
            random order (vLLM's [pages, 16, KVH, D] layout), decoded through
            block tables and per-sequence lengths (paged_kernel.py)
  floor     per-step floors of this box: an empty launch of the decode grid
            and a plain streaming read of each path's algorithmic bytes
            (kvdec_read_probe, best of 512 and 1024 workgroups), timed the
            same way; each path records read_floor_us and frac_of_read_floor
  grid      the reference harness's sweep (benchmark.py:34-169): dense at
            every L of CONTEXT_LENGTHS, sparse at every W of WINDOW_SIZES and
            the fused KIVI decode at W = 32 and every W >= R, with the
            batch-1 host CPU time beside each point.  Sparse and KIVI steps
            read the same bytes at every L >= S + W (steady state), so they
            are timed once per W at L = 163840.

Timing.  Each path keeps enough independent input sets resident in HBM that
one pass over them is >= 1 GiB (more than L2 plus the 256 MB Infinity
Cache), captures G back-to-back calls cycling through every set in one HIP
graph, replays it untimed, then times R back-to-back replays between two
HIP events on the capture stream: ``us_per_step`` = that time / (R * G), the
steady-state cost of a decode step whose inputs are cold in every cache,
with launches pipelined as in a decode loop.  A replay carries a fixed cost
of its own (~20 us measured: a 51-step graph replayed 20 times gave 6.93 us
per KIVI step where a 400-step graph gave 6.49), so the microsecond-scale
paths use G = max(K, sets, 512) and R * G >= 1000 whatever K is; the
millisecond-scale paths use G = min(K, 20) (at least 4) and R = 2.
``latency_us`` is the reference harness's method (triton do_bench): a 1 GiB
buffer write before each single call, events around the call; it adds the
per-call dispatch latency (about 5 us on this system for an empty kernel).

``roofline.traffic`` is the HBM bytes per launch recorded by the rocprofv3
FETCH_SIZE / WRITE_SIZE runs in profiles/hbm_traffic.json; each record
names the kernel sources it was measured on (a hash), and the line reports
null when the sources have changed since.

The CPU baseline times the repository's torch restatement of the
reference's PyTorch test oracles (oracle/torch_ref.py) on the host, float32,
with torch's thread pool as the process finds it (OMP_NUM_THREADS; 16 on
the GPU boxes, which is this process's CPU share there).
"""

from __future__ import annotations

import argparse
import hashlib
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "numerics-and-sparse-attn_amd")
for _p in (PKG, ROOT):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import numpy as np  # noqa: E402
import torch  # noqa: E402

B, H, KVH, D = 32, 64, 8, 128
L = 163840
S, W, R = 4, 256, 128
HBM_PEAK_GBS = 8000.0
REF_KIVI_W256_US = 240.87          # A100 Triton, results/benchmark_results_quantized.csv:43
METRIC = "decode-attn µs/step + achieved HBM TB/s (% of peak), B=32 L=163840 W=256"
COLD_SET_BYTES = 1 << 30           # one pass over a path's input sets reads at least this
MAX_SETS = 512
MIN_TIMED_STEPS = 1000             # microsecond-scale paths: R * G >= this
MIN_GRAPH_STEPS = 512              # and G >= this: each replay costs ~20 us of its own
CONTEXT_LENGTHS = [8192, 16384, 32768, 65536, 131072, 163840]          # constants.py:18
WINDOW_SIZES = [0, 32, 64, 128, 256, 512, 1024, 2048, 4096, 8192, 16384]
KERNEL_SOURCES = ("attn.hip", "kvdec_device.h", "kvdec_stream.h", "quant.hip")


# --------------------------------------------------------------------------
# algorithmic byte models
# --------------------------------------------------------------------------

def bytes_q_o():
    return 2 * B * H * D * 2


def bytes_dense(n_tok):
    """Q + O + K + V: 1,048,576 + 131,072 * L (benchmark.py:30-31,57 of the reference)."""
    return bytes_q_o() + 2 * B * KVH * n_tok * D * 2


def bytes_sparse(window):
    return bytes_dense(S + window)


def bytes_kivi(window, residual=R, sink_tokens=S):
    """Minimal bytes of the fused step: Q, O, fp16 residual K/V, and the 2-bit
    codes + fp16 scale/zero of ``sink_tokens`` sink tokens and the window-old
    tokens.  sink_tokens=32 gives the reference's own accounting (padded sink
    group, benchmark.py:121-129)."""
    pairs = B * KVH
    residual = min(residual, window)          # a window below the residual stays fp16
    quant_tok = sink_tokens + (window - residual)
    k_codes = quant_tok * D // 4
    k_meta = 2 * 2 * D * (-(-sink_tokens // 32) + (window - residual) // 32)
    v_codes = quant_tok * D // 4
    v_meta = 2 * 2 * quant_tok * (D // 32)
    return bytes_q_o() + pairs * (2 * residual * D * 2 + k_codes + k_meta + v_codes + v_meta)


def bytes_stream_step(window, residual=R):
    """One decode step of the streaming KIVI cache, averaged over a group of
    32 steps: attend over sink + window-old + residual .. residual + 31 ring
    rows (residual + 15.5 on average); once per 32 steps read a 32-row block
    and write its codes and scales/zeros (K per channel, V per token).  The
    new token's K/V are written into the ring by their producer."""
    pairs = B * KVH
    attend = bytes_kivi(window, residual) + pairs * 2 * 15.5 * D * 2
    evict = pairs * (2 * 32 * D * 2 + 2 * (32 * D // 4) + 2 * 2 * D + 2 * 2 * 32 * (D // 32))
    return int(attend + evict / 32)


def bytes_paged(n_tok, page_size):
    """bytes_dense plus the block table and the per-sequence lengths."""
    return bytes_dense(n_tok) + B * (-(-n_tok // page_size)) * 4 + B * 4


def bytes_quantize(n_tok):
    """Read fp16 input, write codes and fp16 scale/zero (the same for K and V)."""
    pairs = B * KVH
    return pairs * (n_tok * D * 2 + n_tok * D // 4 + 2 * 2 * (n_tok // 32) * D)


# --------------------------------------------------------------------------
# timing
# --------------------------------------------------------------------------

CLOCK = {"lib": None}              # the timing build's ctypes handle under --kernel-clock
CLOCK_LAUNCHES_PER_STEP = 2        # log slots per captured step (attention launches it may make)
CLOCK_WGS = 1024                   # workgroup records per slot (kClockWgs in attn.hip)


def _capture(body, G):
    """Capture body() (which issues G steps) into one HIP graph; under
    --kernel-clock the timing build's log is armed for the capture, so each
    attention launch of the graph owns one slot.  Returns (graph, log)."""
    lib = CLOCK["lib"]
    log = None
    if lib is not None:
        log = torch.zeros(CLOCK_LAUNCHES_PER_STEP * G * CLOCK_WGS * 4, dtype=torch.int64, device="cuda")
        if lib.kvdec_clock_arm(log.data_ptr(), CLOCK_LAUNCHES_PER_STEP * G) != 0:
            raise RuntimeError("kvdec_clock_arm failed")
    g = torch.cuda.CUDAGraph()
    try:
        with torch.cuda.graph(g):
            out = body()
    finally:
        if lib is not None:
            lib.kvdec_clock_arm(None, 0)
    return g, log, out


def _replay_time(g, G, Rp, warmup):
    for _ in range(max(1, warmup)):
        g.replay()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(Rp):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / (Rp * G)


def _clock_stats(g, log):
    """One more replay with the log cleared: every workgroup of every
    attention launch of the graph has stored the realtime counter at its
    start and end.  Per launch: its own duration (last workgroup end - first
    workgroup start), the gap to the next launch (its first start - this
    launch's last end; negative = overlap), the dispatch ramp (last start -
    first start) and the end spread (last end - first end), in us, and the
    shader clock (MHz) of each workgroup: its core-clock ticks over its
    realtime span.  The realtime counter's rate is checked against HIP
    events around the same replay (nominally 100 MHz)."""
    log.zero_()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    g.replay()
    e1.record()
    torch.cuda.synchronize()
    raw = log.cpu().numpy().view(np.uint64).reshape(-1, CLOCK_WGS, 4).astype(np.float64)
    a, core = raw[:, :, :2], raw[:, :, 2:]
    live = a[:, :, 0] > 0                                # workgroups that ran
    keep = live.any(axis=1)
    a, core, live = a[keep], core[keep], live[keep]
    if len(a) < 2:
        return {"status": "no clocked launches recorded"}
    big = np.where(live, a[:, :, 0], np.inf)
    first = big.min(axis=1)
    last_start = np.where(live, a[:, :, 0], -np.inf).max(axis=1)
    first_end = np.where(live, a[:, :, 1], np.inf).min(axis=1)
    last_end = np.where(live, a[:, :, 1], -np.inf).max(axis=1)
    replay_us = e0.elapsed_time(e1) * 1e3
    ticks = float(last_end[-1] - first[0])
    rate = ticks / replay_us                             # ticks per us, the replay's fixed cost included
    tick_us = 1.0 / 100.0 if abs(rate / 100.0 - 1.0) < 0.05 else 1.0 / rate
    span = (last_end - first) * tick_us
    gap = (first[1:] - last_end[:-1]) * tick_us
    ramp = (last_start - first) * tick_us
    tail = (last_end - first_end) * tick_us
    # shader clock of each workgroup: core-clock ticks over its realtime span
    # (spans of at least 1 us, where the 100 MHz counter's granularity is
    # below 1%)
    rt = (a[:, :, 1] - a[:, :, 0]) * tick_us
    ok = live & (rt >= 1.0)
    sclk = ((core[:, :, 1] - core[:, :, 0])[ok] / rt[ok]) if ok.any() else np.array([np.nan])

    def st(x):
        return {"mean": round(float(np.mean(x)), 3), "median": round(float(np.median(x)), 3),
                "min": round(float(np.min(x)), 3), "max": round(float(np.max(x)), 3)}
    return {"launches": int(len(a)), "workgroups_per_launch": int(live.sum(axis=1).max()),
            "counter_ticks_per_us_measured": round(rate, 2), "tick_us": tick_us,
            "kernel_us": st(span), "gap_us": st(gap), "overlapping_launches": int((gap < 0).sum()),
            "dispatch_ramp_us": st(ramp), "end_spread_us": st(tail), "shader_clock_mhz": st(sclk),
            "first_start_to_last_end_us_per_launch": round(ticks * tick_us / len(a), 3)}


def graph_time(call, nsets, steps, warmup, min_steps=MIN_TIMED_STEPS, replays=None,
               min_graph=MIN_GRAPH_STEPS):
    """Per-step ms of back-to-back calls call(i % nsets), G = max(steps, nsets,
    min_graph) of them captured in one HIP graph (every input set once per
    pass), timed over R back-to-back replays (R * G >= min_steps unless
    `replays` is given).  A replay carries a fixed cost (~20 us measured
    between two back-to-back replays of one graph) that R * G steps share,
    so G is kept long whatever `steps` is.  Returns (ms_per_step,
    {"graph_steps": G, "replays": R}), plus "kernel_clock" under
    --kernel-clock."""
    G = max(steps, nsets, min_graph)
    Rp = replays if replays is not None else max(2, math.ceil(min_steps / G))
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for i in range(min(3, G)):
            call(i % nsets)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()

    def body():
        for i in range(G):
            call(i % nsets)
    g, log, _ = _capture(body, G)
    ms = _replay_time(g, G, Rp, warmup)
    info = {"graph_steps": G, "replays": Rp}
    if log is not None:
        info["kernel_clock"] = _clock_stats(g, log)
    del g
    return ms, info


def chain_time(step, q0, nsets, steps, warmup, min_steps=MIN_TIMED_STEPS):
    """The same timing for a dependent chain: step i attends with the query
    q_i = o_{i-1} (q_0 = q0) over input set i % nsets, so no step can start
    before the previous one has written its output, as in a decode loop
    where each layer's attention waits for the last.  After the timing the
    chain is rerun eagerly from q0 and its final output compared with the
    graph's, bit for bit.  Returns (ms_per_step, info)."""
    G = max(steps, nsets, MIN_GRAPH_STEPS)
    Rp = max(2, math.ceil(min_steps / G))
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        q = q0
        for i in range(min(3, G)):
            q = step(i % nsets, q)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()

    def body():
        q = q0
        for i in range(G):
            q = step(i % nsets, q)
        return q
    g, log, q_graph = _capture(body, G)
    ms = _replay_time(g, G, Rp, warmup)
    info = {"graph_steps": G, "replays": Rp}
    if log is not None:
        info["kernel_clock"] = _clock_stats(g, log)
    q = q0
    for i in range(G):
        q = step(i % nsets, q)
    torch.cuda.synchronize()
    info["final_output_equals_eager_chain"] = bool(torch.equal(q, q_graph))
    info["final_output_max_abs_diff_vs_eager"] = float((q.float() - q_graph.float()).abs().max())
    del g
    return ms, info


def latency_time(call, nsets, reps, flush):
    """Reference-harness latency: 1 GiB write, then events around one call."""
    for i in range(3):
        call(i % nsets)
    torch.cuda.synchronize()
    per = []
    for i in range(reps):
        flush.zero_()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        call(i % nsets)
        e1.record()
        torch.cuda.synchronize()
        per.append(e0.elapsed_time(e1))
    return float(np.mean(per)), float(np.median(per))


def path_record(ms, alg_bytes, nsets, tinfo, alg_bytes_ref=None, latency=None):
    gbs = alg_bytes / (ms * 1e-3) / 1e9
    rec = {"us_per_step": round(ms * 1e3, 3), "input_sets": nsets, **tinfo,
           "alg_bytes": int(alg_bytes), "achieved_GBs": round(gbs, 1),
           "frac_of_peak": round(gbs / HBM_PEAK_GBS, 4)}
    if alg_bytes_ref is not None:
        rec["alg_bytes_ref_accounting"] = int(alg_bytes_ref)
        rec["achieved_GBs_ref_accounting"] = round(alg_bytes_ref / (ms * 1e-3) / 1e9, 1)
    if latency is not None:
        rec["latency_us"] = round(latency[0] * 1e3, 3)
        rec["latency_median_us"] = round(latency[1] * 1e3, 3)
    return rec


def kernel_source_hash():
    """sha256 (first 16 hex) of the kernel sources, in a fixed order."""
    h = hashlib.sha256()
    for name in KERNEL_SOURCES:
        with open(os.path.join(PKG, "csrc", name), "rb") as f:
            h.update(f.read())
    return h.hexdigest()[:16]


def measured_traffic(key):
    """(HBM bytes per launch, provenance) of the path's kernel from the
    rocprofv3 FETCH_SIZE / WRITE_SIZE runs recorded in profiles/
    hbm_traffic.json; bytes are None when nothing is recorded or the record
    was measured on other kernel sources."""
    src = {"file": "profiles/hbm_traffic.json", "key": key, "current_source_sha16": kernel_source_hash()}
    try:
        with open(os.path.join(ROOT, "profiles", "hbm_traffic.json")) as f:
            rec = json.load(f).get(key)
    except (OSError, ValueError):
        rec = None
    if rec is None:
        return None, {**src, "status": "not recorded"}
    src.update(commit=rec.get("commit"), recorded_source_sha16=rec.get("source_sha16"))
    if rec.get("source_sha16") != src["current_source_sha16"]:
        return None, {**src, "status": "stale: recorded on other kernel sources"}
    return int(rec["fetch_bytes_per_launch"] + rec["write_bytes_per_launch"]), {**src, "status": "current"}


def recorded_kernel_clock(key):
    """The path's kernel-only duration recorded by the timing build
    (bench.py --kernel-clock, profiles/kernel_clock.json): the mean over a
    graph's launches of last workgroup end - first workgroup start, and the
    mean gap to the next launch; None when nothing is recorded or the record
    was measured on other kernel sources."""
    src = {"file": "profiles/kernel_clock.json", "key": key, "current_source_sha16": kernel_source_hash()}
    try:
        with open(os.path.join(ROOT, "profiles", "kernel_clock.json")) as f:
            rec = json.load(f).get("paths", {}).get(key)
    except (OSError, ValueError):
        rec = None
    if rec is None:
        return None, {**src, "status": "not recorded"}
    src.update(recorded_source_sha16=rec.get("source_sha16"))
    if rec.get("source_sha16") != src["current_source_sha16"]:
        return None, {**src, "status": "stale: recorded on other kernel sources"}
    return rec, {**src, "status": "current"}


def n_sets(bytes_per_set):
    return int(max(1, min(MAX_SETS, -(-COLD_SET_BYTES // bytes_per_set))))


# --------------------------------------------------------------------------
# CPU baseline: the torch restatement of the reference's test oracles
# --------------------------------------------------------------------------

def host_info():
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        affinity = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        affinity = None
    return {"cpu_model": model, "threads_used": torch.get_num_threads(), "os_cpu_count": os.cpu_count(),
            "affinity_cpus": affinity, "OMP_NUM_THREADS": os.environ.get("OMP_NUM_THREADS")}


def cpu_time(fn, min_reps=5, budget_s=8.0):
    """1 warm-up call, then >= min_reps timed calls (more while within
    budget_s, at most 30); returns (median seconds, reps)."""
    fn()
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < min_reps or (time.perf_counter() < t_end and len(times) < 30):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return float(np.median(times)), len(times)


def cpu_randn(*shape, seed=0):
    return torch.randn(*shape, generator=torch.Generator().manual_seed(seed))


def cpu_dense_b1(n_tok, seed=0):
    """One sequence of the dense step on the host: (median us, reps)."""
    from oracle import torch_ref as T
    q = cpu_randn(1, H, D, seed=seed)
    k = cpu_randn(1, KVH, n_tok, D, seed=seed + 1)
    v = cpu_randn(1, KVH, n_tok, D, seed=seed + 2)
    sec, reps = cpu_time(lambda: T.dense_attention(q, k, v, D**-0.5), min_reps=5, budget_s=2.0)
    return sec * 1e6, reps


def cpu_sparse(batch, window, seed=0):
    from oracle import torch_ref as T
    q = cpu_randn(batch, H, D, seed=seed)
    k = cpu_randn(batch, KVH, S + window, D, seed=seed + 1)
    v = cpu_randn(batch, KVH, S + window, D, seed=seed + 2)
    sec, reps = cpu_time(lambda: T.sparse_attention(q, k, v, L, window, S, D**-0.5), budget_s=2.0)
    return sec * 1e6, reps


def cpu_kivi(q, cache, window, budget_s=2.0):
    """The fused step's dequantize-then-attend on the host, over a cache and
    q given as GPU tensors (copied to the host first, untimed)."""
    from oracle import torch_ref as T
    qh = q.cpu()
    hc = {k: v.cpu() for k, v in cache.items()}
    sec, reps = cpu_time(lambda: T.quantized_attention(qh, max(window - R, 0), hc, D**-0.5),
                         budget_s=budget_s)
    return sec * 1e6, reps


def cpu_config1():
    """B=1, 64q/8kv, d=128, L=8192, Q/K/V ~ N(0,1) fp32
    from a fixed CPU seed; the torch restatement timed and its output
    checked against the fp64 numpy oracle."""
    from oracle import kvdec_oracle as O
    from oracle import torch_ref as T
    g = torch.Generator().manual_seed(0)
    q = torch.randn(1, H, D, generator=g)
    k = torch.randn(1, KVH, 8192, D, generator=g)
    v = torch.randn(1, KVH, 8192, D, generator=g)
    sec, reps = cpu_time(lambda: T.dense_attention(q, k, v, D**-0.5), min_reps=5, budget_s=3.0)
    out = T.dense_attention(q, k, v, D**-0.5).numpy()
    err = float(np.abs(out - O.dense_attention(q.numpy(), k.numpy(), v.numpy(), D**-0.5)).max())
    nbytes = 2 * H * D * 4 + 2 * KVH * 8192 * D * 4
    return {"config": "B=1 H=64 KVH=8 D=128 L=8192, fp32 N(0,1), torch.Generator seed 0",
            "us_per_step": round(sec * 1e6, 1), "reps": reps, "alg_bytes": nbytes,
            "achieved_GBs": round(nbytes / sec / 1e9, 2),
            "max_abs_err_vs_fp64_oracle": err, "check": "pass" if err < 1e-4 else "FAIL"}


# --------------------------------------------------------------------------

KIVI_KEYS = ("k_residual", "v_residual",
             "k_sink_packed", "k_sink_scale", "k_sink_zero",
             "v_sink_packed", "v_sink_scale", "v_sink_zero",
             "k_win_packed", "k_win_scale", "k_win_zero",
             "v_win_packed", "v_win_scale", "v_win_zero")


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--paths", default="kivi,sweep,dense,sparse,quantize,stream,paged,grid,floor")
    ap.add_argument("--sweep-windows", default="32,1024,4096",
                    help="windows of the 'sweep' path (fused KIVI decode, config 5)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-latency", action="store_true", help="skip the per-call latency runs")
    ap.add_argument("--dense-lengths", default="163840,32768",
                    help="context lengths of the 'dense' path (163840: the metric's L; 32768: config 2)")
    ap.add_argument("--chain", choices=("both", "only", "off"), default="both",
                    help="kivi and sparse paths: time the independent-input graph, the dependent chain "
                         "(q <- o of the previous step), or both")
    ap.add_argument("--kernel-clock", action="store_true",
                    help="load the timing build (libkvdec_clock.so) and add each graph's per-launch kernel "
                         "durations and launch gaps, read from the GPU realtime counter, to the paths")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="first copy 256 MiB device-to-device three times: the reference kernel "
                         "for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE counters to bytes")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: every GPU box of this build has one GPU and the "
              "build has no multi-GPU path (run with --gpus 1)", file=sys.stderr)
        sys.exit(2)

    if args.kernel_clock:
        os.environ["KVDEC_LIBRARY"] = "clock"
    import _kvdec
    import dense_kernel
    import quant_kernel
    import sparse_kernel
    if args.kernel_clock:
        CLOCK["lib"] = _kvdec.lib
    dense_lengths = [int(x) for x in args.dense_lengths.split(",") if x.strip()]

    paths = [p.strip() for p in args.paths.split(",") if p.strip()]
    K, Wu = max(1, args.steps), max(1, args.warmup)
    Kms = max(4, min(K, 20))           # graph length of the millisecond-scale paths (2 replays)
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(0)
    outliers = torch.randperm(D, generator=torch.Generator().manual_seed(0))[:4].tolist()
    flush = None if args.no_latency else torch.empty((1 << 30) // 4, dtype=torch.int32, device=dev)
    want_cpu = not args.no_cpu

    def progress(msg):
        print(f"[bench] {msg}", file=sys.stderr, flush=True)

    def randn(*shape):
        return torch.randn(*shape, generator=gen, device=dev, dtype=torch.float16)

    def compacted(window):
        kc = randn(B, KVH, S + window, D)
        kc[..., outliers] *= 10
        return kc, randn(B, KVH, S + window, D)

    out = {}
    cpu = {"host": host_info()} if want_cpu else None
    head_cpu = None

    if args.copy_calibration:
        src = torch.ones((256 << 20) // 4, dtype=torch.int32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    def kivi_sets(window):
        ns = n_sets(bytes_kivi(window))
        sets = []
        for _ in range(ns):
            kc, vc = compacted(window)
            cache = quant_kernel.build_quantized_kv_cache(kc, vc)
            del kc, vc
            sets.append((randn(B, H, D), [cache[k] for k in KIVI_KEYS]))
        return ns, sets

    def kivi_call(sets, window):
        def call(i):
            q, a = sets[i]
            return quant_kernel.sparse_decode_attention_quantized(q, *a, seq_len=L, window=window)
        return call

    def kivi_path(window, name, latency=True, chain=False):
        ns, sets = kivi_sets(window)
        call = kivi_call(sets, window)
        if not (chain and args.chain == "only"):
            ms, ti = graph_time(call, ns, K, Wu)
            lat = None if (flush is None or not latency) else latency_time(call, ns, 50, flush)
            out[name] = path_record(ms, bytes_kivi(window), ns, ti, bytes_kivi(window, sink_tokens=32), lat)
            progress(f"{name}: {out[name]['us_per_step']} us")
        if chain and args.chain != "off":
            def step(i, q):
                return quant_kernel.sparse_decode_attention_quantized(q, *sets[i][1], seq_len=L, window=window)
            ms, ti = chain_time(step, sets[0][0], ns, K, Wu)
            out[name + "_chain"] = path_record(ms, bytes_kivi(window), ns, ti, bytes_kivi(window, sink_tokens=32))
            progress(f"{name}_chain: {out[name + '_chain']['us_per_step']} us")
        return sets

    if "kivi" in paths:
        sets = kivi_path(W, "kivi_w256", chain=True)
        if want_cpu and "kivi_w256" in out:
            q0, parts = sets[0]
            us, reps = cpu_kivi(q0, dict(zip(KIVI_KEYS, parts)), W, budget_s=8.0)
            head_cpu = {"value": round(us, 1), "unit": "us/step", "cores": cpu["host"]["threads_used"],
                        "kind": "port",
                        "sample": f"the whole kivi_w256 step (B=32, all 256 KV heads): oracle/torch_ref.py "
                                  f"dequantize-then-attend in float32 (restates test_quantized_attention_"
                                  f"correctness.py:32-61), median of {reps} reps after 1 warm-up, "
                                  f"{cpu['host']['threads_used']} torch threads on {cpu['host']['cpu_model']}"}
            out["kivi_w256"]["cpu_us_per_step"] = round(us, 1)
        del sets

    if "sweep" in paths:
        for w in [int(x) for x in args.sweep_windows.split(",") if x.strip()]:
            sets = kivi_path(w, f"kivi_w{w}")
            if want_cpu:
                q0, parts = sets[0]
                us, _ = cpu_kivi(q0, dict(zip(KIVI_KEYS, parts)), w)
                out[f"kivi_w{w}"]["cpu_us_per_step"] = round(us, 1)
            del sets

    if "stream" in paths:
        # decode loop over the streaming KIVI cache (kivi_stream.py): each
        # step reserves the next token's ring row (quantizing a block into
        # the window-old ring every 32 steps) and attends; steps rotate over
        # independent caches so that every step starts cold, and each cache
        # advances 32 tokens per pass of the graph
        from kivi_stream import KiviStreamBatch, KiviStreamCache
        ns = n_sets(bytes_stream_step(W))
        caches, toks = [], []
        for _ in range(ns):
            kc, vc = compacted(W)
            caches.append(KiviStreamCache.from_prefill(kc, vc, W))
            del kc, vc
            toks.append(randn(B, H, D))
        ssteps = 32 * ns

        def scall(i):
            # the token's K/V are written into the reserved ring row by their
            # producer (the projection), which is not part of this step
            c = caches[i % ns]
            c.reserve()
            return c.attend(toks[i % ns])

        ms, ti = graph_time(scall, ns, ssteps, Wu)
        out["kivi_stream_w256"] = path_record(ms, bytes_stream_step(W), ns, ti)
        del caches

        # the same loop with one ring state per sequence: per step one launch
        # that writes each sequence's token row, quantizes the blocks due for
        # eviction, keeps the on-GPU bookkeeping and attends
        batches, new_kv = [], []
        for _ in range(ns):
            kc, vc = compacted(W)
            batches.append(KiviStreamBatch.from_prefill(kc, vc, W))
            del kc, vc
            new_kv.append((randn(B, KVH, D), randn(B, KVH, D)))

        def bcall(i):
            kn, vn = new_kv[i % ns]
            return batches[i % ns].step_attend(toks[i % ns], kn, vn)

        ms, ti = graph_time(bcall, ns, ssteps, Wu)
        out["kivi_stream_seqs_w256"] = path_record(ms, bytes_stream_step(W), ns, ti)
        progress("stream done")
        del batches, toks, new_kv

    if "sparse" in paths:
        ns = n_sets(bytes_sparse(W))
        sets = [(randn(B, H, D),) + compacted(W) for _ in range(ns)]

        def call(i):
            q, kc, vc = sets[i]
            return sparse_kernel.sparse_decode_attention(q, kc, vc, seq_len=L, window=W)

        if args.chain != "only":
            ms, ti = graph_time(call, ns, K, Wu)
            lat = None if flush is None else latency_time(call, ns, 50, flush)
            out["sparse_fp16_w256"] = path_record(ms, bytes_sparse(W), ns, ti, latency=lat)

        def sstep(i, q):
            return sparse_kernel.sparse_decode_attention(q, sets[i][1], sets[i][2], seq_len=L, window=W)
        if args.chain != "off":
            ms, ti = chain_time(sstep, sets[0][0], ns, K, Wu)
            out["sparse_fp16_w256_chain"] = path_record(ms, bytes_sparse(W), ns, ti)
        if want_cpu and "sparse_fp16_w256" in out:
            us, reps = cpu_sparse(B, W)
            out["sparse_fp16_w256"]["cpu_us_per_step"] = round(us, 1)
        progress("sparse done: " + ", ".join(f"{k} {v['us_per_step']} us" for k, v in out.items()
                                             if k.startswith("sparse")))
        del sets

    ms_warm = max(2, min(Wu, 3))
    if "quantize" in paths or ("dense" in paths and dense_lengths) or "paged" in paths:
        full = "quantize" in paths or "paged" in paths or ("dense" in paths and L in dense_lengths)
        k = randn(B, KVH, L, D) if full else None
        if full:
            k[..., outliers] *= 10
        v = randn(B, KVH, L, D) if full else None
        q = randn(B, H, D)
        if "quantize" in paths:
            ms, ti = graph_time(lambda i: quant_kernel.quantize_k_cache(k), 1, Kms, ms_warm, replays=2, min_graph=1)
            out["quantize_k_L163840"] = path_record(ms, bytes_quantize(L), 1, ti)
            ms, ti = graph_time(lambda i: quant_kernel.quantize_v_cache(v), 1, Kms, ms_warm, replays=2, min_graph=1)
            out["quantize_v_L163840"] = path_record(ms, bytes_quantize(L), 1, ti)
            progress("quantize done")
        if "dense" in paths and L in dense_lengths:
            ms, ti = graph_time(lambda i: dense_kernel.dense_decode_attention(q, k, v, seq_len=L), 1,
                                Kms, ms_warm, replays=2, min_graph=1)
            out["dense_L163840"] = path_record(ms, bytes_dense(L), 1, ti)
            if want_cpu:
                us, reps = cpu_dense_b1(L)
                out["dense_L163840"]["cpu_b1_us_per_step"] = round(us, 1)
                out["dense_L163840"]["cpu_b32_us_per_step_extrapolated"] = round(us * B, 1)
                out["dense_L163840"]["cpu_note"] = (f"measured on one sequence (B=1, {reps} reps); the B=32 "
                                                    "figure is that x32, extrapolated, not measured")
            progress(f"dense_L163840: {out['dense_L163840']['us_per_step']} us")
        if "paged" in paths:
            # the same cache scattered over 16-token pages ([pages, 16, KVH,
            # D], vLLM's layout) in a random order, every sequence at full
            # length through per-sequence lengths
            import paged_kernel
            ps = 16
            nb = L // ps
            table = torch.randperm(B * nb, generator=torch.Generator().manual_seed(1)).to(dev)
            table = table.view(B, nb).to(torch.int32)
            idx = table.view(-1).long()
            kp = torch.empty(B * nb, ps, KVH, D, dtype=torch.float16, device=dev)
            kp[idx] = k.view(B, KVH, nb, ps, D).permute(0, 2, 3, 1, 4).reshape(-1, ps, KVH, D)
            vp = torch.empty_like(kp)
            vp[idx] = v.view(B, KVH, nb, ps, D).permute(0, 2, 3, 1, 4).reshape(-1, ps, KVH, D)
            lens = torch.full((B,), L, dtype=torch.int32, device=dev)
            ms, ti = graph_time(lambda i: paged_kernel.paged_decode_attention(
                q, kp, vp, table, lens, max_seq_len=L, kv_layout="NHD"), 1, Kms, ms_warm, replays=2, min_graph=1)
            out["paged_nhd16_L163840"] = path_record(ms, bytes_paged(L, ps), 1, ti)
            del kp, vp, table, idx, lens
        del k, v
        if "dense" in paths and 32768 in dense_lengths:
            # config 2: L = 32768 (a prefix view of the same cache would not be
            # contiguous, so the cache is regenerated at that length)
            Ls = 32768
            ns = n_sets(bytes_dense(Ls))
            dsets = [(randn(B, H, D), randn(B, KVH, Ls, D), randn(B, KVH, Ls, D)) for _ in range(ns)]

            def dcall(i):
                qq, kk, vv = dsets[i]
                return dense_kernel.dense_decode_attention(qq, kk, vv, seq_len=Ls)

            ms, ti = graph_time(dcall, ns, Kms, ms_warm, replays=2, min_graph=1)
            out["dense_L32768"] = path_record(ms, bytes_dense(Ls), ns, ti)
            del dsets
        torch.cuda.empty_cache()

    grid = None
    if "grid" in paths:
        grid = {"note": "dense per L; sparse and fused KIVI per W at L=163840 (steady state: the same "
                        "bytes at every L >= S + W); cpu_b1_us = the same step for one sequence "
                        "(B=1) on the host, float32 torch restatement",
                "dense": {}, "sparse": {}, "kivi": {}}
        for Lg in CONTEXT_LENGTHS:
            qq, kk, vv = randn(B, H, D), randn(B, KVH, Lg, D), randn(B, KVH, Lg, D)
            ms, ti = graph_time(lambda i: dense_kernel.dense_decode_attention(qq, kk, vv, seq_len=Lg), 1,
                                Kms, ms_warm, replays=2, min_graph=1)
            rec = path_record(ms, bytes_dense(Lg), 1, ti)
            if want_cpu:
                rec["cpu_b1_us"] = round(cpu_dense_b1(Lg)[0], 1)
            grid["dense"][str(Lg)] = rec
            del qq, kk, vv
            torch.cuda.empty_cache()
        progress("grid dense done")
        for wg in WINDOW_SIZES:
            ns = n_sets(bytes_sparse(wg))
            sets = [(randn(B, H, D),) + compacted(wg) for _ in range(ns)]

            def call(i, sets=sets, wg=wg):
                q, kc, vc = sets[i]
                return sparse_kernel.sparse_decode_attention(q, kc, vc, seq_len=L, window=wg)

            ms, ti = graph_time(call, ns, K, Wu)
            rec = path_record(ms, bytes_sparse(wg), ns, ti)
            if want_cpu:
                rec["cpu_b1_us"] = round(cpu_sparse(1, wg)[0], 1)
            grid["sparse"][str(wg)] = rec
            del sets
        progress("grid sparse done")
        for wg in [32] + [w for w in WINDOW_SIZES if w >= R]:
            ns, sets = kivi_sets(wg)
            ms, ti = graph_time(kivi_call(sets, wg), ns, K, Wu)
            rec = path_record(ms, bytes_kivi(wg), ns, ti, bytes_kivi(wg, sink_tokens=32))
            if want_cpu:
                q0, parts = sets[0]
                cache = {k_: t[:1] for k_, t in zip(KIVI_KEYS, parts)}
                rec["cpu_b1_us"] = round(cpu_kivi(q0[:1], cache, wg, budget_s=1.0)[0], 1)
            grid["kivi"][str(wg)] = rec
            del sets
            torch.cuda.empty_cache()
        progress("grid kivi done")

    floor = None
    if "floor" in paths:
        # what the box itself allows a decode step of each path: empty
        # launches shaped like the decode kernels, and plain streaming reads
        # of the path's algorithmic bytes (kvdec_read_probe_sweep), timed
        # like the paths.  The headline's bytes get the whole sweep (grid x
        # block size x load form); the other paths the sweep's best forms.
        import _kvdec as KV
        sink = torch.zeros(65536, dtype=torch.int32, device=dev)
        kinds = ("global_nt", "global", "buffer_nt", "buffer")

        def cfg_name(blocks, threads, mode):
            return f"{blocks}x{threads}/{kinds[mode & 3]}/{'upfront16' if mode & 4 else 'inflight4'}"

        def probe_sets(nbytes):
            nb = (nbytes + 15) // 16 * 16
            ns = n_sets(nb) if nb else 1
            return nb, [torch.empty(max(nb, 16) // 4, dtype=torch.int32, device=dev) for _ in range(ns)]

        def probe_us(nb, bufs, blocks, threads, mode, lds=0):
            def pcall(i):
                KV.check(KV.lib.kvdec_read_probe_sweep(KV.ptr(bufs[i]), nb, KV.ptr(sink), blocks, threads,
                                                       mode, lds, KV.stream_of(sink)), "read_probe_sweep")
            big = nb > (1 << 30)
            ms, _ = (graph_time(pcall, len(bufs), Kms, ms_warm, replays=2, min_graph=1) if big
                     else graph_time(pcall, len(bufs), K, Wu))
            return round(ms * 1e3, 3)

        nb0, b0 = probe_sets(0)
        floor = {"note": "per-step floors on this box, in the paths' graph timing: launch_us = an empty launch "
                         "of 256 workgroups x 512 threads; launch_us_kivi_lean / _kivi_wide = the same grid "
                         "with the lean (512 threads, 71184 B LDS) and wide (1024 threads, 150272 B LDS) KIVI "
                         "kernels' block and LDS sizes; read_floor_us per path = the fastest plain streaming "
                         "read of the path's algorithmic bytes found by kvdec_read_probe_sweep (the best probe "
                         "form, not a proven bound: a kernel can beat it); frac_of_read_floor = read_floor_us / "
                         "us_per_step",
                 "launch_us": probe_us(nb0, b0, 256, 512, 0),
                 "launch_us_kivi_lean": probe_us(nb0, b0, 256, 512, 0, 71184),
                 "launch_us_kivi_wide": probe_us(nb0, b0, 256, 1024, 0, 150272)}
        del b0
        best_cfgs = [(512, 512, 0), (1024, 512, 0)]
        head_bytes = (out.get("kivi_w256") or out.get("kivi_w256_chain") or {}).get("alg_bytes")
        if head_bytes:
            nb, bufs = probe_sets(head_bytes)
            res = {}
            for blocks in (256, 512, 1024, 2048):
                for threads in (256, 512, 1024):
                    for mode in range(8):
                        res[(blocks, threads, mode)] = probe_us(nb, bufs, blocks, threads, mode)
            del bufs
            order = sorted(res, key=res.get)
            floor["sweep_kivi_w256"] = {"bytes": nb, "best": cfg_name(*order[0]), "best_us": res[order[0]],
                                        "us": {cfg_name(*c): res[c] for c in order}}
            best_cfgs = list(dict.fromkeys(order[:4] + best_cfgs))
            progress(f"floor sweep: best {cfg_name(*order[0])} {res[order[0]]} us")
        probed = {}
        for name, rec in list(out.items()):
            if rec.get("alg_bytes") in probed:
                rec.update(probed[rec["alg_bytes"]])
                rec["frac_of_read_floor"] = round(rec["read_floor_us"] / rec["us_per_step"], 4)
            elif rec.get("alg_bytes"):
                nb, bufs = probe_sets(rec["alg_bytes"])
                tried = {c: probe_us(nb, bufs, *c) for c in best_cfgs
                         if (c[2] & 3) < 2 or -(-nb // c[0]) < (1 << 31)}
                del bufs
                c = min(tried, key=tried.get)
                rec["read_floor_us"] = tried[c]
                rec["read_floor_config"] = cfg_name(*c)
                rec["frac_of_read_floor"] = round(rec["read_floor_us"] / rec["us_per_step"], 4)
                probed[rec["alg_bytes"]] = {"read_floor_us": tried[c], "read_floor_config": cfg_name(*c)}
        torch.cuda.empty_cache()
        progress("floors done")

    if want_cpu:
        cpu["config1_dense_L8192_b1"] = cpu_config1()

    head_key = "kivi_w256" if "kivi_w256" in out else next(iter(out))
    head = out[head_key]
    value = head["us_per_step"]
    traffic, traffic_src = measured_traffic(head_key)
    line = {
        "metric": METRIC,
        "value": value,
        "unit": "us/step",
        "n_gpus": 1,
        "steps": K,
        "warmup": Wu,
        "ms_per_step": round(value / 1e3, 6),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": round(value / REF_KIVI_W256_US, 5) if head_key == "kivi_w256" else None,
        "dtype": "f16",
        "data": "synthetic",
        "config": {"workload": f"{head_key}: B=32 H=64 KVH=8 D=128 L=163840 S=4 W=256 R=128, "
                               "fp16 N(0,1), 4 K channels x10",
                   "timing": f"HIP graph of max(K, input sets) back-to-back steps over rotating cold "
                             f"input sets, R back-to-back replays between two events, time / (R * "
                             f"graph steps); this path: graph_steps={head['graph_steps']}, "
                             f"replays={head['replays']}"},
        "roofline": {"bound": "hbm", "achieved": head["achieved_GBs"], "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": head["frac_of_peak"], "traffic": traffic,
                     "traffic_source": traffic_src},
        "cpu_baseline": head_cpu,
        "paths": out,
    }
    clk, clk_src = recorded_kernel_clock(head_key)
    line["roofline"]["kernel_only"] = (
        {"note": "achieved and frac over the kernel's own duration (first workgroup start to last "
                 "workgroup end, timing build, no profiler), without the gap between launches that "
                 "value includes", "kernel_us": clk["kernel_us_mean"],
         "launch_gap_us": clk["gap_us_mean"],
         "achieved": round(head["alg_bytes"] / (clk["kernel_us_mean"] * 1e-6) / 1e9, 1),
         "frac": round(head["alg_bytes"] / (clk["kernel_us_mean"] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
         "source": clk_src} if clk else {"source": clk_src})
    if floor is not None:
        line["floor"] = floor
    if grid is not None:
        line["grid"] = grid
    if cpu is not None:
        line["cpu"] = cpu
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
