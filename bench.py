"""Decode-attention benchmark on one MI355X: prints ONE JSON line.

    python bench.py [--gpus 1] [--steps K] [--warmup W]
                    [--paths kivi,dense,sparse,quantize,sweep,stream,paged]
                    [--no-cpu] [--no-latency]

Workload (the headline metric's configuration): B=32, 64 query / 8 KV heads,
head_dim 128, logical context L=163840, sink S=4, window W=256, KIVI residual
R=128, fp16 inputs ~ N(0,1) from a fixed seed with 4 of the 128 K channels
scaled x10.  A "step" is one decode call of a path over the whole batch:

  kivi      fused sink+window(W=256)+KIVI-2bit decode (the headline ``value``)
  dense     dense GQA decode over all 163840 tokens (and L=32768, config 2)
  sparse    fp16 sink+window(W=256) decode (config 3)
  quantize  KIVI quantization of the [32, 8, 163840, 128] K and V caches (config 4)
  sweep     the fused decode at W = 32, 1024 and 4096 (config 5; W=32 < R,
            which the reference leaves undefined, keeps the window fp16)
  stream    a decode loop on the streaming KIVI cache (kivi_stream.py, W=256):
            reserve the next token's ring row (quantizing a block every 32
            steps), then attend; each cache advances 32 steps, so the time
            includes one eviction per 32 steps.  Also the same loop with one
            ring state per sequence (KiviStreamBatch.step_attend: the
            token's row write, evictions, bookkeeping and decode in one
            launch)
  paged     the dense L=163840 cache scattered over 16-token pages in a
            random order (vLLM's [pages, 16, KVH, D] layout), decoded through
            block tables and per-sequence lengths (paged_kernel.py)

Timing.  Each path keeps several independent input sets resident in HBM
(together >= 1 GiB, more than L2 plus the 256 MB Infinity Cache) and captures
K back-to-back calls that cycle through them in one HIP graph; the graph is
replayed W times untimed, then once between two HIP events on the capture
stream.  ``ms_per_step`` / ``value`` = that time / K: the steady-state cost
of a decode step whose inputs are cold in every cache, with launches
pipelined as in a decode loop.  A replay also carries a fixed cost of about
30 us (the graph's submission) that K amortises: the default K = 400 puts it
near 0.1 us per microsecond-scale step (at K = 50 it would add 0.6 us).  The
millisecond-scale paths time K/5 (dense, paged), K/10 (quantize) and K/2
(dense L=32768) steps.  ``latency_us`` is the reference harness's
method (triton do_bench): a 1 GiB buffer write before each single call,
events around the call; it adds the per-call dispatch latency (about 5 us
on this system for an empty kernel).

The CPU baseline times the numpy oracle (the repository's own restatement of
the reference's PyTorch formulas) on the host on a bounded sample of the same
workload.
"""

from __future__ import annotations

import argparse
import json
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
COLD_SET_BYTES = 1 << 30           # rotating input sets per path: at least this many bytes
MAX_SETS = 64


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
    append = 0
    attend = bytes_kivi(window, residual) + pairs * 2 * 15.5 * D * 2
    evict = pairs * (2 * 32 * D * 2 + 2 * (32 * D // 4) + 2 * 2 * D + 2 * 2 * 32 * (D // 32))
    return int(append + attend + evict / 32)


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

def graph_time(call, nsets, steps, warmup):
    """Per-step ms of `steps` back-to-back calls call(i % nsets), captured in
    one HIP graph and replayed; returns (ms_per_step, outputs of the capture)."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for i in range(min(3, steps)):
            call(i % nsets)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    outs = []
    with torch.cuda.graph(g):
        for i in range(steps):
            outs.append(call(i % nsets))
    for _ in range(max(1, warmup)):
        g.replay()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps, outs


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


def path_record(ms, alg_bytes, nsets, steps, alg_bytes_ref=None, latency=None):
    gbs = alg_bytes / (ms * 1e-3) / 1e9
    rec = {"us_per_step": round(ms * 1e3, 3), "steps": steps, "input_sets": nsets,
           "alg_bytes": int(alg_bytes), "achieved_GBs": round(gbs, 1),
           "frac_of_peak": round(gbs / HBM_PEAK_GBS, 4)}
    if alg_bytes_ref is not None:
        rec["alg_bytes_ref_accounting"] = int(alg_bytes_ref)
        rec["achieved_GBs_ref_accounting"] = round(alg_bytes_ref / (ms * 1e-3) / 1e9, 1)
    if latency is not None:
        rec["latency_us"] = round(latency[0] * 1e3, 3)
        rec["latency_median_us"] = round(latency[1] * 1e3, 3)
    return rec


def measured_traffic(key):
    """HBM bytes per launch of the path's kernel, as recorded from the
    rocprofv3 FETCH_SIZE / WRITE_SIZE runs in profiles/hbm_traffic.json
    (calibrated against a 256 MiB copy); None when not recorded."""
    try:
        with open(os.path.join(ROOT, "profiles", "hbm_traffic.json")) as f:
            rec = json.load(f).get(key)
        return None if rec is None else int(rec["fetch_bytes_per_launch"] + rec["write_bytes_per_launch"])
    except (OSError, ValueError, KeyError):
        return None


def n_sets(bytes_per_set):
    return int(max(1, min(MAX_SETS, -(-COLD_SET_BYTES // bytes_per_set))))


# --------------------------------------------------------------------------
# CPU baseline (numpy oracle on the host)
# --------------------------------------------------------------------------

def _blas_threads():
    try:
        from threadpoolctl import threadpool_info
        n = [i.get("num_threads", 1) for i in threadpool_info() if i.get("user_api") == "blas"]
        return int(max(n)) if n else 1
    except Exception:
        return 1


def _timed(fn, min_reps=3, budget_s=10.0):
    fn()                                   # warm-up
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < min_reps or time.perf_counter() < t_end:
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
        if len(times) >= 50:
            break
    return float(np.median(times)), len(times)


def cpu_baseline_kivi(q, cache):
    from oracle import kvdec_oracle as O
    qh = q.cpu().numpy()
    hc = {k: v.cpu().numpy() for k, v in cache.items()}
    sec, reps = _timed(lambda: O.quantized_attention(qh, W - R, hc, D**-0.5, dtype=np.float32))
    return sec * 1e6, reps


def cpu_baseline_dense(q, k, v, rows=1):
    from oracle import kvdec_oracle as O
    qh = q[:rows].cpu().numpy()
    kh = k[:rows].cpu().numpy()
    vh = v[:rows].cpu().numpy()
    sec, reps = _timed(lambda: O.dense_attention(qh, kh, vh, D**-0.5, dtype=np.float32),
                       min_reps=2, budget_s=6.0)
    return sec * 1e6 * (B / rows), reps


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
    ap.add_argument("--paths", default="kivi,dense,sparse,quantize,sweep,stream,paged")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-latency", action="store_true", help="skip the per-call latency runs")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="first copy 256 MiB device-to-device three times: the reference kernel "
                         "for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE counters to bytes")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(run with --gpus 1)", file=sys.stderr)
        sys.exit(2)

    import dense_kernel
    import quant_kernel
    import sparse_kernel

    paths = [p.strip() for p in args.paths.split(",") if p.strip()]
    K, Wu = max(1, args.steps), max(1, args.warmup)
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(0)
    outliers = torch.randperm(D, generator=torch.Generator().manual_seed(0))[:4].tolist()
    flush = None if args.no_latency else torch.empty((1 << 30) // 4, dtype=torch.int32, device=dev)

    def randn(*shape):
        return torch.randn(*shape, generator=gen, device=dev, dtype=torch.float16)

    def compacted(window):
        kc = randn(B, KVH, S + window, D)
        kc[..., outliers] *= 10
        return kc, randn(B, KVH, S + window, D)

    out = {}
    cpu = None

    if args.copy_calibration:
        src = torch.ones((256 << 20) // 4, dtype=torch.int32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    def kivi_path(window, steps, name, with_cpu=False):
        nonlocal cpu
        ns = n_sets(bytes_kivi(window))
        sets = []
        for _ in range(ns):
            kc, vc = compacted(window)
            cache = quant_kernel.build_quantized_kv_cache(kc, vc)
            del kc, vc
            sets.append((randn(B, H, D), [cache[k] for k in KIVI_KEYS], cache))

        def call(i):
            q, a, _ = sets[i]
            return quant_kernel.sparse_decode_attention_quantized(q, *a, seq_len=L, window=window)

        ms, _ = graph_time(call, ns, steps, Wu)
        lat = None if flush is None else latency_time(call, ns, 50, flush)
        out[name] = path_record(ms, bytes_kivi(window), ns, steps, bytes_kivi(window, sink_tokens=32), lat)
        if with_cpu and not args.no_cpu:
            us, reps = cpu_baseline_kivi(sets[0][0], sets[0][2])
            cpu = {"value": round(us, 1), "unit": "us/step", "cores": _blas_threads(), "kind": "port",
                   "sample": f"the full kivi_w256 step (B=32, all 256 KV heads), numpy oracle "
                             f"dequantize-then-attend in float32, median of {reps} reps"}
        del sets

    if "kivi" in paths:
        kivi_path(W, K, "kivi_w256", with_cpu=True)

    if "sweep" in paths:
        for w in (32, 1024, 4096):
            kivi_path(w, K, f"kivi_w{w}")

    if "stream" in paths:
        # decode loop over the streaming KIVI cache (kivi_stream.py): each
        # step reserves the next token's ring row (quantizing a block into
        # the window-old ring every 32 steps) and attends; steps rotate over
        # independent caches so that every step starts cold, and each cache
        # advances 32 tokens
        from kivi_stream import KiviStreamCache
        ns = n_sets(bytes_stream_step(W))
        caches, toks = [], []
        for _ in range(ns):
            kc, vc = compacted(W)
            caches.append(KiviStreamCache.from_prefill(kc, vc, W))
            del kc, vc
            toks.append((randn(B, H, D),))
        ssteps = 32 * ns

        def scall(i):
            # the token's K/V are written into the reserved ring row by their
            # producer (the projection), which is not part of this step
            c = caches[i % ns]
            c.reserve()
            return c.attend(toks[i % ns][0])

        ms, _ = graph_time(scall, ns, ssteps, Wu)
        out["kivi_stream_w256"] = path_record(ms, bytes_stream_step(W), ns, ssteps)
        del caches

        # the same loop with one ring state per sequence (kivi_stream.
        # KiviStreamBatch.step_attend): per step one launch that writes each
        # sequence's token row, quantizes the blocks due for eviction, keeps
        # the on-GPU bookkeeping and attends, every sequence active
        from kivi_stream import KiviStreamBatch
        batches, new_kv = [], []
        for _ in range(ns):
            kc, vc = compacted(W)
            batches.append(KiviStreamBatch.from_prefill(kc, vc, W))
            del kc, vc
            new_kv.append((randn(B, KVH, D), randn(B, KVH, D)))

        def bcall(i):
            kn, vn = new_kv[i % ns]
            return batches[i % ns].step_attend(toks[i % ns][0], kn, vn)

        ms, _ = graph_time(bcall, ns, ssteps, Wu)
        out["kivi_stream_seqs_w256"] = path_record(ms, bytes_stream_step(W), ns, ssteps)
        del batches, toks, new_kv

    if "sparse" in paths:
        ns = n_sets(bytes_sparse(W))
        sets = [(randn(B, H, D),) + compacted(W) for _ in range(ns)]

        def call(i):
            q, kc, vc = sets[i]
            return sparse_kernel.sparse_decode_attention(q, kc, vc, seq_len=L, window=W)

        ms, _ = graph_time(call, ns, K, Wu)
        lat = None if flush is None else latency_time(call, ns, 50, flush)
        out["sparse_fp16_w256"] = path_record(ms, bytes_sparse(W), ns, K, latency=lat)
        del sets

    if "quantize" in paths or "dense" in paths or "paged" in paths:
        k = randn(B, KVH, L, D)
        k[..., outliers] *= 10
        v = randn(B, KVH, L, D)
        q = randn(B, H, D)
        dsteps = max(3, K // 5)
        if "quantize" in paths:
            qsteps = max(3, K // 10)
            ms, _ = graph_time(lambda i: quant_kernel.quantize_k_cache(k), 1, qsteps, 1)
            out["quantize_k_L163840"] = path_record(ms, bytes_quantize(L), 1, qsteps)
            ms, _ = graph_time(lambda i: quant_kernel.quantize_v_cache(v), 1, qsteps, 1)
            out["quantize_v_L163840"] = path_record(ms, bytes_quantize(L), 1, qsteps)
        if "dense" in paths:
            ms, _ = graph_time(lambda i: dense_kernel.dense_decode_attention(q, k, v, seq_len=L), 1,
                               dsteps, 1)
            out["dense_L163840"] = path_record(ms, bytes_dense(L), 1, dsteps)
            if not args.no_cpu:
                us, reps = cpu_baseline_dense(q, k, v)
                out["dense_L163840"]["cpu_baseline"] = {
                    "value": round(us, 1), "unit": "us/step", "cores": _blas_threads(), "kind": "port",
                    "sample": f"batch row 0 of 32 at L=163840 (numpy oracle, float32, median of "
                              f"{reps} reps), scaled x32"}
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
            ms, _ = graph_time(lambda i: paged_kernel.paged_decode_attention(
                q, kp, vp, table, lens, max_seq_len=L, kv_layout="NHD"), 1, dsteps, 1)
            out["paged_nhd16_L163840"] = path_record(ms, bytes_paged(L, ps), 1, dsteps)
            del kp, vp, table, idx, lens
        del k, v
        if "dense" in paths:
            # config 2: L = 32768 (a prefix view of the same cache would not be
            # contiguous, so the cache is regenerated at that length)
            Ls = 32768
            ns = n_sets(bytes_dense(Ls))
            dsets = [(randn(B, H, D), randn(B, KVH, Ls, D), randn(B, KVH, Ls, D)) for _ in range(ns)]

            def dcall(i):
                qq, kk, vv = dsets[i]
                return dense_kernel.dense_decode_attention(qq, kk, vv, seq_len=Ls)

            ms, _ = graph_time(dcall, ns, max(3, K // 2), 1)
            out["dense_L32768"] = path_record(ms, bytes_dense(Ls), ns, max(3, K // 2))
            del dsets

    head_key = "kivi_w256" if "kivi_w256" in out else next(iter(out))
    head = out[head_key]
    value = head["us_per_step"]
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
                   "timing": "HIP-graph replay of back-to-back steps over rotating cold input sets"},
        "roofline": {"bound": "hbm", "achieved": head["achieved_GBs"], "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": head["frac_of_peak"], "traffic": measured_traffic(head_key)},
        "cpu_baseline": cpu,
        "paths": out,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
