"""Fused sink + window + KIVI-2bit decode on the GPU vs the CPU oracle
(restates the reference's test_quantized_attention_correctness.py, adds W=R,
the split-K windows, ramp-up and the cache builder's bit-exact codes)."""

import numpy as np
import pytest
import torch

from conftest import load_golden
from helpers import ATTN_TOL, REF_TOL, SCALE, assert_nearly_rounded, dev, host, max_abs, randn, say
from oracle import kvdec_oracle as O

pytestmark = pytest.mark.gpu

S, R = 4, 128


def _attend(q, cache, L, W, device=None, sink=S):
    from quant_kernel import sparse_decode_attention_quantized
    c = cache
    o = sparse_decode_attention_quantized(
        q, c["k_residual"], c["v_residual"],
        c["k_sink_packed"], c["k_sink_scale"], c["k_sink_zero"],
        c["v_sink_packed"], c["v_sink_scale"], c["v_sink_zero"],
        c["k_win_packed"], c["k_win_scale"], c["k_win_zero"],
        c["v_win_packed"], c["v_win_scale"], c["v_win_zero"],
        seq_len=L, window=W, sink=sink)
    torch.cuda.synchronize()
    return host(o)


def _host_cache(cache):
    return {k: host(v) for k, v in cache.items()}


def test_kivi_golden(device):
    g = load_golden("kivi_golden.npz")
    W = int(g["window"])
    from quant_kernel import build_quantized_kv_cache
    say("kivi golden build")
    cache = build_quantized_kv_cache(dev(g["k_compacted"], device), dev(g["v_compacted"], device))
    hc = _host_cache(cache)
    for key in O.CACHE_KEYS:
        np.testing.assert_array_equal(hc[key], g["cache_" + key], err_msg=key)
    q = dev(g["q"], device)
    say("kivi golden attend")
    assert max_abs(_attend(q, cache, S + W + 1000, W), g["o_steady"]) < ATTN_TOL
    assert max_abs(_attend(q, cache, 150, W), g["o_ramp"]) < ATTN_TOL


@pytest.mark.parametrize("W", [160, 192, 224, 288, 320, 384, 448, 480])
def test_quantized_attention_work_splits(W, device):
    """Every static work split of the 8 waves: 1..3 window groups (the
    quantized waves take them all), 5 (one leftover tile: a residual wave
    steps the sink and hands its fp16 tile over), 6 (two leftovers, two
    hand-overs), 7 (three leftovers, no hand-over), 8..11 (every residual
    wave takes a leftover, the quantized waves a second tile); W=512 and up
    run the dynamic queue (above).  B=8 keeps the oracle fast."""
    from quant_kernel import build_quantized_kv_cache
    B, H, KVH, D = 8, 64, 8, 128
    L = S + W + 77
    gen = torch.Generator(device=device).manual_seed(1000 + W)
    q = torch.randn(B, H, D, generator=gen, device=device, dtype=torch.float16)
    kc = torch.randn(B, KVH, S + W, D, generator=gen, device=device, dtype=torch.float16)
    vc = torch.randn(B, KVH, S + W, D, generator=gen, device=device, dtype=torch.float16)
    say(f"kivi work split W={W}")
    cache = build_quantized_kv_cache(kc, vc)
    o = _attend(q, cache, L, W)
    hc = _host_cache(cache)
    ref = O.quantized_attention(host(q), W - R, hc, SCALE)
    assert max_abs(o, ref) < ATTN_TOL
    assert_nearly_rounded(o, ref)


@pytest.mark.parametrize("W", [128, 256, 512, 1024, 4096, 8192])
def test_quantized_attention_steady_state(W, device):
    """Reference case (seed 3 analogue, W in {256, 512, 8192}) plus W = R and
    the split-K windows; q and the compacted cache are fp16 N(0,1)."""
    from quant_kernel import build_quantized_kv_cache
    B, H, KVH, D = 32, 64, 8, 128
    L = S + W + 1000
    gen = torch.Generator(device=device).manual_seed(3 + W)
    q = torch.randn(B, H, D, generator=gen, device=device, dtype=torch.float16)
    kc = torch.randn(B, KVH, S + W, D, generator=gen, device=device, dtype=torch.float16)
    vc = torch.randn(B, KVH, S + W, D, generator=gen, device=device, dtype=torch.float16)
    say(f"kivi steady W={W}")
    cache = build_quantized_kv_cache(kc, vc)
    o = _attend(q, cache, L, W)
    hc = _host_cache(cache)
    qh = host(q)
    # codes built on the GPU equal the oracle's build on the same fp16 cache
    oc = O.build_quantized_kv_cache(host(kc), host(vc))
    for key in O.CACHE_KEYS:
        np.testing.assert_array_equal(hc[key], oc[key], err_msg=key)
    ref = O.quantized_attention(qh, W - R, hc, SCALE)
    assert max_abs(o, ref) < ATTN_TOL
    assert max_abs(o, O.quantized_attention(qh, W - R, hc, SCALE, dtype=np.float32)) < REF_TOL


@pytest.mark.parametrize("G", [1, 4, 16])
@pytest.mark.parametrize("W", [256, 1024])
def test_quantized_attention_query_group_sizes(G, W, device):
    """G = H / KVH query heads per KV head other than 8: one head, a partial
    MFMA column block, all 16 columns (the quantized tiles' publish writes
    16 head rows in their own lane layout).  Static (W=256) and dynamic
    (W=1024) work queues."""
    from quant_kernel import build_quantized_kv_cache
    B, KVH, D = 2, 4, 128
    H = G * KVH
    gen = torch.Generator(device=device).manual_seed(400 + G + W)
    q = torch.randn(B, H, D, generator=gen, device=device, dtype=torch.float16)
    kc = torch.randn(B, KVH, S + W, D, generator=gen, device=device, dtype=torch.float16)
    vc = torch.randn(B, KVH, S + W, D, generator=gen, device=device, dtype=torch.float16)
    say(f"kivi G={G} W={W}")
    cache = build_quantized_kv_cache(kc, vc)
    o = _attend(q, cache, 163840, W)
    ref = O.quantized_attention(host(q), W - R, _host_cache(cache), SCALE)
    assert max_abs(o, ref) < ATTN_TOL
    assert_nearly_rounded(o, ref)


def test_quantized_attention_outlier_keys(device):
    """Config-5 distributions: K with 4 channels x10 (sharper softmax)."""
    from quant_kernel import build_quantized_kv_cache
    B, H, KVH, D, W = 32, 64, 8, 128, 256
    gen = torch.Generator(device=device).manual_seed(11)
    q = torch.randn(B, H, D, generator=gen, device=device, dtype=torch.float16)
    kc = torch.randn(B, KVH, S + W, D, generator=gen, device=device, dtype=torch.float16)
    outl = torch.randperm(D, generator=torch.Generator().manual_seed(0))[:4].tolist()
    kc[..., outl] *= 10
    vc = torch.randn(B, KVH, S + W, D, generator=gen, device=device, dtype=torch.float16)
    say("kivi outliers")
    cache = build_quantized_kv_cache(kc, vc)
    o = _attend(q, cache, 163840, W)
    ref = O.quantized_attention(host(q), W - R, _host_cache(cache), SCALE)
    assert max_abs(o, ref) < ATTN_TOL


@pytest.mark.parametrize("vmul", [1.0, 600.0])
def test_quantized_attention_growing_logits(vmul, device):
    """Logits that grow along the window (K row t scaled by 1 + t/512), so
    the running max rises tile after tile: quantized tiles refresh it
    lazily (up to 2^8 above it) while every V scale is <= 128, and eagerly
    when V is scaled x600 (V scales ~1200: a lazy p * scale could overflow
    fp16).  W=4096 gives each wave a dynamic queue of many tiles."""
    from quant_kernel import build_quantized_kv_cache
    B, H, KVH, D, W = 4, 32, 4, 128, 4096
    gen = torch.Generator(device=device).manual_seed(21)
    q = torch.randn(B, H, D, generator=gen, device=device, dtype=torch.float16)
    ramp = 1 + torch.arange(S + W, device=device, dtype=torch.float32) / 512
    kc = (torch.randn(B, KVH, S + W, D, generator=gen, device=device) * ramp[:, None]).half()
    vc = (torch.randn(B, KVH, S + W, D, generator=gen, device=device) * vmul).half()
    say(f"kivi growing logits vmul={vmul}")
    cache = build_quantized_kv_cache(kc, vc)
    o = _attend(q, cache, 163840, W)
    ref = O.quantized_attention(host(q), W - R, _host_cache(cache), SCALE)
    assert np.all(np.isfinite(o))
    assert max_abs(o, ref) < ATTN_TOL * vmul
    assert_nearly_rounded(o, ref, 5e-5 * vmul)


def test_quantized_attention_large_v_offsets(device):
    """V rows far from zero relative to their spread (100 + 0.05 N(0,1)):
    zero points beyond 1000, which take the separate zero-term path, in
    some groups and tiles next to ordinary ones.  Outputs near 100 are
    checked to half an fp16 ulp."""
    from quant_kernel import build_quantized_kv_cache
    B, H, KVH, D, W = 2, 16, 2, 128, 512
    gen = torch.Generator(device=device).manual_seed(17)
    q = torch.randn(B, H, D, generator=gen, device=device, dtype=torch.float16)
    kc = torch.randn(B, KVH, S + W, D, generator=gen, device=device).half()
    vc = torch.randn(B, KVH, S + W, D, generator=gen, device=device)
    far = torch.zeros(S + W, dtype=torch.bool, device=device)
    far[S + 32:S + 96] = True                   # two whole window-old tiles
    far[S + 200:S + 210] = True                 # part of a tile
    vc[:, :, far] = 100 + 0.05 * vc[:, :, far]
    vc[:, :, :, 64:] = torch.where(far[None, None, :, None], vc[:, :, :, 64:] - 100, vc[:, :, :, 64:])
    vc = vc.half()
    say("kivi large V offsets")
    cache = build_quantized_kv_cache(kc, vc)
    zeros = host(cache["v_win_zero"]).astype(np.float32)
    assert np.abs(zeros).max() > 1000 and (np.abs(zeros) <= 3).any()
    o = _attend(q, cache, 163840, W)
    ref = O.quantized_attention(host(q), W - R, _host_cache(cache), SCALE)
    assert_nearly_rounded(o, ref)


@pytest.mark.parametrize("W", [256, 512])
def test_quantized_attention_large_k_offsets(W, device):
    """K channels far from zero relative to their spread (+-100, +-300 and
    30 plus 0.05 N(0,1), in every token): K zero points of both signs up to
    a few thousand (fp16 integers, even above 2048), in the sink and window
    groups.  1024 + zero and code - zero are then not exact fp16, so those
    tiles take the separate zero-term path; every output must stay within
    half an fp16 ulp of the fp64 oracle (plus 5e-5)."""
    from quant_kernel import build_quantized_kv_cache
    B, H, KVH, D = 2, 16, 2, 128
    gen = torch.Generator(device=device).manual_seed(19 + W)
    q = torch.randn(B, H, D, generator=gen, device=device, dtype=torch.float16)
    kc = torch.randn(B, KVH, S + W, D, generator=gen, device=device)
    for ch, off in [(3, 100.0), (17, -100.0), (40, 300.0), (77, -300.0), (90, 30.0)]:
        kc[..., ch] = off + 0.05 * kc[..., ch]
    kc = kc.half()
    vc = torch.randn(B, KVH, S + W, D, generator=gen, device=device, dtype=torch.float16)
    say(f"kivi large K offsets W={W}")
    cache = build_quantized_kv_cache(kc, vc)
    hc = _host_cache(cache)
    zeros = np.concatenate([hc["k_win_zero"].ravel(), hc["k_sink_zero"].ravel()]).astype(np.float32)
    assert zeros.max() > 2048 and zeros.min() < -2048
    o = _attend(q, cache, 163840, W)
    ref = O.quantized_attention(host(q), W - R, hc, SCALE)
    assert max_abs(o, ref) < ATTN_TOL
    assert_nearly_rounded(o, ref)


@pytest.mark.parametrize("W,varlen", [(32, False), (256, False), (512, False), (1024, False),
                                      (256, True), (1024, True)])
def test_quantized_attention_q_times_k_scale_beyond_fp16(W, varlen, device):
    """|q| = 64 on a K channel whose 32-token groups span 0..30000 (K scale
    10000): the fp16 product q * scale (-640000) is beyond the fp16 range,
    which the kernels' power-of-two Q prescale keeps finite.  The channel's
    other tokens are 0 (code 0 exactly), the outlier tokens (one window-old,
    one sink) get logits of about -2e6 and weight 0, so every output stays
    an ordinary attention result within half an fp16 ulp of the fp64
    oracle.  Covers the lean kernels (W=32, 256), the 16-wave kernel (W=512,
    1024) and the general kernel (per-sequence lengths)."""
    from quant_kernel import build_quantized_kv_cache
    B, H, KVH, D = 2, 16, 2, 128
    gen = torch.Generator(device=device).manual_seed(23 + W)
    q = torch.randn(B, H, D, generator=gen, device=device, dtype=torch.float16)
    q[..., 5] = -64.0
    kc = torch.randn(B, KVH, S + W, D, generator=gen, device=device)
    kc[..., 5] = 0.0
    kc[:, :, 1, 5] = 30000.0                          # sink group
    if W > R:
        kc[:, :, S + 40, 5] = 30000.0                 # a window-old group
    kc = kc.half()
    vc = torch.randn(B, KVH, S + W, D, generator=gen, device=device, dtype=torch.float16)
    say(f"kivi q * k_scale beyond fp16 W={W} varlen={varlen}")
    cache = build_quantized_kv_cache(kc, vc)
    hc = _host_cache(cache)
    assert float(hc["k_sink_scale"][..., 5].astype(np.float32).max()) == 10000.0
    L = 163840
    o = _attend(q, cache, torch.full((B,), L, dtype=torch.int32, device=device) if varlen else L, W)
    ref = O.quantized_attention(host(q), W - R, hc, SCALE)
    assert np.isfinite(o).all()
    assert max_abs(o, ref) < ATTN_TOL
    assert_nearly_rounded(o, ref)


@pytest.mark.parametrize("where", ["window_old", "sink", "residual"])
def test_quantized_attention_dominant_token(where, device):
    """One token carries almost all of a head's softmax weight, so the output
    is (nearly) that token's V row: an fp16 rounding of its probability (or
    of probability x V scale) would show up whole in the output.  Every
    output must be within half an fp16 ulp of the fp64 oracle (plus 5e-5)."""
    from quant_kernel import build_quantized_kv_cache
    B, H, KVH, D, W = 4, 32, 4, 128, 1024
    gen = torch.Generator(device=device).manual_seed(5)
    q = torch.randn(B, H, D, generator=gen, device=device, dtype=torch.float16)
    kc = torch.randn(B, KVH, S + W, D, generator=gen, device=device)
    vc = torch.randn(B, KVH, S + W, D, generator=gen, device=device) * 1.9
    slot = {"window_old": S + 300, "sink": 2, "residual": S + W - 5}[where]
    G = H // KVH
    for kv in range(KVH):                      # query head kv * G of every KV head
        kc[:, kv, slot] = q[:, kv * G].float() * 0.9
    kc, vc = kc.half(), vc.half()
    say(f"kivi dominant token in {where}")
    cache = build_quantized_kv_cache(kc, vc)
    o = _attend(q, cache, 163840, W)
    ref = O.quantized_attention(host(q), W - R, _host_cache(cache), SCALE)
    assert max_abs(o, ref) < ATTN_TOL
    assert_nearly_rounded(o, ref)


@pytest.mark.parametrize("W,L", [(256, L) for L in (1, 3, 4, 5, 60, 131, 200, 259, 260, 261)] +
                         [(384, L) for L in (1, 3, 4, 5, 60, 200, 300, 387, 388, 389)] +
                         [(1024, L) for L in (3, 500, 900, 1027, 1028, 1029)])
def test_quantized_attention_rampup(W, L, device):
    """Ramp-up (seq_len <= S + W): only the slots the _kv_indices rule marks
    valid are attended.  Unwritten slots hold 3.0 before quantization: far
    enough from N(0,1) data that a leak moves the output, small enough that
    the quantization groups they share with real tokens stay well conditioned
    (1e4, as in the fp16 sparse test, would swamp those groups' scales).
    W = 256 runs the 9-wave lean kernel (the sink group on its own wave),
    W = 384 the 8-wave kernel, W = 1024 the 16-wave one."""
    from quant_kernel import build_quantized_kv_cache
    B, H, KVH, D = 2, 16, 2, 128
    kf = randn((B, KVH, max(L, 1), D), 30 + L)
    vf = randn((B, KVH, max(L, 1), D), 31 + L)
    kc, vc = O.build_compacted_cache(kf, vf, L, W, S, garbage=3.0)
    q16 = randn((B, H, D), 32 + L, np.float16)
    say(f"kivi ramp W={W} L={L}")
    cache = build_quantized_kv_cache(dev(kc.astype(np.float16), device), dev(vc.astype(np.float16), device))
    o = _attend(dev(q16, device), cache, L, W)
    ref = O.quantized_attention_masked(q16, _host_cache(cache), L, W, SCALE)
    assert max_abs(o, ref) < ATTN_TOL


@pytest.mark.parametrize("W", [96, 384])
def test_quantized_attention_varlen(W, device):
    """One length per sequence: pre-sink, ramp-up (fp16 residual slots,
    then window-old slots partly unwritten), the last ramp-up length and
    steady state share one launch; each row matches the oracle at its own
    length and the scalar-length call at that length."""
    from quant_kernel import build_quantized_kv_cache
    lens = [1, 3, 60, 200, S + W - 1, S + W, 163840]
    B, H, KVH, D = len(lens), 16, 2, 128
    kc = np.zeros((B, KVH, S + W, D), np.float32)
    vc = np.zeros((B, KVH, S + W, D), np.float32)
    for b, n in enumerate(lens):
        m = min(n, S + W + 64)
        kb, vb = O.build_compacted_cache(randn((1, KVH, m, D), 60 + b), randn((1, KVH, m, D), 70 + b),
                                         min(n, m), W, S, garbage=3.0)
        kc[b], vc[b] = kb[0], vb[0]
    q16 = randn((B, H, D), 80 + W, np.float16)
    say(f"kivi varlen W={W}")
    cache = build_quantized_kv_cache(dev(kc.astype(np.float16), device), dev(vc.astype(np.float16), device))
    o = _attend(dev(q16, device), cache, torch.tensor(lens, dtype=torch.int32, device=device), W)
    ref = O.quantized_attention_varlen(q16, _host_cache(cache), lens, W, SCALE)
    assert max_abs(o, ref) < ATTN_TOL
    qd = dev(q16, device)
    for b, n in enumerate(lens):
        assert max_abs(o[b], _attend(qd, cache, n, W)[b]) < ATTN_TOL, n


@pytest.mark.parametrize("W", [32, 48, 96])
@pytest.mark.parametrize("L", [20, 163840])
def test_quantized_attention_window_below_residual(W, L, device):
    """window < residual_size (config 5's W=32; undefined in the reference):
    the whole window stays fp16, the sink is quantized.  Steady state and
    ramp-up (seq_len 20: the window's first slots are unwritten)."""
    from quant_kernel import build_quantized_kv_cache
    B, H, KVH, D = 4, 32, 4, 128
    if L >= S + W:                                   # steady state: every slot written
        kc = randn((B, KVH, S + W, D), 50 + W)
        vc = randn((B, KVH, S + W, D), 51 + W)
    else:
        kc, vc = O.build_compacted_cache(randn((B, KVH, L, D), 50 + W), randn((B, KVH, L, D), 51 + W),
                                         L, W, S, garbage=3.0)
    q16 = randn((B, H, D), 52 + W, np.float16)
    say(f"kivi W={W} < R, L={L}")
    cache = build_quantized_kv_cache(dev(kc.astype(np.float16), device), dev(vc.astype(np.float16), device))
    hc = _host_cache(cache)
    assert hc["k_residual"].shape[2] == W and hc["k_win_packed"].shape[2] == 0
    oc = O.build_quantized_kv_cache(kc.astype(np.float16), vc.astype(np.float16))
    for key in O.CACHE_KEYS:
        np.testing.assert_array_equal(hc[key], oc[key], err_msg=key)
    o = _attend(dev(q16, device), cache, L, W)
    ref = O.quantized_attention_masked(q16, hc, L, W, SCALE)
    assert max_abs(o, ref) < ATTN_TOL


@pytest.mark.parametrize("G", [1, 12, 16])
@pytest.mark.parametrize("W", [32, 64])
def test_quantized_attention_window_below_residual_groups(G, W, device):
    """W < R (1-2 residual tiles, the sink the only quantized group) with
    query groups of 1, 12 and 16 heads: each output correctly rounded."""
    from quant_kernel import build_quantized_kv_cache
    B, KVH, D = 3, 2, 128
    H = G * KVH
    kc = randn((B, KVH, S + W, D), 60 + W + G, np.float16)
    vc = randn((B, KVH, S + W, D), 61 + W + G, np.float16)
    q16 = randn((B, H, D), 62 + W + G, np.float16)
    say(f"kivi W={W} < R, G={G}")
    cache = build_quantized_kv_cache(dev(kc, device), dev(vc, device))
    o = _attend(dev(q16, device), cache, 163840, W)
    ref = O.quantized_attention_masked(q16, _host_cache(cache), 163840, W, SCALE)
    assert_nearly_rounded(o, ref)


def test_quantized_attention_rejects_small_window(device):
    from quant_kernel import build_quantized_kv_cache
    kc = torch.zeros(1, 2, S + 256, 128, dtype=torch.float16, device=device)
    cache = build_quantized_kv_cache(kc, kc)
    q = torch.zeros(1, 16, 128, dtype=torch.float16, device=device)
    with pytest.raises(ValueError):
        _attend(q, cache, 1000, 64)


@pytest.mark.parametrize("sink", [1, 16, 17, 20, 32])
@pytest.mark.parametrize("W", [256, 1024])
def test_quantized_attention_sink_sizes(sink, W, device):
    """Sink groups of 1 to 32 real tokens (the API's sink argument): the
    9-wave lean kernel (W=256, the sink group on wave 4: a half-group step
    up to 16 tokens, a whole one above), the 16-wave kernel (W=1024 with a sink of at
    most 16 tokens: its half-group step after the loop) and the work-queue
    kernel (W=1024, sink > 16), in steady state and ramp-up.  Each case is
    launched five times and every output checked: a schedule whose result
    depends on how the waves interleave shows as a wrong output on some
    calls only."""
    from quant_kernel import build_quantized_kv_cache
    B, H, KVH, D = 2, 16, 2, 128
    q16 = randn((B, H, D), 60 + sink + W, np.float16)
    for L in (sink + W + 500, sink + W // 2):
        kf = randn((B, KVH, L, D), 61 + sink + L)
        vf = randn((B, KVH, L, D), 62 + sink + L)
        kc, vc = O.build_compacted_cache(kf, vf, L, W, sink, garbage=3.0)
        say(f"kivi sink={sink} W={W} L={L}")
        cache = build_quantized_kv_cache(dev(kc.astype(np.float16), device), dev(vc.astype(np.float16), device),
                                         sink=sink)
        ref = O.quantized_attention_masked(q16, _host_cache(cache), L, W, SCALE, sink=sink)
        qd = dev(q16, device)
        for rep in range(5):
            o = _attend(qd, cache, L, W, sink=sink)
            assert max_abs(o, ref) < ATTN_TOL, rep
            if L > sink + W:
                assert_nearly_rounded(o, ref)


@pytest.mark.parametrize("W,sink", [(32, 4), (160, 4), (256, 4), (256, 20), (352, 4), (1024, 4), (1024, 20)])
def test_kivi_bit_identical_under_concurrent_load(W, sink, device):
    """The fused decode's waves meet only at the Q readiness count (lean
    kernels), the group-queue counter (16-wave kernel) and the merge barrier,
    so a result must not depend on how far each wave has got.  Launches made
    while a second stream (default priority) copies 512 MiB through the same
    CUs and HBM must be bit-identical to a launch on an idle GPU (the lean
    kernel's work split is static; the 16-wave kernel's queue makes the
    summation order vary, so there the outputs must agree within the
    attention gate and the oracle's).  The windows cover the 8-wave lean
    kernel (W=32, 160, 352), the 9-wave one (W=256, with a half- and a
    whole-group sink step) and the 16-wave one (W=1024, sink of 4 and 20)."""
    from quant_kernel import build_quantized_kv_cache, sparse_decode_attention_quantized
    B, H, KVH, D = 32, 64, 8, 128
    L = sink + W + 1000
    gen = torch.Generator(device=device).manual_seed(70 + W + sink)
    kc = torch.randn(B, KVH, sink + W, D, generator=gen, device=device, dtype=torch.float16)
    vc = torch.randn(B, KVH, sink + W, D, generator=gen, device=device, dtype=torch.float16)
    q = torch.randn(B, H, D, generator=gen, device=device, dtype=torch.float16)
    cache = build_quantized_kv_cache(kc, vc, sink=sink)
    args = [cache[k] for k in O.CACHE_KEYS]

    def attend():
        return sparse_decode_attention_quantized(q, *args, seq_len=L, window=W, sink=sink)

    say(f"kivi concurrent-load determinism W={W} sink={sink}")
    ref = attend()
    torch.cuda.synchronize()
    src = torch.ones((512 << 20) // 4, dtype=torch.int32, device=device)
    dst = torch.empty_like(src)
    side = torch.cuda.Stream(device)
    outs = []
    for i in range(24):
        side.wait_stream(torch.cuda.current_stream(device))
        with torch.cuda.stream(side):
            dst.copy_(src)
        if i % 3:
            outs.append(attend())
        else:
            torch.cuda.current_stream(device).wait_stream(side)
            outs.append(attend())
    torch.cuda.synchronize()
    o_ref = host(ref)
    for i, o in enumerate(outs):
        if W <= 352:
            assert torch.equal(o, ref), f"launch {i} differs from the idle-GPU launch"
        else:
            assert max_abs(host(o), o_ref) < 1e-3, f"launch {i}"
    hc = _host_cache(cache)
    ho = O.quantized_attention_masked(host(q)[:2], {k: v[:2] for k, v in hc.items()}, L, W, SCALE, sink=sink)
    assert max_abs(o_ref[:2], ho) < ATTN_TOL
