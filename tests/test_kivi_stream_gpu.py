"""Decode-time KIVI cache (kivi_stream.py) on the GPU: appends with
quantize-on-evict, then the fused decode over the ring state.

Right after each eviction the state must be what the reference's builder
(quant_kernel.py:584-622) makes of the compacted cache at that length: the
same window-old codes (bit-exact, in ring order), the same residual tokens,
and the same decode output as the one-shot path.  Between evictions the
output is checked against the CPU oracle's stream_cache state."""

import numpy as np
import pytest
import torch

from helpers import ATTN_TOL, SCALE, dev, host, max_abs, say
from oracle import kvdec_oracle as O

pytestmark = pytest.mark.gpu

S, R, G = 4, 128, 32


def _stream(B, H, KVH, W, L0, steps, seed):
    from kivi_stream import KiviStreamCache
    gen = torch.Generator(device="cuda").manual_seed(seed)
    D = 128
    kf = torch.randn(B, KVH, L0 + steps, D, generator=gen, device="cuda", dtype=torch.float16)
    vf = torch.randn(B, KVH, L0 + steps, D, generator=gen, device="cuda", dtype=torch.float16)
    q = torch.randn(B, H, D, generator=gen, device="cuda", dtype=torch.float16)
    cache = KiviStreamCache.from_prefill(kf[:, :, :L0], vf[:, :, :L0], W)
    return cache, kf, vf, q


@pytest.mark.parametrize("W", [256, 1024, 128])
def test_stream_matches_builder_after_evictions(W, device):
    from quant_kernel import build_quantized_kv_cache, sparse_decode_attention_quantized
    B, H, KVH = 4, 32, 4
    L0 = S + W + 37
    cache, kf, vf, q = _stream(B, H, KVH, W, L0, 3 * G, 40 + W)
    for step in range(3 * G):
        cache.append(kf[:, :, cache.seq_len], vf[:, :, cache.seq_len])
        if cache.ring.count != R:
            continue
        L = cache.seq_len
        say(f"stream W={W} L={L}")
        comp_k = torch.cat([kf[:, :, :S], kf[:, :, L - W:L]], dim=2)
        comp_v = torch.cat([vf[:, :, :S], vf[:, :, L - W:L]], dim=2)
        ref = build_quantized_kv_cache(comp_k, comp_v)
        o_ref = sparse_decode_attention_quantized(
            q, ref["k_residual"], ref["v_residual"],
            ref["k_sink_packed"], ref["k_sink_scale"], ref["k_sink_zero"],
            ref["v_sink_packed"], ref["v_sink_scale"], ref["v_sink_zero"],
            ref["k_win_packed"], ref["k_win_scale"], ref["k_win_zero"],
            ref["v_win_packed"], ref["v_win_scale"], ref["v_win_zero"], seq_len=L, window=W)
        o = cache.attend(q)
        torch.cuda.synchronize()
        # window-old groups: ring slots in age order hold the builder's groups
        slots = cache.window_old_slots()
        for name, per in (("k_win_packed", G // 4), ("k_win_scale", 1), ("k_win_zero", 1),
                          ("v_win_packed", G), ("v_win_scale", G), ("v_win_zero", G)):
            got = host(cache.t[name])
            want = host(ref[name])
            for age, slot in enumerate(slots):
                np.testing.assert_array_equal(got[:, :, slot * per:(slot + 1) * per],
                                              want[:, :, age * per:(age + 1) * per], err_msg=name)
        rows = cache.residual_rows()
        np.testing.assert_array_equal(host(cache.t["k_ring"])[:, :, rows], host(ref["k_residual"]))
        np.testing.assert_array_equal(host(cache.t["v_ring"])[:, :, rows], host(ref["v_residual"]))
        for name in ("k_sink_packed", "k_sink_scale", "k_sink_zero",
                     "v_sink_packed", "v_sink_scale", "v_sink_zero"):
            np.testing.assert_array_equal(host(cache.t[name]), host(ref[name]), err_msg=name)
        assert max_abs(host(o), host(o_ref)) < 1e-3
        # and the CPU oracle: its builder on the same compacted cache gives
        # the GPU builder's tensors, and its stream_cache state (pinned by a
        # token-by-token model in test_oracle.py) the same attention
        oc = O.build_quantized_kv_cache(host(comp_k), host(comp_v))
        for key in O.CACHE_KEYS:
            np.testing.assert_array_equal(host(ref[key]), oc[key], err_msg=key)
        sc, wlen = O.stream_cache(host(kf), host(vf), L0, L, W)
        for key in O.CACHE_KEYS:
            np.testing.assert_array_equal(sc[key], oc[key], err_msg=key)
        o_orc = O.quantized_attention(host(q), wlen, sc, SCALE)
        assert max_abs(host(o), o_orc) < ATTN_TOL


# the ring decode's kernels: 8 heads per KV head with 4 and 7 window-old
# groups (the lean kernel, packed), 16 heads (lean, unpacked), 8 window-old
# groups (past the lean kernel)
@pytest.mark.parametrize("H,KVH,W", [(16, 2, 256), (16, 2, 352), (32, 2, 256), (16, 2, 384)])
def test_stream_between_evictions_vs_oracle(H, KVH, W, device):
    B = 2
    L0 = S + W + 5
    steps = 70
    cache, kf, vf, q = _stream(B, H, KVH, W, L0, steps, 77 + W + H)
    kh, vh, qh = host(kf), host(vf), host(q)
    for step in range(steps):
        cache.append(kf[:, :, cache.seq_len], vf[:, :, cache.seq_len])
        if step % 9 != 4:
            continue
        L = cache.seq_len
        say(f"stream between evictions H={H} KVH={KVH} W={W} L={L} count={cache.ring.count}")
        o = host(cache.attend(q))
        oc, wlen = O.stream_cache(kh, vh, L0, L, W)
        ref = O.quantized_attention(qh, wlen, oc, SCALE)
        assert max_abs(o, ref) < ATTN_TOL


def test_stream_reserve_equals_append(device):
    """reserve() + writing the row views gives the state append() gives."""
    B, H, KVH, W = 2, 16, 2, 256
    L0 = S + W + 3
    a, kf, vf, q = _stream(B, H, KVH, W, L0, 40, 91)
    from kivi_stream import KiviStreamCache
    b = KiviStreamCache.from_prefill(kf[:, :, :L0], vf[:, :, :L0], W)
    for step in range(40):
        a.append(kf[:, :, a.seq_len], vf[:, :, a.seq_len])
        kv, vv = b.reserve()
        kv.copy_(kf[:, :, b.seq_len - 1])
        vv.copy_(vf[:, :, b.seq_len - 1])
    say("stream reserve vs append")
    for name in a.t:
        np.testing.assert_array_equal(host(a.t[name]), host(b.t[name]), err_msg=name)
    np.testing.assert_array_equal(host(a.attend(q)), host(b.attend(q)))


def test_stream_rejects_short_prefill(device):
    from kivi_stream import KiviStreamCache
    k = torch.zeros(1, 2, S + 255, 128, dtype=torch.float16, device=device)
    with pytest.raises(ValueError):
        KiviStreamCache.from_prefill(k, k, 256)


@pytest.mark.parametrize("per_sequence", [False, True])
def test_stream_attend_bit_identical_under_concurrent_load(per_sequence, device):
    """The ring decode kernel's waves (window-old slots, the sink group, the
    ring tiles) meet only at the Q readiness count, the premerge count and
    the merge barrier, and its work split is static: repeated attends of one
    state, some launched while a second stream copies 512 MiB through the
    same CUs and HBM, must be bit-identical to the first (one ring state for
    all sequences, and one per sequence)."""
    from kivi_stream import KiviStreamBatch, KiviStreamCache
    B, H, KVH, W, D = 32, 64, 8, 256, 128
    L0 = S + W + 40
    gen = torch.Generator(device="cuda").manual_seed(97)
    kf = torch.randn(B, KVH, L0, D, generator=gen, device="cuda", dtype=torch.float16)
    vf = torch.randn(B, KVH, L0, D, generator=gen, device="cuda", dtype=torch.float16)
    q = torch.randn(B, H, D, generator=gen, device="cuda", dtype=torch.float16)
    cls = KiviStreamBatch if per_sequence else KiviStreamCache
    cache = cls.from_prefill(kf, vf, W)
    say(f"stream concurrent-load determinism per_sequence={per_sequence}")
    ref = cache.attend(q)
    torch.cuda.synchronize()
    src = torch.ones((512 << 20) // 4, dtype=torch.int32, device=device)
    dst = torch.empty_like(src)
    side = torch.cuda.Stream(device)
    outs = []
    for i in range(16):
        side.wait_stream(torch.cuda.current_stream(device))
        with torch.cuda.stream(side):
            dst.copy_(src)
        if i % 2:
            torch.cuda.current_stream(device).wait_stream(side)
        outs.append(cache.attend(q))
    torch.cuda.synchronize()
    for i, o in enumerate(outs):
        assert torch.equal(o, ref), f"attend {i} differs from the first"
