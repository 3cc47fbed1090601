"""Decode-time KIVI cache with one ring state per sequence
(kivi_stream.KiviStreamBatch) on the GPU: sequences that sit out steps and a
sequence that joins with its own prefill.  Each sequence must end up where a
single-sequence KiviStreamCache fed the same tokens ends up (ring rows and
window-old codes exactly, decode output to an fp16 ulp), and the on-GPU
bookkeeping must match the host's RingState arithmetic step by step."""

import numpy as np
import pytest
import torch

from helpers import ATTN_TOL, SCALE, assert_nearly_rounded, host, max_abs, say
from oracle import kvdec_oracle as O

pytestmark = pytest.mark.gpu

S, R, G = 4, 128, 32


def test_plan_matches_host_ring_state(device):
    """The on-GPU bookkeeping of kvdec_kivi_stream_step over 150 steps with
    random active masks: the step taken and the ring state after it equal
    RingState.append() per sequence."""
    from kivi_stream import KiviStreamBatch, RingState
    B, KVH, D, W = 6, 3, 128, 256
    k = torch.zeros(B, KVH, S + W, D, dtype=torch.float16, device=device)
    cache = KiviStreamBatch.from_prefill(k, k, W)
    host_rings = [RingState(cap=R + G, residual=R, n_groups=(W - R) // G, count=R) for _ in range(B)]
    rng = np.random.default_rng(0)
    say("stream plan vs host")
    for step in range(150):
        active = rng.random(B) < 0.7
        cache._step(None, None, torch.from_numpy(active).to(device))
        plan, ring = host(cache.plan), host(cache.ring)
        for b in range(B):
            if active[b]:
                row, blk, slot = host_rings[b].append()
                assert tuple(plan[b]) == (row, blk, slot if blk >= 0 else -1), (step, b)
            else:
                assert tuple(plan[b]) == (-1, -1, -1)
            assert (ring[b, 0], ring[b, 1]) == (host_rings[b].start, host_rings[b].count), (step, b)


@pytest.mark.parametrize("W", [256, 1024])
def test_batch_equals_single_sequence_caches(W, device):
    """Random active masks for 90 steps, slot 2 re-admitted at step 33 with a
    prefill of another length: every sequence's ring rows and window-old
    codes equal a one-sequence KiviStreamCache given the same tokens
    (bit-exact), its decode output matches that cache's (to one fp16 ulp:
    the summation order of a dynamic work queue may differ), and one
    sequence per check matches the CPU oracle's stream state."""
    from kivi_stream import KiviStreamBatch, KiviStreamCache
    B, H, KVH, D = 4, 16, 2, 128
    L0, steps = S + W + 21, 90
    gen = torch.Generator(device=device).manual_seed(W)
    kf = torch.randn(B, KVH, L0 + steps, D, generator=gen, device=device, dtype=torch.float16)
    vf = torch.randn(B, KVH, L0 + steps, D, generator=gen, device=device, dtype=torch.float16)
    L2 = S + W + 70                                  # the late joiner's prefill length
    k2 = torch.randn(KVH, L2 + steps, D, generator=gen, device=device, dtype=torch.float16)
    v2 = torch.randn(KVH, L2 + steps, D, generator=gen, device=device, dtype=torch.float16)
    q = torch.randn(B, H, D, generator=gen, device=device, dtype=torch.float16)
    batch = KiviStreamBatch.from_prefill(kf[:, :, :L0], vf[:, :, :L0], W)
    singles = [KiviStreamCache.from_prefill(kf[b:b + 1, :, :L0], vf[b:b + 1, :, :L0], W) for b in range(B)]
    pos = [L0] * B                                   # next position of each sequence
    src_k = [kf[b] for b in range(B)]
    src_v = [vf[b] for b in range(B)]
    rng = np.random.default_rng(W)
    say(f"stream batch W={W}")
    for step in range(steps):
        if step == 33:
            batch.admit(2, k2[:, :L2], v2[:, :L2])
            singles[2] = KiviStreamCache.from_prefill(k2[None, :, :L2], v2[None, :, :L2], W)
            pos[2], src_k[2], src_v[2] = L2, k2, v2
        active = rng.random(B) < 0.75
        kn = torch.stack([src_k[b][:, pos[b]] for b in range(B)])
        vn = torch.stack([src_v[b][:, pos[b]] for b in range(B)])
        batch.append(kn, vn, torch.from_numpy(active).to(device))
        for b in range(B):
            if active[b]:
                singles[b].append(kn[b:b + 1], vn[b:b + 1])
                pos[b] += 1
        if step % 11 != 10:
            continue
        o = host(batch.attend(q))
        for b in range(B):
            one = singles[b]
            rows = one.residual_rows()
            np.testing.assert_array_equal(host(batch.t["k_ring"][b])[:, rows], host(one.t["k_ring"][0])[:, rows])
            np.testing.assert_array_equal(host(batch.t["v_ring"][b])[:, rows], host(one.t["v_ring"][0])[:, rows])
            for name in ("k_win_packed", "k_win_scale", "k_win_zero", "v_win_packed", "v_win_scale",
                         "v_win_zero", "k_sink_packed", "k_sink_scale", "k_sink_zero",
                         "v_sink_packed", "v_sink_scale", "v_sink_zero"):
                np.testing.assert_array_equal(host(batch.t[name][b]), host(one.t[name][0]), err_msg=name)
            # the same arithmetic; with a dynamic work queue (W=1024) the
            # summation order may differ, so allow one fp16 ulp
            assert max_abs(o[b], host(one.attend(q[b:b + 1]))[0]) < ATTN_TOL
        # oracle check of one sequence at this step
        b = step % B
        L = pos[b]
        p0 = L2 if (b == 2 and step >= 33) else L0
        src = (k2[None], v2[None]) if (b == 2 and step >= 33) else (kf[b:b + 1], vf[b:b + 1])
        oc, wlen = O.stream_cache(host(src[0]), host(src[1]), p0, L, W)
        ref = O.quantized_attention(host(q[b:b + 1]), wlen, oc, SCALE)
        assert max_abs(o[b:b + 1], ref) < ATTN_TOL
        assert_nearly_rounded(o[b:b + 1], ref)


def test_batch_reserve_equals_append(device):
    """reserve() returns each sequence's ring row; writing K/V there gives
    the state append() gives."""
    from kivi_stream import KiviStreamBatch
    B, H, KVH, D, W = 3, 16, 2, 128, 256
    L0 = S + W + 3
    gen = torch.Generator(device=device).manual_seed(5)
    kf = torch.randn(B, KVH, L0 + 40, D, generator=gen, device=device, dtype=torch.float16)
    vf = torch.randn(B, KVH, L0 + 40, D, generator=gen, device=device, dtype=torch.float16)
    q = torch.randn(B, H, D, generator=gen, device=device, dtype=torch.float16)
    a = KiviStreamBatch.from_prefill(kf[:, :, :L0], vf[:, :, :L0], W)
    b = KiviStreamBatch.from_prefill(kf[:, :, :L0], vf[:, :, :L0], W)
    active = torch.tensor([1, 0, 1], dtype=torch.int32, device=device)
    say("stream batch reserve vs append")
    for step in range(40):
        kn, vn = kf[:, :, L0 + step], vf[:, :, L0 + step]
        a.append(kn, vn, active)
        rows = b.reserve(active).long()
        for s in range(B):
            if int(rows[s]) >= 0:
                b.t["k_ring"][s, :, rows[s]] = kn[s]
                b.t["v_ring"][s, :, rows[s]] = vn[s]
    torch.cuda.synchronize()
    for name in a.t:
        if name in ("k_ring", "v_ring"):
            continue
        np.testing.assert_array_equal(host(a.t[name]), host(b.t[name]), err_msg=name)
    np.testing.assert_array_equal(host(a.ring), host(b.ring))
    np.testing.assert_array_equal(host(a.attend(q)), host(b.attend(q)))


@pytest.mark.parametrize("W", [160, 256, 288, 1024])
def test_step_attend_equals_append_then_attend(W, device):
    """step_attend (one launch: each workgroup writes its token's row,
    quantizes its evicted block, then attends) against append followed by
    attend on an identical cache, over 75 steps with random active masks
    (every sequence crosses at least one eviction): the same outputs (bit
    for bit with a static work split; W=1024's dynamic work queue may sum in
    another order, so one fp16 ulp), and every cache tensor and the
    bookkeeping bit for bit.  W=160 and 288 take other work splits."""
    from kivi_stream import KiviStreamBatch
    B, H, KVH, D = 5, 16, 2, 128
    L0, steps = S + W + 9, 75
    gen = torch.Generator(device=device).manual_seed(100 + W)
    k = torch.randn(B, KVH, L0, D, generator=gen, device=device, dtype=torch.float16)
    v = torch.randn(B, KVH, L0, D, generator=gen, device=device, dtype=torch.float16)
    kn = torch.randn(steps, B, KVH, D, generator=gen, device=device, dtype=torch.float16)
    vn = torch.randn(steps, B, KVH, D, generator=gen, device=device, dtype=torch.float16) * 3
    q = torch.randn(steps, B, H, D, generator=gen, device=device, dtype=torch.float16)
    two = KiviStreamBatch.from_prefill(k, v, W)
    one = KiviStreamBatch.from_prefill(k, v, W)
    rng = np.random.default_rng(W)
    say(f"stream step_attend W={W}")
    for i in range(steps):
        active = torch.from_numpy(rng.random(B) < 0.8).to(device)
        if i % 5 == 0:
            active = None                      # every sequence takes the token
        two.append(kn[i], vn[i], active)
        o2 = host(two.attend(q[i]))
        o1 = host(one.step_attend(q[i], kn[i], vn[i], active))
        if W < 512:   # static work split: the same summation order
            np.testing.assert_array_equal(o1, o2, err_msg=str(i))
        else:
            assert max_abs(o1, o2) < ATTN_TOL, i
    for name in two.t:
        if name in ("k_ring", "v_ring"):   # free rows hold whatever the allocation held
            for b, (start, count) in enumerate(host(two.ring)):
                rows = [(start + i) % two.cap for i in range(count)]
                np.testing.assert_array_equal(host(one.t[name][b])[:, rows], host(two.t[name][b])[:, rows])
        else:
            np.testing.assert_array_equal(host(one.t[name]), host(two.t[name]), err_msg=name)
    for name in ("appended", "ring", "plan", "arrive"):
        np.testing.assert_array_equal(host(getattr(one, name)), host(getattr(two, name)), err_msg=name)
    assert int(host(one.appended).min()) >= 32


@pytest.mark.parametrize("G", [1, 4, 16])
def test_step_attend_query_group_sizes(G, device):
    """step_attend with G = H / KVH query heads per KV head other than 8
    (one head, a partial MFMA column block, all 16 columns): after every
    step (evictions included) the output matches the CPU oracle's stream
    state to half an fp16 ulp."""
    from kivi_stream import KiviStreamBatch
    B, KVH, D, W = 3, 2, 128, 256
    H = G * KVH
    L0, steps = S + W + 9, 40
    gen = torch.Generator(device=device).manual_seed(300 + G)
    kf = torch.randn(B, KVH, L0 + steps, D, generator=gen, device=device, dtype=torch.float16)
    vf = torch.randn(B, KVH, L0 + steps, D, generator=gen, device=device, dtype=torch.float16)
    q = torch.randn(steps, B, H, D, generator=gen, device=device, dtype=torch.float16)
    batch = KiviStreamBatch.from_prefill(kf[:, :, :L0], vf[:, :, :L0], W)
    kh, vh = host(kf), host(vf)
    say(f"stream step_attend G={G}")
    for i in range(steps):
        o = host(batch.step_attend(q[i], kf[:, :, L0 + i], vf[:, :, L0 + i]))
        if i % 7 != 3 and i != R // 4 + 3:
            continue
        oc, wlen = O.stream_cache(kh, vh, L0, L0 + i + 1, W)
        ref = O.quantized_attention(host(q[i]), wlen, oc, SCALE)
        assert max_abs(o, ref) < ATTN_TOL, i
        assert_nearly_rounded(o, ref)
