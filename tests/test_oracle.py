"""Pins the CPU oracle (oracle/kvdec_oracle.py) without running the reference.

Every oracle function is checked against something other than its own
formula: hand-computed known answers, exact rational arithmetic, brute force
on tiny inputs, a library routine (torch's scaled_dot_product_attention),
the reference tests' own independent constructions (streaming-llm mask,
strided unpack), and invariants chosen so that a plausible mistake (wrong
head mapping, dropped zero-point, banker's rounding, transposed packing,
off-by-one window) fails at least one of them.
"""

import math
from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle import kvdec_oracle as O

F32 = np.float32


def _rng(seed):
    return np.random.default_rng(seed)


# ----------------------------------------------------------------------------
# dense attention
# ----------------------------------------------------------------------------

def _brute_dense(q, k, v, scale):
    """Pure-Python loops, one head at a time (tiny shapes only)."""
    B, H, D = q.shape
    KVH, N = k.shape[1], k.shape[2]
    G = H // KVH
    out = np.zeros((B, H, D))
    for b in range(B):
        for h in range(H):
            kv = h // G
            logits = [sum(float(q[b, h, d]) * float(k[b, kv, n, d]) for d in range(D)) * scale
                      for n in range(N)]
            mx = max(logits)
            w = [math.exp(x - mx) for x in logits]
            den = sum(w)
            for d in range(D):
                out[b, h, d] = sum(w[n] * float(v[b, kv, n, d]) for n in range(N)) / den
    return out


def test_dense_matches_brute_force():
    r = _rng(1)
    q = r.standard_normal((2, 6, 5))
    k = r.standard_normal((2, 3, 7, 5))
    v = r.standard_normal((2, 3, 7, 5))
    got = O.dense_attention(q, k, v, 0.37)
    np.testing.assert_allclose(got, _brute_dense(q, k, v, 0.37), rtol=1e-12, atol=1e-12)


def test_dense_matches_torch_sdpa():
    r = _rng(2)
    B, H, KVH, N, D = 3, 16, 2, 300, 128
    q = r.standard_normal((B, H, D))
    k = r.standard_normal((B, KVH, N, D))
    v = r.standard_normal((B, KVH, N, D))
    scale = D**-0.5
    qt = torch.from_numpy(q)[:, :, None, :]                             # [B,H,1,D]
    kt = torch.from_numpy(k).repeat_interleave(H // KVH, dim=1)        # [B,H,N,D]
    vt = torch.from_numpy(v).repeat_interleave(H // KVH, dim=1)
    ref = torch.nn.functional.scaled_dot_product_attention(qt, kt, vt, scale=scale)[:, :, 0].numpy()
    np.testing.assert_allclose(O.dense_attention(q, k, v, scale), ref, rtol=1e-10, atol=1e-12)


def test_dense_invariants():
    r = _rng(3)
    B, H, KVH, N, D = 2, 8, 2, 40, 16
    q = r.standard_normal((B, H, D))
    k = r.standard_normal((B, KVH, N, D))
    v = r.standard_normal((B, KVH, N, D))
    # a single token: the output is that token's value row
    o1 = O.dense_attention(q, k[:, :, :1], v[:, :, :1], 0.3)
    np.testing.assert_allclose(o1, np.repeat(v[:, :, 0], H // KVH, axis=1), rtol=0, atol=1e-15)
    # constant keys: uniform weights, the output is the mean value row
    kc = np.broadcast_to(k[:, :, :1], k.shape)
    oc = O.dense_attention(q, kc, v, 0.3)
    np.testing.assert_allclose(oc, np.repeat(v.mean(axis=2), H // KVH, axis=1), atol=1e-13)
    # token permutation invariance
    perm = r.permutation(N)
    np.testing.assert_allclose(O.dense_attention(q, k[:, :, perm], v[:, :, perm], 0.3),
                               O.dense_attention(q, k, v, 0.3), atol=1e-13)
    # GQA: the query heads of KV head j equal single-head attention on KV head j
    G = H // KVH
    full = O.dense_attention(q, k, v, 0.3)
    for j in range(KVH):
        part = O.dense_attention(q[:, j * G:(j + 1) * G], k[:, j:j + 1], v[:, j:j + 1], 0.3)
        np.testing.assert_allclose(full[:, j * G:(j + 1) * G], part, atol=1e-15)


def test_masked_attention_ignores_invalid_contents():
    r = _rng(4)
    q = r.standard_normal((1, 4, 8))
    k = r.standard_normal((1, 2, 10, 8))
    v = r.standard_normal((1, 2, 10, 8))
    valid = np.array([1, 0, 1, 1, 0, 0, 1, 1, 1, 0], dtype=bool)
    a = O.masked_attention(q, k, v, valid, 0.5)
    k2, v2 = k.copy(), v.copy()
    k2[:, :, ~valid] = 1e4
    v2[:, :, ~valid] = np.nan
    np.testing.assert_array_equal(a, O.masked_attention(q, k2, v2, valid, 0.5))


# ----------------------------------------------------------------------------
# per-sequence lengths and paged caches
# ----------------------------------------------------------------------------

def test_dense_varlen_brute_force_and_garbage():
    """Each sequence equals brute force over its own first rows; rows past
    the length (NaN here) and a length of 0 (zeros) never leak in."""
    r = _rng(11)
    q = r.standard_normal((3, 4, 5))
    k = r.standard_normal((3, 2, 9, 5))
    v = r.standard_normal((3, 2, 9, 5))
    lens = [9, 4, 0]
    got = O.dense_attention_varlen(q, k, v, lens, 0.4)
    for b, n in enumerate(lens[:2]):
        want = _brute_dense(q[b:b + 1], k[b:b + 1, :, :n], v[b:b + 1, :, :n], 0.4)
        np.testing.assert_allclose(got[b:b + 1], want, rtol=1e-12, atol=1e-12)
    assert np.all(got[2] == 0)
    k2, v2 = k.copy(), v.copy()
    k2[1, :, 4:] = np.nan
    v2[1, :, 4:] = np.nan
    np.testing.assert_array_equal(O.dense_attention_varlen(q, k2, v2, lens, 0.4), got)


@pytest.mark.parametrize("layout", ["NHD", "HND"])
def test_paged_gather_known_answer(layout):
    """Token t of a sequence is row t % P of page table[t // P]: hand-placed
    rows come back in order, and a wrong index (page-major vs row-major,
    heads and tokens swapped) would not."""
    P, KVH, D, num_pages = 4, 2, 3, 5
    shape = (num_pages, P, KVH, D) if layout == "NHD" else (num_pages, KVH, P, D)
    pages = np.zeros(shape)
    table = [3, 0, 4]
    for t in range(10):
        for h in range(KVH):
            val = [1000 * h + t, -t, h]
            if layout == "NHD":
                pages[table[t // P], t % P, h] = val
            else:
                pages[table[t // P], h, t % P] = val
    got = O.gather_pages(pages, table, 10, layout)
    assert got.shape == (KVH, 10, D)
    for t in range(10):
        for h in range(KVH):
            assert list(got[h, t]) == [1000 * h + t, -t, h]


def test_paged_attention_equals_varlen_after_scatter():
    r = _rng(12)
    B, H, KVH, D, L, P = 3, 4, 2, 8, 21, 4
    q = r.standard_normal((B, H, D))
    k = r.standard_normal((B, KVH, L, D))
    v = r.standard_normal((B, KVH, L, D))
    lens = [21, 5, 0]
    nb = (L + P - 1) // P
    perm = r.permutation(B * nb)
    table = perm.reshape(B, nb)
    kp = r.standard_normal((B * nb, P, KVH, D)) * 1e3
    vp = r.standard_normal((B * nb, P, KVH, D)) * 1e3
    for b in range(B):
        for t in range(lens[b]):
            kp[table[b, t // P], t % P] = k[b, :, t]
            vp[table[b, t // P], t % P] = v[b, :, t]
    np.testing.assert_allclose(O.paged_attention(q, kp, vp, table, lens, 0.3),
                               O.dense_attention_varlen(q, k, v, lens, 0.3), rtol=1e-12, atol=1e-12)


def test_sparse_varlen_is_per_sequence_call():
    r = _rng(13)
    B, H, KVH, D, W, S = 3, 4, 2, 8, 6, 2
    q = r.standard_normal((B, H, D))
    kc = r.standard_normal((B, KVH, S + W, D))
    vc = r.standard_normal((B, KVH, S + W, D))
    lens = [1, 5, 40]
    got = O.sparse_attention_varlen(q, kc, vc, lens, W, S, 0.5)
    for b, n in enumerate(lens):
        want = O.sparse_attention_compacted(q[b:b + 1], kc[b:b + 1], vc[b:b + 1], n, W, S, 0.5)
        np.testing.assert_array_equal(got[b:b + 1], want)
    # length 1: only sink slot 0 is valid, so the output is V[slot 0]
    np.testing.assert_allclose(got[0], np.repeat(vc[0, :, 0], H // KVH, axis=0), rtol=1e-12)


def test_quantized_varlen_rows_are_independent():
    """Equal lengths give the batched call; each row at its own length is
    that row of the batched call at that length."""
    r = _rng(14)
    B, H, KVH, D, W, S = 3, 4, 2, 64, 160, 4
    kc = r.standard_normal((B, KVH, S + W, D)).astype(np.float16)
    vc = r.standard_normal((B, KVH, S + W, D)).astype(np.float16)
    cache = O.build_quantized_kv_cache(kc, vc)
    q = r.standard_normal((B, H, D)).astype(np.float16)
    same = O.quantized_attention_varlen(q, cache, [500] * B, W, 0.3)
    np.testing.assert_array_equal(same, O.quantized_attention_masked(q, cache, 500, W, 0.3))
    lens = [2, 100, 500]
    got = O.quantized_attention_varlen(q, cache, lens, W, 0.3)
    for b, n in enumerate(lens):
        np.testing.assert_array_equal(got[b], O.quantized_attention_masked(q, cache, n, W, 0.3)[b])


# ----------------------------------------------------------------------------
# StreamingLLM sink + window
# ----------------------------------------------------------------------------

def test_kv_indices_known_answers():
    # ramp-up: seq_len=2, W=256, S=4 -> only sink slots 0 and 1 are real
    _, valid = O.kv_indices(2, 0, 256, 4, 260)
    assert np.flatnonzero(valid).tolist() == [0, 1]
    # steady state: every slot valid
    _, valid = O.kv_indices(5000, 0, 256, 4, 260)
    assert valid.all()
    # seq_len=100, W=256: sink 0..3 and window slots holding positions 4..99
    # (slot 4 + i holds position (100 - 256) + i >= 4  <=>  i >= 160)
    _, valid = O.kv_indices(100, 0, 256, 4, 260)
    assert np.flatnonzero(valid).tolist() == [0, 1, 2, 3] + list(range(164, 260))
    # out-of-range slots are invalid and address slot 0
    addr, valid = O.kv_indices(5000, 256, 256, 4, 8)
    assert addr.tolist() == [256, 257, 258, 259, 0, 0, 0, 0]
    assert valid.tolist() == [True] * 4 + [False] * 4


@pytest.mark.parametrize("window", [0, 4, 32, 128])
def test_compacted_cache_equals_streaming_llm_mask(window):
    """The kernel's slot mapping over the compacted cache (linear and ring)
    gives the same attention as the streaming-llm mask over the full context,
    for every length from 1 through past the ramp-up."""
    r = _rng(10 + window)
    S, D = 4, 8
    Lmax = S + window + 40
    q = r.standard_normal((2, 4, D))
    kf = r.standard_normal((2, 2, Lmax, D))
    vf = r.standard_normal((2, 2, Lmax, D))
    for L in range(1, Lmax + 1):
        ref = O.sparse_attention_full(q, kf, vf, L, window, S, 0.4)
        kc, vc = O.build_compacted_cache(kf, vf, L, window, S)
        got = O.sparse_attention_compacted(q, kc, vc, L, window, S, 0.4, layout=0)
        np.testing.assert_allclose(got, ref, atol=1e-12, err_msg=f"linear L={L}")
        if window > 0:
            kr, vr = O.build_ring_cache(kf, vf, L, window, S)
            got = O.sparse_attention_compacted(q, kr, vr, L, window, S, 0.4, layout=1)
            np.testing.assert_allclose(got, ref, atol=1e-12, err_msg=f"ring L={L}")


def test_streaming_mask_known_answer():
    assert O.streaming_llm_mask(10, 3, 2).tolist() == [1, 1, 0, 0, 0, 0, 0, 1, 1, 1]
    assert O.streaming_llm_mask(5, 3, 2).all()


# ----------------------------------------------------------------------------
# KIVI quantizers
# ----------------------------------------------------------------------------

def _exact_codes(col):
    """Exact-rational evaluation of clamp(floor(x/s + 1/2) + z, 0, 3)."""
    xs = [Fraction(float(x)) for x in col]
    mn, mx = min(xs), max(xs)
    s = (mx - mn) / 3
    if s == 0:
        s = Fraction(1)
    z = math.floor(-mn / s + Fraction(1, 2))
    out = []
    for x in xs:
        c = math.floor(x / s + Fraction(1, 2)) + z
        out.append(min(max(c, 0), 3))
    return np.array(out), s, z


def _unpack_k_codes(packed, N):
    p = packed.astype(np.int32)
    codes = np.zeros(p.shape[:2] + (N,) + p.shape[3:], dtype=np.int32)
    for j in range(4):
        codes[:, :, j::4] = (p >> (2 * j)) & 3
    return codes


def test_quantize_k_linear_ramp_known_answer():
    # channel values 0..31: mn=0, mx=31, s=31/3, z=0, code = floor(3x/31 + 1/2)
    # (no exact ties: 31(2k-1)/6 is never an integer)
    x = np.arange(32, dtype=F32)[None, None, :, None].repeat(2, axis=3)
    packed, scale, zero = O.quantize_k(x)
    codes = _unpack_k_codes(packed, 32)[0, 0, :, 0]
    expect = [0] * 6 + [1] * 10 + [2] * 10 + [3] * 6
    assert codes.tolist() == expect
    assert float(scale[0, 0, 0, 0]) == float(np.float16(F32(31) / F32(3)))
    assert float(zero[0, 0, 0, 0]) == 0.0


def test_quantize_round_half_up_ties():
    # group spanning [0, 3] -> s = 1 exactly, z = 0; x = k + 0.5 is an exact tie
    col = np.array([0.0, 3.0, 0.5, 1.5, 2.5, 1.0, 2.0] + [0.0] * 25, dtype=F32)
    x = col[None, None, :, None]
    codes = _unpack_k_codes(O.quantize_k(x)[0], 32)[0, 0, :7, 0]
    assert codes.tolist() == [0, 3, 1, 2, 3, 1, 2]     # banker's rounding would give 0,2,2 for the ties
    # the same group along channels for V
    v = col[None, None, None, :]
    vp = O.quantize_v(v)[0]
    vcodes = [(int(vp[0, 0, 0, i // 4]) >> (2 * (i % 4))) & 3 for i in range(7)]
    assert vcodes == [0, 3, 1, 2, 3, 1, 2]


def test_quantize_constant_and_positive_groups():
    # constant group: s = 0 -> 1, z = floor(-c + 0.5)
    for c in (0.7, -2.3, 0.5, 0.0, 100.25):
        x = np.full((1, 1, 32, 1), c, dtype=F32)
        packed, scale, zero = O.quantize_k(x)
        assert float(scale[0, 0, 0, 0]) == 1.0
        z = math.floor(-c + 0.5)
        assert float(zero[0, 0, 0, 0]) == float(np.float16(z))
        code = min(max(math.floor(c + 0.5) + z, 0), 3)
        assert (_unpack_k_codes(packed, 32) == code).all()
    # all-positive narrow group: negative zero-point
    col = np.linspace(5.0, 6.0, 32, dtype=F32)
    packed, scale, zero = O.quantize_k(col[None, None, :, None])
    ec, s, z = _exact_codes(col)
    assert z == -15
    assert float(zero[0, 0, 0, 0]) == -15.0
    assert (_unpack_k_codes(packed, 32)[0, 0, :, 0] == ec).all()


def test_quantize_matches_exact_rational_arithmetic():
    """Random groups (with x10 outlier channels): float32 codes equal the
    exact-rational codes except where x/s + 1/2 is within float32 rounding of
    an integer."""
    r = _rng(20)
    x = r.standard_normal((1, 2, 64, 16)).astype(F32)
    x[..., [3, 11]] *= 10
    packed, scale, zero = O.quantize_k(x)
    codes = _unpack_k_codes(packed, 64)
    mismatches = 0
    for h in range(2):
        for g in range(2):
            for d in range(16):
                col = x[0, h, 32 * g:32 * g + 32, d]
                ec, s, z = _exact_codes(col)
                got = codes[0, h, 32 * g:32 * g + 32, d]
                assert float(scale[0, h, g, d]) == float(np.float16(float(s)))
                assert float(zero[0, h, g, d]) == float(np.float16(z))
                for i in np.flatnonzero(got != ec):
                    t = Fraction(float(col[i])) / s + Fraction(1, 2)
                    assert abs(t - round(t)) < Fraction(1, 10**5), "mismatch away from a boundary"
                    mismatches += 1
    assert mismatches <= 2


def test_quantize_v_matches_exact_rational_arithmetic():
    r = _rng(21)
    x = r.standard_normal((1, 1, 24, 64)).astype(F32)
    packed, scale, zero = O.quantize_v(x)
    for t in range(24):
        for g in range(2):
            col = x[0, 0, t, 32 * g:32 * g + 32]
            ec, s, z = _exact_codes(col)
            got = [(int(packed[0, 0, t, 8 * g + i // 4]) >> (2 * (i % 4))) & 3 for i in range(32)]
            assert got == ec.tolist()
            assert float(scale[0, 0, t, g]) == float(np.float16(float(s)))
            assert float(zero[0, 0, t, g]) == float(np.float16(z))


def test_packing_layout_known_bytes():
    # K: tokens 0..3 of one channel with codes [1, 2, 3, 0] -> 1 | 2<<2 | 3<<4 = 57
    col = np.array([1.0, 2.0, 3.0, 0.0] + [0.0] * 27 + [3.0], dtype=F32)   # mn 0, mx 3, s 1
    packed = O.quantize_k(col[None, None, :, None])[0]
    assert int(packed[0, 0, 0, 0]) == 57
    # V: channels 0..3 of one token with codes [3, 0, 2, 1] -> 3 | 0 | 2<<4 | 1<<6 = 99
    row = np.array([3.0, 0.0, 2.0, 1.0] + [0.0] * 28, dtype=F32)
    packed = O.quantize_v(row[None, None, None, :])[0]
    assert int(packed[0, 0, 0, 0]) == 99


def test_roundtrip_within_reference_tolerance():
    """The reference's round-trip bound (test_quantize_correctness.py:46-55)."""
    r = _rng(22)
    for N in (32, 256):
        k = r.standard_normal((1, 1, N, 128)).astype(F32)
        packed, s, z = O.quantize_k(k)
        rec = O.unpack_dequant(packed, s, z, N, pack_axis=2)
        grouped = k.reshape(1, 1, N // 32, 32, 128)
        tol = (grouped.max(axis=3) - grouped.min(axis=3)).max() / 2 + 1e-3
        assert np.abs(rec - k).max() < tol
        v = r.standard_normal((1, 1, N, 128)).astype(F32)
        packed, s, z = O.quantize_v(v)
        rec = O.unpack_dequant(packed, s, z, 128, pack_axis=3)
        grouped = v.reshape(1, 1, N, 4, 32)
        tol = (grouped.max(axis=4) - grouped.min(axis=4)).max() / 2 + 1e-3
        assert np.abs(rec - v).max() < tol


def test_fp16_and_fp32_inputs_give_identical_codes():
    r = _rng(23)
    x16 = r.standard_normal((2, 2, 64, 128)).astype(np.float16)
    for fn in (O.quantize_k, O.quantize_v):
        a = fn(x16)
        b = fn(x16.astype(F32))
        for u, w in zip(a, b):
            np.testing.assert_array_equal(u, w)


def test_sink_padding_keeps_real_range():
    """Padding 4 sink tokens to 32 by repeating token 0 leaves the per-channel
    min/max of the real tokens unchanged (quant_kernel.py:595-606)."""
    r = _rng(24)
    kc = r.standard_normal((1, 2, 4 + 256, 128)).astype(np.float16)
    vc = r.standard_normal((1, 2, 4 + 256, 128)).astype(np.float16)
    cache = O.build_quantized_kv_cache(kc, vc)
    real = kc[:, :, :4].astype(F32)
    s_expect = (real.max(axis=2) - real.min(axis=2)) / F32(3)
    s_expect = np.where(s_expect == 0, F32(1), s_expect)
    np.testing.assert_array_equal(cache["k_sink_scale"][:, :, 0], s_expect.astype(np.float16))
    np.testing.assert_array_equal(cache["k_residual"], kc[:, :, -128:])
    assert cache["k_win_packed"].shape == (1, 2, 32, 128)
    assert cache["v_win_packed"].shape == (1, 2, 128, 32)
    assert set(cache) == set(O.CACHE_KEYS)


# ----------------------------------------------------------------------------
# tile dequantizers
# ----------------------------------------------------------------------------

def test_dequant_tiles_equal_unpack_when_aligned():
    """The reference's isolated-dequant check (test_dequantize_tile_isolated.py:66-120)."""
    r = _rng(30)
    k = r.standard_normal((1, 1, 256, 128)).astype(F32)
    pk, sk, zk = O.quantize_k(k)
    ref = O.unpack_dequant(pk, sk, zk, 256, pack_axis=2)
    np.testing.assert_array_equal(O.dequant_k_tile(pk, sk, zk, 0, 64, 8), ref[:, :, :128])
    np.testing.assert_array_equal(O.dequant_k_tile(pk, sk, zk, 128, 64, 8), ref[:, :, 128:])
    v = r.standard_normal((1, 1, 256, 128)).astype(F32)
    pv, sv, zv = O.quantize_v(v)
    ref = O.unpack_dequant(pv, sv, zv, 128, pack_axis=3)
    np.testing.assert_array_equal(O.dequant_v_tile(pv, sv, zv, 0, 256), ref[:, :, :128])
    np.testing.assert_array_equal(O.dequant_v_tile(pv, sv, zv, 100, 256), ref[:, :, 100:228])


def test_dequant_tile_clamping():
    r = _rng(31)
    k = r.standard_normal((1, 1, 64, 8)).astype(F32)
    pk, sk, zk = O.quantize_k(k)
    ref = O.unpack_dequant(pk, sk, zk, 64, pack_axis=2)
    # tok_start = -4 (the sink/window-old composer): tokens t >= 4 read token t-4,
    # tokens 0..3 clamp to byte 0 and keep their own sub-position t
    out = O.dequant_k_tile(pk, sk, zk, -4, 16, 2, block_n=32)
    np.testing.assert_array_equal(out[:, :, 4:], ref[:, :, :28])
    np.testing.assert_array_equal(out[:, :, :4], ref[:, :, :4])
    # past the end: every token reads the last byte row with its own sub-position
    out = O.dequant_k_tile(pk, sk, zk, 64, 16, 2, block_n=8)
    np.testing.assert_array_equal(out[:, :, 0], ref[:, :, 60])
    np.testing.assert_array_equal(out[:, :, 5], ref[:, :, 61])
    v = r.standard_normal((1, 1, 40, 32)).astype(F32)
    pv, sv, zv = O.quantize_v(v)
    refv = O.unpack_dequant(pv, sv, zv, 32, pack_axis=3)
    out = O.dequant_v_tile(pv, sv, zv, 30, 40, block_n=16)
    np.testing.assert_array_equal(out[:, :, :10], refv[:, :, 30:40])
    np.testing.assert_array_equal(out[:, :, 10:], np.repeat(refv[:, :, 39:40], 6, axis=2))


# ----------------------------------------------------------------------------
# fused quantized decode
# ----------------------------------------------------------------------------

def test_quantized_attention_composition_and_masking():
    r = _rng(40)
    B, H, KVH, D, S, R = 2, 16, 2, 128, 4, 128
    for W in (128, 256):
        q = r.standard_normal((B, H, D)).astype(np.float16)
        kc = r.standard_normal((B, KVH, S + W, D)).astype(np.float16)
        vc = r.standard_normal((B, KVH, S + W, D)).astype(np.float16)
        cache = O.build_quantized_kv_cache(kc, vc)
        comp = O.quantized_attention(q, W - R, cache, D**-0.5)
        # steady state: the masked (kernel) form equals the composition
        steady = O.quantized_attention_masked(q, cache, S + W + 1000, W, D**-0.5)
        np.testing.assert_allclose(steady, comp, atol=1e-14)
        # composition == dense attention over the dequantized cache, and the
        # residual regime is passed through exactly
        k, v = O.dequantized_regimes(cache, W - R)
        np.testing.assert_array_equal(k[:, :, -R:], kc[:, :, -R:].astype(F32))
        np.testing.assert_allclose(comp, O.dense_attention(q, k, v, D**-0.5), atol=0)
        # quantization error of the window-old regime stays within the
        # reference's round-trip bound (half the largest group range)
        if W > R:
            old_k = kc[:, :, S:S + W - R].astype(F32)
            g = old_k.reshape(B, KVH, (W - R) // 32, 32, D)
            tol = (g.max(axis=3) - g.min(axis=3)).max() / 2 + 1e-3
            assert np.abs(k[:, :, S:S + W - R] - old_k).max() < tol
        # ramp-up: only the slots kv_indices marks valid are attended
        L = 50
        ramp = O.quantized_attention_masked(q, cache, L, W, D**-0.5)
        valid = O.kv_indices(L, 0, W, S, S + W)[1]
        np.testing.assert_allclose(ramp, O.masked_attention(q, k, v, valid, D**-0.5), atol=0)


# ----------------------------------------------------------------------------
# decode-time (streaming) KIVI cache
# ----------------------------------------------------------------------------

def _stream_positions(prefill_len, n_appends, window, sink=4, residual=128, group=32):
    """Token-by-token model of the streaming cache's attended positions: the
    sink, the window-old groups (oldest first) and the fp16 residual.  Each
    append joins the residual; when it holds residual + group tokens its
    oldest `group` form a new window-old group and the oldest window-old
    group leaves (with no window-old part the block leaves at once)."""
    sinks = list(range(sink))
    groups = [list(range(s, s + group))
              for s in range(prefill_len - window, prefill_len - residual, group)]
    res = list(range(prefill_len - residual, prefill_len))
    for p in range(prefill_len, prefill_len + n_appends):
        res.append(p)
        if len(res) == residual + group:
            block, res = res[:group], res[group:]
            if groups:
                groups = groups[1:] + [block]
    return sinks, groups, res


def _padded_sink(x, sink=4, group=32):
    real = x[:, :, :sink]
    return np.concatenate([real, np.repeat(real[:, :, :1], group - sink, axis=2)], axis=2)


@pytest.mark.parametrize("W", [128, 160, 256])
def test_stream_cache_follows_token_by_token_model(W):
    """stream_cache after n = 0..200 appends holds exactly the positions the
    token-by-token model attends, each regime quantized from those positions;
    at every eviction point (n a multiple of 32) it is the reference
    builder's output on the compacted cache [sink, L - W .. L)."""
    S, R = 4, 128
    L0 = S + W + 37
    rng = _rng(500 + W)
    kf = rng.standard_normal((1, 2, L0 + 201, 128)).astype(np.float16)
    vf = rng.standard_normal((1, 2, L0 + 201, 128)).astype(np.float16)
    sink_k = O.quantize_k(_padded_sink(kf).astype(F32))
    sink_v = O.quantize_v(_padded_sink(vf).astype(F32))
    for n in range(201):
        L = L0 + n
        cache, wlen = O.stream_cache(kf, vf, L0, L, W)
        sinks, groups, res = _stream_positions(L0, n, W)
        assert wlen == W - R == 32 * len(groups)
        assert len(res) == R + n % 32 and res[-1] == L - 1
        # every position attended exactly once, none twice
        attended = sinks + sum(groups, []) + res
        assert len(set(attended)) == len(attended) == S + W + n % 32
        np.testing.assert_array_equal(cache["k_residual"], kf[:, :, res])
        np.testing.assert_array_equal(cache["v_residual"], vf[:, :, res])
        for name, (p, s, z) in (("k_sink", sink_k), ("v_sink", sink_v)):
            np.testing.assert_array_equal(cache[name + "_packed"], p)
            np.testing.assert_array_equal(cache[name + "_scale"], s)
            np.testing.assert_array_equal(cache[name + "_zero"], z)
        if groups:
            pos = sum(groups, [])
            for name, fn, src in (("k_win", O.quantize_k, kf), ("v_win", O.quantize_v, vf)):
                p, s, z = fn(src[:, :, pos].astype(F32))
                np.testing.assert_array_equal(cache[name + "_packed"], p)
                np.testing.assert_array_equal(cache[name + "_scale"], s)
                np.testing.assert_array_equal(cache[name + "_zero"], z)
        if n % 32 == 0:
            comp_k = np.concatenate([kf[:, :, :S], kf[:, :, L - W:L]], axis=2)
            comp_v = np.concatenate([vf[:, :, :S], vf[:, :, L - W:L]], axis=2)
            built = O.build_quantized_kv_cache(comp_k, comp_v)
            for key in O.CACHE_KEYS:
                np.testing.assert_array_equal(cache[key], built[key], err_msg=f"{key} n={n}")


# ----------------------------------------------------------------------------
# torch restatement used for the CPU baseline (oracle/torch_ref.py)
# ----------------------------------------------------------------------------

def test_torch_ref_matches_numpy_oracle():
    """The torch CPU restatement that bench.py times as the CPU baseline
    computes what the (independently pinned) numpy oracle computes: dense,
    sink + window through ramp-up, unpack/dequant of both layouts, and the
    quantized composition (float32 vs float64: 1e-5)."""
    from oracle import torch_ref as T
    rng = _rng(900)
    t = torch.from_numpy
    q = rng.standard_normal((2, 16, 128)).astype(F32)
    k = rng.standard_normal((2, 2, 300, 128)).astype(F32)
    v = rng.standard_normal((2, 2, 300, 128)).astype(F32)
    sc = 128 ** -0.5
    np.testing.assert_allclose(T.dense_attention(t(q), t(k), t(v), sc).numpy(),
                               O.dense_attention(q, k, v, sc), atol=1e-5)
    S, W = 4, 256
    kc, vc = k[:, :, :S + W], v[:, :, :S + W]
    for L in (1, 3, 4, 5, 100, 259, 260, 261, 5000):
        want = O.sparse_attention_compacted(q, kc, vc, L, W, S, sc)
        got = T.sparse_attention(t(q), t(kc), t(vc), L, W, S, sc).numpy()
        np.testing.assert_allclose(got, want, atol=1e-5, err_msg=str(L))
        np.testing.assert_array_equal(T.slot_validity(L, W, S, S + W).numpy(), O.slot_validity(L, W, S))
    cache = O.build_quantized_kv_cache(kc.astype(np.float16), vc.astype(np.float16))
    for name, n, axis in (("k_win", W - 128, 2), ("v_win", 128, 3)):
        got = T.unpack_dequant(t(cache[name + "_packed"]), t(cache[name + "_scale"]), t(cache[name + "_zero"]),
                               n, axis).numpy()
        want = O.unpack_dequant(cache[name + "_packed"], cache[name + "_scale"], cache[name + "_zero"], n, axis)
        np.testing.assert_array_equal(got, want)
    tc = {key: t(np.ascontiguousarray(val)) for key, val in cache.items()}
    q16 = q.astype(np.float16)
    np.testing.assert_allclose(T.quantized_attention(t(q16), W - 128, tc, sc).numpy(),
                               O.quantized_attention(q16, W - 128, cache, sc), atol=1e-5)


# ----------------------------------------------------------------------------
# quantizers of any code width (the reference's BITS / GROUP_SIZE parameters)
# ----------------------------------------------------------------------------

def _exact_codes_q(col, qmax):
    """Exact-rational clamp(floor(x/s + 1/2) + z, 0, qmax), s = (mx - mn) / qmax."""
    xs = [Fraction(float(x)) for x in col]
    mn, mx = min(xs), max(xs)
    s = (mx - mn) / qmax
    if s == 0:
        s = Fraction(1)
    z = math.floor(-mn / s + Fraction(1, 2))
    return [min(max(math.floor(x / s + Fraction(1, 2)) + z, 0), qmax) for x in xs], s, z


def _field(byte, j, bits):
    """Code j of a byte, bit by bit (independent of the oracle's shift/mask)."""
    return sum(((int(byte) >> (j * bits + i)) & 1) << i for i in range(bits))


@pytest.mark.parametrize("bits,group", [(1, 16), (3, 16), (4, 32), (4, 64), (8, 16), (2, 64), (5, 8)])
def test_quantize_any_width_matches_exact_rational_arithmetic(bits, group):
    qmax, pf = (1 << bits) - 1, 8 // bits
    r = _rng(40 + bits)
    N, D = 2 * group, 128
    x = r.standard_normal((1, 1, N, D)).astype(F32)
    x[..., 7] *= 10
    packed, scale, zero = O.quantize_k(x, group, bits)
    assert packed.shape == (1, 1, N // pf, D) and scale.shape == (1, 1, N // group, D)
    near = 0
    for g in range(N // group):
        for d in range(0, D, 9):
            col = x[0, 0, group * g:group * (g + 1), d]
            ec, s, z = _exact_codes_q(col, qmax)
            assert float(scale[0, 0, g, d]) == float(np.float16(float(s)))
            assert float(zero[0, 0, g, d]) == float(np.float16(z))
            for t in range(group):
                tok = group * g + t
                got = _field(packed[0, 0, tok // pf, d], tok % pf, bits)
                if got != ec[t]:
                    v = Fraction(float(col[t])) / s + Fraction(1, 2)
                    assert abs(v - round(v)) < Fraction(1, 10**5), "mismatch away from a boundary"
                    near += 1
    assert near <= 2
    v = r.standard_normal((1, 1, 6, D)).astype(F32)
    packed, scale, zero = O.quantize_v(v, group, bits)
    assert packed.shape == (1, 1, 6, D // pf) and scale.shape == (1, 1, 6, D // group)
    for t in range(6):
        for g in range(D // group):
            col = v[0, 0, t, group * g:group * (g + 1)]
            ec, s, z = _exact_codes_q(col, qmax)
            got = [_field(packed[0, 0, t, (group * g + c) // pf], (group * g + c) % pf, bits) for c in range(group)]
            assert got == ec
            assert float(scale[0, 0, t, g]) == float(np.float16(float(s)))


def test_quantize_any_width_known_bytes():
    # bits 1: a group of 8 tokens spanning [0, 1] (s = 1, z = 0): codes = values
    col = np.array([1, 0, 1, 1, 0, 0, 0, 1], dtype=F32)
    assert int(O.quantize_k(col[None, None, :, None], 8, 1)[0][0, 0, 0, 0]) == 1 + 4 + 8 + 128
    # bits 4, two channels per byte: a group of 16 spanning [0, 15]
    row = np.array([15, 3] + [0] * 14, dtype=F32)
    assert int(O.quantize_v(row[None, None, None, :], 16, 4)[0][0, 0, 0, 0]) == 15 | 3 << 4
    # bits 3, two codes per byte at bits 0 and 3: a group of 8 spanning [0, 7]
    row = np.array([5, 7, 0, 0, 0, 0, 0, 0], dtype=F32)
    assert int(O.quantize_v(row[None, None, None, :], 8, 3)[0][0, 0, 0, 0]) == 5 | 7 << 3
    # bits 8: the byte is the code
    col = np.arange(16, dtype=F32) * 17    # 0 .. 255, s = 1
    assert O.quantize_k(col[None, None, :, None], 16, 8)[0][0, 0, :, 0].tolist() == (np.arange(16) * 17).tolist()
    with pytest.raises(ValueError):
        O.quantize_k(np.zeros((1, 1, 8, 4), F32), 4, 1)     # half a byte of 1-bit codes per group


def test_quantized_attention_any_width_is_exact_on_integer_data():
    """8-bit codes of integer data whose groups span 0..255 dequantize
    exactly (s = 1, z = 0), so the regime composition must equal dense
    attention over the original cache: pins the sink padding, window-old and
    residual slots of the generic width path."""
    r = _rng(50)
    B, KVH, G, D, S, W, R, grp = 1, 2, 4, 128, 4, 96, 32, 16
    n = S + W
    kc = r.integers(0, 256, (B, KVH, n, D)).astype(F32)
    vc = r.integers(0, 256, (B, KVH, n, D)).astype(F32)
    kc[:, :, :S] = kc[:, :, :1]            # the sink group is padded with token 0
    kc[:, :, 0, :] = 0
    kc[:, :, 1, :] = 255
    for g0 in range(S, S + W - R, grp):    # every window-old K group spans 0..255
        kc[:, :, g0, :] = 0
        kc[:, :, g0 + 1, :] = 255
    for c in range(0, D, grp):             # every V channel group spans 0..255
        vc[:, :, :, c] = 0
        vc[:, :, :, c + 1] = 255
    kc16, vc16 = kc.astype(np.float16), vc.astype(np.float16)
    cache = O.build_quantized_kv_cache(kc16, vc16, residual_size=R, sink=S, group_size=grp, bits=8)
    q = (r.standard_normal((B, KVH * G, D)) / 64).astype(np.float16)
    got = O.quantized_attention(q, W - R, cache, SCALE_T, sink=S, group_size=grp, bits=8)
    want = O.dense_attention(q, kc16, vc16, SCALE_T)
    assert np.abs(got - want).max() < 1e-9


SCALE_T = 128**-0.5
