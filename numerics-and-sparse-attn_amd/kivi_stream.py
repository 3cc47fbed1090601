"""Decode-time KIVI cache on MI355X: append one token per step, quantize on
eviction, attend with the fused sink + window + KIVI-2bit decode.

The reference builds its quantized cache once, from a compacted
[B, KVH, sink + window, D] cache (build_quantized_kv_cache,
quant_kernel.py:584-622), and leaves the decode loop's write side open.  This
module keeps the same regimes as a streaming state:

  sink        the first `sink` tokens, quantized once as one padded group
              (token 0 repeated), exactly as the reference builds it;
  window-old  a ring of (window - residual) / 32 quantized groups;
  residual    an fp16 ring of residual + 32 rows holding the most recent
              residual .. residual + 31 tokens.

Each new token goes into the residual ring.  When the ring holds
residual + 32 tokens, its oldest 32-row block is quantized (K per channel,
V per token, the quantizers' exact formulas) into the slot of the oldest
window-old group, which leaves the window.

Two ways to add a token: append(k_new, v_new) copies it in; reserve()
returns [B, KVH, D] views of the ring row the token belongs in, so that the
kernel producing K and V (the projection) writes them there directly and the
decode loop costs only attend() plus one quantization every 32 tokens.  So the attended window is
window .. window + 31 tokens: sink + every window-old group + the residual
ring's valid rows.  Right after an eviction (residual count == residual) the
state holds exactly what build_quantized_kv_cache builds from the compacted
cache at that length: the same window-old groups (same token sets, so the
same codes, in ring order) and the same residual tokens.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

import _checks
import _kvdec as K
from constants import D_HEAD, GROUP_SIZE, QUANT_BITS, RESIDUAL_SIZE, SINK_SIZE
from quant_kernel import quantize_k_cache, quantize_v_cache

_WIN_KEYS = ("k_win_packed", "k_win_scale", "k_win_zero", "v_win_packed", "v_win_scale", "v_win_zero")
_SINK_KEYS = ("k_sink_packed", "k_sink_scale", "k_sink_zero", "v_sink_packed", "v_sink_scale",
              "v_sink_zero")


@dataclass
class RingState:
    """Host-side bookkeeping of the residual ring and the window-old ring."""
    cap: int            # residual ring rows (residual + group)
    residual: int
    n_groups: int       # window-old groups
    start: int = 0      # oldest valid residual row
    count: int = 0      # valid residual rows
    next_slot: int = 0  # window-old slot holding the oldest group
    group: int = GROUP_SIZE

    def append(self):
        """Advance by one token; returns (row, evict_block, evict_slot), with
        evict_block = -1 when no block is quantized on this step."""
        row = (self.start + self.count) % self.cap
        self.count += 1
        evict_block, evict_slot = -1, -1
        if self.count == self.cap:
            evict_block = self.start // self.group
            evict_slot = self.next_slot if self.n_groups else -1
            self.start = (self.start + self.group) % self.cap
            self.count -= self.group
            if self.n_groups:
                self.next_slot = (self.next_slot + 1) % self.n_groups
        return row, evict_block, evict_slot


def _prefill_state(k, v, window, sink, residual_size):
    """The quantized sink group, the window-old groups and the residual ring
    (rows 0 .. residual - 1 = the last residual prefill tokens) of a
    [B, KVH, L, D] fp16 prefill."""
    _checks.require_gpu_tensor("k", k, ndim=4, contiguous=False)   # sliced, then copied
    _checks.require_gpu_tensor("v", v, ndim=4, contiguous=False)
    _checks.require_same_device(("k", k), ("v", v))
    B, KVH, L, D = k.shape
    _checks.require_shape("v", v, (B, KVH, L, D))
    R, G = int(residual_size), GROUP_SIZE
    window, sink = int(window), int(sink)
    if window < R or (window - R) % G or R % G or not 1 <= sink <= G:
        raise ValueError(f"unsupported window={window} / residual={R} / sink={sink}")
    if L < sink + window:
        raise ValueError(f"prefill length {L} < sink + window = {sink + window}")
    pad = G - sink
    t = {}

    def padded(x):
        real = x[:, :, :sink]
        return torch.cat([real, real[:, :, :1].expand(-1, -1, pad, -1)], dim=2).contiguous()

    t["k_sink_packed"], t["k_sink_scale"], t["k_sink_zero"] = quantize_k_cache(padded(k))
    t["v_sink_packed"], t["v_sink_scale"], t["v_sink_zero"] = quantize_v_cache(padded(v))
    win = k[:, :, L - window:L - R].contiguous()
    t["k_win_packed"], t["k_win_scale"], t["k_win_zero"] = quantize_k_cache(win)
    win = v[:, :, L - window:L - R].contiguous()
    t["v_win_packed"], t["v_win_scale"], t["v_win_zero"] = quantize_v_cache(win)
    cap = R + G
    t["k_ring"] = torch.empty(B, KVH, cap, D, dtype=torch.float16, device=k.device)
    t["v_ring"] = torch.empty(B, KVH, cap, D, dtype=torch.float16, device=k.device)
    t["k_ring"][:, :, :R] = k[:, :, L - R:]
    t["v_ring"][:, :, :R] = v[:, :, L - R:]
    return t


class KiviStreamCache:
    """Streaming KIVI cache of B sequences that advance together (one scalar
    length, as in the reference's decode calls)."""

    def __init__(self, tensors, ring: RingState, seq_len: int, window: int, sink: int):
        self.t = tensors
        self.ring = ring
        self.seq_len = seq_len
        self.window = window
        self.sink = sink

    @classmethod
    def from_prefill(cls, k, v, window, sink=SINK_SIZE, residual_size=RESIDUAL_SIZE):
        """k, v: [B, KVH, L, D] fp16 of positions 0..L-1 (a prefill), with
        L >= sink + window (steady state: every window slot is filled)."""
        t = _prefill_state(k, v, window, sink, residual_size)
        R, G = int(residual_size), GROUP_SIZE
        ring = RingState(cap=R + G, residual=R, n_groups=(int(window) - R) // G, count=R)
        return cls(t, ring, k.shape[2], int(window), int(sink))

    @property
    def shape(self):
        B, KVH, cap, D = self.t["k_ring"].shape
        return B, KVH, D

    def reserve(self):
        """Advance by one token and return (k_view, v_view), the [B, KVH, D]
        ring-row views to write its K and V into before the next attend().
        A block eviction due at this token is enqueued here, before the
        caller's writes (it never touches the returned row)."""
        B, KVH, D = self.shape
        row, blk, slot = self.ring.append()
        if blk >= 0:
            win = (K._vp * 6)(*[K.ptr(self.t[n]) if self.t[n].numel() else None for n in _WIN_KEYS])
            rc = K.lib.kvdec_kivi_stream_append(None, None, K.ptr(self.t["k_ring"]),
                                                K.ptr(self.t["v_ring"]), win, B, KVH, D, self.ring.cap,
                                                row, blk, slot, self.ring.n_groups, GROUP_SIZE,
                                                QUANT_BITS, K.stream_of(self.t["k_ring"]))
            K.check(rc, "KiviStreamCache.reserve")
        self.seq_len += 1
        return self.t["k_ring"][:, :, row], self.t["v_ring"][:, :, row]

    def append(self, k_new, v_new):
        """Append the token at position seq_len: k_new, v_new [B, KVH, D]
        (or [B, KVH, 1, D]) fp16."""
        B, KVH, D = self.shape
        k_new = k_new.reshape(B, KVH, D)
        v_new = v_new.reshape(B, KVH, D)
        k_new, v_new = k_new.contiguous(), v_new.contiguous()
        _checks.require_gpu_tensor("k_new", k_new, ndim=3)
        _checks.require_gpu_tensor("v_new", v_new, ndim=3)
        _checks.require_same_device(("k_new", k_new), ("v_new", v_new), ("k_ring", self.t["k_ring"]))
        row, blk, slot = self.ring.append()
        win = (K._vp * 6)(*[K.ptr(self.t[n]) if self.t[n].numel() else None for n in _WIN_KEYS])
        rc = K.lib.kvdec_kivi_stream_append(K.ptr(k_new), K.ptr(v_new), K.ptr(self.t["k_ring"]),
                                            K.ptr(self.t["v_ring"]), win, B, KVH, D, self.ring.cap,
                                            row, blk, slot, self.ring.n_groups, GROUP_SIZE,
                                            QUANT_BITS, K.stream_of(k_new))
        K.check(rc, "KiviStreamCache.append")
        self.seq_len += 1

    def attend(self, q, sm_scale=None):
        """Decode attention of q [B, H, D] fp16 over the cache; returns o
        [B, H, D] fp16."""
        B, KVH, D = self.shape
        _checks.require_gpu_tensor("q", q, ndim=3)
        _checks.require_shape("q", q, (B, q.shape[1], D))
        _checks.require_same_device(("q", q), ("k_ring", self.t["k_ring"]))
        o = torch.empty_like(q)
        if sm_scale is None:
            sm_scale = D_HEAD**-0.5
        names = _SINK_KEYS + _WIN_KEYS
        arr = (K._vp * 12)(*[K.ptr(self.t[n]) if self.t[n].numel() else None for n in names])
        r = self.ring
        rc = K.lib.kvdec_kivi_stream_decode(K.ptr(q), K.ptr(self.t["k_ring"]), K.ptr(self.t["v_ring"]),
                                            arr, K.ptr(o), B, q.shape[1], KVH, self.sink, r.n_groups,
                                            r.cap, r.start, r.count, GROUP_SIZE, QUANT_BITS,
                                            float(sm_scale), K.stream_of(q))
        K.check(rc, "KiviStreamCache.attend")
        return o

    def window_old_slots(self):
        """Window-old ring slots from the oldest group to the newest."""
        n = self.ring.n_groups
        return [(self.ring.next_slot + i) % n for i in range(n)]

    def residual_rows(self):
        """Valid residual ring rows from the oldest token to the newest."""
        r = self.ring
        return [(r.start + i) % r.cap for i in range(r.count)]


class KiviStreamBatch:
    """Decode-time KIVI cache whose B sequences keep separate ring states,
    for continuous batching: a sequence can take a new prefill in its batch
    slot (admit) and sit out steps (the `active` mask), while the others go
    on.  The bookkeeping lives on the GPU (a token count per sequence, from
    which each step's ring row, eviction and ring state follow, kept by the
    append kernel itself), so a step is two launches and no host round
    trip: the step (append, quantize-on-evict, bookkeeping) and attend, or
    one (step_attend).  Each sequence's state equals
    a KiviStreamCache of that sequence alone after the same appends."""

    def __init__(self, tensors, window, sink, residual):
        self.t = tensors
        self.window, self.sink, self.residual = int(window), int(sink), int(residual)
        self.cap = self.residual + GROUP_SIZE
        self.n_groups = (self.window - self.residual) // GROUP_SIZE
        B = tensors["k_ring"].shape[0]
        dev = tensors["k_ring"].device
        self.appended = torch.zeros(B, dtype=torch.int32, device=dev)   # tokens since each prefill
        self.arrive = torch.zeros(B, dtype=torch.int32, device=dev)     # kernel scratch, stays zero
        self.plan = torch.full((B, 3), -1, dtype=torch.int32, device=dev)
        self.ring = torch.tensor([[0, self.residual]] * B, dtype=torch.int32, device=dev)

    @classmethod
    def from_prefill(cls, k, v, window, sink=SINK_SIZE, residual_size=RESIDUAL_SIZE):
        """k, v: [B, KVH, L, D] fp16 prefills of one length L >= sink + window
        (sequences of other lengths join with admit())."""
        return cls(_prefill_state(k, v, window, sink, residual_size), window, sink, residual_size)

    @property
    def shape(self):
        B, KVH, cap, D = self.t["k_ring"].shape
        return B, KVH, D

    def admit(self, b, k, v):
        """Start sequence slot b over from a prefill k, v [KVH, L, D] fp16
        (L >= sink + window); the other slots are untouched.  Ordered on
        torch's current stream like every other call."""
        B, KVH, D = self.shape
        if not 0 <= int(b) < B:
            raise ValueError(f"slot {b} outside the batch of {B}")
        one = _prefill_state(k[None], v[None], self.window, self.sink, self.residual)
        for name, x in one.items():
            self.t[name][b] = x[0]
        self.appended[b] = 0
        self.ring[b, 0] = 0
        self.ring[b, 1] = self.residual

    def _step(self, k_new, v_new, active):
        B, KVH, D = self.shape
        act = None
        if active is not None:
            act = active.to(device=self.appended.device, dtype=torch.int32).contiguous()
            _checks.require_gpu_tensor("active", act, dtypes=(torch.int32,), ndim=1)
            _checks.require_shape("active", act, (B,))
        win = (K._vp * 6)(*[K.ptr(self.t[n]) if self.t[n].numel() else None for n in _WIN_KEYS])
        rc = K.lib.kvdec_kivi_stream_step(K.ptr(k_new), K.ptr(v_new), K.ptr(self.t["k_ring"]),
                                          K.ptr(self.t["v_ring"]), win, K.ptr(self.appended), K.ptr(act),
                                          K.ptr(self.arrive), K.ptr(self.plan), K.ptr(self.ring), B, KVH, D,
                                          self.residual, self.cap, self.n_groups, GROUP_SIZE, QUANT_BITS,
                                          K.stream_of(self.t["k_ring"]))
        K.check(rc, "KiviStreamBatch.step")

    def append(self, k_new, v_new, active=None):
        """Append one token to every active sequence: k_new, v_new [B, KVH, D]
        fp16 (rows of inactive sequences are ignored); active: [B] bool or
        int tensor on the GPU, None = all."""
        B, KVH, D = self.shape
        k_new = k_new.reshape(B, KVH, D).contiguous()
        v_new = v_new.reshape(B, KVH, D).contiguous()
        _checks.require_gpu_tensor("k_new", k_new, ndim=3)
        _checks.require_gpu_tensor("v_new", v_new, ndim=3)
        _checks.require_same_device(("k_new", k_new), ("v_new", v_new), ("k_ring", self.t["k_ring"]))
        self._step(k_new, v_new, active)

    def reserve(self, active=None):
        """Advance every active sequence by one token and return the ring row
        each one takes ([B] int32 on the GPU, -1 for inactive sequences): the
        producer of K and V writes them to k_ring[b, :, row[b]] and
        v_ring[b, :, row[b]].  Evictions due at this token are enqueued here."""
        self._step(None, None, active)
        return self.plan[:, 0]

    def step_attend(self, q, k_new, v_new, active=None, sm_scale=None):
        """append(k_new, v_new, active) then attend(q), in one launch (each
        (b, kv) workgroup writes its token's row and quantizes its evicted
        block before it attends); returns o [B, H, D].  Leaves the cache as
        the two calls do."""
        B, KVH, D = self.shape
        k_new = k_new.reshape(B, KVH, D).contiguous()
        v_new = v_new.reshape(B, KVH, D).contiguous()
        _checks.require_gpu_tensor("q", q, ndim=3)
        _checks.require_shape("q", q, (B, q.shape[1], D))
        _checks.require_gpu_tensor("k_new", k_new, ndim=3)
        _checks.require_gpu_tensor("v_new", v_new, ndim=3)
        _checks.require_same_device(("q", q), ("k_new", k_new), ("v_new", v_new), ("k_ring", self.t["k_ring"]))
        act = None
        if active is not None:
            act = active.to(device=self.appended.device, dtype=torch.int32).contiguous()
            _checks.require_gpu_tensor("active", act, dtypes=(torch.int32,), ndim=1)
            _checks.require_shape("active", act, (B,))
        o = torch.empty_like(q)
        if sm_scale is None:
            sm_scale = D_HEAD**-0.5
        names = _SINK_KEYS + _WIN_KEYS
        arr = (K._vp * 12)(*[K.ptr(self.t[n]) if self.t[n].numel() else None for n in names])
        rc = K.lib.kvdec_kivi_stream_step_decode(
            K.ptr(q), K.ptr(k_new), K.ptr(v_new), K.ptr(self.t["k_ring"]), K.ptr(self.t["v_ring"]), arr,
            K.ptr(o), K.ptr(self.appended), K.ptr(act), K.ptr(self.arrive), K.ptr(self.plan),
            K.ptr(self.ring), B, q.shape[1], KVH, self.sink, self.residual, self.n_groups, self.cap,
            GROUP_SIZE, QUANT_BITS, float(sm_scale), K.stream_of(q))
        K.check(rc, "KiviStreamBatch.step_attend")
        return o

    def attend(self, q, sm_scale=None):
        """Decode attention of q [B, H, D] fp16 over each sequence's cache."""
        B, KVH, D = self.shape
        _checks.require_gpu_tensor("q", q, ndim=3)
        _checks.require_shape("q", q, (B, q.shape[1], D))
        _checks.require_same_device(("q", q), ("k_ring", self.t["k_ring"]))
        o = torch.empty_like(q)
        if sm_scale is None:
            sm_scale = D_HEAD**-0.5
        names = _SINK_KEYS + _WIN_KEYS
        arr = (K._vp * 12)(*[K.ptr(self.t[n]) if self.t[n].numel() else None for n in names])
        rc = K.lib.kvdec_kivi_stream_decode_seqs(K.ptr(q), K.ptr(self.t["k_ring"]), K.ptr(self.t["v_ring"]),
                                                 arr, K.ptr(o), K.ptr(self.ring), B, q.shape[1], KVH,
                                                 self.sink, self.n_groups, self.cap, GROUP_SIZE, QUANT_BITS,
                                                 float(sm_scale), K.stream_of(q))
        K.check(rc, "KiviStreamBatch.attend")
        return o
