"""C-ABI checks that need no GPU: the library loads, exports every symbol
include/kvdec.h declares, and rejects bad arguments with the documented
negative codes before any HIP call."""

import ctypes
import os
import re

import pytest

from conftest import ROOT

import _kvdec as K

HEADER = os.path.join(ROOT, "include", "kvdec.h")
# Never dereferenced: every call below is built to fail host-side validation
# before any launch (a launch on these pointers would fault the GPU).
FAKE = ctypes.c_void_p(0x1000)

E = {
    "NULL": -1, "SHAPE": -2, "DTYPE": -3, "GROUP": -4, "DGROUP": -5, "WORKSPACE": -6,
    "WINDOW": -7, "SEQLEN": -8, "BITS": -9, "UNSUPPORTED": -10,
}


def _header_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+char\s*\*|int|size_t)\s+(kvdec_\w+)\s*\(", text, re.M)))


def _header_codes():
    text = open(HEADER).read()
    return {m.group(1): int(m.group(2)) for m in re.finditer(r"#define KVDEC_E_(\w+) \((-\d+)\)", text)}


def test_header_and_binding_agree():
    funcs = _header_functions()
    assert len(funcs) == 25
    assert funcs == sorted(K.SIGNATURES)
    assert _header_codes() == E


def test_library_exports_every_symbol():
    lib = ctypes.CDLL(K.LIB_PATH)
    for name in _header_functions():
        assert hasattr(lib, name), name


def test_strerror_and_version():
    assert K.strerror(0) == "success"
    for code in E.values():
        assert K.strerror(code) and "unknown" not in K.strerror(code)
    assert K.strerror(-999) == "unknown kvdec error"
    assert K.lib.kvdec_version().decode().startswith("kvdec")
    # the reference's assert messages are kept verbatim
    assert K.strerror(E["GROUP"]) == "this simple version assumes seq_len is a multiple of group_size"
    assert K.strerror(E["DGROUP"]) == "this simple version assumes D_HEAD is a multiple of group_size"


def test_split_plan_and_workspace_arithmetic():
    # at the metric shapes (B*KVH = 256 KV heads fill the GPU) every path runs
    # in one pass: no split, no workspace
    for kind, n in ((K.KIND_DENSE, 163840), (K.KIND_DENSE, 32768), (K.KIND_SPARSE, 260),
                    (K.KIND_SPARSE, 16388), (K.KIND_KIVI, 256), (K.KIND_KIVI, 4096)):
        assert K.lib.kvdec_num_splits(kind, 32, 8, n) == 1, (kind, n)
        assert K.lib.kvdec_workspace_bytes(kind, 32, 64, 8, n, 128) == 0, (kind, n)
    # a small batch splits the context and needs G x (128 + 2) floats per split
    s = K.lib.kvdec_num_splits(K.KIND_DENSE, 1, 8, 163840)
    assert s > 1
    assert K.lib.kvdec_workspace_bytes(K.KIND_DENSE, 1, 64, 8, 163840, 128) == 8 * s * 8 * 130 * 4
    # every split keeps at least one tile per wave of an 8-wave workgroup, and
    # splits stop once the work units fill the 256 CUs
    for B in (1, 2, 4, 32):
        for L in (1, 2, 100, 8192, 32768, 131072, 163840):
            s = K.lib.kvdec_num_splits(K.KIND_DENSE, B, 8, L)
            tiles = -(-L // 32)
            assert s == 1 or tiles / s >= 8, (B, L, s)
            assert s == 1 or B * 8 * (s - 1) < 256, (B, L, s)
    # the fused KIVI decode never splits (one work unit per KV head)
    assert K.lib.kvdec_num_splits(K.KIND_KIVI, 1, 8, 4096) == 1
    assert K.lib.kvdec_workspace_bytes(K.KIND_KIVI, 1, 64, 8, 4096, 128) == 0
    # invalid heads -> no workspace
    assert K.lib.kvdec_workspace_bytes(K.KIND_DENSE, 32, 64, 7, 1000, 128) == 0
    assert K.lib.kvdec_workspace_bytes(K.KIND_DENSE, 32, 64, 8, 1000, 64) == 0


def _dense(**kw):
    a = dict(q=FAKE, k=FAKE, v=FAKE, o=FAKE, dtype=K.F16, B=32, H=64, KVH=8, L=1024, D=128,
             scale=0.088, ws=None, wsb=0, stream=None)
    a.update(kw)
    return K.lib.kvdec_dense_decode(a["q"], a["k"], a["v"], a["o"], a["dtype"], a["B"], a["H"],
                                    a["KVH"], a["L"], a["D"], a["scale"], a["ws"], a["wsb"],
                                    a["stream"])


def test_dense_validation():
    assert _dense(q=None) == E["NULL"]
    assert _dense(o=None) == E["NULL"]
    assert _dense(dtype=7) == E["DTYPE"]           # f16 / f32 / bf16 are taken
    assert _dense(KVH=7) == E["SHAPE"]            # H % KVH != 0
    assert _dense(H=8 * 32, KVH=8) == E["SHAPE"]  # group of 32 > 16 MFMA columns
    assert _dense(D=64) == E["SHAPE"]
    assert _dense(B=0) == E["SHAPE"]
    assert _dense(L=0) == E["SEQLEN"]
    assert _dense(L=1 << 23) == E["SHAPE"]        # 32-bit in-head offsets
    # B=1: the long context is split, so a workspace is required (these
    # calls must fail validation: FAKE pointers are never launched on)
    assert _dense(B=1, L=163840) == E["WORKSPACE"]
    assert _dense(B=1, L=163840, ws=FAKE, wsb=16) == E["WORKSPACE"]


def test_dense_noalloc_validation():
    """The workspace-free dense decode rejects bad arguments before it looks
    up its device array or launches anything."""
    def call(**kw):
        a = dict(q=FAKE, k=FAKE, v=FAKE, o=FAKE, dtype=K.F16, B=32, H=64, KVH=8, L=5000, D=128)
        a.update(kw)
        return K.lib.kvdec_dense_decode_noalloc(a["q"], a["k"], a["v"], a["o"], a["dtype"], a["B"], a["H"],
                                                a["KVH"], a["L"], a["D"], 0.088, None)
    assert call(q=None) == E["NULL"]
    assert call(dtype=7) == E["DTYPE"]
    assert call(KVH=7) == E["SHAPE"]
    assert call(D=64) == E["SHAPE"]
    assert call(L=0) == E["SEQLEN"]
    assert call(L=1 << 23) == E["SHAPE"]


def test_read_probe_validation():
    """The bandwidth probe rejects bad sizes before launching anything."""
    probe = K.lib.kvdec_read_probe
    assert probe(FAKE, 1024, None, 256, None) == E["NULL"]
    assert probe(None, 1024, FAKE, 256, None) == E["NULL"]
    assert probe(FAKE, 1000, FAKE, 256, None) == E["SHAPE"]
    assert probe(FAKE, -16, FAKE, 256, None) == E["SHAPE"]
    assert probe(FAKE, 1024, FAKE, 0, None) == E["SHAPE"]
    assert probe(FAKE, 1024, FAKE, 65537, None) == E["SHAPE"]


def test_read_probe_sweep_validation():
    """The sweep form of the probe rejects bad sizes, block sizes, modes and
    LDS reservations before launching anything."""
    probe = K.lib.kvdec_read_probe_sweep
    assert probe(FAKE, 1024, None, 256, 512, 0, 0, None) == E["NULL"]
    assert probe(None, 1024, FAKE, 256, 512, 0, 0, None) == E["NULL"]
    assert probe(FAKE, 1000, FAKE, 256, 512, 0, 0, None) == E["SHAPE"]
    assert probe(FAKE, 1024, FAKE, 0, 512, 0, 0, None) == E["SHAPE"]
    for threads in (0, 64, 128, 768, 2048):
        assert probe(FAKE, 1024, FAKE, 256, threads, 0, 0, None) == E["SHAPE"]
    for mode in (-1, 8):
        assert probe(FAKE, 1024, FAKE, 256, 512, mode, 0, None) == E["SHAPE"]
    assert probe(FAKE, 1024, FAKE, 256, 512, 0, -1, None) == E["SHAPE"]
    assert probe(FAKE, 1024, FAKE, 256, 512, 0, 160 * 1024 + 1, None) == E["SHAPE"]
    # buffer loads address a workgroup's share with 31-bit offsets
    assert probe(FAKE, 1 << 32, FAKE, 1, 512, 2, 0, None) == E["SHAPE"]


def test_clock_arm_only_in_timing_build():
    """The kernel clock exists only in the timing build; the product
    library says so instead of recording anything."""
    if os.path.basename(K.LIB_PATH) == "libkvdec.so":
        assert K.lib.kvdec_clock_arm(FAKE, 16) == E["UNSUPPORTED"]
        assert K.lib.kvdec_clock_arm(None, 0) == E["UNSUPPORTED"]
    else:
        assert K.lib.kvdec_clock_arm(FAKE, 0) == E["SHAPE"]
        assert K.lib.kvdec_clock_arm(None, 0) == 0


def _sparse(**kw):
    a = dict(q=FAKE, k=FAKE, v=FAKE, o=FAKE, dtype=K.F16, B=32, H=64, KVH=8, seq_len=5000, W=256,
             S=4, layout=0, scale=0.088, ws=None, wsb=0, stream=None)
    a.update(kw)
    return K.lib.kvdec_sparse_decode(a["q"], a["k"], a["v"], a["o"], a["dtype"], a["B"], a["H"],
                                     a["KVH"], a["seq_len"], a["W"], a["S"], a["layout"],
                                     a["scale"], a["ws"], a["wsb"], a["stream"])


def test_sparse_validation():
    assert _sparse(v=None) == E["NULL"]
    assert _sparse(dtype=7) == E["DTYPE"]
    assert _sparse(seq_len=0) == E["SEQLEN"]
    assert _sparse(W=-1) == E["WINDOW"]
    assert _sparse(S=-1) == E["WINDOW"]
    assert _sparse(W=0, S=0) == E["WINDOW"]
    assert _sparse(layout=2) == E["UNSUPPORTED"]
    assert _sparse(layout=1, W=0) == E["WINDOW"]
    assert _sparse(B=1, W=16384) == E["WORKSPACE"]


def _kivi(ptrs=None, **kw):
    a = dict(q=FAKE, kr=FAKE, vr=FAKE, o=FAKE, B=32, H=64, KVH=8, seq_len=200000, W=256, S=4, R=128,
             group=32, bits=2, scale=0.088, ws=None, wsb=0, stream=None)
    a.update(kw)
    arr = (K._vp * 12)(*([0x1000] * 12 if ptrs is None else ptrs))
    return K.lib.kvdec_sparse_decode_kivi(a["q"], a["kr"], a["vr"], arr, a["o"], a["B"], a["H"],
                                          a["KVH"], a["seq_len"], a["W"], a["S"], a["R"],
                                          a["group"], a["bits"], a["scale"], a["ws"], a["wsb"],
                                          a["stream"])


def test_kivi_validation():
    assert _kivi(q=None) == E["NULL"]
    assert _kivi(ptrs=[0x1000] * 5 + [None] + [0x1000] * 6) == E["NULL"]
    assert _kivi(ptrs=[0x1000] * 6 + [None] * 6) == E["NULL"]          # window-old needed at W=256
    assert _kivi(bits=9) == E["BITS"]
    assert _kivi(bits=0) == E["BITS"]
    assert _kivi(group=48) == E["GROUP"]                               # does not divide D_HEAD
    assert _kivi(bits=1, group=4) == E["GROUP"]                        # not whole bytes of codes
    # the generic kernel's own checks (widths other than 2, groups other than 32)
    assert _kivi(bits=4, q=None) == E["NULL"]
    assert _kivi(bits=4, ptrs=[0x1000] * 6 + [None] * 6) == E["NULL"]
    assert _kivi(bits=4, S=0) == E["WINDOW"]
    assert _kivi(group=16, S=17) == E["WINDOW"]                        # sink beyond one group
    assert _kivi(bits=4, W=128 + 48) == E["GROUP"]
    assert _kivi(group=64, W=128 + 96) == E["GROUP"]
    assert _kivi(bits=4, seq_len=0) == E["SEQLEN"]
    assert _kivi(bits=4, KVH=3) == E["SHAPE"]
    assert _kivi(W=0) == E["WINDOW"]                                  # empty window
    assert _kivi(S=0) == E["WINDOW"]
    assert _kivi(S=33) == E["WINDOW"]
    assert _kivi(R=100) == E["WINDOW"]
    assert _kivi(W=128 + 48) == E["GROUP"]                            # window-old not whole groups
    assert _kivi(seq_len=0) == E["SEQLEN"]
    assert _kivi(KVH=3) == E["SHAPE"]


def _kivi_varlen(**kw):
    a = dict(q=FAKE, kr=FAKE, vr=FAKE, o=FAKE, lens=FAKE, B=32, H=64, KVH=8, W=256, S=4, R=128,
             group=32, bits=2, scale=0.088, stream=None)
    a.update(kw)
    arr = (K._vp * 12)(*([0x1000] * 12))
    return K.lib.kvdec_sparse_decode_kivi_varlen(a["q"], a["kr"], a["vr"], arr, a["o"], a["lens"],
                                                 a["B"], a["H"], a["KVH"], a["W"], a["S"], a["R"],
                                                 a["group"], a["bits"], a["scale"], a["stream"])


def test_kivi_varlen_validation():
    assert _kivi_varlen(lens=None) == E["NULL"]
    assert _kivi_varlen(q=None) == E["NULL"]
    assert _kivi_varlen(bits=9) == E["BITS"]
    assert _kivi_varlen(group=48) == E["GROUP"]
    assert _kivi_varlen(bits=4, lens=None) == E["NULL"]
    assert _kivi_varlen(bits=8, W=200) == E["GROUP"]
    assert _kivi_varlen(W=0) == E["WINDOW"]
    assert _kivi_varlen(W=200) == E["GROUP"]
    assert _kivi_varlen(H=60) == E["SHAPE"]


def _kivi_typed(**kw):
    a = dict(q=FAKE, kr=FAKE, vr=FAKE, o=FAKE, qdt=K.BF16, rdt=K.F32, lens=None, B=32, H=64, KVH=8,
             seq_len=163840, W=256, S=4, R=128, group=32, bits=2, scale=0.088, stream=None)
    a.update(kw)
    arr = (K._vp * 12)(*([0x1000] * 12))
    return K.lib.kvdec_sparse_decode_kivi_typed(a["q"], a["kr"], a["vr"], arr, a["o"], a["qdt"], a["rdt"],
                                                a["lens"], a["B"], a["H"], a["KVH"], a["seq_len"], a["W"],
                                                a["S"], a["R"], a["group"], a["bits"], a["scale"],
                                                a["stream"])


def test_kivi_typed_validation():
    assert _kivi_typed(q=None) == E["NULL"]
    assert _kivi_typed(qdt=3) == E["DTYPE"]
    assert _kivi_typed(rdt=-1) == E["DTYPE"]
    assert _kivi_typed(qdt=K.F16, rdt=7) == E["DTYPE"]
    assert _kivi_typed(bits=9) == E["BITS"]
    assert _kivi_typed(group=48) == E["GROUP"]
    assert _kivi_typed(W=200) == E["GROUP"]
    assert _kivi_typed(seq_len=0) == E["SEQLEN"]
    assert _kivi_typed(S=0) == E["WINDOW"]
    assert _kivi_typed(KVH=3) == E["SHAPE"]
    # fp16 / fp16 is the fused kernel's, with its checks
    assert _kivi_typed(qdt=K.F16, rdt=K.F16, R=100) == E["WINDOW"]
    assert _kivi_typed(qdt=K.F16, rdt=K.F16, q=None) == E["NULL"]


def _quant(fn, **kw):
    a = dict(x=FAKE, dt=K.F32, p=FAKE, s=FAKE, z=FAKE, B=1, KVH=8, N=256, D=128, group=32, bits=2,
             stream=None)
    a.update(kw)
    return fn(a["x"], a["dt"], a["p"], a["s"], a["z"], a["B"], a["KVH"], a["N"], a["D"], a["group"],
              a["bits"], a["stream"])


@pytest.mark.parametrize("name", ["kvdec_quantize_k", "kvdec_quantize_v"])
def test_quantize_validation(name):
    fn = getattr(K.lib, name)
    assert _quant(fn, x=None) == E["NULL"]
    assert _quant(fn, z=None) == E["NULL"]
    assert _quant(fn, bits=9) == E["BITS"]
    assert _quant(fn, bits=0) == E["BITS"]
    assert _quant(fn, dt=7) == E["DTYPE"]
    assert _quant(fn, N=0) == E["SHAPE"]
    if name == "kvdec_quantize_k":
        assert _quant(fn, N=100) == E["GROUP"]
        assert _quant(fn, D=7) == E["SHAPE"]
        assert _quant(fn, group=48) == E["GROUP"]                 # 256 tokens not whole groups
        assert _quant(fn, bits=1, group=4) == E["GROUP"]          # not whole bytes of codes
    else:
        assert _quant(fn, D=100) == E["DGROUP"]
        assert _quant(fn, group=48) == E["DGROUP"]
        assert _quant(fn, bits=1, group=4) == E["DGROUP"]


def _append(**kw):
    a = dict(kn=FAKE, vn=FAKE, kr=FAKE, vr=FAKE, win=[0x1000] * 6, B=32, KVH=8, D=128, cap=160,
             row=0, blk=-1, slot=0, ng=4, group=32, bits=2, stream=None)
    a.update(kw)
    arr = (K._vp * 6)(*a["win"]) if a["win"] is not None else None
    return K.lib.kvdec_kivi_stream_append(a["kn"], a["vn"], a["kr"], a["vr"], arr, a["B"], a["KVH"],
                                          a["D"], a["cap"], a["row"], a["blk"], a["slot"], a["ng"],
                                          a["group"], a["bits"], a["stream"])


def test_stream_append_validation():
    assert _append(kn=None) == E["NULL"]               # one of the pair missing
    assert _append(kr=None) == E["NULL"]
    assert _append(bits=4) == E["BITS"]
    assert _append(group=64) == E["UNSUPPORTED"]
    assert _append(D=100) == E["DGROUP"]
    assert _append(cap=32) == E["WINDOW"]            # below residual + one group
    assert _append(cap=170) == E["WINDOW"]
    assert _append(row=160) == E["SHAPE"]
    assert _append(blk=5) == E["SHAPE"]
    assert _append(row=40, blk=1) == E["SHAPE"]      # the evicted block holds the new row
    assert _append(blk=1, slot=4) == E["SHAPE"]
    assert _append(blk=1, win=[0x1000] * 5 + [None]) == E["NULL"]
    assert _append(blk=1, win=None) == E["NULL"]


def _sdecode(**kw):
    a = dict(q=FAKE, kr=FAKE, vr=FAKE, o=FAKE, B=32, H=64, KVH=8, S=4, ng=4, cap=160, start=0,
             count=128, group=32, bits=2, scale=0.088, stream=None)
    a.update(kw)
    arr = (K._vp * 12)(*([0x1000] * 12))
    return K.lib.kvdec_kivi_stream_decode(a["q"], a["kr"], a["vr"], arr, a["o"], a["B"], a["H"],
                                          a["KVH"], a["S"], a["ng"], a["cap"], a["start"], a["count"],
                                          a["group"], a["bits"], a["scale"], a["stream"])


def test_stream_decode_validation():
    assert _sdecode(q=None) == E["NULL"]
    assert _sdecode(bits=3) == E["BITS"]
    assert _sdecode(S=0) == E["WINDOW"]
    assert _sdecode(cap=48) == E["WINDOW"]
    assert _sdecode(start=160) == E["WINDOW"]
    assert _sdecode(count=0) == E["WINDOW"]
    assert _sdecode(count=161) == E["WINDOW"]
    assert _sdecode(KVH=3) == E["SHAPE"]


def _paged(**kw):
    a = dict(q=FAKE, k=FAKE, v=FAKE, bt=FAKE, lens=FAKE, o=FAKE, dtype=K.F16, B=4, H=64, KVH=8, D=128,
             L=4096, ps=16, mb=256, np_=1024, sp=16 * 8 * 128, sr=8 * 128, sh=128, scale=0.088, ws=None,
             nbytes=0, stream=None)
    a.update(kw)
    return K.lib.kvdec_paged_decode(a["q"], a["k"], a["v"], a["bt"], a["lens"], a["o"], a["dtype"],
                                    a["B"], a["H"], a["KVH"], a["D"], a["L"], a["ps"], a["mb"],
                                    a["np_"], a["sp"], a["sr"], a["sh"], a["scale"], a["ws"],
                                    a["nbytes"], a["stream"])


def test_paged_validation():
    assert _paged(q=None) == E["NULL"]
    assert _paged(v=None) == E["NULL"]
    assert _paged(dtype=K.BF16) == E["DTYPE"]
    assert _paged(D=64) == E["SHAPE"]
    assert _paged(H=60) == E["SHAPE"]
    assert _paged(L=0) == E["SEQLEN"]
    assert _paged(L=1 << 30) == E["SHAPE"]
    assert _paged(sr=-1) == E["SHAPE"]
    assert _paged(sr=1 << 26) == E["SHAPE"]       # 16 rows past 2^31 bytes
    assert _paged(ps=8) == E["UNSUPPORTED"]
    assert _paged(ps=48) == E["UNSUPPORTED"]
    assert _paged(mb=255) == E["SHAPE"]           # 255 * 16 < 4096 tokens
    assert _paged(np_=0) == E["SHAPE"]
    # B=4, L=4096 splits: a missing workspace is reported, nothing launched
    assert _paged() == E["WORKSPACE"]
    assert _paged(bt=None, ps=0, mb=0, np_=0) == E["WORKSPACE"]


def _svarlen(**kw):
    a = dict(q=FAKE, k=FAKE, v=FAKE, o=FAKE, lens=FAKE, dtype=K.F16, B=4, H=64, KVH=8, W=16384, S=4,
             layout=K.LAYOUT_LINEAR, scale=0.088, ws=None, nbytes=0, stream=None)
    a.update(kw)
    return K.lib.kvdec_sparse_decode_varlen(a["q"], a["k"], a["v"], a["o"], a["lens"], a["dtype"],
                                            a["B"], a["H"], a["KVH"], a["W"], a["S"], a["layout"],
                                            a["scale"], a["ws"], a["nbytes"], a["stream"])


def test_sparse_varlen_validation():
    assert _svarlen(lens=None) == E["NULL"]
    assert _svarlen(dtype=7) == E["DTYPE"]
    assert _svarlen(W=0, S=0) == E["WINDOW"]
    assert _svarlen(W=-1) == E["WINDOW"]
    assert _svarlen(layout=5) == E["UNSUPPORTED"]
    assert _svarlen(layout=K.LAYOUT_RING, W=0) == E["WINDOW"]
    assert _svarlen() == E["WORKSPACE"]


def test_stream_seqs_validation():
    L = K.lib
    win = (K._vp * 6)(*([0x1000] * 6))

    def step(**kw):
        a = dict(kn=None, vn=None, kr=FAKE, vr=FAKE, win=win, app=FAKE, act=None, arr=FAKE, plan=FAKE,
                 ring=FAKE, B=4, KVH=8, D=128, R=128, cap=160, ng=4, group=32, bits=2)
        a.update(kw)
        return L.kvdec_kivi_stream_step(a["kn"], a["vn"], a["kr"], a["vr"], a["win"], a["app"], a["act"],
                                        a["arr"], a["plan"], a["ring"], a["B"], a["KVH"], a["D"], a["R"],
                                        a["cap"], a["ng"], a["group"], a["bits"], None)

    assert step(app=None) == E["NULL"]
    assert step(arr=None) == E["NULL"]
    assert step(kn=FAKE) == E["NULL"]                  # one of the pair missing
    assert step(win=None) == E["NULL"]
    assert step(bits=4) == E["BITS"]
    assert step(group=64) == E["UNSUPPORTED"]
    assert step(B=0) == E["SHAPE"]
    assert step(ng=-1) == E["SHAPE"]
    assert step(D=100) == E["DGROUP"]
    assert step(cap=192) == E["WINDOW"]
    assert step(R=100, cap=132) == E["WINDOW"]
    arr = (K._vp * 12)(*([0x1000] * 12))
    dec = L.kvdec_kivi_stream_decode_seqs
    assert dec(FAKE, FAKE, FAKE, arr, FAKE, None, 4, 64, 8, 4, 4, 160, 32, 2, 0.088, None) == E["NULL"]
    assert dec(FAKE, FAKE, FAKE, arr, FAKE, FAKE, 4, 64, 8, 0, 4, 160, 32, 2, 0.088, None) == E["WINDOW"]
    assert dec(FAKE, FAKE, FAKE, arr, FAKE, FAKE, 4, 64, 8, 4, 4, 48, 32, 2, 0.088, None) == E["WINDOW"]
    assert dec(FAKE, FAKE, FAKE, arr, FAKE, FAKE, 4, 60, 8, 4, 4, 160, 32, 2, 0.088, None) == E["SHAPE"]


def test_stream_step_decode_validation():
    L = K.lib

    def call(**kw):
        a = dict(q=FAKE, kn=FAKE, vn=FAKE, kr=FAKE, vr=FAKE, kivi=[0x1000] * 12, o=FAKE, app=FAKE,
                 act=None, arr=FAKE, plan=FAKE, ring=FAKE, B=4, H=64, KVH=8, sink=4, R=128, ng=4,
                 cap=160, group=32, bits=2)
        a.update(kw)
        arr = (K._vp * 12)(*a["kivi"])
        return L.kvdec_kivi_stream_step_decode(a["q"], a["kn"], a["vn"], a["kr"], a["vr"], arr, a["o"],
                                               a["app"], a["act"], a["arr"], a["plan"], a["ring"], a["B"],
                                               a["H"], a["KVH"], a["sink"], a["R"], a["ng"], a["cap"],
                                               a["group"], a["bits"], 0.088, None)

    assert call(kn=None) == E["NULL"]                   # the token's K / V are required here
    assert call(vn=None) == E["NULL"]
    assert call(app=None) == E["NULL"]
    assert call(ring=None) == E["NULL"]
    assert call(kivi=[0x1000] * 6 + [0] * 6) == E["NULL"]   # window-old tensors with ng > 0
    assert call(bits=4) == E["BITS"]
    assert call(group=64) == E["UNSUPPORTED"]
    assert call(H=60) == E["SHAPE"]
    assert call(sink=0) == E["WINDOW"]
    assert call(cap=192) == E["WINDOW"]
    assert call(R=100, cap=132) == E["WINDOW"]


def _build(**kw):
    a = dict(k=FAKE, v=FAKE, dt=K.F16, rdt=K.F16, B=2, KVH=8, n=4 + 256, D=128, S=4, R=128, group=32,
             bits=2, out=[0x1000] * 14, stream=None)
    a.update(kw)
    arr = (K._vp * 14)(*a["out"]) if a["out"] is not None else None
    return K.lib.kvdec_build_kivi_cache(a["k"], a["v"], a["dt"], a["rdt"], a["B"], a["KVH"], a["n"],
                                        a["D"], a["S"], a["R"], a["group"], a["bits"], arr, a["stream"])


def test_build_cache_validation():
    assert _build(k=None) == E["NULL"]
    assert _build(out=None) == E["NULL"]
    assert _build(out=[0x1000] * 13 + [None]) == E["NULL"]
    assert _build(out=[0x1000] * 8 + [None] * 6) == E["NULL"]   # window-old part needed
    assert _build(bits=4) == E["BITS"]
    assert _build(group=64) == E["UNSUPPORTED"]
    assert _build(dt=7) == E["DTYPE"]
    assert _build(dt=K.F32, rdt=K.BF16) == E["DTYPE"]
    assert _build(D=100) == E["DGROUP"]
    assert _build(S=0) == E["WINDOW"]
    assert _build(S=33) == E["WINDOW"]
    assert _build(n=4) == E["WINDOW"]
    assert _build(n=4 + 144) == E["GROUP"]
    assert _build(B=0) == E["SHAPE"]


def test_dequant_tile_validation():
    assert K.lib.kvdec_dequant_k_tile(None, FAKE, FAKE, FAKE, 0, 8, 1, 1, 1, 128, 128, None) == E["NULL"]
    assert K.lib.kvdec_dequant_k_tile(FAKE, FAKE, FAKE, FAKE, 0, 0, 1, 1, 1, 128, 128, None) == E["SHAPE"]
    assert K.lib.kvdec_dequant_v_tile(FAKE, FAKE, FAKE, FAKE, 0, 0, 1, 1, 128, 128, None) == E["SHAPE"]
    assert K.lib.kvdec_dequant_v_tile(FAKE, FAKE, FAKE, FAKE, 0, 32, 1, 1, 100, 128, None) == E["DGROUP"]


def test_python_wrappers_reject_cpu_tensors():
    import torch
    import dense_kernel
    import quant_kernel
    import sparse_kernel
    q = torch.zeros(2, 16, 128, dtype=torch.float16)
    k = torch.zeros(2, 2, 8, 128, dtype=torch.float16)
    with pytest.raises(ValueError, match="GPU"):
        dense_kernel.dense_decode_attention(q, k, k, seq_len=8)
    with pytest.raises(ValueError, match="GPU"):
        sparse_kernel.sparse_decode_attention(q, k, k, seq_len=8, window=4)
    with pytest.raises(ValueError, match="GPU"):
        quant_kernel.quantize_k_cache(torch.zeros(1, 1, 32, 128))
    with pytest.raises(AssertionError, match="multiple of group_size"):
        quant_kernel.quantize_k_cache(torch.zeros(1, 1, 33, 128))
    with pytest.raises(AssertionError, match="multiple of group_size"):
        quant_kernel.quantize_v_cache(torch.zeros(1, 1, 32, 100))
