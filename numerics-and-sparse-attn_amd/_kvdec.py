"""ctypes binding of libkvdec.so (the C ABI in include/kvdec.h).

The library is loaded from this directory; there is no fallback: importing a
wrapper module when the library has not been built raises ImportError with the
build command.  Negative return codes (host-side validation) become
ValueError, positive ones (HIP launch errors) RuntimeError.

KVDEC_LIBRARY=clock in the environment loads the timing build
libkvdec_clock.so instead (the same kernels, which also record the GPU
realtime counter at their start and end; see kvdec_clock_arm).
"""

from __future__ import annotations

import ctypes
import os

# torch must load its bundled HIP runtime before libkvdec.so is opened: both
# carry the SONAME libamdhip64.so.7, and whichever is loaded first is the one
# the dynamic loader binds libkvdec to.  Opening libkvdec first would pull the
# system runtime in beside torch's and leave two HIP runtimes in one process.
import torch  # noqa: F401

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIBRARIES = {"": "libkvdec.so", "clock": "libkvdec_clock.so"}
_which = os.environ.get("KVDEC_LIBRARY", "")
if _which not in _LIBRARIES:
    raise ImportError(f"KVDEC_LIBRARY={_which!r}: expected one of {sorted(_LIBRARIES)}")
LIB_PATH = os.path.join(_HERE, _LIBRARIES[_which])

# element types / layouts / workspace kinds (include/kvdec.h)
F16, F32, BF16 = 0, 1, 2
LAYOUT_LINEAR, LAYOUT_RING = 0, 1
KIND_DENSE, KIND_SPARSE, KIND_KIVI = 0, 1, 2

_vp = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_f32 = ctypes.c_float
_sz = ctypes.c_size_t

# name -> (restype, argtypes); every symbol include/kvdec.h declares
SIGNATURES = {
    "kvdec_strerror": (ctypes.c_char_p, [ctypes.c_int]),
    "kvdec_version": (ctypes.c_char_p, []),
    "kvdec_num_splits": (ctypes.c_int, [ctypes.c_int, _i64, _i32, _i64]),
    "kvdec_workspace_bytes": (_sz, [ctypes.c_int, _i64, _i32, _i32, _i64, _i32]),
    "kvdec_dense_decode": (ctypes.c_int, [_vp, _vp, _vp, _vp, ctypes.c_int, _i64, _i32, _i32, _i64,
                                          _i32, _f32, _vp, _sz, _vp]),
    "kvdec_dense_decode_noalloc": (ctypes.c_int, [_vp, _vp, _vp, _vp, ctypes.c_int, _i64, _i32, _i32,
                                                  _i64, _i32, _f32, _vp]),
    "kvdec_read_probe": (ctypes.c_int, [_vp, _i64, _vp, _i32, _vp]),
    "kvdec_read_probe_sweep": (ctypes.c_int, [_vp, _i64, _vp, _i32, _i32, _i32, _i32, _vp]),
    "kvdec_clock_arm": (ctypes.c_int, [_vp, _i32]),
    "kvdec_sparse_decode": (ctypes.c_int, [_vp, _vp, _vp, _vp, ctypes.c_int, _i64, _i32, _i32, _i64,
                                           _i32, _i32, _i32, _f32, _vp, _sz, _vp]),
    "kvdec_paged_decode": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, ctypes.c_int, _i64, _i32, _i32,
                                          _i32, _i64, _i32, _i32, _i64, _i64, _i64, _i64, _f32, _vp,
                                          _sz, _vp]),
    "kvdec_sparse_decode_varlen": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, ctypes.c_int, _i64, _i32,
                                                  _i32, _i32, _i32, _i32, _f32, _vp, _sz, _vp]),
    "kvdec_quantize_k": (ctypes.c_int, [_vp, ctypes.c_int, _vp, _vp, _vp, _i64, _i32, _i64, _i32,
                                        _i32, _i32, _vp]),
    "kvdec_quantize_v": (ctypes.c_int, [_vp, ctypes.c_int, _vp, _vp, _vp, _i64, _i32, _i64, _i32,
                                        _i32, _i32, _vp]),
    "kvdec_sparse_decode_kivi": (ctypes.c_int, [_vp, _vp, _vp, ctypes.POINTER(_vp), _vp, _i64, _i32,
                                                _i32, _i64, _i32, _i32, _i32, _i32, _i32, _f32, _vp,
                                                _sz, _vp]),
    "kvdec_sparse_decode_kivi_varlen": (ctypes.c_int, [_vp, _vp, _vp, ctypes.POINTER(_vp), _vp, _vp, _i64,
                                                       _i32, _i32, _i32, _i32, _i32, _i32, _i32, _f32,
                                                       _vp]),
    "kvdec_sparse_decode_kivi_typed": (ctypes.c_int, [_vp, _vp, _vp, ctypes.POINTER(_vp), _vp, ctypes.c_int,
                                                      ctypes.c_int, _vp, _i64, _i32, _i32, _i64, _i32, _i32,
                                                      _i32, _i32, _i32, _f32, _vp]),
    "kvdec_kivi_stream_append": (ctypes.c_int, [_vp, _vp, _vp, _vp, ctypes.POINTER(_vp), _i64, _i32,
                                                _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _vp]),
    "kvdec_kivi_stream_decode": (ctypes.c_int, [_vp, _vp, _vp, ctypes.POINTER(_vp), _vp, _i64, _i32,
                                                _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _f32,
                                                _vp]),
    "kvdec_kivi_stream_step": (ctypes.c_int, [_vp, _vp, _vp, _vp, ctypes.POINTER(_vp), _vp, _vp, _vp, _vp,
                                              _vp, _i64, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _vp]),
    "kvdec_kivi_stream_decode_seqs": (ctypes.c_int, [_vp, _vp, _vp, ctypes.POINTER(_vp), _vp, _vp, _i64,
                                                     _i32, _i32, _i32, _i32, _i32, _i32, _i32, _f32,
                                                     _vp]),
    "kvdec_kivi_stream_step_decode": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, ctypes.POINTER(_vp), _vp, _vp,
                                                     _vp, _vp, _vp, _vp, _i64, _i32, _i32, _i32, _i32,
                                                     _i32, _i32, _i32, _i32, _f32, _vp]),
    "kvdec_build_kivi_cache": (ctypes.c_int, [_vp, _vp, ctypes.c_int, ctypes.c_int, _i64, _i32, _i32,
                                              _i32, _i32, _i32, _i32, _i32, ctypes.POINTER(_vp), _vp]),
    "kvdec_dequant_k_tile": (ctypes.c_int, [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i32, _i32, _i32,
                                            _i32, _vp]),
    "kvdec_dequant_v_tile": (ctypes.c_int, [_vp, _vp, _vp, _vp, _i64, _i64, _i32, _i32, _i32, _i32,
                                            _vp]),
}


def _load() -> ctypes.CDLL:
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} is missing: build it with `python {os.path.join(_HERE, 'build.py')}` "
            "(or __graft_entry__.build()); there is no CPU fallback")
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


lib = _load()


class KvdecLaunchError(RuntimeError):
    """A HIP launch inside libkvdec failed (positive return code)."""


def strerror(code: int) -> str:
    return lib.kvdec_strerror(code).decode()


def check(code: int, what: str) -> None:
    if code == 0:
        return
    msg = f"{what}: {strerror(code)} (kvdec code {code})"
    if code < 0:
        raise ValueError(msg)
    raise KvdecLaunchError(msg)


def ptr(t) -> int | None:
    """Device address of a tensor (None for None)."""
    return None if t is None else t.data_ptr()


def stream_of(t) -> int | None:
    """hipStream_t of torch's current stream on t's device."""
    import torch
    if t is None or not t.is_cuda:
        return None
    return torch.cuda.current_stream(t.device).cuda_stream


def workspace(kind: int, B: int, H: int, KVH: int, n_slots: int, D: int, device):
    """Split-K workspace for one call (None when a single pass suffices)."""
    import torch
    nbytes = lib.kvdec_workspace_bytes(kind, B, H, KVH, n_slots, D)
    if nbytes == 0:
        return None, 0
    return torch.empty(nbytes, dtype=torch.uint8, device=device), nbytes
