"""Argument checks shared by the drop-in wrappers (raise before any launch)."""

from __future__ import annotations

import torch

# dtypes of the attention entry points' q / k / v / o and their kvdec codes
# (include/kvdec.h: KVDEC_F16, KVDEC_F32, KVDEC_BF16)
ATTN_DTYPES = {torch.float16: 0, torch.float32: 1, torch.bfloat16: 2}


def require_gpu_tensor(name: str, t, dtypes=(torch.float16,), ndim: int | None = None,
                       contiguous: bool = True) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor, got {type(t).__name__}")
    if not t.is_cuda:
        raise ValueError(f"{name} must live on the GPU (got device {t.device})")
    if t.dtype not in dtypes:
        raise ValueError(f"{name} must have dtype in {[str(d) for d in dtypes]}, got {t.dtype}")
    if ndim is not None and t.dim() != ndim:
        raise ValueError(f"{name} must be {ndim}-D, got shape {tuple(t.shape)}")
    if contiguous and not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def require_shape(name: str, t, shape) -> None:
    if tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} must have shape {tuple(shape)}, got {tuple(t.shape)}")


def require_same_device(*named) -> None:
    devs = {t.device for _, t in named if t is not None}
    if len(devs) > 1:
        raise ValueError("all tensors must be on the same device: "
                         + ", ".join(f"{n}={t.device}" for n, t in named if t is not None))


def seq_lens_tensor(name: str, t, B: int, device) -> None:
    """Per-sequence lengths: a [B] int32 tensor on the cache's device."""
    require_gpu_tensor(name, t, dtypes=(torch.int32,), ndim=1)
    require_shape(name, t, (B,))
    if t.device != device:
        raise ValueError(f"{name} must be on {device}, got {t.device}")


def row_major_rows(name: str, t) -> None:
    """The head dim (last) must be contiguous; other strides are free."""
    if t.stride(-1) != 1:
        raise ValueError(f"{name} must have a contiguous last dimension, got strides {t.stride()}")
