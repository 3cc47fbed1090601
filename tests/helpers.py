"""Small helpers shared by the GPU parity tests."""

import sys

import numpy as np
import torch

ATTN_TOL = 2e-3      # north-star gate: fp16 outputs vs the fp64 oracle on the fp16 inputs
REF_TOL = 1e-2       # the reference tests' gate vs fp32 originals
SCALE = 128**-0.5


def say(msg):
    """Name the case before a GPU step (flushed, so it survives a crash)."""
    print(msg, file=sys.stderr, flush=True)


def dev(x, device):
    return torch.from_numpy(np.ascontiguousarray(x)).to(device)


def host(t):
    return t.detach().cpu().numpy()


def max_abs(a, b):
    return float(np.max(np.abs(np.asarray(a, dtype=np.float64) - np.asarray(b, dtype=np.float64))))


def randn(shape, seed, dtype=np.float32):
    return np.random.default_rng(seed).standard_normal(shape).astype(dtype)
