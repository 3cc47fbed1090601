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


def assert_nearly_rounded(o, ref, slack=5e-5):
    """Every fp16 output within half an fp16 ulp of the fp64 reference (what
    one rounding of an exact result gives) plus `slack`: the kernel's own
    arithmetic before that rounding must be far more accurate than fp16."""
    o = np.asarray(o, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    half_ulp = np.spacing(np.abs(ref).astype(np.float16)).astype(np.float64) / 2
    excess = np.abs(o - ref) - half_ulp
    worst = np.unravel_index(np.argmax(excess), excess.shape)
    assert excess[worst] <= slack, (f"output {o[worst]} vs reference {ref[worst]} at {worst}: "
                                    f"{excess[worst]:.3g} beyond half an ulp")
