"""Build libkvdec.so, the gfx950 decode-attention library, in-tree with hipcc.

    python build.py [-v]

Each HIP source is compiled for gfx950 only, with packed-fp32 instruction
selection disabled; quant.hip additionally forbids FP contraction so its codes
match the IEEE closed form bit for bit.  The shared library lands next to this
file, where the ctypes loader (_kvdec.py) looks for it.

The same sources also make libkvdec_clock.so, the timing build: attn.hip
compiled with -DKVDEC_CLOCK, whose attention kernels record the GPU realtime
counter at their start and end into a log armed by kvdec_clock_arm (the
loader takes it when KVDEC_LIBRARY=clock; bench.py --kernel-clock).
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(os.path.dirname(HERE), "include")
BUILD_DIR = os.path.join(HERE, "_build")
LIB_PATH = os.path.join(HERE, "libkvdec.so")
ARCH = "gfx950"

SOURCES = (
    ("attn.hip", []),
    ("quant.hip", ["-ffp-contract=off"]),
    ("generic.hip", []),
)
CLOCK_LIB_PATH = os.path.join(HERE, "libkvdec_clock.so")
# object name, source, extra flags; each library links the objects it names
OBJECTS = (
    ("attn", "attn.hip", []),
    ("attn_clock", "attn.hip", ["-DKVDEC_CLOCK"]),
    ("quant", "quant.hip", ["-ffp-contract=off"]),
    ("generic", "generic.hip", []),
)
LIBRARIES = (
    (LIB_PATH, ("attn", "quant", "generic")),
    (CLOCK_LIB_PATH, ("attn_clock", "quant", "generic")),
)

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-Wall",
    # packed fp32 (v_pk_*_f32) stays off: all fp32 math is scalar VALU or MFMA
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", INCLUDE,
    "-I", CSRC,
]


def _hipcc() -> str:
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm toolchain required to build libkvdec.so)")


def _filter_host_feature_warning(text: str) -> str:
    # The host pass does not know the GPU-only target feature; that warning
    # is expected and harmless.
    keep = [ln for ln in text.splitlines() if "is not a recognized feature for this target" not in ln]
    return "\n".join(keep)


def build(verbose: bool = False) -> str:
    """Compile every HIP source and link libkvdec.so and the timing build
    libkvdec_clock.so; returns the product library's path."""
    hipcc = _hipcc()
    os.makedirs(BUILD_DIR, exist_ok=True)
    procs = []
    objs = {}
    for name, src, extra in OBJECTS:
        obj = os.path.join(BUILD_DIR, name + ".o")
        cmd = [hipcc, *COMMON_FLAGS, *extra, "-c", os.path.join(CSRC, src), "-o", obj]
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((name, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)))
        objs[name] = obj
    failed = []
    for name, p in procs:
        out, _ = p.communicate()
        out = _filter_host_feature_warning(out)
        if out.strip() and (verbose or p.returncode):
            print(out, file=sys.stderr)
        if p.returncode:
            failed.append(name)
    if failed:
        raise RuntimeError(f"hipcc failed on {', '.join(failed)}")
    for lib, names in LIBRARIES:
        tmp = lib + ".tmp"
        cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *[objs[n] for n in names]]
        if verbose:
            print(" ".join(cmd), flush=True)
        r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
        if r.returncode:
            print(r.stdout, file=sys.stderr)
            raise RuntimeError(f"linking {os.path.basename(lib)} failed")
        os.replace(tmp, lib)
    return LIB_PATH


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print(path)
