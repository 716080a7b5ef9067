"""Builds libproxima_hip.so in place from proxima_amd/csrc/*.hip with hipcc
for gfx950. Run `python proxima_amd/build.py` (or __graft_entry__.build())."""
import glob
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libproxima_hip.so")
ARCH = os.environ.get("PXG_OFFLOAD_ARCH", "gfx950")

FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # exact kernels restate the reference's arithmetic: no FMA contraction
    "-ffp-contract=off",
    # packed FP32 ops are kept out of every kernel
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-result",
]


def sources():
    return sorted(glob.glob(os.path.join(CSRC, "*.hip")))


NOISE = ("unknown target feature", "packed-fp32-ops", "warning: argument unused")


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    msgs = [ln for ln in (res.stdout + res.stderr).splitlines() if not any(n in ln for n in NOISE)]
    if res.returncode != 0:
        sys.stderr.write("\n".join(msgs) + "\n")
        raise RuntimeError(f"hipcc failed ({res.returncode}): {' '.join(cmd)}")
    if verbose and msgs:
        print("\n".join(msgs))


def build(verbose=False, jobs=None):
    """Compile each source to an object in parallel (every source is
    self-contained: kernels and their device helpers live in one translation
    unit), then link the shared library."""
    hipcc = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
    objdir = os.path.join(HERE, "_build")
    os.makedirs(objdir, exist_ok=True)
    srcs = sources()
    objs = [os.path.join(objdir, os.path.basename(s)[:-4] + ".o") for s in srcs]
    jobs = jobs or min(len(srcs), os.cpu_count() or 4, 8)
    with ThreadPoolExecutor(jobs) as pool:
        for f in [pool.submit(_run, [hipcc, *FLAGS, "-c", s, "-o", o], verbose) for s, o in zip(srcs, objs)]:
            f.result()
    tmp = LIB + ".tmp"
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp], verbose)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
