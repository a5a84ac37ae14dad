"""Build libsimsd_kernels.so (HIP, gfx950) in-tree, next to the Python package.

    python simsd-release_amd/build_lib.py            # build
    python simsd-release_amd/build_lib.py --verbose  # echo the hipcc line

The library is compiled ahead of time, so nothing JIT-compiles at import or
inside a captured graph.  All device code is built with packed-fp32 ops
disabled (the compiler would otherwise form v_pk_*_f32 from plain float code).
"""
from __future__ import annotations

import argparse
import concurrent.futures
import os
import shutil
import subprocess
import sys
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(REPO, "include")
OUT = os.path.join(HERE, "kernels", "libsimsd_kernels.so")

SOURCES = ["capi.cpp", "thin_gemm.hip", "moe.hip", "logits.hip", "attention.hip"]
# gfx950 only: tiles rely on its 160 KiB of LDS per workgroup and on its
# instructions (v_permlane32_swap, the 16x16x32 bf16 MFMA)
ARCH = "gfx950"


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def flags(extra=()) -> list[str]:
    return [
        f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wno-unused-command-line-argument",
        # leading scalar kernel arguments arrive in SGPRs (no kernarg fetch
        # before a kernel's first loads); kernels whose first argument is a
        # struct are unaffected
        "-mllvm", "-amdgpu-kernarg-preload-count=16",
        "-I", INCLUDE, "-I", CSRC, *extra,
    ]


def command(out: str = OUT, extra=()) -> list[str]:
    """The equivalent single hipcc line (what --verbose prints)."""
    srcs = [os.path.join(CSRC, s) for s in SOURCES]
    return [hipcc(), *flags(extra), "-shared", "-o", out, *srcs]


def _run(cmd: list[str]) -> str:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    # The host pass does not know the packed-fp32 feature and says so; that
    # line is expected.  Anything else on stderr is shown.
    noise = "'-packed-fp32-ops' is not a recognized feature"
    errs = "\n".join(l for l in proc.stderr.splitlines() if noise not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{errs}")
    return errs


def build(verbose: bool = False, out: str = OUT, extra=()) -> str:
    """Compile every source to an object in parallel, then link the library
    (same result as the single line from command())."""
    if verbose:
        print(" ".join(command(out, extra)), flush=True)
    with tempfile.TemporaryDirectory(prefix="simsd_build_") as tmpdir:
        objs = [os.path.join(tmpdir, os.path.splitext(s)[0] + ".o") for s in SOURCES]
        jobs = [[hipcc(), *flags(extra), "-c", "-o", o, os.path.join(CSRC, s)] for s, o in zip(SOURCES, objs)]
        workers = max(1, min(len(jobs), os.cpu_count() or 1, 8))
        with concurrent.futures.ThreadPoolExecutor(workers) as pool:
            errs = list(pool.map(_run, jobs))
        tmp = out + ".tmp"
        errs.append(_run([hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]))
    text = "\n".join(e for e in errs if e.strip())
    if text and verbose:
        print(text, file=sys.stderr)
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--verbose", action="store_true")
    args = ap.parse_args()
    print(build(verbose=args.verbose))
