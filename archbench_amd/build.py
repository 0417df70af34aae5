"""Builds the HIP C-ABI library libgdn_mi355x.so in-tree (gfx950 only).

    python -m archbench_amd.build            # compile every .hip under archbench_amd/csrc into one .so
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
import tempfile
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libgdn_mi355x.so")
ARCH = "gfx950"

# -packed-fp32-ops: keep the compiler from emitting packed fp32 VALU ops (v_pk_*_f32).
HIP_FLAGS = ["-O3", "-std=c++17", f"--offload-arch={ARCH}", "-fPIC", "-Wall", "-Wno-unused-function",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-munsafe-fp-atomics"]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm toolchain required to build the gdn kernels)")


def sources() -> list[str]:
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def source_digest() -> str:
    """SHA-256 (first 16 hex digits) over the kernel sources (csrc/*.hip and *.h, names and contents): the build a
    profile under profiles/ was measured on is recorded by it, so that bench.py uses a profile only with the
    sources it was taken from."""
    import hashlib

    h = hashlib.sha256()
    for f in sorted(os.listdir(CSRC)):
        if f.endswith((".hip", ".h")):
            h.update(f.encode() + b"\0")
            with open(os.path.join(CSRC, f), "rb") as fh:
                h.update(fh.read())
    return h.hexdigest()[:16]


def build(verbose: bool = False, jobs: int | None = None) -> str:
    cc = hipcc()
    srcs = sources()
    tmp = tempfile.mkdtemp(prefix="gdn_build_")
    try:
        def compile_one(src):
            obj = os.path.join(tmp, os.path.basename(src) + ".o")
            cmd = [cc, *HIP_FLAGS, "-c", src, "-o", obj]
            r = subprocess.run(cmd, capture_output=True, text=True)
            out = (r.stdout + r.stderr).strip()
            # hipcc's host pass does not know the packed-fp32 feature and says so; drop that line only
            out = "\n".join(x for x in out.splitlines() if "packed-fp32-ops' is not a recognized feature" not in x)
            if r.returncode != 0:
                raise RuntimeError(f"hipcc failed for {os.path.basename(src)}:\n{out}")
            if out and verbose:
                print(out, file=sys.stderr)
            return obj

        n = jobs or min(len(srcs), max(1, (os.cpu_count() or 4) // 2))
        with ThreadPoolExecutor(max_workers=n) as ex:
            objs = list(ex.map(compile_one, srcs))
        tmp_lib = LIB + ".tmp"
        cmd = [cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp_lib]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"link failed:\n{r.stdout}{r.stderr}")
        os.replace(tmp_lib, LIB)
    finally:
        shutil.rmtree(tmp, ignore_errors=True)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
