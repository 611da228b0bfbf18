"""Build the gfx950 HIP library ``catfuse_amd/_lib/libcatfuse_amd.so``.

Every ``catfuse_amd/csrc/*.hip`` file is compiled with hipcc for gfx950 and
linked into one shared library exporting the C-ABI declared in
``include/catfuse_amd.h``.  Numerics flags:

* ``-ffp-contract=off``: no fused multiply-add contraction, so the LIF
  recurrence rounds each operation separately (SpikingJelly op order).
* ``-fhip-fp32-correctly-rounded-divide-sqrt``: ``(x - v) / tau`` is an
  IEEE division.
* ``-fno-gpu-flush-denormals-to-zero``: fp32 denormals are kept.
* ``-Xclang -target-feature -Xclang -packed-fp32-ops``: no packed fp32
  instructions are emitted.

Usage: ``python -m catfuse_amd.build`` (or ``catfuse_amd.build.build()``).
"""
from __future__ import annotations

import concurrent.futures as _cf
import hashlib
import os
import shutil
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG_DIR, "csrc")
INCLUDE = os.path.join(os.path.dirname(PKG_DIR), "include")   # the C-ABI header
LIB_DIR = os.path.join(PKG_DIR, "_lib")
LIB_NAME = "libcatfuse_amd.so"
BUILD_DIR = os.path.join(os.path.dirname(PKG_DIR), "_build", "catfuse_amd")

ARCH = os.environ.get("CATFUSE_AMD_ARCH", "gfx950")

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fvisibility=hidden",
    "-ffp-contract=off",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-fno-gpu-flush-denormals-to-zero",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def sources() -> list:
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def source_digest() -> str:
    """SHA-256 over the HIP sources and headers (with the C-ABI header) the
    library is built from."""
    h = hashlib.sha256()
    files = [os.path.join(CSRC, f) for f in sorted(os.listdir(CSRC)) if f.endswith((".hip", ".h"))]
    files.append(os.path.join(INCLUDE, "catfuse_amd.h"))
    for path in files:
        h.update(os.path.basename(path).encode())
        with open(path, "rb") as fh:
            h.update(fh.read())
    return h.hexdigest()


def stamp_path() -> str:
    return os.path.join(LIB_DIR, LIB_NAME + ".sources")


def _compile(src: str, hipcc: str) -> str:
    obj = os.path.join(BUILD_DIR, os.path.basename(src)[:-4] + ".o")
    cmd = [hipcc, *HIPCC_FLAGS, "-I", CSRC, "-I", INCLUDE, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return obj


def build(verbose: bool = True, jobs: int = 0) -> str:
    """Compile every HIP source and link the shared library; returns its path."""
    hipcc = _hipcc()
    os.makedirs(BUILD_DIR, exist_ok=True)
    os.makedirs(LIB_DIR, exist_ok=True)
    srcs = sources()
    digest = source_digest()
    jobs = jobs or min(len(srcs), max(1, (os.cpu_count() or 4) - 1), 8)
    with _cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, hipcc), srcs))
    out = os.path.join(LIB_DIR, LIB_NAME)
    tmp = out + ".tmp"
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, out)
    with open(stamp_path(), "w") as fh:   # the sources this library was built from
        fh.write(digest + "\n")
    if verbose:
        print(f"[catfuse_amd.build] {len(srcs)} sources -> {out}")
    return out


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
