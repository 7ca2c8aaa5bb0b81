"""Builds libhllm_rocm.so (HIP kernels + stage runtime + C ABI) in-tree for gfx950."""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
LIBRARY = os.path.join(HERE, "libhllm_rocm.so")
SOURCES = ["kernels_misc.hip", "gemm.hip", "attention.hip", "stage.hip"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-Wall",
         # Packed FP32 instructions stay disabled in device code.
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         f"-I{os.path.join(ROOT, 'include')}", f"-I{CSRC}"]


def _quiet(text: str) -> str:
    # hipcc's host pass does not know the device-only feature flag; drop that notice.
    return "\n".join(l for l in text.splitlines() if "packed-fp32-ops" not in l)


def build(jobs: int = 4) -> str:
    os.makedirs(os.path.join(HERE, "_build"), exist_ok=True)
    objects, procs = [], []
    for src in SOURCES:
        obj = os.path.join(HERE, "_build", src.replace(".hip", ".o"))
        objects.append(obj)
        procs.append(subprocess.Popen([HIPCC, *FLAGS, "-c", os.path.join(CSRC, src), "-o", obj],
                                      stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True))
        while len([p for p in procs if p.poll() is None]) >= jobs:
            procs[0].wait()
    failed = False
    for src, p in zip(SOURCES, procs):
        out, _ = p.communicate()
        msg = _quiet(out or "").strip()
        if msg:
            print(f"[{src}]\n{msg}", file=sys.stderr)
        failed |= p.returncode != 0
    if failed:
        raise RuntimeError("HIP compilation failed")
    tmp = LIBRARY + ".tmp"
    r = subprocess.run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objects],
                       capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIBRARY)
    return LIBRARY


if __name__ == "__main__":
    print(build())
