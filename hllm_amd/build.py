"""Builds, in-tree: libhllm_rocm.so (HIP kernels + stage runtime + C ABI, gfx950),
libhllm_rocm_host.so (the C++ stage-backend adapter, loader and scheduler over that ABI)
and the host test program tests/host/host_tests.cpp (into _build/host_tests).

`python -m hllm_amd.build --sanitize address|thread` builds the host test program with the
host layer instrumented by ASan + UBSan (g++) or TSan (clang) into _build/host_tests_<kind>;
tests/test_host.py runs every CPU case under both."""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
LIBRARY = os.path.join(HERE, "libhllm_rocm.so")
SOURCES = ["kernels_misc.hip", "gemm.hip", "attention.hip", "sampling.hip", "sample_static.hip", "stage.hip"]
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
    build_host()
    return LIBRARY


HOST = os.path.join(HERE, "host")
HOST_LIBRARY = os.path.join(HERE, "libhllm_rocm_host.so")
HOST_SOURCES = ["json.cpp", "safetensors.cpp", "dense_loader.cpp", "scheduler.cpp", "rocm_stage.cpp"]
TEST_DIR = os.path.join(ROOT, "tests", "host")
# The host test program: its cases, plus the host sampler they check (not part of the library).
TEST_SOURCES = [os.path.join(TEST_DIR, "host_tests.cpp"), os.path.join(TEST_DIR, "host_sampling.cpp")]
HOST_TESTS = os.path.join(HERE, "_build", "host_tests")
CXX = os.environ.get("CXX", "g++")
CXXFLAGS = ["-std=c++20", "-O2", "-fPIC", "-Wall", "-Wextra", f"-I{os.path.join(ROOT, 'include')}", f"-I{HOST}",
            f"-I{TEST_DIR}"]
# Sanitized host test programs (host code only; the HIP library is linked as built):
# "address" = ASan + UBSan with g++, "thread" = TSan with clang (GCC 11's TSan reports false
# double locks around condition_variable::wait_for).
SANITIZERS = {
    "address": ("g++", ["-fsanitize=address,undefined", "-fno-omit-frame-pointer", "-fno-sanitize-recover=undefined"]),
    "thread": ("/opt/rocm/llvm/bin/clang++", ["-fsanitize=thread", "-fno-omit-frame-pointer"]),
}


def build_host() -> str:
    """The host adapter library (links libhllm_rocm.so) and its test program."""
    tmp = HOST_LIBRARY + ".tmp"
    srcs = [os.path.join(HOST, s) for s in HOST_SOURCES]
    r = subprocess.run([CXX, *CXXFLAGS, "-shared", "-o", tmp, *srcs, f"-L{HERE}", "-lhllm_rocm",
                        "-Wl,-rpath,$ORIGIN", "-pthread"], capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"host library build failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, HOST_LIBRARY)
    r = subprocess.run([CXX, *CXXFLAGS, "-o", HOST_TESTS + ".tmp", *TEST_SOURCES, f"-L{HERE}", "-lhllm_rocm_host",
                        "-lhllm_rocm", "-Wl,-rpath,$ORIGIN/..", "-pthread"], capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"host test build failed:\n{r.stdout}\n{r.stderr}")
    os.replace(HOST_TESTS + ".tmp", HOST_TESTS)
    return HOST_LIBRARY


def build_sanitized_host_tests(kind: str) -> str:
    """The host test program with the host layer compiled in and instrumented by `kind`
    ("address" or "thread"): _build/host_tests_<kind>. Links the built libhllm_rocm.so."""
    compiler, flags = SANITIZERS[kind]
    out = os.path.join(HERE, "_build", f"host_tests_{kind}")
    os.makedirs(os.path.dirname(out), exist_ok=True)
    cxxflags = [f for f in CXXFLAGS if f != "-O2"] + ["-O1", "-g"]
    srcs = [os.path.join(HOST, s) for s in HOST_SOURCES] + TEST_SOURCES
    r = subprocess.run([compiler, *cxxflags, *flags, "-o", out + ".tmp", *srcs, f"-L{HERE}", "-lhllm_rocm",
                        "-Wl,-rpath,$ORIGIN/..", "-pthread"], capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"sanitized host test build failed:\n{r.stdout}\n{r.stderr}")
    os.replace(out + ".tmp", out)
    return out


if __name__ == "__main__":
    import argparse

    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--sanitize", choices=sorted(SANITIZERS),
                    help="build only the sanitized host test program (after a full build)")
    ns = ap.parse_args()
    print(build_sanitized_host_tests(ns.sanitize) if ns.sanitize else build())
