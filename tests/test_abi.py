"""CPU checks of the C ABI: the library loads, exports every function include/hllm_rocm.h
declares, and the ctypes mirrors have the C layouts (gcc compiles the header)."""
import ctypes as C
import os
import re
import subprocess
import tempfile

import pytest

from hllm_amd import capi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "hllm_rocm.h")


def declared_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\**\s+\**(hllm_rocm_\w+)\s*\(", text, re.M)))


def test_library_exports_every_declared_function():
    lib = capi.library()
    names = declared_functions()
    assert len(names) >= 20
    for name in names:
        assert hasattr(lib, name), name
    assert set(names) == set(capi.EXPORTS)
    out = subprocess.run(["nm", "-D", "--defined-only", capi.LIBRARY], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r" T (hllm_rocm_\w+)", out))
    assert set(names) <= exported


def test_abi_version():
    assert capi.library().hllm_rocm_abi_version() == capi.ABI_VERSION


@pytest.mark.parametrize("struct,cname", [(capi.StageConfig, "hllm_rocm_stage_config"),
                                          (capi.Item, "hllm_rocm_item"),
                                          (capi.Pass, "hllm_rocm_pass"),
                                          (capi.Memory, "hllm_rocm_memory"),
                                          (capi.PhaseTime, "hllm_rocm_phase_time")])
def test_struct_layouts_match_header(struct, cname):
    fields = [f for f, _ in struct._fields_]
    body = "\n".join(f'  printf("%zu ", offsetof({cname}, {f}));' for f in fields)
    src = f"""#include <stddef.h>
#include <stdio.h>
#include "hllm_rocm.h"
int main(void) {{
{body}
  printf("%zu\\n", sizeof({cname}));
  return 0;
}}
"""
    with tempfile.TemporaryDirectory() as d:
        c_file, exe = os.path.join(d, "probe.c"), os.path.join(d, "probe")
        open(c_file, "w").write(src)
        subprocess.run(["gcc", "-I", os.path.join(ROOT, "include"), c_file, "-o", exe], check=True)
        got = [int(x) for x in subprocess.run([exe], capture_output=True, text=True,
                                              check=True).stdout.split()]
    expect = [getattr(struct, f).offset for f in fields] + [C.sizeof(struct)]
    assert got == expect


def test_calls_without_a_stage_fail_cleanly():
    lib = capi.library()
    assert lib.hllm_rocm_stage_finalize(None) == capi.INVALID_REQUEST
    assert b"null" in lib.hllm_rocm_last_error()
    assert lib.hllm_rocm_stage_create(None, None) == capi.INVALID_REQUEST


def test_gemm_configuration_hook_validates_and_restores():
    previous = capi.set_gemm_config(-1)
    assert capi.set_gemm_config(previous) == -1
    for bad in (-2, 19):
        with pytest.raises(capi.StageError) as e:
            capi.set_gemm_config(bad)
        assert e.value.status == capi.INVALID_REQUEST


def test_read_probe_validates_sizes_before_touching_a_device():
    for bad in (0, 1000, (1 << 20) + 8, 65 << 30):
        with pytest.raises(capi.StageError) as e:
            capi.measure_read_bandwidth(bad)
        assert e.value.status == capi.INVALID_REQUEST
