"""The C++ host layer over the C ABI (hllm_amd/host): JSON / Safetensors readers, stage
admission, decode-batch packing, host sampling, the pass scheduler, and on a GPU the
RocmStage adapter loading a Safetensors checkpoint through its factory. Each case runs in
tests/host/host_tests.cpp's program (built by __graft_entry__.build())."""
import json
import os
import re
import subprocess

import numpy as np
import pytest

import oracle
from tests import models

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "hllm_amd", "_build", "host_tests")
VECTORS = os.path.join(ROOT, "tests", "golden", "sampling_vectors.json")


def _cases(kind):
    if not os.path.exists(BIN):
        return ["<host_tests not built>"]
    out = subprocess.run([BIN, "--list"], capture_output=True, text=True, check=True).stdout
    return [line.split()[0] for line in out.splitlines() if line.split()[1] == kind]


def _run(case, *args, timeout=60):
    assert os.path.exists(BIN), "host test program missing: run __graft_entry__.build()"
    print(f"[host] {case} {' '.join(map(str, args))}", flush=True)
    r = subprocess.run([BIN, case, *map(str, args)], capture_output=True, text=True, timeout=timeout)
    assert r.returncode == 0 and f"PASS {case}" in r.stdout, r.stdout + r.stderr
    return r.stdout


@pytest.mark.parametrize("case", _cases("cpu"))
def test_host_case(case):
    args = [VECTORS] if case == "host_sampling" else []
    _run(case, *args)


def _write_tiny_checkpoint(path):
    from safetensors.numpy import save_file
    fx = models.tiny_reference()
    w = models.tiny_reference_stage()
    save_file({k: np.ascontiguousarray(v, np.float32) for k, v in w.tensors.items()},
              str(path / "model.safetensors"))
    with open(path / "config.json", "w") as f:
        json.dump(fx["config"], f)
    return w


def _oracle_greedy(w, prompt, decodes):
    st = oracle.OracleStage(w)
    seq = st.allocate_sequence(len(prompt) + decodes + 1)
    tokens = [st.execute(np.array(prompt, np.uint64), 0, seq)[1]]
    for i in range(decodes):
        tokens.append(st.execute(np.array([tokens[-1]], np.uint64), len(prompt) + i, seq)[1])
    return tokens


@pytest.mark.gpu
def test_factory_loads_checkpoint_and_decodes_like_the_oracle(tmp_path):
    w = _write_tiny_checkpoint(tmp_path)
    prompt, decodes = [1, 4, 2, 8, 3], 6
    out = _run("gpu_checkpoint_greedy", tmp_path, "f32", ",".join(map(str, prompt)), decodes, timeout=120)
    got = json.loads(re.search(r"TOKENS (\[.*\])", out).group(1))
    assert got == _oracle_greedy(w, prompt, decodes)
    out = _run("gpu_checkpoint_greedy", tmp_path, "f16", ",".join(map(str, prompt)), decodes, timeout=120)
    got16 = json.loads(re.search(r"TOKENS (\[.*\])", out).group(1))
    assert got16 == _oracle_greedy(w, prompt, decodes)


@pytest.mark.gpu
def test_adapter_decode_batch_contract(tmp_path):
    _write_tiny_checkpoint(tmp_path)
    _run("gpu_decode_batch_contract", tmp_path, timeout=120)


@pytest.mark.gpu
def test_scheduler_runs_a_mixed_pass_on_the_stage(tmp_path):
    _write_tiny_checkpoint(tmp_path)
    _run("gpu_scheduler_mixed_pass", tmp_path, timeout=120)
