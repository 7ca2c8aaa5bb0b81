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


@pytest.mark.parametrize("kind", ["address", "thread"])
def test_host_cases_under_sanitizers(kind):
    """Every CPU case with the host layer built under ASan + UBSan (g++) or TSan (clang);
    any sanitizer report fails the case (ASan, UBSan and TSan exit non-zero on a report)."""
    from hllm_amd import build
    program = build.build_sanitized_host_tests(kind)
    env = dict(os.environ, TSAN_OPTIONS="halt_on_error=1", ASAN_OPTIONS="halt_on_error=1",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
    for case in _cases("cpu"):
        args = [VECTORS] if case == "host_sampling" else []
        r = subprocess.run([program, case, *args], capture_output=True, text=True, timeout=120, env=env)
        assert r.returncode == 0 and f"PASS {case}" in r.stdout, (kind, case, r.stdout + r.stderr)


def _write_tiny_checkpoint(path, max_positions=None):
    """The reference's tiny Qwen3 fixture as a checkpoint (`max_positions` overrides its
    context of 32 positions, for longer passes)."""
    from safetensors.numpy import save_file
    fx = models.tiny_reference()
    w = models.tiny_reference_stage()
    save_file({k: np.ascontiguousarray(v, np.float32) for k, v in w.tensors.items()},
              str(path / "model.safetensors"))
    cfg = dict(fx["config"])
    if max_positions:
        cfg["max_position_embeddings"] = max_positions
    with open(path / "config.json", "w") as f:
        json.dump(cfg, f)
    return w


def _bf16_bits(values):
    """Round-to-nearest-even F32 -> BF16 bits (finite inputs)."""
    bits = np.ascontiguousarray(values, np.float32).view(np.uint32).astype(np.uint64)
    return ((bits + 0x7FFF + ((bits >> 16) & 1)) >> 16).astype(np.uint16)


def _write_safetensors(path, tensors):
    """Writes a Safetensors file from {name: (dtype name, numpy array of its storage)}."""
    header, blobs, offset = {"__metadata__": {"format": "pt"}}, [], 0
    for name, (dtype, arr) in tensors.items():
        data = np.ascontiguousarray(arr).tobytes()
        header[name] = {"dtype": dtype, "shape": list(arr.shape), "data_offsets": [offset, offset + len(data)]}
        blobs.append(data)
        offset += len(data)
    text = json.dumps(header).encode()
    text += b" " * (-len(text) % 8)
    with open(path, "wb") as f:
        f.write(len(text).to_bytes(8, "little") + text + b"".join(blobs))


def _write_variant_checkpoint(path, architecture, tied, storage):
    """The reference's tiny Qwen3 fixture as a {qwen3, llama} x {tied, untied} checkpoint
    stored as F32, F16 or BF16; returns the oracle's weights (the stored values in F32).
    The Llama variant drops the q/k norms; the untied head is the embedding with its rows
    rotated by three and scaled by 0.9."""
    fx = models.tiny_reference()
    base = models.tiny_reference_stage()
    shape = models.tiny_reference_shape()
    qk = architecture == "qwen3"
    names = [n for n in base.tensors if qk or not n.endswith(("q_norm.weight", "k_norm.weight"))]
    names = [n for n in names if n != "lm_head.weight"]
    values = {n: np.asarray(base.tensors[n], np.float32) for n in names}
    if not tied:
        values["lm_head.weight"] = (np.roll(values["model.embed_tokens.weight"], 3, axis=0) * 0.9).astype(np.float32)
    stored, seen = {}, {}
    for n, v in values.items():
        if storage == "F32":
            stored[n], seen[n] = ("F32", v), v
        elif storage == "F16":
            bits = oracle.f16_encode(v)
            stored[n], seen[n] = ("F16", bits), oracle.f16_decode(bits)
        else:
            bits = _bf16_bits(v)
            stored[n], seen[n] = ("BF16", bits), (bits.astype(np.uint32) << 16).view(np.float32)
    _write_safetensors(path / "model.safetensors", stored)
    cfg = dict(fx["config"], model_type=architecture, tie_word_embeddings=tied)
    with open(path / "config.json", "w") as f:
        json.dump(cfg, f)
    oshape = shape.__class__(**{**shape.__dict__, "qk_norm": qk, "tied": tied})
    w = oracle.StageWeights(models.oracle_config(oshape), shape.vocab, 0, shape.layers, True, True, tied)
    w.tensors.update({n: seen[n].reshape(values[n].shape) for n in values})
    return w


def _oracle_greedy(w, prompt, decodes, logprobs=False):
    """Greedy tokens (and, with `logprobs`, each step's five best (id, log-probability))."""
    st = oracle.OracleStage(w)
    seq = st.allocate_sequence(len(prompt) + decodes + 1,
                               oracle.Sampling(return_logprobs=True, top_logprobs=5) if logprobs else None)
    outs = [st.execute(np.array(prompt, np.uint64), 0, seq)]
    for i in range(decodes):
        outs.append(st.execute(np.array([outs[-1][1]], np.uint64), len(prompt) + i, seq))
    tokens = [o[1] for o in outs]
    return (tokens, [o[3] for o in outs]) if logprobs else tokens


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


@pytest.mark.gpu
def test_adapter_execute_profiled_and_factory_diagnostics(tmp_path):
    _write_tiny_checkpoint(tmp_path)
    print(_run("gpu_adapter_profiled_and_diagnostics", tmp_path, timeout=120))


@pytest.mark.gpu
def test_adapter_cancels_inside_a_pass_and_fails_the_sequence(tmp_path):
    _write_tiny_checkpoint(tmp_path, max_positions=1024)
    print(_run("gpu_adapter_cancellation", tmp_path, timeout=120))


@pytest.mark.gpu
@pytest.mark.parametrize("storage", ["F32", "F16", "BF16"])
@pytest.mark.parametrize("tied", [True, False])
@pytest.mark.parametrize("architecture", ["qwen3", "llama"])
def test_factory_storage_matrix_decodes_like_the_oracle(tmp_path, architecture, tied, storage):
    """{Llama, Qwen3} x {tied, untied} x {F32, F16, BF16} storage x {F32, F16} execution,
    loaded through the factory (Safetensors payloads converted on the device): greedy tokens
    equal the oracle's on the stored values (tests/cpp/cuda_stage_test.cpp:150-178)."""
    w = _write_variant_checkpoint(tmp_path, architecture, tied, storage)
    prompt, decodes = [1, 4, 2, 8, 3], 6
    expect, tops = _oracle_greedy(w, prompt, decodes, logprobs=True)
    for execution, tol in (("f32", 1e-4), ("f16", 2e-2)):
        out = _run("gpu_checkpoint_greedy", tmp_path, execution, ",".join(map(str, prompt)), decodes, "logprobs",
                   timeout=120)
        got = json.loads(re.search(r"TOKENS (\[.*\])", out).group(1))
        steps = [dict(json.loads(m)) for m in re.findall(r"TOP (\[.*\])", out)]
        assert len(steps) == len(tops) == len(got)
        # F32 execution gives the oracle's tokens; F16 execution too, or departs at a near
        # tie (the oracle's two best within 4e-2), after which the sequences differ.
        same = next((i for i, (g, e) in enumerate(zip(got, expect)) if g != e), len(expect))
        if same < len(expect):
            margin = tops[same][0][1] - tops[same][1][1]
            assert execution == "f16" and margin <= 4e-2, (architecture, tied, storage, execution, got, expect)
        # Each step's log-probabilities of the oracle's five best tokens (those the GPU also
        # ranks in its five best: near-equal values may swap places at the end).
        for step, (gpu, ref) in enumerate(zip(steps[:same + 1], tops[:same + 1])):
            assert int(ref[0][0]) in gpu, (execution, step)
            common = [(i, lp) for i, lp in ref if int(i) in gpu]
            assert len(common) >= 4, (execution, step, gpu, ref)
            for i, lp in common:
                assert abs(gpu[int(i)] - lp) <= tol, (architecture, tied, storage, execution, step, i, gpu[int(i)], lp)
