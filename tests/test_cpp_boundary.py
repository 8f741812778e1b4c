"""The C++ boundary on the CPU: tests/cpp/boundary_test.cpp compiled with g++ from the product headers and host
sources alone (no HIP), then run. It checks the reference's block-manager unit test, ModelConfig against Qwen3-0.6B's
published parameter counts, the JSON parser, the engine's page logic (admission by prefix match, ensure / seal /
preempt, chunked prefill, speculative verify with rollback) driving a read-back Backend subclass over the product
BlockManager, and reads a model directory written here with the safetensors package."""
import json
import shutil
import subprocess
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
HOST = ROOT / "ember_amd" / "csrc" / "host"
SOURCES = [HOST / "kvcache" / "block_manager.cpp", HOST / "model" / "config.cpp", HOST / "model" / "safetensors.cpp",
           HOST / "common" / "json.cpp", HOST / "common" / "mmap_file.cpp"]


# The plain build, and one with the undefined-behaviour sanitizer (every finding fatal) and libstdc++'s checked
# containers and iterators, over the same host sources and scenarios.
CHECKED = ["-fsanitize=undefined", "-fno-sanitize-recover=all", "-D_GLIBCXX_ASSERTIONS", "-g"]


@pytest.fixture(scope="module", params=["plain", "checked"])
def boundary_binary(request, tmp_path_factory):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ is not installed")
    out = tmp_path_factory.mktemp("cpp") / f"boundary_test_{request.param}"
    extra = CHECKED if request.param == "checked" else []
    cmd = [gxx, "-std=c++20", "-O1", "-Wall", "-Wextra", "-Werror", *extra, f"-I{HOST}", f"-I{ROOT / 'include'}",
           str(ROOT / "tests" / "cpp" / "boundary_test.cpp"), *map(str, SOURCES), "-o", str(out)]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr
    return out


def _model_dir(tmp_path):
    from safetensors.numpy import save_file

    rng = np.random.default_rng(3)
    tensors = {
        "model.embed_tokens.weight": rng.standard_normal((16, 8)).astype(np.float16),
        "model.norm.weight": np.arange(8, dtype=np.float32),
        "model.layers.0.self_attn.q_norm.weight": np.full(4, 0.25, np.float32),
        "ids": np.array([[1, 2, 3], [4, 5, 6]], np.int32),
    }
    save_file(tensors, str(tmp_path / "model.safetensors"))
    (tmp_path / "config.json").write_text(json.dumps({
        "model_type": "qwen3", "vocab_size": 16, "hidden_size": 8, "intermediate_size": 24, "num_hidden_layers": 1,
        "num_attention_heads": 2, "num_key_value_heads": 1, "head_dim": 4, "eos_token_id": 3}))
    (tmp_path / "generation_config.json").write_text(json.dumps({"eos_token_id": [3, 5]}))
    return tmp_path


def test_boundary_program(boundary_binary, tmp_path):
    d = _model_dir(tmp_path)
    r = subprocess.run([str(boundary_binary), str(d)], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    lines = r.stdout.splitlines()
    assert lines[-1] == "boundary ok"
    assert "config qwen3 8 1 2 1 2" in lines  # generation_config's two eos ids
    tensors = {ln.split()[1]: ln.split()[2:] for ln in lines if ln.startswith("tensor ")}
    assert tensors["model.norm.weight"] == ["F32", "[8]", "28"]
    assert tensors["model.layers.0.self_attn.q_norm.weight"] == ["F32", "[4]", "1"]
    assert tensors["ids"] == ["I32", "[2,", "3]", "21"]
    assert tensors["model.embed_tokens.weight"][:3] == ["F16", "[16,", "8]"]


def test_corrupt_safetensors_is_refused(boundary_binary, tmp_path):
    d = _model_dir(tmp_path)
    blob = bytearray((d / "model.safetensors").read_bytes())
    blob[0:8] = (len(blob) + 5).to_bytes(8, "little")  # a header longer than the file
    (d / "model.safetensors").write_bytes(bytes(blob))
    r = subprocess.run([str(boundary_binary), str(d)], capture_output=True, text=True, timeout=300)
    assert r.returncode != 0 and "past the end of the file" in r.stderr
