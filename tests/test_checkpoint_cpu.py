"""Adapter checkpoints (save_checkpoint / load_checkpoint of the C++ host
interface, after src/training/checkpoint.rs) against the safetensors library,
no GPU.

The reference writes checkpoints through the safetensors crate
(safetensors::serialize_to_file, checkpoint.rs:57-63). The Python
`safetensors` package wraps the same crate (0.8 here, the reference pins 0.4;
the container layout is the same), so it serves as the library cross-check:
  * the C++ writer's file for a set of tensors and metadata is byte-identical
    to safetensors.numpy.save_file's for the same tensors and metadata;
  * the C++ reader loads the library's file back exactly (checked inside the
    C++ case), and the library loads the C++ file back exactly.
The tensors are LoRA A / B of a 2-layer adapter (q, v, gate, down at hidden 16,
intermediate 24, rank 4), keyed "layers.{i}.{module}.lora_{a,b}", with values
given by a formula both sides compute; the metadata entry is
CheckpointMetadata {100, 1.5, 1e-4, 1234567890} as serde_json writes it.
"""
import os
import subprocess

import numpy as np
import safetensors.numpy as stn

import host_runner

HIDDEN, INTER, RANK = 16, 24, 4
MODULES = {"q_proj": (HIDDEN, HIDDEN), "v_proj": (HIDDEN, HIDDEN), "gate_proj": (HIDDEN, INTER),
           "down_proj": (INTER, HIDDEN)}
META = '{"global_step":100,"loss":1.5,"learning_rate":0.0001,"timestamp":1234567890}'


def formula_tensors():
    shapes = {}
    for layer in range(2):
        for m, (fin, fout) in MODULES.items():
            key = f"layers.{layer}.{m}"
            shapes[key + ".lora_a"] = (fin, RANK)
            shapes[key + ".lora_b"] = (RANK, fout)
    out = {}
    for k, name in enumerate(sorted(shapes)):
        r, c = shapes[name]
        i = np.arange(r)[:, None]
        j = np.arange(c)[None, :]
        out[name] = (((131 * k + 17 * i + 3 * j) % 97).astype(np.float32) / np.float32(100) - np.float32(0.5))
    return out


def test_checkpoint_bytes_match_safetensors(tmp_path):
    tensors = formula_tensors()
    py = tmp_path / "py.safetensors"
    stn.save_file(tensors, str(py), metadata={"checkpoint_metadata": META})
    env = dict(os.environ, MC_CKPT_DIR=str(tmp_path))
    p = subprocess.run([host_runner.BINARY, "--cpu", "checkpoint_format"], capture_output=True, text=True,
                       timeout=120, env=env)
    assert p.returncode == 0 and "[     OK ] checkpoint_format" in p.stdout, p.stdout[-2000:]
    cpp = tmp_path / "cpp.safetensors"
    assert cpp.read_bytes() == py.read_bytes()
    back = stn.load_file(str(cpp))
    assert sorted(back) == sorted(tensors)
    for k, v in tensors.items():
        assert back[k].dtype == np.float32 and np.array_equal(back[k], v)
