"""The C++ host API (libkuiper_host.so: base::DeviceType::kDeviceHIP, the
pooled HIP allocator, Buffer/Tensor, op:: layers, kernel:: adapters and
model::Model) through its C++ test program tests/cpp/_build/test_host.

* ``cpu_*`` units (no GPU): buffers, tensors, status codes, kernel factories,
  layer checks returning a Status, model-file errors (bad path, truncated
  image, Qwen3 int8 refused).
* ``hip_*`` units (GPU): the reference's op tests (matmul known answers,
  int8 matmul, rmsnorm, per-row rmsnorm, add, in-place SwiGLU, embedding,
  first-max argmax, allocator reuse, tensor moves).
* whole model (GPU): a synthetic image loaded by model::Model, driven the way
  demo/main.cpp drives it, layer by layer and fused; first-step logits within
  1e-4 relative of the CPU oracle and greedy tokens identical to it; the same
  loop through a subclass that overrides the virtual predict().
"""
import json
import os
import subprocess

import numpy as np
import pytest

from conftest import ROOT

BIN = os.path.join(ROOT, "tests", "cpp", "_build", "test_host")
LOGIT_RTOL = 1e-4


def run(args, timeout=120):
    if not os.path.exists(BIN):
        pytest.fail(f"{BIN} is not built (run __graft_entry__.build())")
    p = subprocess.run([BIN] + args, capture_output=True, text=True, timeout=timeout)
    print(p.stdout[-4000:], p.stderr[-4000:], flush=True)
    return p


def test_host_cpu_units():
    p = run(["unit", "cpu_"])
    assert p.returncode == 0, p.stdout + p.stderr
    assert "[FAIL]" not in p.stdout


@pytest.mark.gpu
def test_host_hip_units(gpu):
    p = run(["unit", "hip_"])
    assert p.returncode == 0, p.stdout + p.stderr
    assert "[FAIL]" not in p.stdout and "0 failed" in p.stdout


def rel(a, b):
    return float(np.max(np.abs(a.astype(np.float64) - b)) / max(np.max(np.abs(b)), 1e-30))


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["tiny_llama2", "tiny_llama3", "tiny_q8", "tiny_qwen2",
                                  "tiny_qwen2_q8", "tiny_qwen3"])
def test_host_model_matches_oracle(K, O, gpu, tmp_path, name):
    cfg = K.TINY[name]
    img = K.synth_image(cfg)
    path = str(tmp_path / f"{name}.bin")
    img.tofile(path)
    prompt = [int(t) for t in K.prompt_tokens(cfg, 5)]
    n_new = 8
    print(f"host model {name}: prompt {prompt}", flush=True)
    p = run(["model", path, str(cfg.family), str(int(cfg.quant)), str(n_new)] +
            [str(t) for t in prompt])
    assert p.returncode == 0, p.stdout + p.stderr
    out = json.loads(p.stdout.strip().splitlines()[-1])
    assert out["dims"] == [cfg.dim, cfg.qd, cfg.kv_dim, cfg.hidden_dim, cfg.layers, cfg.heads,
                           cfg.kv_heads, cfg.vocab]

    om = O.Model(img, cfg.family, cfg.quant)
    ref = om.step(prompt[0], 0)
    for kind in ("layered", "fused"):
        lg = np.fromfile(path + ".logits_" + kind, dtype=np.float32)
        assert lg.shape == ref.shape
        r = rel(lg, ref)
        print(f"{name} {kind} first-step logits rel err {r:.2e}", flush=True)
        assert r < LOGIT_RTOL, (name, kind, r)

    want = [int(t) for t in O.Model(img, cfg.family, cfg.quant).generate(prompt, n_new)]
    assert out["layered"] == want, (out["layered"], want)
    assert out["fused"] == want, (out["fused"], want)
    assert out["fused_steps"] == want, (out["fused_steps"], want)
    # a subclass overriding predict() (llama3.h:33-53): generate() reaches it
    # once per position, and its tokens are the oracle's
    assert out["subclass"] == want, (out["subclass"], want)
    assert out["subclass_predict_calls"] == len(prompt) + n_new - 1
