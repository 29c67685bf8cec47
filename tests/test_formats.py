"""The .bin byte layouts against files written by the reference's own
exporters (tests/golden/fmt_*.bin, made by tests/golden/make_format_fixtures.py
with tools/export_llama.py, tools/export_qwen2.py and tools/export_qwen3.py
from the same seeded weights).

* CPU: this backend's image writer (kl_synth_image) produces the same bytes
  for the same spec (the fp32 v0 / Qwen2 freq tables aside: the reference
  writes cos/sin there, this writer zeros, and no loader reads them); the
  oracle parses every fixture and matches the independent fp64 model, which
  takes its weights from the generator streams, not from the file.
* GPU: the engine (both modes) and model::Model load every fixture and match
  the oracle.
"""
import json
import os

import numpy as np
import pytest

from conftest import GOLDEN

MANIFEST = os.path.join(GOLDEN, "fmt_manifest.json")


def fixtures():
    with open(MANIFEST) as f:
        return json.load(f)


NAMES = sorted(fixtures()["files"])


def cfg_of(K, name):
    m = fixtures()
    spec = dict(m["files"][name]["spec"])
    return K.Config(name=name, family=spec["family"], dim=spec["dim"],
                    hidden_dim=spec["hidden_dim"], layers=spec["layers"], heads=spec["heads"],
                    kv_heads=spec["kv_heads"], vocab=spec["vocab"], seq_len=spec["seq_len"],
                    tied=bool(spec["tied"]), q_dim=spec["q_dim"], group_size=spec["group_size"],
                    norm_std=m["norm_stddev"], prompt_len=5, decode_steps=8)


def load(name):
    return np.fromfile(os.path.join(GOLDEN, name + ".bin"), np.uint8)


def freq_region(cfg):
    """Byte range of freq_cos + freq_sin in the fp32 v0 / Qwen2 layouts
    (export_llama.py:124-126), or None for layouts without it."""
    if cfg.family == 3 or cfg.quant:
        return None
    D, Dq, Dkv, F, L, V = cfg.dim, cfg.qd, cfg.kv_dim, cfg.hidden_dim, cfg.layers, cfg.vocab
    b = (Dq + 2 * Dkv) if cfg.family == 2 else 0
    floats = V * D + L * D + L * (Dq * D + 2 * Dkv * D + b) + L * D * Dq + L * D + 3 * L * F * D + D
    off = 28 + 4 * floats
    return off, off + 4 * cfg.seq_len * cfg.head_size


def rel(a, b):
    return float(np.max(np.abs(a.astype(np.float64) - b)) / max(np.max(np.abs(b)), 1e-30))


def test_manifest_names_reference_writers():
    m = fixtures()
    assert m["seed"] == 1234 and m["stddev"] == 0.02 and m["norm_stddev"] == 0.1
    writers = {v["writer"] for v in m["files"].values()}
    assert writers == {"tools/export_llama.py:legacy_export",
                       "tools/export_llama.py:legacy_export_quant",
                       "tools/export_qwen2.py:legacy_export",
                       "tools/export_qwen2.py:legacy_export_quant",
                       "tools/export_qwen3.py:export_qwen3_bin"}


@pytest.mark.parametrize("name", NAMES)
def test_writer_matches_reference_exporter(K, name):
    cfg = cfg_of(K, name)
    ref = load(name)
    mine = K.synth_image(cfg)
    assert mine.size == ref.size, (mine.size, ref.size)
    region = freq_region(cfg)
    if region is None:
        assert np.array_equal(mine, ref)
    else:
        a, b = region
        assert np.array_equal(mine[:a], ref[:a])
        assert np.array_equal(mine[b:], ref[b:])
        # the reference writes real tables there: cos(0) = 1 opens freq_cos
        cos0 = np.frombuffer(ref[a:a + 4].tobytes(), np.float32)[0]
        assert cos0 == 1.0
    # the header the reference wrote
    h = np.frombuffer(ref[:32].tobytes(), np.int32)
    if cfg.family == 3:
        assert list(h[:8]) == [cfg.qd, cfg.dim, cfg.layers, cfg.heads, cfg.kv_heads, cfg.vocab,
                               cfg.seq_len, cfg.hidden_dim]
    else:
        vocab = cfg.vocab if cfg.tied else -cfg.vocab
        assert list(h[:7]) == [cfg.dim, cfg.hidden_dim, cfg.layers, cfg.heads, cfg.kv_heads,
                               vocab, cfg.seq_len]
        if cfg.quant:
            assert h[7] == cfg.group_size


@pytest.mark.parametrize("name", NAMES)
def test_oracle_reads_reference_files(K, O, name):
    from npmodel import NpModel

    cfg = cfg_of(K, name)
    om = O.Model(load(name), cfg.family, cfg.quant)
    nm = NpModel(K, cfg)
    for pos, t in enumerate(K.prompt_tokens(cfg, 8)):
        assert rel(om.step(int(t), pos), nm.step(int(t), pos)) < 2e-5, (name, pos)


@pytest.mark.gpu
@pytest.mark.parametrize("name", NAMES)
def test_engine_reads_reference_files(K, O, gpu, name):
    cfg = cfg_of(K, name)
    img = load(name)
    prompt = K.prompt_tokens(cfg, 5)
    want = O.Model(img, cfg.family, cfg.quant).generate(prompt, 8)
    for mode in (K.MODE_PERSISTENT, K.MODE_MULTI):
        eng = K.Engine(img, cfg)
        eng.set_mode(mode)
        om = O.Model(img, cfg.family, cfg.quant)
        for pos, t in enumerate(prompt):
            _, lg = eng.step(int(t), pos)
            assert rel(lg, om.step(int(t), pos)) < 1e-4, (name, mode, pos)
        eng2 = K.Engine(img, cfg)
        eng2.set_mode(mode)
        got, _ = eng2.generate(prompt, 8)
        assert list(got) == list(want), (name, mode)


@pytest.mark.gpu
@pytest.mark.parametrize("name", NAMES)
def test_host_model_reads_reference_files(K, O, gpu, tmp_path, name):
    import json as js
    import shutil

    from test_host_cpp import run

    cfg = cfg_of(K, name)
    path = str(tmp_path / (name + ".bin"))
    shutil.copyfile(os.path.join(GOLDEN, name + ".bin"), path)
    prompt = [int(t) for t in K.prompt_tokens(cfg, 5)]
    p = run(["model", path, str(cfg.family), str(int(cfg.quant)), "8"] + [str(t) for t in prompt])
    assert p.returncode == 0, p.stdout + p.stderr
    out = js.loads(p.stdout.strip().splitlines()[-1])
    want = [int(t) for t in O.Model(load(name), cfg.family, cfg.quant).generate(prompt, 8)]
    assert out["layered"] == want and out["fused"] == want
