"""Writes tests/golden/fmt_*.bin: tiny model images produced by the
reference's OWN exporters, so the byte layouts this backend reads and writes
are pinned to them rather than to this repository's reading of them.

Run in the build container only (it imports the reference's Python tools from
/root/reference/tools, which never travel to the GPU box):

    python tests/golden/make_format_fixtures.py

Exporters used (the reference's functions, called unchanged):
  * tools/export_llama.py  legacy_export        (fp32 v0, :79-131)
  * tools/export_llama.py  legacy_export_quant  (int8 g64, :134-210)
  * tools/export_qwen2.py  legacy_export        (fp32 + q/k/v bias, :79-134)
  * tools/export_qwen2.py  legacy_export_quant  (int8 g64, :137-210)
  * tools/export_qwen3.py  export_qwen3_bin     (fp32 Qwen3, :193-253, from a
    HuggingFace-style directory: config.json + model.safetensors written here)

Every weight is taken from this repository's seeded generator streams
(kuiperllama_amd.synth_normal: role, layer), the same streams
kl_synth_image writes, so the fixture and this backend's own image of the same
spec can be compared byte for byte.  fmt_manifest.json records each file's
spec and seeds.
"""
from __future__ import annotations

import importlib
import json
import os
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
REF_TOOLS = "/root/reference/tools"

SEED, STD, NORM_STD = 1234, 0.02, 0.1
# synth.cpp roles
EMB, WQ, WK, WV, WO, W1, W2, W3, CLS, BQ, BK, BV = range(1, 13)
RMS_ATT, RMS_FFN, RMS_FINAL, Q_NORM, K_NORM = range(13, 18)

# name -> kl_model_spec fields (family 0 Llama2, 2 Qwen2, 3 Qwen3).  The int8
# images keep every row a whole number of 64-element groups (the decode
# engine's requirement; the reference's group index runs over the flattened
# matrix, the same thing when rows hold whole groups).
SPECS = {
    "fmt_llama_fp32": dict(family=0, dim=64, q_dim=64, hidden_dim=96, layers=2, heads=2,
                           kv_heads=1, vocab=128, seq_len=32, tied=0, group_size=0),
    "fmt_llama_q8": dict(family=0, dim=64, q_dim=64, hidden_dim=128, layers=2, heads=2,
                         kv_heads=1, vocab=128, seq_len=32, tied=0, group_size=64),
    "fmt_qwen2_fp32": dict(family=2, dim=64, q_dim=64, hidden_dim=96, layers=2, heads=2,
                           kv_heads=1, vocab=128, seq_len=32, tied=1, group_size=0),
    "fmt_qwen2_q8": dict(family=2, dim=64, q_dim=64, hidden_dim=128, layers=2, heads=2,
                         kv_heads=1, vocab=128, seq_len=32, tied=0, group_size=64),
    "fmt_qwen3_fp32": dict(family=3, dim=64, q_dim=128, hidden_dim=96, layers=2, heads=4,
                           kv_heads=2, vocab=128, seq_len=32, tied=0, group_size=0),
}


def streams(K):
    import torch

    def mat(role, layer, rows, cols):
        return torch.from_numpy(K.synth_normal(SEED, role, layer, rows * cols, STD).reshape(rows, cols))

    def vec(role, layer, n, std=STD):
        return torch.from_numpy(K.synth_normal(SEED, role, layer, n, std))

    def norm(role, layer, n):
        return 1.0 + vec(role, layer, n, NORM_STD)

    return mat, vec, norm


def llama_like_model(K, mod_name, spec):
    """The reference's llama2.c-style Transformer (tools/model.py or
    tools/model_qwen2.py) with every parameter overwritten from the streams."""
    import torch

    mod = importlib.import_module(mod_name)
    args = mod.ModelArgs(dim=spec["dim"], n_layers=spec["layers"], n_heads=spec["heads"],
                         n_kv_heads=spec["kv_heads"], vocab_size=spec["vocab"],
                         hidden_dim=spec["hidden_dim"], max_seq_len=spec["seq_len"])
    m = mod.Transformer(args)
    mat, vec, norm = streams(K)
    D, F, V = spec["dim"], spec["hidden_dim"], spec["vocab"]
    Dkv = D // spec["heads"] * spec["kv_heads"]
    with torch.no_grad():
        m.tok_embeddings.weight = torch.nn.Parameter(mat(EMB, 0, V, D).clone())
        if spec["tied"]:
            m.output.weight = m.tok_embeddings.weight
        else:
            m.output.weight = torch.nn.Parameter(mat(CLS, 0, V, D).clone())
        for l, layer in enumerate(m.layers):
            a, f = layer.attention, layer.feed_forward
            a.wq.weight.copy_(mat(WQ, l, D, D))
            a.wk.weight.copy_(mat(WK, l, Dkv, D))
            a.wv.weight.copy_(mat(WV, l, Dkv, D))
            a.wo.weight.copy_(mat(WO, l, D, D))
            if a.wq.bias is not None:
                a.wq.bias.copy_(vec(BQ, l, D))
                a.wk.bias.copy_(vec(BK, l, Dkv))
                a.wv.bias.copy_(vec(BV, l, Dkv))
            f.w1.weight.copy_(mat(W1, l, F, D))
            f.w2.weight.copy_(mat(W2, l, D, F))
            f.w3.weight.copy_(mat(W3, l, F, D))
            layer.attention_norm.weight.copy_(norm(RMS_ATT, l, D))
            layer.ffn_norm.weight.copy_(norm(RMS_FFN, l, D))
        m.norm.weight.copy_(norm(RMS_FINAL, 0, D))
    return m


def qwen3_dir(K, spec, path):
    """A HuggingFace-style Qwen3 directory (config.json + model.safetensors)
    holding the stream weights, the input export_qwen3_bin reads."""
    from safetensors.torch import save_file

    mat, vec, norm = streams(K)
    D, Dq, F, V, L = spec["dim"], spec["q_dim"], spec["hidden_dim"], spec["vocab"], spec["layers"]
    hd = Dq // spec["heads"]
    Dkv = hd * spec["kv_heads"]
    t = {"model.embed_tokens.weight": mat(EMB, 0, V, D), "model.norm.weight": norm(RMS_FINAL, 0, D),
         "lm_head.weight": mat(CLS, 0, V, D)}
    for l in range(L):
        p = f"model.layers.{l}."
        t[p + "input_layernorm.weight"] = norm(RMS_ATT, l, D)
        t[p + "post_attention_layernorm.weight"] = norm(RMS_FFN, l, D)
        t[p + "self_attn.q_proj.weight"] = mat(WQ, l, Dq, D)
        t[p + "self_attn.q_norm.weight"] = norm(Q_NORM, l, hd)
        t[p + "self_attn.k_proj.weight"] = mat(WK, l, Dkv, D)
        t[p + "self_attn.k_norm.weight"] = norm(K_NORM, l, hd)
        t[p + "self_attn.v_proj.weight"] = mat(WV, l, Dkv, D)
        t[p + "self_attn.o_proj.weight"] = mat(WO, l, D, Dq)
        t[p + "mlp.gate_proj.weight"] = mat(W1, l, F, D)
        t[p + "mlp.down_proj.weight"] = mat(W2, l, D, F)
        t[p + "mlp.up_proj.weight"] = mat(W3, l, F, D)
    save_file({k: v.contiguous() for k, v in t.items()}, os.path.join(path, "model.safetensors"))
    cfg = {"hidden_size": D, "num_attention_heads": spec["heads"],
           "num_key_value_heads": spec["kv_heads"], "vocab_size": V, "num_hidden_layers": L,
           "intermediate_size": F, "head_dim": hd}
    with open(os.path.join(path, "config.json"), "w") as f:
        json.dump(cfg, f)


def main() -> None:
    from pathlib import Path

    sys.path.insert(0, ROOT)
    sys.path.insert(0, REF_TOOLS)
    import kuiperllama_amd as K

    exp_llama = importlib.import_module("export_llama")
    exp_qwen2 = importlib.import_module("export_qwen2")
    exp_qwen3 = importlib.import_module("export_qwen3")
    manifest = {"seed": SEED, "stddev": STD, "norm_stddev": NORM_STD, "files": {}}
    for name, spec in SPECS.items():
        out = os.path.join(HERE, name + ".bin")
        if spec["family"] == 3:
            with tempfile.TemporaryDirectory() as d:
                qwen3_dir(K, spec, d)
                exp_qwen3.export_qwen3_bin(Path(d), Path(out), spec["seq_len"], overwrite=True)
            writer = "tools/export_qwen3.py:export_qwen3_bin"
        else:
            qwen2 = spec["family"] == 2
            mod = exp_qwen2 if qwen2 else exp_llama
            model = llama_like_model(K, "model_qwen2" if qwen2 else "model", spec)
            if spec["group_size"]:
                mod.legacy_export_quant(model, out)
                fn = "legacy_export_quant"
            else:
                mod.legacy_export(model, out)
                fn = "legacy_export"
            writer = ("tools/export_qwen2.py:" if qwen2 else "tools/export_llama.py:") + fn
        manifest["files"][name] = {"spec": spec, "writer": writer,
                                   "bytes": os.path.getsize(out)}
        print(f"{name}: {os.path.getsize(out)} bytes by {writer}")
    with open(os.path.join(HERE, "fmt_manifest.json"), "w") as f:
        json.dump(manifest, f, indent=1, sort_keys=True)


if __name__ == "__main__":
    main()
