"""kuiper_generate, the generate/serve driver (demo/main.cpp:5-47,
demo/main_qwen.cpp:198-284 and :404-452), on synthetic images: its response
ids equal the oracle's greedy sequence (demo/main.cpp's loop), the decode-phase
stop rules apply, and the --serve protocol answers prompt after prompt."""
import os
import subprocess

import pytest

from conftest import ROOT

BIN = os.path.join(ROOT, "kuiperllama_amd", "lib", "kuiper_generate")
FAMILY = {0: "llama2", 1: "llama3", 2: "qwen2", 3: "qwen3"}


def run(args, stdin=None, timeout=120):
    if not os.path.exists(BIN):
        pytest.fail(f"{BIN} is not built (run __graft_entry__.build())")
    return subprocess.run([BIN] + args, input=stdin, capture_output=True, text=True,
                          timeout=timeout)


def response(stdout):
    lines = stdout.splitlines()
    i = lines.index("[RESPONSE_START]")
    j = lines.index("[RESPONSE_END]", i)
    body = " ".join(lines[i + 1:j]).split()
    return [int(t) for t in body]


def test_usage_and_errors():
    assert run([]).returncode == 2
    assert run(["--family", "gpt"]).returncode == 2
    assert run(["/nonexistent/model.bin", "1,2,3"]).returncode == 1  # init fails before the GPU
    assert run(["m.bin", "1,x,3"]).returncode == 2
    assert run(["--layered", "--prefill", "m.bin", "1,2"]).returncode == 2


@pytest.fixture(scope="module")
def images(K, tmp_path_factory):
    d = tmp_path_factory.mktemp("gen")
    out = {}
    for name in ("tiny_llama3", "tiny_qwen2", "tiny_qwen3"):
        cfg = K.TINY[name]
        p = str(d / f"{name}.bin")
        K.synth_image(cfg).tofile(p)
        out[name] = (cfg, p)
    return out


@pytest.mark.gpu
@pytest.mark.parametrize("name,flags", [("tiny_llama3", []), ("tiny_qwen2", ["--layered"]),
                                        ("tiny_qwen3", ["--prefill"])])
def test_single_shot_matches_oracle(K, O, gpu, images, name, flags):
    cfg, path = images[name]
    prompt = [int(t) for t in K.prompt_tokens(cfg, 6)]
    max_new = 9
    p = run(["--family", FAMILY[cfg.family]] + flags + [path, ",".join(map(str, prompt)),
                                                       str(max_new)])
    assert p.returncode == 0, p.stderr
    assert "[STATS] steps=" in p.stderr
    img = open(path, "rb").read()
    import numpy as np
    want = [int(t) for t in O.Model(np.frombuffer(img, np.uint8), cfg.family, cfg.quant)
            .generate(prompt, max_new + 1)]
    got = response(p.stdout)
    print(name, flags, got, flush=True)
    # The stop rules cannot fire within 10 tokens unless one token repeats 24 times.
    assert got == want


@pytest.mark.gpu
def test_eos_stops_decode(K, O, gpu, images):
    cfg, path = images["tiny_llama3"]
    prompt = [int(t) for t in K.prompt_tokens(cfg, 6)]
    import numpy as np
    want = [int(t) for t in O.Model(np.fromfile(path, np.uint8), cfg.family, cfg.quant)
            .generate(prompt, 10)]
    eos = want[3]
    cut = want.index(eos)
    p = run(["--family", "llama3", "--eos", str(eos), path, ",".join(map(str, prompt)), "9"])
    assert p.returncode == 0, p.stderr
    assert response(p.stdout) == want[:cut]


@pytest.mark.gpu
def test_serve_protocol(K, O, gpu, images):
    cfg, path = images["tiny_qwen3"]
    import numpy as np
    img = np.fromfile(path, np.uint8)
    prompts = [[int(t) for t in K.prompt_tokens(cfg, 5, seed=s)] for s in (11, 12, 13)]

    def request(ids_text):
        return "[PROMPT_START]\n" + ids_text + "\n[PROMPT_END]\n"

    stdin = ""
    for pr in prompts[:2]:
        stdin += request(" ".join(map(str, pr[:3])) + "\n" + ",".join(map(str, pr[3:])))
    # bad requests get an [ERROR] line and the server keeps serving
    stdin += request("not ids")
    stdin += request(f"1 2 {cfg.vocab}")                      # id outside [0, vocab)
    stdin += request(" ".join(["5"] * (cfg.seq_len + 1)))     # longer than seq_len
    stdin += request(" ".join(map(str, prompts[2])))
    stdin += "[EXIT]\n"
    p = run(["--serve", "--family", "qwen3", "--prefill", path, "7"], stdin=stdin)
    assert p.returncode == 0, p.stderr
    assert p.stdout.splitlines()[0] == "[READY]"
    blocks = p.stdout.split("[RESPONSE_START]")[1:]
    assert len(blocks) == 3
    for pr, blk in zip(prompts, blocks):
        got = [int(t) for t in blk.split("[RESPONSE_END]")[0].split()]
        want = [int(t) for t in O.Model(img, cfg.family, cfg.quant).generate(pr, 8)]
        assert got == want
    errors = [l for l in p.stdout.splitlines() if l.startswith("[ERROR]")]
    assert len(errors) == 3, errors
    assert "outside [0, " in errors[1] and "positions" in errors[2]
