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
    # Decoded responses may end inside a UTF-8 sequence: undecodable bytes
    # read as U+FFFD, as the test oracle's decode() reads them.
    return subprocess.run([BIN] + args, input=stdin, capture_output=True, encoding="utf-8",
                          errors="replace", timeout=timeout)


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
    for name in ("tiny_llama3", "tiny_qwen2", "tiny_qwen3", "tiny_q8", "tiny_qwen2_q8"):
        cfg = K.TINY[name]
        p = str(d / f"{name}.bin")
        K.synth_image(cfg).tofile(p)
        out[name] = (cfg, p)
    return out


@pytest.mark.gpu
@pytest.mark.parametrize("name,flags", [("tiny_llama3", []), ("tiny_qwen2", ["--layered"]),
                                        ("tiny_qwen3", ["--prefill"]),
                                        ("tiny_q8", ["--quant", "--prefill"]),
                                        ("tiny_qwen2_q8", ["--quant", "--prefill"])])
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


# ------------------------------------------------------------- text prompts ----
TOK = os.path.join(ROOT, "tests", "golden", "tok")
TOKFILE = {"llama2": "sp_bpe.model", "llama3": "bpe_llama3.json", "qwen2": "bpe_qwen.json",
           "qwen3": "bpe_qwen.json"}
MARKERS = ["<|im_end|>", "<|endoftext|>", "</s>", "<|end|>"]


def response_text(decoded):
    """main_qwen.cpp:94-148 (remove_end_markers, collapse_repeated_lines)."""
    strip = lambda t: t.strip(" \t\r\n")  # noqa: E731
    for mk in MARKERS:
        if mk in decoded:
            decoded = decoded[:decoded.index(mk)]
    kept, prev, run = [], "", 0
    for line in strip(decoded).split("\n"):
        norm = strip(line)
        if norm and norm == prev and len(norm) <= 48:
            run += 1
            if run >= 2 and len(norm) <= 32:
                if kept and strip(kept[-1]) == norm:
                    kept.pop()
                break
            if run >= 3:
                continue
        else:
            prev, run = norm, 1
        kept.append(line)
    return strip("\n".join(kept))


def test_response_text_rules():
    """The restated post-processing on hand-made cases."""
    assert response_text("  hi <|im_end|> junk") == "hi"
    assert response_text("a</s>b<|endoftext|>c") == "a"
    assert response_text("x\nab\nab\nab\ny") == "x"                 # short line repeated twice more
    long = "l" * 40
    assert response_text(f"{long}\n{long}\n{long}\n{long}\nz") == f"{long}\n{long}\nz"
    assert response_text("\n\n") == ""


def tokenizer_for(family):
    """(oracle encode, oracle decode, stop ids) for the family's fixture tokenizer."""
    path = os.path.join(TOK, TOKFILE[family])
    if family == "llama2":
        spm = pytest.importorskip("sentencepiece")
        sp = spm.SentencePieceProcessor(model_file=path)
        return (lambda s: [sp.bos_id()] + sp.encode(s, out_type=int)), sp.decode, {sp.eos_id()}
    import sys
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import tokenizer as T
    bt = T.BpeTokenizer(path, qwen=family.startswith("qwen"))
    return bt.encode, bt.decode, {bt.eos, bt.stop2}


def ids_line(stderr, tag):
    line = next(l for l in stderr.splitlines() if l.startswith(tag))
    return [int(t) for t in line[len(tag):].split()]


def test_tokenizer_errors_before_the_gpu(K, tmp_path):
    """A missing tokenizer file, or one with more ids than the model's
    vocabulary, fails init() before any GPU call."""
    cfg = K.TINY["tiny_qwen3"]            # vocab 640 < the fixture's 903 ids
    p = str(tmp_path / "q3.bin")
    K.synth_image(cfg).tofile(p)
    r = run(["--family", "qwen3", "--tokenizer", str(tmp_path / "missing.json"), p, "hi"])
    assert r.returncode == 1 and "init failed" in r.stderr, r.stderr
    r = run(["--family", "qwen3", "--tokenizer", os.path.join(TOK, TOKFILE["qwen3"]), p, "hi"])
    assert r.returncode == 1 and "vocabulary" in r.stderr, r.stderr


@pytest.fixture(scope="module")
def text_images(K, tmp_path_factory):
    """Tiny images with the fixture tokenizers' vocabulary sizes, so that
    every generated id decodes."""
    d = tmp_path_factory.mktemp("gentext")
    out = {}
    for fam, name, vocab in (("llama2", "tiny_llama2", 700), ("llama3", "tiny_llama3", 903),
                             ("qwen2", "tiny_qwen2", 903)):
        cfg = K.TINY[name].with_(vocab=vocab, seq_len=128)
        p = str(d / f"{name}_v{vocab}.bin")
        K.synth_image(cfg).tofile(p)
        out[fam] = (cfg, p)
    return out


def expected(O, cfg, path, prompt, max_new, stops):
    import numpy as np
    ids = [int(t) for t in O.Model(np.fromfile(path, np.uint8), cfg.family, cfg.quant)
           .generate(prompt, max_new + 1)]
    for i, t in enumerate(ids):
        if t in stops:
            return ids[:i]
    return ids


@pytest.mark.gpu
@pytest.mark.parametrize("family,flags", [("llama2", []), ("llama3", ["--prefill"]),
                                          ("qwen2", ["--layered"])])
def test_text_prompt_single_shot(O, gpu, text_images, family, flags):
    cfg, path = text_images[family]
    enc, dec, stops = tokenizer_for(family)
    text = "The quick brown fox's 42 jumps\tover the lazy dog."
    max_new = 9
    p = run(["--family", family, "--tokenizer", os.path.join(TOK, TOKFILE[family])] + flags +
            [path, text, str(max_new)])
    assert p.returncode == 0, p.stderr
    prompt = ids_line(p.stderr, "[PROMPT_IDS]")
    assert prompt == enc(text)
    got = ids_line(p.stderr, "[RESPONSE_IDS]")
    want = expected(O, cfg, path, prompt, max_new, stops)
    print(family, flags, prompt, got, flush=True)
    # Within 10 tokens only an end marker in the decoded tail could stop
    # earlier; the fixture vocabularies decode no token to one.
    assert got == want
    body = p.stdout.split("[RESPONSE_START]\n")[1].split("\n[RESPONSE_END]")[0]
    assert body == response_text(dec(got))


@pytest.mark.gpu
def test_text_serve_protocol(O, gpu, text_images):
    cfg, path = text_images["qwen2"]
    enc, dec, stops = tokenizer_for("qwen2")
    prompts = ["<|im_start|>user\nHello there, how are you?<|im_end|>\n<|im_start|>assistant\n",
               "",
               "single line"]
    stdin = "".join("[PROMPT_START]\n" + t + "\n[PROMPT_END]\n" for t in prompts) + "[EXIT]\n"
    p = run(["--serve", "--family", "qwen2", "--tokenizer", os.path.join(TOK, TOKFILE["qwen2"]),
             path, "6"], stdin=stdin)
    assert p.returncode == 0, p.stderr
    blocks = [b.split("[RESPONSE_END]")[0] for b in p.stdout.split("[RESPONSE_START]\n")[1:]]
    assert len(blocks) == 3
    got_prompts = [[int(t) for t in l.split()[1:]] for l in p.stderr.splitlines()
                   if l.startswith("[PROMPT_IDS]")]
    got_resp = [[int(t) for t in l.split()[1:]] for l in p.stderr.splitlines()
                if l.startswith("[RESPONSE_IDS]")]
    assert got_prompts == [enc(t) for t in prompts]
    assert got_prompts[1] == [] and blocks[1] == "\n"   # an empty prompt: an empty response
    for k in (0, 2):
        want = expected(O, cfg, path, got_prompts[k], 6, stops)
        assert got_resp[k] == want
        assert blocks[k] == response_text(dec(want)) + "\n"


def profile_lines(stderr):
    out = {}
    for line in stderr.splitlines():
        if line.startswith("[PROFILE] "):
            kv = dict(f.split("=", 1) for f in line[len("[PROFILE] "):].split())
            out[kv["op"]] = (int(kv["calls"]), float(kv["total_ms"]), float(kv["avg_ms"]))
    return out


@pytest.mark.gpu
@pytest.mark.parametrize("flags", [["--layered"], [], ["--prefill"]])
def test_profile_counts_operations(K, gpu, images, flags):
    """--profile (the reference's per-operation profile, timed on the device):
    the layer-by-layer step reports every operation once per layer and
    position, the sampler once per decode step; the fused step one
    "fused.step" per position (the batched prefill one "prefill.batched")."""
    cfg, path = images["tiny_llama3"]
    P, max_new = 6, 9
    prompt = [int(t) for t in K.prompt_tokens(cfg, P)]
    p = run(["--family", "llama3", "--profile"] + flags + [path, ",".join(map(str, prompt)), str(max_new)])
    assert p.returncode == 0, p.stderr
    steps = int(p.stderr.split("[STATS] steps=")[1].split()[0])
    prof = profile_lines(p.stderr)
    print(flags, steps, prof, flush=True)
    assert prof and all(t >= 0 and n > 0 for n, t, _ in prof.values())
    decode = len(response(p.stdout))  # sampled positions that produced a response token
    if flags == ["--layered"]:
        L = cfg.layers
        for op in ("attn.rmsnorm", "attn.wq", "attn.wk", "attn.wv", "attn.rope", "attn.mha", "attn.wo",
                   "ffn.rmsnorm", "ffn.w1", "ffn.w3", "ffn.swiglu", "ffn.w2", "ffn.residual_add1",
                   "ffn.residual_add2"):
            assert prof[op][0] == steps * L, op
        assert prof["output.cls"][0] == steps
        assert prof["sampler.argmax"][0] == steps - (P - 1)
        assert prof["attn.wq"][1] > 0
    elif flags == ["--prefill"]:
        assert prof["prefill.batched"][0] == 1 and prof["prefill.batched"][1] > 0
        assert prof["fused.step"][0] == steps - P
    else:
        assert prof["fused.step"][0] == steps and prof["fused.step"][1] > 0
    assert decode >= 1
