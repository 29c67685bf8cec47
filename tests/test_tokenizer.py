"""Tokenizers (kuiper/source/op/encode.cpp:14-182) on the CPU: the C++
layers of libkuiper_host.so (op::SpeEncodeLayer, op::BpeEncodeLayer,
op::QwenEncodeLayer, driven through tests/cpp/_build/test_host tok) against

* the committed fixtures of tests/golden/tok (make_tokenizer_fixtures.py):
  SentencePiece ids and decodings written by the sentencepiece library the
  reference wraps, byte-level BPE ids written by oracle/tokenizer.py;
* seeded random strings over letters, digits, punctuation, ASCII and
  non-ASCII whitespace, apostrophes and non-Latin scripts: the C++ BPE
  against oracle/tokenizer.py, the C++ SentencePiece layer against the
  sentencepiece library (skipped where it is not importable).

oracle/tokenizer.py is pinned here too: its byte-pair merge on a hand-built
vocabulary, and its ids against HF tokenizers' own BPE on text that has no
spaces (where the reference's U+0120 replacement and pre-tokenizer make no
difference).
"""
import json
import os
import random
import subprocess
import sys

import pytest
import regex

from conftest import ROOT

sys.path.insert(0, os.path.join(ROOT, "oracle"))
import tokenizer as T  # noqa: E402

BIN = os.path.join(ROOT, "tests", "cpp", "_build", "test_host")
TOK = os.path.join(ROOT, "tests", "golden", "tok")
FILES = {"spe": "sp_bpe.model", "llama3": "bpe_llama3.json", "qwen": "bpe_qwen.json"}
KIND = {"spe": "spe", "llama3": "bpe", "qwen": "qwen"}


def run_cpp(name, texts, tmp_path):
    """(meta line, [(ids, decoded text, ends_sentence)]) from the C++ layer."""
    if not os.path.exists(BIN):
        pytest.fail(f"{BIN} is not built (run __graft_entry__.build())")
    cases = tmp_path / f"cases_{name}.txt"
    cases.write_text("".join((t.encode("utf-8").hex() or "-") + "\n" for t in texts))
    p = subprocess.run([BIN, "tok", KIND[name], os.path.join(TOK, FILES[name]), str(cases)],
                       capture_output=True, text=True, timeout=120)
    assert p.returncode == 0, p.stdout + p.stderr
    lines = p.stdout.splitlines()
    ids = [list(map(int, ln.split()[1:])) for ln in lines if ln.startswith("ids")]
    dec = [bytes.fromhex(ln[4:]).decode("utf-8", "replace") for ln in lines if ln.startswith("dec")]
    end = [ln.split()[1] == "1" for ln in lines if ln.startswith("end")]
    assert len(ids) == len(texts)
    return lines[0], list(zip(ids, dec, end))


def fixtures():
    with open(os.path.join(TOK, "tok_cases.json"), encoding="utf-8") as f:
        return json.load(f)


@pytest.mark.parametrize("name", ["spe", "llama3", "qwen"])
def test_layers_match_fixtures(tmp_path, name):
    d = fixtures()
    cases = d["cases"][name]
    meta, got = run_cpp(name, [c["text"] for c in cases], tmp_path)
    assert f"vocab {d['meta'][name]['vocab_size']}" in meta
    for c, (ids, dec, _) in zip(cases, got):
        assert ids == c["ids"], (c["text"], ids, c["ids"])
        assert dec == c["decoded"], (c["text"], dec, c["decoded"])


def random_texts(seed, n=300):
    alphabet = (list("abcdefghijklmnopqrstuvwxyzABCDEFGHIJKLMNOPQRSTUVWXYZ") * 3 + list("0123456789") * 2 +
                list(" " * 12) + list("\t\n\r\f") + list("'''") + list(".,;:!?-_()[]{}<>/\\\"#$%&*+=@^`|~") +
                ["é", "ü", "ß", "ñ", "ø", "ſ", "İ", "日", "本", "語", "中", "テ", "ス", "ト", "П", "р", "и",
                 "²", "½", "٣", "Ⅻ", " ", "　", "​", "😀", "👍", "́", "\x0b", "ŉ"])
    rng = random.Random(seed)
    words = ["'s", "'t", "'re", "'ve", "'m", "'ll", "'d", "'S", "'LL", "'Re", "<|eot_id|>",
             "<|im_start|>", "<|end_of_text|>"]
    out = []
    for _ in range(n):
        k = rng.randint(0, 40)
        s = "".join(rng.choice(words) if rng.random() < 0.05 else rng.choice(alphabet) for _ in range(k))
        out.append(s)
    return out


@pytest.mark.parametrize("name", ["llama3", "qwen"])
def test_bpe_random_strings_match_oracle(tmp_path, name):
    texts = random_texts(11 if name == "llama3" else 12)
    bt = T.BpeTokenizer(os.path.join(TOK, FILES[name]), qwen=name == "qwen")
    _, got = run_cpp(name, texts, tmp_path)
    for s, (ids, dec, end) in zip(texts, got):
        want = bt.encode(s)
        assert ids == want, (s, ids, want)
        assert dec == bt.decode(want), (s, dec)
        assert end == (bool(want) and want[-1] in (bt.eos, bt.stop2))


def test_spe_random_strings_match_sentencepiece(tmp_path):
    spm = pytest.importorskip("sentencepiece")
    sp = spm.SentencePieceProcessor(model_file=os.path.join(TOK, FILES["spe"]))
    texts = random_texts(13)
    _, got = run_cpp("spe", texts, tmp_path)
    for s, (ids, dec, _) in zip(texts, got):
        want = [sp.bos_id()] + sp.encode(s, out_type=int)
        assert ids == want, (s, ids, want)
        assert dec == sp.decode(want), (s, dec, sp.decode(want))


def test_round_trips(tmp_path):
    """decode(encode(s)) == s for text the vocabularies cover (byte-level BPE:
    every text; SentencePiece with byte fallback: every text)."""
    texts = [c["text"] for c in fixtures()["cases"]["spe"]] + random_texts(14, 80)
    for name in ("spe", "qwen"):
        _, got = run_cpp(name, texts, tmp_path)
        for s, (_, dec, _) in zip(texts, got):
            if name == "spe":
                # SentencePiece's identity normaliser keeps every character;
                # decode drops the dummy-prefix space only.
                assert dec == s.replace("▁", " "), (name, s, dec)
            else:
                assert dec == s, (name, s, dec)


def test_bad_files_are_reported(tmp_path):
    for kind in ("spe", "bpe", "qwen"):
        cases = tmp_path / "c.txt"
        cases.write_text("-\n")
        p = subprocess.run([BIN, "tok", kind, str(tmp_path / "missing"), str(cases)],
                           capture_output=True, text=True, timeout=60)
        assert p.returncode == 1 and "meta init 2" in p.stdout, p.stdout
    bad = tmp_path / "bad.json"
    bad.write_text("{ not json")
    p = subprocess.run([BIN, "tok", "bpe", str(bad), str(cases)], capture_output=True, text=True, timeout=60)
    assert p.returncode == 1 and "meta init 3" in p.stdout, p.stdout
    # a byte-level vocabulary without all 256 byte tokens
    nobytes = tmp_path / "nobytes.json"
    nobytes.write_text(json.dumps({"added_tokens": [], "model": {"vocab": {"a": 0, "b": 1, "ab": 2}}}))
    p = subprocess.run([BIN, "tok", "qwen", str(nobytes), str(cases)], capture_output=True, text=True,
                       timeout=60)
    assert p.returncode == 1 and "meta init 3" in p.stdout and "byte-level" in p.stdout, p.stdout
    # an added token with empty content (it would match at every position, and
    # an encoder that took it would never advance): refused at init, no hang
    with open(os.path.join(TOK, FILES["qwen"]), encoding="utf-8") as f:
        src = json.load(f)
    src["added_tokens"].append({"id": len(src["model"]["vocab"]) + len(src["added_tokens"]),
                                "content": "", "special": True})
    empty = tmp_path / "empty_added.json"
    empty.write_text(json.dumps(src))
    cases.write_text("hello world\n")
    for kind in ("bpe", "qwen"):
        p = subprocess.run([BIN, "tok", kind, str(empty), str(cases)], capture_output=True, text=True,
                           timeout=60)
        assert p.returncode == 1 and "meta init 3" in p.stdout and "empty content" in p.stdout, p.stdout


# ----------------------------------------------- pinning the BPE oracle ----
def test_oracle_byte_pair_merge_hand_vocabulary():
    """Ranks a=0 b=1 c=2 d=3, ab=4, cd=5, abcd=6, bc=7: "abcd" merges the
    lowest-ranked pair first (ab), then cd, then abcd -- never bc (rank 7)."""
    ranks = {b"a": 0, b"b": 1, b"c": 2, b"d": 3, b"ab": 4, b"cd": 5, b"abcd": 6, b"bc": 7}
    assert T.byte_pair_merge(b"abcd", ranks) == [6]
    assert T.byte_pair_merge(b"abc", ranks) == [4, 2]       # ab (4) before bc (7)
    assert T.byte_pair_merge(b"bcd", ranks) == [1, 5]       # cd (5) before bc (7)
    assert T.byte_pair_merge(b"dcba", ranks) == [3, 2, 1, 0]
    ranks2 = {b"x": 0, b"y": 1, b"xy": 2, b"yx": 3}
    assert T.byte_pair_merge(b"xyx", ranks2) == [2, 0]      # equal start: the lower rank, leftmost


def test_oracle_pre_tokenizer_pattern():
    """The reference's pattern (RE2 semantics) on hand-checked strings."""
    import regex
    f = lambda s: regex.findall(T.PAT_STR, s)  # noqa: E731
    assert f("Hello world's") == ["Hello", " world", "'s"]
    assert f("it's ME'LL") == ["it", "'s", " ME", "'LL"]
    assert f("a  b") == ["a", "  ", "b"]          # \s+(?:$|[^\S]) takes both spaces
    assert f("a \n\nb") == ["a", " \n\n", "b"]    # \s*[\r\n]+
    assert f("x123") == ["x", "1", "2", "3"]
    assert f("x!!\n y") == ["x", "!!\n", " y"]
    assert f("trail  ") == ["trail", "  "]
    assert f(" word") == [" word"]      # NBSP is not \s in RE2


def test_oracle_matches_hf_bpe_without_spaces():
    """On text without spaces the reference's path is plain byte-level BPE:
    the oracle's ids equal HF tokenizers' own encoding (merges applied by
    rank) for every word of the fixture corpus alphabet."""
    tk = pytest.importorskip("tokenizers")
    path = os.path.join(TOK, FILES["qwen"])
    hf = tk.Tokenizer.from_file(path)
    bt = T.BpeTokenizer(path, qwen=True)
    rng = random.Random(5)
    syl = ["ka", "to", "ri", "me", "lo", "sa", "ne", "qu", "th", "ing", "er", "an", "st", "ou", "ch",
           "pre", "con", "tion", "al", "ly", "be", "de", "ex", "un", "re", "ight", "ow", "ea"]
    words = ["".join(rng.choice(syl) for _ in range(rng.randint(1, 5))) for _ in range(400)]
    words += ["café", "naïve", "Zürich", "straße", "Привет", "日本語"]
    agree = 0
    for w in words:
        if hf.encode(w).ids == bt.encode(w):
            agree += 1
    # tiktoken merges by the rank of the joined bytes, HF by merge order; on
    # this HF-trained vocabulary they coincide on every word.
    assert agree == len(words), agree


def test_spe_decodes_invalid_byte_runs_like_sentencepiece(tmp_path):
    """Byte pieces that do not form valid UTF-8 (overlong forms, surrogates,
    values above U+10FFFF, stray continuation bytes, truncated sequences)
    decode to U+FFFD per byte, as the sentencepiece library does; valid runs
    decode to their character."""
    spm = pytest.importorskip("sentencepiece")
    sp = spm.SentencePieceProcessor(model_file=os.path.join(TOK, FILES["spe"]))
    byte_id = {sp.id_to_piece(i): i for i in range(sp.get_piece_size()) if sp.is_byte(i)}
    lead = next(i for i in range(sp.get_piece_size())
                if sp.id_to_piece(i).startswith("▁") and len(sp.id_to_piece(i)) > 2)
    runs = [b"\xc1\x80", b"\xc0\xaf", b"\xe0\x80\x80", b"\xed\xa0\x80", b"\xf4\x90\x80\x80",
            b"\xf5\x80\x80\x80", b"\x80", b"\xe6\x97", b"\xe6\x97\xa5", b"\xf0\x9f\x98\x80",
            b"\xc3\xa9\x80\xc3", b"\xef\xbf\xbf", b"\xf0\x90\x80\x80"]
    cases = []
    for r in runs:
        ids = [byte_id[f"<0x{b:02X}>"] for b in r]
        cases.append(ids)
        cases.append([lead] + ids + [sp.piece_to_id("a")])
    f = tmp_path / "dec.txt"
    f.write_text("".join("#" + " ".join(map(str, ids)) + "\n" for ids in cases))
    p = subprocess.run([BIN, "tok", "spe", os.path.join(TOK, FILES["spe"]), str(f)],
                       capture_output=True, text=True, timeout=60)
    assert p.returncode == 0, p.stdout + p.stderr
    got = [bytes.fromhex(ln[5:]).decode("utf-8") for ln in p.stdout.splitlines() if ln.startswith("only")]
    assert len(got) == len(cases)
    for ids, g in zip(cases, got):
        assert g == sp.decode(ids), (ids, g, sp.decode(ids))


def test_space_replacement_pin(tmp_path):
    """encode.cpp:110-112 replaces every " " with U+0120 before the split:
    a text and its replaced twin encode alike (oracle and C++), and since
    U+0120 is a letter, words joined by spaces form one pre-tokenizer piece.
    decode() maps U+0120 back to " " (encode.cpp:129-131), so a literal
    U+0120 in the input also comes back as a space."""
    bt = T.BpeTokenizer(os.path.join(TOK, FILES["qwen"]), qwen=True)
    texts = ["hello world", "a b  c", " lead", "tail ", "xĠy z", "it's a 12 test"]
    twins = [s.replace(" ", "Ġ") for s in texts]
    for s, t in zip(texts, twins):
        assert bt.encode(s) == bt.encode(t)
        assert bt.decode(bt.encode(t)) == s.replace("Ġ", " ")
    assert regex.findall(T.PAT_STR, "helloĠworld") == ["helloĠworld"]
    assert regex.findall(T.PAT_STR, "hello world") == ["hello", " world"]
    _, got = run_cpp("qwen", texts + twins, tmp_path)
    n = len(texts)
    for k in range(n):
        assert got[k][0] == got[n + k][0] == bt.encode(texts[k])
        assert got[n + k][1] == texts[k].replace("Ġ", " ")


@pytest.mark.parametrize("opts", [
    dict(remove_extra_whitespaces=True, byte_fallback=False, add_dummy_prefix=True),
    dict(remove_extra_whitespaces=False, byte_fallback=False, add_dummy_prefix=False),
])
def test_spe_other_model_options_match_sentencepiece(tmp_path, opts):
    """SentencePiece BPE models trained here with the options the fixture model
    does not use: extra-whitespace removal, no byte fallback (pieces outside
    the vocabulary become the unknown id, decoded as " \\u2047 "), no dummy
    prefix.  The C++ layer must give the library's ids and decodings."""
    spm = pytest.importorskip("sentencepiece")
    import io
    rng = random.Random(21)
    words = ["the", "quick", "brown", "fox", "jumps", "over", "lazy", "dog", "and", "runs", "far",
             "away", "from", "home", "while", "singing", "songs", "of", "old", "days", "42", "7"]
    corpus = [" ".join(rng.choice(words) for _ in range(rng.randint(3, 12))) for _ in range(2000)]
    buf = io.BytesIO()
    spm.SentencePieceTrainer.train(
        sentence_iterator=iter(corpus), model_writer=buf, vocab_size=120, model_type="bpe",
        normalization_rule_name="identity", split_digits=True, character_coverage=1.0,
        unk_id=0, bos_id=1, eos_id=2, pad_id=-1, num_threads=1, minloglevel=2, **opts)
    path = tmp_path / "m.model"
    path.write_bytes(buf.getvalue())
    sp = spm.SentencePieceProcessor(model_file=str(path))
    texts = random_texts(31, 200) + ["  the  quick   fox  ", "\tlazy dog\n", "", " ", "over home"]
    cases = tmp_path / "cases.txt"
    cases.write_text("".join((t.encode("utf-8").hex() or "-") + "\n" for t in texts))
    p = subprocess.run([BIN, "tok", "spe", str(path), str(cases)], capture_output=True, text=True,
                       timeout=120)
    assert p.returncode == 0, p.stdout + p.stderr
    lines = p.stdout.splitlines()
    ids = [list(map(int, ln.split()[1:])) for ln in lines if ln.startswith("ids")]
    dec = [bytes.fromhex(ln[4:]).decode("utf-8") for ln in lines if ln.startswith("dec")]
    assert len(ids) == len(texts)
    for s, i, d in zip(texts, ids, dec):
        want = [sp.bos_id()] + sp.encode(s, out_type=int)
        assert i == want, (s, i, want)
        assert d == sp.decode(want), (s, d, sp.decode(want))


def test_bpe_full_size_vocabulary(tmp_path):
    """A tokenizer.json the size of Qwen's (151643 byte-level entries + the
    special tokens) loads and encodes 20k characters in well under a second
    and agrees with the oracle id for id."""
    import time
    b2u = T.bytes_to_unicode()
    alpha = [b2u[b] for b in range(256)]
    rng = random.Random(1)
    vocab = {c: i for i, c in enumerate(alpha)}
    while len(vocab) < 151643:
        k = "".join(rng.choice(alpha[:200]) for _ in range(rng.randint(2, 8)))
        vocab.setdefault(k, len(vocab))
    added = [{"id": 151643 + i, "content": c}
             for i, c in enumerate(["<|endoftext|>", "<|im_start|>", "<|im_end|>"])]
    path = tmp_path / "big.json"
    path.write_text(json.dumps({"added_tokens": added, "model": {"type": "BPE", "vocab": vocab}},
                               ensure_ascii=False), encoding="utf-8")
    text = "".join(rng.choice("abcdefghijklmnopqrstuvwxyz      .,'\n0123456789") for _ in range(20000))
    text += "<|im_start|>assistant\n" + text[:500] + "<|im_end|>"
    cases = tmp_path / "c.txt"
    cases.write_text(text.encode("utf-8").hex() + "\n")
    t0 = time.time()
    p = subprocess.run([BIN, "tok", "qwen", str(path), str(cases)], capture_output=True, text=True,
                       timeout=60)
    dt = time.time() - t0
    assert p.returncode == 0, p.stdout + p.stderr
    lines = p.stdout.splitlines()
    assert "vocab 151646" in lines[0]
    got = [int(x) for x in lines[1].split()[1:]]
    assert got == T.BpeTokenizer(str(path), qwen=True).encode(text)
    assert dt < 5.0, dt
