"""Writes the tokenizer fixtures under tests/golden/tok/ (run in the build
container; nothing on the GPU box runs it).

* sp_bpe.model: a SentencePiece BPE model trained here on a seeded synthetic
  corpus with the options of the Llama-2 tokenizer (identity normalisation,
  dummy prefix, byte fallback, split digits); sentencepiece is the library
  the reference's SpeEncodeLayer wraps (kuiper/source/op/encode.cpp:14-57).
* bpe_llama3.json / bpe_qwen.json: byte-level BPE tokenizer.json files
  trained here with HF tokenizers, with the Llama-3 and Qwen special tokens
  (what BpeEncodeLayer / QwenEncodeLayer read, encode.cpp:64-182).
* tok_cases.json: test sentences and the expected ids / decoded text:
  SentencePiece cases from the sentencepiece library itself (EncodeAsIds
  with BOS, as SpeEncodeLayer::encode; DecodeIds); BPE cases from
  oracle/tokenizer.py, the restatement of the reference's tiktoken path.
"""
from __future__ import annotations

import io
import json
import os
import random
import sys

import sentencepiece as spm
from tokenizers import Tokenizer, decoders, models, pre_tokenizers, trainers

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
import tokenizer as T  # noqa: E402

OUT = os.path.join(HERE, "tok")

SYL = ["ka", "to", "ri", "me", "lo", "sa", "ne", "qu", "th", "ing", "er", "an", "st", "ou", "ch",
       "pre", "con", "tion", "al", "ly", "be", "de", "ex", "un", "re", "ight", "ow", "ea"]
EXTRA = ["café", "naïve", "Zürich", "straße", "日本語", "中文", "テスト", "Привет", "мир", "😀", "👍🏽",
         "don't", "we're", "I'll", "it's", "THE", "Hello", "World", "3.14", "2024", "x=y+1;", "(a,b)",
         "--", "...", "!?", "#tag", "@user", "\t", "e-mail", "co-op"]


def corpus(seed: int = 7, lines: int = 3000) -> list[str]:
    rng = random.Random(seed)
    out = []
    for _ in range(lines):
        words = []
        for _ in range(rng.randint(3, 14)):
            r = rng.random()
            if r < 0.75:
                w = "".join(rng.choice(SYL) for _ in range(rng.randint(1, 4)))
                if rng.random() < 0.15:
                    w = w.capitalize()
            elif r < 0.9:
                w = rng.choice(EXTRA)
            else:
                w = str(rng.randint(0, 99999))
            words.append(w)
        sep = rng.choice([" ", " ", " ", "  ", ", ", ". "])
        out.append(sep.join(words))
    return out


CASES = [
    "hello", "Hello world", "the quick brown fox", "  leading spaces", "trailing spaces   ",
    "multiple   inner   spaces", "line one\nline two\n\nline four", "tabs\tand\ttabs",
    "numbers 12345 and 3.14159", "don't we're I'll it's IT'S", "café naïve Zürich straße",
    "日本語のテスト 中文", "Привет, мир!", "emoji 😀👍🏽 end", "punctuation!?... --- ###",
    "x=y+1; f(a,b) == [1, 2, 3]", "", " ", "a", "katomeri stloing", "\n", "end with newline\n",
    "<|begin_of_text|>special inside<|eot_id|>text", "<|im_start|>user\nhi<|im_end|>",
    "mixed 123abc456def", "UPPER lower MiXeD", " nbsp here", "zero​width",
]


def main() -> None:
    os.makedirs(OUT, exist_ok=True)
    text = corpus()
    # SentencePiece BPE with the Llama-2 tokenizer's options.
    buf = io.BytesIO()
    spm.SentencePieceTrainer.train(
        sentence_iterator=iter(text), model_writer=buf, vocab_size=700, model_type="bpe",
        byte_fallback=True, normalization_rule_name="identity", add_dummy_prefix=True,
        remove_extra_whitespaces=False, split_digits=True, allow_whitespace_only_pieces=True,
        character_coverage=0.9995, unk_id=0, bos_id=1, eos_id=2, pad_id=-1, num_threads=1,
        minloglevel=2)
    sp_path = os.path.join(OUT, "sp_bpe.model")
    with open(sp_path, "wb") as f:
        f.write(buf.getvalue())
    sp = spm.SentencePieceProcessor(model_file=sp_path)
    # Byte-level BPE tokenizer.json files with the Llama-3 / Qwen specials.
    specials = {"llama3": ["<|begin_of_text|>", "<|end_of_text|>", "<|eot_id|>"],
                "qwen": ["<|endoftext|>", "<|im_start|>", "<|im_end|>"]}
    bpe_paths = {}
    for name, sp_tokens in specials.items():
        tok = Tokenizer(models.BPE())
        tok.pre_tokenizer = pre_tokenizers.ByteLevel(add_prefix_space=False)
        tok.decoder = decoders.ByteLevel()
        trainer = trainers.BpeTrainer(vocab_size=900, initial_alphabet=pre_tokenizers.ByteLevel.alphabet(),
                                      show_progress=False)
        tok.train_from_iterator(text, trainer)
        tok.add_special_tokens(sp_tokens)
        path = os.path.join(OUT, f"bpe_{name}.json")
        tok.save(path)
        bpe_paths[name] = path
    cases = {"spe": [], "llama3": [], "qwen": []}
    for s in CASES:
        ids = [sp.bos_id()] + sp.encode(s, out_type=int)
        cases["spe"].append({"text": s, "ids": ids, "decoded": sp.decode(ids)})
    for name in ("llama3", "qwen"):
        bt = T.BpeTokenizer(bpe_paths[name], qwen=name == "qwen")
        for s in CASES:
            ids = bt.encode(s)
            cases[name].append({"text": s, "ids": ids, "decoded": bt.decode(ids)})
    meta = {"spe": {"vocab_size": sp.get_piece_size(), "bos": sp.bos_id(), "eos": sp.eos_id()}}
    for name in ("llama3", "qwen"):
        bt = T.BpeTokenizer(bpe_paths[name], qwen=name == "qwen")
        meta[name] = {"vocab_size": bt.vocab_size(), "bos": bt.bos, "eos": bt.eos, "stop2": bt.stop2}
    with open(os.path.join(OUT, "tok_cases.json"), "w", encoding="utf-8") as f:
        json.dump({"meta": meta, "cases": cases}, f, ensure_ascii=False, indent=1)
    print("wrote", sorted(os.listdir(OUT)))


if __name__ == "__main__":
    main()
