"""CPU restatement of the reference's byte-level BPE tokenizers (test
infrastructure: only tests/ and the fixture script use it).

Follows kuiper/source/op/encode.cpp:64-182 (BpeEncodeLayer, QwenEncodeLayer)
over kuiper/include/base/tiktoken.h:17-268 (tiktoken's rank-based byte-pair
merge) as the reference builds it:

* the vocabulary of a HF tokenizer.json ("model" -> "vocab") is converted
  from the byte-level alphabet back to raw bytes (encode.cpp:86-98); a
  token's id is its merge rank;
* "added_tokens" are the special tokens, matched anywhere in the text
  (tiktoken.h:167-187);
* the text between special tokens is split by the reference's pattern
  PAT_STR (encode.cpp:61-62), an RE2 pattern: \\s is ASCII whitespace
  [\\t\\n\\f\\r ], \\p{L} / \\p{N} are Unicode letters / numbers; each piece is
  looked up whole, else byte-pair merged (tiktoken.h:17-108);
* encode replaces every " " by "\\u0120" first and decode does the reverse
  (encode.cpp:110-112, :129-131) -- a reference behaviour kept as is;
* BOS (Llama-3: <|begin_of_text|>) is prepended when has_bos; Qwen has none.

Parity of the pre-tokenizer: the `regex` module stands in for RE2 (same
leftmost-first semantics for this pattern, which has no backreferences);
Unicode categories come from that module's tables (a newer Unicode version
than RE2's may classify recently added code points differently).
"""
from __future__ import annotations

import json

import regex

# encode.cpp:61-62 with RE2's \s spelled out (RE2: \s == [\t\n\f\r ]) and its $ as
# \Z (RE2's $ matches only at the end of the text).
_WS = r"\t\n\f\r "
PAT_STR = (r"(?i:'s|'t|'re|'ve|'m|'ll|'d)|[^\r\n\p{L}\p{N}]?\p{L}+|\p{N}|"
           r" ?[^" + _WS + r"\p{L}\p{N}]+[\r\n]*|[" + _WS + r"]*[\r\n]+|[" + _WS + r"]+(?:\Z|[" + _WS +
           r"])|[" + _WS + r"]+")


def bytes_to_unicode() -> dict[int, str]:
    """The GPT-2 byte-level alphabet: printable Latin-1 bytes map to
    themselves, the other bytes to U+0100 upwards, in byte order."""
    keep = list(range(ord("!"), ord("~") + 1)) + list(range(0xA1, 0xAC + 1)) + list(range(0xAE, 0xFF + 1))
    table, extra = {}, 0
    for b in range(256):
        if b in keep:
            table[b] = chr(b)
        else:
            table[b] = chr(256 + extra)
            extra += 1
    return table


_U2B = {u: b for b, u in bytes_to_unicode().items()}


def _raw(key: str) -> bytes:
    """A vocabulary key in the byte-level alphabet -> its raw bytes
    (encode.cpp:89-95: unicode_utf8_to_byte per code point)."""
    return bytes(_U2B[c] for c in key)


def byte_pair_merge(piece: bytes, ranks: dict[bytes, int]) -> list[int]:
    """tiktoken.h:17-108: repeatedly merge the adjacent parts whose joined
    bytes have the lowest rank (the first such pair on ties)."""
    if len(piece) == 1:
        return [ranks[piece]]
    bounds = list(range(len(piece) + 1))
    inf = float("inf")

    def rank_of(i: int, skip: int):
        if i + skip + 2 < len(bounds):
            return ranks.get(piece[bounds[i]:bounds[i + skip + 2]], inf)
        return inf

    r = [rank_of(i, 0) for i in range(len(bounds) - 1)]
    while len(bounds) > 2:
        best, bi = inf, -1
        for i in range(len(bounds) - 1):
            if r[i] < best:
                best, bi = r[i], i
        if bi < 0:
            break
        r[bi] = rank_of(bi, 1)
        if bi > 0:
            r[bi - 1] = rank_of(bi - 1, 1)
        del bounds[bi + 1]
        del r[bi + 1]
    return [ranks[piece[bounds[i]:bounds[i + 1]]] for i in range(len(bounds) - 1)]


class BpeTokenizer:
    """BpeEncodeLayer (Llama-3 specials) or QwenEncodeLayer (qwen=True)."""

    def __init__(self, path: str, qwen: bool = False, has_bos: bool | None = None):
        with open(path, encoding="utf-8") as f:
            data = json.load(f)
        self.special = {t["content"]: int(t["id"]) for t in data["added_tokens"]}
        self.ranks = {_raw(k): int(v) for k, v in data["model"]["vocab"].items()}
        self.decoder = {v: k for k, v in self.ranks.items()}
        self.special_dec = {v: k.encode() for k, v in self.special.items()}
        if qwen:
            self.bos, self.eos = self.special.get("<|im_start|>", 0), self.special.get("<|im_end|>", 0)
            self.stop2 = self.special.get("<|endoftext|>", 0)
        else:
            self.bos, self.eos = self.special.get("<|begin_of_text|>", 0), self.special.get("<|end_of_text|>", 0)
            self.stop2 = self.special.get("<|eot_id|>", 0)
        self.has_bos = (not qwen) if has_bos is None else has_bos
        self.pat = regex.compile(PAT_STR)
        # Longest special first: the reference's alternation order follows a
        # hash map, so overlapping specials are left out of the fixtures.
        self.spat = regex.compile("|".join(regex.escape(s) for s in sorted(self.special, key=len, reverse=True))) \
            if self.special else None

    def _ordinary(self, text: str) -> list[int]:
        out = []
        for m in self.pat.finditer(text):
            piece = m.group(0).encode("utf-8")
            if piece in self.ranks:
                out.append(self.ranks[piece])
            else:
                out.extend(byte_pair_merge(piece, self.ranks))
        return out

    def encode(self, sentence: str) -> list[int]:
        text = sentence.replace(" ", "Ġ")  # encode.cpp:110-112
        out = []
        pos = 0
        while True:
            m = self.spat.search(text, pos) if self.spat else None
            out.extend(self._ordinary(text[pos:m.start() if m else len(text)]))
            if not m:
                break
            out.append(self.special[m.group(0)])
            pos = m.end()
        if self.has_bos:
            out.insert(0, self.bos)
        return out

    def decode(self, ids) -> str:
        b = b"".join(self.decoder[i] if i in self.decoder else self.special_dec[i] for i in ids)
        return b.decode("utf-8", errors="replace").replace("Ġ", " ")

    def vocab_size(self) -> int:
        return len(self.ranks) + len(self.special)
