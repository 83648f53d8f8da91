"""Pure-Python restatement of the reference tokenizer (Sources/M1MoE/Tokenizer.swift).

TEST INFRASTRUCTURE ONLY: the checker m1moe_tokenizer_* is compared against.
Only tests/ may import it.

  load            Tokenizer.init(url:)            :35-62
  encode          encode(_:addBOS:bos:)           :66-72
  byte-level      encodeByteLevelBPE / decode...  :86-130
  SentencePiece   encodeSentencePiece / decode... :134-207
  BPE             applyBPE                        :212-228
  byte table      makeByteLevelEncoder            :232-248

Strings are Python str (code points); merges split at the first space after
any leading spaces (Swift's split(separator:maxSplits: 1) omits empty
leading parts).  Pinned in tests/test_tokenizer.py against the HuggingFace
`tokenizers` library (its GPT-2 byte alphabet and its BPE model, with and
without byte fallback, on pre-split words), known answers of the byte table,
and round-trip identities of both modes.
"""
from __future__ import annotations

import json
from typing import Dict, List, Tuple

META = "▁"  # '▁'


def byte_table() -> Dict[int, str]:
    """GPT-2's byte -> character table: printable Latin-1 bytes map to
    themselves, the remaining 68 bytes to U+0100.. in byte order."""
    own = set(range(33, 127)) | set(range(161, 173)) | set(range(174, 256))
    table, extra = {}, 0
    for b in range(256):
        if b in own:
            table[b] = chr(b)
        else:
            table[b] = chr(256 + extra)
            extra += 1
    return table


_ENC = byte_table()
_DEC = {c: b for b, c in _ENC.items()}


def _split_merge(line: str):
    s = line.lstrip(" ")
    i = s.find(" ")
    if i < 0 or i + 1 >= len(s):
        return None
    return s[:i], s[i + 1:]


class OracleTokenizer:
    def __init__(self, path: str):
        with open(path, "rb") as f:
            root = json.loads(f.read().decode("utf-8"))
        model = root.get("model") if isinstance(root, dict) else None
        if not isinstance(model, dict) or not isinstance(model.get("vocab"), dict):
            raise ValueError("invalid format")
        merges = model.get("merges")
        if not isinstance(merges, list) or not all(isinstance(m, str) for m in merges):
            raise ValueError("invalid format")
        bf = model.get("byte_fallback", False)
        self.sentencepiece = bf is True or (type(bf) in (int, float) and bf == 1)
        self.vocab: Dict[str, int] = {}
        for k, v in model["vocab"].items():
            if type(v) in (int, float) and float(v).is_integer():
                self.vocab[k] = int(v)
        self.piece: Dict[int, str] = {}
        for k, v in self.vocab.items():
            if v not in self.piece or k.encode() < self.piece[v].encode():
                self.piece[v] = k
        self.rank: Dict[Tuple[str, str], int] = {}
        for r, m in enumerate(merges):
            ab = _split_merge(m)
            if ab is not None:
                self.rank[ab] = r

    # ---- BPE -------------------------------------------------------------
    def bpe(self, syms: List[str]) -> List[str]:
        syms = list(syms)
        while len(syms) > 1:
            best, at = None, -1
            for i in range(len(syms) - 1):
                r = self.rank.get((syms[i], syms[i + 1]))
                if r is not None and (best is None or r < best):
                    best, at = r, i
            if at < 0:
                break
            syms[at:at + 2] = [syms[at] + syms[at + 1]]
        return syms

    # ---- words ---------------------------------------------------------------
    @staticmethod
    def byte_level_words(text: str) -> List[str]:
        words, cur = [], ""
        for i, ch in enumerate(text):
            if ch == " " and cur:
                words.append(cur)
                cur = _ENC[0x20]
            elif i == 0 and ch == " ":
                cur = _ENC[0x20]
            else:
                cur += "".join(_ENC[b] for b in ch.encode("utf-8"))
        if cur:
            words.append(cur)
        return words

    @staticmethod
    def sentencepiece_words(text: str) -> List[str]:
        return [META + w for w in text.split(" ") if w]

    def encode(self, text: str, add_bos: bool = True, bos: int = 1) -> List[int]:
        ids = [bos] if add_bos else []
        if not text:
            return ids
        if not self.sentencepiece:
            for w in self.byte_level_words(text):
                ids += [self.vocab[s] for s in self.bpe(list(w)) if s in self.vocab]
            return ids
        for w in self.sentencepiece_words(text):
            for s in self.bpe(list(w)):
                if s in self.vocab:
                    ids.append(self.vocab[s])
                else:
                    ids += [self.vocab[t] for t in ("<0x%02X>" % b for b in s.encode("utf-8"))
                            if t in self.vocab]
        return ids

    # ---- decode ----------------------------------------------------------------
    @staticmethod
    def _special(p: str) -> bool:
        return p in ("<s>", "</s>", "<unk>", "<pad>") or (p.startswith("<|") and p.endswith("|>"))

    @staticmethod
    def _byte_piece(p: str):
        if len(p) != 6 or not p.startswith("<0x") or not p.endswith(">"):
            return None
        h = p[3:5]
        digits = "0123456789abcdefABCDEF"
        if h[0] in "+-" and h[1] in digits:
            v = int(h[1], 16)
            return v if h[0] == "+" or v == 0 else None
        if h[0] in digits and h[1] in digits:
            return int(h, 16)
        return None

    def decode(self, ids, skip_special: bool = True) -> str:
        out = bytearray()
        for i in ids:
            p = self.piece.get(int(i))
            if p is None:
                continue
            if not self.sentencepiece:
                out += bytes(_DEC[c] for c in p if c in _DEC)
                continue
            if self._special(p):
                if not skip_special:
                    out += p.encode("utf-8")
                continue
            b = self._byte_piece(p)
            if b is not None:
                out.append(b)
                continue
            out += p.replace(META, " ").encode("utf-8")
        try:
            return bytes(out).decode("utf-8")
        except UnicodeDecodeError:
            return bytes(out).decode("latin-1")


__all__ = ["OracleTokenizer", "byte_table", "META"]
