"""The BPE tokenizer (Sources/M1MoE/Tokenizer.swift) on the CPU.

Vocabularies are trained here with the HuggingFace `tokenizers` library on a
seeded synthetic corpus (ASCII, accented Latin, Greek, CJK, emoji): a GPT-2
style byte-level BPE (the OLMoE mode) and a SentencePiece-style BPE with
'▁' words and <0xNN> byte fallback (the Mixtral mode), each written as a
tokenizer.json with merges as "a b" strings, the form the reference reads.

The oracle (oracle/tokenizer_oracle.py) is pinned against `tokenizers`
itself: its byte table against ByteLevel.alphabet() and known answers, its
merge loop against the library's BPE model on the same pre-split words
(with and without byte fallback), plus the round-trip identities of both
modes.  The library (m1moe_tokenizer_*) must then equal the oracle on every
string and id list here.
"""
from __future__ import annotations

import ctypes
import json

import numpy as np
import pytest

from m1moe_amd import _lib
from m1moe_amd._lib import M1MoEError
from m1moe_amd.tokenizer import Tokenizer
from oracle.tokenizer_oracle import META, OracleTokenizer, byte_table

tokenizers = pytest.importorskip("tokenizers")
from tokenizers import models, pre_tokenizers, trainers  # noqa: E402

_WORDS = ["the", "model", "expert", "router", "token", "layer", "gate", "merge", "shard",
          "résumé", "naïve", "Ærø", "straße", "λόγος", "μοντέλο", "東京", "模型", "专家",
          "🙂", "🚀x", "á", "tab\there", "line\nbreak", "1234", "3.14", "e=mc²",
          # repeated pairs: the leftmost of equal ranks must merge first
          "aaaa", "aaaaaa", "kakaka", "erer", "ooo", "🙂🙂🙂", "ééé", "tetete"]


_SYLLABLES = ["ka", "ro", "mi", "tes", "un", "ex", "pert", "ou", "ter", "shar", "lay", "é", "ß",
               "λο", "γο", "東", "京", "模", "型", "🙂", "qu", "ing", "tion", "st", "a", "e"]


def _corpus(seed=0, n=1500):
    """Lines of known words and seeded random syllable words (so that the
    trainer learns several hundred merges of varied lengths)."""
    rng = np.random.default_rng(seed)
    made = ["".join(_SYLLABLES[int(j)] for j in rng.integers(0, len(_SYLLABLES),
                                                              int(rng.integers(1, 5))))
            for _ in range(400)]
    pool = _WORDS + made
    lines = []
    for _ in range(n):
        k = int(rng.integers(1, 12))
        lines.append(" ".join(pool[int(i)] for i in rng.integers(0, len(pool), k)))
    return lines


def _strings(seed=1, n=150):
    rng = np.random.default_rng(seed)
    out = ["", " ", "  ", "a", " a", "a ", "a  b", "   lead", "trail   ", "\n", " \n ",
           "Hello world", "expert router", "東京 模型🙂", "á b́", "<s>", "<|endoftext|>",
           "x" * 300, "🚀" * 40, "tokens nbsp", "zero​width",
           "aaa", "aaaaa", "aaaaaaa", "kakak", "erererer", "oooo ooooo", "🙂🙂", "éééé"]
    pool = _WORDS + ["", " ", "  ", "unseen", "ÿþ", "́", "€", "𝔘𝔫𝔦", "\t"]
    for _ in range(n):
        k = int(rng.integers(0, 10))
        out.append("".join(pool[int(i)] + (" " if rng.random() < 0.6 else "")
                           for i in rng.integers(0, len(pool), k)))
    return out


def _write(path, tok, byte_fallback):
    js = json.loads(tok.to_str())
    m = js["model"]
    m["merges"] = [" ".join(p) if isinstance(p, list) else p for p in m["merges"]]
    m["byte_fallback"] = byte_fallback
    path.write_text(json.dumps(js, ensure_ascii=bool(byte_fallback)), encoding="utf-8")
    return js


@pytest.fixture(scope="module")
def byte_level(tmp_path_factory):
    tok = tokenizers.Tokenizer(models.BPE())
    tok.pre_tokenizer = pre_tokenizers.ByteLevel(add_prefix_space=False)
    tr = trainers.BpeTrainer(vocab_size=700, initial_alphabet=pre_tokenizers.ByteLevel.alphabet(),
                             special_tokens=["<|endoftext|>", "<|pad|>"], show_progress=False)
    tok.train_from_iterator(_corpus(0), tr)
    path = tmp_path_factory.mktemp("bl") / "tokenizer.json"
    js = _write(path, tok, False)
    return str(path), js


@pytest.fixture(scope="module")
def sentencepiece(tmp_path_factory):
    tok = tokenizers.Tokenizer(models.BPE(byte_fallback=True, unk_token="<unk>"))
    tok.pre_tokenizer = pre_tokenizers.Metaspace(replacement=META, prepend_scheme="always")
    specials = ["<unk>", "<s>", "</s>", "<pad>", "<|im_end|>"] + ["<0x%02X>" % b for b in range(256)]
    tr = trainers.BpeTrainer(vocab_size=900, special_tokens=specials, show_progress=False)
    tok.train_from_iterator(_corpus(3), tr)
    path = tmp_path_factory.mktemp("sp") / "tokenizer.json"
    js = _write(path, tok, True)
    return str(path), js


def _hf_bpe(js, byte_fallback):
    m = js["model"]
    merges = [tuple(s.split(" ", 1)) for s in m["merges"]]
    kw = dict(byte_fallback=True, unk_token="<unk>") if byte_fallback else {}
    return tokenizers.Tokenizer(models.BPE(vocab=m["vocab"], merges=merges, **kw))


# ---- the oracle, pinned ------------------------------------------------------------

def test_byte_table_is_gpt2s():
    t = byte_table()
    assert set(t.values()) == set(pre_tokenizers.ByteLevel.alphabet())
    assert len(set(t.values())) == 256
    assert t[0x20] == "Ġ" and t[0x0A] == "Ċ" and t[0x00] == "Ā"
    assert t[0xAD] == "Ń" and t[ord("A")] == "A" and t[0xFF] == "ÿ"


def test_oracle_merges_match_the_bpe_model_byte_level(byte_level):
    path, js = byte_level
    o, hf = OracleTokenizer(path), _hf_bpe(js, False)
    n = 0
    for s in _strings():
        for w in o.byte_level_words(s):
            got = o.bpe(list(w))
            assert got == hf.encode(w).tokens, (s, w)
            n += 1
    assert n > 300


def test_oracle_merges_match_the_bpe_model_with_byte_fallback(sentencepiece):
    path, js = sentencepiece
    o, hf = OracleTokenizer(path), _hf_bpe(js, True)
    assert o.sentencepiece
    n = 0
    for s in _strings():
        for w in o.sentencepiece_words(s):
            want = hf.encode(w).ids
            assert o.encode(w[len(META):], add_bos=False) == want, (s, w)
            n += 1
    assert n > 300


def test_oracle_round_trips(byte_level, sentencepiece):
    bl, sp = OracleTokenizer(byte_level[0]), OracleTokenizer(sentencepiece[0])
    for s in _strings():
        assert bl.decode(bl.encode(s, add_bos=False)) == s
        want = "".join(" " + w for w in s.split(" ") if w)
        assert sp.decode(sp.encode(s, add_bos=True)) == want


# ---- the library against the oracle ---------------------------------------------------

@pytest.mark.parametrize("mode", ["byte_level", "sentencepiece"])
def test_encode_equals_oracle(mode, request):
    path, _ = request.getfixturevalue(mode)
    o, t = OracleTokenizer(path), Tokenizer(path)
    assert t.mode == mode and t.vocab_size == len(o.vocab)
    for s in _strings():
        for add_bos, bos in ((True, 1), (False, 1), (True, 7)):
            assert t.encode(s, add_bos, bos) == o.encode(s, add_bos, bos), repr(s)


@pytest.mark.parametrize("mode", ["byte_level", "sentencepiece"])
def test_decode_equals_oracle(mode, request):
    path, _ = request.getfixturevalue(mode)
    o, t = OracleTokenizer(path), Tokenizer(path)
    rng = np.random.default_rng(9)
    n = len(o.vocab)
    lists = [[], [0], [1, 2, 3], [n + 5], [2**32 - 1], list(range(n))]
    lists += [list(rng.integers(0, n + 20, int(rng.integers(1, 30)))) for _ in range(300)]
    for s in _strings()[:60]:
        lists.append(o.encode(s))
    for ids in lists:
        for skip in (True, False):
            assert t.decode(ids, skip) == o.decode(ids, skip), ids


def test_decode_falls_back_to_latin1(byte_level, sentencepiece):
    sp = Tokenizer(sentencepiece[0])
    o = OracleTokenizer(sentencepiece[0])
    lone = [o.vocab["<0xC3>"]]
    assert sp.decode(lone) == "Ã" == o.decode(lone)
    pair = [o.vocab["<0xC3>"], o.vocab["<0xA9>"]]
    assert sp.decode(pair) == "é"
    bl = Tokenizer(byte_level[0])
    ob = OracleTokenizer(byte_level[0])
    lone = [ob.vocab[byte_table()[0xE6]]]
    assert bl.decode(lone) == "æ" == ob.decode(lone)


def test_special_tokens_in_both_modes(byte_level, sentencepiece):
    sp, o = Tokenizer(sentencepiece[0]), OracleTokenizer(sentencepiece[0])
    ids = [o.vocab["<s>"], o.vocab["▁the"] if "▁the" in o.vocab else o.vocab["<0x41>"],
           o.vocab["<|im_end|>"], o.vocab["</s>"]]
    kept = sp.decode(ids, skip_special=False)
    assert kept.startswith("<s>") and kept.endswith("<|im_end|></s>")
    assert "<" not in sp.decode(ids, skip_special=True)
    # byte-level keeps special tokens as text either way (its decoder has no special list)
    bl, ob = Tokenizer(byte_level[0]), OracleTokenizer(byte_level[0])
    assert bl.decode([ob.vocab["<|endoftext|>"]]) == "<|endoftext|>"


def test_reference_merge_line_split(tmp_path):
    """Leading spaces produce no part; the second part keeps further spaces;
    a line without two parts is ignored but still takes a rank."""
    js = {"model": {"vocab": {"a": 0, "b": 1, "ab": 2, "c": 3, "bc": 4, "abc": 5},
                    "merges": ["  b c", "nospace", "a b", "ab c"]}}
    p = tmp_path / "t.json"
    p.write_text(json.dumps(js))
    t, o = Tokenizer(str(p)), OracleTokenizer(str(p))
    assert t.num_merges == 3
    # 'b c' has rank 0 and wins over 'a b' (rank 2): a|bc, and no 'a bc' merge
    assert t.encode("abc", add_bos=False) == o.encode("abc", add_bos=False) == [0, 4]


def test_bad_inputs_are_refused(tmp_path, byte_level):
    lib = _lib.load()
    h = ctypes.c_void_p()
    cases = {"missing.json": None,
             "notjson.json": "{\"model\": ",
             "nomodel.json": json.dumps({"x": 1}),
             "novocab.json": json.dumps({"model": {"merges": []}}),
             "nomerges.json": json.dumps({"model": {"vocab": {"a": 0}}}),
             "mergenum.json": json.dumps({"model": {"vocab": {"a": 0}, "merges": ["a b", 3]}}),
             "negid.json": json.dumps({"model": {"vocab": {"a": -1}, "merges": []}}),
             "surrogate.json": '{"model": {"vocab": {"\\ud800": 0}, "merges": []}}'}
    for name, text in cases.items():
        p = tmp_path / name
        if text is not None:
            p.write_text(text)
        assert lib.m1moe_tokenizer_load(str(p).encode(), ctypes.byref(h)) == _lib.M1MOE_ERR_INVALID, name
        assert not h.value
    ok = tmp_path / "ok.json"
    ok.write_text(json.dumps({"model": {"vocab": {"a": 0, "b": 1.0, "c": 2.5, "d": "x"},
                                        "merges": [], "byte_fallback": None}}))
    t = Tokenizer(str(ok))
    assert t.vocab_size == 2 and t.mode == "byte_level"     # 2.5 and "x" are not Int ids
    t = Tokenizer(byte_level[0])
    n = ctypes.c_uint64()
    bad = b"\xff\xfe"
    assert lib.m1moe_tokenizer_encode(t.handle, bad, 2, 1, 1, None, 0, ctypes.byref(n)) == \
        _lib.M1MOE_ERR_INVALID
    ids = np.zeros(1, np.uint32)
    assert lib.m1moe_tokenizer_encode(t.handle, b"hello world", 11, 1, 1, ids.ctypes.data, 1,
                                      ctypes.byref(n)) == _lib.M1MOE_ERR_INVALID
    assert n.value == len(t.encode("hello world"))
    with pytest.raises(M1MoEError):
        Tokenizer(str(tmp_path / "missing.json"))
