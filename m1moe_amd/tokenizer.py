"""Tokenizer (Sources/M1MoE/Tokenizer.swift) over the C ABI.

``Tokenizer(path)`` reads a HuggingFace tokenizer.json; ``encode(text,
add_bos=True, bos=1)`` and ``decode(ids, skip_special=True)`` are
encode(_:addBOS:bos:) and decode(_:skipSpecial:) of the reference (:66-81).
The work is done by the library's host code (m1moe_amd/csrc/tokenizer.cpp):
byte-level BPE for GPT-2 style vocabularies (OLMoE), SentencePiece BPE with
byte fallback when model.byte_fallback is true (Mixtral).
"""
from __future__ import annotations

import ctypes
from typing import Iterable, List

import numpy as np

from . import _lib
from ._lib import check


class Tokenizer:
    def __init__(self, path: str):
        self.lib = _lib.load()
        h = ctypes.c_void_p()
        check(self.lib.m1moe_tokenizer_load(str(path).encode(), ctypes.byref(h)),
              "m1moe_tokenizer_load")
        self.handle = h
        sp, nv, nm = ctypes.c_int32(), ctypes.c_uint64(), ctypes.c_uint64()
        check(self.lib.m1moe_tokenizer_info(self.handle, ctypes.byref(sp), ctypes.byref(nv),
                                            ctypes.byref(nm)), "m1moe_tokenizer_info")
        self.sentencepiece = bool(sp.value)
        self.vocab_size = int(nv.value)
        self.num_merges = int(nm.value)

    @property
    def mode(self) -> str:
        return "sentencepiece" if self.sentencepiece else "byte_level"

    def close(self) -> None:
        if getattr(self, "handle", None):
            self.lib.m1moe_tokenizer_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def encode(self, text: str, add_bos: bool = True, bos: int = 1) -> List[int]:
        data = text.encode("utf-8")
        n = ctypes.c_uint64()
        # at most 4 ids per byte (a SentencePiece word of one unknown byte: the
        # three bytes of U+2581 and its own, by byte fallback) + the BOS: one call
        ids = np.empty(4 * len(data) + 8, np.uint32)
        check(self.lib.m1moe_tokenizer_encode(self.handle, data, len(data), int(add_bos),
                                              int(bos), ids.ctypes.data, ids.size,
                                              ctypes.byref(n)), "m1moe_tokenizer_encode")
        return ids[:n.value].tolist()

    def decode(self, ids: Iterable[int], skip_special: bool = True) -> str:
        a = np.ascontiguousarray(list(ids), dtype=np.uint32)
        n = ctypes.c_uint64()
        check(self.lib.m1moe_tokenizer_decode(self.handle, a.ctypes.data if a.size else None,
                                              a.size, int(skip_special), None, 0,
                                              ctypes.byref(n)), "m1moe_tokenizer_decode")
        buf = ctypes.create_string_buffer(int(n.value) + 1)
        check(self.lib.m1moe_tokenizer_decode(self.handle, a.ctypes.data if a.size else None,
                                              a.size, int(skip_special), buf, len(buf),
                                              ctypes.byref(n)), "m1moe_tokenizer_decode")
        return buf.raw[:n.value].decode("utf-8")


__all__ = ["Tokenizer"]
