"""The converters' 4-bit group quantizer over the C ABI (m1moe_quantize_4bit).

``quantize_4bit(w, group_size)`` is quantize_4bit of
scripts/extract_olmoe.py:116-159 (and extract_mixtral.py:93-116): packed u32
nibbles [rows, cols/8], bf16 scales and biases [rows, cols/group_size], as
the library's host code (m1moe_amd/csrc/quant.cpp) computes them.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

from . import _lib
from ._lib import MoEShape, check


def _threads(threads: int | None) -> int:
    return int(threads) if threads else min(16, os.cpu_count() or 1)


def quantize_4bit(w: np.ndarray, group_size: int = 64, threads: int | None = None):
    """(packed u32 [rows, cols/8], scales bf16 bits [rows, cols/gs], biases
    bf16 bits [rows, cols/gs]) of a 2-D f32 matrix."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    if w.ndim != 2:
        raise ValueError(f"quantize_4bit: a 2-D matrix is needed, got shape {w.shape}")
    rows, cols = w.shape
    packed = np.empty((rows, max(cols // 8, 0)), np.uint32)
    ng = cols // group_size if group_size > 0 and cols % group_size == 0 else 0
    scales = np.empty((rows, ng), np.uint16)
    biases = np.empty((rows, ng), np.uint16)
    check(_lib.load().m1moe_quantize_4bit(
        w.ctypes.data, rows, cols, int(group_size), packed.ctypes.data, scales.ctypes.data,
        biases.ctypes.data, _threads(threads)), "m1moe_quantize_4bit")
    return packed, scales, biases


def quantize_expert(shape: MoEShape, gate: np.ndarray, up: np.ndarray, down: np.ndarray,
                    threads: int | None = None) -> np.ndarray:
    """One expert block (u8 bytes, [gate W|S|B][up W|S|B][down W|S|B]) from
    f32 gate [I, h], up [I, h], down [h, I]."""
    from .engine import expert_bytes

    h, inter = shape.hidden, shape.intermediate
    mats = []
    for name, m, want in (("gate", gate, (inter, h)), ("up", up, (inter, h)),
                          ("down", down, (h, inter))):
        m = np.ascontiguousarray(m, dtype=np.float32)
        if m.shape != want:
            raise ValueError(f"quantize_expert: {name} has shape {m.shape}, expected {want}")
        mats.append(m)
    out = np.empty(expert_bytes(shape), np.uint8)
    check(_lib.load().m1moe_quantize_expert(
        ctypes.byref(shape), mats[0].ctypes.data, mats[1].ctypes.data, mats[2].ctypes.data,
        out.ctypes.data, out.size, _threads(threads)), "m1moe_quantize_expert")
    return out


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """f32_to_bf16 of extract_olmoe.py:104-111 (round to nearest even)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint16)
    check(_lib.load().m1moe_f32_to_bf16(x.ctypes.data, x.size, out.ctypes.data),
          "m1moe_f32_to_bf16")
    return out


__all__ = ["quantize_4bit", "quantize_expert", "f32_to_bf16"]
