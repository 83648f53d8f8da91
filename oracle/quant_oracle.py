"""numpy restatement of the reference converters' 4-bit group quantizer.

TEST INFRASTRUCTURE ONLY: the checker m1moe_quantize_4bit /
m1moe_quantize_expert / m1moe_f32_to_bf16 are compared against.  Only
tests/ may import it.

  f32_to_bf16    scripts/extract_olmoe.py:104-111
  quantize_4bit  scripts/extract_olmoe.py:116-159 (extract_mixtral.py:93-116)
  expert block   scripts/extract_olmoe.py:322-338 (gate, up, down; W, S, B)

Pinned in tests/test_quant.py by known answers (exactly representable
groups, round-half-even ties, constant groups, bf16 rounding ties), by
torch's own f32 -> bf16 conversion, and by the dequantisation error bound
|nibble * s + lo - w| <= s / 2.
"""
from __future__ import annotations

import numpy as np


def f32_to_bf16(x) -> np.ndarray:
    """Round-to-nearest-even bf16 bits of f32 values: the f32 bits plus
    0x7FFF plus the kept least significant bit, top half kept (u32 wrap)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    lsb = (u >> np.uint32(16)) & np.uint32(1)
    return ((u + np.uint32(0x7FFF) + lsb) >> np.uint32(16)).astype(np.uint16)


def quantize_4bit(w, group_size: int = 64):
    """(packed u32 [rows, cols/8], scales bf16 [rows, G], biases bf16 [rows, G])
    with G = cols / group_size, all arithmetic in f32."""
    w = np.asarray(w, dtype=np.float32)
    rows, cols = w.shape
    if cols % group_size or cols % 8:
        raise ValueError("cols must be a multiple of group_size and of 8")
    groups = w.reshape(rows, cols // group_size, group_size)
    lo = groups.min(axis=2)
    s = (groups.max(axis=2) - lo) / np.float32(15.0)
    s = np.where(s == np.float32(0), np.float32(1), s).astype(np.float32)
    t = (groups - lo[:, :, None]) / s[:, :, None]
    nib = np.clip(np.rint(t), 0, 15).astype(np.uint32).reshape(rows, cols // 8, 8)
    shifts = (np.arange(8, dtype=np.uint32) * np.uint32(4))
    packed = np.bitwise_or.reduce(nib << shifts, axis=2).astype(np.uint32)
    return packed, f32_to_bf16(s), f32_to_bf16(lo)


def nibbles(packed: np.ndarray) -> np.ndarray:
    """[rows, cols] nibble values of packed [rows, cols/8] words."""
    p = np.asarray(packed, dtype=np.uint32)
    shifts = np.arange(8, dtype=np.uint32) * np.uint32(4)
    return ((p[:, :, None] >> shifts) & np.uint32(15)).reshape(p.shape[0], -1)


def expert_block(gate, up, down, group_size: int = 64) -> np.ndarray:
    """u8 bytes of one expert: gate, up, down, each packed|scales|biases."""
    parts = []
    for m in (gate, up, down):
        for a in quantize_4bit(m, group_size):
            parts.append(np.ascontiguousarray(a).view(np.uint8).reshape(-1))
    return np.concatenate(parts)


__all__ = ["f32_to_bf16", "quantize_4bit", "nibbles", "expert_block"]
