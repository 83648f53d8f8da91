"""Checkpoint converter: HuggingFace safetensors -> the reference's on-disk format.

The offline step of scripts/extract_olmoe.py and scripts/extract_mixtral.py
(the two differ only in the expert tensor names):

  <out>/model_weights.bin   every non-expert tensor, in the order the
                            reference writes them (non-expert names sorted,
                            grouped by the shard of their first appearance,
                            each shard's tensors in its header order), each
                            start 4-byte aligned (extract_olmoe.py:216-262);
                            BF16 kept, F16 -> f32 -> bf16, F32 kept as f32
  <out>/model_weights.json  {name: {offset, shape, dtype}} (json.dump, indent 2)
  <out>/packed_experts/layer_NN.bin
                            per layer, experts in index order, per expert
                            gate, up, down, each W|S|B from the 4-bit group
                            quantizer (extract_olmoe.py:268-345)

Expert names: OLMoE ``model.layers.L.mlp.experts.E.{gate,up,down}_proj.weight``
(extract_olmoe.py:203-206, 289-300), Mixtral
``model.layers.L.block_sparse_moe.experts.E.{w1,w3,w2}.weight`` with w1 =
gate, w3 = up, w2 = down (extract_mixtral.py:144-146, 215-235).  The
quantizer is the library's (m1moe_quantize_4bit, host threads); tensors are
read through memory maps one matrix at a time, so a 47 B-parameter
checkpoint converts in bounded memory.

  python -m m1moe_amd.convert --model-dir CKPT --out-dir OUT [--group-size 64]
"""
from __future__ import annotations

import argparse
import json
import os
import struct
import sys
from collections import defaultdict
from pathlib import Path

import numpy as np

from .quant import f32_to_bf16, quantize_4bit

_DTYPES = {"BF16": np.uint16, "F16": np.float16, "F32": np.float32}

# expert tensor naming per architecture: (marker, {name part: projection})
_EXPERT_NAMING = {
    "olmoe": (".mlp.experts.", {"gate_proj": "gate", "up_proj": "up", "down_proj": "down"}),
    "mixtral": (".block_sparse_moe.experts.", {"w1": "gate", "w3": "up", "w2": "down"}),
}


class Shard:
    """One .safetensors file: its header (in file order) and memory-mapped tensors."""

    def __init__(self, path: Path):
        self.path = path
        with open(path, "rb") as f:
            (n,) = struct.unpack("<Q", f.read(8))
            self.header = json.loads(f.read(n))
        self.data_offset = 8 + n
        self._map = None

    def names(self):
        return [k for k in self.header if k != "__metadata__"]

    def tensor(self, name: str):
        """The tensor as numpy (BF16 as its u16 bits), or None for a dtype
        the converter does not handle (the reference skips those too)."""
        info = self.header[name]
        dt = _DTYPES.get(info["dtype"])
        if dt is None:
            return None
        if self._map is None:
            self._map = np.memmap(self.path, dtype=np.uint8, mode="r")
        a, b = info["data_offsets"]
        raw = self._map[self.data_offset + a:self.data_offset + b]
        return raw.view(dt).reshape(info["shape"])


def _as_f32(arr: np.ndarray) -> np.ndarray:
    if arr.dtype == np.uint16:  # BF16 bits
        return (arr.astype(np.uint32) << 16).view(np.float32)
    return arr.astype(np.float32)


def detect_architecture(names) -> str:
    return "mixtral" if any(_EXPERT_NAMING["mixtral"][0] in n for n in names) else "olmoe"


def convert(model_dir: str, out_dir: str, group_size: int = 64, architecture: str | None = None,
            threads: int | None = None, verbose: bool = True) -> dict:
    """Converts every *.safetensors of model_dir; returns the manifest."""
    model_dir, out_dir = Path(model_dir).expanduser(), Path(out_dir).expanduser()
    paths = sorted(model_dir.glob("*.safetensors"))
    if not paths:
        raise FileNotFoundError(f"no .safetensors files in {model_dir}")
    shards = {str(p): Shard(p) for p in paths}
    where = {}
    for key, sh in shards.items():
        for n in sh.names():
            where[n] = key
    arch = architecture or detect_architecture(where)
    if arch not in _EXPERT_NAMING:
        raise ValueError(f"unknown architecture {arch!r} (olmoe or mixtral)")
    marker, projs = _EXPERT_NAMING[arch]
    out_dir.mkdir(parents=True, exist_ok=True)
    (out_dir / "packed_experts").mkdir(exist_ok=True)

    # -- non-expert tensors -------------------------------------------------
    by_shard: dict = {}
    for n in sorted(k for k in where if marker not in k):
        by_shard.setdefault(where[n], []).append(n)
    manifest, offset = {}, 0
    with open(out_dir / "model_weights.bin", "wb") as f:
        for key, names in by_shard.items():
            sh, wanted = shards[key], set(names)
            for n in sh.names():
                if n not in wanted:
                    continue
                arr = sh.tensor(n)
                if arr is None:
                    print(f"  [skip] {n}: unsupported dtype {sh.header[n]['dtype']}",
                          file=sys.stderr)
                    continue
                if arr.dtype == np.uint16:
                    dtype, raw = "bf16", np.ascontiguousarray(arr).tobytes()
                elif arr.dtype == np.float16:
                    dtype, raw = "bf16", f32_to_bf16(arr.astype(np.float32)).tobytes()
                else:
                    dtype, raw = "f32", np.ascontiguousarray(arr, np.float32).tobytes()
                if offset % 4:
                    pad = 4 - offset % 4
                    f.write(b"\x00" * pad)
                    offset += pad
                manifest[n] = {"offset": offset, "shape": list(arr.shape), "dtype": dtype}
                f.write(raw)
                offset += len(raw)
    with open(out_dir / "model_weights.json", "w") as f:
        json.dump(manifest, f, indent=2)
    if verbose:
        print(f"[convert] {arch}: {len(manifest)} non-expert tensors, {offset / 2**20:.1f} MiB")

    # -- experts ------------------------------------------------------------
    experts = defaultdict(dict)  # (layer, expert) -> {proj: name}
    for n in sorted(k for k in where if marker in k):
        parts = n.split(".")
        try:
            layer, e, proj = int(parts[2]), int(parts[5]), projs.get(parts[6])
        except (IndexError, ValueError):
            print(f"  [warn] unexpected expert tensor name: {n}", file=sys.stderr)
            continue
        if proj is not None:
            experts[(layer, e)][proj] = n
    if not experts:
        return manifest
    first = experts[min(experts)]["gate"]
    inter, hidden = shards[where[first]].header[first]["shape"]
    eb = 0
    for rows, cols in ((inter, hidden), (inter, hidden), (hidden, inter)):
        eb += rows * cols // 2 + 2 * 2 * rows * (cols // group_size)
    for layer in sorted({l for l, _ in experts}):
        ids = sorted(e for l, e in experts if l == layer)
        path = out_dir / "packed_experts" / f"layer_{layer:02d}.bin"
        with open(path, "wb") as f:
            for e in ids:
                for proj in ("gate", "up", "down"):
                    n = experts[(layer, e)][proj]
                    arr = shards[where[n]].tensor(n)
                    packed, scales, biases = quantize_4bit(_as_f32(arr), group_size, threads)
                    f.write(packed.tobytes())
                    f.write(scales.tobytes())
                    f.write(biases.tobytes())
        size = os.path.getsize(path)
        if size != len(ids) * eb:
            raise RuntimeError(f"layer {layer:02d}: {size} bytes, expected {len(ids) * eb}")
        if verbose:
            print(f"[convert] layer {layer:02d}: {len(ids)} experts, {size / 2**20:.0f} MiB")
    return manifest


def main(argv=None) -> int:
    p = argparse.ArgumentParser(description="Convert a safetensors MoE checkpoint "
                                            "(OLMoE or Mixtral) to the M1MoE format")
    p.add_argument("--model-dir", required=True)
    p.add_argument("--out-dir", required=True)
    p.add_argument("--group-size", type=int, default=64)
    p.add_argument("--architecture", choices=sorted(_EXPERT_NAMING), default=None,
                   help="expert naming (default: detected from the tensor names)")
    p.add_argument("--threads", type=int, default=None)
    p.add_argument("--quiet", action="store_true")
    a = p.parse_args(argv)
    convert(a.model_dir, a.out_dir, a.group_size, a.architecture, a.threads, not a.quiet)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
