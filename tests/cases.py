"""Shared set-up of seeded MoE-layer cases for the GPU parity tests."""
from __future__ import annotations

import os
import sys
from dataclasses import dataclass, field

import numpy as np

import m1moe_amd as m
from m1moe_amd import synth
from oracle import oracle as orc

REL_L2_TOL = 1e-2  # layer outputs vs the oracle


def rel_l2(got, want) -> float:
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    return float(np.linalg.norm(got - want) / max(np.linalg.norm(want), 1e-300))


_PROGRESS = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "gpurun_out")


def say(msg: str) -> None:
    """Names the case before a GPU step (flushed, in case the step never
    returns); also appended to gpurun_out/test_progress.log when that folder
    exists, so a long test shows progress while pytest holds its output."""
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()
    if os.path.isdir(_PROGRESS):
        try:
            with open(os.path.join(_PROGRESS, "test_progress.log"), "a") as f:
                f.write(f"[case] {msg}\n")
        except OSError:
            pass


@dataclass
class Case:
    name: str
    shape: m.MoEShape
    seed: int
    ctx: m.HIPContext
    images: list
    routers: list
    biases: list = field(default_factory=list)

    @property
    def oshape(self):
        return orc.from_moe_shape(self.shape)

    def x_bf16(self, T: int, stream: int = 0) -> np.ndarray:
        return synth.activations_bf16(self.shape, self.seed, T, stream)

    def residual(self, T: int, stream: int = 0) -> np.ndarray:
        return synth.residual_f32(self.shape, self.seed, T, stream)

    def close(self):
        self.ctx.close()


def make_case(name: str, seed: int = 1234, num_layers: int = 1, router_override=None,
              bias=None) -> Case:
    wl = synth.CONFIGS[name]
    shape = wl.shape(num_layers)
    say(f"create context {name} seed={seed} layers={num_layers}")
    ctx = m.HIPContext(shape)
    images, routers, biases = [], [], []
    for layer in range(num_layers):
        img = synth.layer_image(shape, seed, layer)
        r = synth.router(shape, seed, layer) if router_override is None else router_override
        ctx.upload_layer_experts(layer, img)
        ctx.upload_router(layer, r)
        if bias is not None:
            ctx.set_logit_bias(layer, bias)
        images.append(img)
        routers.append(np.ascontiguousarray(r))
        biases.append(bias)
    return Case(name, shape, seed, ctx, images, routers, biases)


# ---- a small byte-level tokenizer.json (chat tests) -----------------------------------------

_BYTE_MERGES = [("Ġ", "t"), ("h", "e"), ("Ġt", "he"), ("i", "n"), ("e", "r"), ("Ġ", "a"),
                ("o", "u"), ("Ġ", "s"), ("r", "e"), ("o", "n"), ("Ġ", "w"), ("a", "t"),
                ("e", "n"), ("Ġ", "b"), ("Ġ", "m"), ("in", "g"), ("Ġ", "o"), ("Ġ", "h"),
                ("l", "l"), ("|", ">"), ("<", "|"), ("Ċ", "<|"), ("u", "s"), ("us", "er")]


def write_byte_tokenizer(path, eos_id: int = 299) -> dict:
    """A GPT-2 style tokenizer.json whose ids fit a 300-entry vocabulary:
    the 256 byte characters at ids 0..255, one id per merge after them, and
    "<|endoftext|>" at eos_id.  Merges are "a b" strings (the form the
    reference reads)."""
    import json as _json

    own = set(range(33, 127)) | set(range(161, 173)) | set(range(174, 256))
    chars, extra = [], 0
    for b in range(256):
        if b in own:
            chars.append(chr(b))
        else:
            chars.append(chr(256 + extra))
            extra += 1
    vocab = {c: i for i, c in enumerate(chars)}
    for a, b in _BYTE_MERGES:
        vocab.setdefault(a + b, len(vocab))
    assert len(vocab) < eos_id
    vocab["<|endoftext|>"] = eos_id
    js = {"version": "1.0", "added_tokens": [], "normalizer": None,
          "model": {"type": "BPE", "dropout": None, "unk_token": None, "byte_fallback": False,
                    "vocab": vocab, "merges": [f"{a} {b}" for a, b in _BYTE_MERGES]}}
    with open(path, "w", encoding="utf-8") as f:
        _json.dump(js, f, ensure_ascii=False)
    return js
