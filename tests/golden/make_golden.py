#!/usr/bin/env python3
"""Writes the committed golden fixtures of tests/golden/.

The expected outputs come from the scalar CPU oracle (oracle/), which
tests/test_oracle.py pins against closed forms, special cases and brute
force before any fixture is trusted.  The reference has no golden vectors
or tests of its own for this path, so these fixtures pin the oracle and the
seeded generator against silent drift, and give the GPU tests fixed cases.

  tiny.npz         h128 E8 K2 I64 gs64: full inputs + outputs for 6 tokens
  tiny_renorm.npz  h256 E16 K4 I128 gs32 with renormalisation, 6 tokens
  cfg0_token.npz   OLMoE-shaped layer, seed 1234: outputs for 2 tokens;
                   inputs are regenerated from the seed and pinned by
                   SHA-256 of the generated layer image and router
  synth.json       SHA-256 of generator outputs (pins the generator)

Usage: python tests/golden/make_golden.py   (from the repository root)
"""
import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from m1moe_amd import synth  # noqa: E402
from oracle import oracle as orc  # noqa: E402


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def small_case(name: str, seed: int, tokens: int, with_bias: bool):
    wl = synth.CONFIGS[name]
    shape = wl.shape()
    s = orc.from_moe_shape(shape)
    img = synth.layer_image(shape, seed, 0)
    router = synth.router(shape, seed, 0)
    xb = synth.activations_bf16(shape, seed, tokens)
    res = synth.residual_f32(shape, seed, tokens)
    bias = synth.zipf_logit_bias(shape.num_experts, 1.1) if with_bias else None
    outs, idxs, ws, lgs = [], [], [], []
    for t in range(tokens):
        o, i, w, lg = orc.moe_decode(s, img, router, synth.bf16_to_f32(xb[t]), res[t], bias)
        outs.append(o)
        idxs.append(i)
        ws.append(w)
        lgs.append(lg)
    eb = orc.offsets(s).expert_bytes
    e = shape.num_experts - 1
    deq = [orc.dequant_proj(s, img[e * eb:(e + 1) * eb], p) for p in range(3)]
    arrays = dict(
        shape=np.array([shape.hidden, shape.num_experts, shape.top_k, shape.intermediate,
                        shape.group_size, shape.norm_topk_prob], np.int32),
        seed=np.array([seed], np.int64), image=img, router=router, x_bf16=xb, residual=res,
        out=np.stack(outs), topk_idx=np.stack(idxs), topk_w=np.stack(ws), logits=np.stack(lgs),
        dequant_expert=np.array([e], np.int32), dequant_gate=deq[0], dequant_up=deq[1],
        dequant_down=deq[2])
    if bias is not None:
        arrays["logit_bias"] = bias
    np.savez_compressed(os.path.join(HERE, f"{name}.npz"), **arrays)


def cfg0_case():
    seed, tokens = 1234, 2
    shape = synth.CONFIGS["cfg0"].shape()
    s = orc.from_moe_shape(shape)
    img = synth.layer_image(shape, seed, 0)
    router = synth.router(shape, seed, 0)
    xb = synth.activations_bf16(shape, seed, tokens)
    res = synth.residual_f32(shape, seed, tokens)
    outs, idxs, ws, lgs = [], [], [], []
    for t in range(tokens):
        o, i, w, lg = orc.moe_decode(s, img, router, synth.bf16_to_f32(xb[t]), res[t])
        outs.append(o)
        idxs.append(i)
        ws.append(w)
        lgs.append(lg)
    np.savez_compressed(
        os.path.join(HERE, "cfg0_token.npz"), seed=np.array([seed], np.int64),
        image_sha256=np.array(sha(img)), router_sha256=np.array(sha(router)),
        x_bf16=xb, residual=res, out=np.stack(outs), topk_idx=np.stack(idxs),
        topk_w=np.stack(ws), logits=np.stack(lgs))


def synth_checksums():
    shape = synth.CONFIGS["tiny"].shape()
    d = {
        "layer_image(tiny, seed=5, layer=3)": sha(synth.layer_image(shape, 5, 3)),
        "router(tiny, seed=5, layer=3)": sha(synth.router(shape, 5, 3)),
        "activations_bf16(tiny, seed=5, T=7)": sha(synth.activations_bf16(shape, 5, 7)),
        "residual_f32(tiny, seed=5, T=7)": sha(synth.residual_f32(shape, 5, 7)),
        "normal_bf16(seed=9, id=77, n=1000, sigma=0.5)": sha(synth.normal_bf16(9, 77, 1000, 0.5)),
        "normal_f32(seed=9, id=78, n=1000, sigma=2.0)": sha(synth.normal_f32(9, 78, 1000, 2.0)),
    }
    with open(os.path.join(HERE, "synth.json"), "w") as f:
        json.dump(d, f, indent=1, sort_keys=True)


if __name__ == "__main__":
    small_case("tiny", 11, 6, with_bias=False)
    small_case("tiny_renorm", 12, 6, with_bias=True)
    cfg0_case()
    synth_checksums()
    for f in sorted(os.listdir(HERE)):
        if f.endswith((".npz", ".json")):
            print(f, os.path.getsize(os.path.join(HERE, f)), "bytes")
