"""Seeded synthetic workloads of the benchmark configurations.

All tensors come from the library's counter-based generator
(m1moe_synth_*), so the same (seed, tensor id, index) gives the same value
on every machine and any slice can be regenerated on its own.

Distributions (2, 3):
  expert nibbles  uniform 0..15, 8 per u32 (reference packing)
  expert scales   bf16 |N(0, 0.02)|
  expert biases   bf16 N(0, 0.01)
  router          bf16 N(0, 0.02)   [E x h]
  x               bf16 N(0, 1)      [T x h]
  residual        f32  N(0, 1)      [T x h]
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass
from typing import Optional

import numpy as np

from . import _lib
from ._lib import MoEShape, check
from .engine import expert_bytes, make_shape

SCALE_SIGMA = 0.02
BIAS_SIGMA = 0.01
ROUTER_SIGMA = 0.02

# tensor-id namespaces of the non-expert tensors
_TID_ROUTER = 2 << 56
_TID_X = 3 << 56
_TID_RESIDUAL = 4 << 56


@dataclass(frozen=True)
class Workload:
    name: str
    shape_kwargs: dict
    T: int = 1             # tokens per call (1 = decode)
    zipf_s: float = 0.0    # router logit bias for a Zipf(s) expert load; 0 = none
    description: str = ""

    def shape(self, num_layers: int = 1) -> MoEShape:
        return make_shape(num_layers=num_layers, **self.shape_kwargs)


CONFIGS = {
    "cfg0": Workload("cfg0", dict(hidden=2048, num_experts=64, top_k=8, intermediate=1024,
                                  group_size=64, norm_topk_prob=False),
                     description="OLMoE-shaped MoE layer, batch-1 decode (h2048 E64 top-8 I1024)"),
    "cfg2": Workload("cfg2", dict(hidden=4096, num_experts=8, top_k=2, intermediate=14336,
                                  group_size=64, norm_topk_prob=True),
                     description="Mixtral-shaped MoE layer, batch-1 decode (h4096 E8 top-2 "
                                 "renorm I14336)"),
    "cfg3": Workload("cfg3", dict(hidden=2048, num_experts=64, top_k=8, intermediate=1024,
                                  group_size=64, norm_topk_prob=False),
                     T=512, zipf_s=1.1,
                     description="OLMoE-shaped MoE layer prefill, 512 tokens, Zipf(1.1) loads"),
    # small shapes for tests
    "tiny": Workload("tiny", dict(hidden=128, num_experts=8, top_k=2, intermediate=64,
                                  group_size=64, norm_topk_prob=False)),
    "tiny_renorm": Workload("tiny_renorm", dict(hidden=256, num_experts=16, top_k=4,
                                                intermediate=128, group_size=32,
                                                norm_topk_prob=True)),
}


@dataclass(frozen=True)
class DecoderWorkload:
    """A full decoder: the MoE layers of `moe` stacked num_layers deep, dense
    weights random-init, `prompt` random token ids then `gen` greedy steps."""
    name: str
    moe: Workload
    num_layers: int
    vocab: int
    num_heads: int
    num_kv_heads: int
    head_dim: int
    rope_theta: float
    qk_norm: bool
    prompt: int
    gen: int
    rms_eps: float = 1e-5
    description: str = ""

    def shape(self) -> MoEShape:
        return self.moe.shape(self.num_layers)

    def dec_shape(self, max_seq: Optional[int] = None):
        from ._lib import DecShape
        return DecShape(self.vocab, self.num_heads, self.num_kv_heads, self.head_dim,
                        int(max_seq or (self.prompt + self.gen)), 1 if self.qk_norm else 0,
                        self.rope_theta, self.rms_eps)


_OLMOE_MOE = Workload("olmoe", dict(hidden=2048, num_experts=64, top_k=8, intermediate=1024,
                                    group_size=64, norm_topk_prob=False))
_MIXTRAL_MOE = Workload("mixtral", dict(hidden=4096, num_experts=8, top_k=2, intermediate=14336,
                                        group_size=64, norm_topk_prob=False))

# BASELINE.json configs 1 and 4 (architecture values of configs/olmoe-1b-7b.json and
# configs/mixtral-8x7b.json; Mixtral's norm_topk_prob is that file's false)
DECODERS = {
    "cfg1": DecoderWorkload("cfg1", _OLMOE_MOE, 16, 50304, 16, 16, 128, 10000.0, True, 128, 128,
                            description="OLMoE-1B-7B-shaped decoder, 16 layers, 128-token "
                                        "prompt then 128 greedy steps, batch 1"),
    "cfg4": DecoderWorkload("cfg4", _MIXTRAL_MOE, 32, 32000, 32, 8, 128, 1e6, False, 2048, 64,
                            description="Mixtral-8x7B-shaped decoder, 32 layers, 2048-token "
                                        "context then 64 greedy steps, batch 1"),
    # small decoders for tests: GQA 2:1, KV cache over two attention chunks
    "tiny_dec": DecoderWorkload("tiny_dec", CONFIGS["tiny"], 2, 300, 2, 1, 64, 10000.0, True,
                                8, 8),
}


def _threads() -> int:
    return max(1, min(16, os.cpu_count() or 1))


def layer_image(shape: MoEShape, seed: int, layer: int) -> np.ndarray:
    """One layer_NN.bin image (E expert blocks) as uint8."""
    nbytes = shape.num_experts * expert_bytes(shape)
    out = np.empty(nbytes, dtype=np.uint8)
    check(_lib.load().m1moe_synth_layer_image(
        ctypes.byref(shape), ctypes.c_uint64(seed), int(layer), ctypes.c_float(SCALE_SIGMA),
        ctypes.c_float(BIAS_SIGMA), ctypes.c_void_p(out.ctypes.data), ctypes.c_uint64(nbytes),
        _threads()), "m1moe_synth_layer_image")
    return out


def normal_bf16(seed: int, tensor_id: int, n: int, sigma: float, absval: bool = False) -> np.ndarray:
    out = np.empty(n, dtype=np.uint16)
    check(_lib.load().m1moe_synth_normal_bf16(ctypes.c_uint64(seed), ctypes.c_uint64(tensor_id),
                                              ctypes.c_uint64(n), ctypes.c_float(sigma),
                                              1 if absval else 0, ctypes.c_void_p(out.ctypes.data)),
          "m1moe_synth_normal_bf16")
    return out


def normal_f32(seed: int, tensor_id: int, n: int, sigma: float) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    check(_lib.load().m1moe_synth_normal_f32(ctypes.c_uint64(seed), ctypes.c_uint64(tensor_id),
                                             ctypes.c_uint64(n), ctypes.c_float(sigma),
                                             ctypes.c_void_p(out.ctypes.data)),
          "m1moe_synth_normal_f32")
    return out


def router(shape: MoEShape, seed: int, layer: int) -> np.ndarray:
    """bf16 router [E x h] as uint16."""
    n = shape.num_experts * shape.hidden
    return normal_bf16(seed, _TID_ROUTER | layer, n, ROUTER_SIGMA).reshape(shape.num_experts,
                                                                           shape.hidden)


def activations_bf16(shape: MoEShape, seed: int, T: int, stream: int = 0) -> np.ndarray:
    """x bf16 N(0,1) [T x h] as uint16."""
    return normal_bf16(seed, _TID_X | stream, T * shape.hidden, 1.0).reshape(T, shape.hidden)


def residual_f32(shape: MoEShape, seed: int, T: int, stream: int = 0) -> np.ndarray:
    return normal_f32(seed, _TID_RESIDUAL | stream, T * shape.hidden, 1.0).reshape(T, shape.hidden)


def zipf_logit_bias(num_experts: int, s: float) -> Optional[np.ndarray]:
    """Per-expert logit bias -s*ln(rank) (rank = expert index + 1): with the
    router's own logits added, expert loads follow roughly a Zipf(s) law."""
    if s <= 0:
        return None
    ranks = np.arange(1, num_experts + 1, dtype=np.float64)
    return (-s * np.log(ranks)).astype(np.float32)


_TID_DENSE = 5 << 56
NORM_SIGMA = 0.1       # norm weights bf16 1 + N(0, 0.1)


def dense_weight(wl: DecoderWorkload, seed: int, which: int, layer: int) -> np.ndarray:
    """Dense tensor `which` (m1moe_amd._lib.W_*) of `layer` as bf16 bits, shaped
    [rows, cols] for matrices.  Embedding N(0, 1); projections and lm_head
    N(0, 1/sqrt(cols)), so every projection keeps unit-RMS inputs at unit
    scale; norm weights 1 + N(0, 0.1)."""
    from . import _lib as L
    h = wl.moe.shape_kwargs["hidden"]
    qd, kvd, hd = wl.num_heads * wl.head_dim, wl.num_kv_heads * wl.head_dim, wl.head_dim
    dims = {L.W_EMBED: (wl.vocab, h), L.W_LM_HEAD: (wl.vocab, h), L.W_FINAL_NORM: (h,),
            L.W_IN_NORM: (h,), L.W_POST_NORM: (h,), L.W_Q: (qd, h), L.W_K: (kvd, h),
            L.W_V: (kvd, h), L.W_O: (h, qd), L.W_Q_NORM: (hd,), L.W_K_NORM: (hd,)}[which]
    n = int(np.prod(dims))
    tid = _TID_DENSE | (which << 32) | (layer if which in L.W_PER_LAYER else 0)
    if len(dims) == 1:
        return f32_to_bf16(normal_f32(seed, tid, n, NORM_SIGMA) + np.float32(1.0))
    sigma = 1.0 if which == L.W_EMBED else 1.0 / float(np.sqrt(dims[1]))
    return normal_bf16(seed, tid, n, sigma).reshape(dims)


def prompt_tokens(wl: DecoderWorkload, seed: int, n: Optional[int] = None) -> np.ndarray:
    """n (default wl.prompt) token ids uniform in [0, vocab), int32."""
    rng = np.random.Generator(np.random.PCG64(seed))
    return rng.integers(0, wl.vocab, size=int(n or wl.prompt), dtype=np.int64).astype(np.int32)


def write_model_dir(wl: DecoderWorkload, seed: int, path: str, num_layers: Optional[int] = None,
                    architecture: str = "olmoe") -> dict:
    """Writes a converted model directory of the seeded synthetic model in the
    format scripts/extract_olmoe.py produces (:216-266, :268-345):
    model_weights.bin (tensors in sorted-name order, each 4-byte aligned) +
    model_weights.json ({name: {offset, shape, dtype}}) and
    packed_experts/layer_NN.bin.  Norm vectors are written as f32 (the
    converter keeps f32 sources as f32), the q/k norms at their Hugging Face
    length (q_dim / kv_dim) with the first head_dim values the decoder uses,
    the router under the reference's key for `architecture`.  Returns the
    manifest."""
    import json

    from . import _lib as L
    L_ = int(num_layers or wl.num_layers)
    shape = wl.moe.shape(L_)
    os.makedirs(os.path.join(path, "packed_experts"), exist_ok=True)
    for layer in range(L_):
        layer_image(shape, seed, layer).tofile(
            os.path.join(path, "packed_experts", f"layer_{layer:02d}.bin"))
    qd, kvd, hd = wl.num_heads * wl.head_dim, wl.num_kv_heads * wl.head_dim, wl.head_dim
    tensors = {}

    def as_f32(bits):
        return bf16_to_f32(bits)

    tensors["model.embed_tokens.weight"] = dense_weight(wl, seed, L.W_EMBED, 0)
    tensors["lm_head.weight"] = dense_weight(wl, seed, L.W_LM_HEAD, 0)
    tensors["model.norm.weight"] = as_f32(dense_weight(wl, seed, L.W_FINAL_NORM, 0))
    gate = "block_sparse_moe.gate" if architecture == "mixtral" else "mlp.gate"
    for layer in range(L_):
        pre = f"model.layers.{layer}."
        tensors[pre + "input_layernorm.weight"] = as_f32(dense_weight(wl, seed, L.W_IN_NORM, layer))
        tensors[pre + "post_attention_layernorm.weight"] = as_f32(
            dense_weight(wl, seed, L.W_POST_NORM, layer))
        tensors[pre + "self_attn.q_proj.weight"] = dense_weight(wl, seed, L.W_Q, layer)
        tensors[pre + "self_attn.k_proj.weight"] = dense_weight(wl, seed, L.W_K, layer)
        tensors[pre + "self_attn.v_proj.weight"] = dense_weight(wl, seed, L.W_V, layer)
        tensors[pre + "self_attn.o_proj.weight"] = dense_weight(wl, seed, L.W_O, layer)
        if wl.qk_norm:
            for which, n, name in ((L.W_Q_NORM, qd, "q_norm"), (L.W_K_NORM, kvd, "k_norm")):
                full = np.concatenate([dense_weight(wl, seed, which, layer),
                                       f32_to_bf16(normal_f32(seed, _TID_DENSE | (which << 32) |
                                                              (1 << 31) | layer, n - hd, 0.1) + 1)])
                tensors[pre + "self_attn." + name + ".weight"] = as_f32(full)
        tensors[pre + gate + ".weight"] = router(shape, seed, layer)
    manifest, offset = {}, 0
    with open(os.path.join(path, "model_weights.bin"), "wb") as f:
        for name in sorted(tensors):
            arr = tensors[name]
            dtype = "bf16" if arr.dtype == np.uint16 else "f32"
            if offset % 4:
                f.write(b"\x00" * (4 - offset % 4))
                offset += 4 - offset % 4
            manifest[name] = {"offset": offset, "shape": list(arr.shape), "dtype": dtype}
            raw = np.ascontiguousarray(arr).tobytes()
            f.write(raw)
            offset += len(raw)
    with open(os.path.join(path, "model_weights.json"), "w") as f:
        json.dump(manifest, f, indent=2)
    return manifest


def bf16_to_f32(a: np.ndarray) -> np.ndarray:
    """Exact bf16 (uint16 bits) -> f32."""
    return (np.asarray(a, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(a: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even f32 -> bf16 bits (scripts/extract_olmoe.py:104-111)."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = u + 0x7FFF + ((u >> 16) & 1)
    return (u >> 16).astype(np.uint16)
