"""Host-side mirror of the reference decoder (InferenceEngine) over the C ABI.

``Decoder.forward(token)`` is InferenceEngine.forward(token:) at temperature
0 (Sources/M1MoE/InferenceEngine.swift:125-156): embed, every layer's
attention and MoE block, final norm, lm_head, greedy token.  The whole step
runs on the GPU (m1moe_dec_step) with the token and the position in device
memory; ``forward`` adds the one host round-trip the reference's API implies
(the token in, the token out).  ``step_device`` is the same step without it,
for graph-captured loops.

The dense building blocks (RMSNorm, bf16 matvec, decode attention, argmax)
are exposed one by one in ``DenseOps`` for tests and for callers that
compose their own layers.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Optional

import numpy as np

from . import _lib
from ._lib import (DecShape, W_EMBED, W_FINAL_NORM, W_IN_NORM, W_K, W_K_NORM, W_LM_HEAD, W_O,
                   W_PER_LAYER, W_POST_NORM, W_Q, W_Q_NORM, W_V, check)
from .engine import DeviceBuffer, HIPContext, _ptr
from .sampling import sample_token

WEIGHT_NAMES = {
    W_EMBED: "model.embed_tokens.weight",
    W_LM_HEAD: "lm_head.weight",
    W_FINAL_NORM: "model.norm.weight",
    W_IN_NORM: "model.layers.{}.input_layernorm.weight",
    W_POST_NORM: "model.layers.{}.post_attention_layernorm.weight",
    W_Q: "model.layers.{}.self_attn.q_proj.weight",
    W_K: "model.layers.{}.self_attn.k_proj.weight",
    W_V: "model.layers.{}.self_attn.v_proj.weight",
    W_O: "model.layers.{}.self_attn.o_proj.weight",
    W_Q_NORM: "model.layers.{}.self_attn.q_norm.weight",
    W_K_NORM: "model.layers.{}.self_attn.k_norm.weight",
}  # InferenceEngine.swift:580-599 (WeightKeys)


@dataclass(frozen=True)
class AttentionSpec:
    """AttentionSpec, ModelSpec.swift:62-75."""

    num_heads: int
    num_kv_heads: int
    head_dim: int
    rope_theta: float
    max_seq_len: int
    gpu_kv_seq_prealloc: int

    @property
    def q_dim(self) -> int:
        return self.num_heads * self.head_dim

    @property
    def kv_dim(self) -> int:
        return self.num_kv_heads * self.head_dim

    @property
    def hpkv(self) -> int:
        return self.num_heads // self.num_kv_heads


@dataclass(frozen=True)
class DecoderSpec:
    """The dense part of ModelSpec (ModelSpec.swift:14-22): vocabulary, norm
    epsilon, attention, and whether the model has per-head q/k RMSNorm (the
    reference sets it for architecture "olmoe", InferenceEngine.swift:55)."""

    architecture: str
    vocab_size: int
    rms_norm_eps: float
    attention: AttentionSpec

    @property
    def qk_norm(self) -> bool:
        return self.architecture == "olmoe"

    @staticmethod
    def from_dict(d: dict) -> "DecoderSpec":
        a = d["attention"]
        return DecoderSpec(
            architecture=str(d.get("architecture", "")),
            vocab_size=int(d["vocab_size"]),
            rms_norm_eps=float(d["rms_norm_eps"]),
            attention=AttentionSpec(int(a["num_heads"]), int(a["num_kv_heads"]),
                                    int(a["head_dim"]), float(a["rope_theta"]),
                                    int(a["max_seq_len"]), int(a["gpu_kv_seq_prealloc"])))

    def dec_shape(self, max_seq: Optional[int] = None) -> DecShape:
        """KV cache of gpu_kv_seq_prealloc positions unless max_seq is given
        (MetalContext preallocates that many, InferenceEngine.swift:353)."""
        a = self.attention
        return DecShape(self.vocab_size, a.num_heads, a.num_kv_heads, a.head_dim,
                        int(max_seq if max_seq is not None else a.gpu_kv_seq_prealloc),
                        1 if self.qk_norm else 0, a.rope_theta, self.rms_norm_eps)


def weight_count(which: int, hidden: int, s: DecShape) -> int:
    """Element count of dense tensor `which` (include/m1moe_hip.h, M1MOE_W_*)."""
    qd, kvd = s.num_heads * s.head_dim, s.num_kv_heads * s.head_dim
    return {W_EMBED: s.vocab * hidden, W_LM_HEAD: s.vocab * hidden, W_FINAL_NORM: hidden,
            W_IN_NORM: hidden, W_POST_NORM: hidden, W_Q: qd * hidden, W_K: kvd * hidden,
            W_V: kvd * hidden, W_O: hidden * qd, W_Q_NORM: s.head_dim,
            W_K_NORM: s.head_dim}[which]


class DenseOps:
    """The dense kernels one by one (asynchronous on the context stream)."""

    def __init__(self, ctx: HIPContext):
        self.ctx = ctx
        self.lib = ctx.lib

    def rmsnorm(self, x, w, out, n: int, eps: float) -> None:
        check(self.lib.m1moe_rmsnorm(self.ctx.handle, _ptr(x), _ptr(w), _ptr(out), int(n),
                                     ctypes.c_float(eps)), "m1moe_rmsnorm")

    def matvec_bf16(self, w, x, residual, y, rows: int, cols: int) -> None:
        check(self.lib.m1moe_matvec_bf16(self.ctx.handle, _ptr(w), _ptr(x), _ptr(residual),
                                         _ptr(y), int(rows), int(cols)), "m1moe_matvec_bf16")

    def attention_decode(self, q, kcache, vcache, out, num_heads: int, num_kv_heads: int,
                         head_dim: int, seq_len: int) -> None:
        check(self.lib.m1moe_attention_decode(self.ctx.handle, _ptr(q), _ptr(kcache),
                                              _ptr(vcache), _ptr(out), int(num_heads),
                                              int(num_kv_heads), int(head_dim), int(seq_len)),
              "m1moe_attention_decode")

    def argmax(self, x, n: int, idx) -> None:
        check(self.lib.m1moe_argmax(self.ctx.handle, _ptr(x), int(n), _ptr(idx)), "m1moe_argmax")


class Decoder:
    """InferenceEngine (InferenceEngine.swift:19-156) over a HIPContext that
    holds the MoE layers: dense weights resident in HBM, f32 KV cache of
    max_seq positions per layer."""

    def __init__(self, ctx: HIPContext, shape: DecShape):
        self.ctx = ctx
        self.lib = ctx.lib
        self.shape = shape
        self.hidden = ctx.shape.hidden
        self.num_layers = ctx.shape.num_layers
        h = ctypes.c_void_p()
        check(self.lib.m1moe_dec_create(ctx.handle, ctypes.byref(shape), ctypes.byref(h)),
              "m1moe_dec_create")
        self.handle = h
        self._tok = ctx.alloc(16)     # token in/out of forward()
        self._logits = ctx.alloc(4 * shape.vocab)

    def close(self) -> None:
        if self.handle:
            self.lib.m1moe_dec_destroy(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def upload(self, which: int, layer: int, bf16: np.ndarray) -> None:
        a = np.ascontiguousarray(bf16, dtype=np.uint16).reshape(-1)
        check(self.lib.m1moe_dec_upload(self.handle, int(which), int(layer),
                                        a.ctypes.data_as(ctypes.POINTER(ctypes.c_uint16)),
                                        ctypes.c_uint64(a.size)), "m1moe_dec_upload")

    def upload_all(self, weights) -> None:
        """weights(which, layer) -> bf16 array, for every tensor of the model."""
        for which in range(11):
            if which in (W_Q_NORM, W_K_NORM) and not self.shape.qk_norm:
                continue
            layers = range(self.num_layers) if which in W_PER_LAYER else [0]
            for layer in layers:
                self.upload(which, layer, weights(which, layer))

    def reset(self) -> None:
        """InferenceEngine.reset (InferenceEngine.swift:159-163)."""
        check(self.lib.m1moe_dec_reset(self.handle), "m1moe_dec_reset")

    def position(self) -> int:
        p = ctypes.c_int32()
        check(self.lib.m1moe_dec_position(self.handle, ctypes.byref(p)), "m1moe_dec_position")
        return int(p.value)

    def step_device(self, token_in, token_out, logits=None) -> None:
        """One step with the tokens in device memory (asynchronous)."""
        check(self.lib.m1moe_dec_step(self.handle, _ptr(token_in), _ptr(token_out),
                                      _ptr(logits)), "m1moe_dec_step")

    def step_seq(self, seq, n_prompt: int, seq_cap: int, logits=None) -> None:
        """Sequence-mode step (asynchronous): embeds seq[pos]; past the prompt
        stores the greedy token at seq[pos + 1].  n_prompt + n_gen calls after
        reset() run prompt-then-generate with no host round trip."""
        check(self.lib.m1moe_dec_step_seq(self.handle, _ptr(seq), int(n_prompt), int(seq_cap),
                                          _ptr(logits)), "m1moe_dec_step_seq")

    def prefill_device(self, tokens, T: int, token_out, logits=None) -> None:
        """The T prompt tokens (device int32) through the decoder in one batch
        per layer (asynchronous); token_out receives the greedy next token."""
        check(self.lib.m1moe_dec_prefill(self.handle, _ptr(tokens), int(T), _ptr(token_out),
                                         _ptr(logits)), "m1moe_dec_prefill")

    def prefill(self, prompt, return_logits: bool = False):
        """The prompt at once from the current position; returns the greedy
        token after its last token (and that token's logits when asked)."""
        prompt = np.ascontiguousarray(prompt, dtype=np.int32)
        d = self.ctx.to_device(prompt)
        self.prefill_device(d, prompt.size, self._tok, self._logits)
        self.ctx.sync()
        d.free()
        nxt = int(self._tok.download(np.int32, 1)[0])
        if return_logits:
            return nxt, self._logits.download(np.float32, self.shape.vocab)
        return nxt

    def generate(self, prompt, n_gen: int):
        """Sources/bench/main.swift:136-163 at temperature 0: the prompt
        forwarded token by token, then n_gen greedy steps; returns the
        n_gen + 1 greedy tokens (the prompt's own prediction first)."""
        prompt = np.ascontiguousarray(prompt, dtype=np.int32)
        P, cap = prompt.size, prompt.size + n_gen + 1
        seq = self.ctx.alloc(4 * cap)
        seq.upload(np.concatenate([prompt, np.zeros(cap - P, np.int32)]))
        self.reset()
        for _ in range(P + n_gen):
            self.step_seq(seq, P, cap)
        self.ctx.sync()
        out = seq.download(np.int32)[P:]
        seq.free()
        return out

    def forward(self, token: int, return_logits: bool = False, temperature: float = 0.0,
                top_p: float = 1.0, rng: Optional[np.random.Generator] = None):
        """InferenceEngine.forward(token:temperature:topP:) (:125-156): the next
        token — greedy on the GPU at temperature <= 0, else sampled on the host
        from the step's logits as the reference does (sampling.sample_token) —
        and the f32 logits when asked."""
        self._tok.upload(np.array([token, 0, 0, 0], dtype=np.int32))
        self.step_device(self._tok, self._tok, self._logits)
        self.ctx.sync()
        logits = None
        if temperature > 0:
            logits = self._logits.download(np.float32, self.shape.vocab)
            nxt = sample_token(logits, temperature, top_p, rng=rng)
        else:
            nxt = int(self._tok.download(np.int32, 1)[0])
        if return_logits:
            if logits is None:
                logits = self._logits.download(np.float32, self.shape.vocab)
            return nxt, logits
        return nxt


__all__ = ["AttentionSpec", "DecoderSpec", "DenseOps", "Decoder", "DeviceBuffer",
           "WEIGHT_NAMES", "weight_count"]
