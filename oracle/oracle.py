"""ctypes wrapper of the scalar CPU oracle (oracle/liboracle_m1moe.so).

TEST INFRASTRUCTURE ONLY: the checker the HIP path is compared against.
Only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg may
import this module.  The reference arithmetic it restates is cited per
function in m1moe_oracle.c.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from ctypes import POINTER, c_float, c_int32, c_uint16, c_uint32, c_uint8

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle_m1moe.so")

KEY_LOGIT = 0
KEY_PROB = 1


class OrcShape(ctypes.Structure):
    _fields_ = [("hidden", c_int32), ("num_experts", c_int32), ("top_k", c_int32),
                ("intermediate", c_int32), ("group_size", c_int32), ("norm_topk_prob", c_int32)]


class OrcOffsets(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint64) for n in
                ("gate_w", "gate_s", "gate_b", "up_w", "up_s", "up_b", "down_w", "down_s",
                 "down_b", "expert_bytes")]


_lib = None


def build() -> None:
    subprocess.run(["make", "-B", "-C", HERE], check=True, stdout=subprocess.DEVNULL)


def load() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        build()
    lib = ctypes.CDLL(LIB_PATH)
    P = ctypes.c_void_p
    sig = {
        "orc_bf16_to_f32": (c_float, [c_uint16]),
        "orc_expert_offsets": (None, [POINTER(OrcShape), POINTER(OrcOffsets)]),
        "orc_dequant_proj": (None, [POINTER(OrcShape), P, c_int32, P]),
        "orc_matvec4bit": (None, [P, P, P, P, P, c_int32, c_int32, c_int32]),
        "orc_matvec4bit_lanes": (None, [P, P, P, P, P, c_int32, c_int32, c_int32]),
        "orc_set_scalar": (None, [c_int32]),
        "orc_matvec4bit_f64": (None, [P, P, P, P, P, c_int32, c_int32, c_int32]),
        "orc_swiglu": (None, [P, P, P, c_int32]),
        "orc_router_logits": (None, [P, P, c_int32, c_int32, P]),
        "orc_router_logits_seq_f32": (None, [P, P, c_int32, c_int32, P]),
        "orc_softmax": (None, [P, c_int32, P]),
        "orc_select_topk": (None, [P, P, c_int32, c_int32, c_int32, c_int32, P, P]),
        "orc_combine": (None, [P, P, P, P, c_int32, c_int32]),
        "orc_expert_forward": (None, [POINTER(OrcShape), P, P, P]),
        "orc_moe_decode": (c_int32, [POINTER(OrcShape), P, P, P, P, P, P, P, P, P]),
        "orc_moe_decode_given_topk": (c_int32, [POINTER(OrcShape), P, P, P, P, P, P]),
        "orc_moe_prefill": (c_int32, [POINTER(OrcShape), P, P, P, c_int32, P, P, P, P, P,
                                      c_int32]),
        "orc_embed": (None, [P, c_int32, c_int32, P]),
        "orc_rmsnorm": (None, [P, P, P, c_int32, c_float]),
        "orc_matvec_bf16": (None, [P, P, P, P, c_int32, c_int32]),
        "orc_head_rmsnorm": (None, [P, c_int32, c_int32, P, c_float]),
        "orc_rope": (None, [P, c_int32, c_int32, c_float, c_int32]),
        "orc_attention": (c_int32, [P, P, P, P, c_int32, c_int32, c_int32, c_int32, P]),
        "orc_argmax": (c_int32, [P, c_int32]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def _p(a):
    if a is None:
        return None
    if not a.flags["C_CONTIGUOUS"]:
        raise ValueError("oracle inputs must be C-contiguous")
    return ctypes.c_void_p(a.ctypes.data)


def shape(hidden, num_experts, top_k, intermediate, group_size=64, norm_topk_prob=False):
    return OrcShape(hidden, num_experts, top_k, intermediate, group_size,
                    1 if norm_topk_prob else 0)


def from_moe_shape(s) -> OrcShape:
    """From an m1moe_amd MoEShape (or anything with the same field names)."""
    return OrcShape(s.hidden, s.num_experts, s.top_k, s.intermediate, s.group_size,
                    s.norm_topk_prob)


def offsets(s: OrcShape) -> OrcOffsets:
    o = OrcOffsets()
    load().orc_expert_offsets(ctypes.byref(s), ctypes.byref(o))
    return o


def dequant_proj(s: OrcShape, block: np.ndarray, proj: int) -> np.ndarray:
    rows = s.hidden if proj == 2 else s.intermediate
    cols = s.intermediate if proj == 2 else s.hidden
    out = np.empty((rows, cols), dtype=np.float32)
    load().orc_dequant_proj(ctypes.byref(s), _p(block), proj, _p(out))
    return out


def set_scalar(on: bool) -> None:
    """Every matvec4bit (and so every expert, decode and prefill) runs the
    lane-by-lane scalar restatement while on (the benchmark's scalar CPU
    baseline); the same bits either way."""
    load().orc_set_scalar(1 if on else 0)


def matvec4bit(w, sc, bi, x, out_dim, in_dim, gs, lanes=False) -> np.ndarray:
    """Shaders.metal:39-92; lanes=True runs the lane-by-lane restatement
    instead of its eight-lanes-at-a-time form (same bits)."""
    y = np.empty(out_dim, dtype=np.float32)
    fn = load().orc_matvec4bit_lanes if lanes else load().orc_matvec4bit
    fn(_p(w), _p(sc), _p(bi), _p(np.ascontiguousarray(x, np.float32)), _p(y), out_dim, in_dim, gs)
    return y


def matvec4bit_f64(w, sc, bi, x, out_dim, in_dim, gs) -> np.ndarray:
    y = np.empty(out_dim, dtype=np.float64)
    load().orc_matvec4bit_f64(_p(w), _p(sc), _p(bi), _p(np.ascontiguousarray(x, np.float32)),
                              _p(y), out_dim, in_dim, gs)
    return y


def swiglu(g, u) -> np.ndarray:
    g = np.ascontiguousarray(g, np.float32)
    u = np.ascontiguousarray(u, np.float32)
    out = np.empty_like(g)
    load().orc_swiglu(_p(g), _p(u), _p(out), g.size)
    return out


def router_logits(router_bf16, x, seq_f32=False) -> np.ndarray:
    r = np.ascontiguousarray(router_bf16, np.uint16)
    x = np.ascontiguousarray(x, np.float32)
    E, h = r.shape
    out = np.empty(E, dtype=np.float32)
    fn = load().orc_router_logits_seq_f32 if seq_f32 else load().orc_router_logits
    fn(_p(r), _p(x), E, h, _p(out))
    return out


def softmax(logits) -> np.ndarray:
    lg = np.ascontiguousarray(logits, np.float32)
    out = np.empty_like(lg)
    load().orc_softmax(_p(lg), lg.size, _p(out))
    return out


def select_topk(logits, probs, k, norm, key_mode=KEY_LOGIT):
    lg = np.ascontiguousarray(logits, np.float32)
    pr = np.ascontiguousarray(probs, np.float32)
    idx = np.empty(k, dtype=np.int32)
    w = np.empty(k, dtype=np.float32)
    load().orc_select_topk(_p(lg), _p(pr), lg.size, k, 1 if norm else 0, key_mode, _p(idx), _p(w))
    return idx, w


def combine(expert_outs, w, residual) -> np.ndarray:
    eo = np.ascontiguousarray(expert_outs, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    K, h = eo.shape
    out = np.empty(h, dtype=np.float32)
    res = None if residual is None else np.ascontiguousarray(residual, np.float32)
    load().orc_combine(_p(eo), _p(w), _p(res), _p(out), K, h)
    return out


def expert_forward(s: OrcShape, block: np.ndarray, x) -> np.ndarray:
    out = np.empty(s.hidden, dtype=np.float32)
    load().orc_expert_forward(ctypes.byref(s), _p(block), _p(np.ascontiguousarray(x, np.float32)),
                              _p(out))
    return out


def moe_decode(s: OrcShape, image, router_bf16, x, residual=None, logit_bias=None):
    """Returns (out [h], idx [K], w [K], logits [E])."""
    out = np.empty(s.hidden, dtype=np.float32)
    idx = np.empty(s.top_k, dtype=np.int32)
    w = np.empty(s.top_k, dtype=np.float32)
    lg = np.empty(s.num_experts, dtype=np.float32)
    r = np.ascontiguousarray(router_bf16, np.uint16)
    res = None if residual is None else np.ascontiguousarray(residual, np.float32)
    bias = None if logit_bias is None else np.ascontiguousarray(logit_bias, np.float32)
    rc = load().orc_moe_decode(ctypes.byref(s), _p(image), _p(r), _p(bias),
                               _p(np.ascontiguousarray(x, np.float32)), _p(res), _p(out), _p(idx),
                               _p(w), _p(lg))
    if rc:
        raise ValueError(f"orc_moe_decode returned {rc}")
    return out, idx, w, lg


def moe_decode_given_topk(s: OrcShape, image, x, idx, w, residual=None) -> np.ndarray:
    out = np.empty(s.hidden, dtype=np.float32)
    res = None if residual is None else np.ascontiguousarray(residual, np.float32)
    rc = load().orc_moe_decode_given_topk(ctypes.byref(s), _p(image),
                                          _p(np.ascontiguousarray(x, np.float32)),
                                          _p(np.ascontiguousarray(idx, np.int32)),
                                          _p(np.ascontiguousarray(w, np.float32)), _p(res), _p(out))
    if rc:
        raise ValueError(f"orc_moe_decode_given_topk returned {rc}")
    return out


def moe_prefill(s: OrcShape, image, router_bf16, x, residual=None, logit_bias=None, nthreads=1):
    """x [T x h] f32; returns (out [T x h], idx [T x K], w [T x K])."""
    x = np.ascontiguousarray(x, np.float32)
    T = x.shape[0]
    out = np.empty((T, s.hidden), dtype=np.float32)
    idx = np.empty((T, s.top_k), dtype=np.int32)
    w = np.empty((T, s.top_k), dtype=np.float32)
    r = np.ascontiguousarray(router_bf16, np.uint16)
    res = None if residual is None else np.ascontiguousarray(residual, np.float32)
    bias = None if logit_bias is None else np.ascontiguousarray(logit_bias, np.float32)
    rc = load().orc_moe_prefill(ctypes.byref(s), _p(image), _p(r), _p(bias), T, _p(x), _p(res),
                                _p(out), _p(idx), _p(w), int(nthreads))
    if rc:
        raise ValueError(f"orc_moe_prefill returned {rc}")
    return out, idx, w


def proj_arrays(s: OrcShape, block: np.ndarray, proj: int):
    """(words u32 [rows, cols/8], scales u16 [rows, groups], biases u16) views of a block."""
    o = offsets(s)
    rows = s.hidden if proj == 2 else s.intermediate
    cols = s.intermediate if proj == 2 else s.hidden
    base = [(o.gate_w, o.gate_s, o.gate_b), (o.up_w, o.up_s, o.up_b),
            (o.down_w, o.down_s, o.down_b)][proj]
    g = cols // s.group_size
    w = block[base[0]:base[0] + rows * cols // 2].view(np.uint32).reshape(rows, cols // 8)
    sc = block[base[1]:base[1] + rows * g * 2].view(np.uint16).reshape(rows, g)
    bi = block[base[2]:base[2] + rows * g * 2].view(np.uint16).reshape(rows, g)
    return w, sc, bi


# ---- dense decoder step (dense_oracle.c) -------------------------------------------------

def _f32(a):
    return np.ascontiguousarray(a, np.float32)


def _u16(a):
    return np.ascontiguousarray(a, np.uint16)


def embed(table_bf16, token: int) -> np.ndarray:
    t = _u16(table_bf16)
    h = t.shape[-1]
    out = np.empty(h, dtype=np.float32)
    load().orc_embed(_p(t), int(token), h, _p(out))
    return out


def rmsnorm(x, w_bf16, eps: float) -> np.ndarray:
    x = _f32(x)
    out = np.empty_like(x)
    load().orc_rmsnorm(_p(x), _p(_u16(w_bf16)), _p(out), x.size, float(eps))
    return out


def matvec_bf16(w_bf16, x, residual=None) -> np.ndarray:
    w = _u16(w_bf16)
    rows, cols = w.shape
    y = np.empty(rows, dtype=np.float32)
    res = None if residual is None else _f32(residual)
    load().orc_matvec_bf16(_p(w), _p(_f32(x)), _p(res), _p(y), rows, cols)
    return y


def head_rmsnorm(x, num_heads: int, head_dim: int, w_bf16, eps: float) -> np.ndarray:
    out = _f32(x).copy()
    load().orc_head_rmsnorm(_p(out), num_heads, head_dim, _p(_u16(w_bf16)), float(eps))
    return out


def rope(x, num_heads: int, head_dim: int, theta: float, pos: int) -> np.ndarray:
    out = _f32(x).copy()
    load().orc_rope(_p(out), num_heads, head_dim, float(theta), int(pos))
    return out


def attention(q, kcache, vcache, num_heads: int, num_kv_heads: int, head_dim: int,
              seq_len: int) -> np.ndarray:
    """kcache/vcache [>= seq_len x num_kv_heads*head_dim] f32."""
    out = np.empty(num_heads * head_dim, dtype=np.float32)
    scratch = np.empty(max(1, seq_len), dtype=np.float64)
    rc = load().orc_attention(_p(_f32(q)), _p(_f32(kcache)), _p(_f32(vcache)), _p(out),
                              num_heads, num_kv_heads, head_dim, int(seq_len), _p(scratch))
    if rc:
        raise ValueError(f"orc_attention returned {rc}")
    return out


def argmax(x) -> int:
    x = _f32(x)
    return int(load().orc_argmax(_p(x), x.size))


class DecoderOracle:
    """InferenceEngine.forward at temperature 0 (InferenceEngine.swift:125-266)
    composed from the oracle's functions, with an f32 KV cache of max_seq
    positions per layer.

    tensors[name] for name in embed, lm_head, final_norm (model level) and
    tensors[name][layer] for in_norm, post_norm, q, k, v, o, q_norm, k_norm:
    bf16 (uint16) arrays, matrices as [rows x cols].  images[layer] and
    routers[layer]: the MoE block's expert image and bf16 router.

    nthreads > 1 spreads work that is independent in the restated arithmetic
    over threads: the rows of a large matvec, the selected experts of a MoE
    block, and the tokens of a prompt in prefill().  Every value is computed
    by the same functions on the same operands as with one thread, so the
    results are the same bits."""

    def __init__(self, moe: OrcShape, num_layers: int, vocab: int, num_heads: int,
                 num_kv_heads: int, head_dim: int, max_seq: int, qk_norm: bool,
                 rope_theta: float, eps: float, tensors: dict, images, routers,
                 nthreads: int = 1):
        self.moe, self.L = moe, num_layers
        self.vocab, self.nh, self.nkv, self.hd = vocab, num_heads, num_kv_heads, head_dim
        self.max_seq, self.qk_norm = max_seq, bool(qk_norm)
        self.theta, self.eps = float(rope_theta), float(eps)
        self.t, self.images, self.routers = tensors, images, routers
        kvd = num_kv_heads * head_dim
        self.kc = np.zeros((num_layers, max_seq, kvd), dtype=np.float32)
        self.vc = np.zeros((num_layers, max_seq, kvd), dtype=np.float32)
        self.pos = 0
        self.nthreads = max(1, int(nthreads))
        self._pool = None
        self._eb = None
        self.split_min = 1 << 22     # matvecs with fewer weights stay on one thread
        # smallest gap, over the layers of the last step, between the K-th and
        # (K+1)-th router logit: where it is tiny the selected set (and so the
        # step's output) changes under arbitrarily small input perturbations
        self.route_margin = np.inf

    def _map(self, fn, items):
        items = list(items)
        if self.nthreads == 1 or len(items) < 2:
            return [fn(i) for i in items]
        if self._pool is None:
            from concurrent.futures import ThreadPoolExecutor
            self._pool = ThreadPoolExecutor(self.nthreads)
        return list(self._pool.map(fn, items))

    def close(self) -> None:
        if self._pool is not None:
            self._pool.shutdown()
            self._pool = None

    def _matvec(self, w, x, residual=None, par=True) -> np.ndarray:
        """matvec_bf16, its rows split over the threads when it is large."""
        rows = w.shape[0]
        if not par or self.nthreads == 1 or w.size < self.split_min:
            return matvec_bf16(w, x, residual)
        n = self.nthreads
        cuts = [rows * i // n for i in range(n + 1)]
        parts = self._map(lambda i: matvec_bf16(
            w[cuts[i]:cuts[i + 1]], x,
            None if residual is None else residual[cuts[i]:cuts[i + 1]]), range(n))
        return np.concatenate(parts)

    def _moe(self, layer: int, x, residual, par=True):
        """moe_decode, the selected experts run on the threads (the same
        router, top-K, expert_forward and combine as orc_moe_decode)."""
        if not par or self.nthreads == 1:
            out, _, _, lg = moe_decode(self.moe, self.images[layer], self.routers[layer], x,
                                       residual=residual)
            return out, lg
        if self._eb is None:
            self._eb = offsets(self.moe).expert_bytes
        lg = router_logits(self.routers[layer], x)
        idx, w = select_topk(lg, softmax(lg), self.moe.top_k, bool(self.moe.norm_topk_prob))
        img, eb = self.images[layer], self._eb
        outs = self._map(lambda e: expert_forward(self.moe, img[e * eb:(e + 1) * eb], x),
                         [int(e) for e in idx])
        return combine(np.stack(outs), w, residual), lg

    def _note_margin(self, lg) -> float:
        if self.moe.top_k >= self.moe.num_experts:
            return np.inf
        srt = np.sort(lg)[::-1]
        k = self.moe.top_k
        return float(srt[k - 1] - srt[k])

    def reset(self) -> None:
        """InferenceEngine.reset (:159-163)."""
        self.pos = 0
        self.kc[:] = 0
        self.vc[:] = 0

    def _qkv(self, layer: int, res, pos: int, par=True):
        """:181-220: the normed input's q (returned) and k/v (into the cache)."""
        t, nh, nkv, hd = self.t, self.nh, self.nkv, self.hd
        xn = rmsnorm(res, t["in_norm"][layer], self.eps)                        # :181-184
        q = self._matvec(t["q"][layer], xn, par=par)                            # :185-190
        k = self._matvec(t["k"][layer], xn, par=par)
        v = self._matvec(t["v"][layer], xn, par=par)
        if self.qk_norm:                                                        # :199-208
            q = head_rmsnorm(q, nh, hd, t["q_norm"][layer], self.eps)
            k = head_rmsnorm(k, nkv, hd, t["k_norm"][layer], self.eps)
        q = rope(q, nh, hd, self.theta, pos)                                    # :210-213
        k = rope(k, nkv, hd, self.theta, pos)
        self.kc[layer, pos] = k                                                 # :215-220
        self.vc[layer, pos] = v
        return q

    def _after_attention(self, layer: int, res, q, pos: int, par=True):
        """:226-266: attention over positions 0..pos, o_proj + residual, the
        post-attention norm and the MoE block (with its residual).  Returns
        the layer output and the router's K-th/(K+1)-th logit gap."""
        t = self.t
        a = attention(q, self.kc[layer], self.vc[layer], self.nh, self.nkv, self.hd, pos + 1)
        res2 = self._matvec(t["o"][layer], a, residual=res, par=par)            # :227-233
        hmid = rmsnorm(res2, t["post_norm"][layer], self.eps)                   # :234-236
        out, lg = self._moe(layer, hmid, res2, par=par)                         # :240-266
        return out, self._note_margin(lg)

    def _logits(self, res):
        xn = rmsnorm(res, self.t["final_norm"], self.eps)                       # :142-144
        logits = self._matvec(self.t["lm_head"], xn)                            # :145-147
        return argmax(logits), logits                                           # :151-155

    def step(self, token: int):
        """One forward step; returns (greedy next token, logits f32 [vocab])."""
        if self.pos >= self.max_seq:
            raise ValueError("KV cache full")
        pos = self.pos
        res = embed(self.t["embed"], token)                                     # :129-131
        self.route_margin = np.inf
        for layer in range(self.L):
            q = self._qkv(layer, res, pos)
            res, m = self._after_attention(layer, res, q, pos)
            self.route_margin = min(self.route_margin, m)
        self.pos += 1                                                           # :138
        return self._logits(res)

    def prefill(self, tokens, log=None):
        """The prompt, as len(tokens) step() calls would run it (the
        reference forwards a prompt token by token, Sources/bench/main.swift:
        139-141), but layer by layer with the tokens of a layer on the
        threads: token i's values depend only on the cache rows of tokens
        <= i of the same layer, and all of a layer's rows are written before
        any of its attention runs.  Returns the last token's (greedy next
        token, logits); the KV cache and position end as after the steps, bit
        for bit, and route_margin is the last token's."""
        tokens = [int(t) for t in tokens]
        T, p0 = len(tokens), self.pos
        if T < 1 or p0 + T > self.max_seq:
            raise ValueError("KV cache full")
        res = [embed(self.t["embed"], tok) for tok in tokens]                   # :129-131
        margins = [np.inf] * T
        for layer in range(self.L):
            qs = self._map(lambda i: self._qkv(layer, res[i], p0 + i, par=False), range(T))
            outs = self._map(lambda i: self._after_attention(layer, res[i], qs[i], p0 + i,
                                                             par=False), range(T))
            res = [o for o, _ in outs]
            margins = [min(a, m) for a, (_, m) in zip(margins, outs)]
            if log:
                log(f"  oracle prefill: layer {layer + 1}/{self.L} of {T} tokens done")
        self.route_margin = margins[-1]
        self.pos += T
        return self._logits(res[-1])
