"""Host-side mirror of the reference engine's MoE block over the C ABI.

Python counterpart of what the Swift engine does around its MoE block
(Sources/M1MoE/InferenceEngine.swift:240-266) once the Metal backend is
replaced: a ``ModelSpec`` read from the reference's JSON config
(ModelSpec.swift:56-61, snake_case keys), a ``HIPContext`` that owns the
resident experts, routers and scratch (in place of MetalContext,
MetalContext.swift:69-185), and ``MoEBlock.forward`` for one token through
one layer's MoE block.  Device memory is managed through the library
(m1moe_alloc/copy); no other GPU runtime is loaded into the process.
"""
from __future__ import annotations

import ctypes
import json
from dataclasses import dataclass
from typing import Optional

import numpy as np

from . import _lib
from ._lib import M1MOE_BF16, M1MOE_F32, MoEShape, check


@dataclass(frozen=True)
class MoESpec:
    """MoESpec, ModelSpec.swift:82-87."""

    num_experts: int
    top_k: int
    intermediate_dim: int
    norm_topk_prob: bool


@dataclass(frozen=True)
class QuantSpec:
    """QuantSpec, ModelSpec.swift:91-94 (only 4-bit is meaningful)."""

    bits: int
    group_size: int


@dataclass(frozen=True)
class ModelSpec:
    """The MoE-relevant part of ModelSpec (ModelSpec.swift:11-52)."""

    name: str
    architecture: str
    hidden_dim: int
    num_layers: int
    moe: MoESpec
    quantization: QuantSpec

    @staticmethod
    def load(path: str) -> "ModelSpec":
        """ModelSpec.load(from:), ModelSpec.swift:56-61 (snake_case JSON)."""
        with open(path, "r", encoding="utf-8") as f:
            d = json.load(f)
        return ModelSpec.from_dict(d)

    @staticmethod
    def from_dict(d: dict) -> "ModelSpec":
        m, q = d["moe"], d["quantization"]
        if int(q["bits"]) != 4:
            raise ValueError(f"quantization.bits={q['bits']}: only 4-bit experts exist")
        return ModelSpec(
            name=str(d.get("name", "")),
            architecture=str(d.get("architecture", "")),
            hidden_dim=int(d["hidden_dim"]),
            num_layers=int(d["num_layers"]),
            moe=MoESpec(int(m["num_experts"]), int(m["top_k"]), int(m["intermediate_dim"]),
                        bool(m["norm_topk_prob"])),
            quantization=QuantSpec(int(q["bits"]), int(q["group_size"])),
        )

    def shape(self, num_layers: Optional[int] = None) -> MoEShape:
        return MoEShape(self.hidden_dim, self.moe.num_experts, self.moe.top_k,
                        self.moe.intermediate_dim, self.quantization.group_size,
                        self.num_layers if num_layers is None else num_layers,
                        1 if self.moe.norm_topk_prob else 0)

    @property
    def expert_bytes_4bit(self) -> int:
        """ModelSpec.expertBytes4Bit, ModelSpec.swift:36-52 (computed by the library)."""
        return expert_bytes(self.shape())


def make_shape(hidden: int, num_experts: int, top_k: int, intermediate: int,
               group_size: int = 64, num_layers: int = 1, norm_topk_prob: bool = False) -> MoEShape:
    return MoEShape(hidden, num_experts, top_k, intermediate, group_size, num_layers,
                    1 if norm_topk_prob else 0)


def expert_bytes(shape: MoEShape) -> int:
    lib = _lib.load()
    out = ctypes.c_uint64()
    check(lib.m1moe_expert_bytes(ctypes.byref(shape), ctypes.byref(out)), "m1moe_expert_bytes")
    return int(out.value)


def expert_offsets(shape: MoEShape) -> list:
    lib = _lib.load()
    out = (ctypes.c_uint64 * 9)()
    check(lib.m1moe_expert_offsets(ctypes.byref(shape), out), "m1moe_expert_offsets")
    return [int(v) for v in out]


DECODE_KERNELS = ("moe_decode_kernel", "moe_decode_cu_kernel", "moe_decode_cuw_kernel")


def decode_kernel_for(shape: MoEShape, cus: int = 256, blocks_per_cu: int = 1) -> str:
    """Name of the decode kernel the library runs for `shape` on a device of
    `cus` CUs each holding `blocks_per_cu` per-CU workgroups
    (m1moe_decode_kernel_for; host only)."""
    k = ctypes.c_int32(-1)
    lib = _lib.load()
    check(lib.m1moe_decode_kernel_for(ctypes.byref(shape), int(cus), int(blocks_per_cu),
                                      ctypes.byref(k)), "m1moe_decode_kernel_for")
    return DECODE_KERNELS[k.value]


def check_shape(shape: MoEShape) -> None:
    check(_lib.load().m1moe_check_shape(ctypes.byref(shape)), "m1moe_check_shape")


def _host_ptr(a: np.ndarray) -> ctypes.c_void_p:
    if not a.flags["C_CONTIGUOUS"]:
        raise ValueError("host arrays passed to the library must be C-contiguous")
    return ctypes.c_void_p(a.ctypes.data)


class DeviceBuffer:
    """A device allocation owned by a HIPContext (m1moe_alloc)."""

    def __init__(self, ctx: "HIPContext", nbytes: int):
        self.ctx = ctx
        self.nbytes = int(nbytes)
        p = ctypes.c_void_p()
        check(ctx.lib.m1moe_alloc(ctx.handle, ctypes.c_uint64(self.nbytes), ctypes.byref(p)),
              "m1moe_alloc")
        self.ptr = p

    @property
    def addr(self) -> int:
        return int(self.ptr.value or 0)

    def upload(self, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        if a.nbytes > self.nbytes:
            raise ValueError(f"{a.nbytes} bytes do not fit a {self.nbytes}-byte buffer")
        check(self.ctx.lib.m1moe_copy_h2d(self.ctx.handle, self.ptr, _host_ptr(a),
                                          ctypes.c_uint64(a.nbytes)), "m1moe_copy_h2d")
        return self

    def download(self, dtype, count: Optional[int] = None) -> np.ndarray:
        dtype = np.dtype(dtype)
        n = self.nbytes // dtype.itemsize if count is None else int(count)
        out = np.empty(n, dtype=dtype)
        check(self.ctx.lib.m1moe_copy_d2h(self.ctx.handle, _host_ptr(out), self.ptr,
                                          ctypes.c_uint64(out.nbytes)), "m1moe_copy_d2h")
        return out

    def free(self) -> None:
        if self.ptr is not None and self.ctx.handle:
            check(self.ctx.lib.m1moe_free(self.ctx.handle, self.ptr), "m1moe_free")
        self.ptr = None


class HIPContext:
    """Owns the device state of the MoE block (replaces MetalContext for it)."""

    def __init__(self, shape: MoEShape, device: int = 0):
        self.lib = _lib.load()
        self.shape = shape
        h = ctypes.c_void_p()
        check(self.lib.m1moe_create(int(device), ctypes.byref(shape), ctypes.byref(h)),
              "m1moe_create")
        self.handle = h
        self.expert_bytes = expert_bytes(shape)

    def close(self) -> None:
        if self.handle:
            self.lib.m1moe_destroy(self.handle)
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

    # ---- uploads ---------------------------------------------------------
    def upload_layer_experts(self, layer: int, image: np.ndarray) -> None:
        image = np.ascontiguousarray(image)
        check(self.lib.m1moe_upload_layer_experts(self.handle, int(layer), _host_ptr(image),
                                                  ctypes.c_uint64(image.nbytes)),
              "m1moe_upload_layer_experts")

    def upload_router(self, layer: int, router_bf16: np.ndarray) -> None:
        r = np.ascontiguousarray(router_bf16, dtype=np.uint16)
        check(self.lib.m1moe_upload_router(
            self.handle, int(layer), r.ctypes.data_as(ctypes.POINTER(ctypes.c_uint16)),
            ctypes.c_uint64(r.size)), "m1moe_upload_router")

    def set_logit_bias(self, layer: int, bias: Optional[np.ndarray]) -> None:
        if bias is None:
            check(self.lib.m1moe_set_logit_bias(self.handle, int(layer), None, 0),
                  "m1moe_set_logit_bias")
            return
        b = np.ascontiguousarray(bias, dtype=np.float32)
        check(self.lib.m1moe_set_logit_bias(
            self.handle, int(layer), b.ctypes.data_as(ctypes.POINTER(ctypes.c_float)),
            int(b.size)), "m1moe_set_logit_bias")

    def load_model(self, model_dir: str, decoder=None, threads: int = 8) -> None:
        """Uploads a converted model directory (model_weights.bin/.json and
        packed_experts/layer_NN.bin, as scripts/extract_olmoe.py writes them):
        every layer's experts and router, and the dense tensors into `decoder`
        (a m1moe_amd.decoder.Decoder) when given."""
        check(self.lib.m1moe_load_model(self.handle, decoder.handle if decoder is not None else None,
                                        model_dir.encode(), int(threads)), "m1moe_load_model")

    # ---- memory ----------------------------------------------------------
    def alloc(self, nbytes: int) -> DeviceBuffer:
        return DeviceBuffer(self, nbytes)

    def to_device(self, a: np.ndarray) -> DeviceBuffer:
        a = np.ascontiguousarray(a)
        return DeviceBuffer(self, a.nbytes).upload(a)

    def sync(self) -> None:
        check(self.lib.m1moe_sync(self.handle), "m1moe_sync")

    # ---- events / graphs ---------------------------------------------------
    def event(self) -> "Event":
        return Event(self)

    def graph_begin(self) -> None:
        check(self.lib.m1moe_graph_begin(self.handle), "m1moe_graph_begin")

    def graph_end(self) -> "Graph":
        g = ctypes.c_void_p()
        check(self.lib.m1moe_graph_end(self.handle, ctypes.byref(g)), "m1moe_graph_end")
        return Graph(self, g)


class Event:
    def __init__(self, ctx: HIPContext):
        self.ctx = ctx
        e = ctypes.c_void_p()
        check(ctx.lib.m1moe_event_create(ctx.handle, ctypes.byref(e)), "m1moe_event_create")
        self.handle = e

    def record(self) -> None:
        check(self.ctx.lib.m1moe_event_record(self.ctx.handle, self.handle), "m1moe_event_record")

    def elapsed_ms(self, end: "Event") -> float:
        ms = ctypes.c_float()
        check(self.ctx.lib.m1moe_event_elapsed_ms(self.handle, end.handle, ctypes.byref(ms)),
              "m1moe_event_elapsed_ms")
        return float(ms.value)

    def __del__(self):
        try:
            self.ctx.lib.m1moe_event_destroy(self.handle)
        except Exception:
            pass


class Graph:
    def __init__(self, ctx: HIPContext, handle: ctypes.c_void_p):
        self.ctx = ctx
        self.handle = handle

    def launch(self) -> None:
        check(self.ctx.lib.m1moe_graph_launch(self.ctx.handle, self.handle), "m1moe_graph_launch")

    def __del__(self):
        try:
            self.ctx.lib.m1moe_graph_destroy(self.handle)
        except Exception:
            pass


def _dtype_code(x_dtype) -> int:
    if x_dtype in ("bf16", M1MOE_BF16):
        return M1MOE_BF16
    if x_dtype in ("f32", M1MOE_F32):
        return M1MOE_F32
    raise ValueError(f"unknown activation dtype {x_dtype!r}")


def _ptr(buf) -> Optional[ctypes.c_void_p]:
    if buf is None:
        return None
    if isinstance(buf, DeviceBuffer):
        return buf.ptr
    return ctypes.c_void_p(int(buf))


class MoEBlock:
    """The MoE block of a decoder layer (InferenceEngine.swift:240-266) on the GPU."""

    def __init__(self, ctx: HIPContext):
        self.ctx = ctx
        self.lib = ctx.lib

    def forward(self, layer: int, x, x_dtype, residual, out, topk_idx=None, topk_w=None) -> None:
        """One token: router, top-K, experts, combine, residual (asynchronous)."""
        check(self.lib.m1moe_moe_decode(self.ctx.handle, int(layer), _ptr(x), _dtype_code(x_dtype),
                                        _ptr(residual), _ptr(out), _ptr(topk_idx), _ptr(topk_w)),
              "m1moe_moe_decode")

    def forward_given_topk(self, layer: int, x, x_dtype, topk_idx, topk_w, residual, out) -> None:
        check(self.lib.m1moe_moe_decode_given_topk(
            self.ctx.handle, int(layer), _ptr(x), _dtype_code(x_dtype), _ptr(topk_idx),
            _ptr(topk_w), _ptr(residual), _ptr(out)), "m1moe_moe_decode_given_topk")

    def router_topk(self, layer: int, T: int, x, x_dtype, topk_idx, topk_w, logits=None) -> None:
        check(self.lib.m1moe_router_topk(self.ctx.handle, int(layer), int(T), _ptr(x),
                                         _dtype_code(x_dtype), _ptr(topk_idx), _ptr(topk_w),
                                         _ptr(logits)), "m1moe_router_topk")

    def prefill(self, layer: int, T: int, x, x_dtype, residual, out, topk_idx=None,
                topk_w=None) -> None:
        check(self.lib.m1moe_moe_prefill(self.ctx.handle, int(layer), int(T), _ptr(x),
                                         _dtype_code(x_dtype), _ptr(residual), _ptr(out),
                                         _ptr(topk_idx), _ptr(topk_w)), "m1moe_moe_prefill")

    def prefill_noalloc(self, layer: int, T: int, x, x_dtype, residual, out, topk_idx=None,
                        topk_w=None) -> None:
        """prefill() on the device's fixed static scratch: allocates nothing,
        T limited by that scratch's 64 MiB (776 tokens at the OLMoE shape,
        676 at the Mixtral shape)."""
        check(self.lib.m1moe_moe_prefill_noalloc(
            self.ctx.handle, int(layer), int(T), _ptr(x), _dtype_code(x_dtype), _ptr(residual),
            _ptr(out), _ptr(topk_idx), _ptr(topk_w)), "m1moe_moe_prefill_noalloc")

    def dequant(self, layer: int, expert: int, proj: int, out) -> None:
        check(self.lib.m1moe_dequant_debug(self.ctx.handle, int(layer), int(expert), int(proj),
                                           _ptr(out)), "m1moe_dequant_debug")
