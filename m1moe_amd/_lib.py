"""ctypes binding of libm1moe_hip.so (the C ABI declared in include/m1moe_hip.h).

The library is built in-tree (``make -C m1moe_amd/csrc``) and loaded from
this package directory only.  There is no fallback: if the shared library is
missing, importing the binding raises, so a GPU run can never silently take
another code path.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_char_p, c_float, c_int32, c_uint16, c_uint64, c_void_p

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libm1moe_hip.so")

M1MOE_OK = 0
M1MOE_ERR_INVALID = 1
M1MOE_ERR_HIP = 2
M1MOE_ERR_OOM = 3
M1MOE_ERR_DEVICE = 4

M1MOE_F32 = 0
M1MOE_BF16 = 1

PROJ_GATE, PROJ_UP, PROJ_DOWN = 0, 1, 2


class MoEShape(ctypes.Structure):
    """m1moe_moe_shape: ModelSpec.hiddenDim/numLayers + MoESpec + QuantSpec.groupSize."""

    _fields_ = [
        ("hidden", c_int32),
        ("num_experts", c_int32),
        ("top_k", c_int32),
        ("intermediate", c_int32),
        ("group_size", c_int32),
        ("num_layers", c_int32),
        ("norm_topk_prob", c_int32),
    ]


class DecShape(ctypes.Structure):
    """m1moe_dec_shape: ModelSpec.vocabSize/rmsNormEps + AttentionSpec (ModelSpec.swift:19-22,
    62-75); qk_norm = the OLMoE per-head q/k RMSNorm (InferenceEngine.swift:55)."""

    _fields_ = [
        ("vocab", c_int32),
        ("num_heads", c_int32),
        ("num_kv_heads", c_int32),
        ("head_dim", c_int32),
        ("max_seq", c_int32),
        ("qk_norm", c_int32),
        ("rope_theta", c_float),
        ("rms_eps", c_float),
    ]


# dtypes of the on-disk manifest (m1moe_store_tensor)
DT_BF16, DT_F32, DT_U32 = 0, 1, 2

# dense tensor ids of m1moe_dec_upload
(W_EMBED, W_LM_HEAD, W_FINAL_NORM, W_IN_NORM, W_POST_NORM, W_Q, W_K, W_V, W_O, W_Q_NORM,
 W_K_NORM) = range(11)
W_PER_LAYER = (W_IN_NORM, W_POST_NORM, W_Q, W_K, W_V, W_O, W_Q_NORM, W_K_NORM)


class M1MoEError(RuntimeError):
    """A non-zero status from the C ABI, with m1moe_last_error()'s message."""

    def __init__(self, code: int, where: str, message: str):
        super().__init__(f"{where} -> status {code}: {message}")
        self.code = code
        self.where = where
        self.message = message


# (name, restype, argtypes) of every exported function of include/m1moe_hip.h
_PROTOTYPES = [
    ("m1moe_abi_version", c_int32, []),
    ("m1moe_last_error", c_char_p, []),
    ("m1moe_check_shape", c_int32, [POINTER(MoEShape)]),
    ("m1moe_expert_bytes", c_int32, [POINTER(MoEShape), POINTER(c_uint64)]),
    ("m1moe_expert_offsets", c_int32, [POINTER(MoEShape), POINTER(c_uint64)]),
    ("m1moe_decode_kernel_for", c_int32, [POINTER(MoEShape), c_int32, c_int32, POINTER(c_int32)]),
    ("m1moe_create", c_int32, [c_int32, POINTER(MoEShape), POINTER(c_void_p)]),
    ("m1moe_destroy", None, [c_void_p]),
    ("m1moe_upload_layer_experts", c_int32, [c_void_p, c_int32, c_void_p, c_uint64]),
    ("m1moe_upload_router", c_int32, [c_void_p, c_int32, POINTER(c_uint16), c_uint64]),
    ("m1moe_set_logit_bias", c_int32, [c_void_p, c_int32, POINTER(c_float), c_int32]),
    ("m1moe_expert_block", c_int32, [c_void_p, c_int32, c_int32, POINTER(c_void_p)]),
    ("m1moe_alloc", c_int32, [c_void_p, c_uint64, POINTER(c_void_p)]),
    ("m1moe_free", c_int32, [c_void_p, c_void_p]),
    ("m1moe_copy_h2d", c_int32, [c_void_p, c_void_p, c_void_p, c_uint64]),
    ("m1moe_copy_d2h", c_int32, [c_void_p, c_void_p, c_void_p, c_uint64]),
    ("m1moe_copy_d2d", c_int32, [c_void_p, c_void_p, c_void_p, c_uint64]),
    ("m1moe_set_stream", c_int32, [c_void_p, c_void_p]),
    ("m1moe_get_stream", c_int32, [c_void_p, POINTER(c_void_p)]),
    ("m1moe_sync", c_int32, [c_void_p]),
    ("m1moe_event_create", c_int32, [c_void_p, POINTER(c_void_p)]),
    ("m1moe_event_record", c_int32, [c_void_p, c_void_p]),
    ("m1moe_event_elapsed_ms", c_int32, [c_void_p, c_void_p, POINTER(c_float)]),
    ("m1moe_event_destroy", None, [c_void_p]),
    ("m1moe_graph_begin", c_int32, [c_void_p]),
    ("m1moe_graph_end", c_int32, [c_void_p, POINTER(c_void_p)]),
    ("m1moe_graph_launch", c_int32, [c_void_p, c_void_p]),
    ("m1moe_graph_destroy", None, [c_void_p]),
    ("m1moe_router_topk", c_int32,
     [c_void_p, c_int32, c_int32, c_void_p, c_int32, c_void_p, c_void_p, c_void_p]),
    ("m1moe_moe_decode", c_int32,
     [c_void_p, c_int32, c_void_p, c_int32, c_void_p, c_void_p, c_void_p, c_void_p]),
    ("m1moe_moe_decode_given_topk", c_int32,
     [c_void_p, c_int32, c_void_p, c_int32, c_void_p, c_void_p, c_void_p, c_void_p]),
    ("m1moe_moe_prefill", c_int32,
     [c_void_p, c_int32, c_int32, c_void_p, c_int32, c_void_p, c_void_p, c_void_p, c_void_p]),
    ("m1moe_moe_prefill_noalloc", c_int32,
     [c_void_p, c_int32, c_int32, c_void_p, c_int32, c_void_p, c_void_p, c_void_p, c_void_p]),
    ("m1moe_dequant_debug", c_int32, [c_void_p, c_int32, c_int32, c_int32, c_void_p]),
    ("m1moe_rmsnorm", c_int32, [c_void_p, c_void_p, c_void_p, c_void_p, c_int32, c_float]),
    ("m1moe_matvec_bf16", c_int32,
     [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int32, c_int32]),
    ("m1moe_attention_decode", c_int32,
     [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_int32, c_int32]),
    ("m1moe_argmax", c_int32, [c_void_p, c_void_p, c_int32, c_void_p]),
    ("m1moe_dec_create", c_int32, [c_void_p, POINTER(DecShape), POINTER(c_void_p)]),
    ("m1moe_dec_destroy", None, [c_void_p]),
    ("m1moe_dec_upload", c_int32, [c_void_p, c_int32, c_int32, POINTER(c_uint16), c_uint64]),
    ("m1moe_dec_reset", c_int32, [c_void_p]),
    ("m1moe_dec_step", c_int32, [c_void_p, c_void_p, c_void_p, c_void_p]),
    ("m1moe_dec_step_seq", c_int32, [c_void_p, c_void_p, c_int32, c_int32, c_void_p]),
    ("m1moe_dec_prefill", c_int32, [c_void_p, c_void_p, c_int32, c_void_p, c_void_p]),
    ("m1moe_dec_position", c_int32, [c_void_p, POINTER(c_int32)]),
    ("m1moe_store_open", c_int32, [c_char_p, c_char_p, POINTER(c_void_p)]),
    ("m1moe_store_close", None, [c_void_p]),
    ("m1moe_store_count", c_int32, [c_void_p, POINTER(c_int32)]),
    ("m1moe_store_tensor", c_int32,
     [c_void_p, c_char_p, POINTER(c_void_p), POINTER(c_int32), POINTER(ctypes.c_int64),
      POINTER(c_int32)]),
    ("m1moe_load_model", c_int32, [c_void_p, c_void_p, c_char_p, c_int32]),
    ("m1moe_quantize_4bit", c_int32,
     [c_void_p, ctypes.c_int64, ctypes.c_int64, c_int32, c_void_p, c_void_p, c_void_p, c_int32]),
    ("m1moe_quantize_expert", c_int32,
     [POINTER(MoEShape), c_void_p, c_void_p, c_void_p, c_void_p, c_uint64, c_int32]),
    ("m1moe_f32_to_bf16", c_int32, [c_void_p, c_uint64, c_void_p]),
    ("m1moe_tokenizer_load", c_int32, [c_char_p, POINTER(c_void_p)]),
    ("m1moe_tokenizer_free", None, [c_void_p]),
    ("m1moe_tokenizer_info", c_int32,
     [c_void_p, POINTER(c_int32), POINTER(c_uint64), POINTER(c_uint64)]),
    ("m1moe_tokenizer_encode", c_int32,
     [c_void_p, c_char_p, c_uint64, c_int32, ctypes.c_uint32, c_void_p, c_uint64,
      POINTER(c_uint64)]),
    ("m1moe_tokenizer_decode", c_int32,
     [c_void_p, c_void_p, c_uint64, c_int32, c_void_p, c_uint64, POINTER(c_uint64)]),
    ("m1moe_synth_normal_bf16", c_int32,
     [c_uint64, c_uint64, c_uint64, c_float, c_int32, c_void_p]),
    ("m1moe_synth_normal_f32", c_int32, [c_uint64, c_uint64, c_uint64, c_float, c_void_p]),
    ("m1moe_synth_layer_image", c_int32,
     [POINTER(MoEShape), c_uint64, c_int32, c_float, c_float, c_void_p, c_uint64, c_int32]),
]

EXPORTED_NAMES = [p[0] for p in _PROTOTYPES]

_lib = None


def load() -> ctypes.CDLL:
    """Loads the in-tree library once; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} is missing: build it with `make -C m1moe_amd/csrc` "
            "(or __graft_entry__.build()); there is no fallback implementation")
    lib = ctypes.CDLL(LIB_PATH)
    for name, restype, argtypes in _PROTOTYPES:
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    _lib = lib
    return lib


def last_error() -> str:
    msg = load().m1moe_last_error()
    return msg.decode() if msg else ""


def check(code: int, where: str) -> None:
    """Raises M1MoEError for a non-zero status."""
    if code != M1MOE_OK:
        raise M1MoEError(code, where, last_error())
