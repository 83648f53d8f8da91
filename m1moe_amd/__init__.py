"""m1moe_amd — MI355X (gfx950) MoE-layer decode path of koaWood/M1MoE.

The compute lives in libm1moe_hip.so (hand-written HIP kernels behind the C
ABI in include/m1moe_hip.h).  This package is the host-side mirror of the
reference's MoE-block interface over that ABI (engine.py), the decoder
around it (decoder.py: InferenceEngine.forward on the GPU), plus the seeded
synthetic workloads (synth.py).
"""
from ._lib import (M1MOE_BF16, M1MOE_F32, M1MoEError, MoEShape, PROJ_DOWN, PROJ_GATE,
                   PROJ_UP, load)
from .engine import (DeviceBuffer, HIPContext, MoEBlock, ModelSpec, check_shape, expert_bytes,
                     expert_offsets, make_shape)
from .decoder import AttentionSpec, Decoder, DecoderSpec, DenseOps

__all__ = [
    "M1MOE_BF16", "M1MOE_F32", "M1MoEError", "MoEShape", "PROJ_DOWN", "PROJ_GATE", "PROJ_UP",
    "load", "DeviceBuffer", "HIPContext", "MoEBlock", "ModelSpec", "check_shape",
    "expert_bytes", "expert_offsets", "make_shape", "AttentionSpec", "Decoder", "DecoderSpec",
    "DenseOps",
]
