"""The C ABI library without a GPU: it loads, exports every declared
symbol, and validates arguments on the host.  CPU only (no compute calls)."""
import ctypes
import os
import re
import subprocess

import numpy as np
import pytest

import m1moe_amd as m
from m1moe_amd import _lib
from m1moe_amd.engine import expert_bytes, expert_offsets, make_shape

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "m1moe_hip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(m1moe_[a-z0-9_]+)\s*\(", text)))


def test_every_declared_symbol_is_exported_and_bound():
    names = declared_functions()
    assert len(names) >= 30
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\bT (m1moe_\w+)", out))
    missing = [n for n in names if n not in exported]
    assert not missing, missing
    assert sorted(_lib.EXPORTED_NAMES) == names
    lib = _lib.load()
    for n in names:
        assert getattr(lib, n) is not None


def test_swift_binding_names_only_declared_symbols():
    """The uncompiled SwiftPM binding and the Swift check executable (no
    Swift toolchain here) call only functions and constants the header
    declares, and the binding links the library's own name."""
    sw = os.path.join(ROOT, "Sources")
    mm = open(os.path.join(sw, "CM1MoEHIP", "module.modulemap")).read()
    assert 'link "m1moe_hip"' in mm and 'header "shim.h"' in mm
    assert os.path.basename(_lib.LIB_PATH) == "libm1moe_hip.so"
    assert "#include <m1moe_hip.h>" in open(os.path.join(sw, "CM1MoEHIP", "shim.h")).read()
    swift = "".join(re.sub(r"//[^\n]*", "", open(os.path.join(sw, *f)).read())
                    for f in (("M1MoE", "HIPMoE.swift"), ("hipcheck", "main.swift")))
    header = open(HEADER).read()
    calls = set(re.findall(r"\b(m1moe_[a-z0-9_]+)\s*\(", swift))
    calls -= {"m1moe_moe_shape", "m1moe_dec_shape"}     # struct initialisers, checked below
    assert calls and calls <= set(declared_functions()), calls - set(declared_functions())
    for c in set(re.findall(r"\b(M1MOE_[A-Z0-9_]+)\b", swift)):
        assert re.search(r"\b%s\s*=" % c, header), c
    for t in set(re.findall(r"\b(m1moe_[a-z_]+_t|m1moe_[a-z_]+_shape)\b", swift)):
        assert re.search(r"\b%s;" % t, header), t


def _gfx950_code_objects(so_path):
    """The gfx950 code objects embedded in a library built here (the
    .hip_fatbin section holds one clang offload bundle per .hip file)."""
    import struct
    data = subprocess.run(["objcopy", "-O", "binary", "--only-section=.hip_fatbin", so_path,
                           "/dev/stdout"], capture_output=True, check=True).stdout
    magic = b"__CLANG_OFFLOAD_BUNDLE__"
    out = []
    for m in re.finditer(re.escape(magic), data):
        p = m.start()
        (n,) = struct.unpack_from("<Q", data, p + len(magic))
        q = p + len(magic) + 8
        for _ in range(n):
            off, size, tl = struct.unpack_from("<QQQ", data, q)
            triple = data[q + 24:q + 24 + tl].decode()
            q += 24 + tl
            if triple.endswith("gfx950"):
                out.append(data[p + off:p + off + size])
    return out


def test_device_code_has_no_packed_fp32(tmp_path):
    """Packed-FP32 VALU instructions are disabled for every device pass."""
    objdump = "/opt/rocm/lib/llvm/bin/llvm-objdump"
    if not os.path.exists(objdump):
        pytest.skip("llvm-objdump not installed")
    cos = _gfx950_code_objects(_lib.LIB_PATH)
    assert len(cos) >= 7
    for i, co in enumerate(cos):
        f = tmp_path / f"co{i}.o"
        f.write_bytes(co)
        dis = subprocess.run([objdump, "-d", str(f)], capture_output=True, text=True,
                             check=True).stdout
        assert dis.count("\n") > 0
        assert not re.search(r"\bv_pk_(fma|mul|add)_f32\b", dis), f"code object {i}"


def test_abi_version():
    assert _lib.load().m1moe_abi_version() == 1


def test_no_oracle_linkage():
    out = subprocess.run(["ldd", _lib.LIB_PATH], capture_output=True, text=True).stdout
    assert "oracle" not in out
    dyn = subprocess.run(["nm", "-D", _lib.LIB_PATH], capture_output=True, text=True).stdout
    assert "orc_" not in dyn


@pytest.mark.parametrize("kw,frag", [
    (dict(hidden=2000), "hidden"),
    (dict(hidden=0), "hidden"),
    (dict(intermediate=96), "intermediate"),
    (dict(group_size=48), "group_size"),
    (dict(group_size=128, hidden=192), "group_size"),
    (dict(num_experts=0), "num_experts"),
    (dict(num_experts=300), "num_experts"),
    (dict(top_k=9, num_experts=8), "top_k"),
    (dict(top_k=0), "top_k"),
    (dict(num_layers=0), "num_layers"),
    (dict(norm_topk_prob=2), "norm_topk_prob"),
])
def test_shape_validation(kw, frag):
    base = dict(hidden=2048, num_experts=64, top_k=8, intermediate=1024, group_size=64,
                num_layers=1, norm_topk_prob=0)
    base.update(kw)
    s = _lib.MoEShape(base["hidden"], base["num_experts"], base["top_k"], base["intermediate"],
                      base["group_size"], base["num_layers"], base["norm_topk_prob"])
    rc = _lib.load().m1moe_check_shape(ctypes.byref(s))
    assert rc == _lib.M1MOE_ERR_INVALID
    assert frag in _lib.last_error()


def test_valid_shapes_and_expert_bytes():
    olmoe = make_shape(2048, 64, 8, 1024, 64)
    mixtral = make_shape(4096, 8, 2, 14336, 64, norm_topk_prob=True)
    m.check_shape(olmoe)
    m.check_shape(mixtral)
    assert expert_bytes(olmoe) == 3538944
    assert expert_bytes(mixtral) == 99090432
    off = expert_offsets(olmoe)
    assert off == [0, 1048576, 1114112, 1179648, 2228224, 2293760, 2359296, 3407872, 3473408]


def test_null_context_is_rejected_everywhere():
    lib = _lib.load()
    buf = np.zeros(16, np.float32)
    p = ctypes.c_void_p(buf.ctypes.data)
    calls = [
        lambda: lib.m1moe_upload_layer_experts(None, 0, p, 64),
        lambda: lib.m1moe_upload_router(None, 0, None, 0),
        lambda: lib.m1moe_moe_decode(None, 0, p, 0, None, p, None, None),
        lambda: lib.m1moe_moe_decode_given_topk(None, 0, p, 0, p, p, None, p),
        lambda: lib.m1moe_moe_prefill(None, 0, 1, p, 0, None, p, None, None),
        lambda: lib.m1moe_router_topk(None, 0, 1, p, 0, p, p, None),
        lambda: lib.m1moe_dequant_debug(None, 0, 0, 0, p),
        lambda: lib.m1moe_sync(None),
        lambda: lib.m1moe_alloc(None, 16, ctypes.byref(ctypes.c_void_p())),
        lambda: lib.m1moe_graph_begin(None),
    ]
    for c in calls:
        assert c() == _lib.M1MOE_ERR_INVALID
        assert "null context" in _lib.last_error()
    lib.m1moe_destroy(None)  # no-op


def test_synth_layer_image_rejects_wrong_size():
    s = make_shape(128, 8, 2, 64, 64)
    buf = np.zeros(10, np.uint8)
    rc = _lib.load().m1moe_synth_layer_image(ctypes.byref(s), 1, 0, ctypes.c_float(0.02),
                                             ctypes.c_float(0.01), ctypes.c_void_p(buf.ctypes.data),
                                             10, 1)
    assert rc == _lib.M1MOE_ERR_INVALID
    assert "layer image is" in _lib.last_error()


def test_error_raises_with_message():
    with pytest.raises(m.M1MoEError) as ei:
        m.check_shape(make_shape(100, 8, 2, 64, 64))
    assert ei.value.code == _lib.M1MOE_ERR_INVALID
    assert "hidden=100" in str(ei.value)


def test_modelspec_loads_reference_config_format(tmp_path):
    cfg = {
        "name": "OLMoE-1B-7B-0924", "architecture": "olmoe", "hidden_dim": 2048,
        "vocab_size": 50304, "num_layers": 16, "rms_norm_eps": 1e-5,
        "attention": {"num_heads": 16, "num_kv_heads": 16, "head_dim": 128,
                      "rope_theta": 10000.0, "max_seq_len": 4096, "gpu_kv_seq_prealloc": 4096},
        "moe": {"num_experts": 64, "top_k": 8, "intermediate_dim": 1024,
                "norm_topk_prob": False},
        "quantization": {"bits": 4, "group_size": 64},
        "special_tokens": {"eos": [50279], "bos": 1},
        "runtime": {"expert_window_size": 1024, "io_threads": 8},
    }
    import json
    p = tmp_path / "olmoe.json"
    p.write_text(json.dumps(cfg))
    spec = m.ModelSpec.load(str(p))
    assert spec.expert_bytes_4bit == 3538944
    sh = spec.shape()
    assert (sh.hidden, sh.num_experts, sh.top_k, sh.intermediate, sh.group_size,
            sh.num_layers, sh.norm_topk_prob) == (2048, 64, 8, 1024, 64, 16, 0)


@pytest.mark.parametrize("shape,cus,blocks,want", [
    (make_shape(2048, 64, 8, 1024, 64), 256, 1, "moe_decode_cu_kernel"),
    (make_shape(2048, 64, 8, 1024, 64), 255, 1, "moe_decode_kernel"),   # one workgroup unplaced
    (make_shape(2048, 64, 8, 1024, 64), 128, 2, "moe_decode_cu_kernel"),
    (make_shape(2048, 64, 8, 1024, 64), 256, 0, "moe_decode_kernel"),   # does not fit a CU
    (make_shape(2048, 64, 8, 1024, 64), 32, 1, "moe_decode_kernel"),    # a 32-CU partition
    (make_shape(4096, 8, 2, 14336, 64, norm_topk_prob=True), 256, 1, "moe_decode_cuw_kernel"),
    (make_shape(4096, 8, 2, 14336, 64, norm_topk_prob=True), 240, 1, "moe_decode_kernel"),
    (make_shape(128, 8, 2, 64, 64), 256, 1, "moe_decode_kernel"),       # shape outside both
    (make_shape(2048, 64, 8, 1024, 128), 256, 1, "moe_decode_cu_kernel"),
])
def test_decode_kernel_choice(shape, cus, blocks, want):
    """The per-CU decode kernels wait for all 256 of their workgroups, so the
    library picks them only when the device holds all 256 at once."""
    from m1moe_amd.engine import decode_kernel_for
    assert decode_kernel_for(shape, cus, blocks) == want


def test_decode_kernel_choice_rejects_bad_arguments():
    lib = _lib.load()
    k = ctypes.c_int32()
    s = make_shape(2048, 64, 8, 1024, 64)
    assert lib.m1moe_decode_kernel_for(ctypes.byref(s), -1, 1, ctypes.byref(k)) == \
        _lib.M1MOE_ERR_INVALID
    assert lib.m1moe_decode_kernel_for(ctypes.byref(s), 256, 1, None) == _lib.M1MOE_ERR_INVALID
    bad = make_shape(100, 8, 2, 64, 64)
    assert lib.m1moe_decode_kernel_for(ctypes.byref(bad), 256, 1, ctypes.byref(k)) == \
        _lib.M1MOE_ERR_INVALID
