"""The on-disk model format and its reader (m1moe_store_*), on the CPU.

A manifest and a .bin written the way scripts/extract_olmoe.py:216-266 writes
them (sorted names, 4-byte alignment, bf16 / f32 / u32 tensors) are read
back through the library: every tensor's bytes, dtype and shape.  Broken
inputs (missing files, malformed JSON, a tensor past the end of the file, an
unknown dtype) are rejected with a message.
"""
import ctypes
import json
import os

import numpy as np
import pytest

from m1moe_amd import _lib, synth

RNG = np.random.default_rng(5)


def write_store(path, tensors, pad_byte_first=False):
    manifest, offset = {}, 0
    with open(os.path.join(path, "w.bin"), "wb") as f:
        if pad_byte_first:
            f.write(b"\0\0")
            offset = 2
        for name in sorted(tensors):
            arr = tensors[name]
            dtype = {np.dtype(np.uint16): "bf16", np.dtype(np.float32): "f32",
                     np.dtype(np.uint32): "u32"}[arr.dtype]
            if offset % 4:
                f.write(b"\0" * (4 - offset % 4))
                offset += 4 - offset % 4
            manifest[name] = {"offset": offset, "shape": list(arr.shape), "dtype": dtype}
            f.write(arr.tobytes())
            offset += arr.nbytes
    with open(os.path.join(path, "w.json"), "w") as f:
        json.dump(manifest, f, indent=2)
    return manifest


def open_store(path, bin_name="w.bin", json_name="w.json"):
    h = ctypes.c_void_p()
    rc = _lib.load().m1moe_store_open(os.path.join(path, bin_name).encode(),
                                      os.path.join(path, json_name).encode(), ctypes.byref(h))
    return rc, h


def get(h, name):
    data = ctypes.c_void_p()
    dtype = ctypes.c_int32()
    shape = (ctypes.c_int64 * 4)()
    ndim = ctypes.c_int32()
    _lib.check(_lib.load().m1moe_store_tensor(h, name.encode(), ctypes.byref(data), ctypes.byref(dtype),
                                              shape, ctypes.byref(ndim)), "m1moe_store_tensor")
    return data.value, dtype.value, [shape[i] for i in range(ndim.value)]


def test_round_trip_of_every_dtype(tmp_path):
    tensors = {
        "model.embed_tokens.weight": RNG.integers(0, 65535, (37, 24), dtype=np.uint16),
        "model.norm.weight": RNG.normal(0, 1, 24).astype(np.float32),
        "model.layers.0.mlp.gate.weight": RNG.integers(0, 65535, (8, 24), dtype=np.uint16),
        "odd": RNG.integers(0, 65535, 3, dtype=np.uint16),  # 6 bytes: the next is padded
        "packed": RNG.integers(0, 2**32 - 1, (4, 3), dtype=np.uint32),
        "scalar_shape": np.zeros(0, dtype=np.float32),
    }
    manifest = write_store(str(tmp_path), tensors)
    assert manifest["packed"]["offset"] % 4 == 0
    rc, h = open_store(str(tmp_path))
    assert rc == 0, _lib.last_error()
    try:
        n = ctypes.c_int32()
        _lib.check(_lib.load().m1moe_store_count(h, ctypes.byref(n)), "count")
        assert n.value == len(tensors)
        for name, arr in tensors.items():
            ptr, dt, shape = get(h, name)
            assert shape == list(arr.shape)
            assert dt == {"bf16": _lib.DT_BF16, "f32": _lib.DT_F32, "u32": _lib.DT_U32}[manifest[name]["dtype"]]
            got = np.ctypeslib.as_array((ctypes.c_uint8 * arr.nbytes).from_address(ptr)) if arr.nbytes else b""
            assert bytes(got) == arr.tobytes(), name
        with pytest.raises(_lib.M1MoEError, match="not in the manifest"):
            get(h, "missing")
    finally:
        _lib.load().m1moe_store_close(h)


@pytest.mark.parametrize("case,frag", [
    ("no_json", "cannot read"),
    ("no_bin", "cannot open"),
    ("bad_json", "manifest"),
    ("past_end", "past the end"),
    ("bad_dtype", "dtype"),
    ("no_offset", "lacks offset"),
])
def test_broken_stores_are_rejected(tmp_path, case, frag):
    write_store(str(tmp_path), {"a": np.arange(4, dtype=np.float32)})
    j = os.path.join(str(tmp_path), "w.json")
    if case == "no_json":
        os.remove(j)
    elif case == "no_bin":
        os.remove(os.path.join(str(tmp_path), "w.bin"))
    elif case == "bad_json":
        open(j, "w").write('{"a": {"offset": 0, "shape": [4], "dtype": "f32"')
    elif case == "past_end":
        open(j, "w").write('{"a": {"offset": 8, "shape": [4], "dtype": "f32"}}')
    elif case == "bad_dtype":
        open(j, "w").write('{"a": {"offset": 0, "shape": [4], "dtype": "f64"}}')
    elif case == "no_offset":
        open(j, "w").write('{"a": {"shape": [4], "dtype": "f32", "extra": [1, {"x": null}]}}')
    rc, h = open_store(str(tmp_path))
    assert rc == _lib.M1MOE_ERR_INVALID
    assert frag in _lib.last_error()


def test_synthetic_model_dir_matches_the_converter_layout(tmp_path):
    wl = synth.DECODERS["tiny_dec"]
    manifest = synth.write_model_dir(wl, 3, str(tmp_path))
    shape = wl.shape()
    import m1moe_amd as m
    eb = m.expert_bytes(shape)
    for layer in range(wl.num_layers):
        f = os.path.join(str(tmp_path), "packed_experts", f"layer_{layer:02d}.bin")
        assert os.path.getsize(f) == shape.num_experts * eb
        assert np.array_equal(np.fromfile(f, np.uint8), synth.layer_image(shape, 3, layer))
    names = sorted(manifest)
    offs = [manifest[n]["offset"] for n in names]
    assert offs == sorted(offs) and all(o % 4 == 0 for o in offs)
    assert manifest["model.norm.weight"]["dtype"] == "f32"
    assert manifest["model.layers.1.self_attn.q_norm.weight"]["shape"] == [wl.num_heads * wl.head_dim]
    rc, h = open_store(str(tmp_path), "model_weights.bin", "model_weights.json")
    assert rc == 0, _lib.last_error()
    try:
        ptr, dt, shp = get(h, "model.layers.0.mlp.gate.weight")
        assert dt == _lib.DT_BF16 and shp == [shape.num_experts, shape.hidden]
        got = np.ctypeslib.as_array((ctypes.c_uint16 * (shp[0] * shp[1])).from_address(ptr))
        assert np.array_equal(got.reshape(shp), synth.router(shape, 3, 0))
    finally:
        _lib.load().m1moe_store_close(h)
