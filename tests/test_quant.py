"""The converters' 4-bit quantizer and the checkpoint converter (CPU only).

The oracle (oracle/quant_oracle.py, a numpy restatement of
scripts/extract_olmoe.py:104-159) is pinned first: known answers where the
quantisation is exact, round-half-even ties, constant groups, bf16 rounding
ties, torch's own f32 -> bf16 conversion and the dequantisation error bound.
Then the library's m1moe_quantize_4bit / m1moe_quantize_expert /
m1moe_f32_to_bf16 must equal it bit for bit, and m1moe_amd.convert must
write the files extract_olmoe.py / extract_mixtral.py would write.
"""
from __future__ import annotations

import json
import struct

import numpy as np
import pytest

from m1moe_amd import _lib
from m1moe_amd._lib import M1MoEError
from m1moe_amd.engine import make_shape
from m1moe_amd import quant
from oracle import quant_oracle as qo


def bf16_bits(x) -> int:
    return int(qo.f32_to_bf16(np.array([x], np.float32))[0])


def bits_to_f32(u) -> np.ndarray:
    return (np.asarray(u, np.uint32) << 16).view(np.float32)


# ---- the oracle, pinned ------------------------------------------------------

def test_oracle_bf16_known_answers():
    f = lambda bits: np.array([bits], np.uint32).view(np.float32)[0]
    assert bf16_bits(1.0) == 0x3F80
    assert bf16_bits(-2.0) == 0xC000
    assert bf16_bits(f(0x3F808000)) == 0x3F80       # tie, even stays
    assert bf16_bits(f(0x3F818000)) == 0x3F82       # tie, odd rounds up
    assert bf16_bits(f(0x3F808001)) == 0x3F81       # above the tie
    assert bf16_bits(f(0x3F807FFF)) == 0x3F80       # below the tie
    assert bf16_bits(f(0x7F7FFFFF)) == 0x7F80       # max finite rounds to inf
    assert bf16_bits(np.inf) == 0x7F80
    assert bf16_bits(0.0) == 0 and bf16_bits(-0.0) == 0x8000


def test_oracle_bf16_matches_torch():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(50000).astype(np.float32) * 10.0 ** rng.integers(-30, 30, 50000),
                        rng.integers(0, 2**31 - 2**23, 50000, dtype=np.uint32).view(np.float32)])
    x = x[np.isfinite(x)].astype(np.float32)
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(qo.f32_to_bf16(x), want)


def test_oracle_exact_groups_give_their_nibbles():
    """w = lo + q * s with s a power of two and q spanning 0..15: the
    quantizer must return q, bf16(s) and bf16(lo) exactly."""
    rng = np.random.default_rng(1)
    rows, gs = 12, 32
    q = rng.integers(0, 16, (rows, 2 * gs))
    q[:, 0], q[:, 1], q[:, gs], q[:, gs + 1] = 0, 15, 15, 0     # each group spans 0..15
    s = np.float32(2.0) ** rng.integers(-12, 4, (rows, 2)).astype(np.float32)
    lo = (rng.integers(-64, 64, (rows, 2)) * np.float32(0.125)).astype(np.float32)
    w = (lo.repeat(gs, 1) + q * s.repeat(gs, 1)).astype(np.float32)
    packed, sc, bi = qo.quantize_4bit(w, gs)
    np.testing.assert_array_equal(qo.nibbles(packed), q)
    np.testing.assert_array_equal(sc, qo.f32_to_bf16(s))
    np.testing.assert_array_equal(bi, qo.f32_to_bf16(lo))
    # nibble j of word c is column 8c + j, in bits 4j..4j+3
    assert int(packed[0, 0]) == sum(int(q[0, j]) << (4 * j) for j in range(8))


def test_oracle_rounds_half_to_even_and_keeps_constant_groups():
    g = np.array([0.0, 15.0, 0.5, 1.5, 2.5, 7.5, 14.5, 3.0], np.float32)
    packed, sc, bi = qo.quantize_4bit(g[None, :], 8)
    assert list(qo.nibbles(packed)[0]) == [0, 15, 0, 2, 2, 8, 14, 3]
    assert int(sc[0, 0]) == 0x3F80 and int(bi[0, 0]) == 0
    c = np.full((1, 16), -0.3, np.float32)
    packed, sc, bi = qo.quantize_4bit(c, 16)
    assert (qo.nibbles(packed) == 0).all()
    assert int(sc[0, 0]) == 0x3F80                     # scale 0 becomes 1
    assert int(bi[0, 0]) == bf16_bits(-0.3)


def test_oracle_dequant_error_bound():
    rng = np.random.default_rng(2)
    w = (rng.standard_normal((64, 256)) * 0.05).astype(np.float32)
    packed, sc, bi = qo.quantize_4bit(w, 64)
    g = w.reshape(64, 4, 64)
    lo, s = g.min(2), (g.max(2) - g.min(2)) / np.float32(15)
    deq = qo.nibbles(packed).reshape(64, 4, 64) * s[:, :, None] + lo[:, :, None]
    assert (np.abs(deq - g) <= s[:, :, None] * 0.5 * (1 + 1e-5) + 1e-12).all()
    # the stored bf16 pair is the f32 pair rounded
    assert (np.abs(bits_to_f32(sc) - s) <= np.abs(s) * 2.0 ** -8).all()


# ---- the library against the oracle -------------------------------------------

def _random_matrix(rng, rows, cols, gs):
    w = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
    w[0, :gs] = 0.25                                    # constant group
    w[1, :gs] = 0.0                                     # all-zero group
    w[2, :gs] = np.linspace(-1, 1, gs, dtype=np.float32) * 7.5   # many ties
    w[3] *= 1e4                                         # large values
    w[4] *= 1e-6                                        # tiny values
    return w


@pytest.mark.parametrize("gs", [32, 64, 128])
@pytest.mark.parametrize("threads", [1, 7])
def test_quantize_4bit_equals_oracle(gs, threads):
    rng = np.random.default_rng(gs + threads)
    w = _random_matrix(rng, 37, 4 * gs, gs)
    got = quant.quantize_4bit(w, gs, threads)
    want = qo.quantize_4bit(w, gs)
    for g, o in zip(got, want):
        np.testing.assert_array_equal(g, o)


def test_f32_to_bf16_equals_oracle():
    rng = np.random.default_rng(5)
    x = rng.integers(0, 2**32, 200000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    np.testing.assert_array_equal(quant.f32_to_bf16(x), qo.f32_to_bf16(x))


@pytest.mark.parametrize("h,inter,gs", [(512, 256, 64), (1024, 512, 32), (512, 1024, 128)])
def test_quantize_expert_equals_oracle_block(h, inter, gs):
    rng = np.random.default_rng(h + inter + gs)
    shape = make_shape(h, 8, 2, inter, gs)
    gate = _random_matrix(rng, inter, h, gs)
    up = _random_matrix(rng, inter, h, gs)
    down = _random_matrix(rng, h, inter, gs)
    blk = quant.quantize_expert(shape, gate, up, down, threads=4)
    np.testing.assert_array_equal(blk, qo.expert_block(gate, up, down, gs))


def test_quantizer_refuses_what_the_reference_asserts_and_non_finite():
    w = np.zeros((4, 96), np.float32)
    with pytest.raises(M1MoEError, match="not divisible by group_size"):
        quant.quantize_4bit(w, 64)
    with pytest.raises(M1MoEError, match="not divisible by 8"):
        quant.quantize_4bit(np.zeros((4, 12), np.float32), 4)
    for bad in (np.nan, np.inf, -np.inf):
        w = np.zeros((4, 64), np.float32)
        w[2, 17] = bad
        with pytest.raises(M1MoEError, match="row 2 holds a non-finite"):
            quant.quantize_4bit(w, 64)
    shape = make_shape(512, 8, 2, 256, 64)
    lib = _lib.load()
    buf = np.zeros(16, np.uint8)
    g = np.zeros((256, 512), np.float32)
    rc = lib.m1moe_quantize_expert(__import__("ctypes").byref(shape), g.ctypes.data,
                                   g.ctypes.data, g.ctypes.data, buf.ctypes.data, buf.size, 1)
    assert rc == _lib.M1MOE_ERR_INVALID and "expert block is" in _lib.last_error()


# ---- the converter -----------------------------------------------------------------

def write_safetensors(path, tensors):
    """A .safetensors file of (name, dtype, array) in the given header order;
    BF16 arrays are given as their u16 bits."""
    header, blobs, off = {}, [], 0
    for name, dt, a in tensors:
        raw = np.ascontiguousarray(a).tobytes()
        header[name] = {"dtype": dt, "shape": list(a.shape), "data_offsets": [off, off + len(raw)]}
        blobs.append(raw)
        off += len(raw)
    header["__metadata__"] = {"format": "pt"}
    h = json.dumps(header).encode()
    h += b" " * (-len(h) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)))
        f.write(h)
        for b in blobs:
            f.write(b)


def _checkpoint(tmp_path, arch, rng, h=512, inter=256, E=4, L=2):
    """Two shards: dense tensors of mixed dtypes spread over both (in
    unsorted header order), experts of both layers split across them."""
    names = {"olmoe": ("mlp.experts.{e}.gate_proj", "mlp.experts.{e}.up_proj",
                       "mlp.experts.{e}.down_proj", "mlp.gate"),
             "mixtral": ("block_sparse_moe.experts.{e}.w1", "block_sparse_moe.experts.{e}.w3",
                         "block_sparse_moe.experts.{e}.w2", "block_sparse_moe.gate")}[arch]
    shard = [[], []]
    experts = {}
    bf16 = lambda a: qo.f32_to_bf16(a)
    shard[1].append(("model.norm.weight", "F32", rng.standard_normal(h).astype(np.float32)))
    shard[0].append(("model.embed_tokens.weight", "BF16",
                     bf16(rng.standard_normal((64, h)).astype(np.float32))))
    shard[1].append(("lm_head.weight", "F16", rng.standard_normal((64, h)).astype(np.float16)))
    shard[0].append(("model.layers.0.odd.weight", "F16",
                     rng.standard_normal(3).astype(np.float16)))   # 6 bytes: next one is padded
    shard[0].append(("model.layers.0.skipped", "I64", np.arange(4, dtype=np.int64)))
    for l in range(L):
        for e in range(E):
            for k, (rows, cols) in enumerate(((inter, h), (inter, h), (h, inter))):
                n = f"model.layers.{l}.{names[k].format(e=e)}.weight"
                a = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
                dt = ("BF16", "F16", "F32")[(l + e + k) % 3]
                if dt == "BF16":
                    bits = bf16(a)
                    shard[(e + k) % 2].append((n, dt, bits))
                    experts[n] = bits_to_f32(bits)
                elif dt == "F16":
                    a16 = a.astype(np.float16)
                    shard[(e + k) % 2].append((n, dt, a16))
                    experts[n] = a16.astype(np.float32)
                else:
                    shard[(e + k) % 2].append((n, dt, a))
                    experts[n] = a
        shard[l % 2].append((f"model.layers.{l}.{names[3]}.weight", "BF16",
                             bf16(rng.standard_normal((E, h)).astype(np.float32))))
    src = tmp_path / "ckpt"
    src.mkdir()
    for i, t in enumerate(shard):
        write_safetensors(src / f"model-{i:05d}-of-00002.safetensors", t[::-1])
    return src, shard, experts, names


@pytest.mark.parametrize("arch", ["olmoe", "mixtral"])
def test_converter_writes_the_reference_layout(tmp_path, arch):
    from m1moe_amd.convert import convert

    rng = np.random.default_rng(11)
    h, inter, E, L, gs = 512, 256, 4, 2, 64
    src, shard, experts, names = _checkpoint(tmp_path, arch, rng, h, inter, E, L)
    out = tmp_path / "out"
    manifest = convert(str(src), str(out), gs, verbose=False)

    # non-expert tensors: sorted names grouped by shard of first appearance,
    # each shard in its header order, 4-byte aligned, converted by dtype
    marker = names[0].split("{")[0]
    dense = sorted(n for t in shard for n, _, _ in t if marker not in n)
    order = []
    for s in sorted({i for i, t in enumerate(shard) for n, _, _ in t if n in dense},
                    key=lambda i: min(dense.index(n) for n, _, _ in shard[i] if n in dense)):
        order += [n for n, dt, _ in shard[s][::-1] if n in dense and dt != "I64"]
    assert list(manifest) == order
    assert json.load(open(out / "model_weights.json")) == manifest
    blob = open(out / "model_weights.bin", "rb").read()
    arrays = {n: (dt, a) for t in shard for n, dt, a in t}
    off = 0
    for n in order:
        dt, a = arrays[n]
        off += -off % 4
        want_dt, raw = {"BF16": ("bf16", a.tobytes()), "F32": ("f32", a.tobytes()),
                        "F16": ("bf16", qo.f32_to_bf16(a.astype(np.float32)).tobytes())}[dt]
        assert manifest[n] == {"offset": off, "shape": list(a.shape), "dtype": want_dt}
        assert blob[off:off + len(raw)] == raw
        off += len(raw)
    assert len(blob) == off

    # experts: per layer, experts in order, gate/up/down each W|S|B
    for l in range(L):
        got = np.fromfile(out / "packed_experts" / f"layer_{l:02d}.bin", np.uint8)
        want = np.concatenate([qo.expert_block(
            *[experts[f"model.layers.{l}.{names[k].format(e=e)}.weight"] for k in range(3)], gs)
            for e in range(E)])
        np.testing.assert_array_equal(got, want)

    # and the library's store reads the manifest back
    lib = _lib.load()
    import ctypes
    st = ctypes.c_void_p()
    _lib.check(lib.m1moe_store_open(str(out / "model_weights.bin").encode(),
                                    str(out / "model_weights.json").encode(), ctypes.byref(st)),
               "m1moe_store_open")
    n = ctypes.c_int32()
    _lib.check(lib.m1moe_store_count(st, ctypes.byref(n)), "m1moe_store_count")
    assert n.value == len(order)
    lib.m1moe_store_close(st)
