"""Golden fixtures (tests/golden/) against the oracle and the generator.  CPU.

The fixtures were written by tests/golden/make_golden.py from the oracle
after tests/test_oracle.py pinned it; these tests catch any later drift of
the oracle's arithmetic or of the seeded generator, bit for bit.
"""
import hashlib
import json
import os

import numpy as np
import pytest

from m1moe_amd import synth
from oracle import oracle as orc

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def load(name):
    return np.load(os.path.join(GOLDEN, name), allow_pickle=False)


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.mark.parametrize("name", ["tiny.npz", "tiny_renorm.npz"])
def test_small_fixture_oracle_bit_exact(name):
    f = load(name)
    h, E, K, I, gs, norm = (int(v) for v in f["shape"])
    s = orc.shape(h, E, K, I, gs, bool(norm))
    bias = f["logit_bias"] if "logit_bias" in f.files else None
    for t in range(f["x_bf16"].shape[0]):
        out, idx, w, lg = orc.moe_decode(s, f["image"], f["router"],
                                         synth.bf16_to_f32(f["x_bf16"][t]), f["residual"][t], bias)
        assert np.array_equal(idx, f["topk_idx"][t])
        assert np.array_equal(bits(w), bits(f["topk_w"][t]))
        assert np.array_equal(bits(lg), bits(f["logits"][t]))
        assert np.array_equal(bits(out), bits(f["out"][t]))
    e = int(f["dequant_expert"][0])
    eb = orc.offsets(s).expert_bytes
    blk = f["image"][e * eb:(e + 1) * eb]
    for p, key in enumerate(["dequant_gate", "dequant_up", "dequant_down"]):
        assert np.array_equal(bits(orc.dequant_proj(s, blk, p)), bits(f[key]))


@pytest.mark.parametrize("name", ["tiny.npz", "tiny_renorm.npz"])
def test_small_fixture_inputs_regenerate(name):
    f = load(name)
    cfg = name[:-4]
    shape = synth.CONFIGS[cfg].shape()
    seed = int(f["seed"][0])
    T = f["x_bf16"].shape[0]
    assert np.array_equal(synth.layer_image(shape, seed, 0), f["image"])
    assert np.array_equal(synth.router(shape, seed, 0), f["router"])
    assert np.array_equal(synth.activations_bf16(shape, seed, T), f["x_bf16"])
    assert np.array_equal(bits(synth.residual_f32(shape, seed, T)), bits(f["residual"]))


def test_cfg0_fixture():
    f = load("cfg0_token.npz")
    seed = int(f["seed"][0])
    shape = synth.CONFIGS["cfg0"].shape()
    img = synth.layer_image(shape, seed, 0)
    router = synth.router(shape, seed, 0)
    assert sha(img) == str(f["image_sha256"])
    assert sha(router) == str(f["router_sha256"])
    s = orc.from_moe_shape(shape)
    for t in range(f["x_bf16"].shape[0]):
        out, idx, w, lg = orc.moe_decode(s, img, router, synth.bf16_to_f32(f["x_bf16"][t]),
                                         f["residual"][t])
        assert np.array_equal(idx, f["topk_idx"][t])
        assert np.array_equal(bits(out), bits(f["out"][t]))
        assert np.array_equal(bits(lg), bits(f["logits"][t]))


def test_generator_checksums():
    with open(os.path.join(GOLDEN, "synth.json")) as fh:
        want = json.load(fh)
    shape = synth.CONFIGS["tiny"].shape()
    got = {
        "layer_image(tiny, seed=5, layer=3)": sha(synth.layer_image(shape, 5, 3)),
        "router(tiny, seed=5, layer=3)": sha(synth.router(shape, 5, 3)),
        "activations_bf16(tiny, seed=5, T=7)": sha(synth.activations_bf16(shape, 5, 7)),
        "residual_f32(tiny, seed=5, T=7)": sha(synth.residual_f32(shape, 5, 7)),
        "normal_bf16(seed=9, id=77, n=1000, sigma=0.5)": sha(synth.normal_bf16(9, 77, 1000, 0.5)),
        "normal_f32(seed=9, id=78, n=1000, sigma=2.0)": sha(synth.normal_f32(9, 78, 1000, 2.0)),
    }
    assert got == want


def test_generator_distributions():
    # nibbles uniform in 0..15; scales |N(0,0.02)|; biases N(0,0.01)
    shape = synth.CONFIGS["tiny"].shape()
    img = synth.layer_image(shape, 3, 0)
    s = orc.from_moe_shape(shape)
    eb = orc.offsets(s).expert_bytes
    w, sc, bi = orc.proj_arrays(s, img[:eb], 0)
    nib = np.stack([(w >> (4 * j)) & 0xF for j in range(8)]).ravel()
    counts = np.bincount(nib, minlength=16)
    assert counts.min() > 0.8 * nib.size / 16 and counts.max() < 1.2 * nib.size / 16
    many = synth.normal_f32(1, 2, 200000, 1.0)
    assert abs(many.mean()) < 0.01 and abs(many.std() - 1.0) < 0.01
    sc_all = synth.bf16_to_f32(synth.normal_bf16(1, 3, 100000, 0.02, absval=True))
    assert sc_all.min() >= 0 and abs(sc_all.mean() - 0.02 * np.sqrt(2 / np.pi)) < 5e-4
    # bf16 rounding is round-to-nearest-even of the f32 value
    f32 = synth.normal_f32(7, 8, 5000, 1.0)
    assert np.array_equal(synth.f32_to_bf16(f32), synth.normal_bf16(7, 8, 5000, 1.0))
