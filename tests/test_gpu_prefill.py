"""GPU parity of the multi-token MoE prefill against the CPU oracle.

The reference has no batched path: prefill is T independent token-by-token
forwards (Sources/bench/main.swift:139-141), so the oracle is the per-token
decode (orc_moe_prefill runs it over T tokens).  Bars: top-K indices
bit-exact per token (same router arithmetic as decode); layer outputs within
1e-2 relative L2 of the oracle (f16 operands with f32 accumulation on the
GPU: weights f16(n*s+b), x exact after a per-token power-of-two scale, act
rounded to f16).  Every call goes through the C ABI.
"""
import os

import numpy as np
import pytest

import m1moe_amd as m
from m1moe_amd import synth
from m1moe_amd.engine import MoEBlock
from oracle import oracle as orc

from cases import REL_L2_TOL, make_case, rel_l2, say

pytestmark = pytest.mark.gpu

NTHREADS = max(1, min(16, os.cpu_count() or 1))


def _run_prefill(c, T, x_dtype="bf16", stream=3, with_residual=True, layer=0):
    blk = MoEBlock(c.ctx)
    h, K = c.shape.hidden, c.shape.top_k
    xb = c.x_bf16(T, stream=stream)
    x32 = synth.bf16_to_f32(xb)
    xin = xb if x_dtype == "bf16" else np.ascontiguousarray(x32)
    res = c.residual(T, stream=stream) if with_residual else None
    dx = c.ctx.to_device(xin)
    dres = c.ctx.to_device(res) if with_residual else None
    dout = c.ctx.alloc(T * h * 4)
    didx, dw = c.ctx.alloc(T * K * 4), c.ctx.alloc(T * K * 4)
    say(f"prefill {c.name} T={T} x={x_dtype} residual={with_residual} layer={layer}")
    blk.prefill(layer, T, dx, x_dtype, dres, dout, didx, dw)
    c.ctx.sync()
    got = dout.download(np.float32).reshape(T, h)
    gidx = didx.download(np.int32).reshape(T, K)
    gw = dw.download(np.float32).reshape(T, K)
    for b in (dx, dres, dout, didx, dw):
        if b is not None:
            b.free()
    return got, gidx, gw, x32, res


def _check(c, T, got, gidx, gw, x32, res, layer=0):
    want, widx, ww = orc.moe_prefill(c.oshape, c.images[layer], c.routers[layer], x32, res,
                                     c.biases[layer], nthreads=NTHREADS)
    assert np.array_equal(gidx, widx), "top-K differs from the oracle"
    np.testing.assert_allclose(gw, ww, rtol=2e-6, atol=1e-7)
    err = rel_l2(got, want)
    per_tok = max(rel_l2(got[t], want[t]) for t in range(T))
    # the MoE contribution alone (the residual would dilute the error)
    r = 0.0 if res is None else res
    moe = rel_l2(got - r, want - r)
    say(f"  rel L2 {err:.3e}, worst token {per_tok:.3e}, MoE part {moe:.3e}")
    assert err <= REL_L2_TOL and per_tok <= REL_L2_TOL and moe <= REL_L2_TOL, (err, per_tok, moe)
    return err


@pytest.mark.parametrize("name,T", [("tiny", 1), ("tiny", 5), ("tiny", 64), ("tiny", 77),
                                    ("tiny_renorm", 3), ("tiny_renorm", 130)])
def test_prefill_small(name, T):
    c = make_case(name, seed=31)
    try:
        _check(c, T, *_run_prefill(c, T))
    finally:
        c.close()


@pytest.fixture(scope="module")
def cfg3():
    wl = synth.CONFIGS["cfg3"]
    bias = synth.zipf_logit_bias(wl.shape().num_experts, wl.zipf_s)
    c = make_case("cfg3", seed=2026, bias=bias)
    yield c
    c.close()


def test_prefill_cfg3_zipf_512(cfg3):
    T = synth.CONFIGS["cfg3"].T
    got, gidx, gw, x32, res = _run_prefill(cfg3, T)
    counts = np.bincount(gidx.ravel(), minlength=cfg3.shape.num_experts)
    say(f"  expert loads: max {counts.max()} min {counts.min()} "
        f"top-4 {np.sort(counts)[::-1][:4].tolist()}")
    assert counts.max() > 4 * counts.mean(), "Zipf bias should skew the loads"
    _check(cfg3, T, got, gidx, gw, x32, res)


@pytest.mark.parametrize("T", [1, 63, 65, 200])
def test_prefill_cfg3_ragged_f32_no_residual(cfg3, T):
    _check(cfg3, T, *_run_prefill(cfg3, T, x_dtype="f32", stream=9, with_residual=False))


def test_prefill_cfg2_mixtral_shape():
    c = make_case("cfg2", seed=5)
    try:
        _check(c, 24, *_run_prefill(c, 24))
    finally:
        c.close()


def test_prefill_cfg2_shape_2048_tokens():
    """cfg4's MoE prefill regime: the Mixtral MoE shape at T=2048 (about 512
    (token, slot) pairs per expert, eight 64-pair tiles each), every token
    against the oracle."""
    c = make_case("cfg2", seed=2048)
    try:
        got, gidx, gw, x32, res = _run_prefill(c, 2048)
        counts = np.bincount(gidx.ravel(), minlength=c.shape.num_experts)
        say(f"  pairs per expert: {counts.tolist()}")
        _check(c, 2048, got, gidx, gw, x32, res)
    finally:
        c.close()


@pytest.mark.parametrize("kw", [
    dict(hidden=1024, num_experts=16, top_k=4, intermediate=512, group_size=128),
    dict(hidden=1152, num_experts=8, top_k=2, intermediate=640, group_size=64),
])
def test_prefill_group_and_block_shapes(kw):
    # gate/up on 256-wide k-blocks at group size 128 (two lanes' 64 columns
    # share a scale group); h % 256 != 0 (gate/up back on 128-wide blocks)
    synth.CONFIGS["_pf_shape"] = synth.Workload("_pf_shape", dict(kw, norm_topk_prob=False))
    c = make_case("_pf_shape", seed=43)
    try:
        _check(c, 100, *_run_prefill(c, 100))
    finally:
        c.close()
        del synth.CONFIGS["_pf_shape"]


def test_prefill_is_deterministic(cfg3):
    a = _run_prefill(cfg3, 300, stream=4)[0]
    b = _run_prefill(cfg3, 300, stream=4)[0]
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_prefill_agrees_with_decode(cfg3):
    """T tokens at once vs T batch-1 decodes on the GPU (same routing)."""
    T = 40
    got, gidx, _, _, res = _run_prefill(cfg3, T, stream=6)
    blk = MoEBlock(cfg3.ctx)
    h, K = cfg3.shape.hidden, cfg3.shape.top_k
    xb = cfg3.x_bf16(T, stream=6)
    out = cfg3.ctx.alloc(h * 4)
    didx = cfg3.ctx.alloc(K * 4)
    dec = np.empty((T, h), np.float32)
    for t in range(T):
        dx, dres = cfg3.ctx.to_device(xb[t]), cfg3.ctx.to_device(res[t])
        blk.forward(0, dx, "bf16", dres, out, didx, None)
        cfg3.ctx.sync()
        dec[t] = out.download(np.float32)
        assert np.array_equal(didx.download(np.int32), gidx[t])
        dx.free()
        dres.free()
    assert rel_l2(got, dec) <= REL_L2_TOL


def _set_groups(img, base, row, groups, first, count, bf16_bits):
    """bf16 words [first, first + count) of row `row` of the [rows][groups]
    scale or bias array at byte offset `base` of a layer image."""
    v = img[base:].view(np.uint16)
    v[row * groups + first:row * groups + first + count] = bf16_bits


def _scale_pow2(img, base, count, p):
    """Multiplies `count` bf16 scales at byte offset `base` by 2^p (exponent
    field + p; the synthetic scales are normal and nonzero)."""
    v = img[base:base + 2 * count].view(np.uint16)
    v[:] = (v.astype(np.int32) + (p << 7)).astype(np.uint16)


def test_prefill_takes_large_scales():
    """Group scales |s| >= 0.25 (s * 2^18 alone would overflow f16) go through
    the per-row power of two: whole matrices scaled by 2^6 .. 2^12 (down of
    experts 0 and 4, gate of 1 and 5, up of 2 and 6) and single rows set to
    s = 0.5 and 8 (gate of 3 and 7), against the oracle at the usual bar."""
    c = make_case("tiny", seed=8)
    try:
        s = c.shape
        eb = c.ctx.expert_bytes
        offs = m.expert_offsets(s)  # gate_w, gate_s, gate_b, up_w, up_s, up_b, down_w, down_s, down_b
        gh = s.hidden // s.group_size
        n_gu, n_d = s.intermediate * gh, s.hidden * (s.intermediate // s.group_size)
        img = c.images[0].copy()
        for e in range(s.num_experts):
            o = e * eb
            if e % 4 == 0:
                _scale_pow2(img, o + offs[7], n_d, 12)      # down s ~ 0.02 * 4096
            elif e % 4 == 1:
                _scale_pow2(img, o + offs[1], n_gu, 6)      # gate s ~ 0.02 * 64
            elif e % 4 == 2:
                _scale_pow2(img, o + offs[4], n_gu, 8)      # up s ~ 0.02 * 256
            else:
                _set_groups(img, o + offs[1], 0, gh, 0, gh, 0x3F00)   # gate row 0: s = 0.5
                _set_groups(img, o + offs[1], 1, gh, 0, 1, 0x4100)    # gate row 1, group 0: s = 8
        c.ctx.upload_layer_experts(0, img)
        c.images[0] = img
        c.ctx.sync()
        T = 64
        say("prefill with group scales up to ~100")
        got, gidx, gw, x32, res = _run_prefill(c, T, stream=12)
        assert np.all(np.isfinite(got))
        _check(c, T, got, gidx, gw, x32, res)
    finally:
        c.close()


def test_prefill_upload_refuses_a_non_finite_scale():
    c = make_case("tiny", seed=9)
    try:
        s = c.shape
        offs = m.expert_offsets(s)
        img = c.images[0].copy()
        _set_groups(img, 3 * c.ctx.expert_bytes + offs[1], 7, s.hidden // s.group_size, 1, 1,
                    0x7F80)  # +inf
        say("upload with an infinite gate scale (expect the upload to refuse it)")
        with pytest.raises(m.M1MoEError, match="non-finite"):
            c.ctx.upload_layer_experts(0, img)
        c.ctx.sync()  # nothing left for the next sync
        # the layer stays unloaded until a good image arrives
        with pytest.raises(m.M1MoEError, match="never uploaded"):
            MoEBlock(c.ctx).prefill(0, 1, c.ctx.alloc(2 * s.hidden), "bf16", None,
                                    c.ctx.alloc(4 * s.hidden))
        c.ctx.upload_layer_experts(0, c.images[0])
    finally:
        c.close()


def test_prefill_graph_replay_matches_eager(cfg3):
    blk = MoEBlock(cfg3.ctx)
    T, h = 96, cfg3.shape.hidden
    xs = [cfg3.x_bf16(T, stream=20 + i) for i in range(2)]
    dx = cfg3.ctx.to_device(xs[0])
    dout = cfg3.ctx.alloc(T * h * 4)
    say("prefill eager reference")
    eager = []
    for xb in xs:
        dx.upload(xb)
        blk.prefill(0, T, dx, "bf16", None, dout)
        cfg3.ctx.sync()
        eager.append(dout.download(np.float32).copy())
    say("prefill graph capture + replays")
    cfg3.ctx.graph_begin()
    blk.prefill(0, T, dx, "bf16", None, dout)
    g = cfg3.ctx.graph_end()
    for rep in range(4):
        dx.upload(xs[rep % 2])
        g.launch()
        cfg3.ctx.sync()
        got = dout.download(np.float32)
        assert np.array_equal(got.view(np.uint32), eager[rep % 2].view(np.uint32)), rep


def test_prefill_takes_act_beyond_f16():
    """Gate and up scales of the even experts times 2^10: their SwiGLU
    products pass the f16 range (checked below on the oracle's own act).  The
    prefill stores each 32-value block of act times its own power of two,
    brings a pair's blocks to one exponent and scales the pair's output back;
    against the oracle at the usual bar, with the odd experts' pairs
    (unscaled) in the same call, and no device error."""
    c = make_case("tiny", seed=12)
    try:
        s = c.shape
        eb = c.ctx.expert_bytes
        offs = m.expert_offsets(s)
        gh = s.hidden // s.group_size
        img = c.images[0].copy()
        for e in range(0, s.num_experts, 2):
            for k in (1, 4):  # gate_s, up_s
                _scale_pow2(img, e * eb + offs[k], s.intermediate * gh, 10)
        c.ctx.upload_layer_experts(0, img)
        c.images[0] = img
        c.ctx.sync()
        T = 48
        say("prefill with SwiGLU products beyond the f16 range")
        got, gidx, gw, x32, res = _run_prefill(c, T, stream=5)
        assert np.all(np.isfinite(got))
        # the oracle's act of the routed pairs: some past 65504, some within
        big = small = 0
        for t in range(T):
            for e in gidx[t]:
                blk = img[int(e) * eb:(int(e) + 1) * eb]
                g = orc.dequant_proj(c.oshape, blk, 0) @ x32[t]
                u = orc.dequant_proj(c.oshape, blk, 1) @ x32[t]
                a = np.abs(orc.swiglu(g.astype(np.float32), u.astype(np.float32))).max()
                big += int(a > 65504.0)
                small += int(a <= 65504.0)
        say(f"  pairs with max |act| past f16: {big}, within: {small}")
        assert big > 0 and small > 0
        _check(c, T, got, gidx, gw, x32, res)
    finally:
        c.close()
