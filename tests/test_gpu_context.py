"""Context-level guarantees of the C ABI on the GPU: one stream per device,
graphs refused once their scratch was reallocated, uploads that refuse a
non-finite scale, writes through m1moe_expert_block, and inputs whose
magnitude is near the bottom of the f32 range.  Every call goes through
the C ABI; results are checked against the CPU oracle."""
import ctypes
import gc

import numpy as np
import pytest

import m1moe_amd as m
from m1moe_amd import _lib, synth
from m1moe_amd.engine import MoEBlock
from oracle import oracle as orc

from cases import REL_L2_TOL, make_case, rel_l2, say

pytestmark = pytest.mark.gpu


def _stream(ctx):
    s = ctypes.c_void_p()
    _lib.check(ctx.lib.m1moe_get_stream(ctx.handle, ctypes.byref(s)), "m1moe_get_stream")
    return s.value


def _decode_vs_oracle(c, stream=0, layer=0):
    blk = MoEBlock(c.ctx)
    h, K = c.shape.hidden, c.shape.top_k
    xb = c.x_bf16(1, stream=stream)[0]
    res = c.residual(1, stream=stream)[0]
    dx, dres = c.ctx.to_device(xb), c.ctx.to_device(res)
    out, didx = c.ctx.alloc(h * 4), c.ctx.alloc(K * 4)
    blk.forward(layer, dx, "bf16", dres, out, didx)
    c.ctx.sync()
    want, widx = orc.moe_decode(c.oshape, c.images[layer], c.routers[layer],
                                   synth.bf16_to_f32(xb), res)[:2]
    assert np.array_equal(didx.download(np.int32), widx)
    assert rel_l2(out.download(np.float32), want) <= REL_L2_TOL


def test_contexts_on_one_device_share_one_stream():
    """Two live contexts on a device enqueue on the same stream (their
    launches cannot overlap), a caller stream is refused while both are live,
    and both decode correctly when used in turn."""
    a = make_case("cfg0", seed=21)
    b = make_case("tiny", seed=22)
    try:
        assert _stream(a.ctx) == _stream(b.ctx) != 0
        rc = a.ctx.lib.m1moe_set_stream(a.ctx.handle, ctypes.c_void_p(_stream(b.ctx)))
        assert rc == _lib.M1MOE_ERR_INVALID
        assert "share device" in _lib.last_error()
        for turn in range(2):
            say(f"contexts in turn: cfg0 then tiny, turn {turn}")
            _decode_vs_oracle(a, stream=turn)
            _decode_vs_oracle(b, stream=turn)
    finally:
        b.close()
    # alone on the device, the context may take a caller stream; no second
    # context is created while it does (contexts other tests left for the
    # garbage collector are collected first)
    gc.collect()
    try:
        s = _stream(a.ctx)
        rc = a.ctx.lib.m1moe_set_stream(a.ctx.handle, ctypes.c_void_p(s))
        if rc != _lib.M1MOE_OK:
            assert "share device" in _lib.last_error()
            pytest.skip("another test's context is still alive on the device")
        with pytest.raises(m.M1MoEError) as ei:
            m.HIPContext(m.make_shape(128, 8, 2, 64, 64))
        assert "caller stream" in str(ei.value)
        assert a.ctx.lib.m1moe_set_stream(a.ctx.handle, None) == _lib.M1MOE_OK
        c = m.HIPContext(m.make_shape(128, 8, 2, 64, 64))
        assert _stream(c) == _stream(a.ctx)
        c.close()
        _decode_vs_oracle(a, stream=5)
    finally:
        a.close()


def test_graph_refused_after_scratch_growth():
    """A graph holds the scratch addresses of its capture: after an eager
    call reallocates that scratch, launching it is refused; a new capture
    works and matches the eager result."""
    c = make_case("tiny", seed=31)
    try:
        blk = MoEBlock(c.ctx)
        h = c.shape.hidden
        T0, T1 = 8, 64
        xb = c.x_bf16(T1, stream=4)
        dx = c.ctx.to_device(xb)
        out = c.ctx.alloc(T1 * h * 4)
        say(f"prefill T={T0} eager, then captured")
        blk.prefill(0, T0, dx, "bf16", None, out)
        c.ctx.sync()
        eager = out.download(np.float32)[:T0 * h].copy()
        c.ctx.graph_begin()
        blk.prefill(0, T0, dx, "bf16", None, out)
        g = c.ctx.graph_end()
        g.launch()
        c.ctx.sync()
        assert np.array_equal(out.download(np.float32)[:T0 * h], eager)
        say(f"prefill T={T1} eager (scratch grows)")
        blk.prefill(0, T1, dx, "bf16", None, out)
        c.ctx.sync()
        with pytest.raises(m.M1MoEError) as ei:
            g.launch()
        assert ei.value.code == _lib.M1MOE_ERR_INVALID and "capture it again" in str(ei.value)
        c.ctx.graph_begin()
        blk.prefill(0, T0, dx, "bf16", None, out)
        g2 = c.ctx.graph_end()
        out.upload(np.zeros(T1 * h, np.float32))
        g2.launch()
        c.ctx.sync()
        assert np.array_equal(out.download(np.float32)[:T0 * h], eager)
    finally:
        c.close()


def test_upload_refuses_non_finite_scale():
    shape = synth.CONFIGS["tiny"].shape(1)
    img = synth.layer_image(shape, 41, 0)
    off = m.expert_offsets(shape)
    eb = m.expert_bytes(shape)
    bad = img.copy()
    # expert 1's first down scale: a bf16 NaN
    bad[eb + off[7]: eb + off[7] + 2] = np.frombuffer(np.uint16(0x7FC0).tobytes(), np.uint8)
    say("upload of an image with a NaN scale")
    with m.HIPContext(shape) as ctx:
        with pytest.raises(m.M1MoEError) as ei:
            ctx.upload_layer_experts(0, bad)
        assert ei.value.code == _lib.M1MOE_ERR_INVALID and "non-finite" in str(ei.value)
        ctx.sync()  # the flag was taken back: nothing left for the next sync
        ctx.upload_layer_experts(0, img)
        ctx.upload_router(0, synth.router(shape, 41, 0))
        ctx.sync()


def test_writes_through_expert_block_reach_decode_and_prefill():
    """An expert block rewritten on the device through m1moe_expert_block is
    what the next decode and prefill use (their repacked copies are rebuilt),
    bit for bit in the routing and to the oracle's bar in the outputs."""
    c = make_case("cfg0", seed=51)
    try:
        blk = MoEBlock(c.ctx)
        h, K = c.shape.hidden, c.shape.top_k
        eb = c.ctx.expert_bytes
        xb = c.x_bf16(4, stream=9)
        x32 = synth.bf16_to_f32(xb)
        dx = c.ctx.to_device(xb)
        out, didx = c.ctx.alloc(4 * h * 4), c.ctx.alloc(4 * K * 4)
        blk.forward(0, dx, "bf16", None, out, didx)
        c.ctx.sync()
        sel = didx.download(np.int32)[:K]
        # replace every selected expert of token 0 with another seed's blocks
        other = synth.layer_image(c.shape, 52, 0)
        img = c.images[0].copy()
        for e in sel:
            p = ctypes.c_void_p()
            _lib.check(c.ctx.lib.m1moe_expert_block(c.ctx.handle, 0, int(e), ctypes.byref(p)),
                       "m1moe_expert_block")
            blkbytes = np.ascontiguousarray(other[e * eb:(e + 1) * eb])
            _lib.check(c.ctx.lib.m1moe_copy_h2d(c.ctx.handle, p, blkbytes.ctypes.data_as(
                ctypes.c_void_p), eb), "m1moe_copy_h2d")
            img[e * eb:(e + 1) * eb] = blkbytes
        say("decode after writes through m1moe_expert_block")
        blk.forward(0, dx, "bf16", None, out, didx)
        c.ctx.sync()
        want, widx = orc.moe_decode(c.oshape, img, c.routers[0], x32[0])[:2]
        assert np.array_equal(didx.download(np.int32)[:K], widx)
        assert rel_l2(out.download(np.float32)[:h], want) <= REL_L2_TOL
        # the old blocks would fail the same bar
        old = orc.moe_decode(c.oshape, c.images[0], c.routers[0], x32[0])[0]
        assert rel_l2(old, want) > 10 * REL_L2_TOL
        say("prefill T=4 after the writes")
        blk.prefill(0, 4, dx, "bf16", None, out, didx)
        c.ctx.sync()
        wp, wpi, _ = orc.moe_prefill(c.oshape, img, c.routers[0], x32)
        assert np.array_equal(didx.download(np.int32).reshape(4, K), wpi)
        assert rel_l2(out.download(np.float32).reshape(4, h), wp) <= REL_L2_TOL
    finally:
        c.close()


@pytest.mark.parametrize("name", ["cfg0", "cfg2"])
def test_tiny_input_chunks_stay_finite(name):
    """Input chunks near the bottom of the f32 range (max |x| ~ 1e-36, whose
    power-of-two staging scale would be 2^133) next to ordinary ones: the
    output is finite and matches the oracle; a whole token that small gives
    the residual."""
    c = make_case(name, seed=61)
    try:
        blk = MoEBlock(c.ctx)
        h = c.shape.hidden
        x = synth.bf16_to_f32(c.x_bf16(1, stream=2)[0]).copy()
        x[160:192] *= np.float32(1e-36)       # one 32-column chunk
        xb = synth.f32_to_bf16(x)
        x32 = synth.bf16_to_f32(xb)
        res = c.residual(1, stream=2)[0]
        dres, out = c.ctx.to_device(res), c.ctx.alloc(h * 4)
        for dt, xin in (("bf16", xb), ("f32", x32)):
            say(f"decode {name} with a 1e-36 chunk, x {dt}")
            dx = c.ctx.to_device(np.ascontiguousarray(xin))
            blk.forward(0, dx, dt, dres, out)
            c.ctx.sync()
            got = out.download(np.float32)
            assert np.isfinite(got).all()
            want = orc.moe_decode(c.oshape, c.images[0], c.routers[0], x32, res)[0]
            assert rel_l2(got - res, want - res) <= REL_L2_TOL
        T = 4
        xs = synth.bf16_to_f32(c.x_bf16(T, stream=3)).copy()
        xs[1] *= np.float32(1e-36)             # a whole token
        xs[2, 64:96] *= np.float32(1e-36)
        xsb = synth.f32_to_bf16(xs)
        xs32 = synth.bf16_to_f32(xsb)
        rs = c.residual(T, stream=3)
        dx, dres, out = c.ctx.to_device(xsb), c.ctx.to_device(rs), c.ctx.alloc(T * h * 4)
        say(f"prefill {name} T={T} with tiny rows")
        blk.prefill(0, T, dx, "bf16", dres, out)
        c.ctx.sync()
        got = out.download(np.float32).reshape(T, h)
        assert np.isfinite(got).all()
        want = orc.moe_prefill(c.oshape, c.images[0], c.routers[0], xs32, rs)[0]
        assert rel_l2(got - rs, want - rs) <= REL_L2_TOL
        np.testing.assert_allclose(got[1], want[1], rtol=0, atol=1e-30)
    finally:
        c.close()
