"""m1moe_moe_prefill_noalloc, the prefill entry point that allocates nothing,
against m1moe_moe_prefill (the same kernels on the context's own scratch):
bit-identical outputs, top-K indices and weights on two calls in a row, the
second with fewer tokens and other inputs (the static scratch keeps the first
call's contents); a graph captured around it with no earlier call of that
size, replayed with eager work between replays; and the size limit.  Every
call goes through the C ABI.
"""
import numpy as np
import pytest

from m1moe_amd import synth
from m1moe_amd._lib import M1MOE_ERR_INVALID, M1MoEError
from m1moe_amd.engine import MoEBlock

from cases import make_case, say

pytestmark = pytest.mark.gpu

T_LIMIT_CFG3 = 776     # 64 MiB of static scratch at hidden 2048, 8 x 1024 experts


@pytest.fixture(scope="module")
def cfg3():
    wl = synth.CONFIGS["cfg3"]
    bias = synth.zipf_logit_bias(wl.shape().num_experts, wl.zipf_s)
    c = make_case("cfg3", seed=2026, bias=bias)
    yield c
    c.close()


def _both(c, T, stream):
    """Runs both entry points on the same inputs; returns (noalloc, alloc)
    as (out, idx, w) host arrays."""
    blk = MoEBlock(c.ctx)
    h, K = c.shape.hidden, c.shape.top_k
    dx = c.ctx.to_device(c.x_bf16(T, stream=stream))
    dres = c.ctx.to_device(c.residual(T, stream=stream))
    res = []
    for fn in (blk.prefill_noalloc, blk.prefill):
        dout, didx, dw = c.ctx.alloc(T * h * 4), c.ctx.alloc(T * K * 4), c.ctx.alloc(T * K * 4)
        say(f"{fn.__name__} cfg3 T={T} stream={stream}")
        fn(0, T, dx, "bf16", dres, dout, didx, dw)
        c.ctx.sync()
        res.append((dout.download(np.float32).reshape(T, h),
                    didx.download(np.int32).reshape(T, K),
                    dw.download(np.float32).reshape(T, K)))
        for b in (dout, didx, dw):
            b.free()
    dx.free()
    dres.free()
    return res


def _same(a, b):
    for u, v in zip(a, b):
        assert np.array_equal(u.view(np.uint32), v.view(np.uint32))


def test_noalloc_prefill_matches_prefill_twice(cfg3):
    # 512 tokens, then 200 other tokens: the second call finds the first
    # call's routing and expert outputs in the static scratch
    for T, stream in ((512, 41), (200, 42)):
        na, ref = _both(cfg3, T, stream)
        _same(na, ref)
        assert np.abs(na[0]).max() > 0


def test_noalloc_prefill_in_graph_without_warmup(cfg3):
    """Captured at a T no earlier call used (m1moe_moe_prefill would have to
    grow its scratch there and refuses during capture)."""
    blk = MoEBlock(cfg3.ctx)
    T, h = 640, cfg3.shape.hidden
    xs = [cfg3.x_bf16(T, stream=50 + i) for i in range(2)]
    dx = cfg3.ctx.to_device(xs[0])
    dout = cfg3.ctx.alloc(T * h * 4)
    say("noalloc prefill: graph capture at T=640")
    cfg3.ctx.graph_begin()
    blk.prefill_noalloc(0, T, dx, "bf16", None, dout)
    g = cfg3.ctx.graph_end()
    eager = []
    for xb in xs:
        dx.upload(xb)
        blk.prefill(0, T, dx, "bf16", None, dout)
        cfg3.ctx.sync()
        eager.append(dout.download(np.float32).copy())
    for rep in range(4):
        say(f"  replay {rep}")
        dx.upload(xs[rep % 2])
        g.launch()
        cfg3.ctx.sync()
        got = dout.download(np.float32)
        assert np.array_equal(got.view(np.uint32), eager[rep % 2].view(np.uint32)), rep
        # eager work on the same scratch between replays
        blk.prefill_noalloc(0, 17, dx, "bf16", None, dout)
        cfg3.ctx.sync()
    del g
    dx.free()
    dout.free()


def test_noalloc_prefill_rejects_a_T_beyond_its_scratch(cfg3):
    blk = MoEBlock(cfg3.ctx)
    h = cfg3.shape.hidden
    T = T_LIMIT_CFG3 + 1
    dx = cfg3.ctx.alloc(T * h * 2)
    dout = cfg3.ctx.alloc(T * h * 4)
    with pytest.raises(M1MoEError) as e:
        blk.prefill_noalloc(0, T, dx, "bf16", None, dout)
    assert e.value.code == M1MOE_ERR_INVALID
    assert f"T <= {T_LIMIT_CFG3}" in str(e.value)
    cfg3.ctx.sync()
    dx.free()
    dout.free()
