"""GPU parity of the dense decoder step and the whole decoder against the CPU
oracle (oracle/dense_oracle.c, oracle.DecoderOracle), through the C ABI.

Tolerances: every sum on the GPU is f32 in its own order against the
oracle's f64, so the building blocks are held to relative L2 1e-5 (argmax
bit-exact).  The MoE decode splits its f32 inputs and activations into hi +
lo f16 halves for the nibble dot products, the MoE prefill rounds them to
one f16 (its own parity bar is relative L2 1e-2), so decoder logits are held
to the north-star bar of relative L2 1e-2, and greedy tokens must agree
wherever the oracle's top-2 logit margin exceeds the logit error bound.
The long cases (cfg4 widths at 2048 positions, cfg1 at 16 layers and 128 +
128 tokens) run the oracle's prompt layer by layer on up to 16 threads.
"""
import os

import numpy as np
import pytest

import m1moe_amd as m
from m1moe_amd import M1MoEError, _lib, synth
from m1moe_amd.decoder import Decoder, DenseOps
from oracle import oracle as orc

from cases import rel_l2, say

pytestmark = pytest.mark.gpu

RNG = np.random.default_rng(77)
NAMES = {_lib.W_EMBED: "embed", _lib.W_LM_HEAD: "lm_head", _lib.W_FINAL_NORM: "final_norm",
         _lib.W_IN_NORM: "in_norm", _lib.W_POST_NORM: "post_norm", _lib.W_Q: "q", _lib.W_K: "k",
         _lib.W_V: "v", _lib.W_O: "o", _lib.W_Q_NORM: "q_norm", _lib.W_K_NORM: "k_norm"}
LOGIT_TOL = 1e-2
NTHREADS = max(1, min(16, os.cpu_count() or 1))


def bf16(a):
    return synth.f32_to_bf16(np.asarray(a, np.float32))


@pytest.fixture(scope="module")
def ops_ctx():
    say("dense ops context")
    ctx = m.HIPContext(m.make_shape(128, 8, 2, 64, 64))
    yield ctx, DenseOps(ctx)
    ctx.close()


# ---- building blocks --------------------------------------------------------------------

@pytest.mark.parametrize("n", [1, 100, 2048, 4096, 5000])
def test_rmsnorm(ops_ctx, n):
    ctx, ops = ops_ctx
    x = RNG.normal(0, 3, n).astype(np.float32)
    w = bf16(RNG.normal(1, 0.1, n))
    dx, dw, dout = ctx.to_device(x), ctx.to_device(w), ctx.alloc(4 * n)
    say(f"rmsnorm n={n}")
    ops.rmsnorm(dx, dw, dout, n, 1e-5)
    ctx.sync()
    assert rel_l2(dout.download(np.float32), orc.rmsnorm(x, w, 1e-5)) < 1e-6


@pytest.mark.parametrize("rows,cols,with_res", [(1, 8, False), (37, 200, True), (2048, 2048, True),
                                                (6144, 2048, False), (2048, 4096, True),
                                                (50304, 2048, False), (33000, 2560, True),
                                                (40001, 4096, True), (40001, 4096, False),
                                                (131075, 1024, False), (3, 65536, False)])
def test_matvec_bf16(ops_ctx, rows, cols, with_res):
    ctx, ops = ops_ctx
    w = bf16(RNG.normal(0, 1 / np.sqrt(cols), (rows, cols)))
    x = RNG.normal(0, 1, cols).astype(np.float32)
    r = RNG.normal(0, 1, rows).astype(np.float32) if with_res else None
    dw, dx, dy = ctx.to_device(w), ctx.to_device(x), ctx.alloc(4 * rows)
    dr = ctx.to_device(r) if with_res else None
    say(f"matvec_bf16 {rows}x{cols} residual={with_res}")
    ops.matvec_bf16(dw, dx, dr, dy, rows, cols)
    ctx.sync()
    got = dy.download(np.float32)
    want = orc.matvec_bf16(w, x, residual=r)
    assert rel_l2(got, want) < 1e-5


@pytest.mark.parametrize("nh,nkv,hd,sl", [(16, 16, 128, 1), (4, 2, 64, 255), (4, 2, 64, 256),
                                           (4, 2, 64, 257), (32, 8, 128, 1000), (2, 1, 256, 700),
                                           (16, 16, 128, 4096), (32, 8, 128, 2112),
                                           (32, 4, 128, 2112), (16, 2, 64, 4096),
                                           (8, 2, 128, 5000), (4, 4, 64, 8300),
                                           # one wide sub-chunk per workgroup (65..80
                                           # positions: the grid fits the CUs)
                                           (32, 8, 64, 2100), (32, 8, 256, 2100),
                                           (64, 64, 128, 300)])
def test_attention_decode(ops_ctx, nh, nkv, hd, sl):
    """The attention building block against the oracle: one chunk, 64-position
    chunks up to 64 per kv head, chunks of several 64-position sub-chunks
    (two K/V register sets), chunks of one wide sub-chunk (65..80
    positions, when 64-position chunks would put more workgroups than CUs:
    the Mixtral grouping at 2100-2112 positions, 64 single-head groups at
    300), head_dim 64 / 128 / 256."""
    ctx, ops = ops_ctx
    kvd = nkv * hd
    q = RNG.normal(0, 1, nh * hd).astype(np.float32)
    kc = RNG.normal(0, 1, (sl, kvd)).astype(np.float32)
    vc = RNG.normal(0, 1, (sl, kvd)).astype(np.float32)
    dq, dk, dv, dout = ctx.to_device(q), ctx.to_device(kc), ctx.to_device(vc), ctx.alloc(4 * nh * hd)
    say(f"attention nh={nh} nkv={nkv} hd={hd} seq={sl}")
    ops.attention_decode(dq, dk, dv, dout, nh, nkv, hd, sl)
    ctx.sync()
    want = orc.attention(q, kc, vc, nh, nkv, hd, sl)
    assert rel_l2(dout.download(np.float32), want) < 1e-5


@pytest.mark.parametrize("nh,nkv,hd", [(2048, 1, 64), (1024, 8, 128)])
def test_attention_decode_rejects_too_many_heads(ops_ctx, nh, nkv, hd):
    """num_heads * head_dim > 65536 is refused before any launch (the launch
    keeps one counter per q-head group, 1024 of them)."""
    ctx, ops = ops_ctx
    buf = ctx.alloc(1 << 16)
    with pytest.raises(M1MoEError) as ei:
        ops.attention_decode(buf, buf, buf, buf, nh, nkv, hd, 100)
    assert ei.value.code == _lib.M1MOE_ERR_INVALID
    assert "exceeds 65536" in str(ei.value)


@pytest.mark.parametrize("case", ["random", "ties", "nan0", "nan_mid", "neg_inf", "one"])
def test_argmax(ops_ctx, case):
    ctx, ops = ops_ctx
    n = 50304
    x = RNG.normal(0, 1, n).astype(np.float32)
    if case == "ties":
        x[[7, 3000, 50000]] = 9.0
    elif case == "nan0":
        x[0] = np.nan
    elif case == "nan_mid":
        x[[5, 60, 40000]] = np.nan
    elif case == "neg_inf":
        x[:] = -np.inf
    elif case == "one":
        x = x[:1]
        n = 1
    dx, di = ctx.to_device(x), ctx.alloc(16)
    say(f"argmax {case}")
    ops.argmax(dx, n, di)
    ctx.sync()
    assert int(di.download(np.int32, 1)[0]) == orc.argmax(x)


# ---- the decoder -------------------------------------------------------------------------

class Pair:
    """The same seeded model on the GPU (Decoder) and in the oracle."""

    def __init__(self, wl, seed, max_seq, num_layers=None, nthreads=1):
        self.wl = wl
        L = num_layers or wl.num_layers
        shape = wl.moe.shape(L)
        say(f"decoder {wl.name} layers={L} max_seq={max_seq} seed={seed}")
        self.ctx = m.HIPContext(shape)
        ds = wl.dec_shape(max_seq)
        self.dec = Decoder(self.ctx, ds)
        tensors = {}
        for which, name in NAMES.items():
            if which in _lib.W_PER_LAYER:
                tensors[name] = [synth.dense_weight(wl, seed, which, l) for l in range(L)]
            else:
                tensors[name] = synth.dense_weight(wl, seed, which, 0)
        self.dec.upload_all(lambda which, l: tensors[NAMES[which]][l]
                            if which in _lib.W_PER_LAYER else tensors[NAMES[which]])
        images, routers = [], []
        for l in range(L):
            img = synth.layer_image(shape, seed, l)
            r = synth.router(shape, seed, l)
            self.ctx.upload_layer_experts(l, img)
            self.ctx.upload_router(l, r)
            images.append(img)
            routers.append(r)
        self.orc = orc.DecoderOracle(orc.from_moe_shape(shape), L, wl.vocab, wl.num_heads,
                                     wl.num_kv_heads, wl.head_dim, max_seq, wl.qk_norm,
                                     wl.rope_theta, wl.rms_eps, tensors, images, routers,
                                     nthreads=nthreads)

    def close(self):
        self.orc.close()
        self.dec.close()
        self.ctx.close()


def check_step(got_tok, got_logits, want_tok, want_logits, where):
    rel = rel_l2(got_logits, want_logits)
    assert rel < LOGIT_TOL, f"{where}: logits rel L2 {rel:.2e}"
    if got_tok != want_tok:
        top2 = np.sort(want_logits.astype(np.float64))[-2:]
        bound = 4 * LOGIT_TOL * np.linalg.norm(want_logits) / np.sqrt(want_logits.size)
        assert top2[1] - top2[0] < bound, f"{where}: token {got_tok} != {want_tok}"
    return rel


def test_decoder_tiny_teacher_forced_over_two_attention_chunks():
    """280 forced tokens: the cache crosses the 256-position attention chunk."""
    p = Pair(synth.DECODERS["tiny_dec"], seed=11, max_seq=300)
    try:
        toks = synth.prompt_tokens(p.wl, 5, 280)
        rels = []
        for i, t in enumerate(toks):
            g_tok, g_lg = p.dec.forward(int(t), return_logits=True)
            w_tok, w_lg = p.orc.step(int(t))
            rels.append(check_step(g_tok, g_lg, w_tok, w_lg, f"step {i}"))
        assert p.dec.position() == 280
        rels = np.array(rels)
        say(f"tiny decoder logits rel L2: median {np.median(rels):.2e}, worst before "
            f"position 256 {rels[:256].max():.2e}, from 256 on {rels[256:].max():.2e}")
    finally:
        p.close()


def test_decoder_forward_samples_from_its_logits():
    """forward(temperature > 0) samples on the host from the step's logits
    (InferenceEngine.swift:557-574) with the caller's generator."""
    from m1moe_amd.sampling import sample_token
    p = Pair(synth.DECODERS["tiny_dec"], seed=17, max_seq=16)
    try:
        toks = synth.prompt_tokens(p.wl, 2, 4)
        for i, t in enumerate(toks):
            tok, lg = p.dec.forward(int(t), return_logits=True, temperature=0.8, top_p=0.9,
                                    rng=np.random.default_rng(i))
            assert tok == sample_token(lg, 0.8, 0.9, rng=np.random.default_rng(i))
        assert p.dec.position() == len(toks)
    finally:
        p.close()


def test_decoder_reset_restarts_the_sequence():
    p = Pair(synth.DECODERS["tiny_dec"], seed=12, max_seq=32)
    try:
        toks = synth.prompt_tokens(p.wl, 6, 6)
        first = [p.dec.forward(int(t), return_logits=True)[1] for t in toks]
        p.dec.reset()
        assert p.dec.position() == 0
        again = [p.dec.forward(int(t), return_logits=True)[1] for t in toks]
        for a, b in zip(first, again):
            np.testing.assert_array_equal(a, b)
    finally:
        p.close()


def test_decoder_greedy_loop_in_a_graph():
    """Prompt steps read &prompt[i]; greedy steps chain toks[i] -> toks[i+1];
    the captured loop is replayed three times against the eager run."""
    p = Pair(synth.DECODERS["tiny_dec"], seed=13, max_seq=64)
    try:
        ctx, dec = p.ctx, p.dec
        prompt = synth.prompt_tokens(p.wl, 7, 8)
        n_gen = 24
        # eager reference run through forward() (one host round trip per step)
        eager = []
        tok = None
        for t in prompt:
            tok = dec.forward(int(t))
        for _ in range(n_gen):
            eager.append(tok)
            tok = dec.forward(tok)
        eager.append(tok)
        P = len(prompt)
        dprompt = ctx.to_device(prompt)
        dpred = ctx.alloc(4 * P)
        dtoks = ctx.alloc(4 * (n_gen + 1))  # toks[i+1] = greedy(toks[i]); toks[0] unused
        ctx.graph_begin()
        dec.reset()
        for i in range(P):
            dec.step_device(dprompt.addr + 4 * i, dpred.addr + 4 * i)
        for i in range(n_gen):
            src = dpred.addr + 4 * (P - 1) if i == 0 else dtoks.addr + 4 * i
            dec.step_device(src, dtoks.addr + 4 * (i + 1))
        graph = ctx.graph_end()
        for rep in range(3):
            say(f"graph replay {rep}")
            graph.launch()
            ctx.sync()
            assert int(dpred.download(np.int32)[P - 1]) == eager[0], f"replay {rep}"
            assert dtoks.download(np.int32).tolist()[1:] == eager[1:], f"replay {rep}"
            assert dec.position() == P + n_gen
            dtoks.upload(np.zeros(n_gen + 1, np.int32))  # eager work between replays
        # the oracle, fed the same tokens, picks the same ones wherever its
        # top-2 margin is clear of the logit error
        p.orc.reset()
        for t in prompt:
            w, lg = p.orc.step(int(t))
        for i in range(n_gen + 1):
            top2 = np.sort(lg.astype(np.float64))[-2:]
            assert w == eager[i] or top2[1] - top2[0] < 1e-2, f"greedy step {i}"
            if i < n_gen:
                w, lg = p.orc.step(eager[i])
    finally:
        p.close()


def test_decoder_sequence_mode_and_one_step_graph():
    """m1moe_dec_step_seq: eager calls, and one captured step replayed P + G
    times, give the tokens of the forward() loop (prompt then greedy)."""
    p = Pair(synth.DECODERS["tiny_dec"], seed=16, max_seq=40)
    try:
        ctx, dec = p.ctx, p.dec
        prompt = synth.prompt_tokens(p.wl, 9, 7)
        P, G = len(prompt), 20
        want = []
        tok = None
        for t in prompt:
            tok = dec.forward(int(t))
        for _ in range(G):
            want.append(tok)
            tok = dec.forward(tok)
        want.append(tok)
        assert dec.generate(prompt, G).tolist() == want
        cap = P + G + 1
        seq = ctx.alloc(4 * cap)
        init = np.concatenate([prompt, np.full(cap - P, -7, np.int32)])
        ctx.graph_begin()
        dec.step_seq(seq, P, cap)
        graph = ctx.graph_end()
        for rep in range(3):
            seq.upload(init)
            dec.reset()
            say(f"one-step graph, {P + G} replays, round {rep}")
            for _ in range(P + G):
                graph.launch()
            ctx.sync()
            got = seq.download(np.int32)
            assert got[:P].tolist() == prompt.tolist()  # the prompt is never overwritten
            assert got[P:].tolist() == want, f"round {rep}"
            assert dec.position() == P + G
    finally:
        p.close()


def test_decoder_dense_only_is_tight():
    """With the MoE block's expert weights all zero (scales and biases 0) the
    block adds only the residual, so the step is the dense kernels alone:
    logits to relative L2 1e-5 over positions on both sides of 256."""
    wl = synth.DECODERS["tiny_dec"]
    p = Pair(wl, seed=15, max_seq=300)
    try:
        zero = np.zeros_like(p.orc.images[0])
        for l in range(wl.num_layers):
            p.ctx.upload_layer_experts(l, zero)
            p.orc.images[l] = zero
        worst = 0.0
        for i, t in enumerate(synth.prompt_tokens(wl, 8, 270)):
            g_tok, g_lg = p.dec.forward(int(t), return_logits=True)
            w_tok, w_lg = p.orc.step(int(t))
            rel = rel_l2(g_lg, w_lg)
            assert rel < 1e-5, f"step {i}: rel L2 {rel:.2e}"
            worst = max(worst, rel)
            if g_tok != w_tok:
                top2 = np.sort(w_lg.astype(np.float64))[-2:]
                assert top2[1] - top2[0] < 1e-4, f"step {i}: token {g_tok} != {w_tok}"
        say(f"dense-only decoder worst logits rel L2 {worst:.2e}")
    finally:
        p.close()


def _zero_experts(p):
    zero = np.zeros_like(p.orc.images[0])
    for l in range(p.orc.L):
        p.ctx.upload_layer_experts(l, zero)
        p.orc.images[l] = zero


@pytest.mark.parametrize("Ts", [(1,), (17,), (130,), (5, 7)])
def test_prefill_dense_path_is_tight(Ts):
    """Batched prefill with the MoE block zeroed (it then adds only the
    residual): the f32 GEMMs, causal attention, RoPE and KV rows against the
    oracle's token-by-token run, logits of each prefill's last token to
    relative L2 1e-5, then a greedy step from the prefilled cache."""
    wl = synth.DECODERS["tiny_dec"]
    p = Pair(wl, seed=31, max_seq=160)
    try:
        _zero_experts(p)
        toks = synth.prompt_tokens(wl, 12, sum(Ts))
        off = 0
        for T in Ts:
            say(f"prefill T={T} at position {off}")
            g_tok, g_lg = p.dec.prefill(toks[off:off + T], return_logits=True)
            for t in toks[off:off + T]:
                w_tok, w_lg = p.orc.step(int(t))
            off += T
            rel = rel_l2(g_lg, w_lg)
            assert rel < 1e-5, f"T={T}: rel L2 {rel:.2e}"
            assert g_tok == w_tok or np.ptp(np.sort(w_lg)[-2:]) < 1e-4
            assert p.dec.position() == off
        g_tok, g_lg = p.dec.forward(int(toks[0]), return_logits=True)
        w_tok, w_lg = p.orc.step(int(toks[0]))
        assert rel_l2(g_lg, w_lg) < 1e-5
    finally:
        p.close()


def test_prefill_split_k_gemms_are_tight():
    """OLMoE widths (h = q = kv = 2048), one layer, MoE block zeroed.  A
    100-token prefill: q, k and v as one launch over three weight segments
    (192 tiles of 64 x 64, 4 shares of 8 k-blocks), o_proj 64 tiles in 8
    shares of 4 k-blocks, summed with the residual and normalised in one
    kernel; a second 200-token prefill: q/k/v 384 tiles in 2 shares, o_proj
    128 tiles in 6 shares of 5-6 k-blocks.  Partials summed in a fixed order;
    last logits against the oracle's token-by-token run to relative L2 1e-5."""
    p = Pair(synth.DECODERS["cfg1"], seed=53, max_seq=310, num_layers=1, nthreads=8)
    try:
        _zero_experts(p)
        toks = synth.prompt_tokens(p.wl, 23, 300)
        off = 0
        for T in (100, 200):
            say(f"olmoe-width split-K prefill T={T} at position {off}")
            g_tok, g_lg = p.dec.prefill(toks[off:off + T], return_logits=True)
            for t in toks[off:off + T]:
                w_tok, w_lg = p.orc.step(int(t))
            off += T
            rel = rel_l2(g_lg, w_lg)
            assert rel < 1e-5, f"T={T}: rel L2 {rel:.2e}"
            assert p.dec.position() == off
    finally:
        p.close()


def test_prefill_longer_than_one_piece():
    """A 4100-token prompt goes through m1moe_dec_prefill in two pieces (4096
    + 4): last logits against the oracle's token-by-token run to 1e-5 (MoE
    block zeroed), and the position reaches 4100."""
    wl = synth.DECODERS["tiny_dec"]
    p = Pair(wl, seed=43, max_seq=4110)
    try:
        _zero_experts(p)
        toks = synth.prompt_tokens(wl, 19, 4100)
        say("prefill of 4100 tokens (two pieces)")
        g_tok, g_lg = p.dec.prefill(toks, return_logits=True)
        for t in toks:
            w_tok, w_lg = p.orc.step(int(t))
        rel = rel_l2(g_lg, w_lg)
        assert rel < 1e-5, f"rel L2 {rel:.2e}"
        assert p.dec.position() == 4100
    finally:
        p.close()


@pytest.mark.parametrize("Ts", [(150,), (40, 90)])
def test_prefill_dense_path_head_dim_128_gqa(Ts):
    """The MFMA prefill attention at head_dim 128 with 4 q heads per kv head
    (the Mixtral grouping), T crossing several 64-query and 32-key blocks,
    a second prefill over a past context: last logits against the oracle's
    token-by-token run to relative L2 1e-5 (MoE block zeroed)."""
    wl = synth.DecoderWorkload("hd128_gqa", synth.CONFIGS["tiny_renorm"], 1, 300, 8, 2, 128,
                               1e6, False, 8, 8)
    p = Pair(wl, seed=41, max_seq=200)
    try:
        _zero_experts(p)
        toks = synth.prompt_tokens(wl, 14, sum(Ts))
        off = 0
        for T in Ts:
            say(f"prefill head_dim 128 T={T} at position {off}")
            g_tok, g_lg = p.dec.prefill(toks[off:off + T], return_logits=True)
            for t in toks[off:off + T]:
                w_tok, w_lg = p.orc.step(int(t))
            off += T
            rel = rel_l2(g_lg, w_lg)
            assert rel < 1e-5, f"T={T}: rel L2 {rel:.2e}"
            assert p.dec.position() == off
    finally:
        p.close()


def test_prefill_whole_decoder_then_greedy():
    """The whole decoder (MoE prefill included): the prompt's last logits and
    the greedy steps after it against the oracle at the decoder bar."""
    wl = synth.DECODERS["tiny_dec"]
    p = Pair(wl, seed=32, max_seq=80)
    try:
        prompt = synth.prompt_tokens(wl, 13, 48)
        say("prefill 48 + 8 greedy")
        tok, g_lg = p.dec.prefill(prompt, return_logits=True)
        for t in prompt:
            w_tok, w_lg = p.orc.step(int(t))
        check_step(tok, g_lg, w_tok, w_lg, "prefill")
        for i in range(8):
            feed = w_tok  # the oracle's token, so both see the same sequence
            g_tok, g_lg = p.dec.forward(int(feed), return_logits=True)
            w_tok, w_lg = p.orc.step(int(feed))
            check_step(g_tok, g_lg, w_tok, w_lg, f"greedy {i}")
    finally:
        p.close()


def test_prefill_past_the_cache_is_reported():
    wl = synth.DECODERS["tiny_dec"]
    p = Pair(wl, seed=33, max_seq=10)
    try:
        p.dec.prefill(synth.prompt_tokens(wl, 3, 6))
        say("prefill past max_seq")
        with pytest.raises(m.M1MoEError, match="KV cache full"):
            p.dec.prefill(synth.prompt_tokens(wl, 4, 6))
        p.dec.reset()
        p.dec.prefill(synth.prompt_tokens(wl, 3, 10))  # exactly full is fine
        assert p.dec.position() == 10
    finally:
        p.close()


def test_decoder_olmoe_dims_two_layers():
    """Full OLMoE widths (h 2048, 16x128 heads, vocab 50304, 64 experts top-8),
    two layers, four prompt tokens and four greedy steps."""
    p = Pair(synth.DECODERS["cfg1"], seed=2026, max_seq=16, num_layers=2)
    try:
        toks = synth.prompt_tokens(p.wl, 2026, 4)
        tok = None
        for i, t in enumerate(toks):
            g_tok, g_lg = p.dec.forward(int(t), return_logits=True)
            w_tok, w_lg = p.orc.step(int(t))
            check_step(g_tok, g_lg, w_tok, w_lg, f"prompt {i}")
            tok = w_tok
        for i in range(4):
            g_tok, g_lg = p.dec.forward(tok, return_logits=True)
            w_tok, w_lg = p.orc.step(tok)
            check_step(g_tok, g_lg, w_tok, w_lg, f"greedy {i}")
            tok = w_tok
        # the same prompt through the batched prefill
        p.dec.reset()
        p.orc.reset()
        say("olmoe-width prefill of 8")
        tok, g_lg = p.dec.prefill(synth.prompt_tokens(p.wl, 7, 8), return_logits=True)
        for t in synth.prompt_tokens(p.wl, 7, 8):
            w_tok, w_lg = p.orc.step(int(t))
        check_step(tok, g_lg, w_tok, w_lg, "prefill")
    finally:
        p.close()


def test_decoder_olmoe_dims_past_one_attention_chunk():
    """OLMoE widths, two layers: a 100-token batched prefill, then greedy
    steps at positions 100..103.  Two 64-position attention chunks are
    active, 16 heads x 2 chunks: the attention launch leaves the chunk merge
    to the o_proj launch, which merges the partials as its input."""
    p = Pair(synth.DECODERS["cfg1"], seed=2027, max_seq=130, num_layers=2)
    try:
        prompt = synth.prompt_tokens(p.wl, 17, 100)
        say("olmoe-width prefill of 100, then 4 greedy steps")
        tok, g_lg = p.dec.prefill(prompt, return_logits=True)
        for t in prompt:
            w_tok, w_lg = p.orc.step(int(t))
        check_step(tok, g_lg, w_tok, w_lg, "prefill")
        for i in range(4):
            feed = w_tok
            g_tok, g_lg = p.dec.forward(int(feed), return_logits=True)
            w_tok, w_lg = p.orc.step(int(feed))
            check_step(g_tok, g_lg, w_tok, w_lg, f"greedy {i} (position {100 + i})")
    finally:
        p.close()


def test_decoder_mixtral_gqa_dims_one_layer():
    """Mixtral widths (h 4096, 32 q / 8 kv heads, vocab 32000, 8 experts
    top-2, intermediate 14336), one layer, three steps."""
    p = Pair(synth.DECODERS["cfg4"], seed=5, max_seq=8, num_layers=1)
    try:
        for i, t in enumerate(synth.prompt_tokens(p.wl, 5, 3)):
            g_tok, g_lg = p.dec.forward(int(t), return_logits=True)
            w_tok, w_lg = p.orc.step(int(t))
            check_step(g_tok, g_lg, w_tok, w_lg, f"step {i}")
    finally:
        p.close()


def _greedy_against_oracle(p, tok, n, pos0, where):
    """n greedy steps, both sides fed the oracle's token; returns the logits
    relative L2 of each step and the number of steps whose greedy tokens
    differ (allowed only inside the top-2 margin, check_step)."""
    errs, differ = [], 0
    for i in range(n):
        g_tok, g_lg = p.dec.forward(int(tok), return_logits=True)
        w_tok, w_lg = p.orc.step(int(tok))
        errs.append(check_step(g_tok, g_lg, w_tok, w_lg, f"{where} step {i} (position {pos0 + i})"))
        differ += int(g_tok != w_tok)
        tok = w_tok
        if (i + 1) % 32 == 0:
            say(f"  {where}: {i + 1}/{n} greedy steps, logits rel L2 max {max(errs):.2e}")
    return errs, differ


def test_decoder_mixtral_width_long_context():
    """cfg4's regime at two of its 32 layers: Mixtral widths, a 2048-token
    batched prefill (attention over 32 chunks of 64 positions, RoPE at theta
    1e6, the grouped MoE prefill at about 512 (token, slot) pairs per
    expert), then greedy steps at positions 2048..2051 against the oracle."""
    wl = synth.DECODERS["cfg4"]
    p = Pair(wl, seed=2048, max_seq=2056, num_layers=2, nthreads=NTHREADS)
    try:
        prompt = synth.prompt_tokens(wl, 2048, 2048)
        say("mixtral-width prefill of 2048 tokens (GPU)")
        tok, g_lg = p.dec.prefill(prompt, return_logits=True)
        w_tok, w_lg = p.orc.prefill(prompt, log=say)
        pre = check_step(tok, g_lg, w_tok, w_lg, "prefill of 2048")
        assert p.dec.position() == 2048
        errs, differ = _greedy_against_oracle(p, w_tok, 4, 2048, "mixtral")
        say(f"  logits rel L2: prefill {pre:.2e}, greedy max {max(errs):.2e}, "
            f"tokens differing {differ}/4")
    finally:
        p.close()


def test_decoder_olmoe_16_layers_128_prompt_128_greedy():
    """cfg1 at full depth and length: 16 OLMoE-width layers, the 128-token
    prompt in one batch, then 128 greedy steps (positions 128..255)."""
    wl = synth.DECODERS["cfg1"]
    p = Pair(wl, seed=2026, max_seq=256, num_layers=16, nthreads=NTHREADS)
    try:
        prompt = synth.prompt_tokens(wl, 2026, 128)
        say("olmoe 16 layers: prefill of 128 tokens")
        tok, g_lg = p.dec.prefill(prompt, return_logits=True)
        w_tok, w_lg = p.orc.prefill(prompt, log=say)
        pre = check_step(tok, g_lg, w_tok, w_lg, "prefill of 128")
        errs, differ = _greedy_against_oracle(p, w_tok, 128, 128, "olmoe-16")
        say(f"[depth] layers=16 prefill {pre:.2e} greedy median {np.median(errs):.2e} "
            f"max {max(errs):.2e} tokens differing {differ}/128")
    finally:
        p.close()


@pytest.mark.parametrize("layers", [2, 8])
def test_decoder_olmoe_logit_error_by_depth(layers):
    """The same model family at 2 and 8 layers (16: the test above): 32-token
    prompt, 32 greedy steps; records how the logits error grows with depth."""
    wl = synth.DECODERS["cfg1"]
    p = Pair(wl, seed=2026, max_seq=64, num_layers=layers, nthreads=NTHREADS)
    try:
        prompt = synth.prompt_tokens(wl, 2026, 32)
        tok, g_lg = p.dec.prefill(prompt, return_logits=True)
        w_tok, w_lg = p.orc.prefill(prompt)
        pre = check_step(tok, g_lg, w_tok, w_lg, "prefill of 32")
        errs, differ = _greedy_against_oracle(p, w_tok, 32, 32, f"olmoe-{layers}")
        say(f"[depth] layers={layers} prefill {pre:.2e} greedy median {np.median(errs):.2e} "
            f"max {max(errs):.2e} tokens differing {differ}/32")
    finally:
        p.close()


def test_decoder_reports_bad_token_and_full_cache():
    p = Pair(synth.DECODERS["tiny_dec"], seed=14, max_seq=3)
    try:
        say("bad token")
        with pytest.raises(m.M1MoEError, match="vocabulary"):
            p.dec.forward(p.wl.vocab + 5)
        p.dec.reset()
        for t in (1, 2, 3):
            p.dec.forward(t)
        assert p.dec.position() == 3
        say("full cache")
        with pytest.raises(m.M1MoEError, match="KV cache full"):
            p.dec.forward(4)
        assert p.dec.position() == 3
        p.dec.reset()
        p.dec.forward(1)  # usable again after the error
        assert p.dec.position() == 1
    finally:
        p.close()


@pytest.mark.parametrize("arch", ["olmoe", "mixtral"])
def test_load_model_dir_equals_direct_upload(tmp_path, arch):
    """A converted model directory (model_weights.bin/.json + packed_experts,
    written in the converter's format with f32 norms and HF-length q/k
    norms) loaded by m1moe_load_model gives the same logits, bit for bit, as
    the same tensors uploaded directly."""
    wl = synth.DECODERS["tiny_dec"]
    synth.write_model_dir(wl, 21, str(tmp_path), architecture=arch)
    p = Pair(wl, seed=21, max_seq=16)
    ctx2 = m.HIPContext(wl.shape())
    try:
        dec2 = Decoder(ctx2, wl.dec_shape(16))
        say(f"load_model {arch}")
        ctx2.load_model(str(tmp_path), dec2, threads=4)
        for t in synth.prompt_tokens(wl, 4, 6):
            a_tok, a_lg = p.dec.forward(int(t), return_logits=True)
            b_tok, b_lg = dec2.forward(int(t), return_logits=True)
            assert a_tok == b_tok
            np.testing.assert_array_equal(a_lg, b_lg)
        # a layer file of the wrong size is rejected before anything is uploaded
        f = tmp_path / "packed_experts" / "layer_01.bin"
        f.write_bytes(f.read_bytes()[:-4])
        with pytest.raises(m.M1MoEError, match="layer_01.bin"):
            ctx2.load_model(str(tmp_path), dec2)
        dec2.close()
    finally:
        ctx2.close()
        p.close()


def test_decoder_rejects_missing_weights_and_bad_shapes():
    ctx = m.HIPContext(m.make_shape(128, 8, 2, 64, 64))
    try:
        wl = synth.DECODERS["tiny_dec"]
        dec = Decoder(ctx, wl.dec_shape(8))
        tok = ctx.to_device(np.zeros(4, np.int32))
        with pytest.raises(m.M1MoEError, match="not uploaded"):
            dec.step_device(tok, tok)
        bad = wl.dec_shape(8)
        bad.head_dim = 96
        with pytest.raises(m.M1MoEError, match="head_dim"):
            Decoder(ctx, bad)
        with pytest.raises(m.M1MoEError, match="count"):
            dec.upload(_lib.W_Q, 0, np.zeros(5, np.uint16))
        with pytest.raises(m.M1MoEError, match="n_prompt"):
            dec.step_seq(tok, 5, 4)
        dec.close()
    finally:
        ctx.close()


@pytest.mark.timeout(1200)
def test_decoder_mixtral_32_layers_2048_prompt_64_greedy():
    """cfg4 at full depth and length (Sources/bench/main.swift:133-185): 32
    Mixtral-width layers, a 2048-token prompt in one batch, then 64 greedy
    steps.  The oracle would take hours here, so the batched prefill (f16
    MFMA operands) is held against the same prompt fed token by token
    through the decode step, which the tests above pin to the oracle at
    ~1e-7: the last position's logits within 1e-2 relative L2 (the greedy
    tokens may differ only inside that margin).  Every logit is finite, and
    a second prefill-then-generate run is bit-identical."""
    wl = synth.DECODERS["cfg4"]
    L, P, G, seed = wl.num_layers, 2048, 64, 404
    shape = wl.moe.shape(L)
    say(f"cfg4 full depth: {L} layers, prompt {P}, {G} greedy steps")
    ctx = m.HIPContext(shape)
    dec = None
    try:
        dec = Decoder(ctx, wl.dec_shape(P + G + 1))
        dec.upload_all(lambda which, l: synth.dense_weight(wl, seed, which, l))
        for l in range(L):
            ctx.upload_layer_experts(l, synth.layer_image(shape, seed, l))
            ctx.upload_router(l, synth.router(shape, seed, l))
        say("  weights uploaded")
        prompt = synth.prompt_tokens(wl, seed, P)
        runs = []
        for run in range(2):
            dec.reset()
            tok, lg = dec.prefill(prompt, return_logits=True)
            toks, lgs = [tok], [lg]
            for _ in range(G):
                tok, lg = dec.forward(tok, return_logits=True)
                toks.append(tok)
                lgs.append(lg)
            assert all(np.isfinite(x).all() for x in lgs), f"run {run}: non-finite logits"
            assert dec.position() == P + G
            runs.append((toks, lgs))
            say(f"  run {run}: prefill + {G} greedy steps, tokens {toks[:6]}...")
        assert runs[0][0] == runs[1][0]
        for a, b in zip(runs[0][1], runs[1][1]):
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
        # the same prompt through the decode step, token by token
        seq = ctx.to_device(np.concatenate([prompt, np.zeros(1, np.int32)]).astype(np.int32))
        lgbuf = ctx.alloc(4 * wl.vocab)
        dec.reset()
        for i in range(P):
            dec.step_seq(seq, P, P + 1, lgbuf if i == P - 1 else None)
            if i % 512 == 511:
                ctx.sync()
                say(f"  token by token: {i + 1}/{P}")
        ctx.sync()
        step_tok = int(seq.download(np.int32)[P])
        step_lg = lgbuf.download(np.float32)
        rel = check_step(runs[0][0][0], runs[0][1][0], step_tok, step_lg,
                         "batched prefill vs token-by-token decode at position 2047")
        say(f"  last-position logits rel L2 (batched prefill vs decode steps): {rel:.3e}")
    finally:
        if dec is not None:
            dec.close()
        ctx.close()


@pytest.mark.parametrize("layers", [2, 4, 8])
def test_decoder_mixtral_width_error_against_depth(layers):
    """How the batched prefill's error grows with depth at Mixtral widths:
    a 256-token prompt through `layers` layers in one batch per layer
    against the oracle fed token by token (the last position's logits,
    then two greedy steps), each within the 1e-2 bar."""
    wl = synth.DECODERS["cfg4"]
    p = Pair(wl, seed=77, max_seq=264, num_layers=layers, nthreads=NTHREADS)
    try:
        prompt = synth.prompt_tokens(wl, 77, 256)
        say(f"mixtral width, {layers} layers: prefill of 256 tokens (GPU, then oracle)")
        tok, g_lg = p.dec.prefill(prompt, return_logits=True)
        w_tok, w_lg = p.orc.prefill(prompt)
        pre = check_step(tok, g_lg, w_tok, w_lg, f"{layers}-layer prefill of 256")
        errs, differ = _greedy_against_oracle(p, w_tok, 2, 256, f"{layers} layers")
        say(f"  depth {layers}: logits rel L2 prefill {pre:.2e}, greedy max {max(errs):.2e}")
    finally:
        p.close()
