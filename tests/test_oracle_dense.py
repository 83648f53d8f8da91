"""Pins the dense decoder-step functions of the CPU oracle (test
infrastructure) against closed forms, invariants, library routines and an
independent whole-sequence formulation.  CPU only.

Each check is chosen so a plausible restatement mistake fails it: a dropped
norm weight or epsilon, a mean over the wrong length, the wrong RoPE pairing
(interleaved instead of half-split) or frequency exponent, a position off by
one, a GQA head mapping h % n_kv instead of h / hpkv, a missing 1/sqrt(d)
scale, the softmax over a cache row that includes unwritten positions, a tie
broken to the higher index, a residual dropped around attention or the MoE
block.
"""
import numpy as np
import pytest
from scipy.special import softmax

from oracle import oracle as orc

RNG = np.random.default_rng(20261202)


def bf16_bits(a):
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def bf16_val(bits):
    return (np.asarray(bits, np.uint16).astype(np.uint32) << 16).view(np.float32)


ONES = lambda n: np.full(n, 0x3F80, np.uint16)  # bf16 1.0


# ---- embedding -----------------------------------------------------------------------

def test_embed_is_the_exact_row():
    table = bf16_bits(RNG.normal(0, 1, (37, 64)))
    for t in (0, 5, 36):
        np.testing.assert_array_equal(orc.embed(table, t), bf16_val(table[t]))


# ---- RMSNorm -------------------------------------------------------------------------

def test_rmsnorm_constant_vector_closed_form():
    n, c, eps = 512, 3.0, 1e-5
    w = bf16_bits(RNG.normal(1, 0.1, n))
    out = orc.rmsnorm(np.full(n, c, np.float32), w, eps)
    want = c / np.sqrt(c * c + eps) * bf16_val(w).astype(np.float64)
    np.testing.assert_allclose(out, want, rtol=2e-7)


def test_rmsnorm_unit_rms_and_scale_invariance():
    n = 2048
    x = RNG.normal(0, 5, n).astype(np.float32)
    out = orc.rmsnorm(x, ONES(n), 0.0)
    assert abs(np.sqrt(np.mean(out.astype(np.float64) ** 2)) - 1.0) < 1e-6
    out2 = orc.rmsnorm(x * np.float32(8.0), ONES(n), 0.0)  # exact power-of-two scale
    np.testing.assert_array_equal(out, out2)


def test_rmsnorm_epsilon_and_weight_enter():
    n = 256
    x = np.full(n, 1e-3, np.float32)
    # eps dominates: out = 1e-3 / sqrt(1e-6 + 1e-2) * w
    w = bf16_bits(np.linspace(0.5, 2, n))
    out = orc.rmsnorm(x, w, 1e-2)
    np.testing.assert_allclose(out, 1e-3 / np.sqrt(1e-6 + 1e-2) * bf16_val(w), rtol=2e-6)


# ---- bf16 matvec ---------------------------------------------------------------------

@pytest.mark.parametrize("rows,cols", [(1, 8), (37, 200), (128, 2048)])
def test_matvec_bf16_against_numpy(rows, cols):
    w = bf16_bits(RNG.normal(0, 1, (rows, cols)))
    x = RNG.normal(0, 1, cols).astype(np.float32)
    r = RNG.normal(0, 1, rows).astype(np.float32)
    want = bf16_val(w).astype(np.float64) @ x.astype(np.float64)
    np.testing.assert_allclose(orc.matvec_bf16(w, x), want, rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(orc.matvec_bf16(w, x, residual=r), want + r, rtol=1e-6,
                               atol=1e-5)


def test_matvec_bf16_identity_picks_columns():
    n = 64
    w = bf16_bits(np.eye(n)[::-1])  # anti-diagonal: y = reversed x
    x = bf16_val(bf16_bits(RNG.normal(0, 1, n)))
    np.testing.assert_array_equal(orc.matvec_bf16(w, x), x[::-1])


# ---- per-head q/k RMSNorm --------------------------------------------------------------

def test_head_rmsnorm_each_head_unit_rms_and_independent():
    nh, hd = 4, 64
    x = (RNG.normal(0, 1, nh * hd) * np.repeat([0.1, 1, 10, 100], hd)).astype(np.float32)
    w = bf16_bits(RNG.normal(1, 0.2, hd))
    out = orc.head_rmsnorm(x, nh, hd, w, 0.0).reshape(nh, hd)
    unweighted = out / bf16_val(w)  # every head shares the head_dim-long weight
    np.testing.assert_allclose(np.sqrt(np.mean(unweighted.astype(np.float64) ** 2, 1)), 1.0,
                               rtol=1e-5)
    x2 = x.copy()
    x2[:hd] *= 3  # head 0 changed: the other heads are not
    out2 = orc.head_rmsnorm(x2, nh, hd, w, 0.0).reshape(nh, hd)
    np.testing.assert_array_equal(out[1:], out2[1:])


# ---- RoPE ----------------------------------------------------------------------------

def rope_complex(x, nh, hd, theta, pos):
    """Half-split RoPE as a complex rotation of (x[p], x[p+hd/2]) by pos*theta^(-2p/hd)."""
    half = hd // 2
    v = x.reshape(nh, hd).astype(np.float64)
    z = v[:, :half] + 1j * v[:, half:]
    ang = pos * theta ** (-2.0 * np.arange(half) / hd)
    z = z * np.exp(1j * ang)
    return np.concatenate([z.real, z.imag], 1).reshape(-1)


def test_rope_position_zero_is_identity():
    x = RNG.normal(0, 1, 3 * 128).astype(np.float32)
    np.testing.assert_array_equal(orc.rope(x, 3, 128, 10000.0, 0), x)


@pytest.mark.parametrize("pos", [1, 7, 300, 4095])
def test_rope_matches_complex_rotation(pos):
    nh, hd, theta = 2, 128, 10000.0
    x = RNG.normal(0, 1, nh * hd).astype(np.float32)
    got = orc.rope(x, nh, hd, theta, pos)
    # the f32 angle pos*freq carries ~pos*2^-24 rad of rounding
    np.testing.assert_allclose(got, rope_complex(x, nh, hd, theta, pos),
                               atol=4e-6 * max(1, pos) ** 0.5 + 2e-6 * pos / 64)


def test_rope_relative_position_property():
    hd, theta = 64, 500.0
    q = RNG.normal(0, 1, hd).astype(np.float32)
    k = RNG.normal(0, 1, hd).astype(np.float32)
    d1 = np.dot(orc.rope(q, 1, hd, theta, 10).astype(np.float64),
                orc.rope(k, 1, hd, theta, 3))
    d2 = np.dot(orc.rope(q, 1, hd, theta, 27).astype(np.float64),
                orc.rope(k, 1, hd, theta, 20))
    assert abs(d1 - d2) < 1e-4 * np.linalg.norm(q) * np.linalg.norm(k)


# ---- attention -----------------------------------------------------------------------

def attention_softmax_ref(q, kc, vc, nh, nkv, hd, sl):
    """Scores for all heads as one matrix product, softmax from scipy."""
    hpkv = nh // nkv
    Q = q.reshape(nh, hd).astype(np.float64)
    K = kc[:sl].reshape(sl, nkv, hd).astype(np.float64)
    V = vc[:sl].reshape(sl, nkv, hd).astype(np.float64)
    kvh = np.arange(nh) // hpkv
    S = np.einsum("hd,phd->hp", Q, K[:, kvh, :]) / np.sqrt(hd)
    P = softmax(S, axis=1)
    return np.einsum("hp,phd->hd", P, V[:, kvh, :]).reshape(-1)


@pytest.mark.parametrize("nh,nkv,hd,sl", [(4, 4, 64, 1), (4, 2, 64, 17), (8, 2, 128, 300),
                                           (2, 1, 256, 5)])
def test_attention_against_softmax_library(nh, nkv, hd, sl):
    kvd = nkv * hd
    q = RNG.normal(0, 1, nh * hd).astype(np.float32)
    kc = RNG.normal(0, 1, (sl + 3, kvd)).astype(np.float32)  # rows past sl must be ignored
    vc = RNG.normal(0, 1, (sl + 3, kvd)).astype(np.float32)
    kc[sl:] = 1e4
    vc[sl:] = np.nan
    got = orc.attention(q, kc, vc, nh, nkv, hd, sl)
    np.testing.assert_allclose(got, attention_softmax_ref(q, kc, vc, nh, nkv, hd, sl),
                               rtol=1e-5, atol=1e-6)


def test_attention_single_position_returns_v_of_its_kv_head():
    nh, nkv, hd = 8, 2, 64
    q = RNG.normal(0, 1, nh * hd).astype(np.float32)
    kc = RNG.normal(0, 1, (1, nkv * hd)).astype(np.float32)
    vc = RNG.normal(0, 1, (1, nkv * hd)).astype(np.float32)
    out = orc.attention(q, kc, vc, nh, nkv, hd, 1).reshape(nh, hd)
    for h in range(nh):  # heads 0..3 read kv head 0, heads 4..7 kv head 1
        np.testing.assert_array_equal(out[h], vc[0, (h // 4) * hd:(h // 4 + 1) * hd])


def test_attention_equal_keys_average_values():
    nh, hd, sl = 2, 64, 9
    q = RNG.normal(0, 1, nh * hd).astype(np.float32)
    kc = np.tile(RNG.normal(0, 1, (1, nh * hd)).astype(np.float32), (sl, 1))
    vc = RNG.normal(0, 1, (sl, nh * hd)).astype(np.float32)
    np.testing.assert_allclose(orc.attention(q, kc, vc, nh, nh, hd, sl), vc.mean(0), rtol=1e-5,
                               atol=1e-6)


# ---- greedy argmax --------------------------------------------------------------------

def test_argmax_ties_go_to_the_lower_index():
    x = np.array([0, 5, 1, 5, 5], np.float32)
    assert orc.argmax(x) == 1
    assert orc.argmax(np.full(10, -np.inf, np.float32)) == 0


def test_argmax_nan_semantics_of_the_strict_scan():
    assert orc.argmax(np.array([np.nan, 1, 2], np.float32)) == 0
    assert orc.argmax(np.array([1, np.nan, 2, np.nan], np.float32)) == 2


def test_argmax_matches_numpy_on_random():
    for _ in range(20):
        x = RNG.normal(0, 1, 50304).astype(np.float32)
        assert orc.argmax(x) == int(np.argmax(x))


# ---- the whole decoder: incremental with a KV cache == whole-sequence causal ----------

TINY_MOE = orc.shape(128, 8, 2, 64, 64, False)


def tiny_decoder(seed=5, qk_norm=True, nh=2, nkv=1, hd=64, L=2, vocab=97):
    rng = np.random.default_rng(seed)
    h = TINY_MOE.hidden
    qd, kvd = nh * hd, nkv * hd
    mat = lambda r, c: bf16_bits(rng.normal(0, 1 / np.sqrt(c), (r, c)))
    vec = lambda n: bf16_bits(rng.normal(1, 0.1, n))
    t = {"embed": bf16_bits(rng.normal(0, 1, (vocab, h))), "lm_head": mat(vocab, h),
         "final_norm": vec(h), "in_norm": [vec(h) for _ in range(L)],
         "post_norm": [vec(h) for _ in range(L)], "q": [mat(qd, h) for _ in range(L)],
         "k": [mat(kvd, h) for _ in range(L)], "v": [mat(kvd, h) for _ in range(L)],
         "o": [mat(h, qd) for _ in range(L)], "q_norm": [vec(hd) for _ in range(L)],
         "k_norm": [vec(hd) for _ in range(L)]}
    from test_oracle import make_block
    o = orc.offsets(TINY_MOE)
    images = [np.concatenate([make_block(TINY_MOE, rng) for _ in range(TINY_MOE.num_experts)])
              for _ in range(L)]
    assert images[0].size == TINY_MOE.num_experts * o.expert_bytes
    routers = [bf16_bits(rng.normal(0, 0.02, (TINY_MOE.num_experts, h))) for _ in range(L)]
    return t, images, routers, dict(nh=nh, nkv=nkv, hd=hd, L=L, vocab=vocab, qk_norm=qk_norm)


def whole_sequence_logits(t, images, routers, cfg, tokens, theta, eps):
    """All positions at once: [T x h] activations, causal-masked attention
    over the full sequence, RoPE as complex rotations, MoE through the
    oracle's T-token entry.  Returns logits [T x vocab]."""
    nh, nkv, hd, L = cfg["nh"], cfg["nkv"], cfg["hd"], cfg["L"]
    T = len(tokens)
    f = lambda b: bf16_val(b).astype(np.float64)

    def norm(X, w):
        return X / np.sqrt(np.mean(X * X, -1, keepdims=True) + eps) * f(w)

    def head_norm(X, w, n):
        Y = X.reshape(T, n, hd)
        return (Y / np.sqrt(np.mean(Y * Y, -1, keepdims=True) + eps) * f(w)).reshape(T, -1)

    X = f(t["embed"])[tokens]
    mask = np.tril(np.ones((T, T), bool))
    caches = []
    for layer in range(L):
        Xn = norm(X, t["in_norm"][layer])
        Q, K, V = (Xn @ f(t[n][layer]).T for n in ("q", "k", "v"))
        if cfg["qk_norm"]:
            Q, K = head_norm(Q, t["q_norm"][layer], nh), head_norm(K, t["k_norm"][layer], nkv)
        Q = np.stack([rope_complex(Q[p], nh, hd, theta, p) for p in range(T)])
        K = np.stack([rope_complex(K[p], nkv, hd, theta, p) for p in range(T)])
        caches.append((K, V))
        kvh = np.arange(nh) // (nh // nkv)
        Qh, Kh, Vh = Q.reshape(T, nh, hd), K.reshape(T, nkv, hd)[:, kvh], V.reshape(T, nkv, hd)[:, kvh]
        S = np.einsum("qhd,khd->hqk", Qh, Kh) / np.sqrt(hd)
        S = np.where(mask[None], S, -np.inf)
        A = np.einsum("hqk,khd->qhd", softmax(S, axis=-1), Vh).reshape(T, nh * hd)
        X2 = X + A @ f(t["o"][layer]).T
        Hm = norm(X2, t["post_norm"][layer])
        X, _, _ = orc.moe_prefill(TINY_MOE, images[layer], routers[layer],
                                  Hm.astype(np.float32), residual=X2.astype(np.float32))
        X = X.astype(np.float64)
    return norm(X, t["final_norm"]) @ f(t["lm_head"]).T, caches


@pytest.mark.parametrize("qk_norm,nh,nkv", [(True, 2, 1), (False, 4, 2)])
def test_decoder_incremental_equals_whole_sequence(qk_norm, nh, nkv):
    theta, eps = 10000.0, 1e-5
    t, images, routers, cfg = tiny_decoder(qk_norm=qk_norm, nh=nh, nkv=nkv)
    tokens = np.random.default_rng(9).integers(0, cfg["vocab"], 12)
    dec = orc.DecoderOracle(TINY_MOE, cfg["L"], cfg["vocab"], nh, nkv, cfg["hd"], 16, qk_norm,
                            theta, eps, t, images, routers)
    inc = np.stack([dec.step(int(tok))[1] for tok in tokens])
    whole, caches = whole_sequence_logits(t, images, routers, cfg, tokens, theta, eps)
    rel = np.linalg.norm(inc - whole) / np.linalg.norm(whole)
    assert rel < 1e-4, rel
    # the cache rows themselves: RoPE at the absolute position (a uniform
    # position offset would leave the logits unchanged)
    T = len(tokens)
    for layer, (K, V) in enumerate(caches):
        np.testing.assert_allclose(dec.kc[layer, :T], K, rtol=1e-4, atol=1e-4)
        np.testing.assert_allclose(dec.vc[layer, :T], V, rtol=1e-4, atol=1e-4)
    # the greedy token is the argmax of those logits
    dec.reset()
    for p, tok in enumerate(tokens[:4]):
        nxt, lg = dec.step(int(tok))
        assert nxt == int(np.argmax(lg))
    assert dec.pos == 4


@pytest.mark.parametrize("qk_norm,nh,nkv", [(True, 2, 1), (False, 4, 2)])
def test_decoder_threads_and_prefill_equal_single_thread_steps(qk_norm, nh, nkv):
    """Threaded steps (rows of every matvec and the selected experts on four
    threads) and the batched prefill (tokens of a layer on four threads)
    produce step()'s bits: logits, greedy tokens and every cache row."""
    theta, eps = 10000.0, 1e-5
    t, images, routers, cfg = tiny_decoder(qk_norm=qk_norm, nh=nh, nkv=nkv)
    tokens = [int(v) for v in np.random.default_rng(11).integers(0, cfg["vocab"], 10)]

    def make(n):
        d = orc.DecoderOracle(TINY_MOE, cfg["L"], cfg["vocab"], nh, nkv, cfg["hd"], 16, qk_norm,
                              theta, eps, t, images, routers, nthreads=n)
        d.split_min = 0
        return d
    one, four, pre = make(1), make(4), make(4)
    try:
        for tok in tokens[:7]:
            a, b = one.step(tok), four.step(tok)
            assert a[0] == b[0] and np.array_equal(a[1].view(np.uint32), b[1].view(np.uint32))
        c = pre.prefill(tokens[:7])
        assert c[0] == a[0] and np.array_equal(c[1].view(np.uint32), a[1].view(np.uint32))
        assert pre.pos == one.pos == 7
        assert np.array_equal(pre.kc.view(np.uint32), one.kc.view(np.uint32))
        assert np.array_equal(pre.vc.view(np.uint32), one.vc.view(np.uint32))
        # a second piece from position 7, then a step
        c = pre.prefill(tokens[7:])
        for tok in tokens[7:]:
            a = one.step(tok)
        assert c[0] == a[0] and np.array_equal(c[1].view(np.uint32), a[1].view(np.uint32))
        a, c = one.step(tokens[0]), pre.step(tokens[0])
        assert np.array_equal(c[1].view(np.uint32), a[1].view(np.uint32))
        with pytest.raises(ValueError):
            pre.prefill(list(range(6)))            # 11 + 6 > 16 positions
    finally:
        four.close()
        pre.close()
