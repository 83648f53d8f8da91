"""Pins the CPU oracle (test infrastructure) against closed forms, special
cases, invariants and brute force.  CPU only.

Each check is chosen so a plausible restatement mistake fails it: wrong
nibble order or group index, a dropped bias term, f32-vs-f64 router
accumulation, a wrong tie rule, missing renormalisation, a combine that
skips the residual or mis-weights a slot.
"""
import numpy as np
import pytest

from oracle import oracle as orc

RNG = np.random.default_rng(20261201)


def bf16_bits(a):
    """Round-to-nearest-even f32 -> bf16 bits."""
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def bf16_val(bits):
    return (np.asarray(bits, np.uint16).astype(np.uint32) << 16).view(np.float32)


def pack_like_converter(q):
    """Nibble packing of scripts/extract_olmoe.py:145-150, restated:
    column 8w+j goes to bits 4j..4j+3 of word w."""
    rows, cols = q.shape
    q8 = q.reshape(rows, cols // 8, 8).astype(np.uint32)
    packed = np.zeros((rows, cols // 8), dtype=np.uint32)
    for b in range(8):
        packed |= q8[:, :, b] << (4 * b)
    return packed


def make_block(s, rng=RNG, nib=None, scale=None, bias=None):
    """An expert block in the reference layout with optional fixed fields."""
    o = orc.offsets(s)
    blk = np.zeros(o.expert_bytes, dtype=np.uint8)
    for proj in range(3):
        rows = s.hidden if proj == 2 else s.intermediate
        cols = s.intermediate if proj == 2 else s.hidden
        g = cols // s.group_size
        q = rng.integers(0, 16, size=(rows, cols), dtype=np.uint8) if nib is None else \
            np.full((rows, cols), nib, np.uint8)
        sc = bf16_bits(np.abs(rng.normal(0, 0.02, (rows, g)))) if scale is None else \
            np.full((rows, g), bf16_bits(np.float32(scale)), np.uint16)
        bi = bf16_bits(rng.normal(0, 0.01, (rows, g))) if bias is None else \
            np.full((rows, g), bf16_bits(np.float32(bias)), np.uint16)
        w, s_, b_ = orc.proj_arrays(s, blk, proj)
        w[...] = pack_like_converter(q)
        s_[...] = sc
        b_[...] = bi
    return blk


TINY = orc.shape(128, 8, 2, 64, 64, False)


# ---- layout -------------------------------------------------------------

@pytest.mark.parametrize("h,i,gs,want", [
    (2048, 1024, 64, 3538944),     # OLMoE-1B-7B, 3.375 MiB
    (4096, 14336, 64, 99090432),   # Mixtral-8x7B, 94.5 MiB
])
def test_expert_bytes_match_modelspec(h, i, gs, want):
    # ModelSpec.swift:36-52: 2*(i*h/2 + 2*i*(h/gs)*2) + h*i/2 + 2*h*(i/gs)*2
    o = orc.offsets(orc.shape(h, 8, 2, i, gs))
    assert o.expert_bytes == want
    assert o.gate_s == i * h // 2
    assert o.up_w == i * h // 2 + 2 * i * (h // gs) * 2
    assert o.down_w == 2 * (i * h // 2 + 2 * i * (h // gs) * 2)


# ---- dequant ---------------------------------------------------------------

def test_dequant_nibble_order_and_group_index():
    s = orc.shape(128, 2, 1, 64, 32)
    blk = np.zeros(orc.offsets(s).expert_bytes, dtype=np.uint8)
    w, sc, bi = orc.proj_arrays(s, blk, 0)
    # word w holds columns 8w..8w+7; nibble j = (column % 8) + 1 mod 16 pattern
    cols = np.arange(128)
    q = np.tile(((cols % 8) + 3 * (cols // 8)) % 16, (64, 1)).astype(np.uint8)
    w[...] = pack_like_converter(q)
    # distinct power-of-two scale per group, bias = group index
    g = np.arange(128 // 32)
    sc[...] = bf16_bits(np.ldexp(1.0, -g).astype(np.float32))[None, :]
    bi[...] = bf16_bits(g.astype(np.float32))[None, :]
    W = orc.dequant_proj(s, blk, 0)
    want = q.astype(np.float32) * np.ldexp(1.0, -(cols // 32)).astype(np.float32) + (cols // 32)
    assert np.array_equal(W, want.astype(np.float32))


def test_dequant_is_single_rounding_of_exact_product():
    s = orc.shape(256, 2, 1, 128, 64)
    blk = make_block(s)
    for proj in range(3):
        W = orc.dequant_proj(s, blk, proj)
        w, sc, bi = orc.proj_arrays(s, blk, proj)
        rows, cols = W.shape
        q = np.stack([(w >> (4 * j)) & 0xF for j in range(8)], axis=-1).reshape(rows, cols)
        S = np.repeat(bf16_val(sc), s.group_size, axis=1).astype(np.float64)
        B = np.repeat(bf16_val(bi), s.group_size, axis=1).astype(np.float64)
        exact = q * S + B                   # n*s exact; the sum is rounded once
        assert np.array_equal(W, exact.astype(np.float32))


@pytest.mark.parametrize("nib", [0, 15])
def test_dequant_constant_nibbles(nib):
    s = orc.shape(128, 2, 1, 64, 64)
    blk = make_block(s, nib=nib, scale=0.25, bias=-1.5)
    W = orc.dequant_proj(s, blk, 1)
    assert np.all(W == np.float32(nib * 0.25 - 1.5))


# ---- matvec --------------------------------------------------------------

@pytest.mark.parametrize("lanes", [False, True])
def test_matvec_integer_special_case_is_exact(lanes):
    # s = 1, b = 0, small integer x: an integer matvec, exact in f32
    s = orc.shape(2048, 2, 1, 64, 64)
    blk = make_block(s, scale=1.0, bias=0.0)
    w, sc, bi = orc.proj_arrays(s, blk, 0)
    x = RNG.integers(-3, 4, size=2048).astype(np.float32)
    q = np.stack([(w >> (4 * j)) & 0xF for j in range(8)], axis=-1).reshape(64, 2048)
    want = (q.astype(np.int64) @ x.astype(np.int64)).astype(np.float32)
    got = orc.matvec4bit(w, sc, bi, x, 64, 2048, 64, lanes=lanes)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("lanes", [False, True])
def test_matvec_all_zero_nibbles_reduces_to_bias_times_group_sums(lanes):
    s = orc.shape(1024, 2, 1, 64, 64)
    blk = make_block(s, nib=0)
    w, sc, bi = orc.proj_arrays(s, blk, 0)
    x = RNG.normal(size=1024).astype(np.float32)
    gsum = x.astype(np.float64).reshape(16, 64).sum(axis=1)
    want = bf16_val(bi).astype(np.float64) @ gsum
    got = orc.matvec4bit(w, sc, bi, x, 64, 1024, 64, lanes=lanes)
    assert np.allclose(got, want, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("gs", [32, 64, 128])
def test_matvec_matches_f64_brute_force(gs):
    s = orc.shape(512, 2, 1, 256, gs)
    blk = make_block(s)
    for proj in range(3):
        w, sc, bi = orc.proj_arrays(s, blk, proj)
        rows, cols = w.shape[0], w.shape[1] * 8
        q = np.stack([(w >> (4 * j)) & 0xF for j in range(8)], axis=-1).reshape(rows, cols)
        W = q * np.repeat(bf16_val(sc), gs, axis=1).astype(np.float64) + \
            np.repeat(bf16_val(bi), gs, axis=1).astype(np.float64)   # unrounded weights
        x = RNG.normal(size=cols).astype(np.float32)
        want = W @ x.astype(np.float64)
        got = orc.matvec4bit(w, sc, bi, x, rows, cols, gs, lanes=True)
        got64 = orc.matvec4bit_f64(w, sc, bi, x, rows, cols, gs)
        assert np.allclose(got64, want, rtol=1e-12, atol=1e-12)
        assert np.linalg.norm(got - want) / np.linalg.norm(want) < 1e-6


@pytest.mark.parametrize("cols,gs", [(64, 32), (128, 64), (576, 64), (1024, 32), (2048, 128),
                                     (14336, 64)])
def test_matvec_vector_form_equals_lanes_bit_for_bit(cols, gs):
    """The eight-lanes-at-a-time form against the lane-by-lane restatement:
    fewer words than lanes (64, 128 columns), a partial last stride (576),
    two scale groups per eight words (gs 32), the Mixtral down row (14336).
    x spans 2^-20..2^20 so any change of operation order changes bits."""
    rows = 96
    w = RNG.integers(0, 2**32, size=(rows, cols // 8), dtype=np.uint64).astype(np.uint32)
    sc = (RNG.normal(size=(rows, cols // gs)).astype(np.float32).view(np.uint32) >> 16) \
        .astype(np.uint16)
    bi = (RNG.normal(size=(rows, cols // gs)).astype(np.float32).view(np.uint32) >> 16) \
        .astype(np.uint16)
    x = (RNG.normal(size=cols) * 2.0 ** RNG.integers(-20, 21, size=cols)).astype(np.float32)
    a = orc.matvec4bit(w, sc, bi, x, rows, cols, gs)
    b = orc.matvec4bit(w, sc, bi, x, rows, cols, gs, lanes=True)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


# ---- SwiGLU ------------------------------------------------------------------

def test_swiglu_against_f64_libm():
    g = np.concatenate([RNG.normal(0, 4, 4096), [0.0, -0.0, 80.0, -80.0, 1e-30]]).astype(np.float32)
    u = RNG.normal(0, 2, g.size).astype(np.float32)
    got = orc.swiglu(g, u)
    g64 = g.astype(np.float64)
    want = g64 / (1.0 + np.exp(-g64)) * u.astype(np.float64)
    assert np.allclose(got, want, rtol=4e-7, atol=1e-30)


# ---- router ----------------------------------------------------------------

def test_router_logits_are_rounded_exact_sums():
    E, h = 64, 2048
    r = bf16_bits(RNG.normal(0, 0.02, (E, h)))
    x = RNG.normal(size=h).astype(np.float32)
    got = orc.router_logits(r, x)
    # exact rational sum via Python integers (bf16 x f32 products are dyadic)
    from fractions import Fraction
    W = bf16_val(r)
    for e in range(0, E, 9):
        exact = sum(Fraction(float(a)) * Fraction(float(b)) for a, b in zip(W[e], x))
        nearest = np.float32(float(exact))   # float(Fraction) rounds correctly to f64
        assert abs(float(got[e]) - float(nearest)) <= float(np.spacing(np.float32(abs(nearest))))


def test_router_one_hot_input_selects_a_column():
    E, h = 16, 256
    r = bf16_bits(RNG.normal(0, 0.02, (E, h)))
    x = np.zeros(h, np.float32)
    x[37] = 1.0
    assert np.array_equal(orc.router_logits(r, x), bf16_val(r[:, 37]))
    assert np.array_equal(orc.router_logits(r, x, seq_f32=True), bf16_val(r[:, 37]))


def test_router_seq_f32_differs_from_f64_only_in_low_bits():
    E, h = 64, 2048
    r = bf16_bits(RNG.normal(0, 0.02, (E, h)))
    x = RNG.normal(size=h).astype(np.float32)
    a = orc.router_logits(r, x)
    b = orc.router_logits(r, x, seq_f32=True)
    assert np.allclose(a, b, rtol=0, atol=1e-4)


def test_softmax_sums_to_one_and_matches_f64():
    lg = RNG.normal(0, 1, 64).astype(np.float32)
    p = orc.softmax(lg)
    l64 = lg.astype(np.float64)
    want = np.exp(l64 - l64.max())
    want /= want.sum()
    assert abs(p.astype(np.float64).sum() - 1.0) < 1e-6
    assert np.allclose(p, want, rtol=2e-6)


def test_topk_equals_stable_sort_and_ties_go_low():
    for trial in range(200):
        E, K = 64, 8
        lg = RNG.normal(0, 1, E).astype(np.float32)
        if trial % 2:
            lg[RNG.integers(0, E, 10)] = lg[3]   # engineered exact ties
        p = orc.softmax(lg)
        idx, w = orc.select_topk(lg, p, K, False)
        want = np.argsort(-lg.astype(np.float64), kind="stable")[:K]
        assert np.array_equal(idx, want)
        assert np.array_equal(w, p[want])


def test_topk_by_logit_equals_reference_prob_order_on_random_inputs():
    for _ in range(300):
        lg = RNG.normal(0, 1, 64).astype(np.float32)
        p = orc.softmax(lg)
        a, _ = orc.select_topk(lg, p, 8, False, orc.KEY_LOGIT)
        b, _ = orc.select_topk(lg, p, 8, False, orc.KEY_PROB)
        assert np.array_equal(a, b)


def test_topk_documented_divergence_on_probability_ties():
    # two distinct logits one f32 ulp apart whose probabilities round equal:
    # the reference's stable probability sort keeps index order (1 before 2),
    # the logit key puts the larger logit (index 2) first
    lg = np.zeros(4, np.float32)
    lg[0] = 5.0
    lg[1] = 1.0
    lg[2] = np.nextafter(np.float32(1.0), np.float32(2.0))
    p = orc.softmax(lg)
    assert p[1] == p[2] and lg[2] > lg[1]
    by_logit, _ = orc.select_topk(lg, p, 3, False, orc.KEY_LOGIT)
    by_prob, _ = orc.select_topk(lg, p, 3, False, orc.KEY_PROB)
    assert list(by_logit) == [0, 2, 1]
    assert list(by_prob) == [0, 1, 2]


def test_topk_k_equals_e_is_a_permutation():
    lg = RNG.normal(0, 1, 16).astype(np.float32)
    idx, _ = orc.select_topk(lg, orc.softmax(lg), 16, False)
    assert sorted(idx.tolist()) == list(range(16))


def test_topk_renormalisation():
    lg = RNG.normal(0, 1, 8).astype(np.float32)
    p = orc.softmax(lg)
    idx, w = orc.select_topk(lg, p, 2, True)
    assert abs(float(w.sum()) - 1.0) < 1e-6
    sel = lg[idx].astype(np.float64)
    want = np.exp(sel - sel.max())
    want /= want.sum()      # softmax over only the selected logits
    assert np.allclose(w, want, rtol=1e-6)
    _, w0 = orc.select_topk(lg, p, 2, False)
    assert np.allclose(w0, p[idx]) and w0.sum() < 1.0


# ---- combine -----------------------------------------------------------------

def test_combine_single_slot_unit_weight_is_expert_plus_residual():
    eo = RNG.normal(size=(1, 256)).astype(np.float32)
    res = RNG.normal(size=256).astype(np.float32)
    assert np.array_equal(orc.combine(eo, np.ones(1, np.float32), res), eo[0] + res)
    assert np.array_equal(orc.combine(eo, np.ones(1, np.float32), None), eo[0])


def test_combine_is_linear_in_weights():
    eo = RNG.normal(size=(4, 512)).astype(np.float32)
    w = RNG.random(4).astype(np.float32)
    res = RNG.normal(size=512).astype(np.float32)
    got = orc.combine(eo, w, res).astype(np.float64)
    want = res.astype(np.float64) + w.astype(np.float64) @ eo.astype(np.float64)
    assert np.allclose(got, want, rtol=1e-5, atol=1e-5)
    assert np.array_equal(orc.combine(eo, np.zeros(4, np.float32), res), res)


# ---- composed block ------------------------------------------------------------

def _f64_expert(s, blk, x):
    def mv(proj, v):
        return orc.dequant_proj(s, blk, proj).astype(np.float64) @ v
    g, u = mv(0, x), mv(1, x)
    act = g / (1 + np.exp(-g)) * u
    return mv(2, act)


def test_expert_forward_matches_f64_composition():
    s = orc.shape(256, 4, 2, 128, 64)
    blk = make_block(s)
    x = RNG.normal(size=256).astype(np.float32)
    got = orc.expert_forward(s, blk, x)
    want = _f64_expert(s, blk, x.astype(np.float64))
    assert np.linalg.norm(got - want) / np.linalg.norm(want) < 1e-5


@pytest.mark.parametrize("norm", [False, True])
def test_moe_decode_matches_f64_composition(norm):
    s = orc.shape(256, 8, 3, 128, 64, norm)
    o = orc.offsets(s)
    img = np.concatenate([make_block(s) for _ in range(8)])
    r = bf16_bits(RNG.normal(0, 0.05, (8, 256)))
    x = RNG.normal(size=256).astype(np.float32)
    res = RNG.normal(size=256).astype(np.float32)
    out, idx, w, lg = orc.moe_decode(s, img, r, x, res)
    # f64 composition: logits, stable top-K, softmax weights, combine
    l64 = bf16_val(r).astype(np.float64) @ x.astype(np.float64)
    sel = np.argsort(-l64, kind="stable")[:3]
    assert np.array_equal(idx, sel)
    p = np.exp(l64 - l64.max())
    p /= p.sum()
    ww = p[sel] / p[sel].sum() if norm else p[sel]
    assert np.allclose(w, ww, rtol=1e-5)
    want = res.astype(np.float64)
    for k, e in enumerate(sel):
        want = want + ww[k] * _f64_expert(s, img[e * o.expert_bytes:(e + 1) * o.expert_bytes],
                                          x.astype(np.float64))
    assert np.linalg.norm(out - want) / np.linalg.norm(want) < 1e-5


def test_logit_bias_shifts_selection():
    s = orc.shape(128, 8, 2, 64, 64)
    img = np.concatenate([make_block(s) for _ in range(8)])
    r = bf16_bits(RNG.normal(0, 0.02, (8, 128)))
    x = RNG.normal(size=128).astype(np.float32)
    bias = np.full(8, -100.0, np.float32)
    bias[[6, 3]] = 0.0
    _, idx, _, lg = orc.moe_decode(s, img, r, x, None, logit_bias=bias)
    assert sorted(idx.tolist()) == [3, 6]
    assert np.array_equal(lg, orc.router_logits(r, x) + bias)


def test_prefill_threads_equal_per_token_decode():
    s = orc.shape(128, 8, 2, 64, 64)
    img = np.concatenate([make_block(s) for _ in range(8)])
    r = bf16_bits(RNG.normal(0, 0.02, (8, 128)))
    X = RNG.normal(size=(9, 128)).astype(np.float32)
    out, idx, w = orc.moe_prefill(s, img, r, X, None, None, nthreads=4)
    for t in range(9):
        o1, i1, w1, _ = orc.moe_decode(s, img, r, X[t])
        assert np.array_equal(out[t], o1) and np.array_equal(idx[t], i1)
        assert np.array_equal(w[t], w1)


def test_given_topk_rejects_out_of_range_expert():
    s = TINY
    img = np.concatenate([make_block(s) for _ in range(8)])
    with pytest.raises(ValueError):
        orc.moe_decode_given_topk(s, img, np.zeros(128, np.float32), np.array([0, 8], np.int32),
                                  np.ones(2, np.float32))
