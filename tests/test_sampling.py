"""Host-side sampling (m1moe_amd/sampling.py) against a literal restatement
of sampleToken (InferenceEngine.swift:550-575) on small vocabularies, and
against its distribution.  CPU only."""
import numpy as np
import pytest

from m1moe_amd.sampling import greedy, sample_token

RNG = np.random.default_rng(99)


def sample_literal(logits, temperature, top_p, u):
    """The reference's loops one by one in f32 (small vocabularies only)."""
    f = np.float32
    if temperature <= 0:
        best, bv = 0, f(logits[0])
        for i in range(1, len(logits)):
            if f(logits[i]) > bv:
                bv, best = f(logits[i]), i
        return best
    mx = f(logits[0])
    for i in range(1, len(logits)):
        if f(logits[i]) > mx:
            mx = f(logits[i])
    probs, s = [], f(0)
    for v in logits:
        e = f(np.exp(f((f(v) - mx) / f(temperature))))
        probs.append(e)
        s = f(s + e)
    inv = f(f(1.0) / s)
    probs = [f(p * inv) for p in probs]
    order = sorted(range(len(probs)), key=lambda i: (-probs[i], i))
    cumul, nucleus = f(0), []
    for i in order:
        nucleus.append(i)
        cumul = f(cumul + probs[i])
        if cumul >= f(top_p):
            break
    ns = f(0)
    for i in nucleus:
        ns = f(ns + probs[i])
    r = f(f(u) * ns)
    for i in nucleus:
        r = f(r - probs[i])
        if r <= 0:
            return i
    return nucleus[-1]


@pytest.mark.parametrize("n,temp,top_p", [(7, 0.7, 0.9), (50, 1.0, 1.0), (50, 0.3, 0.5),
                                          (200, 1.5, 0.95), (13, 2.0, 0.0)])
def test_matches_the_literal_restatement(n, temp, top_p):
    for _ in range(200):
        logits = RNG.normal(0, 2, n).astype(np.float32)
        if RNG.random() < 0.3:
            logits[RNG.integers(0, n, 3)] = logits.max()  # ties at the top
        u = float(RNG.random(dtype=np.float32))
        assert sample_token(logits, temp, top_p, u=u) == sample_literal(logits, temp, top_p, u)


def test_greedy_at_zero_temperature_and_nan_rules():
    x = np.array([1, 5, 5, 2], np.float32)
    assert sample_token(x, 0.0, 0.9) == 1 == sample_literal(x, 0.0, 0.9, 0.5)
    assert greedy(np.array([np.nan, 3, 4], np.float32)) == 0
    assert greedy(np.array([1, np.nan, 4, np.nan], np.float32)) == 2


def test_tiny_top_p_is_the_most_probable_token():
    for _ in range(50):
        logits = RNG.normal(0, 1, 100).astype(np.float32)
        for u in (0.0, 0.5, 0.999):
            assert sample_token(logits, 0.8, 1e-9, u=u) == int(np.argmax(logits))


def test_frequencies_follow_the_tempered_softmax():
    logits = np.array([0.0, 1.0, 2.0, -1.0, 0.5], np.float32)
    temp = 1.3
    p = np.exp(logits / temp)
    p /= p.sum()
    rng = np.random.default_rng(7)
    n = 40000
    counts = np.bincount([sample_token(logits, temp, 1.0, rng=rng) for _ in range(n)], minlength=5)
    chi2 = float((((counts - n * p) ** 2) / (n * p)).sum())
    assert chi2 < 25.0, (counts, n * p)  # 4 degrees of freedom: p(chi2 > 25) ~ 5e-5


def test_nucleus_excludes_the_tail():
    logits = np.array([5.0, 4.9, 0.0, -1.0, -2.0], np.float32)
    rng = np.random.default_rng(3)
    seen = {sample_token(logits, 1.0, 0.9, rng=rng) for _ in range(2000)}
    assert seen <= {0, 1}
