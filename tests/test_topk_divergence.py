"""How often the reference's own routing order picks a different expert than
the pinned one, on the seeded workload inputs.

The reference sums the router logits sequentially in f32
(InferenceEngine.swift:495-500) and ranks experts by softmax probability with
a stable sort (:510-519).  The pinned semantics (oracle and GPU) sum exact
products in f64, round once, and rank by logit with ties to the lower index.
The two agree except where two of the top-(K+1) logits are closer than the
f32 summation error (or round to the same probability).  These tests count
the disagreements over the seeded cfg0, cfg2 and cfg3 token sets (the same
inputs bench.py and the GPU tests draw) and over a larger random sample at
the cfg0 shape, and record the smallest K-th/(K+1)-th logit gap seen.
"""
import numpy as np

from m1moe_amd import synth
from oracle import oracle as orc


def _divergence(name, seed, layers, tokens, extra_random=0):
    wl = synth.CONFIGS[name]
    shape = wl.shape(max(layers, 1))
    K, E = shape.top_k, shape.num_experts
    norm = bool(shape.norm_topk_prob)
    bias = synth.zipf_logit_bias(E, wl.zipf_s) if wl.zipf_s else None
    xs = synth.bf16_to_f32(synth.activations_bf16(shape, seed, layers * tokens))
    rng = np.random.default_rng(seed)
    stats = dict(n=0, sets=0, order=0, max_logit_diff=0.0, min_gap=np.inf)

    def one(router, x):
        a = orc.router_logits(router, x)                 # pinned: f64 sum, one rounding
        b = orc.router_logits(router, x, seq_f32=True)   # reference: sequential f32
        if bias is not None:
            a = (a + bias).astype(np.float32)
            b = (b + bias).astype(np.float32)
        ia, _ = orc.select_topk(a, orc.softmax(a), K, norm, orc.KEY_LOGIT)
        ib, _ = orc.select_topk(b, orc.softmax(b), K, norm, orc.KEY_PROB)
        stats["n"] += 1
        stats["sets"] += int(set(ia.tolist()) != set(ib.tolist()))
        stats["order"] += int(not np.array_equal(ia, ib))
        stats["max_logit_diff"] = max(stats["max_logit_diff"], float(np.max(np.abs(a - b))))
        if K < E:
            srt = np.sort(a)[::-1]
            stats["min_gap"] = min(stats["min_gap"], float(srt[K - 1] - srt[K]))

    for layer in range(layers):
        router = synth.router(shape, seed, layer)
        for t in range(tokens):
            one(router, xs[layer * tokens + t])
    router = synth.router(shape, seed, 0)
    for _ in range(extra_random):
        one(router, rng.normal(0, 1, shape.hidden).astype(np.float32))
    print(f"[topk] {name}: {stats}", flush=True)
    return stats


def test_cfg0_replicas_route_identically():
    # bench.py's cfg0 inputs: 38 layer replicas, one token each (seed 2026),
    # plus 4096 random tokens at the same shape
    s = _divergence("cfg0", 2026, 38, 1, extra_random=4096)
    assert s["sets"] == 0 and s["order"] == 0
    assert s["max_logit_diff"] < 1e-5


def test_cfg2_routes_identically():
    s = _divergence("cfg2", 2026, 64, 1)
    assert s["sets"] == 0 and s["order"] == 0


def test_cfg3_zipf_prefill_routes_identically():
    # 512 tokens with the Zipf(1.1) logit bias: near-ties are common here
    # (smallest K-th/(K+1)-th gap ~2e-6), still no disagreement
    s = _divergence("cfg3", 2026, 1, 512)
    assert s["sets"] == 0 and s["order"] == 0
