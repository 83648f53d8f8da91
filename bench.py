#!/usr/bin/env python3
"""MoE-layer decode benchmark on one MI355X.

Metric: MoE-layer decode tok/s at batch 1, and achieved HBM
GB/s as a fraction of the 8 TB/s peak.

Workload (default cfg0): one OLMoE-shaped MoE layer (h 2048, 64 experts,
top-8, SwiGLU intermediate 1024, 4-bit group-64 experts), batch-1 decode.
To keep the expert weights out of the 256 MB Infinity Cache, R distinct
layer replicas (R * 216 MiB) are resident and each step runs one token
through all R of them in order (one HIP graph launch); `value` counts
layer-tokens per second.  All inputs are resident in HBM before timing.
The inputs rotate over four graphs (graph j gives replica r the input drawn
for replica (r + j) % R), so the expert selection changes from step to step;
the replicas are not chained output -> input (the configured input is a bf16
N(0,1) activation; the chained form is the whole decoder, cfg1 / cfg4).

A step = one token through the MoE block of each of the R replicas
(router + top-K, expert dispatch, gate/up/SwiGLU, down, combine + residual).

The CPU baseline is the scalar oracle (oracle/, its lane-by-lane matvec)
timed on bounded samples of the same workload in the same run: one thread
(`cpu_baseline`) and the box's 16-thread share (`cpu_baseline_all_cores`).
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_HBM_GBS = 8000.0
PEAK_F16_TFLOPS = 2500.0  # MI355X dense f16/bf16 MFMA
METRIC = "MoE-layer decode tok/s at batch 1; achieved HBM GB/s as % of peak"
PREFILL_METRIC = "MoE-layer prefill tok/s (512 tokens, Zipf(1.1) expert loads); MFMA utilisation"


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def decode_kernel_name(shape) -> str:
    """The decode kernel the library selects for this shape on a 256-CU
    MI355X (m1moe_decode_kernel_for, one per-CU workgroup per CU)."""
    from m1moe_amd.engine import decode_kernel_for
    return decode_kernel_for(shape, 256, 1)


def cpu_threads() -> int:
    """Host threads for the all-cores CPU baseline: the box's CPU share."""
    return max(1, min(16, os.cpu_count() or 1))


def cpu_decode_baselines(args, synth, orc, oshape, img, router, xs, res):
    """The scalar oracle (lane-by-lane matvec restatement) timed on the host:
    one thread, token after token (BASELINE's primary figure), then all the
    threads of the box's share, tokens in parallel (orc.moe_prefill: per-token
    decode on each thread).  About args.cpu_seconds of work each."""
    orc.set_scalar(True)
    try:
        x32 = synth.bf16_to_f32(xs)
        n, t_cpu = 0, 0.0
        while t_cpu < args.cpu_seconds:
            t1 = time.perf_counter()
            orc.moe_decode(oshape, img, router, x32[n % len(x32)], res[n % len(res)])
            t_cpu += time.perf_counter() - t1
            n += 1
        one = {"value": round(n / t_cpu, 3), "unit": "layer-tok/s", "cores": 1, "kind": "port",
               "sample": f"{n} tokens of {args.config} decode (replica-0 experts, the bench's "
                         f"inputs) through the scalar oracle on 1 thread ({t_cpu:.1f}s); "
                         f"host CPU: {cpu_model()}"}
        log(f"cpu baseline (1 thread): {one['value']} layer-tok/s")
        nt = cpu_threads()
        T = 2 * nt
        X = np.stack([x32[i % len(x32)] for i in range(T)])
        Rs = np.stack([res[i % len(res)] for i in range(T)])
        n, t_cpu = 0, 0.0
        while t_cpu < args.cpu_seconds:
            t1 = time.perf_counter()
            orc.moe_prefill(oshape, img, router, X, Rs, nthreads=nt)
            t_cpu += time.perf_counter() - t1
            n += T
        allc = {"value": round(n / t_cpu, 3), "unit": "layer-tok/s", "cores": nt, "kind": "port",
                "sample": f"{n} tokens of {args.config} decode through the scalar oracle, "
                          f"{T} tokens at a time on {nt} threads ({t_cpu:.1f}s); "
                          f"host CPU: {cpu_model()}"}
        log(f"cpu baseline ({nt} threads): {allc['value']} layer-tok/s")
    finally:
        orc.set_scalar(False)
    return one, allc


def algorithmic_bytes(shape, expert_bytes: int, x_bytes: int, with_residual: bool) -> int:
    """Bytes one token must move through one MoE layer: the K selected expert
    blocks, the bf16 router, the input, the residual and the output."""
    h = shape.hidden
    return (shape.top_k * expert_bytes + shape.num_experts * h * 2 + h * x_bytes
            + (h * 4 if with_residual else 0) + h * 4)


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def copy_calibration(m, nbytes: int, reps: int) -> int:
    """Plain device-to-device copies of a known size, so a profiler's
    FETCH_SIZE / WRITE_SIZE for this copy kernel give the counter's scale."""
    shape = m.make_shape(64, 1, 1, 64, 64)
    with m.HIPContext(shape) as ctx:
        a, b = ctx.alloc(nbytes), ctx.alloc(nbytes)
        for _ in range(reps):
            ctx.lib.m1moe_copy_d2d(ctx.handle, b.ptr, a.ptr, nbytes)
        ctx.sync()
    print(json.dumps({"copy_calibration_bytes": nbytes, "copies": reps}), flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawTextHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None,
                    help="timed steps (default 200; cfg1: 5 jobs, cfg4: 1 job)")
    ap.add_argument("--warmup", type=int, default=None,
                    help="untimed steps (default 20; cfg1/cfg4: 1 job)")
    ap.add_argument("--config", default="cfg0",
                    choices=["cfg0", "cfg1", "cfg2", "cfg3", "cfg4", "quant", "tokenizer"],
                    help="cfg0/cfg2: MoE-layer batch-1 decode; cfg3: 512-token MoE prefill; "
                         "cfg1/cfg4: whole decoder, prompt then greedy steps (a step is one "
                         "such job); quant / tokenizer: the host rows (converter's 4-bit "
                         "quantizer over one OLMoE layer, BPE encode), no GPU")
    ap.add_argument("--replicas", type=int, default=0,
                    help="distinct layer replicas (default: >= 1 GiB of selected experts per pass)")
    ap.add_argument("--cpu-seconds", type=float, default=8.0,
                    help="bound on each CPU-baseline sample, one thread and all threads "
                         "(0 disables them)")
    ap.add_argument("--seed", type=int, default=2026)
    ap.add_argument("--eager", action="store_true",
                    help="cfg1/cfg4: launch every step's kernels from the host instead of "
                         "replaying the captured one-step graph (for kernel traces)")
    ap.add_argument("--repeats", type=int, default=20,
                    help="cfg0/cfg2: repeats of a few steps each after the timed region, "
                         "their median reported beside it (0: none; the kernel-trace "
                         "profiles run without them)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="BYTES",
                    help="only run device-to-device copies of BYTES bytes (to scale HBM "
                         "byte counters against a plain copy of known size), then exit")
    args = ap.parse_args()
    job_defaults = {"cfg1": (5, 1), "cfg4": (1, 1), "quant": (3, 1),
                    "tokenizer": (3, 1)}.get(args.config, (200, 20))
    if args.steps is None:
        args.steps = job_defaults[0]
    if args.warmup is None:
        args.warmup = job_defaults[1]

    if args.gpus != 1:
        print(f"bench.py: --gpus {args.gpus} is not supported: this build measures one GPU "
              "(the MoE layer's multi-GPU sharding is a design, not a run). Use --gpus 1.",
              file=sys.stderr)
        return 2

    import m1moe_amd as m
    from m1moe_amd import synth
    from m1moe_amd.engine import MoEBlock

    if args.copy_calibration:
        return copy_calibration(m, args.copy_calibration, max(1, args.steps))

    if args.config == "quant":
        return bench_quant(args, m, synth)
    if args.config == "tokenizer":
        return bench_tokenizer(args, m)
    if args.config == "cfg3":
        return bench_prefill(args, m, synth)
    if args.config in ("cfg1", "cfg4"):
        return bench_decoder(args, m, synth)

    wl = synth.CONFIGS[args.config]
    one = wl.shape(1)
    eb = m.expert_bytes(one)
    layer_bytes = one.num_experts * eb
    # enough replicas that the expert blocks one pass touches (R * K blocks)
    # are far beyond the 256 MB Infinity Cache
    touched = one.top_k * eb
    R = args.replicas or max(2, -(-1024 ** 3 // touched))
    shape = wl.shape(R)
    h, K = shape.hidden, shape.top_k
    log(f"{wl.description}: {R} replicas x {layer_bytes / 2**20:.0f} MiB")

    ctx = m.HIPContext(shape, device=0)
    blk = MoEBlock(ctx)
    t0 = time.time()
    img0 = router0 = None
    for r in range(R):
        img = synth.layer_image(shape, args.seed, r)
        router = synth.router(shape, args.seed, r)
        ctx.upload_layer_experts(r, img)
        ctx.upload_router(r, router)
        if r == 0:
            img0, router0 = img, router
        del img
    log(f"uploaded {R} layers in {time.time() - t0:.1f}s")

    xs = synth.activations_bf16(shape, args.seed, R)
    res = synth.residual_f32(shape, args.seed, R)
    dx = [ctx.to_device(xs[r]) for r in range(R)]
    dres = [ctx.to_device(res[r]) for r in range(R)]
    dout = [ctx.alloc(h * 4) for _ in range(R)]
    didx = ctx.alloc(K * 4)

    # parity of replica 0 before any timing
    from oracle import oracle as orc
    oshape = orc.from_moe_shape(shape)
    blk.forward(0, dx[0], "bf16", dres[0], dout[0], didx, None)
    ctx.sync()
    got = dout[0].download(np.float32)
    want, widx, _, _ = orc.moe_decode(oshape, img0, router0, synth.bf16_to_f32(xs[0]), res[0])
    rel = float(np.linalg.norm(got - want) / np.linalg.norm(want))
    idx_ok = bool(np.array_equal(didx.download(np.int32), widx))
    log(f"parity replica 0: top-K exact={idx_ok} rel L2={rel:.2e}")
    if not idx_ok or rel > 1e-2:
        log("parity FAILED; not reporting throughput")
        return 1

    # The replicas are not chained output -> input: the configured input is a
    # bf16 N(0,1) activation while a layer's output is the f32 residual stream,
    # which without the decoder's RMSNorm grows from layer to layer (the chained
    # form is the whole decoder, --config cfg1 / cfg4).  The inputs rotate
    # instead: graph j feeds replica r the input and residual drawn for replica
    # (r + j) % R, and the graphs are replayed in turn, so every replica's
    # expert selection changes from step to step.
    G = min(4, R)
    sel = []
    for j in range(G):
        q = j % R
        blk.forward(0, dx[q], "bf16", dres[q], dout[0], didx, None)
        ctx.sync()
        sel.append(sorted(didx.download(np.int32).tolist()))
    log(f"replica 0 selects, over the {G} input rotations: {sel}")
    graphs = []
    for j in range(G):
        ctx.graph_begin()
        for r in range(R):
            q = (r + j) % R
            blk.forward(r, dx[q], "bf16", dres[q], dout[r])
        graphs.append(ctx.graph_end())

    for i in range(args.warmup):
        graphs[i % G].launch()
    ctx.sync()
    ev0, ev1 = ctx.event(), ctx.event()
    ctx.sync()
    ev0.record()
    for i in range(args.steps):
        graphs[i % G].launch()
    ev1.record()
    ctx.sync()
    ms = ev0.elapsed_ms(ev1)
    ms_per_step = ms / args.steps
    layer_us = ms_per_step * 1e3 / R
    tok_s = R * args.steps / (ms * 1e-3)
    bytes_tok = algorithmic_bytes(shape, eb, 2, True)
    gbs = bytes_tok / (layer_us * 1e-6) / 1e9
    log(f"{ms_per_step:.4f} ms/step, {layer_us:.3f} us/layer-token, {gbs:.0f} GB/s")

    # the measurement protocol of the baseline beside the timed region above
    # (which `value` comes from): the median of 20 repeats of a few steps each
    rep_steps = max(1, min(10, args.steps))
    rep_us = []
    for _ in range(max(0, args.repeats)):
        ev0.record()
        for i in range(rep_steps):
            graphs[i % G].launch()
        ev1.record()
        ctx.sync()
        rep_us.append(ev0.elapsed_ms(ev1) * 1e3 / (rep_steps * R))
    rep_us.sort()
    repeats = None
    if rep_us:
        repeats = {"n": len(rep_us), "steps_each": rep_steps,
                   "median_us_per_layer_token": round(float(np.median(rep_us)), 4),
                   "min_us": round(rep_us[0], 4), "max_us": round(rep_us[-1], 4)}
        log(f"{len(rep_us)} repeats of {rep_steps} steps: median "
            f"{repeats['median_us_per_layer_token']:.3f} us/layer-token (min {rep_us[0]:.3f}, "
            f"max {rep_us[-1]:.3f})")

    cpu = cpu_all = None
    if args.cpu_seconds > 0:
        cpu, cpu_all = cpu_decode_baselines(args, synth, orc, oshape, img0, router0, xs, res)

    traffic = None
    tpath = os.path.join(ROOT, "profiles", "traffic.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            rec = json.load(f).get(args.config)
        if rec:  # measured by rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE, copy-calibrated
            traffic = int(rec["hbm_bytes_per_launch"])

    line = {
        "metric": METRIC,
        "value": round(tok_s, 1),
        "unit": "layer-tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u4 weights x f16 pairs (bf16 x exact in f16; f32 act as hi+lo f16) -> f32",
        "data": "synthetic (seeded; random-init experts/router)",
        "config": {"workload": wl.description, "config": args.config, "hidden": h,
                   "num_experts": shape.num_experts, "top_k": K,
                   "intermediate": shape.intermediate, "group_size": shape.group_size,
                   "replicas": R, "tokens_per_step": 1, "x_dtype": "bf16",
                   "residual": "f32", "input_rotations": G},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": traffic,
                     "kernel": decode_kernel_name(shape) + " (the whole MoE block, one "
                                                             "launch per layer-token)",
                     "bytes_per_launch": bytes_tok, "us_per_launch": round(layer_us, 4)},
        "cpu_baseline": cpu,
        "cpu_baseline_all_cores": cpu_all,
        "parity": {"topk_exact": idx_ok, "rel_l2": rel},
        "repeats": repeats,
    }
    print(json.dumps(line), flush=True)
    ctx.close()
    return 0


DECODER_METRIC = "decoder greedy decode tok/s at batch 1 (prompt then greedy steps)"


def decoder_step_bytes(wl, eb: int, pos: int) -> int:
    """HBM bytes one decode step at position pos must move: every dense
    weight once (lm_head, q/k/v/o, norms, one embedding row), each layer's
    MoE block (K expert blocks, bf16 router, f32 input/residual/output), and
    the K/V cache rows 0..pos of every layer (read) plus row pos (written)."""
    s = wl.shape()
    h, L, V = s.hidden, s.num_layers, wl.vocab
    qd, kvd = wl.num_heads * wl.head_dim, wl.num_kv_heads * wl.head_dim
    dense = 2 * (V * h + h + L * (2 * h + 2 * qd * h + 2 * kvd * h)
                 + (2 * L * wl.head_dim if wl.qk_norm else 0)) + 2 * h
    moe = L * (s.top_k * eb + s.num_experts * h * 2 + 3 * h * 4)
    kv = L * 2 * kvd * 4 * (pos + 2)
    return dense + moe + kv


def bench_decoder(args, m, synth) -> int:
    """cfg1 / cfg4: the whole decoder (Decoder, m1moe_dec_*), seeded random
    weights, a random prompt then greedy steps (Sources/bench/main.swift:
    136-163; the reference forwards the prompt token by token, here it goes
    through m1moe_dec_prefill in one batch per layer).  One HIP graph holds
    one sequence-mode step, replayed once per greedy token."""
    from m1moe_amd import _lib
    from m1moe_amd.decoder import Decoder
    from oracle import oracle as orc

    wl = synth.DECODERS[args.config]
    shape = wl.shape()
    L, P, G = shape.num_layers, wl.prompt, wl.gen
    eb = m.expert_bytes(shape)
    log(f"{wl.description}: {L} layers, {L * shape.num_experts * eb / 2**30:.1f} GiB of experts")
    t0 = time.time()
    ctx = m.HIPContext(shape, device=0)
    dec = Decoder(ctx, wl.dec_shape(P + G))
    keep = args.cpu_seconds > 0
    tensors = {}
    names = {_lib.W_EMBED: "embed", _lib.W_LM_HEAD: "lm_head", _lib.W_FINAL_NORM: "final_norm",
             _lib.W_IN_NORM: "in_norm", _lib.W_POST_NORM: "post_norm", _lib.W_Q: "q",
             _lib.W_K: "k", _lib.W_V: "v", _lib.W_O: "o", _lib.W_Q_NORM: "q_norm",
             _lib.W_K_NORM: "k_norm"}
    for which, name in names.items():
        if which in (_lib.W_Q_NORM, _lib.W_K_NORM) and not wl.qk_norm:
            continue
        layers = range(L) if which in _lib.W_PER_LAYER else [0]
        arrs = []
        for layer in layers:
            w = synth.dense_weight(wl, args.seed, which, layer)
            dec.upload(which, layer, w)
            arrs.append(w if keep else None)
        tensors[name] = arrs if which in _lib.W_PER_LAYER else arrs[0]
    images, routers = [], []
    for layer in range(L):
        img = synth.layer_image(shape, args.seed, layer)
        r = synth.router(shape, args.seed, layer)
        ctx.upload_layer_experts(layer, img)
        ctx.upload_router(layer, r)
        images.append(img if keep else None)
        routers.append(r)
        del img
    log(f"weights synthesised and uploaded in {time.time() - t0:.1f}s")
    prompt = synth.prompt_tokens(wl, args.seed)

    # parity (and the CPU baseline): the first prompt tokens through the GPU
    # decoder eagerly and through the scalar oracle on one thread
    cpu = None
    parity = None
    if keep:
        oracle = orc.DecoderOracle(orc.from_moe_shape(shape), L, wl.vocab, wl.num_heads,
                                   wl.num_kv_heads, wl.head_dim, P + G, wl.qk_norm,
                                   wl.rope_theta, wl.rms_eps, tensors, images, routers)
        dec.reset()
        worst, n, t_cpu, tok_ok = 0.0, 0, 0.0, True
        orc.set_scalar(True)  # the lane-by-lane matvec restatement, as the cfg0 baseline
        while n < P and (n == 0 or t_cpu < args.cpu_seconds):
            g_tok, g_lg = dec.forward(int(prompt[n]), return_logits=True)
            t1 = time.perf_counter()
            w_tok, w_lg = oracle.step(int(prompt[n]))
            t_cpu += time.perf_counter() - t1
            rel = float(np.linalg.norm(g_lg - w_lg) / np.linalg.norm(w_lg))
            worst = max(worst, rel)
            top2 = np.sort(w_lg.astype(np.float64))[-2:]
            tok_ok &= g_tok == w_tok or bool(top2[1] - top2[0] < 1e-2)
            n += 1
        orc.set_scalar(False)
        parity = {"steps_checked": n, "logits_rel_l2_max": worst, "greedy_tokens_agree": tok_ok}
        log(f"parity over {n} steps: logits rel L2 max {worst:.2e}, tokens agree {tok_ok}")
        if worst > 1e-2 or not tok_ok:
            log("parity FAILED; not reporting throughput")
            return 1
        cpu = {"value": round(n / t_cpu, 4), "unit": "tok/s", "cores": 1, "kind": "port",
               "sample": f"{n} decoder steps of {args.config} (positions 0..{n - 1}) through the "
                         f"scalar oracle on 1 thread ({t_cpu:.1f}s); host CPU: {cpu_model()}"}
        log(f"cpu baseline: {cpu['value']} tok/s")
        del oracle, images, tensors

    cap = P + G + 1
    seq = ctx.alloc(4 * cap)
    init = np.concatenate([prompt, np.zeros(cap - P, np.int32)])
    dprompt = ctx.to_device(prompt)

    def prefill():
        # the prompt in one batch per layer; its greedy token lands at seq[P]
        dec.prefill_device(dprompt, P, seq.addr + 4 * P)

    # eager run (batched prefill, then sequence-mode steps): the reference
    # tokens for the graph replays; it also grows the prefill scratch
    seq.upload(init)
    dec.reset()
    prefill()
    for _ in range(G):
        dec.step_seq(seq, P, cap)
    ctx.sync()
    want = seq.download(np.int32)[P:]
    if args.eager:
        class _Eager:
            @staticmethod
            def launch():
                dec.step_seq(seq, P, cap)
        graph = _Eager()
    else:
        ctx.graph_begin()
        dec.step_seq(seq, P, cap)
        graph = ctx.graph_end()
    ev = [ctx.event() for _ in range(3)]
    t_pre = t_gen = 0.0
    same = True
    for it in range(args.warmup + args.steps):
        seq.upload(init)
        dec.reset()
        ctx.sync()
        ev[0].record()
        prefill()
        ev[1].record()
        for _ in range(G):
            graph.launch()
        ev[2].record()
        ctx.sync()
        same &= seq.download(np.int32)[P:].tolist() == want.tolist()
        if it >= args.warmup:
            t_pre += ev[0].elapsed_ms(ev[1])
            t_gen += ev[1].elapsed_ms(ev[2])
    if not same:
        log("graph replays produced other tokens than the eager run")
        return 1
    jobs = args.steps
    gen_tok_s = G * jobs / (t_gen * 1e-3)
    pre_tok_s = P * jobs / (t_pre * 1e-3)
    us_gen = t_gen * 1e3 / (G * jobs)
    bytes_step = sum(decoder_step_bytes(wl, eb, P + i) for i in range(G)) / G
    gbs = bytes_step / (us_gen * 1e-6) / 1e9
    log(f"prefill {P} tok: {t_pre / jobs:.2f} ms ({pre_tok_s:.1f} tok/s); decode {G} tok: "
        f"{t_gen / jobs:.2f} ms ({gen_tok_s:.1f} tok/s, {us_gen:.1f} us/token, {gbs:.0f} GB/s)")
    line = {
        "metric": DECODER_METRIC, "value": round(gen_tok_s, 2), "unit": "tok/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round((t_pre + t_gen) / jobs, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16 dense weights, u4 experts x f16 pairs -> f32; f32 KV cache",
        "data": "synthetic (seeded; random-init weights, random prompt ids)",
        "config": {"workload": wl.description, "config": args.config, "layers": L,
                   "hidden": shape.hidden, "vocab": wl.vocab, "num_heads": wl.num_heads,
                   "num_kv_heads": wl.num_kv_heads, "head_dim": wl.head_dim,
                   "num_experts": shape.num_experts, "top_k": shape.top_k,
                   "intermediate": shape.intermediate, "prompt_tokens": P, "gen_tokens": G,
                   "step": "one job = reset, the prompt in one batch per layer "
                           "(m1moe_dec_prefill), then each greedy token one " +
                           ("host launch of its kernels" if args.eager else
                            "replay of a one-step HIP graph"),
                   "prefill_tok_s": round(pre_tok_s, 2)},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": None,
                     "kernel": "decoder step (all kernels of one greedy token)",
                     "bytes_per_launch": int(bytes_step), "us_per_launch": round(us_gen, 3)},
        "cpu_baseline": cpu,
        "parity": parity,
    }
    print(json.dumps(line), flush=True)
    dec.close()
    ctx.close()
    return 0


def bench_prefill(args, m, synth) -> int:
    """cfg3: T tokens through the MoE block of R distinct layer replicas per
    step (one HIP graph).  The MFMA work that counts is the useful one:
    T*K pairs x (gate + up + down) = 6*h*I FLOPs per pair."""
    from m1moe_amd.engine import MoEBlock
    from oracle import oracle as orc

    wl = synth.CONFIGS["cfg3"]
    one = wl.shape(1)
    eb = m.expert_bytes(one)
    layer_bytes = one.num_experts * eb
    R = args.replicas or 4
    shape = wl.shape(R)
    T, h, K, I, E = wl.T, shape.hidden, shape.top_k, shape.intermediate, shape.num_experts
    log(f"{wl.description}: {R} replicas x {layer_bytes / 2**20:.0f} MiB")
    bias = synth.zipf_logit_bias(E, wl.zipf_s)
    ctx = m.HIPContext(shape, device=0)
    blk = MoEBlock(ctx)
    img0 = router0 = None
    for r in range(R):
        img = synth.layer_image(shape, args.seed, r)
        router = synth.router(shape, args.seed, r)
        ctx.upload_layer_experts(r, img)
        ctx.upload_router(r, router)
        ctx.set_logit_bias(r, bias)
        if r == 0:
            img0, router0 = img, router
        del img
    xs = [synth.activations_bf16(shape, args.seed, T, r) for r in range(R)]
    res = [synth.residual_f32(shape, args.seed, T, r) for r in range(R)]
    dx = [ctx.to_device(x) for x in xs]
    dres = [ctx.to_device(x) for x in res]
    dout = [ctx.alloc(T * h * 4) for _ in range(R)]
    didx = ctx.alloc(T * K * 4)

    # parity of replica 0 before timing
    blk.prefill(0, T, dx[0], "bf16", dres[0], dout[0], didx, None)
    ctx.sync()
    got = dout[0].download(np.float32).reshape(T, h)
    gidx = didx.download(np.int32).reshape(T, K)
    want, widx, _ = orc.moe_prefill(orc.from_moe_shape(shape), img0, router0,
                                    synth.bf16_to_f32(xs[0]), res[0], bias,
                                    nthreads=min(16, os.cpu_count() or 1))
    rel = float(np.linalg.norm(got - want) / np.linalg.norm(want))
    moe_rel = float(np.linalg.norm((got - res[0]) - (want - res[0]))
                    / np.linalg.norm(want - res[0]))
    idx_ok = bool(np.array_equal(gidx, widx))
    counts = np.bincount(gidx.ravel(), minlength=E)
    log(f"parity replica 0: top-K exact={idx_ok} rel L2={rel:.2e} (MoE part {moe_rel:.2e}); "
        f"expert loads max {counts.max()} min {counts.min()}")
    if not idx_ok or moe_rel > 1e-2:
        log("parity FAILED; not reporting throughput")
        return 1

    ctx.graph_begin()
    for r in range(R):
        blk.prefill(r, T, dx[r], "bf16", dres[r], dout[r])
    graph = ctx.graph_end()
    for _ in range(args.warmup):
        graph.launch()
    ctx.sync()
    ev0, ev1 = ctx.event(), ctx.event()
    ev0.record()
    for _ in range(args.steps):
        graph.launch()
    ev1.record()
    ctx.sync()
    ms = ev0.elapsed_ms(ev1)
    us_layer = ms * 1e3 / (args.steps * R)
    tok_s = T / (us_layer * 1e-6)
    flops = 6.0 * h * I * T * K
    tflops = flops / (us_layer * 1e-6) / 1e12
    used = int((counts > 0).sum())
    wbytes = used * eb + E * h * 2 + T * h * 2 + 2 * T * h * 4
    gbs = wbytes / (us_layer * 1e-6) / 1e9
    log(f"{us_layer:.2f} us per 512-token layer prefill, {tok_s:.0f} tok/s, "
        f"{tflops:.1f} TFLOP/s ({100 * tflops / PEAK_F16_TFLOPS:.1f}% of f16 MFMA peak), "
        f"{gbs:.0f} GB/s of weights+activations")
    cpu = cpu_all = None
    if args.cpu_seconds > 0:
        # the 512-token prefill is 512 independent token decodes on the CPU (the
        # reference forwards a prompt token by token): a bounded prefix of
        # replica 0's tokens, one thread, then all threads
        oshape = orc.from_moe_shape(shape)
        x32, base = synth.bf16_to_f32(xs[0]), []
        orc.set_scalar(True)
        try:
            for nt in (1, cpu_threads()):
                n, t_cpu = 0, 0.0
                while t_cpu < args.cpu_seconds and n < T:
                    m_ = min(2 * nt, T - n)
                    t1 = time.perf_counter()
                    orc.moe_prefill(oshape, img0, router0, x32[n:n + m_], res[0][n:n + m_], bias,
                                    nthreads=nt)
                    t_cpu += time.perf_counter() - t1
                    n += m_
                base.append({"value": round(n / t_cpu, 3), "unit": "tok/s", "cores": nt,
                             "kind": "port",
                             "sample": f"the first {n} of the {T} cfg3 tokens (replica 0, Zipf "
                                       f"bias) through the scalar oracle on {nt} thread(s) "
                                       f"({t_cpu:.1f}s); host CPU: {cpu_model()}"})
                log(f"cpu baseline ({nt} threads): {base[-1]['value']} tok/s")
        finally:
            orc.set_scalar(False)
        cpu, cpu_all = base
    line = {
        "metric": PREFILL_METRIC, "value": round(tok_s, 1), "unit": "tok/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms / args.steps, 5), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "u4 weights -> f16 MFMA, f32 accumulate",
        "data": "synthetic (seeded; random-init experts/router, Zipf(1.1) router bias)",
        "config": {"workload": wl.description, "config": "cfg3", "tokens": T, "hidden": h,
                   "num_experts": E, "top_k": K, "intermediate": I, "replicas": R},
        "roofline": {"bound": "mfma", "achieved": round(tflops, 2), "peak": PEAK_F16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(tflops / PEAK_F16_TFLOPS, 4),
                     "traffic": None, "flops_per_launch": flops,
                     "us_per_launch": round(us_layer, 3),
                     "hbm_gbs_of_algorithmic_bytes": round(gbs, 1)},
        "cpu_baseline": cpu,
        "cpu_baseline_all_cores": cpu_all,
        "parity": {"topk_exact": idx_ok, "rel_l2": rel, "moe_part_rel_l2": moe_rel},
    }
    print(json.dumps(line), flush=True)
    ctx.close()
    return 0


def bench_quant(args, m, synth) -> int:
    """The converters' quantizer (extract_olmoe.py:116-159, quantize_4bit per
    expert matrix, then the expert block layout) over one OLMoE layer: 64
    experts of f32 gate [1024, 2048], up [1024, 2048], down [2048, 1024] to the
    packed layer image, on the host's threads.  A step = one layer.  Eight
    distinct seeded experts are cycled (the work does not depend on the
    values).  CPU baseline: the numpy restatement (oracle/quant_oracle.py)
    on a bounded number of experts, one thread."""
    from m1moe_amd import quant
    from oracle import quant_oracle as qo

    shape = synth.CONFIGS["cfg0"].shape(1)
    h, inter, E = shape.hidden, shape.intermediate, shape.num_experts
    rng = np.random.default_rng(args.seed)
    experts = [tuple((rng.standard_normal(s, dtype=np.float32) * 0.02)
                     for s in ((inter, h), (inter, h), (h, inter))) for _ in range(8)]
    eb = m.expert_bytes(shape)
    image = np.empty((E, eb), np.uint8)
    nt = cpu_threads()
    f32_bytes = E * 3 * inter * h * 4

    def layer():
        for e in range(E):
            image[e] = quant.quantize_expert(shape, *experts[e % 8], threads=nt)

    for _ in range(args.warmup):
        layer()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        layer()
    dt = (time.perf_counter() - t0) / args.steps
    want = qo.expert_block(*experts[0], shape.group_size)
    exact = bool(np.array_equal(image[0], want) and np.array_equal(image[8], want))
    log(f"quantizer: {dt * 1e3:.1f} ms per layer, {f32_bytes / dt / 1e9:.2f} GB/s of f32 "
        f"input on {nt} threads; expert blocks equal to the oracle's: {exact}")
    cpu = None
    if args.cpu_seconds > 0:
        n, t_cpu = 0, 0.0
        while t_cpu < args.cpu_seconds and n < E:
            t1 = time.perf_counter()
            qo.expert_block(*experts[n % 8], shape.group_size)
            t_cpu += time.perf_counter() - t1
            n += 1
        cpu = {"value": round(n / t_cpu / E, 4), "unit": "layers/s", "cores": 1, "kind": "port",
               "sample": f"{n} of the 64 experts through the numpy restatement "
                         f"(oracle/quant_oracle.py) on 1 thread ({t_cpu:.1f}s); "
                         f"host CPU: {cpu_model()}"}
        log(f"cpu baseline: {cpu['value']} layers/s")
    print(json.dumps({
        "metric": "4-bit group-64 quantization of one OLMoE layer's experts (host)",
        "value": round(1.0 / dt, 3), "unit": "layers/s", "n_gpus": 0, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(dt * 1e3, 3), "higher_is_better": True,
        "scaling": "strong", "vs_baseline": None, "dtype": "f32 -> u4 + bf16 scale/bias",
        "data": "synthetic (seeded N(0, 0.02) expert matrices)",
        "config": {"workload": "OLMoE layer: 64 experts x (gate, up [1024, 2048], down "
                               "[2048, 1024]), group 64", "threads": nt},
        "roofline": None, "host_gbs_of_f32_input": round(f32_bytes / dt / 1e9, 2),
        "cpu_baseline": cpu, "parity": {"expert_blocks_equal_oracle": exact}}), flush=True)
    return 0


def _bench_corpus(seed: int, lines: int):
    """Seeded lines of syllable words, English-like words, digits and
    punctuation, some non-ASCII."""
    syl = ["ex", "per", "rout", "er", "to", "ken", "mo", "del", "la", "yer", "in", "ter", "ca",
           "ti", "on", "ma", "tri", "x", "gra", "ph", "é", "ü", "東", "京", "σ", "λ"]
    rng = np.random.default_rng(seed)
    words = ["".join(syl[int(j)] for j in rng.integers(0, len(syl), int(rng.integers(1, 5))))
             for _ in range(3000)] + ["the", "of", "and", "a", "to", "is", "2024", "3.14", "--"]
    out = []
    for _ in range(lines):
        k = int(rng.integers(3, 20))
        w = [words[int(i)] for i in rng.integers(0, len(words), k)]
        out.append(" ".join(w) + rng.choice([".", ",", "!", "?", ":", ""]))
    return out


def bench_tokenizer(args, m) -> int:
    """BPE encode (Tokenizer.swift:34-259) of a seeded synthetic text with
    vocabularies trained here by the HuggingFace `tokenizers` library: GPT-2
    byte-level (OLMoE) and SentencePiece with byte fallback (Mixtral), 8000
    tokens each.  A step = encoding the whole text (4 MiB) with each; one
    thread, as the reference.  CPU baseline: the pure-Python restatement
    (oracle/tokenizer_oracle.py) on a bounded prefix."""
    import tempfile

    import tokenizers
    from tokenizers import models, pre_tokenizers, trainers

    from m1moe_amd.tokenizer import Tokenizer
    from oracle.tokenizer_oracle import OracleTokenizer

    corpus = _bench_corpus(args.seed, 20000)
    text = "\n".join(_bench_corpus(args.seed + 1, 60000))
    text = text.encode("utf-8")[:4 << 20].decode("utf-8", "ignore")
    nbytes = len(text.encode("utf-8"))
    res = {}
    with tempfile.TemporaryDirectory() as d:
        for mode in ("byte_level", "sentencepiece"):
            if mode == "byte_level":
                hf = tokenizers.Tokenizer(models.BPE())
                hf.pre_tokenizer = pre_tokenizers.ByteLevel(add_prefix_space=False)
                tr = trainers.BpeTrainer(vocab_size=8000, show_progress=False,
                                         initial_alphabet=pre_tokenizers.ByteLevel.alphabet(),
                                         special_tokens=["<|endoftext|>"])
            else:
                hf = tokenizers.Tokenizer(models.BPE(byte_fallback=True, unk_token="<unk>"))
                hf.pre_tokenizer = pre_tokenizers.Metaspace(replacement="\u2581",
                                                            prepend_scheme="always")
                specials = ["<unk>", "<s>", "</s>"] + ["<0x%02X>" % b for b in range(256)]
                tr = trainers.BpeTrainer(vocab_size=8000, special_tokens=specials,
                                         show_progress=False)
            hf.train_from_iterator(corpus, tr)
            js = json.loads(hf.to_str())
            js["model"]["merges"] = [" ".join(p) if isinstance(p, list) else p
                                     for p in js["model"]["merges"]]
            js["model"]["byte_fallback"] = mode == "sentencepiece"
            path = os.path.join(d, f"{mode}.json")
            with open(path, "w", encoding="utf-8") as f:
                json.dump(js, f)
            tok = Tokenizer(path)
            for _ in range(args.warmup):
                ids = tok.encode(text, add_bos=False)
            t0 = time.perf_counter()
            for _ in range(args.steps):
                ids = tok.encode(text, add_bos=False)
            dt = (time.perf_counter() - t0) / args.steps
            orc = OracleTokenizer(path)
            n, t_cpu, same = 0, 0.0, True
            pieces = text.split("\n")
            while n < len(pieces) and (t_cpu < max(args.cpu_seconds, 0.5) / 2):
                t1 = time.perf_counter()
                want = orc.encode(pieces[n], add_bos=False)
                t_cpu += time.perf_counter() - t1
                same = same and want == tok.encode(pieces[n], add_bos=False)
                n += 1
            sample = sum(len(p.encode("utf-8")) + 1 for p in pieces[:n])
            res[mode] = {"mib_s": nbytes / dt / 2**20, "tokens": len(ids),
                         "oracle_mib_s": sample / t_cpu / 2**20, "oracle_lines": n,
                         "oracle_s": t_cpu, "lines_equal_oracle": same}
            log(f"{mode}: {nbytes / dt / 2**20:.2f} MiB/s ({len(ids)} tokens); oracle "
                f"{res[mode]['oracle_mib_s']:.3f} MiB/s on {n} lines, equal: {same}")
            tok.close()
    bl = res["byte_level"]
    print(json.dumps({
        "metric": "BPE encode throughput, byte-level (OLMoE) vocabulary (host, one thread)",
        "value": round(bl["mib_s"], 3), "unit": "MiB/s", "n_gpus": 0, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(nbytes / bl["mib_s"] / 2**20 * 1e3, 3),
        "higher_is_better": True, "scaling": "strong", "vs_baseline": None, "dtype": "u8 text",
        "data": "synthetic (seeded syllable-word text; vocabularies trained here)",
        "config": {"workload": "4 MiB of text, 8000-token BPE vocabularies", "bytes": nbytes},
        "roofline": None,
        "sentencepiece_mib_s": round(res["sentencepiece"]["mib_s"], 3),
        "cpu_baseline": {"value": round(bl["oracle_mib_s"], 4), "unit": "MiB/s", "cores": 1,
                         "kind": "port",
                         "sample": f"the first {bl['oracle_lines']} lines through the "
                                   f"pure-Python restatement (oracle/tokenizer_oracle.py), "
                                   f"{bl['oracle_s']:.1f}s; host CPU: {cpu_model()}"},
        "cpu_baseline_sentencepiece": round(res["sentencepiece"]["oracle_mib_s"], 4),
        "parity": {"byte_level_lines_equal_oracle": bl["lines_equal_oracle"],
                   "sentencepiece_lines_equal_oracle":
                       res["sentencepiece"]["lines_equal_oracle"]}}), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
