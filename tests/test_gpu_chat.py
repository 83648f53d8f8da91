"""The chat REPL end to end on the GPU against the decoder oracle.

chat.serve() loads a converted model directory (the seeded tiny decoder,
written in the converter's format) and a byte-level tokenizer.json, and runs
a scripted conversation at temperature 0 with a 300-token context: a system
prompt, turns long enough to hit the context limit, a sliding-window trim
with its re-prefill, /stats, /system, /quit.  The same script runs through
ChatSession over the decoder oracle (oracle.DecoderOracle, token by token).
Replies must be the same tokens up to the first step whose oracle top-2
logit margin is within the decoder's logit error bound (relative L2 1e-2),
as in the decoder's own greedy tests.
"""
from __future__ import annotations

import io

import numpy as np
import pytest

from m1moe_amd import _lib, chat, synth
from oracle import oracle as orc

from cases import say, write_byte_tokenizer

pytestmark = pytest.mark.gpu

NAMES = {_lib.W_EMBED: "embed", _lib.W_LM_HEAD: "lm_head", _lib.W_FINAL_NORM: "final_norm",
         _lib.W_IN_NORM: "in_norm", _lib.W_POST_NORM: "post_norm", _lib.W_Q: "q", _lib.W_K: "k",
         _lib.W_V: "v", _lib.W_O: "o", _lib.W_Q_NORM: "q_norm", _lib.W_K_NORM: "k_norm"}
LOGIT_TOL = 1e-2


class OracleEngine:
    def __init__(self, dec):
        self.o = dec
        self.steps = []   # (token, bound exceeded by the top-2 margin?)

    def reset(self):
        self.o.reset()

    def prefill(self, tokens):
        if len(tokens):
            self.o.prefill(tokens)

    def forward(self, token, temperature, top_p):
        tok, lg = self.o.step(int(token))
        top2 = np.sort(lg.astype(np.float64))[-2:]
        bound = 4 * LOGIT_TOL * np.linalg.norm(lg) / np.sqrt(lg.size)
        self.steps.append((int(tok), top2[1] - top2[0] >= bound))
        return int(tok)


def test_chat_session_on_the_gpu_matches_the_oracle(tmp_path):
    wl, seed, kv = synth.DECODERS["tiny_dec"], 31, 400
    L = wl.num_layers
    synth.write_model_dir(wl, seed, str(tmp_path))
    write_byte_tokenizer(str(tmp_path / "tokenizer.json"), eos_id=299)
    moe = wl.moe.shape(L)
    config = {"name": "tiny", "architecture": "olmoe", "hidden_dim": moe.hidden,
              "vocab_size": wl.vocab, "num_layers": L, "rms_norm_eps": wl.rms_eps,
              "attention": {"num_heads": wl.num_heads, "num_kv_heads": wl.num_kv_heads,
                            "head_dim": wl.head_dim, "rope_theta": wl.rope_theta,
                            "max_seq_len": kv, "gpu_kv_seq_prealloc": kv},
              "moe": {"num_experts": moe.num_experts, "top_k": moe.top_k,
                      "intermediate_dim": moe.intermediate, "norm_topk_prob": False},
              "quantization": {"bits": 4, "group_size": moe.group_size},
              "special_tokens": {"eos": [299], "bos": 1}}
    lines = ["hello there, tell me about the experts", "/stats",
             "and what routes the tokens?", "/system be brief", "third turn", "/quit"]
    args = chat.parse_args(["--temp", "0", "--max-ctx", "300", "--system", "you are a test"])
    out = io.StringIO()
    say("chat.serve tiny decoder, max_ctx 300")
    gpu = chat.serve(config, str(tmp_path), args, io.StringIO("\n".join(lines) + "\n"), out)
    text = out.getvalue()
    assert "[chat] context trimmed to 150 tokens" in text and "Bye." in text
    assert "[chat] last turn: " in text and "[chat] system prompt updated" in text

    tensors = {}
    for which, name in NAMES.items():
        if which in _lib.W_PER_LAYER:
            tensors[name] = [synth.dense_weight(wl, seed, which, l) for l in range(L)]
        else:
            tensors[name] = synth.dense_weight(wl, seed, which, 0)
    images = [synth.layer_image(moe, seed, l) for l in range(L)]
    routers = [synth.router(moe, seed, l) for l in range(L)]
    dec = orc.DecoderOracle(orc.from_moe_shape(moe), L, wl.vocab, wl.num_heads,
                            wl.num_kv_heads, wl.head_dim, kv, wl.qk_norm, wl.rope_theta,
                            wl.rms_eps, tensors, images, routers, nthreads=8)
    try:
        eng = OracleEngine(dec)
        ref = chat.ChatSession(eng, gpu.tok, gpu.tmpl, [299], 1, 0.0, 0.9, 300, out=io.StringIO())
        ref.start("you are a test")
        for ln in lines:
            if not ref.handle(ln):
                break
    finally:
        dec.close()

    got = [t for r in gpu.replies for t in r]
    want = [t for r in ref.replies for t in r]
    assert len(want) > 200
    agree = 0
    for g, (w, clear) in zip(got, eng.steps):
        if g != w:
            assert not clear, f"step {agree}: GPU token {g}, oracle {w} with a clear margin"
            break
        agree += 1
    say(f"chat: {agree} of {len(want)} generated tokens identical")
    if agree == len(want):
        assert gpu.replies == ref.replies and gpu.context == ref.context


def test_converted_checkpoint_decodes_like_the_oracle(tmp_path):
    """A safetensors checkpoint with f32 experts (OLMoE naming, two shards)
    goes through m1moe_amd.convert (the library's quantizer), is loaded by
    m1moe_load_model, and decodes 6 greedy steps within the logit bar of
    the oracle built from the converted files."""
    import m1moe_amd as m
    from m1moe_amd.convert import convert
    from m1moe_amd.decoder import Decoder
    from test_quant import write_safetensors

    wl, seed = synth.DECODERS["tiny_dec"], 41
    L, moe = wl.num_layers, wl.moe.shape(wl.num_layers)
    h, inter, E = moe.hidden, moe.intermediate, moe.num_experts
    rng = np.random.default_rng(seed)
    dense = {}
    for which, name in NAMES.items():
        for l in (range(L) if which in _lib.W_PER_LAYER else [0]):
            dense[(name, l)] = synth.dense_weight(wl, seed, which, l)
    hf = {"embed": "model.embed_tokens.weight", "lm_head": "lm_head.weight",
          "final_norm": "model.norm.weight", "in_norm": "model.layers.{}.input_layernorm.weight",
          "post_norm": "model.layers.{}.post_attention_layernorm.weight",
          "q": "model.layers.{}.self_attn.q_proj.weight", "k": "model.layers.{}.self_attn.k_proj.weight",
          "v": "model.layers.{}.self_attn.v_proj.weight", "o": "model.layers.{}.self_attn.o_proj.weight",
          "q_norm": "model.layers.{}.self_attn.q_norm.weight",
          "k_norm": "model.layers.{}.self_attn.k_norm.weight"}
    shards = [[], []]
    for (name, l), bits in dense.items():
        if name in ("q_norm", "k_norm"):   # Hugging Face length: q_dim / kv_dim
            n = (wl.num_heads if name == "q_norm" else wl.num_kv_heads) * wl.head_dim
            bits = np.concatenate([bits, synth.f32_to_bf16(np.ones(n - bits.size, np.float32))])
        shards[l % 2].append((hf[name].format(l), "BF16", bits))
    routers = []
    for l in range(L):
        r = synth.router(moe, seed, l)
        routers.append(r)
        shards[l % 2].append((f"model.layers.{l}.mlp.gate.weight", "BF16", r.reshape(E, h)))
        for e in range(E):
            for proj, (rows, cols) in (("gate_proj", (inter, h)), ("up_proj", (inter, h)),
                                       ("down_proj", (h, inter))):
                w = (rng.standard_normal((rows, cols)) * 0.05).astype(np.float32)
                shards[e % 2].append((f"model.layers.{l}.mlp.experts.{e}.{proj}.weight", "F32", w))
    src = tmp_path / "ckpt"
    src.mkdir()
    for i, t in enumerate(shards):
        write_safetensors(src / f"model-{i}.safetensors", t)
    out = tmp_path / "conv"
    convert(str(src), str(out), moe.group_size, verbose=False)

    images = [np.fromfile(out / "packed_experts" / f"layer_{l:02d}.bin", np.uint8) for l in range(L)]
    tensors = {name: ([dense[(name, l)] for l in range(L)] if which in _lib.W_PER_LAYER
                      else dense[(name, 0)]) for which, name in NAMES.items()}
    odec = orc.DecoderOracle(orc.from_moe_shape(moe), L, wl.vocab, wl.num_heads, wl.num_kv_heads,
                             wl.head_dim, 16, wl.qk_norm, wl.rope_theta, wl.rms_eps, tensors,
                             images, routers)
    say("converted checkpoint: load_model + 6 decoder steps")
    ctx = m.HIPContext(moe)
    try:
        dec = Decoder(ctx, wl.dec_shape(16))
        ctx.load_model(str(out), dec, threads=2)
        tok = 5
        for step in range(6):
            g_tok, g_lg = dec.forward(tok, return_logits=True)
            w_tok, w_lg = odec.step(tok)
            rel = np.linalg.norm(g_lg - w_lg) / np.linalg.norm(w_lg)
            assert rel < LOGIT_TOL, f"step {step}: rel L2 {rel:.2e}"
            if g_tok != w_tok:
                top2 = np.sort(w_lg.astype(np.float64))[-2:]
                assert top2[1] - top2[0] < 4 * LOGIT_TOL * np.linalg.norm(w_lg) / np.sqrt(w_lg.size)
            tok = w_tok
        dec.close()
    finally:
        ctx.close()
        odec.close()
