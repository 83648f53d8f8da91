"""The chat REPL (Sources/chat/main.swift) on the CPU.

A recording engine stands in for the decoder: it logs every reset, prefill
and forward and answers forwards from a script, so each test pins one rule
of the reference's loop exactly (what is prefilled, which token each step
feeds, where generation stops, how the context is trimmed, what the
commands do).  The GPU test (test_gpu_chat.py) runs the same loop on the
real decoder against the decoder oracle.
"""
from __future__ import annotations

import io
import json

import pytest

from m1moe_amd import chat
from m1moe_amd.tokenizer import Tokenizer

from cases import write_byte_tokenizer

EOS = 299


class ScriptEngine:
    def __init__(self, replies):
        self.replies = list(replies)
        self.log = []

    def reset(self):
        self.log.append(("reset",))

    def prefill(self, tokens):
        self.log.append(("prefill", list(tokens)))

    def forward(self, token, temperature, top_p):
        self.log.append(("forward", int(token), temperature, top_p))
        return self.replies.pop(0)


@pytest.fixture(scope="module")
def tok(tmp_path_factory):
    p = tmp_path_factory.mktemp("tok") / "tokenizer.json"
    write_byte_tokenizer(str(p), EOS)
    return Tokenizer(str(p))


def session(tok, replies, max_ctx=2048, arch="olmoe", **kw):
    out = io.StringIO()
    eng = ScriptEngine(replies)
    s = chat.ChatSession(eng, tok, chat.chat_template({"architecture": arch}), [EOS], 1,
                         temperature=kw.get("temp", 0.0), top_p=kw.get("top_p", 0.9),
                         max_ctx=max_ctx, out=out)
    return s, eng, out


def test_templates_follow_the_config():
    o = chat.chat_template({"architecture": "olmoe"})
    assert (o.user_prefix, o.user_suffix, o.assistant_suffix) == \
        ("<|user|>\n", "\n<|assistant|>\n", "<|endoftext|>\n")
    assert o.system_prefix == "<|system|>\n" and o.system_suffix == "\n"
    m = chat.chat_template({"architecture": "mixtral"})
    assert (m.user_prefix, m.user_suffix, m.assistant_prefix, m.assistant_suffix) == \
        ("[INST] ", " [/INST]", " ", "</s>")
    assert m.system_prefix is None
    c = chat.chat_template({"architecture": "mixtral", "chat": {
        "user_prefix": "U:", "user_suffix": ";", "assistant_prefix": "A:", "assistant_suffix": "."}})
    assert (c.user_prefix, c.assistant_prefix, c.system_prefix) == ("U:", "A:", None)


def test_turn_prefills_feeds_the_last_token_again_and_stops_at_eos(tok):
    s, eng, out = session(tok, [104, 105, EOS])
    s.start("be brief")
    sys_ids = tok.encode("<|system|>\nbe brief\n", add_bos=False)
    user_ids = tok.encode("<|user|>\nhi\n<|assistant|>\n", add_bos=False)
    sfx_ids = tok.encode("<|endoftext|>\n", add_bos=False)
    assert s.handle("  hi\t")
    assert eng.log == [("prefill", sys_ids), ("prefill", user_ids),
                       ("forward", user_ids[-1], 0.0, 0.9),     # the last context token again
                       ("forward", 104, 0.0, 0.9), ("forward", 105, 0.0, 0.9),
                       ("prefill", sfx_ids)]
    assert s.context == sys_ids + user_ids + [104, 105, EOS] + sfx_ids
    assert s.replies == [[104, 105, EOS]]
    text = out.getvalue()
    assert "Bot: hi\n" in text and "ctx %d]" % len(s.context) in text
    assert s.last_stats[0] == 3


def test_first_step_of_an_empty_context_feeds_bos_and_prefix_is_prefilled(tok):
    s, eng, out = session(tok, [EOS], arch="mixtral")
    s.tmpl = chat.ChatSpec("", "", " ", "", None, None)
    s.handle("x")
    assert eng.log[0] == ("prefill", tok.encode("x", add_bos=False))
    assert eng.log[1] == ("prefill", tok.encode(" ", add_bos=False))   # assistant prefix
    assert eng.log[2][:2] == ("forward", tok.encode(" ", add_bos=False)[-1])  # the prefix's last
    s2, eng2, _ = session(tok, [EOS])
    s2.tmpl = chat.ChatSpec("", "", "", "", None, None)
    s2.turn("")
    assert eng2.log == [("prefill", []), ("forward", 1, 0.0, 0.9)]    # bos


def test_stop_string_in_the_reply_tail_ends_the_turn(tok):
    stop = tok.encode("<|user|>", add_bos=False)
    s, eng, out = session(tok, [104, 105] + stop + [106, 107])
    s.handle("q")
    assert s.replies[0] == [104, 105] + stop        # stops right after the stop string
    assert "<|user|>" in out.getvalue()
    # Mixtral's user prefix "[INST] " stops at "[INST]"
    inst = tok.encode("[INST]", add_bos=False)
    s, eng, _ = session(tok, [104] + inst + [105], arch="mixtral")
    s.handle("q")
    assert s.replies[0] == [104] + inst


def test_generation_stops_at_the_context_limit(tok):
    s, eng, _ = session(tok, [104] * 400, max_ctx=300)
    s.handle("hello")
    n_user = len(tok.encode("<|user|>\nhello\n<|assistant|>\n", add_bos=False))
    assert len(s.replies[0]) == 300 - n_user            # context + gen reaches max_ctx


def test_sliding_window_keeps_the_last_half_and_prefills_it_again(tok):
    s, eng, out = session(tok, [104] * 1000, max_ctx=300)
    s.handle("hello")
    before = list(s.context)
    assert len(before) > 150
    eng.log.clear()
    s.handle("again")
    kept = before[-150:]
    assert eng.log[0] == ("reset",) and eng.log[1] == ("prefill", kept)
    assert "[chat] context trimmed to 150 tokens" in out.getvalue()
    user = tok.encode("<|user|>\nagain\n<|assistant|>\n", add_bos=False)
    assert eng.log[2] == ("prefill", user)
    assert s.context[:150] == kept


def test_commands(tok):
    s, eng, out = session(tok, [EOS] * 10)
    s.start(None)
    assert eng.log == []                                  # no system prompt, nothing prefilled
    assert s.handle("/stats")
    assert s.handle("/system")
    assert s.handle("/system   be terse")
    assert s.system_prompt == "  be terse"                # Swift's split keeps the extra spaces
    assert eng.log[-2:] == [("reset",), ("prefill", tok.encode("<|system|>\n  be terse\n",
                                                                add_bos=False))]
    assert s.handle("hi")
    assert s.handle("/stats")
    eng.log.clear()
    assert s.handle("/reset")
    assert eng.log == [("reset",), ("prefill", tok.encode("<|system|>\n  be terse\n",
                                                          add_bos=False))]
    assert s.handle("/nope") and s.handle("/") and s.handle("   ")
    assert not s.handle("/quit")
    assert not s.handle("/q") and not s.handle("/exit")
    text = out.getvalue()
    for want in ("[chat] no stats yet", "[chat] usage: /system <prompt>",
                 "[chat] system prompt updated", "[chat] conversation reset",
                 "[chat] last turn: 1 tokens", "[chat] unknown command: /nope",
                 "[chat] unknown command: /\n", "Bye."):
        assert want in text, want


def test_sampling_arguments_reach_the_engine(tok):
    s, eng, _ = session(tok, [104, EOS], temp=0.7, top_p=0.5)
    s.handle("x")
    assert all(e[2:] == (0.7, 0.5) for e in eng.log if e[0] == "forward")


def test_main_argument_errors(tmp_path, capsys):
    assert chat.main([], io.StringIO(), io.StringIO()) == 1
    assert "--config PATH required" in capsys.readouterr().err
    out = io.StringIO()
    assert chat.main(["--help"], io.StringIO(), out) == 0 and "--max-ctx N" in out.getvalue()
    cfg = tmp_path / "c.json"
    cfg.write_text(json.dumps({"architecture": "olmoe"}))
    assert chat.main(["--config", str(cfg)], io.StringIO(), io.StringIO()) == 1
    assert "no model_dir" in capsys.readouterr().err
    assert chat.main(["--config", str(cfg), "--model", str(tmp_path)], io.StringIO(),
                     io.StringIO()) == 1
    assert "tokenizer.json not found" in capsys.readouterr().err
    a = chat.parse_args(["--temp", "hot", "--top-p", "0.5", "--max-ctx", "64", "--config", "c"])
    assert (a["temp"], a["top_p"], a["max_ctx"], a["config"]) == (0.7, 0.5, 64, "c")
