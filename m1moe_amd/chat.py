"""Interactive multi-turn chat over the decoder (Sources/chat/main.swift).

  python -m m1moe_amd.chat --config PATH [--model DIR] [--system TEXT]
                           [--temp T] [--top-p P] [--max-ctx N]

Commands during chat: /reset, /system TEXT, /stats, /quit (also /exit, /q).

The loop is the reference's (:177-321): the user turn wrapped in the chat
template is encoded and prefilled; the assistant prefix is printed and
prefilled; tokens are generated until an EOS id, a stop string in the last
64 characters of the reply, or the context limit, each decoded on its own
and streamed; the reply's tokens join the context and the assistant suffix
is prefilled.  When context + turn + 256 would exceed --max-ctx, the context
keeps its last max_ctx / 2 tokens and is prefilled again from an empty KV
cache (:252-263).  As in the reference, each reply's first step feeds the
last context token once more (:279), and prompts, templates, special tokens
and the system prompt (--system, else ~/.m1moe/system.md) follow the config
file (ModelSpec.swift:96-146).

What differs is where the work runs: every prefill (system prompt, user
turn, assistant prefix and suffix, the re-prefill after a trim) is one
batched m1moe_dec_prefill on the GPU instead of one forward per token, and
each generated token is one m1moe_dec_step (greedy on the GPU at
temperature 0, else sampled on the host from its logits).
"""
from __future__ import annotations

import json
import os
import sys
import time
from dataclasses import dataclass
from typing import List, Optional, Sequence

import numpy as np

# Swift's CharacterSet.whitespaces: tab and the space separators (Zs)
_WHITESPACE = ("\t\u0020\u00a0\u1680\u2000\u2001\u2002\u2003\u2004\u2005\u2006"
               "\u2007\u2008\u2009\u200a\u202f\u205f\u3000")
# and CharacterSet.newlines
_NEWLINES = "\n\u000b\u000c\r\u0085\u2028\u2029"


@dataclass(frozen=True)
class ChatSpec:
    """ChatSpec (ModelSpec.swift:104-117)."""

    user_prefix: str
    user_suffix: str
    assistant_prefix: str
    assistant_suffix: str
    system_prefix: Optional[str] = None
    system_suffix: Optional[str] = None


def chat_template(config: dict) -> ChatSpec:
    """ModelSpec.chatTemplate (ModelSpec.swift:122-146): the config's "chat"
    object if present, else the architecture's default."""
    c = config.get("chat")
    if isinstance(c, dict):
        return ChatSpec(c["user_prefix"], c["user_suffix"], c["assistant_prefix"],
                        c["assistant_suffix"], c.get("system_prefix"), c.get("system_suffix"))
    if config.get("architecture") == "mixtral":
        return ChatSpec("[INST] ", " [/INST]", " ", "</s>", None, None)
    return ChatSpec("<|user|>\n", "\n<|assistant|>\n", "", "<|endoftext|>\n", "<|system|>\n", "\n")


def split_command(text: str):
    """Swift's split(separator: " ", maxSplits: 1) of the text after '/':
    leading spaces give no part, the second part keeps further spaces."""
    s = text.lstrip(" ")
    if not s:
        return []
    i = s.find(" ")
    if i < 0 or i + 1 >= len(s):
        return [s[:i] if i >= 0 else s]
    return [s[:i], s[i + 1:]]


class DecoderEngine:
    """InferenceEngine's forward / reset over a Decoder, with batched prefill."""

    def __init__(self, decoder, seed: Optional[int] = None):
        self.dec = decoder
        self.rng = np.random.default_rng(seed)

    def reset(self) -> None:
        self.dec.reset()

    def prefill(self, tokens: Sequence[int]) -> None:
        if len(tokens):
            self.dec.prefill(np.asarray(tokens, np.int32))

    def forward(self, token: int, temperature: float, top_p: float) -> int:
        return int(self.dec.forward(int(token), temperature=temperature, top_p=top_p,
                                    rng=self.rng))


class ChatSession:
    """The REPL state of Sources/chat/main.swift (:146-321) over any engine
    with reset(), prefill(tokens) and forward(token, temperature, top_p)."""

    def __init__(self, engine, tokenizer, template: ChatSpec, eos: Sequence[int], bos: int,
                 temperature: float = 0.7, top_p: float = 0.9, max_ctx: int = 2048,
                 out=None, clock=time.perf_counter):
        self.engine, self.tok, self.tmpl = engine, tokenizer, template
        self.eos, self.bos = set(int(e) for e in eos), int(bos)
        self.temperature, self.top_p, self.max_ctx = float(temperature), float(top_p), int(max_ctx)
        self.out = out or sys.stdout
        self.clock = clock
        self.context: List[int] = []
        self.system_prompt: Optional[str] = None
        self.last_stats = (0, 0.0)
        self.replies: List[List[int]] = []   # generated ids per turn

    def say(self, text: str = "", end: str = "\n") -> None:
        self.out.write(text + end)
        self.out.flush()

    def prefill_tokens(self, tokens: Sequence[int]) -> int:
        self.engine.prefill(list(tokens))
        self.context.extend(int(t) for t in tokens)
        return len(tokens)

    def reset_conversation(self) -> None:
        self.engine.reset()
        self.context.clear()
        self.say("[chat] conversation reset")

    def reprefill_context(self) -> None:
        self.engine.reset()
        self.engine.prefill(list(self.context))

    def _prefill_system(self, text: Optional[str]) -> None:
        t = self.tmpl
        if text is not None and t.system_prefix is not None and t.system_suffix is not None:
            self.prefill_tokens(self.tok.encode(t.system_prefix + text + t.system_suffix,
                                                add_bos=False))

    def start(self, system_prompt: Optional[str]) -> None:
        self.system_prompt = system_prompt
        self._prefill_system(system_prompt)

    def handle(self, line: str) -> bool:
        """One input line; False when the chat should end."""
        text = line.strip(_WHITESPACE)
        if not text:
            return True
        if text.startswith("/"):
            parts = split_command(text[1:])
            cmd = parts[0] if parts else ""
            arg = parts[1] if len(parts) > 1 else ""
            if cmd in ("quit", "exit", "q"):
                self.say("Bye.")
                return False
            if cmd == "reset":
                self.reset_conversation()
                self._prefill_system(self.system_prompt)
            elif cmd == "system":
                if not arg:
                    self.say("[chat] usage: /system <prompt>")
                    return True
                self.system_prompt = arg
                self.reset_conversation()
                self._prefill_system(arg)
                self.say("[chat] system prompt updated")
            elif cmd == "stats":
                n, ms = self.last_stats
                if n > 0:
                    per = ms / n
                    self.say("[chat] last turn: %d tokens, %.1f ms/tok (%.2f tok/s)"
                             % (n, per, 1000.0 / per if per > 0 else float("inf")))
                else:
                    self.say("[chat] no stats yet")
            else:
                self.say(f"[chat] unknown command: /{cmd}")
            return True
        self.turn(text)
        return True

    def turn(self, text: str) -> List[int]:
        t = self.tmpl
        user = self.tok.encode(t.user_prefix + text + t.user_suffix, add_bos=False)
        if len(self.context) + len(user) + 256 > self.max_ctx:
            keep = self.max_ctx // 2
            if len(self.context) > keep:
                self.context = self.context[len(self.context) - keep:]
                self.say("[chat] context trimmed to %d tokens" % len(self.context))
                self.reprefill_context()
        self.prefill_tokens(user)
        self.say("Bot: " + t.assistant_prefix, end="")
        if t.assistant_prefix:
            self.prefill_tokens(self.tok.encode(t.assistant_prefix, add_bos=False))
        gen: List[int] = []
        ms: List[float] = []
        reply = ""
        stops = [s for s in (t.user_prefix.strip(_WHITESPACE + _NEWLINES), "<|user|>", "[INST]",
                             "<|endoftext|>") if s]
        while True:
            t0 = self.clock()
            feed = gen[-1] if gen else (self.context[-1] if self.context else self.bos)
            tok = self.engine.forward(feed, self.temperature, self.top_p)
            ms.append((self.clock() - t0) * 1000.0)
            gen.append(int(tok))
            if tok in self.eos:
                break
            piece = self.tok.decode([tok], skip_special=True)
            reply += piece
            self.say(piece, end="")
            tail = reply[-64:]
            if any(s in tail for s in stops):
                break
            if len(self.context) + len(gen) >= self.max_ctx:
                break
        self.say()
        self.context.extend(gen)
        if t.assistant_suffix:
            self.prefill_tokens(self.tok.encode(t.assistant_suffix, add_bos=False))
        self.last_stats = (len(gen), float(sum(ms)))
        if len(ms) > 1:
            mean = sum(ms) / len(ms)
            self.say("  [%.0f ms/tok · %.1f tok/s · ctx %d]"
                     % (mean, 1000.0 / mean if mean > 0 else float("inf"), len(self.context)))
        self.replies.append(gen)
        return gen


_USAGE = """\
M1MoE chat — interactive multi-turn conversation

--config  PATH   Model JSON config (required)
--model   PATH   Override model_dir from config
--system  TEXT   System prompt text
--temp    T      Sampling temperature (default: 0.7)
--top-p   P      Nucleus threshold (default: 0.9)
--max-ctx N      Max context tokens before sliding window (default: 2048)

During chat:
  /reset         Clear history and KV cache
  /system TEXT   Set new system prompt
  /stats         Show last-turn timing
  /quit          Exit"""


def parse_args(argv: Sequence[str]) -> dict:
    """The reference's argument loop (:24-56): a flag whose value is missing
    or does not parse is skipped and the value is read as the next flag."""
    a = {"config": None, "model": None, "system": None, "temp": 0.7, "top_p": 0.9,
         "max_ctx": 2048, "help": False}
    rest = list(argv)
    conv = {"--temp": ("temp", float), "--top-p": ("top_p", float), "--max-ctx": ("max_ctx", int),
            "--config": ("config", str), "--model": ("model", str), "--system": ("system", str)}
    while rest:
        f = rest.pop(0)
        if f in ("--help", "-h"):
            a["help"] = True
            return a
        if f in conv and rest:
            key, ty = conv[f]
            try:
                a[key] = ty(rest[0])
            except ValueError:
                continue
            rest.pop(0)
    return a


def main(argv: Optional[Sequence[str]] = None, stdin=None, stdout=None) -> int:
    stdin, stdout = stdin or sys.stdin, stdout or sys.stdout
    a = parse_args(sys.argv[1:] if argv is None else argv)
    if a["help"]:
        stdout.write(_USAGE + "\n")
        return 0
    if not a["config"]:
        sys.stderr.write("ERROR: --config PATH required\n")
        return 1
    try:
        with open(a["config"], "r", encoding="utf-8") as f:
            config = json.load(f)
    except (OSError, ValueError) as e:
        sys.stderr.write(f"ERROR: {e}\n")
        return 1
    model_dir = a["model"] or config.get("model_dir")
    if not model_dir:
        sys.stderr.write("ERROR: no model_dir — set in config or pass --model\n")
        return 1
    tok_path = os.path.join(model_dir, "tokenizer.json")
    if not os.path.exists(tok_path):
        sys.stderr.write(f"ERROR: tokenizer.json not found in {model_dir}\n")
        return 1

    try:
        serve(config, model_dir, a, stdin, stdout)
    except ValueError as e:
        sys.stderr.write(f"ERROR: {e}\n")
        return 1
    return 0


def repl(session: ChatSession, stdin, stdout) -> None:
    """Reads lines until EOF or /quit (:198-320)."""
    stdout.write("Type your message. Commands: /reset /system /stats /quit\n\n")
    while True:
        stdout.write("You: ")
        stdout.flush()
        line = stdin.readline()
        if not line:
            break
        # readLine(strippingNewline: true) drops one "\n" or "\r\n"
        line = line[:-2] if line.endswith("\r\n") else line[:-1] if line.endswith("\n") else line
        if not session.handle(line):
            break


def serve(config: dict, model_dir: str, args: dict, stdin, stdout) -> ChatSession:
    """Loads the converted model directory and its tokenizer.json onto the
    GPU, runs the REPL over stdin/stdout, frees the device; returns the
    session (its context and replies) for inspection."""
    from .decoder import Decoder, DecoderSpec
    from .engine import HIPContext, ModelSpec
    from .tokenizer import Tokenizer

    t0 = time.perf_counter()
    spec, dspec = ModelSpec.from_dict(config), DecoderSpec.from_dict(config)
    kv = dspec.attention.gpu_kv_seq_prealloc
    if args["max_ctx"] > kv - 64:
        raise ValueError(f"--max-ctx {args['max_ctx']} needs a KV cache of at least "
                         f"{args['max_ctx'] + 64} positions; the config preallocates {kv}")
    tok = Tokenizer(os.path.join(model_dir, "tokenizer.json"))
    ctx = HIPContext(spec.shape())
    try:
        dec = Decoder(ctx, dspec.dec_shape())
        ctx.load_model(model_dir, dec)
        st = config.get("special_tokens", {})
        stdout.write("[chat] %s ready in %.0f ms  (temp=%.1f top-p=%.1f)\n"
                     % (config.get("name", ""), (time.perf_counter() - t0) * 1000.0,
                        args["temp"], args["top_p"]))
        system = args["system"]
        sys_file = os.path.join(os.path.expanduser("~"), ".m1moe", "system.md")
        if system is None and os.path.exists(sys_file):
            with open(sys_file, "r", encoding="utf-8") as f:
                system = f.read().strip(_WHITESPACE + _NEWLINES)
            stdout.write(f"[chat] system prompt loaded from ~/.m1moe/system.md "
                         f"({len(system)} chars)\n")
        session = ChatSession(DecoderEngine(dec), tok, chat_template(config),
                              st.get("eos", []), int(st.get("bos", 1)), args["temp"],
                              args["top_p"], args["max_ctx"], out=stdout)
        session.start(system)
        repl(session, stdin, stdout)
        dec.close()
    finally:
        ctx.close()
    return session


if __name__ == "__main__":
    raise SystemExit(main())
