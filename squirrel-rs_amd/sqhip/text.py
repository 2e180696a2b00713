"""Text front end: the tokenizer.json BPE tokenizer, the streaming text
generator and the `main.rs` command line.

The reference tokenizes with the `tokenizers` crate (0.23.1, BPE from
tokenizer.json: Cargo.toml:16, src/models/llama/model.rs:21-22); here the
same library's Python binding does, on the host, outside the timed region as
in the reference (text_generator.rs:42-46,84-94).  Every forward and every
greedy sample runs on the GPU through the C ABI.

    python -m sqhip.text --model Llama-3.2-1B-Instruct-Q8_0.gguf \\
        --prompt "The capital of France is" [--max-tokens 512] [--assets DIR]
"""
from __future__ import annotations

import json
import sys
import time

from .cli import assets_dir, env_switch, parse_flag
from .model import Llama3_2


class Tokenizer:
    """A tokenizer.json tokenizer (encode with or without special tokens,
    decode skipping them), as the reference calls it."""

    def __init__(self, path: str):
        try:
            from tokenizers import Tokenizer as _Tok
        except ImportError as e:  # the text front end needs the library; ids do not
            raise RuntimeError("the text front end needs the `tokenizers` package") from e
        self._t = _Tok.from_file(path)

    def encode(self, text: str, add_special_tokens: bool) -> list[int]:
        return list(self._t.encode(text, add_special_tokens=add_special_tokens).ids)

    def decode(self, ids, skip_special_tokens: bool = True) -> str:
        return self._t.decode([int(i) for i in ids], skip_special_tokens=skip_special_tokens)


def generate_text(model, tokenizer, prompt: str, max_tokens: int, ctx=None, out=None, log=None) -> str:
    """TextTokenGenerator::generate (text_generator.rs:38-101) with greedy
    sampling: encode with special tokens, one prefill, then one decode step
    per token; each step's new text is printed as soon as it is decoded and
    its latency (forward + sample) goes to the log.  SQUIRREL_IGNORE_EOS and
    SQUIRREL_NO_KV_CACHE act as in the reference.  Returns the generated
    text."""
    out = sys.stdout if out is None else out
    log = sys.stderr if log is None else log
    ids = tokenizer.encode(prompt, True)
    prompt_len = len(ids)
    print(f"[prompt: {prompt_len} tokens]", file=log)
    no_kv, ignore_eos = env_switch("SQUIRREL_NO_KV_CACHE"), env_switch("SQUIRREL_IGNORE_EOS")
    eos = model.eos_token_id()
    if ctx is None:
        # The reference's context grows; this one holds the whole sequence.
        ctx = model.new_context(max(1, min(prompt_len + max_tokens, model.info.context_length)))
    tokens = list(ids)
    inp = list(tokens)
    printed = ""
    for step in range(1, max_tokens + 1):
        t0 = time.perf_counter()
        ctx.forward(inp)
        nxt = ctx.argmax()
        ms = (time.perf_counter() - t0) * 1000.0
        if nxt == eos and not ignore_eos:
            print(f"[step {step:>3}: {ms:>7.1f}ms]  <eos>", file=log)
            break
        tokens.append(nxt)
        if no_kv:
            ctx.reset_cache()
            inp = list(tokens)
        else:
            inp = [nxt]
        full = tokenizer.decode(tokens[prompt_len:], True)
        new_text = full[len(printed):]
        print(f"[step {step:>3}: {ms:>7.1f}ms]  {json.dumps(new_text)}", file=log)
        out.write(new_text)
        out.flush()
        printed = full
    out.write("\n")
    return printed


def main(argv=None) -> int:
    """main.rs:7-39."""
    assets = assets_dir(argv)
    model_file = parse_flag("--model", "Llama-3.2-1B-Instruct-Q8_0.gguf", argv)
    prompt_file = parse_flag("--prompt-file", "", argv)
    if prompt_file:
        with open(prompt_file) as fh:
            prompt = fh.read().rstrip()
    else:
        prompt = parse_flag("--prompt", "The capital of France is", argv)
    max_tokens = int(parse_flag("--max-tokens", "512", argv))
    model = Llama3_2(f"{assets}/{model_file}")
    tokenizer = Tokenizer(f"{assets}/tokenizer.json")
    output = generate_text(model, tokenizer, prompt, max_tokens)
    print(f"{prompt}{output}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
