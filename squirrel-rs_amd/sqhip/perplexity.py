"""Perplexity harness (src/bin/perplexity.rs): teacher-forced NLL over
windows of a token stream, f64 log-softmax per scored position.

Windows of n_ctx tokens: BOS followed by the next n_ctx - 1 tokens of the
stream (only whole windows).  Each window runs on a fresh cache: a prefill
of the first n_ctx / 2 tokens (the burn-in), then every later token is scored
from the current logits and fed as the next decode step.  One window is one
sq_ctx_score call: the whole loop stays on the GPU and the window's
log-probabilities come back with one copy; they are summed here in the
reference's order (window_nll -= each value, total_nll += window_nll).

    python -m sqhip.perplexity --model Llama-3.2-1B-Instruct-Q8_0.gguf \\
        --text wikitext2-raw-test.txt [--ctx 512] [--windows 0] [--assets DIR]
    python -m sqhip.perplexity --model M.gguf --ids ids.npy ...   (token ids)
"""
from __future__ import annotations

import math
import sys
import time

import numpy as np

from .cli import assets_dir, env_switch, parse_flag
from .model import Llama3_2


def windows(ids, n_ctx: int, max_windows: int = 0) -> tuple[int, int, int]:
    """(per_window, n_windows, n_windows_total) as perplexity.rs:42-49."""
    if n_ctx < 4:
        raise ValueError("--ctx must be at least 4")
    per_window = n_ctx - 1
    total = len(ids) // per_window
    n = total if max_windows == 0 else min(max_windows, total)
    return per_window, n, total


def perplexity(model, ids, n_ctx: int = 512, max_windows: int = 0, ctx=None, log=None) -> dict:
    """perplexity.rs:42-101 on token ids; returns the summary values."""
    ids = np.ascontiguousarray(ids, dtype=np.uint32)
    per_window, n_windows, total = windows(ids, n_ctx, max_windows)
    burn = n_ctx // 2
    bos = model.bos_token_id()
    if ctx is None:
        ctx = model.new_context(n_ctx)
    t0 = time.perf_counter()
    total_nll, scored = 0.0, 0
    for w in range(n_windows):
        window = np.empty(n_ctx, np.uint32)
        window[0] = bos
        window[1:] = ids[w * per_window:(w + 1) * per_window]
        logp = ctx.score(window, burn)
        window_nll = 0.0
        for v in logp:
            window_nll -= float(v)
        scored += logp.size
        total_nll += window_nll
        if log is not None:
            print(f"[window {w + 1:>4}/{n_windows}] ppl so far: {math.exp(total_nll / scored):.4f}  "
                  f"({time.perf_counter() - t0:.1f}s)", file=log)
    nll = total_nll / scored if scored else float("nan")
    return dict(windows=n_windows, windows_total=total, burn=burn, scored_tokens=scored, nll_per_token=nll,
                ppl=math.exp(nll) if scored else float("nan"), time_s=time.perf_counter() - t0)


def main(argv=None) -> int:
    assets = assets_dir(argv)
    model_file = parse_flag("--model", "Llama-3.2-1B-Instruct-Q8_0.gguf", argv)
    ids_path = parse_flag("--ids", "", argv)
    n_ctx = int(parse_flag("--ctx", "512", argv))
    max_windows = int(parse_flag("--windows", "0", argv))
    if n_ctx < 4:
        raise SystemExit("--ctx must be at least 4")
    model = Llama3_2(f"{assets}/{model_file}")
    if ids_path:
        ids = np.load(ids_path) if ids_path.endswith(".npy") else np.loadtxt(ids_path, dtype=np.int64)
        ids = np.asarray(ids, dtype=np.uint32).ravel()
    else:
        from .text import Tokenizer
        text_path = parse_flag("--text", f"{assets}/wikitext2-raw-test.txt", argv)
        with open(text_path) as fh:
            text = fh.read()
        ids = np.asarray(Tokenizer(f"{assets}/tokenizer.json").encode(text, False), dtype=np.uint32)
    # The f32-activation path is switched off in this build; the run uses the
    # integer path and says so.
    acts = "f32" if env_switch("SQUIRREL_F32_ACTS") else "int8(where applicable)"
    if acts == "f32":
        raise SystemExit("SQUIRREL_F32_ACTS: the f32-activation kernels are switched off in this build")
    per_window, n_windows, total = windows(ids, n_ctx, max_windows)
    print(f"model={model_file} acts={acts} corpus={ids.size} tokens ctx={n_ctx} burn-in={n_ctx // 2} "
          f"windows={n_windows}/{total}", file=sys.stderr)
    r = perplexity(model, ids, n_ctx, max_windows, log=sys.stderr)
    print(f"model={model_file} acts={acts} ctx={n_ctx} windows={r['windows']} scored_tokens={r['scored_tokens']} "
          f"nll_per_token={r['nll_per_token']:.6f} ppl={r['ppl']:.4f} time_s={r['time_s']:.1f}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
