"""Host logic of the text front end and the perplexity harness on the CPU:
flag parsing (src/cli.rs), the streaming generator's input construction,
EOS handling and text deltas (src/text_generator.rs:38-101) and the
perplexity windowing and NLL accumulation (src/bin/perplexity.rs).  The
model is a stub that returns scripted tokens or log-probabilities; nothing
here launches a kernel.  The tokenizer's own parity is unpinned: the
reference holds no tokenizer fixture, so these tests use a tokenizer.json
written with the same library."""
import io
import math
import os

import numpy as np
import pytest

from sqhip.cli import assets_dir, env_switch, parse_flag
from sqhip import perplexity as P

pytest.importorskip("tokenizers")
from sqhip.text import Tokenizer, generate_text  # noqa: E402
from tokenizer_fixture import CORPUS, write_tokenizer  # noqa: E402


def test_parse_flag_forms():
    argv = ["--model", "a.gguf", "--ctx=256", "--model", "b.gguf", "--prompt"]
    assert parse_flag("--model", "x", argv) == "a.gguf"      # first occurrence
    assert parse_flag("--ctx", "512", argv) == "256"          # --flag=value
    assert parse_flag("--windows", "0", argv) == "0"          # default
    assert parse_flag("--prompt", "dflt", argv) == "dflt"     # flag without a value


def test_assets_dir(tmp_path, monkeypatch):
    monkeypatch.delenv("SQUIRREL_ASSETS", raising=False)
    assert assets_dir(["--assets", str(tmp_path)]) == str(tmp_path)
    monkeypatch.setenv("SQUIRREL_ASSETS", str(tmp_path))
    assert assets_dir([]) == str(tmp_path)
    with pytest.raises(SystemExit):
        assets_dir(["--assets", str(tmp_path / "missing")])


def test_env_switch(monkeypatch):
    monkeypatch.setenv("SQUIRREL_IGNORE_EOS", "0")
    assert not env_switch("SQUIRREL_IGNORE_EOS")
    monkeypatch.setenv("SQUIRREL_IGNORE_EOS", "yes")
    assert env_switch("SQUIRREL_IGNORE_EOS")
    monkeypatch.delenv("SQUIRREL_IGNORE_EOS")
    assert not env_switch("SQUIRREL_IGNORE_EOS")


@pytest.fixture(scope="module")
def tok(tmp_path_factory):
    p = str(tmp_path_factory.mktemp("tok") / "tokenizer.json")
    bos, eos = write_tokenizer(p)
    return Tokenizer(p), bos, eos


def test_tokenizer_round_trip(tok):
    t, bos, eos = tok
    for s in CORPUS[:5] + ["ünïcödé and emoji \U0001F600 survive byte-level BPE"]:
        ids = t.encode(s, False)
        assert t.decode(ids) == s
        with_bos = t.encode(s, True)
        assert with_bos[0] == bos and with_bos[1:] == ids


class StubCtx:
    """Scripted decode: argmax() returns the next scripted token; forward()
    records its input."""

    def __init__(self, script):
        self.script = list(script)
        self.inputs, self.resets = [], 0

    def forward(self, ids):
        self.inputs.append([int(i) for i in ids])

    def argmax(self):
        return self.script.pop(0)

    def reset_cache(self):
        self.resets += 1


class StubModel:
    def __init__(self, eos):
        self.eos = eos

    def eos_token_id(self):
        return self.eos


def scripted(t, text):
    return t.encode(text, False)


def test_generate_text_streams_deltas_and_stops_at_eos(tok, monkeypatch):
    t, bos, eos = tok
    monkeypatch.delenv("SQUIRREL_IGNORE_EOS", raising=False)
    monkeypatch.delenv("SQUIRREL_NO_KV_CACHE", raising=False)
    body = scripted(t, " Paris. The dog sleeps.")
    ctx = StubCtx(body + [eos, 5, 6])
    out, log = io.StringIO(), io.StringIO()
    text = generate_text(StubModel(eos), t, "The capital of France is", 50, ctx=ctx, out=out, log=log)
    assert text == " Paris. The dog sleeps."
    assert out.getvalue() == text + "\n"                 # deltas concatenate to the decoded text
    prompt = t.encode("The capital of France is", True)
    assert ctx.inputs[0] == prompt                       # step 1: the whole prompt with BOS
    assert ctx.inputs[1:] == [[x] for x in body]         # then one token per step
    lines = log.getvalue().splitlines()
    assert lines[0] == f"[prompt: {len(prompt)} tokens]"
    assert lines[-1].endswith("<eos>") and len(lines) == 2 + len(body)


def test_generate_text_ignore_eos_and_max_tokens(tok, monkeypatch):
    t, bos, eos = tok
    monkeypatch.setenv("SQUIRREL_IGNORE_EOS", "1")
    monkeypatch.delenv("SQUIRREL_NO_KV_CACHE", raising=False)
    ctx = StubCtx([eos, 70, eos, 71, 72])
    text = generate_text(StubModel(eos), t, "A", 4, ctx=ctx, out=io.StringIO(), log=io.StringIO())
    assert len(ctx.inputs) == 4                          # max_tokens steps
    assert text == t.decode([eos, 70, eos, 71])          # special tokens skipped in the text


def test_generate_text_no_kv_cache_refeeds_everything(tok, monkeypatch):
    t, bos, eos = tok
    monkeypatch.setenv("SQUIRREL_NO_KV_CACHE", "1")
    monkeypatch.delenv("SQUIRREL_IGNORE_EOS", raising=False)
    ctx = StubCtx([40, 41, 42, eos])
    generate_text(StubModel(eos), t, "A", 10, ctx=ctx, out=io.StringIO(), log=io.StringIO())
    p = t.encode("A", True)
    assert ctx.inputs == [p, p + [40], p + [40, 41], p + [40, 41, 42]]
    assert ctx.resets == 3


# ----------------------------------------------------------------- perplexity

class ScoreCtx:
    def __init__(self, fn):
        self.fn, self.calls = fn, []

    def score(self, window, burn):
        self.calls.append((np.array(window), burn))
        return self.fn(np.array(window), burn)


class PplModel:
    def bos_token_id(self):
        return 7


def test_perplexity_windows_match_the_reference_log():
    """results/perplexity.log: ctx=512, windows=128 -> scored_tokens=32768."""
    ids = np.arange(128 * 511 + 300, dtype=np.uint32) % 1000
    ctx = ScoreCtx(lambda w, b: np.full(w.size - b, -1.0))
    r = P.perplexity(PplModel(), ids, 512, 128, ctx=ctx)
    assert r["windows"] == 128 and r["scored_tokens"] == 32768 and r["burn"] == 256
    assert r["nll_per_token"] == 1.0 and r["ppl"] == math.e
    w0, b0 = ctx.calls[0]
    assert b0 == 256 and w0.size == 512 and w0[0] == 7 and np.array_equal(w0[1:], ids[:511])
    w1, _ = ctx.calls[1]
    assert np.array_equal(w1[1:], ids[511:1022])


def test_perplexity_window_count_and_accumulation():
    ids = np.arange(100, dtype=np.uint32)
    assert P.windows(ids, 16) == (15, 6, 6)
    assert P.windows(ids, 16, 4) == (15, 4, 6)
    assert P.windows(ids, 16, 40) == (15, 6, 6)
    with pytest.raises(ValueError):
        P.windows(ids, 3)
    rng = np.random.default_rng(1)
    vals = {}

    def fn(w, b):
        v = -rng.random(w.size - b) * 5
        vals[len(vals)] = v
        return v

    r = P.perplexity(PplModel(), ids, 16, 0, ctx=ScoreCtx(fn))
    allv = np.concatenate([vals[k] for k in sorted(vals)])
    assert r["scored_tokens"] == 6 * 8 == allv.size
    assert abs(r["nll_per_token"] - (-math.fsum(allv) / allv.size)) < 1e-12
