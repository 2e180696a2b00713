"""Command-line helpers shared by the text generator and the perplexity
harness: parse_flag and assets_dir (src/cli.rs:3-33) and the reference's
environment switches."""
from __future__ import annotations

import os
import sys


def parse_flag(flag: str, default: str, argv=None) -> str:
    """`--flag value` or `--flag=value`, the first occurrence (cli.rs:3-16)."""
    args = list(sys.argv[1:] if argv is None else argv)
    prefix = flag + "="
    i = 0
    while i < len(args):
        a = args[i]
        if a == flag:
            if i + 1 < len(args):
                return args[i + 1]
        elif a.startswith(prefix):
            return a[len(prefix):]
        i += 1
    return default


def assets_dir(argv=None) -> str:
    """--assets, else SQUIRREL_ASSETS, else ./assets; it must exist (cli.rs:19-33)."""
    d = parse_flag("--assets", "", argv)
    if not d:
        d = os.environ.get("SQUIRREL_ASSETS", "") or "assets"
    if not os.path.isdir(d):
        raise SystemExit(f"Unable to find assets directory {d!r}. Please use the --assets flag or the "
                         "SQUIRREL_ASSETS environment variable to point to the GGUF and tokenizer files.")
    return d


def env_switch(name: str) -> bool:
    """Set and not "0" (text_generator.rs:10-20, linear.rs:14-19)."""
    v = os.environ.get(name)
    return v is not None and v != "0"
