#!/usr/bin/env python3
"""Benchmark: batch-1 greedy decode of the Llama-3.2-1B-shaped Q8_0 model.

`python bench.py [--gpus 1] [--steps K] [--warmup W] [--config q8|q4|bf16|long|prefill]`

A step is one decode token (forward + greedy sample) of the token loop,
timed with HIP events on the context stream; the prompt's prefill is step 0
and is reported separately as prefill tok/s (the reference's convention:
decode throughput excludes step 1, scripts/bench.py:68-71).  Weights are
random-init from a fixed seed (synthetic data; no checkpoint is available).

One JSON line is printed.  `roofline` prices the dominant kernel against
MI355X's 8 TB/s HBM peak using its algorithmic bytes and its mean duration
measured here with HIP events: the persistent decode-step kernel (one launch
per token), or with --multi-kernel the fused gate/up matvec; `cpu_baseline` is the
oracle (the C restatement of the reference's x86 scalar path) timed on this
host over a bounded sample of the same workload.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
for _p in (REPO, os.path.join(REPO, "squirrel-rs_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import numpy as np  # noqa: E402

METRIC = "decode tok/s batch-1 (1B Q8_0/Q4_0) + % HBM roofline; prefill tok/s"
HBM_PEAK_GBS = 8000.0
CONFIGS = {
    "q8": dict(wtype="Q8_0", prompt=32, gen=64,
               workload="Llama-3.2-1B arch, Q8_0 GGUF, 32-token prompt then 64 greedy tokens"),
    "q4": dict(wtype="Q4_0", prompt=128, gen=256,
               workload="Llama-3.2-1B arch, Q4_0 GGUF, 128-token prompt then 256 greedy tokens"),
    "bf16": dict(wtype="BF16", prompt=128, gen=256,
                 workload="Llama-3.2-1B arch, BF16 GGUF, 128-token prompt then 256 greedy tokens"),
    "long": dict(wtype="Q8_0", prompt=4096, gen=128,
                 workload="Llama-3.2-1B arch, Q8_0, 4096-token fp32 KV cache then 128 greedy tokens"),
    "prefill": dict(wtype="Q8_0", prompt=2048, gen=16,
                    workload="Llama-3.2-1B arch, Q8_0, 2048-token batched prefill then 16 greedy tokens"),
}
KERNELS = {0: "gate_up_matvec", 1: "lm_head_matvec", 2: "down_matvec", 3: "qkv_matvec",
           4: "attention_split", 5: "o_proj_matvec"}


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def model_path(wtype: str, seed: int) -> str:
    import sqhip
    d = os.environ.get("SQHIP_MODEL_DIR", "/tmp/sqhip_models")
    os.makedirs(d, exist_ok=True)
    p = os.path.join(d, f"llama1b_{wtype}_seed{seed}.gguf")
    if not os.path.exists(p):
        t0 = time.time()
        sqhip.write_synthetic_gguf(p + ".tmp", wtype, seed=seed)
        os.replace(p + ".tmp", p)
        log(f"wrote {p} in {time.time() - t0:.1f}s")
    return p


def bytes_per_token(info, P: int) -> int:
    """Algorithmic HBM bytes of one decode step at P attended positions:
    every matrix once, 2L+1 norm vectors, one embedding row, K/V reads of P
    rows and one K/V row write per layer, the logits write."""
    D, L = info.dim, info.n_layers
    kvd = info.n_kv_heads * info.head_dim
    emb_row = {8: D // 32 * 34, 2: D // 32 * 18, 30: D * 2}[info.wtype]
    return (info.weight_bytes + (2 * L + 1) * D * 4 + emb_row + 2 * L * kvd * 4 * P
            + 2 * L * kvd * 4 + info.vocab * 4)


def cpu_baseline(path: str, prompt: np.ndarray, n_decode: int, reps: int = 4) -> dict:
    """The oracle's W8A32 decode rate: `reps` runs of the workload's decode
    steps, each after an untimed prefill of the same prompt (about 10 s of
    CPU work at the default workload)."""
    from oracle import oracle as O
    threads = min(16, os.cpu_count() or 1)
    O.set_threads(threads)
    m = O.OracleModel(path)
    dt = 0.0
    for _ in range(reps):
        c = m.new_context(len(prompt) + n_decode + 1, O.W8A32)
        c.forward(prompt)
        tok = O.greedy(c.logits())
        t0 = time.perf_counter()
        for _ in range(n_decode):
            c.forward([tok])
            tok = O.greedy(c.logits())
        dt += time.perf_counter() - t0
        c.close()
    return {"value": round(reps * n_decode / dt, 3), "unit": "tok/s", "cores": threads, "kind": "port",
            "sample": f"{reps} x ({len(prompt)}-token prefill, untimed, then {n_decode} timed decode steps) "
                      f"of the same GGUF; C restatement of the reference's x86 scalar-fallback path "
                      f"(f32 activations, W8A32), {threads} threads"}


def copy_calibration(mib: int) -> int:
    """A plain HBM-to-HBM copy of known size, for scaling PMC byte counters."""
    import torch
    n = mib << 20
    src = torch.empty(n, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    src.fill_(1)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    log(f"copy calibration: 5 copies of {n} bytes (read {n}, write {n} per copy)")
    return 0


def measured_traffic(kernel: str, config: str):
    """HBM bytes per launch of the dominant kernel from the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE runs (scaled by the copy calibration),
    or None when no measurement exists for this kernel and workload."""
    path = os.path.join(REPO, "profiles", f"traffic_{kernel}_{config}.json")
    try:
        with open(path) as f:
            return int(json.load(f)["traffic_bytes_per_launch"])
    except (OSError, ValueError, KeyError):
        return None


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None, help="decode steps timed")
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--config", default="q8", choices=sorted(CONFIGS))
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-steps", type=int, default=None,
                    help="decode steps timed on the CPU (default: the same count as the GPU run)")
    ap.add_argument("--kernel-iters", type=int, default=200)
    ap.add_argument("--multi-kernel", action="store_true",
                    help="decode with one kernel per op (hipGraph) instead of the persistent step kernel")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run a plain device-to-device copy of MIB MiB five times (the known-size "
                         "reference that scales rocprofv3 FETCH_SIZE / WRITE_SIZE readings), then exit")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (the token loop is a "
              "batch-1 single-device workload); run with --gpus 1", file=sys.stderr)
        return 2

    if args.copy_calibration:
        return copy_calibration(args.copy_calibration)

    import sqhip
    cfg = CONFIGS[args.config]
    K = args.steps if args.steps is not None else cfg["gen"] - 1
    W = args.warmup
    path = model_path(cfg["wtype"], args.seed)
    t0 = time.time()
    model = sqhip.Llama3_2(path)
    info = model.info
    log(f"loaded {path} ({info.weight_bytes / 1e6:.1f} MB of matrices) in {time.time() - t0:.1f}s")
    S = cfg["prompt"]
    prompt = np.random.default_rng(args.seed).integers(0, info.vocab, S).astype(np.uint32)
    ctx = model.new_context(S + max(K, W) + 2, persistent=not args.multi_kernel)
    gen = sqhip.TextTokenGenerator(model, ctx)

    if W > 0:
        gen.generate(prompt, W + 1, ignore_eos=True)
        log(f"warmup: {W} decode steps")
    sqhip.check(sqhip.lib().sq_synchronize())
    wall0 = time.perf_counter()
    toks, ms = gen.generate(prompt, K + 1, ignore_eos=True)
    sqhip.check(sqhip.lib().sq_synchronize())
    wall = time.perf_counter() - wall0
    assert len(toks) == K + 1, "generation stopped early"
    prefill_ms = float(ms[0])
    decode_ms = float(np.sum(ms[1:K + 1]))
    tok_s = K / (decode_ms / 1e3)
    log(f"prefill {S} tokens: {prefill_ms:.2f} ms; decode {K} steps: {decode_ms:.2f} ms "
        f"({tok_s:.1f} tok/s); wall {wall * 1e3:.1f} ms")

    avg_bytes = np.mean([bytes_per_token(info, S + k) for k in range(1, K + 1)])
    step_gbs = avg_bytes / (decode_ms / K / 1e3) / 1e9

    kernels = {}
    for which, name in KERNELS.items():
        us, nbytes = ctx.time_kernel(which, args.kernel_iters)
        kernels[name] = {"mean_us": round(us, 3), "bytes": int(nbytes),
                         "gbs": round(nbytes / us / 1e3, 1)}
    if ctx.persistent:
        # The whole decode step is one kernel: its algorithmic bytes per launch
        # over its mean duration from the HIP events around every step.
        roofline = {"bound": "hbm", "achieved": round(step_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": round(step_gbs / HBM_PEAK_GBS, 4),
                    "traffic": measured_traffic("decode_step", args.config),
                    "kernel": "decode_step_kernel (persistent: one launch per token, all 16 layers + "
                              "LM head + argmax)",
                    "bytes_per_launch": int(avg_bytes)}
    else:
        dom = kernels["gate_up_matvec"]
        roofline = {"bound": "hbm", "achieved": dom["gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": round(dom["gbs"] / HBM_PEAK_GBS, 4),
                    "traffic": measured_traffic("gate_up_matvec", args.config),
                    "kernel": "gate_up_matvec (RMSNorm+Q8 prologue, 16384x2048 Q8_0 matvec, "
                              "SiLU*up+Q8 epilogue)"}

    cpu = None
    if not args.no_cpu:
        t1 = time.time()
        cpu = cpu_baseline(path, prompt[:32], args.cpu_steps if args.cpu_steps is not None else min(K, 64))
        log(f"cpu baseline {cpu['value']} tok/s in {time.time() - t1:.1f}s")

    line = {
        "metric": METRIC, "value": round(tok_s, 2), "unit": "tok/s", "n_gpus": 1, "steps": K,
        "warmup": W, "ms_per_step": round(decode_ms / K, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "int8" if cfg["wtype"] != "BF16" else "f32",
        "data": "synthetic (seeded random-init weights, random prompt ids)",
        "config": {"workload": cfg["workload"], "weights": cfg["wtype"], "prompt_tokens": S,
                   "generated_tokens": K + 1, "batch": 1, "kv_cache": "fp32", "parallelism": "none"},
        "prefill_tok_s": round(S / (prefill_ms / 1e3), 1),
        "decode_step_hbm": {"bytes_per_token": int(avg_bytes), "achieved_gbs": round(step_gbs, 1),
                            "frac": round(step_gbs / HBM_PEAK_GBS, 4)},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "kernels": kernels,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
