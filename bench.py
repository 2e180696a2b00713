#!/usr/bin/env python3
"""Benchmark: batch-1 prefill + greedy decode of the Llama-3.2-1B-shaped model.

`python bench.py [--gpus 1] [--steps K] [--warmup W] [--config q8|q4|q8_q4|long|prefill] [--only]`

The headline is the Q8_0 workload (32-token prompt, then greedy tokens): a
step is one decode token (forward + greedy sample), timed with HIP events on
the context stream; the prompt's prefill is step 0 and is reported separately
as prefill tok/s (the reference's convention: decode throughput excludes step
1, scripts/bench.py:68-71).  Unless --only is given, the same run then
measures the other workloads -- Q4_0 (128 + 256, and the same on the Q8_0
weights), a 4096-position context (+128) and a 2048-token batched prefill
(+16) -- each in its own block of
`configs` with its own roofline.  The BF16 workload is reported as not run
(its kernels are switched off on the device).  Weights are random-init from a
fixed seed (synthetic data; no checkpoint is available).

One JSON line is printed.  `roofline` prices the decode step (one persistent
kernel launch per token) against MI355X's 8 TB/s HBM peak using its
algorithmic bytes and its mean duration measured here with HIP events; the
prefill block prices its integer matmuls against the 5.0 POP/s int8 peak and
its attention (f32 operands split into f16 halves, three f16 products per
f32 product) against the 2.5 PFLOP/s f16 matrix-core peak.
`cpu_baseline` is the oracle (the C restatement of the reference's x86 scalar
path) timed on this host, on the reference's thread count (all available
logical cores), over a bounded sample of the headline workload.
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
INT8_PEAK_TOPS = 5000.0     # dense int8 matrix-core peak
FP32_MFMA_PEAK_TFLOPS = 157.3
F16_MFMA_PEAK_TFLOPS = 2500.0  # dense f16 matrix-core peak
# f16 matrix products per f32 product in the prefill attention (hi*hi,
# hi*lo, lo*hi of the split operands); SQUIRREL_ATTN_F32=1 runs it on the
# fp32 matrix instructions instead
ATTN_F16_PRODUCTS = 3
# Matrix elements per layer of the 1B shape: QKV 2048x3072, o 2048x2048,
# gate/up 2048x16384, down 8192x2048.
MATMUL_ELEMS_PER_LAYER = 60817408
# per output element per 32-block in the int8 matmul: the convert of the
# integer block sum and the fused multiply-add (the scale product comes from
# the f16 matrix instruction)
VALU_RESCALE_OPS = 2
CONFIGS = {
    "q8": dict(wtype="Q8_0", prompt=32, gen=64,
               workload="Llama-3.2-1B arch, Q8_0 GGUF, 32-token prompt then 64 greedy tokens"),
    "q4": dict(wtype="Q4_0", prompt=128, gen=256,
               workload="Llama-3.2-1B arch, Q4_0 GGUF, 128-token prompt then 256 greedy tokens"),
    # the Q4_0 workload on Q8_0 weights: the two weight types at the same positions
    "q8_q4": dict(wtype="Q8_0", prompt=128, gen=256,
                  workload="Llama-3.2-1B arch, Q8_0 GGUF, 128-token prompt then 256 greedy tokens"),
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


def available_parallelism() -> int:
    """The thread count the reference's rayon pool takes off macOS
    (src/cli.rs:37-47,59-62, std::thread::available_parallelism): the CPUs
    this process may run on, limited by a cgroup CPU quota when one is set."""
    n = len(os.sched_getaffinity(0))
    try:
        quota, period = open("/sys/fs/cgroup/cpu.max").read().split()[:2]
        if quota != "max":
            n = min(n, max(1, int(int(quota) // int(period))))
    except (OSError, ValueError):
        pass
    return max(1, n)


def cpu_baseline(path: str, prompt: np.ndarray, n_decode: int, reps: int = 4) -> dict:
    """The oracle's W8A32 decode rate: `reps` runs of the workload's decode
    steps, each after an untimed prefill of the same prompt (about 10 s of
    CPU work at the default workload)."""
    from oracle import oracle as O
    threads = available_parallelism()
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
            "nproc": os.cpu_count(),
            "sample": f"{reps} x ({len(prompt)}-token prefill, untimed, then {n_decode} timed decode steps) "
                      f"of the same GGUF; C restatement of the reference's x86 scalar-fallback path "
                      f"(f32 activations, W8A32), {threads} threads = the available parallelism of this "
                      f"process ({os.cpu_count()} logical CPUs on the host)"}


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


def source_digest(*names: str) -> str:
    import hashlib
    h = hashlib.sha256()
    for n in names:
        with open(os.path.join(REPO, "squirrel-rs_amd", "csrc", n), "rb") as f:
            h.update(f.read())
    return h.hexdigest()[:16]


def measured_traffic(kernel: str, config: str):
    """HBM bytes per launch of the dominant kernel from the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE runs (scaled by the copy calibration),
    with the digest of the kernel source it was measured on: (bytes, None),
    or (None, reason) when there is no measurement for this kernel and
    workload or the source has changed since."""
    path = os.path.join(REPO, "profiles", f"traffic_{kernel}_{config}.json")
    try:
        with open(path) as f:
            rec = json.load(f)
        b = int(rec["traffic_bytes_per_launch"])
    except (OSError, ValueError, KeyError):
        return None, "no counter measurement for this kernel and workload"
    want = rec.get("source_digest")
    have = source_digest(*rec.get("source_files", ["k_step.hip"]))
    if want != have:
        return None, f"counter measurement is stale (kernel source {have}, measured on {want})"
    return b, None


def run_workload(name: str, cfg: dict, K: int, W: int, seed: int, kernel_iters: int, multi_kernel: bool) -> dict:
    """One workload: prefill + K timed decode steps (after W warmup steps);
    returns its block of the JSON line."""
    import sqhip
    path = model_path(cfg["wtype"], seed)
    t0 = time.time()
    model = sqhip.Llama3_2(path)
    info = model.info
    log(f"[{name}] loaded {path} ({info.weight_bytes / 1e6:.1f} MB of matrices) in {time.time() - t0:.1f}s")
    S = cfg["prompt"]
    prompt = np.random.default_rng(seed).integers(0, info.vocab, S).astype(np.uint32)
    ctx = model.new_context(S + max(K, W) + 2, persistent=not multi_kernel)
    gen = sqhip.TextTokenGenerator(model, ctx)
    if W > 0:
        gen.generate(prompt, W + 1, ignore_eos=True)
    sqhip.check(sqhip.lib().sq_synchronize())
    wall0 = time.perf_counter()
    toks, ms = gen.generate(prompt, K + 1, ignore_eos=True)
    sqhip.check(sqhip.lib().sq_synchronize())
    wall = time.perf_counter() - wall0
    assert len(toks) == K + 1, "generation stopped early"
    prefill_ms = float(ms[0])
    decode_ms = float(np.sum(ms[1:K + 1]))
    tok_s = K / (decode_ms / 1e3)
    log(f"[{name}] prefill {S} tokens: {prefill_ms:.2f} ms; decode {K} steps: {decode_ms:.2f} ms "
        f"({tok_s:.1f} tok/s); wall {wall * 1e3:.1f} ms")
    avg_bytes = float(np.mean([bytes_per_token(info, S + k) for k in range(1, K + 1)]))
    step_gbs = avg_bytes / (decode_ms / K / 1e3) / 1e9
    block = {
        "workload": cfg["workload"], "weights": cfg["wtype"], "prompt_tokens": S, "decode_steps": K,
        "generated_tokens": K + 1, "positions_attended": [S + 1, S + K],
        "decode_tok_s": round(tok_s, 2), "ms_per_step": round(decode_ms / K, 4),
        "prefill_tok_s": round(S / (prefill_ms / 1e3), 1), "prefill_ms": round(prefill_ms, 3),
        "decode_kernel": "persistent decode step" if ctx.persistent else "one kernel per op (hipGraph)",
    }
    traffic, why = measured_traffic("decode_step", name) if ctx.persistent else (None, "multi-kernel path")
    block["roofline"] = {"bound": "hbm", "achieved": round(step_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(step_gbs / HBM_PEAK_GBS, 4), "traffic": traffic,
                         "bytes_per_launch": int(avg_bytes)}
    if why:
        block["roofline"]["traffic_note"] = why
    if name == "prefill":
        ph = ctx.prefill_phases(prompt)
        L = info.n_layers
        mm_ops = 2.0 * S * MATMUL_ELEMS_PER_LAYER * L
        attn_flops = 4.0 * info.head_dim * S * (S + 1) / 2 * info.n_heads * L
        mm_tops = mm_ops / (ph["matmul"] / 1e3) / 1e12
        at_tflops = attn_flops / (ph["attention"] / 1e3) / 1e12
        # VALU ceiling of the int8 matmul's per-block rescale: 256 CUs x 64
        # lanes x 2.4 GHz element operations, VALU_RESCALE_OPS per 64 int8 ops
        valu_ceiling = 256 * 64 * 2.4e9 / VALU_RESCALE_OPS * 64 / 1e12
        block["prefill_phases_ms"] = {k: round(v, 3) for k, v in ph.items()}
        block["prefill_mfma"] = {
            "matmul_int8_tops": round(mm_tops, 1), "matmul_frac_of_int8_peak": round(mm_tops / INT8_PEAK_TOPS, 4),
            "matmul_valu_rescale_ceiling_tops": round(valu_ceiling, 1),
            "matmul_frac_of_rescale_ceiling": round(mm_tops / valu_ceiling, 4),
            "attention_tflops": round(at_tflops, 1),
            "matmul_ops": mm_ops, "attention_flops": attn_flops}
        if os.environ.get("SQUIRREL_ATTN_F32") == "1":
            block["prefill_mfma"]["attention_frac_of_fp32_mfma_peak"] = round(at_tflops / FP32_MFMA_PEAK_TFLOPS, 4)
        else:
            f16_tflops = ATTN_F16_PRODUCTS * at_tflops
            block["prefill_mfma"]["attention_f16_mfma_tflops"] = round(f16_tflops, 1)
            block["prefill_mfma"]["attention_frac_of_f16_mfma_peak"] = round(f16_tflops / F16_MFMA_PEAK_TFLOPS, 4)
        block["prefill_roofline"] = {"bound": "mfma", "achieved": round(mm_tops, 1), "peak": INT8_PEAK_TOPS,
                                     "unit": "TOP/s", "frac": round(mm_tops / INT8_PEAK_TOPS, 4),
                                     "kernel": "gemm_dma_kernel (v_mfma_i32_32x32x32_i8 on 128x128 tiles staged "
                                               "by direct global-to-LDS loads; gate/up with the fused SiLU*up "
                                               "epilogue, q|k|v, o and down with K split 2-3 ways and their "
                                               "partial sums)"}
        log(f"[{name}] prefill phases {ph}; int8 matmul {mm_tops:.0f} TOP/s, attention {at_tflops:.1f} TFLOP/s")
    if kernel_iters and name == "q8":
        kernels = {}
        for which, kname in KERNELS.items():
            us, nbytes = ctx.time_kernel(which, kernel_iters)
            kernels[kname] = {"mean_us": round(us, 3), "bytes": int(nbytes), "gbs": round(nbytes / us / 1e3, 1)}
        block["multi_kernel_path_kernels"] = kernels
    block["_info"] = info
    block["_path"] = path
    block["_prompt"] = prompt
    ctx.close()
    model.close()
    return block


# Stamps of the persistent step's timeline per layer (sq_ctx_step_trace), in
# the order the critical path passes them; each phase ends at its stamp.
TIMELINE_PHASES = [
    ("hidden-row gather + norm (QKV input)", 0), ("QKV rows", 1), ("q -> attention -> attention output", 2),
    ("tile merge", 3), ("attention-output gather (o input)", 4), ("o rows", 5),
    ("hidden-row gather + norm (gate/up input)", 6), ("gate/up rows", 7), ("SiLU + Q8_0", 8),
    ("FFN-activation gather (down input)", 9), ("down rows", 10)]


def step_timeline(config: str, seed: int, steps: int = 4) -> int:
    """Per-phase timeline of the persistent decode step: for every layer and
    phase, the median over workgroups of the time from the workgroup's
    previous stamp to the phase's stamp (the first phase starts at the
    previous layer's down-rows stamp), averaged over the inner layers."""
    import ctypes as C
    import sqhip
    from sqhip._lib import check, lib
    cfg = CONFIGS[config]
    path = model_path(cfg["wtype"], seed)
    model = sqhip.Llama3_2(path)
    S = cfg["prompt"]
    ctx = model.new_context(S + 64)
    if not ctx.persistent:
        print("the persistent decode step does not serve this workload", file=sys.stderr)
        return 2
    khz = C.c_int()
    check(lib().sq_device_wall_clock_khz(C.byref(khz)))
    us_per_tick = 1e3 / khz.value
    prompt = np.random.default_rng(seed).integers(0, model.info.vocab, S).astype(np.uint32)
    ctx.forward(prompt)
    tok = ctx.argmax()
    for _ in range(4):
        ctx.forward([tok])
        tok = ctx.argmax()
    ctx.step_trace(True)
    L = model.info.n_layers
    per = {name: [] for name, _ in TIMELINE_PHASES}
    layer_us, step_us, head_us = [], [], []
    for _ in range(steps):
        ctx.forward([tok])
        tok = ctx.argmax()
        t = ctx.step_trace_read().astype(np.int64)
        for l in range(1, L - 1):
            base = 1 + 20 * l
            prev = t[:, base - 20 + 10]
            for name, j in TIMELINE_PHASES:
                cur = t[:, base + j]
                ok = (cur > 0) & (prev > 0)
                if ok.any():
                    per[name].append(float(np.median(cur[ok] - prev[ok])) * us_per_tick)
                prev = np.where(cur > 0, cur, prev)
            layer_us.append(float(np.median(t[:, base + 10] - t[:, base - 20 + 10])) * us_per_tick)
        end = t[0, 3 + 20 * L]
        step_us.append(float(end - t[:, 0].min()) * us_per_tick)
        head_us.append(float(end - np.median(t[:, 1 + 20 * (L - 1) + 10])) * us_per_tick)
    print(f"# Persistent decode step timeline: {cfg['workload']}, {steps} traced steps, layers 1-{L - 2}")
    print()
    print("| phase | median over workgroups, mean over layers (us) |")
    print("|---|---:|")
    for name, _ in TIMELINE_PHASES:
        v = per[name]
        print(f"| {name} | {np.mean(v):.2f} |" if v else f"| {name} | - |")
    print(f"| **layer** (down rows to down rows) | **{np.mean(layer_us):.2f}** |")
    print(f"| last layer's down rows to the token (final norm, LM head, argmax) | {np.mean(head_us):.2f} |")
    print(f"| whole step (first workgroup start to the token) | {np.mean(step_us):.2f} |")
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None, help="decode steps timed (headline workload)")
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--config", default="q8", choices=sorted(CONFIGS), help="the headline workload")
    ap.add_argument("--only", action="store_true", help="measure the headline workload only")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-steps", type=int, default=None,
                    help="decode steps timed on the CPU (default: the same count as the GPU run, at most 64)")
    ap.add_argument("--kernel-iters", type=int, default=200)
    ap.add_argument("--multi-kernel", action="store_true",
                    help="decode with one kernel per op (hipGraph) instead of the persistent step kernel")
    ap.add_argument("--step-timeline", action="store_true",
                    help="only print the persistent decode step's per-phase timeline for --config, then exit")
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
    if args.step_timeline:
        return step_timeline(args.config, args.seed)
    if args.config == "bf16":
        print("the BF16 workload's kernels (f32 activations) are switched off on the device", file=sys.stderr)
        return 2

    cfg = CONFIGS[args.config]
    K = args.steps if args.steps is not None else cfg["gen"] - 1
    W = args.warmup
    head = run_workload(args.config, cfg, K, W, args.seed, args.kernel_iters, args.multi_kernel)
    info, path, prompt = head.pop("_info"), head.pop("_path"), head.pop("_prompt")

    configs = {}
    if not args.only:
        for name in ("q8", "q4", "q8_q4", "long", "prefill"):
            if name == args.config:
                continue
            c = CONFIGS[name]
            blk = run_workload(name, c, c["gen"] - 1, min(W, 8), args.seed, 0, args.multi_kernel)
            for k in ("_info", "_path", "_prompt"):
                blk.pop(k)
            configs[name] = blk
        if "q4" in configs and "q8_q4" in configs:
            # Q4_0 against Q8_0 at the same positions (decode tok/s ratio)
            configs["q4"]["vs_q8_same_workload"] = round(
                configs["q4"]["decode_tok_s"] / configs["q8_q4"]["decode_tok_s"], 4)
        configs["bf16"] = {"workload": CONFIGS["bf16"]["workload"], "status": "not run",
                           "reason": "the f32-activation kernels (BF16 weights) are switched off on the device"}

    cpu = None
    if not args.no_cpu:
        t1 = time.time()
        cpu = cpu_baseline(path, prompt[:32], args.cpu_steps if args.cpu_steps is not None else min(K, 64))
        log(f"cpu baseline {cpu['value']} tok/s in {time.time() - t1:.1f}s")

    line = {
        "metric": METRIC, "value": head["decode_tok_s"], "unit": "tok/s", "n_gpus": 1, "steps": K,
        "warmup": W, "ms_per_step": head["ms_per_step"], "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "int8" if cfg["wtype"] != "BF16" else "f32",
        "data": "synthetic (seeded random-init weights, random prompt ids)",
        "config": {"workload": cfg["workload"] if K == cfg["gen"] - 1 else
                   f"{cfg['workload'].split(' then ')[0]} then {K + 1} greedy tokens",
                   "weights": cfg["wtype"], "prompt_tokens": cfg["prompt"], "generated_tokens": K + 1,
                   "positions_attended": head["positions_attended"], "batch": 1, "kv_cache": "fp32",
                   "parallelism": "none"},
        "prefill_tok_s": head["prefill_tok_s"],
        "roofline": dict(head["roofline"], kernel="decode_step_kernel (persistent: one launch per token, all "
                         "layers + LM head + argmax)"),
        "cpu_baseline": cpu,
        "configs": configs,
    }
    if "multi_kernel_path_kernels" in head:
        line["multi_kernel_path_kernels"] = head["multi_kernel_path_kernels"]
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
