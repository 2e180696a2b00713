"""The library's HIP kernels run on the CPU under the emulator in tests/emu.

Every kernel except the persistent decode step is compiled for the host
against an emulated HIP device (one fiber per work-item, cross-lane
operations as wavefront collectives, streams that run their queued copies
and launches only when synchronized) with AddressSanitizer, and driven
through the C ABI by tests/emu/emu_model.cpp.  These tests check, without a
GPU:
  * that the emulator itself catches an out-of-bounds read, a cross-lane
    operation reached by only part of a wavefront, and a host or freed
    pointer handed to a kernel (device memory is host memory here, so every
    kernel argument is checked against the live device allocations);
  * that whole teacher-forced model runs (prefill, then the captured
    one-kernel-per-op decode step) make no out-of-bounds access, in every
    weight type and activation mode, including the f32-activation kernels
    that the library refuses on the device;
  * that their logits match the oracle in the same arithmetic mode: the
    integer path (Q8_0 / Q4_0, W8A8) phase-locked -- the oracle checks the
    device's Q8_0 blocks at every quantization site (oracle.h or_lock: only
    one-step flips within 0.02 quanta of a rounding midpoint pass) and then
    continues with them -- within 1e-6 relative L2 and with no bad block;
    W8A32 (BF16 weights and the SQUIRREL_F32_ACTS ablation) within 1e-5;
  * that the lock reports a single planted error (one element off by two, or
    one block scale off by 1%) at the layer and site where it was planted;
  * that the greedy token sequence of sq_generate equals the oracle's.
The emulated run uses the host's libm, so it checks indexing and arithmetic
order, not the device's transcendental functions.
"""
import os
import re
import subprocess
import sys

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "emu"))
import build_emu  # noqa: E402
from lock_bar import FLIP_RATE, LOCK_TOL  # noqa: E402

ENV = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=0")
Q8_0, Q4_0, BF16 = 8, 2, 30
F32_ACTS, NO_GRAPH, MULTI_KERNEL = 1, 2, 4
W8A32, W8A8 = 0, 1


@pytest.fixture(scope="module")
def emu():
    return build_emu.build(asan=True)


@pytest.fixture(scope="module")
def models(emu, tmp_path_factory):
    d = tmp_path_factory.mktemp("emu_models")
    out = {}
    for name, wt in (("Q8_0", Q8_0), ("Q4_0", Q4_0), ("BF16", BF16)):
        path = str(d / f"g4_{name}.gguf")
        subprocess.run([emu, "--write", path, str(wt), "7", "2", "512", "1024", "8", "2", "2048"],
                       check=True, env=ENV)
        out[name] = path
    return out


def run(emu, args, timeout=600, env=None):
    p = subprocess.run([emu, *map(str, args)], capture_output=True, text=True, env={**ENV, **(env or {})},
                       timeout=timeout)
    assert p.returncode == 0, p.stdout[-2000:] + p.stderr[-4000:]
    assert "AddressSanitizer" not in p.stderr
    steps = [(int(m[1]), float(m[2]), float(m[3]), int(m[4]), int(m[5]))
             for m in re.finditer(r"^step (\d+) rel_l2 (\S+) max_abs (\S+) argmax (\d+) (\d+)", p.stdout, re.M)]
    return steps, p.stdout


def locks(out):
    """Per step: (values, flips, scale_flips, bad, (layer, site, index))."""
    return [(int(m[2]), int(m[3]), int(m[4]), int(m[5]), (int(m[6]), int(m[7]), int(m[8])))
            for m in re.finditer(r"^lock step (\d+) values (\d+) flips (\d+) scale_flips (\d+) bad (\d+) "
                                 r"first_bad (-?\d+)/(-?\d+)/(\d+)/", out, re.M)]


def test_emulator_catches_out_of_bounds_and_divergence(emu):
    st = build_emu.SELFTEST
    ok = subprocess.run([st, "ok"], capture_output=True, text=True, env=ENV)
    assert ok.returncode == 0 and "sum 256" in ok.stdout
    oob = subprocess.run([st, "oob"], capture_output=True, text=True, env=ENV)
    assert oob.returncode != 0 and "heap-buffer-overflow" in oob.stderr
    div = subprocess.run([st, "diverge"], capture_output=True, text=True, env=ENV)
    assert div.returncode != 0 and "cross-lane" in div.stderr


@pytest.mark.parametrize("case,want", [("pinned", "sum 512"), ("nullstream", "sum 256"), ("synced", "sum 64")])
def test_emulator_streams_are_asynchronous(emu, case, want):
    """Queued copies and launches run only when their stream is synchronized,
    in stream order: a pinned source rewritten before its copy ran is read as
    rewritten, and hipMemcpy on the null stream does not wait for a
    non-blocking stream.  A missing synchronization in the library's host
    code therefore shows up in the emulated runs as wrong data."""
    p = subprocess.run([build_emu.SELFTEST, case], capture_output=True, text=True, env=ENV)
    assert p.returncode == 0 and want in p.stdout, p.stdout + p.stderr


def test_noalloc_allocates_nothing(emu):
    """sq_linear_noalloc's contract: a warm call allocates no device memory,
    on the single-row matvec path and on the K-split matmul path (sq_linear,
    beside it, allocates its scratch on every call)."""
    p = subprocess.run([emu, "--noalloc-count"], capture_output=True, text=True, env=ENV)
    assert p.returncode == 0 and "AddressSanitizer" not in p.stderr, p.stdout + p.stderr
    got = {int(m[1]): (int(m[2]), int(m[3]))
           for m in re.finditer(r"^m (\d+) noalloc_mallocs (\d+) linear_mallocs (\d+)$", p.stdout, re.M)}
    assert set(got) == {1, 67}, p.stdout
    for m, (noalloc, linear) in got.items():
        assert noalloc == 0 and linear > 0, (m, noalloc, linear)


def test_device_token_id_past_the_table_is_an_error(emu):
    """An id past the embedding table that reaches a kernel from device
    memory (the host validates the ids it is given) is an error status, as
    the reference's slice index panics (embedding.rs:43-44), and the row read
    stays in bounds (AddressSanitizer watches every access here)."""
    p = subprocess.run([emu, "--embed-guard"], capture_output=True, text=True, env=ENV)
    assert p.returncode == 0 and "AddressSanitizer" not in p.stderr, p.stdout + p.stderr
    got = re.findall(r"^embed ids (\d+) (\d+) (\d+) status (\d+)$", p.stdout, re.M)
    assert got == [("3", "63", "0", "0"), ("3", "64", "0", "22"), ("4294967295", "1", "2", "22")], p.stdout


@pytest.mark.parametrize("case,where", [("host", "stack"), ("hoststruct", "stack"), ("freed", "heap")])
def test_emulator_refuses_host_and_freed_pointers(emu, case, where):
    """Device memory is host memory in the emulator, so a host pointer or a
    pointer into a freed allocation handed to a kernel would simply work
    there.  Every argument word of every launch (and of every graph replay)
    is checked against the live device allocations instead."""
    p = subprocess.run([build_emu.SELFTEST, case], capture_output=True, text=True, env=ENV)
    assert p.returncode != 0, p.stdout + p.stderr
    assert "outside every live device allocation" in p.stderr and f"({where})" in p.stderr, p.stderr


@pytest.mark.parametrize("wtype,mode,flags,bar", [
    ("Q8_0", W8A8, MULTI_KERNEL, 1e-6),
    ("Q4_0", W8A8, MULTI_KERNEL, 1e-6),
    ("Q8_0", W8A8, MULTI_KERNEL | NO_GRAPH, 1e-6),
    ("BF16", W8A32, 0, 1e-5),
    ("Q8_0", W8A32, F32_ACTS, 1e-5),
    ("Q4_0", W8A32, F32_ACTS, 1e-5),
])
def test_teacher_forced_run_in_bounds_and_matches_oracle(emu, models, wtype, mode, flags, bar):
    steps, out = run(emu, [models[wtype], mode, flags, 13, 3, 0, 256, f"tol={LOCK_TOL}"])
    assert len(steps) == 4, out
    for step, rel, mx, dev, ora in steps:
        print(f"{wtype} flags={flags} step {step}: rel_l2 {rel:.2e} max_abs {mx:.2e}")
        assert rel <= bar, f"step {step}: rel_l2 {rel:.3e} > {bar}"
        assert dev == ora, f"step {step}: device argmax {dev} vs oracle {ora}"
    if mode == W8A8:
        lk = locks(out)
        assert len(lk) == len(steps)
        assert all(bad == 0 for _, _, _, bad, _ in lk), lk
        assert sum(l[1] for l in lk) <= FLIP_RATE[wtype] * sum(l[0] for l in lk), lk


@pytest.mark.parametrize("attn", ["auto", "split"])
def test_long_prefill_in_bounds(emu, models, attn):
    """70 prompt rows: the unsplit matrix-core matmul tiles (m >= 64) with
    a ragged 6-row tail, and two 64-query tiles of the prefill attention
    (the fp32 kernel the size selects, or the K/V split pass and the
    split-f16 kernel, SQUIRREL_ATTN_F32=0)."""
    env = {"SQUIRREL_ATTN_F32": "0"} if attn == "split" else None
    steps, out = run(emu, [models["Q8_0"], W8A8, MULTI_KERNEL, 70, 1, 1, 128], env=env)
    assert len(steps) == 2 and all(rel <= 1e-6 and dev == ora for _, rel, _, dev, ora in steps), out
    assert all(bad == 0 for _, _, _, bad, _ in locks(out)), out


@pytest.mark.parametrize("tile", ["128", "128x64"])
@pytest.mark.parametrize("wtype", ["Q8_0", "Q4_0"])
def test_long_prefill_full_rate_tiles_in_bounds(emu, models, wtype, tile):
    """The same prefill with every matmul on the full-rate kernel's 128 x 128
    or 128 x 64 tiles (SQUIRREL_GEMM_TILE=128 / 128x64): 70 of a tile's 128
    rows exist, and the grids split K over the workspace."""
    steps, out = run(emu, [models[wtype], W8A8, MULTI_KERNEL, 70, 1, 1, 128], env={"SQUIRREL_GEMM_TILE": tile})
    assert len(steps) == 2 and all(rel <= 1e-6 and dev == ora for _, rel, _, dev, ora in steps), out
    assert all(bad == 0 for _, _, _, bad, _ in locks(out)), out


@pytest.mark.parametrize("unfused", ["0", "1"])
def test_long_prefill_fused_epilogues_in_bounds(emu, models, unfused):
    """A 140-row prefill on an emulated 8-CU device (SQEMU_CUS=8), so that the
    grid-size rules pick the direct-to-LDS kernel's 128 x 128 tiles for the
    FFN gate/up projection and its 128 x 64 tiles for the q|k|v projection:
    with the fused epilogues (SiLU * up with its Q8_0 blocks; RoPE and the
    KV-cache append) and without them (SQUIRREL_PREFILL_UNFUSED=1), with the
    attention on the K/V split pass and the split-f16 kernel
    (SQUIRREL_ATTN_F32=0), every access stays in bounds and the logits and
    quantization sites match the oracle."""
    steps, out = run(emu, [models["Q8_0"], W8A8, MULTI_KERNEL, 140, 1, 1, 160],
                     env={"SQEMU_CUS": "8", "SQUIRREL_PREFILL_UNFUSED": unfused, "SQUIRREL_ATTN_F32": "0"})
    assert len(steps) == 2 and all(rel <= 1e-6 and dev == ora for _, rel, _, dev, ora in steps), out
    assert all(bad == 0 for _, _, _, bad, _ in locks(out)), out


@pytest.fixture(scope="module")
def wide_model(emu, tmp_path_factory):
    """One layer at Llama-3.2-1B's width (dim 2048, 32 heads, 8 KV heads; a
    256-wide FFN keeps the emulated run short): the q|k|v projection has
    3072 rows and K = 2048."""
    path = str(tmp_path_factory.mktemp("emu_wide") / "w2k_Q8_0.gguf")
    subprocess.run([emu, "--write", path, str(Q8_0), "7", "1", "2048", "256", "32", "8", "512"], check=True, env=ENV)
    return path


def gemm_counts(out):
    m = re.search(r"^gemm launches (\d+) split (\d+) tile128 (\d+) max_splits (\d+) tile128x64 (\d+) rows (\d+)",
                  out, re.M)
    return dict(zip(("launches", "split", "tile128", "max_splits", "tile128x64", "rows"), map(int, m.groups())))


@pytest.mark.parametrize("cus,want", [
    # 48 tiles of 128 x 128 fill 8 CUs twice: the q|k|v projection with
    # RoPE and the KV append in the 128 x 128 kernel's epilogue
    (8, {"launches": 4, "split": 1, "tile128": 4, "tile128x64": 0}),
    # 48 tiles on 32 CUs: K split two ways, RoPE and the KV append in the
    # kernel that sums the partials (the o projection splits three ways)
    (32, {"launches": 4, "split": 3, "tile128": 2, "tile128x64": 1}),
])
def test_wide_prefill_qkv_epilogues(emu, wide_model, cus, want):
    """A 140-row prefill of the full-width layer on an emulated 8- and
    32-CU device: the fused q|k|v forms (the 128 x 128 epilogue; the K-split
    sum with RoPE) stay in bounds, match the oracle, and give the same
    logits, hidden state and quantization-site flips as the separate
    launches (SQUIRREL_PREFILL_UNFUSED=1)."""
    lines = {}
    for unfused in ("0", "1"):
        steps, out = run(emu, [wide_model, W8A8, MULTI_KERNEL, 140, 0, 1, 160],
                         env={"SQEMU_CUS": str(cus), "SQUIRREL_PREFILL_UNFUSED": unfused})
        assert len(steps) == 1 and steps[0][1] <= 1e-6 and steps[0][3] == steps[0][4], out
        assert all(bad == 0 for _, _, _, bad, _ in locks(out)), out
        n = gemm_counts(out)
        assert {k: n[k] for k in want} == want, n
        lines[unfused] = re.findall(r"^(?:step|lock step) .*$", out, re.M)
    assert lines["0"] == lines["1"], lines


@pytest.mark.parametrize("step,layer,site,element,kind", [
    (0, 0, 0, 100, 0),   # prefill, attention-norm output, one element
    (0, 1, 3, 700, 1),   # prefill, FFN activation, one block scale
    (1, 1, 1, 37, 0),    # decode, attention output, one element
    (2, 0, 2, 511, 1),   # decode, FFN-norm output, one block scale
])
def test_lock_reports_a_planted_error(emu, models, step, layer, site, element, kind):
    """A single wrong element or block scale at any site fails the lock,
    reported at the place it was planted (the oracle side of the check runs
    on the corrupted copy; the device run itself is correct)."""
    _, out = run(emu, [models["Q8_0"], W8A8, MULTI_KERNEL, 13, 2, 0, 64,
                       f"corrupt={step},{layer},{site},{element},{kind}"])
    lk = locks(out)
    assert all(l[3] == 0 for l in lk[:step]), lk
    values, flips, scale_flips, bad, first = lk[step]
    rows = 13 if step == 0 else 1
    assert bad > 0 and first[:2] == (layer, site), lk
    assert first[2] // 32 == element // 32 if rows == 1 else True, lk


@pytest.mark.parametrize("step,layer,site", [
    (0, 0, 2),   # prefill, FFN-norm output
    (1, 1, 0),   # decode, attention-norm output
    (2, 1, 3),   # decode, FFN activation
])
def test_lock_catches_a_planted_systematic_bias(emu, models, step, layer, site):
    """A systematic error of 0.005 quanta over one whole site (every scaled
    value moved by 0.005 before rounding, so only elements within 0.005 of a
    midpoint change, each by one step) is a bad block at that site under
    LOCK_TOL; under the former bar of 0.02 quanta the same site passes (the
    planted blocks, substituted on the oracle's side only, then show up
    downstream, where the device did not use them)."""
    plant = f"plant={step},{layer},{site},0.005"
    _, tight = run(emu, [models["Q8_0"], W8A8, MULTI_KERNEL, 13, 2, 0, 64, plant, f"tol={LOCK_TOL}"])
    _, loose = run(emu, [models["Q8_0"], W8A8, MULTI_KERNEL, 13, 2, 0, 64, plant, "tol=0.02"])
    lt, ll = locks(tight), locks(loose)
    assert all(l[3] == 0 for l in lt[:step]) and all(l[3] == 0 for l in ll[:step]), (lt, ll)
    assert lt[step][3] > 0 and lt[step][4][:2] == (layer, site), lt
    assert ll[step][3] == 0 or ll[step][4][:2] != (layer, site), ll


def test_generate_matches_oracle_greedy(emu, models):
    _, out = run(emu, [models["Q8_0"], W8A8, MULTI_KERNEL, 9, 5, 2, 64, "generate"])
    got = re.search(r"^generated (.*)$", out, re.M).group(1).split()
    want = re.search(r"^oracle_generated (.*)$", out, re.M).group(1).split()
    assert got == want
