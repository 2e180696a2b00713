"""Model-level parity on the GPU: full forward passes vs the oracle.

The oracle runs the same GGUF file in the matching arithmetic mode (W8A8
integer path for Q8_0 / Q4_0, f32 activations for BF16 and the
SQUIRREL_F32_ACTS ablation).  Logits are compared teacher-forced: both sides
consume the same token ids at every step, so one rounding difference cannot
snowball into a different continuation.

Tolerance rule (integer path).  Activation quantization makes W8A8 logits
discontinuous in f32 rounding: a 1-ulp difference before a Q8 rounding step
moves that activation by a whole quantum.  The reference's own two builds (the
aarch64 NEON combine order vs its scalar twin) therefore either agree to
~1e-7 relative or differ by 0.7-1.0x the whole W8A8-vs-W8A32 quantization
error (measured on these models, 8 seeds).  The bar for the GPU is the same:
per step, the relative L2 error of the GPU logits against the oracle's W8A8
logits must not exceed the reference's own W8A8-vs-W8A32 relative L2 error on
the same inputs.  Two bars follow from that:
  * the GPU's W8A8 logits are as close to the f32-activation (W8A32) logits as
    the oracle's W8A8 logits are: rel_l2(gpu, W8A32) <= F32_FACTOR * gap;
  * the GPU and the oracle differ by no more than two independent W8A8
    roundings would: rel_l2(gpu, W8A8) <= PAIR_FACTOR * gap (sqrt(2) plus
    margin).
Where no flip happens the two agree to f32 rounding (~1e-7 relative; printed).
Integer parity itself is pinned bit for bit at the kernel level (quantizer,
block sums, fused norm+quantize).
"""
import os

import numpy as np
import pytest

from oracle import oracle as O

pytestmark = pytest.mark.gpu

sq = pytest.importorskip("sqhip")

F32_FACTOR = 1.25
PAIR_FACTOR = 1.5
LOGIT_ABS_FLOOR = 2e-4
MODES = {"Q8_0": O.W8A8, "Q4_0": O.W8A8, "BF16": O.W8A32}
A32_SKIP = ("f32-activation kernels (BF16, SQUIRREL_F32_ACTS) are switched off after a GPU "
            "memory fault in a BF16 model prefill whose cause is not identified yet")


def run_oracle(path, seq, mode, max_pos=256):
    m = O.OracleModel(path)
    c = m.new_context(max_pos, mode)
    outs = []
    c.forward(seq[0])
    outs.append(c.logits())
    for t in seq[1:]:
        c.forward([t])
        outs.append(c.logits())
    return outs


def run_gpu(path, seq, f32_acts=False, graph=True, max_pos=256, persistent=True):
    m = sq.Llama3_2(path)
    c = m.new_context(max_pos, f32_acts=f32_acts, graph=graph, persistent=persistent)
    outs, toks = [], []
    c.forward(seq[0])
    outs.append(c.logits())
    toks.append(c.argmax())
    for t in seq[1:]:
        c.forward([t])
        outs.append(c.logits())
        toks.append(c.argmax())
    return outs, toks, (m, c)


def teacher_seq(vocab, n_prompt=13, n_decode=6, seed=0):
    r = np.random.default_rng(seed)
    prompt = r.integers(0, vocab, n_prompt).astype(np.uint32)
    return [prompt] + [int(t) for t in r.integers(0, vocab, n_decode)]


def rel_l2(a, b):
    return float(np.linalg.norm(a.astype(np.float64) - b) / np.linalg.norm(b))


def check_logits(path, seq, got, label, max_pos=256):
    want = run_oracle(path, seq, O.W8A8, max_pos)
    f32 = run_oracle(path, seq, O.W8A32, max_pos)
    neon = run_oracle(path, seq, O.W8A8_NEON, max_pos)
    rows = []
    for step, (g, w, f, n) in enumerate(zip(got, want, f32, neon)):
        rows.append((step, rel_l2(g, w), rel_l2(g, f), rel_l2(w, f), rel_l2(n, w),
                     float(np.abs(g - w).max())))
    print(f"{label}: step, rel_l2(gpu, W8A8), rel_l2(gpu, W8A32), rel_l2(W8A8, W8A32) = gap, "
          f"rel_l2(neon order, scalar), max|gpu - W8A8|")
    for r in rows:
        print("   %2d  %.2e  %.2e  %.2e  %.2e  %.2e" % r)
    for step, e_pair, e_f32, gap, e_ref, mx in rows:
        assert e_f32 <= F32_FACTOR * gap, f"step {step}: {e_f32:.3e} > {F32_FACTOR} x {gap:.3e}"
        assert e_pair <= PAIR_FACTOR * gap, f"step {step}: {e_pair:.3e} > {PAIR_FACTOR} x {gap:.3e}"
    return rows


@pytest.mark.parametrize("decode", ["persistent", "multi_kernel"])
@pytest.mark.parametrize("wtype", ["Q8_0", "Q4_0", "BF16"])
@pytest.mark.parametrize("variant", ["g4", "g2"])
def test_teacher_forced_logits(tiny_gguf, wtype, variant, decode):
    if wtype == "BF16":
        pytest.skip(A32_SKIP)
    path = tiny_gguf(wtype, variant)
    cfg = O.OracleModel(path).cfg
    seq = teacher_seq(cfg.vocab)
    got, toks, (m, c) = run_gpu(path, seq, persistent=decode == "persistent")
    assert c.persistent == (decode == "persistent")
    check_logits(path, seq, got, f"{wtype}/{variant}/{decode}")
    for g, t in zip(got, toks):
        assert t == O.greedy(g), "device argmax disagrees with the greedy rule on its own logits"


@pytest.mark.skip(reason=A32_SKIP)
def test_f32_acts_ablation(tiny_gguf):
    """SQUIRREL_F32_ACTS=1 (linear.rs:14-19): W8A32 on both sides."""
    path = tiny_gguf("Q8_0", "g4")
    seq = teacher_seq(2048, seed=3)
    want = run_oracle(path, seq, O.W8A32)
    got, _, _ = run_gpu(path, seq, f32_acts=True)
    err = max(float(np.abs(g - w).max()) for g, w in zip(got, want))
    print(f"W8A32 max|dlogit| {err:.2e}")
    assert err <= LOGIT_ABS_FLOOR * 5


def test_fused_norm_quantize_bit_exact(tiny_gguf):
    """The decode step's fused RMSNorm+quantize prologue: its Q8_0 blocks are
    bit-identical to the reference quantizer applied to its f32 output, and
    that f32 output matches the oracle's RMSNorm within rounding."""
    path = tiny_gguf("Q8_0", "g4")
    m = sq.Llama3_2(path)
    c = m.new_context(64)
    c.forward(np.array([5, 6, 7], np.uint32))
    c.forward([11])
    normed, blocks = c.debug_act()
    want = O.quantize_row_q8_0(normed)
    assert np.array_equal(blocks["d"], want["d"]) and np.array_equal(blocks["qs"], want["qs"])
    om = O.OracleModel(path)
    x = O.embed([11], om.wtype, om.g.tensor_bytes("token_embd.weight"), om.cfg.embed_dim, om.cfg.vocab)
    w = np.frombuffer(om.g.tensor_bytes("blk.0.attn_norm.weight").tobytes(), np.float32)
    ref = O.rms_norm(x, w, om.cfg.rms_eps)[0]
    assert np.allclose(normed, ref, rtol=2e-6, atol=1e-7)


def test_graph_matches_eager(tiny_gguf):
    """The multi-kernel decode step replayed as a hipGraph == launched eagerly."""
    path = tiny_gguf("Q8_0", "g4")
    seq = teacher_seq(2048, seed=5)
    a, ta, _ = run_gpu(path, seq, graph=True, persistent=False)
    b, tb, _ = run_gpu(path, seq, graph=False, persistent=False)
    for x, y in zip(a, b):
        assert np.array_equal(x, y)
    assert ta == tb


@pytest.mark.parametrize("wtype", ["Q8_0", "Q4_0"])
def test_persistent_step_across_attention_tiles(tiny_gguf, wtype):
    """Decode positions 60..140 cross the 64-position attention tiles, which
    adds the persistent kernel's tile-merge phase (and its extra barrier)."""
    path = tiny_gguf(wtype, "g4")
    seq = teacher_seq(2048, n_prompt=60, n_decode=80, seed=11)
    got, toks, (m, c) = run_gpu(path, seq, max_pos=160)
    assert c.persistent
    rows = check_logits(path, seq, got, f"{wtype}/tiles")
    assert len(rows) == 81
    for g, t in zip(got, toks):
        assert t == O.greedy(g)


@pytest.mark.parametrize("wtype", ["Q8_0", "Q4_0"])
def test_persistent_step_multi_tile_chunks(tiny_gguf, wtype, monkeypatch):
    """On a 32-CU grid, contexts past 16 tiles give each (KV head, chunk)
    item several 64-position tiles (an online softmax inside the item), and
    chunks of unequal length, before the merge phase."""
    monkeypatch.setenv("SQUIRREL_STEP_GRID", "32")
    path = tiny_gguf(wtype, "g2")
    seq = teacher_seq(1000, n_prompt=1050, n_decode=40, seed=13)
    got, toks, (m, c) = run_gpu(path, seq, max_pos=1100)
    assert c.persistent
    rows = check_logits(path, seq, got, f"{wtype}/chunks", max_pos=1100)
    assert len(rows) == 41
    for g, t in zip(got, toks):
        assert t == O.greedy(g)


@pytest.mark.parametrize("wtype", ["Q8_0", "Q4_0"])
def test_long_prefill_unsplit_matrix_core_tiles(tiny_gguf, wtype):
    """A 2048-token prompt gives every prefill matmul of the g4 model at least
    256 output tiles (8 x 32 for the o and down projections), so they run on
    the matrix cores without the K split, accumulating the residual in place;
    shorter prompts take the split path."""
    path = tiny_gguf(wtype, "g4")
    seq = teacher_seq(2048, n_prompt=2048, n_decode=2, seed=17)
    got, toks, _ = run_gpu(path, seq, max_pos=2056)
    rows = check_logits(path, seq, got, f"{wtype}/long prefill", max_pos=2056)
    assert len(rows) == 3
    for g, t in zip(got, toks):
        assert t == O.greedy(g)


def test_persistent_deterministic_across_resets(tiny_gguf):
    """Back-to-back generations, with and without a reset in between, give
    the same tokens and logits (barrier epochs carry over between launches)."""
    path = tiny_gguf("Q8_0", "g2")
    m = sq.Llama3_2(path)
    c = m.new_context(96)
    assert c.persistent
    gen = sq.TextTokenGenerator(m, c)
    prompt = np.arange(1, 9, dtype=np.uint32)
    t1, _ = gen.generate(prompt, 40, ignore_eos=True)
    l1 = c.logits()
    t2, _ = gen.generate(prompt, 40, ignore_eos=True)
    l2 = c.logits()
    c.reset_cache()
    t3, _ = gen.generate(prompt, 40, ignore_eos=True)
    l3 = c.logits()
    assert list(t1) == list(t2) == list(t3)
    assert np.array_equal(l1, l2) and np.array_equal(l1, l3)


def test_persistent_matches_multi_kernel_generation(tiny_gguf):
    """Greedy generations of the two decode paths agree token for token
    until a step whose top-2 margin is within rounding noise."""
    path = tiny_gguf("Q8_0", "g4")
    m = sq.Llama3_2(path)
    prompt = np.arange(3, 15, dtype=np.uint32)
    outs = []
    for persistent in (True, False):
        c = m.new_context(64, persistent=persistent)
        toks, _ = sq.TextTokenGenerator(m, c).generate(prompt, 24, ignore_eos=True)
        outs.append(list(toks))
    a, b = outs
    n = next((i for i, (x, y) in enumerate(zip(a, b)) if x != y), len(a))
    print(f"persistent vs multi-kernel: first divergence at step {n} of {len(a)}")
    if n < len(a):
        # replay the common prefix through the oracle and check the margin
        om = O.OracleModel(path)
        oc = om.new_context(64, O.W8A8)
        oc.forward(prompt)
        for t in a[:n]:
            oc.forward([t])
        lg = np.sort(oc.logits())
        print(f"top-2 margin at the divergence: {lg[-1] - lg[-2]:.3e}")
        assert lg[-1] - lg[-2] < 5e-2 * max(1.0, abs(lg[-1]))


@pytest.mark.parametrize("wtype", ["Q8_0", "BF16"])
def test_generate_matches_forward_loop(tiny_gguf, wtype):
    """TextTokenGenerator::generate == forward/sample loop, and the greedy
    sequence vs the oracle's (first divergence reported, not asserted beyond
    the steps whose top-2 margin exceeds the logit tolerance)."""
    if wtype == "BF16":
        pytest.skip(A32_SKIP)
    path = tiny_gguf(wtype, "g4")
    m = sq.Llama3_2(path)
    c = m.new_context(128)
    prompt = np.random.default_rng(1).integers(0, 2048, 9).astype(np.uint32)
    gen, ms = sq.TextTokenGenerator(m, c).generate(prompt, 20, ignore_eos=True)
    assert len(gen) == 20 and np.all(ms > 0)
    c2 = m.new_context(128)
    c2.forward(prompt)
    loop = [c2.argmax()]
    for _ in range(19):
        c2.forward([loop[-1]])
        loop.append(c2.argmax())
    assert gen == loop
    om = O.OracleModel(path)
    oc = om.new_context(128, MODES[wtype])
    oc.forward(prompt)
    ref = []
    for step in range(20):
        lg = oc.logits()
        ref.append(O.greedy(lg))
        srt = np.sort(lg)
        if ref[-1] != gen[step]:
            margin = float(srt[-1] - srt[-2])
            print(f"greedy diverges at step {step} (oracle top-2 margin {margin:.2e})")
            assert margin <= 0.1
            break
        oc.forward([ref[-1]])


def test_eos_stops_generation(tiny_gguf, model_dir):
    """EOS handling (text_generator.rs:68-74): the same weights with EOS set to
    a token the model emits stop the loop just before it; IGNORE_EOS runs on."""
    from conftest import TINY
    path = tiny_gguf("Q8_0", "g4")
    prompt = np.array([1, 2, 3, 4], np.uint32)
    m = sq.Llama3_2(path)
    full, _ = sq.TextTokenGenerator(m, m.new_context(64)).generate(prompt, 12, ignore_eos=True)
    eos = full[3]
    cut = full.index(eos)
    path2 = str(model_dir / "tiny_eos.gguf")
    sq.write_synthetic_gguf(path2, "Q8_0", seed=7, eos=eos, **TINY)
    m2 = sq.Llama3_2(path2)
    stopped, _ = sq.TextTokenGenerator(m2, m2.new_context(64)).generate(prompt, 12)
    assert stopped == full[:cut]
    ran, _ = sq.TextTokenGenerator(m2, m2.new_context(64)).generate(prompt, 12, ignore_eos=True)
    assert ran == full


def test_no_kv_cache_mode(tiny_gguf):
    """SQUIRREL_NO_KV_CACHE=1 (text_generator.rs:76-78) recomputes the whole
    sequence every step and yields the same tokens as the cached loop."""
    path = tiny_gguf("Q8_0", "g4")
    m = sq.Llama3_2(path)
    prompt = np.random.default_rng(2).integers(0, 2048, 6).astype(np.uint32)
    a, _ = sq.TextTokenGenerator(m, m.new_context(64)).generate(prompt, 6, ignore_eos=True)
    b, _ = sq.TextTokenGenerator(m, m.new_context(64)).generate(prompt, 6, ignore_eos=True,
                                                                 no_kv_cache=True)
    # Prefill and decode use different kernels, so a near-tie can flip; the
    # first token (identical computation) must agree.
    assert a[0] == b[0]


def test_a32_paths_refuse_loudly(tiny_gguf):
    """The switched-off paths fail with an error instead of running."""
    with pytest.raises(sq.LLMError) as e:
        sq.Llama3_2(tiny_gguf("BF16", "g4"))
    assert e.value.code == 20
    m = sq.Llama3_2(tiny_gguf("Q8_0", "g4"))
    with pytest.raises(sq.LLMError):
        m.new_context(16, f32_acts=True)


def test_errors(tiny_gguf):
    path = tiny_gguf("Q8_0", "g4")
    m = sq.Llama3_2(path)
    c = m.new_context(8)
    with pytest.raises(sq.KernelError) as e:
        c.forward(np.array([], np.uint32))
    assert e.value.kind == "EmptyInput"
    with pytest.raises(sq.LLMError):
        c.forward(np.arange(9, dtype=np.uint32))  # more positions than the cache holds
    c.forward(np.arange(8, dtype=np.uint32))
    with pytest.raises(sq.LLMError):
        c.forward([1])


@pytest.mark.skipif(os.environ.get("SQHIP_SKIP_FULL") == "1", reason="full-size model skipped")
def test_full_size_q8_0_prefill_and_decode(model_dir):
    """Llama-3.2-1B shape, Q8_0: 32-token prefill then 3 decode steps,
    teacher-forced against the oracle's W8A8 path."""
    path = str(model_dir / "llama1b_q8_0.gguf")
    if not os.path.exists(path):
        sq.write_synthetic_gguf(path, "Q8_0", seed=0)
    r = np.random.default_rng(0)
    seq = [r.integers(0, 128256, 32).astype(np.uint32)] + [int(t) for t in r.integers(0, 128256, 3)]
    O.set_threads(min(16, os.cpu_count() or 1))
    got, toks, _ = run_gpu(path, seq, max_pos=64)
    want = run_oracle(path, seq, O.W8A8, max_pos=64)
    f32 = run_oracle(path, seq, O.W8A32, max_pos=64)
    neon = run_oracle(path, seq, O.W8A8_NEON, max_pos=64)
    for step, (g, w, f, n) in enumerate(zip(got, want, f32, neon)):
        e_pair, e_f32, gap, e_ref = rel_l2(g, w), rel_l2(g, f), rel_l2(w, f), rel_l2(n, w)
        print(f"full-size Q8_0 step {step}: rel_l2 gpu/W8A8 {e_pair:.2e}, gpu/W8A32 {e_f32:.2e}, "
              f"gap W8A8/W8A32 {gap:.2e}, neon/scalar {e_ref:.2e}, max|d| {float(np.abs(g - w).max()):.2e}, "
              f"top1 gpu {int(np.argmax(g))} oracle {int(np.argmax(w))} neon {int(np.argmax(n))}")
        assert e_f32 <= F32_FACTOR * gap and e_pair <= PAIR_FACTOR * gap
    for g, t in zip(got, toks):
        assert t == O.greedy(g)
