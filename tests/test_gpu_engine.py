"""GPU tests of the GPT-2 decode engine (ie_engine.h over the HIP kernels).

Mirrors the reference's engine tests (tests/test_engine.cu:34-74: greedy
determinism, metrics populated, generation stops) and adds parity with the
CPU decode-step oracle (oracle/gpt2_step.py), graph-replay and batch
invariance (both bit-exact), and the bf16-KV / INT8-head variants.

Parity bar for the engine against the oracle: the oracle's LayerNorm runs in
fp64 and the device's in fp32, so an activation can land on the other side of
an int8 rounding boundary.  For the 128-wide model logits are held to
max|diff| <= 2e-3 * max|logits| and the greedy token must agree whenever the
oracle's top-2 gap exceeds 1e-2 of the logit scale; for the 768-wide model see
check_steps.  The fused step is held to bit-identity with the unfused one.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

TINY = dict(n_layers=2, n_heads=2, d_model=128, d_ff=512, vocab_size=1000, max_seq_len=64)
# GPT-2 widths (the fused step's kernels), few layers, small vocabulary; 256
# positions give 4 attention splits of 64 tokens.
MID = dict(n_layers=2, n_heads=12, d_model=768, d_ff=3072, vocab_size=1000, max_seq_len=256)


@pytest.fixture(scope="module")
def tiny_dir(tmp_path_factory, ie):
    d = tmp_path_factory.mktemp("gpt2_tiny")
    ie.write_random_model(d, seed=11, **TINY)
    return d


@pytest.fixture(scope="module")
def long_dir(tmp_path_factory, ie):
    d = tmp_path_factory.mktemp("gpt2_long")
    ie.write_random_model(d, seed=13, **dict(MID, max_seq_len=1024))
    return d


@pytest.fixture(scope="module")
def mid_dir(tmp_path_factory, ie):
    d = tmp_path_factory.mktemp("gpt2_mid")
    ie.write_random_model(d, seed=12, **MID)
    return d


def run_steps(eng, toks):
    return [eng.step(t) for t in toks]


def test_engine_matches_oracle(ie, tiny_dir):
    from oracle.gpt2_step import OracleGPT2

    B = 2
    rng = np.random.default_rng(0)
    toks = rng.integers(0, TINY["vocab_size"], (12, B)).astype(np.int32)
    eng = ie.Engine(tiny_dir, max_batch=B, use_graph=True)
    orc_m = OracleGPT2(str(tiny_dir), batch=B)
    agree = checked = 0
    for t in toks:
        got = eng.step(t)
        want = orc_m.step(t)
        scale = np.abs(want).max()
        assert np.abs(got - want).max() <= 2e-3 * scale, np.abs(got - want).max() / scale
        for b in range(B):
            top = np.sort(want[b])[-2:]
            if top[1] - top[0] > 1e-2 * scale:
                checked += 1
                agree += int(np.argmax(got[b]) == np.argmax(want[b]))
    assert agree == checked and checked > 0
    eng.close()


def test_graph_replay_is_bit_identical_to_eager(ie, tiny_dir):
    rng = np.random.default_rng(1)
    toks = rng.integers(0, TINY["vocab_size"], (10, 3)).astype(np.int32)
    a = run_steps(ie.Engine(tiny_dir, max_batch=3, use_graph=True), toks)
    b = run_steps(ie.Engine(tiny_dir, max_batch=3, use_graph=False), toks)
    for x, y in zip(a, b):
        assert np.array_equal(x, y)


def test_batch_invariance_bit_exact(ie, tiny_dir):
    rng = np.random.default_rng(2)
    prompts = rng.integers(0, TINY["vocab_size"], (5, 7)).astype(np.int32)
    out_b, _ = ie.Engine(tiny_dir, max_batch=5).generate(prompts, 12, ignore_eos=True)
    for i in range(5):
        single, _ = ie.Engine(tiny_dir, max_batch=1).generate(prompts[i:i + 1], 12, ignore_eos=True)
        assert np.array_equal(single[0], out_b[i])


def test_determinism_and_metrics(ie, tiny_dir):
    eng = ie.Engine(tiny_dir, max_batch=1)
    prompt = np.array([[5, 17, 256, 999, 3]], dtype=np.int32)
    t1, m1 = eng.generate(prompt, 20)
    t2, m2 = eng.generate(prompt, 20)
    assert np.array_equal(t1, t2)
    assert m1["ttft_ms"] > 0 and m1["tps"] > 0 and m1["kv_cache_pct"] > 0
    assert 0 < m1["tokens_generated"] <= 20
    assert m1["itl_min_ms"] <= m1["itl_p95_ms"] <= m1["itl_max_ms"]
    assert eng.session_tokens() == 5 + 19  # prompt + fed-back tokens


def test_context_full_stops_cleanly(ie, tiny_dir):
    eng = ie.Engine(tiny_dir, max_batch=1)
    prompt = np.arange(60, dtype=np.int32)[None, :]
    out, m = eng.generate(prompt, 20, ignore_eos=True)
    assert m["tokens_generated"] <= 5  # 64-token context: 60 prompt + at most 4 steps
    assert eng.session_tokens() == 64


def test_bf16_kv_and_int8_head_vs_oracle(ie, tiny_dir):
    from oracle.gpt2_step import OracleGPT2

    rng = np.random.default_rng(3)
    toks = rng.integers(0, TINY["vocab_size"], (8, 2)).astype(np.int32)
    for kw, okw in [(dict(kv_dtype=ie.KV_BF16), dict(kv_bf16=True)),
                    (dict(int8_lm_head=True), dict(int8_lm_head=True))]:
        eng = ie.Engine(tiny_dir, max_batch=2, **kw)
        om = OracleGPT2(str(tiny_dir), batch=2, **okw)
        for t in toks:
            got, want = eng.step(t), om.step(t)
            assert np.abs(got - want).max() <= 2e-3 * np.abs(want).max(), kw
        eng.close()


def test_gpt2_small_random_generates(ie):
    """Full GPT-2 Small shape (12 layers, d 768, vocab 50257), batch 1 and 16."""
    eng = ie.Engine(None, seed=1, max_batch=16)
    rng = np.random.default_rng(4)
    prompt = rng.integers(0, 50257, (16, 16)).astype(np.int32)
    a, m = eng.generate(prompt, 8, ignore_eos=True)
    b, _ = eng.generate(prompt, 8, ignore_eos=True)
    assert np.array_equal(a, b) and (a >= 0).all() and (a < 50257).all()
    one, _ = eng.generate(prompt[:1], 8, ignore_eos=True)
    assert np.array_equal(one[0], a[0])
    assert m["tps"] > 0


def check_steps(errs):
    """Per-step max |diff| / max |logits| of a free-running engine against the
    free-running oracle, 768-wide model.  At this width an activation now and
    then lies within fp32-vs-fp64 noise of an int8 rounding boundary and is
    quantized one step apart; the step's K/V then stay in the cache, so the
    sequence's later logits move too.  Running the oracle itself with 1e-7
    relative noise on its LayerNorm outputs (3 sequences x 60 steps, this
    model) moves logits by up to 2.1e-2 of their scale, and the device shows
    the same events.  Bar: every step within 3e-2.  This is a drift bound for
    long free runs; the op-by-op parity bar (every op on the device's own
    inputs, bit-exact or within 1e-5) is test_gpu_engine_parity.py's
    teacher-forced test."""
    errs = np.asarray(errs)
    assert errs.max() <= 3e-2, errs


def check_vs_oracle(ie, model_dir, B, steps, seed, eng_kw, orc_kw):
    from oracle.gpt2_step import OracleGPT2

    rng = np.random.default_rng(seed)
    toks = rng.integers(0, 1000, (steps, B)).astype(np.int32)
    eng = ie.Engine(model_dir, max_batch=B, **eng_kw)
    om = OracleGPT2(str(model_dir), batch=B, **orc_kw)
    errs = []
    for t in toks:
        got, want = eng.step(t), om.step(t)
        sc = np.abs(want).max()
        errs.append([np.abs(got[b] - want[b]).max() / sc for b in range(B)])
        # the greedy token agrees wherever a quantization flip cannot reorder it
        for b in range(B):
            top = np.sort(want[b])[-2:]
            if top[1] - top[0] > 6e-2 * sc:
                assert np.argmax(got[b]) == np.argmax(want[b])
    eng.close()
    for b in range(B):
        check_steps([e[b] for e in errs])


@pytest.mark.parametrize("B", [1, 3, 6])
def test_gpt2_width_step_matches_oracle(ie, mid_dir, B):
    """The (fused) step against the oracle; 70 steps cross the first 64-token
    split boundary."""
    check_vs_oracle(ie, mid_dir, B, 70, 20 + B, {}, {})


def test_gpt2_width_bf16_kv_and_int8_head(ie, mid_dir):
    check_vs_oracle(ie, mid_dir, 2, 20, 5, dict(kv_dtype=ie.KV_BF16), dict(kv_bf16=True))
    check_vs_oracle(ie, mid_dir, 5, 20, 6, dict(int8_lm_head=True), dict(int8_lm_head=True))


@pytest.mark.parametrize("B", [1, 2, 3, 4, 6, 16])
def test_fused_step_bit_identical_to_unfused_step(ie, mid_dir, B):
    """The fused kernels (LayerNorm/quantizer prologues, QKV append epilogue)
    against the step built from the public C ABI
    operations: same arithmetic in the same order, so bit-identical logits,
    including past the first 64-token split boundary."""
    rng = np.random.default_rng(30 + B)
    toks = rng.integers(0, 1000, (70, B)).astype(np.int32)
    for kw in (dict(), dict(kv_dtype=ie.KV_BF16, int8_lm_head=True)):
        a = run_steps(ie.Engine(mid_dir, max_batch=B, fuse=True, **kw), toks)
        b = run_steps(ie.Engine(mid_dir, max_batch=B, fuse=False, **kw), toks)
        for i, (x, y) in enumerate(zip(a, b)):
            assert np.array_equal(x, y), (kw, i, np.abs(x - y).max())


def test_fused_graph_replay_and_batch_invariance(ie, mid_dir):
    rng = np.random.default_rng(7)
    toks = rng.integers(0, 1000, (12, 5)).astype(np.int32)
    a = run_steps(ie.Engine(mid_dir, max_batch=5, use_graph=True), toks)
    b = run_steps(ie.Engine(mid_dir, max_batch=5, use_graph=False), toks)
    for x, y in zip(a, b):
        assert np.array_equal(x, y)
    # rows of a batch-5 step equal the batch-1 runs bit for bit (the fixed and
    # the MFMA GEMV stage activation rows identically)
    for i in (0, 4):
        one = run_steps(ie.Engine(mid_dir, max_batch=1), toks[:, i:i + 1])
        for x, y in zip(a, one):
            assert np.array_equal(x[i], y[0])


def test_split_plan_change_past_384_tokens(ie, long_dir):
    """The engine picks its attention split plan from the context length (one
    split, written directly, up to 384 tokens; two up to 768 ...) and keeps a
    captured step per plan.  420 steps cross the switch: the fused and the
    C ABI steps stay bit-identical, graph replay equals eager execution, and
    the logits follow the oracle (check_steps)."""
    from oracle.gpt2_step import OracleGPT2

    B, steps = 2, 420
    rng = np.random.default_rng(40)
    toks = rng.integers(0, 1000, (steps, B)).astype(np.int32)
    fused = ie.Engine(long_dir, max_batch=B)
    plain = ie.Engine(long_dir, max_batch=B, fuse=False)
    eager = ie.Engine(long_dir, max_batch=B, use_graph=False)
    om = OracleGPT2(str(long_dir), batch=B)
    errs = []
    for i, t in enumerate(toks):
        a, b, c = fused.step(t), plain.step(t), eager.step(t)
        assert np.array_equal(a, b), i
        assert np.array_equal(a, c), i
        want = om.step(t)
        sc = np.abs(want).max()
        errs.append([np.abs(a[j] - want[j]).max() / sc for j in range(B)])
    for j in range(B):
        check_steps([e[j] for e in errs])


# ---------------------------------------------------------------- prefill
def prefill_vs_oracle(ie, model_dir, B, P, steps, seed, eng_kw, orc_kw):
    """Prefill of a P-token prompt, then decode steps, against the oracle fed
    the same tokens one position at a time (causal attention over the prompt is
    the same function either way).  Returns per-sequence error lists: the
    prefill's last-token logits first, then one per decode step."""
    from oracle.gpt2_step import OracleGPT2

    rng = np.random.default_rng(seed)
    prompt = rng.integers(0, 1000, (B, P)).astype(np.int32)
    toks = rng.integers(0, 1000, (steps, B)).astype(np.int32)
    eng = ie.Engine(model_dir, max_batch=B, **eng_kw)
    om = OracleGPT2(str(model_dir), batch=B, **orc_kw)
    got = eng.prefill(prompt)
    assert eng.session_tokens() == P
    for t in range(P):
        want = om.step(prompt[:, t])
    errs = []
    for i in range(steps + 1):
        if i > 0:
            got, want = eng.step(toks[i - 1]), om.step(toks[i - 1])
        sc = np.abs(want).max()
        errs.append([np.abs(got[b] - want[b]).max() / sc for b in range(B)])
        for b in range(B):
            top = np.sort(want[b])[-2:]
            if top[1] - top[0] > 6e-2 * sc:
                assert np.argmax(got[b]) == np.argmax(want[b])
    eng.close()
    return [[e[b] for e in errs] for b in range(B)]


def test_prefill_tiny_matches_oracle(ie, tiny_dir):
    """128-wide model.  The per-step 2e-3 bar of the decode tests does not
    hold here: this prompt has an activation within fp32 noise of an int8
    rounding boundary (the oracle itself, with 1e-7 relative noise on the
    prompt's attention outputs, moves these logits by up to 7.6e-3 in two of
    three noise draws), so the bar is check_steps'."""
    for seq in prefill_vs_oracle(ie, tiny_dir, 2, 30, 10, 50, {}, {}):
        check_steps(seq)


@pytest.mark.parametrize("B", [1, 3])
def test_prefill_then_decode_matches_oracle(ie, mid_dir, B):
    """GPT-2 widths: a 40-token prompt through the M = B x 40 GEMMs and the
    prefill attention, then 20 decode steps over the cache it wrote."""
    for seq in prefill_vs_oracle(ie, mid_dir, B, 40, 20, 60 + B, {}, {}):
        check_steps(seq)


def test_prefill_bf16_kv_and_int8_head(ie, mid_dir):
    for seq in prefill_vs_oracle(ie, mid_dir, 2, 33, 8, 70, dict(kv_dtype=ie.KV_BF16), dict(kv_bf16=True)):
        check_steps(seq)
    for seq in prefill_vs_oracle(ie, mid_dir, 2, 33, 8, 71, dict(int8_lm_head=True), dict(int8_lm_head=True)):
        check_steps(seq)


@pytest.mark.parametrize("kv", ["f32", "bf16"])
def test_prefill_batch16_rows_equal_single_prompts(ie, mid_dir, kv):
    """768-wide model, 16 prompts of 40 tokens: the batch's prefill GEMMs run
    on the 64x64 / 128x64 tile kernels (M = 640; the QKV projection storing Q
    and the fp32 or bf16 K/V rows through its routed epilogue, slots in LDS),
    a single prompt's on the small-grid K-split kernel (M = 40).  Both give
    exact int32 sums and the same per-element epilogue, and attention, the
    LayerNorms and the head work per sequence, so each sequence's prefill
    logits, and the decode steps over the cache its prefill wrote, are
    bit-identical either way."""
    kw = dict(kv_dtype=ie.KV_BF16) if kv == "bf16" else {}
    rng = np.random.default_rng(90)
    prompts = rng.integers(0, 1000, (16, 40)).astype(np.int32)
    toks = rng.integers(0, 1000, (3, 16)).astype(np.int32)
    eng = ie.Engine(mid_dir, max_batch=16, **kw)
    batch = [eng.prefill(prompts)] + [eng.step(toks[i]) for i in range(3)]
    eng.close()
    for b in (0, 7, 15):
        one = ie.Engine(mid_dir, max_batch=1, **kw)
        single = [one.prefill(prompts[b:b + 1])] + [one.step(toks[i, b:b + 1]) for i in range(3)]
        one.close()
        for i, (got, want) in enumerate(zip(single, batch)):
            assert np.array_equal(got[0], want[b]), (kv, b, i, np.abs(got[0] - want[b]).max())


def test_prefill_chunking_and_batch_invariance_bit_exact(ie, mid_dir):
    """Every prefill row is computed independently of the others: GEMM rows
    are exact int32 sums with a per-row epilogue, and a query's attention
    walks the cached keys in an order fixed by their positions.  So a prompt
    prefilled whole, in 16- or 37-token chunks (each chunk attending to the
    earlier ones through the cache), or as a batch of one, gives the same bits,
    and so does the decode step after it."""
    rng = np.random.default_rng(80)
    B, P = 3, 100
    prompt = rng.integers(0, 1000, (B, P)).astype(np.int32)
    nxt = rng.integers(0, 1000, B).astype(np.int32)
    runs = []
    for chunk in (0, 16, 37):
        eng = ie.Engine(mid_dir, max_batch=B, prefill_chunk=chunk)
        runs.append((eng.prefill(prompt), eng.step(nxt)))
        eng.close()
    for a, b in runs[1:]:
        assert np.array_equal(runs[0][0], a) and np.array_equal(runs[0][1], b)
    for i in (0, 2):
        eng = ie.Engine(mid_dir, max_batch=1)
        one = eng.prefill(prompt[i:i + 1])
        assert np.array_equal(one[0], runs[0][0][i])
        assert np.array_equal(eng.step(nxt[i:i + 1])[0], runs[0][1][i])
        eng.close()


def test_generate_uses_prefill_and_matches_stepwise_prompt(ie, mid_dir):
    """generate() prefills the prompt; with prefill off it feeds the prompt
    through decode steps.  Both see the same function of the prompt (first-token
    logits within the check_steps bar of each other), the prefill one sooner."""
    rng = np.random.default_rng(90)
    prompt = rng.integers(0, 1000, (2, 64)).astype(np.int32)
    a = ie.Engine(mid_dir, max_batch=2)
    b = ie.Engine(mid_dir, max_batch=2, prefill=False)
    la = a.prefill(prompt)
    for t in range(prompt.shape[1]):
        lb = b.step(prompt[:, t])
    for r in range(2):
        assert np.abs(la[r] - lb[r]).max() <= 3e-2 * np.abs(lb[r]).max()
    a.reset()
    b.reset()
    ta, ma = a.generate(prompt, 4, ignore_eos=True)
    tb, mb = b.generate(prompt, 4, ignore_eos=True)
    assert a.session_tokens() == b.session_tokens() == 64 + 3
    assert ma["ttft_ms"] < mb["ttft_ms"]


# ---------------------------------------------------------------- EOS, sessions
EOS = 50256


def echo_cfg(d=64):
    return dict(n_layers=1, n_heads=d // 64, d_model=d, d_ff=4 * d if d > 64 else 64, vocab_size=EOS + 1,
                max_seq_len=128)


def echo_model(path, eos_from, d=64):
    """Zero-weight model over the GPT-2 vocabulary (one layer, width d): the
    final hidden row at position p is wte[t] + wpe[p].  wte rows are N(0, 1),
    so LN(wte[t]) . wte[t] ~ d beats every other row (~sqrt(d) per unit of
    Gaussian tail, under 5 sqrt(d) over 50k rows) and greedy decoding repeats
    its input; from position eos_from on, wpe adds 20 wte[EOS] and
    <|endoftext|> wins.  Returns the tensors."""
    from gpt2_model import random_tensors, write_model

    cfg = echo_cfg(d)
    t = random_tensors(cfg, 77, zero_weights=True, zero_biases=True, ln_jitter=0)
    t["wte"] = np.random.default_rng(78).standard_normal((EOS + 1, d)).astype(np.float32)
    t["wpe"] = np.zeros((128, d), np.float32)
    t["wpe"][eos_from:] = 20 * t["wte"][EOS]
    write_model(str(path), cfg, t, fp32_weights=False)
    return t


def echo_expected(t, last_token, last_pos, max_new):
    """Greedy continuation from the token at last_pos, in float64 (the closed
    form of the zero-weight model); every pick's top-2 gap must be wide."""
    out, tok, p = [], last_token, last_pos
    while len(out) < max_new:
        x = (t["wte"][tok] + t["wpe"][p]).astype(np.float64)
        xf = (x - x.mean()) / np.sqrt(x.var() + 1e-5)
        logits = t["wte"].astype(np.float64) @ xf
        top = np.sort(logits)[-2:]
        assert top[1] - top[0] > 5.0
        nxt = int(np.argmax(logits))
        if nxt == EOS:
            break
        out.append(nxt)
        tok, p = nxt, p + 1
    return out


def test_eos_stops_generation(ie, tmp_path):
    """tests/test_engine.cu:65-74 (EosStopsGeneration): generation ends at
    <|endoftext|> (src/gpt2_engine.cu:717) after at least one token and within
    max_new; greedy, sampled and batched."""
    P, eos_from = 12, 20
    t = echo_model(tmp_path / "echo", eos_from)
    prompt = np.random.default_rng(5).integers(0, EOS, P).astype(np.int32)
    want = echo_expected(t, int(prompt[-1]), P - 1, 64)
    assert 0 < len(want) < 64 and len(want) == eos_from - P + 1
    eng = ie.Engine(tmp_path / "echo", max_batch=2)
    got, m = eng.generate_one(prompt, 64, greedy=True)
    assert got == want and m["tokens_generated"] == len(want)
    got_s, _ = eng.generate_one(prompt, 64, temperature=0.8, top_k=40, greedy=False)
    assert got_s == want
    prompts = np.stack([prompt, np.roll(prompt, 1)])
    out, m = eng.generate(prompts, 64)
    for b in range(2):
        w = echo_expected(t, int(prompts[b, -1]), P - 1, 64)
        assert out[b, :len(w)].tolist() == w and (out[b, len(w):] == -1).all()
    eng.close()


def test_session_continuation_positions(ie, tmp_path):
    """generate(..., reset_kv=false) continues the session
    (src/gpt2_engine.cu:680-698): the new prompt's positions follow the cached
    ones, so <|endoftext|> arrives where the position law puts it."""
    t = echo_model(tmp_path / "echo", 40)
    r = np.random.default_rng(6)
    p1, p2 = r.integers(0, EOS, 10).astype(np.int32), r.integers(0, EOS, 20).astype(np.int32)
    eng = ie.Engine(tmp_path / "echo", max_batch=1)
    t1, _ = eng.generate_one(p1, 3, greedy=True, reset=True)
    assert t1 == echo_expected(t, int(p1[-1]), 9, 3) and eng.session_tokens() == 13
    t2, _ = eng.generate_one(p2, 64, greedy=True, reset=False)
    want = echo_expected(t, int(p2[-1]), 13 + 20 - 1, 64)
    # picks from positions 32 .. 39 repeat the last prompt token; 40 gives EOS
    assert t2 == want and len(want) == 40 - 32
    assert eng.session_tokens() == 33 + len(want)  # every emitted token was fed
    eng.close()


@pytest.mark.parametrize("prefill", [True, False])
def test_session_continuation_attends_to_the_cache(ie, mid_dir, prefill):
    """A continuation prompt attends to the cached session: the engine's
    greedy picks across two generate() calls (the second with reset=False,
    through prefill or, as the reference does, through decode steps) equal the
    oracle's argmax over the whole token history, fed one position at a time,
    wherever the oracle's top-2 gap exceeds 6e-2 of the logit scale."""
    from oracle.gpt2_step import OracleGPT2

    r = np.random.default_rng(91)
    p1, p2 = r.integers(0, 1000, 20).astype(np.int32), r.integers(0, 1000, 15).astype(np.int32)
    eng = ie.Engine(mid_dir, max_batch=1, prefill=prefill)
    t1, _ = eng.generate_one(p1, 6, greedy=True, reset=True)
    t2, _ = eng.generate_one(p2, 6, greedy=True, reset=False)
    assert len(t1) == len(t2) == 6 and eng.session_tokens() == 20 + 6 + 15 + 6
    eng.close()
    seq = list(p1) + t1 + list(p2) + t2
    picks = {19 + j: t1[j] for j in range(6)}
    picks.update({40 + j: t2[j] for j in range(6)})
    om = OracleGPT2(str(mid_dir), batch=1)
    checked = 0
    for p, tok in enumerate(seq):
        want = om.step(np.array([tok], np.int32))[0]
        if p in picks:
            top = np.sort(want)[-2:]
            if top[1] - top[0] > 6e-2 * np.abs(want).max():
                assert picks[p] == int(np.argmax(want)), p
                checked += 1
    assert checked >= 6


def test_greedy_ties_take_the_lowest_index(ie, tmp_path):
    """Equal logits: the greedy token is the first index of the maximum
    (src/sampler.cu:10-14, std::max_element), also in the fused head, which
    merges per-workgroup maxima with a 64-bit atomic max.  The echo model with
    wte rows 5001 and 40000 copies of row 5000 gives those three rows equal
    logits whenever the input is any of them (rows 5000 and 5001 share a
    16-row vocabulary tile; 40000 is in another workgroup's).  Width 768, so
    the fused step and its fused head apply."""
    from gpt2_model import write_model

    t = echo_model(tmp_path / "base", 100, d=768)
    t["wte"][5001] = t["wte"][5000]
    t["wte"][40000] = t["wte"][5000]
    write_model(str(tmp_path / "ties"), echo_cfg(768), t, fp32_weights=False)
    prompts = np.array([[7, 40000], [9, 5001]], np.int32)
    for kw in (dict(), dict(fuse=False), dict(use_graph=False)):
        eng = ie.Engine(tmp_path / "ties", max_batch=2, **kw)
        out, _ = eng.generate(prompts, 4, ignore_eos=True)
        assert (out == 5000).all(), (kw, out)
        eng.close()


def test_text_prompt_path(ie, tmp_path):
    """The reference's text path (src/main.cpp:224-230): the prompt encoded by
    the BPE tokenizer from the model directory's vocab.json / merges.txt,
    generated from, and the ids decoded; the echo law gives the ids."""
    import json

    from oracle.bpe_tokenizer import byte_table

    d = tmp_path / "echo"
    t = echo_model(d, 40)
    sym = byte_table()
    vocab = {sym[b]: b for b in range(256)}
    vocab.update({"He": 256, "llo": 257, "Hello": 258, sym[0x20] + "world": 259, "<|endoftext|>": EOS})
    merges = [("H", "e"), ("l", "l"), ("ll", "o"), ("He", "llo"), (sym[0x20], "w"), (sym[0x20] + "w", "o"),
              (sym[0x20] + "wo", "r"), (sym[0x20] + "wor", "l"), (sym[0x20] + "worl", "d")]
    (d / "vocab.json").write_text(json.dumps(vocab))
    (d / "merges.txt").write_text("#version: 0.2\n" + "".join(f"{a} {b}\n" for a, b in merges), encoding="utf-8")
    tok = ie.Tokenizer(d)
    text = "Hello world, says the\techo"
    ids = tok.encode(text)
    assert ids[:2] == [258, 259] and tok.decode(ids) == b"Hello world, says the echo"
    eng = ie.Engine(d, max_batch=1)
    out, got, m = eng.generate_text(tok, text, 64, greedy=True)
    want = echo_expected(t, ids[-1], len(ids) - 1, 64)
    assert got == want and out == tok.decode(want) and m["tokens_generated"] == len(want)
    eng.close()
