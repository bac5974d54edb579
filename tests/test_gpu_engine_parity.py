"""GPT-2 Small engine parity that can fail at its stated bar.

* Teacher-forced, op by op: the engine's unfused decode step
  (GPT2Engine::Impl::enqueue_step_unfused, the reference's forward_layer decode
  branch src/gpt2_engine.cu:447-528 and :612-620) is driven from here through
  the public C ABI at full GPT-2 Small size (12 layers, d 768, 12 heads, vocab
  50257).  Every operation's output is checked against the oracle applied to
  the device's own input of that operation: embedding, quantizer and the
  Plain/Bias/Residual GEMMs bit-exact, the GELU GEMM within 2e-6 relative,
  LayerNorm, attention and the LM head within 1e-5 of their output scale.  The
  composed logits are then bit-identical to the engine's unfused and fused
  steps.  Together with the oracle's own pin (tests/test_oracle_gpt2_step.py:
  an independent float64 torch restatement, closed forms, planted mistakes)
  this holds the engine to the reference's composition op by op.
* Closed forms on the engine itself, GPT-2 Small shape: all linear weights
  zero -> logits = LN_f(wte[t] + wpe[p]) wte^T; weights zero, biases random ->
  x_L = x_0 + sum_l (out_bias_l + down_bias_l); LayerNorm gamma/beta random.
* The same op-by-op check at BASELINE configs[4]'s context: a 128-token
  prompt through the prefill path (all rows of every op), decode steps at
  positions 128-131, 255 and 380-383 with the context between advanced by
  prefill chunks, at batch 2 and 16; every composed result equal to the
  engine's prefill and decode steps (unfused and fused) bit for bit.
* BASELINE configs[4] at its stated length (prompt 128, 256 greedy tokens,
  batch 1 and 16): determinism, batch-16 rows equal to batch-1 runs, the
  fused step equal to the unfused one, graph replay equal to eager.
"""
import json
import os

import numpy as np
import pytest

from gpt2_model import random_tensors, write_model

pytestmark = pytest.mark.gpu

GPT2_SMALL = dict(n_layers=12, n_heads=12, d_model=768, d_ff=3072, vocab_size=50257, max_seq_len=1024)
BLOCK = 16


@pytest.fixture(scope="module")
def small_dir(tmp_path_factory):
    d = tmp_path_factory.mktemp("gpt2_small_ln")
    write_model(str(d), GPT2_SMALL, random_tensors(GPT2_SMALL, 31), fp32_weights=False)
    return d


def _rel(got, want):
    return float(np.abs(got - want).max() / max(np.abs(want).max(), 1e-30))


class CAbiStep:
    """The unfused decode step, op by op through the C ABI, with each op's
    output checked against the oracle on the op's device input."""

    def __init__(self, ie, orc, model_dir, B):
        import torch

        self.ie, self.orc, self.torch = ie, orc, torch
        c = json.load(open(os.path.join(model_dir, "config.json")))
        self.c = c
        d, ff, V, S, H = c["d_model"], c["d_ff"], c["vocab_size"], c["max_seq_len"], c["n_heads"]
        self.d, self.ff, self.V, self.S, self.H, self.dh = d, ff, V, S, H, c["d_head"]
        dev = torch.device("cuda:0")

        def f32(rel, n):
            return np.fromfile(os.path.join(model_dir, rel), np.float32).reshape(n)

        def i32(rel, n):
            return np.fromfile(os.path.join(model_dir, rel), np.int32).reshape(n)

        self.h = {"wte": f32("wte.bin", (V, d)), "wpe": f32("wpe.bin", (S, d)),
                  "lnf_g": f32("ln_f_gamma.bin", d), "lnf_b": f32("ln_f_beta.bin", d)}
        self.layers_h = []
        for i in range(c["n_layers"]):
            p = f"layer_{i:02d}/"
            L = {k: f32(p + f"{k}.bin", d) for k in ("ln1_gamma", "ln1_beta", "ln2_gamma", "ln2_beta")}
            for name, N, K in (("qkv", 3 * d, d), ("out", d, d), ("ffn_up", ff, d), ("ffn_down", d, ff)):
                L[name] = (i32(p + f"{name}_weight.bin", (N, K // 4)), f32(p + f"{name}_scale.bin", N),
                           f32(p + f"{name}_bias.bin", N))
            self.layers_h.append(L)

        def t(a):
            return torch.from_numpy(np.ascontiguousarray(a)).to(dev)

        self.g = {k: t(v) for k, v in self.h.items()}
        self.layers = [{k: (tuple(t(x) for x in v) if isinstance(v, tuple) else t(v)) for k, v in L.items()}
                       for L in self.layers_h]
        self.B = B
        self.nbps = (S + BLOCK - 1) // BLOCK
        self.table_h = np.arange(B * self.nbps, dtype=np.int32).reshape(B, self.nbps)
        self.table = t(self.table_h)
        P = B * self.nbps
        self.kc = [torch.zeros((P, BLOCK, H, self.dh), device=dev) for _ in range(c["n_layers"])]
        self.vc = [torch.zeros((P, BLOCK, H, self.dh), device=dev) for _ in range(c["n_layers"])]
        self.positions = torch.zeros(B, dtype=torch.int32, device=dev)
        self.ctx_lens = torch.zeros(B, dtype=torch.int32, device=dev)
        self.ws = torch.empty(ie.workspace_bytes(B, H, self.dh, 16) // 4, device=dev)
        self.pos = 0
        self.worst = {}

    def plan(self, ctx):
        """The engine's split plan (GPT2Engine::Impl::plan_for): one split per
        384 tokens, at most 16."""
        splits = max(1, min((ctx + 383) // 384, 16))
        max_ctx = self.S if splits == 16 else min(splits * 384, self.S)
        return splits, max_ctx

    def _note(self, what, v):
        self.worst[what] = max(self.worst.get(what, 0.0), v)

    def _ln(self, x, g, b, gh, bh):
        y = self.ie.layernorm(x, g, b)
        err = _rel(y.cpu().numpy(), self.orc.layernorm(x.cpu().numpy(), gh, bh))
        self._note("layernorm", err)
        assert err <= 1e-5, ("layernorm", err)
        return y

    def _quant(self, x):
        q, s = self.ie.quantize(x)
        wq, ws = self.orc.quantize(x.cpu().numpy())
        assert np.array_equal(q.cpu().numpy(), wq) and np.array_equal(s.cpu().numpy(), ws), "quantize"
        return q, s

    def _gemm(self, q, s, w, wh, epi, residual=None, out=None):
        res_h = None if residual is None else residual.cpu().numpy()  # before an in-place update
        got = self.ie.int8_gemm(q, w[0], s, w[1], epi, w[2], residual, out=out)
        want = self.orc.gemm(q.cpu().numpy(), wh[0], s.cpu().numpy(), wh[1], epi, wh[2], res_h)
        g = got.cpu().numpy()
        if epi == self.ie.EPI_BIAS_GELU:
            assert np.allclose(g, want, rtol=2e-6, atol=1e-7), ("gelu gemm", np.abs(g - want).max())
        else:
            assert np.array_equal(g, want), ("gemm", epi, np.abs(g - want).max())
        return got

    def prefill(self, tokens, check=True):
        """A prompt chunk of P tokens per sequence at positions pos .. pos + P - 1
        (GPT2Engine::Impl::prefill: M = B x P rows per op, the K/V of the chunk
        appended, causal prefill attention over the cache; the reference's
        is_prefill branch, src/gpt2_engine.cu:447-528 and :660-676).  Every op
        is checked on all its rows against the oracle on its device input
        (check=False runs the same ops unchecked, to advance the context);
        returns the last token's logits [B, V]."""
        ie, orc, torch = self.ie, self.orc, self.torch
        tokens = np.asarray(tokens, np.int32)
        B, P = tokens.shape
        assert B == self.B
        d, H, dh, start, M = self.d, self.H, self.dh, self.pos, B * P
        ids = torch.from_numpy(tokens.reshape(-1).copy()).cuda()
        x = torch.empty((M, d), device="cuda")
        for b in range(B):
            ie.embedding(ids[b * P:(b + 1) * P], start, self.g["wte"], self.g["wpe"], out=x[b * P:(b + 1) * P])
        if check:
            want = np.concatenate([orc.embedding(tokens[b], start, self.h["wte"], self.h["wpe"]) for b in range(B)])
            assert np.array_equal(x.cpu().numpy(), want), "embedding"
        pos_bt = start + np.arange(P)
        lens = np.tile(pos_bt + 1, B).astype(np.int32)   # query (b, t) sees start + t + 1 tokens
        table_rep = np.repeat(self.table_h, P, axis=0)
        saved = (self._ln, self._quant, self._gemm)
        if not check:
            self._ln = lambda x_, g, b_, gh, bh: ie.layernorm(x_, g, b_)
            self._quant = lambda x_: ie.quantize(x_)
            self._gemm = lambda q_, s_, w, wh, epi, residual=None, out=None: ie.int8_gemm(
                q_, w[0], s_, w[1], epi, w[2], residual, out=out)
        try:
            for l, (L, Lh) in enumerate(zip(self.layers, self.layers_h)):
                xn = self._ln(x, L["ln1_gamma"], L["ln1_beta"], Lh["ln1_gamma"], Lh["ln1_beta"])
                q8, s8 = self._quant(xn)
                qkv = self._gemm(q8, s8, L["qkv"], Lh["qkv"], ie.EPI_BIAS)
                q = qkv[:, :d].contiguous().view(B, P, H, dh)
                k = qkv[:, d:2 * d].contiguous().view(B, P, H, dh)
                v = qkv[:, 2 * d:].contiguous().view(B, P, H, dh)
                for b in range(B):
                    ie.kv_cache_write(k[b], v[b], self.kc[l], self.vc[l], self.table[b], start, BLOCK)
                attn = ie.prefill_attn(q, self.kc[l], self.vc[l], self.table, start, BLOCK, H).view(M, d)
                if check:
                    kc_h, vc_h = self.kc[l].cpu().numpy(), self.vc[l].cpu().numpy()
                    slots = self.table_h[:, pos_bt // BLOCK]                      # [B, P]
                    assert np.array_equal(kc_h[slots, pos_bt % BLOCK], k.cpu().numpy()), "kv write"
                    assert np.array_equal(vc_h[slots, pos_bt % BLOCK], v.cpu().numpy()), "kv write"
                    want = orc.decode_attn(q.cpu().numpy().reshape(M, H, dh), kc_h, vc_h, table_rep, lens,
                                           start + P, BLOCK, H).reshape(M, d)
                    err = _rel(attn.cpu().numpy(), want)
                    self._note("prefill_attn", err)
                    assert err <= 1e-5, ("prefill_attn", l, err)
                q8, s8 = self._quant(attn)
                self._gemm(q8, s8, L["out"], Lh["out"], ie.EPI_BIAS_RESIDUAL, residual=x, out=x)
                xn = self._ln(x, L["ln2_gamma"], L["ln2_beta"], Lh["ln2_gamma"], Lh["ln2_beta"])
                q8, s8 = self._quant(xn)
                hdn = self._gemm(q8, s8, L["ffn_up"], Lh["ffn_up"], ie.EPI_BIAS_GELU)
                q8, s8 = self._quant(hdn)
                self._gemm(q8, s8, L["ffn_down"], Lh["ffn_down"], ie.EPI_BIAS_RESIDUAL, residual=x, out=x)
        finally:
            self._ln, self._quant, self._gemm = saved
        last = x.view(B, P, d)[:, P - 1].contiguous()
        xf = self._ln(last, self.g["lnf_g"], self.g["lnf_b"], self.h["lnf_g"], self.h["lnf_b"])
        logits = ie.vocab_proj(xf, self.g["wte"]).cpu().numpy()
        want = np.stack([orc.vocab_proj(row, self.h["wte"]) for row in xf.cpu().numpy()])
        err = _rel(logits, want)
        self._note("lm_head", err)
        assert err <= 1e-5, ("lm_head", err)
        self.pos = start + P
        self.positions.fill_(self.pos)
        return logits

    def step(self, tokens):
        ie, orc, torch = self.ie, self.orc, self.torch
        B, d, H, dh = self.B, self.d, self.H, self.dh
        tok = torch.tensor(np.asarray(tokens, np.int32), device="cuda")
        x = torch.empty((B, d), device="cuda")
        ie.check("ie_embedding_batch", B, ie._ptr(tok), ie._ptr(self.positions), d, ie._ptr(self.g["wte"]),
                 ie._ptr(self.g["wpe"]), ie._ptr(x), ie._stream())
        want = np.concatenate([orc.embedding(np.asarray(tokens[b:b + 1], np.int32), self.pos, self.h["wte"],
                                             self.h["wpe"]) for b in range(B)])
        assert np.array_equal(x.cpu().numpy(), want), "embedding"
        ctx = self.pos + 1
        splits, max_ctx = self.plan(ctx)
        for l, (L, Lh) in enumerate(zip(self.layers, self.layers_h)):
            xn = self._ln(x, L["ln1_gamma"], L["ln1_beta"], Lh["ln1_gamma"], Lh["ln1_beta"])
            q8, s8 = self._quant(xn)
            qkv = self._gemm(q8, s8, L["qkv"], Lh["qkv"], ie.EPI_BIAS)
            q = qkv[:, :d].contiguous()
            k = qkv[:, d:2 * d].contiguous().view(B, H, dh)
            v = qkv[:, 2 * d:].contiguous().view(B, H, dh)
            ie.kv_cache_append_batch(k, v, self.kc[l], self.vc[l], self.table, self.positions, BLOCK)
            self.ctx_lens.copy_(self.positions + 1)
            kc_h, vc_h = self.kc[l].cpu().numpy(), self.vc[l].cpu().numpy()
            for b in range(B):
                slot = self.table_h[b, self.pos // BLOCK]
                assert np.array_equal(kc_h[slot, self.pos % BLOCK], k[b].cpu().numpy()), "kv append"
                assert np.array_equal(vc_h[slot, self.pos % BLOCK], v[b].cpu().numpy()), "kv append"
            attn = ie.decode_attn(q.view(B, H, dh), self.kc[l], self.vc[l], self.table, self.ctx_lens, max_ctx,
                                  BLOCK, H, splits=splits, workspace=self.ws).view(B, d)
            want = orc.decode_attn(q.cpu().numpy().reshape(B, H, dh), kc_h, vc_h, self.table_h,
                                   np.full(B, ctx, np.int32), max_ctx, BLOCK, H).reshape(B, d)
            err = _rel(attn.cpu().numpy(), want)
            self._note("decode_attn", err)
            assert err <= 1e-5, ("decode_attn", l, err)
            q8, s8 = self._quant(attn)
            self._gemm(q8, s8, L["out"], Lh["out"], ie.EPI_BIAS_RESIDUAL, residual=x, out=x)
            xn = self._ln(x, L["ln2_gamma"], L["ln2_beta"], Lh["ln2_gamma"], Lh["ln2_beta"])
            q8, s8 = self._quant(xn)
            hdn = self._gemm(q8, s8, L["ffn_up"], Lh["ffn_up"], ie.EPI_BIAS_GELU)
            q8, s8 = self._quant(hdn)
            self._gemm(q8, s8, L["ffn_down"], Lh["ffn_down"], ie.EPI_BIAS_RESIDUAL, residual=x, out=x)
        xf = self._ln(x, self.g["lnf_g"], self.g["lnf_b"], self.h["lnf_g"], self.h["lnf_b"])
        logits = ie.vocab_proj(xf, self.g["wte"])
        xf_h = xf.cpu().numpy()
        got = logits.cpu().numpy()
        want = np.stack([orc.vocab_proj(xf_h[b], self.h["wte"]) for b in range(B)])
        err = _rel(got, want)
        self._note("lm_head", err)
        assert err <= 1e-5, ("lm_head", err)
        self.positions += 1
        self.pos += 1
        return got


def test_teacher_forced_gpt2_small_every_op(ie, orc, small_dir):
    """Four decode steps at batch 2 through all 12 layers: every op matches
    the oracle on its own input, and the composed logits equal the engine's
    unfused and fused steps bit for bit."""
    B, steps = 2, 4
    rng = np.random.default_rng(17)
    toks = rng.integers(0, GPT2_SMALL["vocab_size"], (steps, B)).astype(np.int32)
    cabi = CAbiStep(ie, orc, str(small_dir), B)
    unfused = ie.Engine(small_dir, max_batch=B, fuse=False)
    fused = ie.Engine(small_dir, max_batch=B)
    for t in toks:
        want = cabi.step(t)
        assert np.array_equal(unfused.step(t), want)
        assert np.array_equal(fused.step(t), want)
    print("worst relative error per op:", cabi.worst)
    unfused.close()
    fused.close()


# BASELINE configs[4]'s context: a 128-token prompt prefilled, then decode
# steps at positions 128-131 (the first block after the prompt), 255 (the last
# slot of block 15) and 380-383 (the run's last positions), the context
# between them advanced by prefill chunks continuing the session.
CFG5_SCHEDULE = [("prefill", 128, True), ("decode", 4), ("prefill", 123, True), ("decode", 1),
                 ("prefill", 124, True), ("decode", 4)]


def run_schedule(ie, orc, small_dir, B, schedule, seed):
    """Drive the op-by-op C ABI model and the engine (unfused and fused)
    through the same prompt chunks and decode tokens; every composed result
    must equal the engines' bit for bit."""
    rng = np.random.default_rng(seed)
    cabi = CAbiStep(ie, orc, str(small_dir), B)
    engines = [ie.Engine(small_dir, max_batch=B, fuse=False), ie.Engine(small_dir, max_batch=B)]
    try:
        for item in schedule:
            if item[0] == "prefill":
                _, P, check = item
                toks = rng.integers(0, GPT2_SMALL["vocab_size"], (B, P)).astype(np.int32)
                want = cabi.prefill(toks, check=check)
                for e in engines:
                    assert np.array_equal(e.prefill(toks), want), ("prefill", cabi.pos)
            else:
                for _ in range(item[1]):
                    at = cabi.pos
                    t = rng.integers(0, GPT2_SMALL["vocab_size"], B).astype(np.int32)
                    want = cabi.step(t)
                    for e in engines:
                        assert np.array_equal(e.step(t), want), ("decode", at)
        # the last decode step ran at position 383: 384 tokens in the session
        assert cabi.pos == 384 and all(e.session_tokens() == cabi.pos for e in engines)
    finally:
        for e in engines:
            e.close()
    print("worst relative error per op:", cabi.worst)


def test_teacher_forced_cfg5_context_batch2(ie, orc, small_dir):
    """GPT-2 Small at BASELINE configs[4]'s context, batch 2: the prompt's
    prefill and every decode step checked op by op on all rows."""
    run_schedule(ie, orc, small_dir, 2, CFG5_SCHEDULE, 23)


def test_teacher_forced_cfg5_context_batch16(ie, orc, small_dir):
    """The same at batch 16 (the configs[4] batch): the 128-token prompt
    (2048 rows per op) and every decode step checked on all rows; the two
    chunks that advance the context between the decode positions run the
    same ops unchecked (checked at batch 2 above) and still must equal the
    engines' prefill bit for bit."""
    sched = [("prefill", 128, True), ("decode", 4), ("prefill", 123, False), ("decode", 1),
             ("prefill", 124, False), ("decode", 4)]
    run_schedule(ie, orc, small_dir, 16, sched, 29)


def closed_form_logits(t, tokens, pos):
    """LN_f(x_L) wte^T in float64; x_L is the fp32 embedding plus, per layer,
    out_bias then down_bias (fp32 adds: the residual epilogue when the GEMM
    term is exactly 0)."""
    x = (t["wte"][tokens] + t["wpe"][pos][None, :]).astype(np.float32)
    for lay in t["layers"]:
        x = (x + lay["out_b"][None, :]).astype(np.float32)
        x = (x + lay["ffn_down_b"][None, :]).astype(np.float32)
    x = x.astype(np.float64)
    mu = x.mean(axis=1, keepdims=True)
    var = ((x - mu) ** 2).mean(axis=1, keepdims=True)
    xf = (x - mu) / np.sqrt(var + 1e-5) * t["ln_f_gamma"].astype(np.float64) + t["ln_f_beta"].astype(np.float64)
    return xf @ t["wte"].astype(np.float64).T


@pytest.mark.parametrize("biases", [False, True])
def test_closed_form_zero_weight_models(ie, tmp_path, biases):
    """GPT-2 Small shape with every linear weight zero, fused and unfused
    steps, graph replay: the layers add exactly their out and down biases (or
    nothing), so the logits have a closed form."""
    t = random_tensors(GPT2_SMALL, 41 + biases, zero_weights=True, zero_biases=not biases, b_std=0.5)
    d = write_model(str(tmp_path / "m"), GPT2_SMALL, t, fp32_weights=False)
    B = 3
    rng = np.random.default_rng(9)
    toks = rng.integers(0, GPT2_SMALL["vocab_size"], (5, B)).astype(np.int32)
    for kw in (dict(), dict(fuse=False)):
        eng = ie.Engine(d, max_batch=B, **kw)
        for p, tk in enumerate(toks):
            got = eng.step(tk)
            want = closed_form_logits(t, tk, p)
            assert _rel(got, want) <= 1e-5, (kw, p, _rel(got, want))
        eng.close()


def test_baseline_cfg5_full_length(ie):
    """GPT-2 Small random-init, prompt of 128 random ids,
    256 greedy tokens at batch 16 and 1."""
    rng = np.random.default_rng(128)
    prompts = rng.integers(0, 50257, (16, 128)).astype(np.int32)
    eng = ie.Engine(None, seed=1234, max_batch=16)
    a, m = eng.generate(prompts, 256, ignore_eos=True)
    b, _ = eng.generate(prompts, 256, ignore_eos=True)
    assert np.array_equal(a, b) and (a >= 0).all() and (a < 50257).all()
    assert m["tokens_generated"] == 256 and eng.session_tokens() == 128 + 255
    for i in (0, 9, 15):
        one, _ = eng.generate(prompts[i:i + 1], 256, ignore_eos=True)
        assert np.array_equal(one[0], a[i]), i
    eng.close()
    for kw in (dict(fuse=False), dict(use_graph=False)):
        other = ie.Engine(None, seed=1234, max_batch=16, **kw)
        c, _ = other.generate(prompts, 256, ignore_eos=True)
        assert np.array_equal(c, a), kw
        other.close()
