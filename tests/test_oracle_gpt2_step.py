"""Pins the decode-step oracle (oracle/gpt2_step.py, the composition of the
reference's GPT2Engine::forward_layer decode branch, src/gpt2_engine.cu:447-528,
forward_final_ln / forward_logits :612-620) without trusting it:

* against TorchRefGPT2 (tests/gpt2_model.py), a float64 torch restatement of
  the GPT-2 block written independently (its own loader, contiguous K/V, torch
  layer_norm / softmax / tanh-GELU), quantizing where the reference quantizes;
* against closed forms: with every linear weight zero the layers pass the
  residual stream through unchanged, so logits = LN_f(wte[t] + wpe[p]) wte^T;
  with weights zero and biases set, x_L = x_0 + sum_l (out_bias_l + down_bias_l);
* planted mistakes (in the oracle, on the CPU) that the comparison must catch:
  LayerNorms swapped, a bias dropped, K and V exchanged, the final LayerNorm
  replaced, positions shifted by one, heads misaligned.

The models have non-trivial LayerNorm gamma/beta and biases, so each of those
mistakes changes the output.  Bar: with every quantizer input at least 5e-5
of a step from a rounding boundary (asserted; the two implementations' inputs
differ by about 1e-7 relative, at most ~2.5e-5 of a step at |q| = 127, so no
quantized value can differ) the logits agree within 2e-6 of their scale.
The models' seeds are ones that meet the margin (most do not: a flip is a
one-step change of one int8 value, after which the logits legitimately move
by up to ~1e-2 of their scale).
"""
import numpy as np
import pytest

from gpt2_model import TorchRefGPT2, random_tensors, write_model

ONE_HEAD = dict(n_layers=2, n_heads=1, d_model=64, d_ff=128, vocab_size=97, max_seq_len=32)
TWO_HEADS = dict(n_layers=2, n_heads=2, d_model=128, d_ff=256, vocab_size=101, max_seq_len=40)
BAR = 2e-6
MARGIN = 5e-5


def compare(model_dir, B, steps, seed, okw=None, rkw=None, mutate=None):
    from oracle.gpt2_step import OracleGPT2

    o = OracleGPT2(str(model_dir), batch=B, **(okw or {}))
    r = TorchRefGPT2(str(model_dir), batch=B, **(rkw or {}))
    if mutate:
        mutate(o)
    V = r.c["vocab_size"]
    rng = np.random.default_rng(seed)
    err = 0.0
    for _ in range(steps):
        t = rng.integers(0, V, B)
        a, b = o.step(t), r.step(t)
        err = max(err, float(np.abs(a - b).max() / np.abs(b).max()))
    return err, r.min_margin


def make(tmp_path, cfg, seed, **kw):
    return write_model(str(tmp_path / f"m{seed}"), cfg, random_tensors(cfg, seed, **kw), fp32_weights=False)


@pytest.mark.parametrize("cfg,seed", [(ONE_HEAD, 2), (ONE_HEAD, 9), (TWO_HEADS, 6), (TWO_HEADS, 11)])
def test_oracle_step_matches_torch_fp64(orc, tmp_path, cfg, seed):
    d = make(tmp_path, cfg, seed)
    err, margin = compare(d, 2, 6, 100 + seed)
    assert margin > MARGIN, margin
    assert err <= BAR, err


@pytest.mark.parametrize("seed,kw", [(2, dict(int8_lm_head=True)), (7, dict(kv_bf16=True))])
def test_oracle_step_variants_match_torch_fp64(orc, tmp_path, seed, kw):
    d = make(tmp_path, ONE_HEAD, seed)
    err, margin = compare(d, 2, 6, 100 + seed, kw, kw)
    assert margin > MARGIN, margin
    assert err <= BAR, err


def _swap_ln(o):
    for L in o.layers:
        L["ln1"], L["ln2"] = L["ln2"], L["ln1"]


def _drop_out_bias(o):
    w, s, b = o.layers[1]["out"]
    o.layers[1]["out"] = (w, s, np.zeros_like(b))


def _swap_kv(o):
    d = o.d
    w, s, b = o.layers[0]["qkv"]
    perm = np.r_[0:d, 2 * d:3 * d, d:2 * d]
    o.layers[0]["qkv"] = (w[perm].copy(), s[perm].copy(), b[perm].copy())


def _final_ln_from_layer(o):
    o.lnf = o.layers[-1]["ln2"]


def _shift_positions(o):
    o.pos = 1


def _misalign_heads(o):
    # Q's two head blocks exchanged: query head h meets key head 1 - h
    d, dh = o.d, o.dh
    w, s, b = o.layers[0]["qkv"]
    perm = np.r_[dh:2 * dh, 0:dh, d:3 * d]
    o.layers[0]["qkv"] = (w[perm].copy(), s[perm].copy(), b[perm].copy())


@pytest.mark.parametrize("mutate", [_swap_ln, _drop_out_bias, _swap_kv, _final_ln_from_layer,
                                    _shift_positions, _misalign_heads])
def test_planted_composition_mistakes_are_caught(orc, tmp_path, mutate):
    d = make(tmp_path, TWO_HEADS, 4)
    err, _ = compare(d, 2, 6, 104, mutate=mutate)
    assert err > 100 * BAR, (mutate.__name__, err)


def test_zero_weights_pass_the_residual_stream_through(orc, tmp_path):
    """All linear weights and biases zero: Q = K = V = 0, attention returns 0,
    and each residual epilogue adds exactly 0, so the hidden row leaving the
    last layer is the embedding itself."""
    from oracle.gpt2_step import OracleGPT2

    cfg = TWO_HEADS
    t = random_tensors(cfg, 21, zero_weights=True, zero_biases=True)
    d = write_model(str(tmp_path / "zero"), cfg, t, fp32_weights=False)
    o = OracleGPT2(d, batch=3)
    rng = np.random.default_rng(5)
    for p in range(5):
        tok = rng.integers(0, cfg["vocab_size"], 3)
        got = o.step(tok)
        want = closed_form_logits(t, tok, p)
        assert np.abs(got - want).max() <= 1e-6 * np.abs(want).max()


def test_biases_only_add_to_the_residual_stream(orc, tmp_path):
    """Weights zero, biases random: each layer adds out_bias and then
    down_bias to x (the attention and FFN paths end in zero weights)."""
    from oracle.gpt2_step import OracleGPT2

    cfg = TWO_HEADS
    t = random_tensors(cfg, 22, zero_weights=True, b_std=0.5)
    d = write_model(str(tmp_path / "bias"), cfg, t, fp32_weights=False)
    o = OracleGPT2(d, batch=2)
    rng = np.random.default_rng(6)
    for p in range(4):
        tok = rng.integers(0, cfg["vocab_size"], 2)
        got = o.step(tok)
        want = closed_form_logits(t, tok, p)
        assert np.abs(got - want).max() <= 1e-6 * np.abs(want).max()


def closed_form_logits(t, tokens, pos):
    """LN_f(x_L) wte^T in float64 for the zero-weight models: x_L = fp32
    embedding plus, per layer in order, the out and down biases (fp32 adds,
    the residual epilogue's arithmetic when the GEMM term is 0)."""
    x = (t["wte"][tokens] + t["wpe"][pos][None, :]).astype(np.float32)
    for lay in t["layers"]:
        x = (x + lay["out_b"][None, :]).astype(np.float32)
        x = (x + lay["ffn_down_b"][None, :]).astype(np.float32)
    x = x.astype(np.float64)
    mu = x.mean(axis=1, keepdims=True)
    var = ((x - mu) ** 2).mean(axis=1, keepdims=True)
    xf = (x - mu) / np.sqrt(var + 1e-5) * t["ln_f_gamma"].astype(np.float64) + t["ln_f_beta"].astype(np.float64)
    return xf @ t["wte"].astype(np.float64).T
