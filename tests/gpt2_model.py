"""Test helpers: GPT-2 models with chosen tensors, written in the reference's
on-disk format (python/export_gpt2.py:73-167), and an independent float64
torch restatement of the quantized decode step used to pin the oracle.

Model tensors are held in the exporter's source layout: linear weights as
fp32 [K=in, N=out] ("x @ W", HF Conv1D), transposed to [N, K] and quantized
per output row before they are written (export_gpt2.py:116-167), with the
fp32 [K, N] copy written beside them as `{name}_weight_fp32.bin`
(export_gpt2.py:48-57).
"""
from __future__ import annotations

import json
import math
import os

import numpy as np

LINEARS = ("qkv", "out", "ffn_up", "ffn_down")


def linear_shapes(d, ff):
    """name -> (K, N) of each linear in a layer."""
    return {"qkv": (d, 3 * d), "out": (d, d), "ffn_up": (d, ff), "ffn_down": (ff, d)}


def random_tensors(cfg, seed, w_std=0.02, b_std=0.02, ln_jitter=0.1, zero_weights=False,
                   zero_biases=False):
    """Random model tensors (fp32).  ln_jitter > 0 gives LayerNorm gamma
    1 + N(0, jitter) and beta N(0, jitter / 2), so that mixing up the two
    LayerNorms of a layer (or the final one) changes the output."""
    r = np.random.default_rng(seed)
    d, ff, V, S, L = cfg["d_model"], cfg["d_ff"], cfg["vocab_size"], cfg["max_seq_len"], cfg["n_layers"]

    def nrm(*shape, std):
        return (r.standard_normal(shape) * std).astype(np.float32)

    def ln():
        if ln_jitter == 0:
            return np.ones(d, np.float32), np.zeros(d, np.float32)
        return 1 + nrm(d, std=ln_jitter), nrm(d, std=ln_jitter / 2)

    t = {"wte": nrm(V, d, std=0.02), "wpe": nrm(S, d, std=0.02)}
    t["ln_f_gamma"], t["ln_f_beta"] = ln()
    t["layers"] = []
    for _ in range(L):
        lay = {}
        lay["ln1_gamma"], lay["ln1_beta"] = ln()
        lay["ln2_gamma"], lay["ln2_beta"] = ln()
        for name, (K, N) in linear_shapes(d, ff).items():
            lay[name + "_w"] = np.zeros((K, N), np.float32) if zero_weights else nrm(K, N, std=w_std)
            lay[name + "_b"] = np.zeros(N, np.float32) if zero_biases else nrm(N, std=b_std)
        t["layers"].append(lay)
    return t


def quantize_per_row(w):
    """export_gpt2.py:10-40 in numpy float32: scale = max|row| / 127 (1 for a
    zero row), q = clip(round(row * (1 / scale)), -128, 127) with round half
    to even, packed four per int32 little-endian."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    m = np.abs(w).max(axis=1)
    scale = np.where(m > 0, m / np.float32(127.0), np.float32(1.0)).astype(np.float32)
    inv = (np.float32(1.0) / scale).astype(np.float32)
    q = np.clip(np.rint(w * inv[:, None]), -128, 127).astype(np.int8)
    return q.view(np.int32).reshape(w.shape[0], -1).copy(), scale


def write_model(path, cfg, t, fp32_weights=True):
    """Writes tensors t (random_tensors layout) to directory `path`."""
    os.makedirs(path, exist_ok=True)
    c = dict(cfg)
    c["d_head"] = c["d_model"] // c["n_heads"]
    keys = ("n_layers", "n_heads", "d_model", "d_ff", "vocab_size", "max_seq_len", "d_head")
    with open(os.path.join(path, "config.json"), "w") as f:
        json.dump({k: c[k] for k in keys}, f, indent=2)
    for k in ("wte", "wpe", "ln_f_gamma", "ln_f_beta"):
        np.ascontiguousarray(t[k], np.float32).tofile(os.path.join(path, f"{k}.bin"))
    for i, lay in enumerate(t["layers"]):
        p = os.path.join(path, f"layer_{i:02d}")
        os.makedirs(p, exist_ok=True)
        for k in ("ln1_gamma", "ln1_beta", "ln2_gamma", "ln2_beta"):
            np.ascontiguousarray(lay[k], np.float32).tofile(os.path.join(p, f"{k}.bin"))
        for name in LINEARS:
            w = lay[name + "_w"]
            packed, scale = quantize_per_row(w.T)
            packed.tofile(os.path.join(p, f"{name}_weight.bin"))
            scale.tofile(os.path.join(p, f"{name}_scale.bin"))
            np.ascontiguousarray(lay[name + "_b"], np.float32).tofile(os.path.join(p, f"{name}_bias.bin"))
            if fp32_weights:
                np.ascontiguousarray(w, np.float32).tofile(os.path.join(p, f"{name}_weight_fp32.bin"))
    return path


class TorchRefGPT2:
    """The quantized GPT-2 decode step restated in float64 torch, written
    independently of oracle/gpt2_step.py: it reads the model directory itself,
    keeps a contiguous per-sequence K/V history (no paging), and takes every
    step from the published GPT-2 block (Radford et al. 2019; the reference's
    src/gpt2_engine.cu:447-528,612-620) with the reference's W8A8 arithmetic
    at the points where it quantizes:
      x = wte[t] + wpe[p]
      per layer: a = LN1(x); q,k,v = Lin_qkv(a); o = softmax(q k^T / sqrt(dh)) v
                 x = x + Lin_out(o); h = GELU_tanh(Lin_up(LN2(x))); x = x + Lin_down(h)
      logits = LN_f(x) wte^T      (or the INT8 head: Lin over quantized wte)
    where Lin_w(a) = (int8(a) . int8(W)) * s_a * s_w + bias, int8() being the
    per-row symmetric quantizer applied to the fp32 rounding of `a`.  All other
    arithmetic is float64.  With quantized=False the linears are plain
    float64 x @ W + b on the exporter's fp32 [K, N] weights (the reference's
    fp32 cuBLAS backend, src/gpt2_engine.cu:530-610).  `min_margin` records the smallest distance (in
    quantization steps) of any quantizer input from a rounding boundary:
    float32-level differences between two implementations cannot change a
    quantized value while it stays above ~1e-4.
    """

    def __init__(self, path, batch=1, int8_lm_head=False, kv_bf16=False, quantized=True):
        import torch

        self.torch = torch
        c = json.load(open(os.path.join(path, "config.json")))
        self.c = c
        d, ff, V, S = c["d_model"], c["d_ff"], c["vocab_size"], c["max_seq_len"]
        self.H, self.dh = c["n_heads"], c["d_head"]

        def f(rel, shape):
            a = np.fromfile(os.path.join(path, rel), np.float32).reshape(shape)
            return torch.from_numpy(a).double()

        def q(p, name, N, K):
            b = f(f"{p}/{name}_bias.bin", (N,))
            if not quantized:  # the exporter's fp32 [K, N] weights
                return (f(f"{p}/{name}_weight_fp32.bin", (K, N)), b)
            w = np.fromfile(os.path.join(path, p, f"{name}_weight.bin"), np.int8).reshape(N, K)
            s = np.fromfile(os.path.join(path, p, f"{name}_scale.bin"), np.float32)
            return (torch.from_numpy(w.astype(np.int64)), torch.from_numpy(s).double(), b)

        self.wte = f("wte.bin", (V, d))
        self.wpe = f("wpe.bin", (S, d))
        self.lnf = (f("ln_f_gamma.bin", (d,)), f("ln_f_beta.bin", (d,)))
        self.layers = []
        for i in range(c["n_layers"]):
            p = f"layer_{i:02d}"
            self.layers.append(dict(
                ln1=(f(f"{p}/ln1_gamma.bin", (d,)), f(f"{p}/ln1_beta.bin", (d,))),
                ln2=(f(f"{p}/ln2_gamma.bin", (d,)), f(f"{p}/ln2_beta.bin", (d,))),
                qkv=q(p, "qkv", 3 * d, d), out=q(p, "out", d, d),
                up=q(p, "ffn_up", ff, d), down=q(p, "ffn_down", d, ff)))
        self.int8_lm_head = int8_lm_head
        if int8_lm_head:
            w = self.wte.float().numpy()
            packed, s = quantize_per_row(w)
            self.head = (torch.from_numpy(packed.view(np.int8).astype(np.int64)), torch.from_numpy(s).double())
        self.kv_bf16 = kv_bf16
        self.B = batch
        self.K = [[[] for _ in range(batch)] for _ in range(c["n_layers"])]
        self.V = [[[] for _ in range(batch)] for _ in range(c["n_layers"])]
        self.pos = 0
        self.min_margin = math.inf

    def quant(self, a):
        """[rows, cols] float64 -> (int64 q, float64 scale) of a's fp32 rounding."""
        torch = self.torch
        x = a.float()
        m = x.abs().amax(dim=1)
        scale = torch.where(m > 0, m / torch.tensor(127.0), torch.tensor(1.0))
        inv = torch.tensor(1.0) / scale
        t = x * inv[:, None]                      # float32 product, as the quantizer forms it
        frac = (t.double() - torch.floor(t.double())).sub(0.5).abs()
        self.min_margin = min(self.min_margin, float(frac.min()))
        qv = torch.clamp(torch.round(t), -128, 127).long()
        return qv, scale.double()

    def lin(self, a, w):
        if len(w) == 2:  # unquantized: x @ W + b in float64
            return a @ w[0] + w[1][None, :]
        qa, sa = self.quant(a)
        wq, ws, b = w
        return (qa @ wq.T).double() * sa[:, None] * ws[None, :] + b[None, :]

    def ln(self, x, gb):
        return self.torch.nn.functional.layer_norm(x, (x.shape[-1],), gb[0], gb[1], eps=1e-5)

    def step(self, tokens):
        torch = self.torch
        B, H, dh, d = self.B, self.H, self.dh, self.c["d_model"]
        tok = torch.as_tensor(np.asarray(tokens, np.int64))
        x = self.wte[tok] + self.wpe[self.pos][None, :]
        for li, L in enumerate(self.layers):
            qkv = self.lin(self.ln(x, L["ln1"]), L["qkv"])
            q, k, v = qkv[:, :d], qkv[:, d:2 * d], qkv[:, 2 * d:]
            if self.kv_bf16:
                k, v = k.float().bfloat16().double(), v.float().bfloat16().double()
            o = torch.empty(B, d, dtype=torch.float64)
            for b in range(B):
                self.K[li][b].append(k[b].reshape(H, dh))
                self.V[li][b].append(v[b].reshape(H, dh))
                Kb = torch.stack(self.K[li][b])          # [t, H, dh]
                Vb = torch.stack(self.V[li][b])
                s = torch.einsum("hd,thd->ht", q[b].reshape(H, dh), Kb) / math.sqrt(dh)
                p = torch.softmax(s, dim=1)
                o[b] = torch.einsum("ht,thd->hd", p, Vb).reshape(d)
            x = x + self.lin(o, L["out"])
            h = torch.nn.functional.gelu(self.lin(self.ln(x, L["ln2"]), L["up"]), approximate="tanh")
            x = x + self.lin(h, L["down"])
        xf = self.ln(x, self.lnf)
        if self.int8_lm_head:
            qa, sa = self.quant(xf)
            logits = (qa @ self.head[0].T).double() * sa[:, None] * self.head[1][None, :]
        else:
            logits = xf @ self.wte.T
        self.pos += 1
        return logits.numpy()
