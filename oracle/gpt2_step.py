"""CPU restatement of the reference engine's decode step — TEST INFRASTRUCTURE.

Composes the oracle's functions (oracle/orc.py) in the order of
GPT2Engine::forward_layer's decode branch (src/gpt2_engine.cu:447-528),
forward_final_ln (:612-616) and forward_logits (:618-620), on a model
directory in the reference's on-disk format (python/export_gpt2.py:73-167).
Used only by tests to check the HIP engine.  Batch b keeps its own paged KV
cache rows: physical block = b * blocks_per_seq + logical block, as the engine
lays them out (the reference engine has one sequence and an identity table,
src/gpt2_engine.cu:420-429).
"""
from __future__ import annotations

import json
import os

import numpy as np

from oracle import orc

BLOCK = 16


def _f32(path, n):
    a = np.fromfile(path, dtype=np.float32)
    assert a.size == n, path
    return a


def _i32(path, n):
    a = np.fromfile(path, dtype=np.int32)
    assert a.size == n, path
    return a


def bf16_round(x: np.ndarray) -> np.ndarray:
    """fp32 -> nearest bf16 (ties to even), returned as fp32 (finite inputs)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)


class OracleGPT2:
    def __init__(self, model_dir: str, batch: int = 1, int8_lm_head: bool = False, kv_bf16: bool = False):
        c = json.load(open(os.path.join(model_dir, "config.json")))
        self.c = c
        d, ff, V, L, S = c["d_model"], c["d_ff"], c["vocab_size"], c["n_layers"], c["max_seq_len"]
        self.d, self.ff, self.V, self.H, self.dh = d, ff, V, c["n_heads"], c["d_head"]
        self.wte = _f32(os.path.join(model_dir, "wte.bin"), V * d).reshape(V, d)
        self.wpe = _f32(os.path.join(model_dir, "wpe.bin"), S * d).reshape(S, d)
        self.lnf = (_f32(os.path.join(model_dir, "ln_f_gamma.bin"), d), _f32(os.path.join(model_dir, "ln_f_beta.bin"), d))
        self.layers = []
        for i in range(L):
            p = os.path.join(model_dir, f"layer_{i:02d}")

            def q(name, N, K):
                return (_i32(os.path.join(p, f"{name}_weight.bin"), N * K // 4).reshape(N, K // 4),
                        _f32(os.path.join(p, f"{name}_scale.bin"), N),
                        _f32(os.path.join(p, f"{name}_bias.bin"), N))

            self.layers.append(dict(
                ln1=(_f32(os.path.join(p, "ln1_gamma.bin"), d), _f32(os.path.join(p, "ln1_beta.bin"), d)),
                ln2=(_f32(os.path.join(p, "ln2_gamma.bin"), d), _f32(os.path.join(p, "ln2_beta.bin"), d)),
                qkv=q("qkv", 3 * d, d), out=q("out", d, d), up=q("ffn_up", ff, d), down=q("ffn_down", d, ff)))
        self.int8_lm_head = int8_lm_head
        self.kv_bf16 = kv_bf16
        if int8_lm_head:
            self.head = orc.quantize(self.wte)
        self.B = batch
        self.nbps = (S + BLOCK - 1) // BLOCK
        P = batch * self.nbps
        self.table = np.arange(P, dtype=np.int32).reshape(batch, self.nbps)
        self.kc = [np.zeros((P, BLOCK, self.H, self.dh), np.float32) for _ in range(L)]
        self.vc = [np.zeros((P, BLOCK, self.H, self.dh), np.float32) for _ in range(L)]
        self.pos = 0

    def step(self, tokens) -> np.ndarray:
        """One decode step for every sequence at position self.pos; returns logits [B, V]."""
        B, d, H, dh = self.B, self.d, self.H, self.dh
        tokens = np.asarray(tokens, dtype=np.int32)
        pos = self.pos
        x = np.concatenate([orc.embedding(tokens[b:b + 1], pos, self.wte, self.wpe) for b in range(B)])
        for li, Lw in enumerate(self.layers):
            xn = orc.layernorm(x, *Lw["ln1"])
            ap, asc = orc.quantize(xn)
            w, s, bias = Lw["qkv"]
            qkv = orc.gemm(ap, w, asc, s, 1, bias)
            Q, K, V = qkv[:, :d], qkv[:, d:2 * d], qkv[:, 2 * d:]
            if self.kv_bf16:  # a bf16 cache stores the nearest bf16 value
                K, V = bf16_round(K), bf16_round(V)
            for b in range(B):
                orc.kv_cache_write(K[b].reshape(1, H, dh), V[b].reshape(1, H, dh), self.kc[li], self.vc[li],
                                   self.table[b], pos, BLOCK)
            lens = np.full(B, pos + 1, dtype=np.int32)
            attn = orc.decode_attn(Q.reshape(B, H, dh), self.kc[li], self.vc[li], self.table, lens,
                                   self.c["max_seq_len"], BLOCK, H).reshape(B, d)
            ap, asc = orc.quantize(attn)
            w, s, bias = Lw["out"]
            x = orc.gemm(ap, w, asc, s, 3, bias, x)
            xn = orc.layernorm(x, *Lw["ln2"])
            ap, asc = orc.quantize(xn)
            w, s, bias = Lw["up"]
            h = orc.gemm(ap, w, asc, s, 2, bias)
            ap, asc = orc.quantize(h)
            w, s, bias = Lw["down"]
            x = orc.gemm(ap, w, asc, s, 3, bias, x)
        xf = orc.layernorm(x, *self.lnf)
        if self.int8_lm_head:
            ap, asc = orc.quantize(xf)
            logits = orc.gemm(ap, self.head[0], asc, self.head[1], 0)
        else:
            logits = np.stack([orc.vocab_proj(xf[b], self.wte) for b in range(B)])
        self.pos += 1
        return logits
