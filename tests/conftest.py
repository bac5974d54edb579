"""Shared pytest setup.

Markers: `gpu` tests need an MI355X and call the HIP library through its C ABI;
everything else runs on the CPU (oracle pins, boundary validation, host logic).
"""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "cuda-llm-inference-engine_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def orc():
    from oracle import orc as m

    m.load()
    return m


@pytest.fixture(scope="session")
def ie():
    import ie_amd

    ie_amd.load()
    return ie_amd


@pytest.fixture(scope="session")
def dev():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("gpu test selected but no GPU is visible")
    return torch.device("cuda:0")


def rng(seed: int) -> np.random.Generator:
    return np.random.default_rng(seed)


def unpack_i8(packed: np.ndarray) -> np.ndarray:
    """int32 words [R, K/4] -> int8 [R, K], byte k%4 of word k/4 (little-endian)."""
    return np.ascontiguousarray(packed).view(np.int8).reshape(packed.shape[0], -1)


def pack_i8(q: np.ndarray) -> np.ndarray:
    """int8 [R, K] -> int32 words [R, K/4] (little-endian byte order)."""
    q = np.ascontiguousarray(q, dtype=np.int8)
    return q.view(np.int32).reshape(q.shape[0], -1).copy()


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """fp32 -> bfloat16 bit patterns, round to nearest even (via torch)."""
    import torch

    t = torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(torch.bfloat16)
    return t.view(torch.int16).numpy().view(np.uint16)


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (bits.astype(np.uint32) << 16).view(np.float32)


def make_paged_cache(rng_, B, H_kv, d, ctx_lens, bs, shuffle=True, dtype=np.float32,
                     spare_blocks=3, fill=None):
    """Random K/V per sequence laid out in a paged cache [P, bs, H_kv, d].

    Returns (k_cache, v_cache, block_table [B, nbps], K_seq, V_seq) where
    K_seq[b] is the logical [ctx_b, H_kv, d] data.  Unused slots hold NaN so a
    kernel that reads past a sequence's end is caught.
    """
    ctx_lens = np.asarray(ctx_lens, dtype=np.int64)
    nbs = (ctx_lens + bs - 1) // bs
    nbps = int(max(1, nbs.max()))
    P = int(nbs.sum()) + spare_blocks
    Ks, Vs = [], []
    for b in range(B):
        c = int(ctx_lens[b])
        if fill is None:
            Kb = rng_.standard_normal((c, H_kv, d), dtype=np.float32)
            Vb = rng_.standard_normal((c, H_kv, d), dtype=np.float32)
        else:
            Kb, Vb = fill(b, c)
        Ks.append(Kb)
        Vs.append(Vb)
    # placement is drawn after the data, so shuffle=False/True share the data
    perm = rng_.permutation(P) if shuffle else np.arange(P)
    k_cache = np.full((P, bs, H_kv, d), np.nan, dtype=np.float32)
    v_cache = np.full((P, bs, H_kv, d), np.nan, dtype=np.float32)
    table = np.full((B, nbps), -1, dtype=np.int32)
    nxt = 0
    for b in range(B):
        c = int(ctx_lens[b])
        Kb, Vb = Ks[b], Vs[b]
        for blk in range(int(nbs[b])):
            phys = int(perm[nxt])
            nxt += 1
            table[b, blk] = phys
            lo, hi = blk * bs, min(c, (blk + 1) * bs)
            k_cache[phys, : hi - lo] = Kb[lo:hi]
            v_cache[phys, : hi - lo] = Vb[lo:hi]
    # table entries past a sequence's blocks point at block 0 (valid memory)
    table[table < 0] = 0
    return k_cache, v_cache, table, Ks, Vs
