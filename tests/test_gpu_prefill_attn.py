"""GPU parity of the causal prefill attention (ie_prefill_attn over the paged
cache, ie_flash_attn over contiguous [B, H, N, d]) against the CPU oracle.

Causal attention of query t (position start + t) is exactly decode attention
over the first start + t + 1 cached tokens, so the oracle is the pinned fp64
decode-attention restatement evaluated once per query position.  Bar as for
decode attention: max |O_gpu - O_oracle| <= 1e-5 * max |O_oracle| (fp32, and
bf16 KV against the oracle run on the same bf16 values).
"""
import numpy as np
import pytest

from conftest import bf16_bits, make_paged_cache, rng

pytestmark = pytest.mark.gpu
REL = 1e-5


def dev(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    import torch

    torch.cuda.synchronize()
    return t.cpu().numpy()


def rel_err(got, want):
    return np.abs(got - want).max() / max(np.abs(want).max(), 1e-30)


def oracle_prefill(orc, Q, kc, vc, table, start, bs, H_kv, kv_dtype=0, causal=True):
    """Q [B, P, H_q, d] -> O [B, P, H_q, d], one decode-oracle call per position."""
    B, P = Q.shape[:2]
    out = np.empty_like(Q)
    for t in range(P):
        n = start + t + 1 if causal else start + P
        lens = np.full(B, n, dtype=np.int32)
        out[:, t] = orc.decode_attn(Q[:, t], kc, vc, table, lens, n, bs, H_kv, kv_dtype=kv_dtype)
    return out


def case(seed, B, P, start, H_kv, G, d, bs, kvdt):
    r = rng(seed)
    lens = np.full(B, start + P)
    kc, vc, table, _, _ = make_paged_cache(r, B, H_kv, d, lens, bs)
    Q = r.standard_normal((B, P, H_kv * G, d)).astype(np.float32)
    if kvdt:
        kc, vc = bf16_bits(kc), bf16_bits(vc)
    return Q, kc, vc, table


@pytest.mark.parametrize("kvdt", [0, 1])
@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("G", [1, 4])
@pytest.mark.parametrize("start", [0, 37])
def test_prefill_matches_oracle(ie, orc, start, G, d, kvdt):
    """Fresh prompt (start 0) and a chunk continuing a 37-token context; P=50
    leaves a partial last query tile and a partial last KV chunk."""
    B, P, H_kv = 2, 50, 2
    Q, kc, vc, table = case(100 + start + G + d + kvdt, B, P, start, H_kv, G, d, 16, kvdt)
    want = oracle_prefill(orc, Q, kc, vc, table, start, 16, H_kv, kvdt)
    got = host(ie.prefill_attn(dev(Q), dev(kc), dev(vc), dev(table), start, 16, H_kv, kv_dtype=kvdt))
    assert rel_err(got, want) < REL


@pytest.mark.parametrize("bs", [1, 8, 48])
def test_prefill_other_block_sizes(ie, orc, bs):
    B, P, start, H_kv, G, d = 3, 70, 5, 2, 2, 64
    Q, kc, vc, table = case(200 + bs, B, P, start, H_kv, G, d, bs, 0)
    want = oracle_prefill(orc, Q, kc, vc, table, start, bs, H_kv)
    got = host(ie.prefill_attn(dev(Q), dev(kc), dev(vc), dev(table), start, bs, H_kv))
    assert rel_err(got, want) < REL


@pytest.mark.parametrize("B", [4, 16])
def test_prefill_gpt2_prompt(ie, orc, B):
    """The BASELINE prompt shape: 128 tokens, 12 heads of 64, batch 4 and the
    engine's batch 16 (192 (sequence, head) pairs: every tile of a pair on one
    XCD)."""
    P, H, d = 128, 12, 64
    Q, kc, vc, table = case(300 + B, B, P, 0, H, 1, d, 16, 0)
    want = oracle_prefill(orc, Q, kc, vc, table, 0, 16, H)
    got = host(ie.prefill_attn(dev(Q), dev(kc), dev(vc), dev(table), 0, 16, H))
    assert rel_err(got, want) < REL
    # the first query attends to itself only: O = V0 of its head
    V0 = vc[table[:, 0], 0]  # [B, H, d]
    assert np.allclose(got[:, 0], V0, rtol=0, atol=1e-6)


def test_prefill_single_token_equals_decode(ie):
    """P = 1 at position start is one decode query over start + 1 tokens."""
    B, H_kv, G, d, start = 2, 4, 2, 128, 300
    Q, kc, vc, table = case(400, B, 1, start, H_kv, G, d, 16, 0)
    got = host(ie.prefill_attn(dev(Q), dev(kc), dev(vc), dev(table), start, 16, H_kv))
    lens = np.full(B, start + 1, dtype=np.int32)
    dec = host(ie.decode_attn(dev(Q[:, 0]), dev(kc), dev(vc), dev(table), dev(lens), start + 1, 16, H_kv))
    assert rel_err(got[:, 0], dec) < 2 * REL


def test_prefill_deterministic_and_placement_invariant(ie):
    B, P, H_kv, d = 2, 96, 2, 128
    lens = np.full(B, P)
    kc, vc, table, _, _ = make_paged_cache(rng(5), B, H_kv, d, lens, 16, shuffle=True)
    kc2, vc2, table2, _, _ = make_paged_cache(rng(5), B, H_kv, d, lens, 16, shuffle=False)
    Q = rng(6).standard_normal((B, P, 8, d)).astype(np.float32)
    a = host(ie.prefill_attn(dev(Q), dev(kc), dev(vc), dev(table), 0, 16, H_kv))
    b = host(ie.prefill_attn(dev(Q), dev(kc2), dev(vc2), dev(table2), 0, 16, H_kv))
    c = host(ie.prefill_attn(dev(Q), dev(kc), dev(vc), dev(table), 0, 16, H_kv))
    assert np.array_equal(a, b) and np.array_equal(a, c)


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("N", [1, 17, 130])
def test_flash_attn_contiguous(ie, orc, N, d, causal):
    """run_flash_attn_v2's layout [B, H, N, d]; the oracle sees the same data
    as a paged cache with one N-token block per sequence."""
    r = rng(N * 10 + d + causal)
    B, H = 2, 3
    Q = r.standard_normal((B, H, N, d)).astype(np.float32)
    K = r.standard_normal((B, H, N, d)).astype(np.float32)
    V = r.standard_normal((B, H, N, d)).astype(np.float32)
    kc = np.ascontiguousarray(K.transpose(0, 2, 1, 3))  # [B blocks, N, H, d]
    vc = np.ascontiguousarray(V.transpose(0, 2, 1, 3))
    table = np.arange(B, dtype=np.int32).reshape(B, 1)
    want = oracle_prefill(orc, np.ascontiguousarray(Q.transpose(0, 2, 1, 3)), kc, vc, table, 0, N, H,
                          causal=causal).transpose(0, 2, 1, 3)
    got = host(ie.flash_attn(dev(Q), dev(K), dev(V), causal=causal))
    assert rel_err(got, want) < REL


K10_CASES = [(1, 1, 128, 64), (1, 12, 128, 64), (1, 12, 256, 64), (1, 12, 512, 64), (2, 12, 256, 64)]


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("case", K10_CASES)
def test_reference_k10_cases(ie, orc, case, causal):
    """The reference's own FlashAttention tests (tests/test_attention.cu:82-109,
    156-159 and the multi-batch case): srand(42), Q, K, V drawn interleaved per
    element as rand()/RAND_MAX*2-1 in [B, H, N, d], max |O - O_ref| < 1e-5
    (:93, :109); here also within 1e-5 of the output scale."""
    B, H, N, d = case
    u = orc.GlibcRand(42).uniform(3 * B * H * N * d)
    Q = np.ascontiguousarray(u[0::3].reshape(B, H, N, d))
    K = np.ascontiguousarray(u[1::3].reshape(B, H, N, d))
    V = np.ascontiguousarray(u[2::3].reshape(B, H, N, d))
    kc = np.ascontiguousarray(K.transpose(0, 2, 1, 3))
    vc = np.ascontiguousarray(V.transpose(0, 2, 1, 3))
    table = np.arange(B, dtype=np.int32).reshape(B, 1)
    want = oracle_prefill(orc, np.ascontiguousarray(Q.transpose(0, 2, 1, 3)), kc, vc, table, 0, N, H,
                          causal=causal).transpose(0, 2, 1, 3)
    got = host(ie.flash_attn(dev(Q), dev(K), dev(V), causal=causal))
    assert np.abs(got - want).max() < 1e-5
    assert rel_err(got, want) < REL


K12_CASES = [(1, 8, 8, 128), (1, 8, 4, 128), (1, 8, 2, 128), (1, 16, 4, 256), (1, 8, 1, 128), (2, 8, 4, 128)]


@pytest.mark.parametrize("case", K12_CASES)
def test_reference_gqa_paged_cases(ie, orc, case):
    """The reference's paged GQA prefill tests (tests/test_paged_attention.cu:
    184-284, causal cases): srand(42), Q [B, H_q, N, d] drawn first, then K and V
    [B, H_kv, N, d] interleaved per element, block size 16, identity block table,
    max |O - O_ref| < 1e-5.  Q and O are token-major here (transposed)."""
    B, H_q, H_kv, N = case
    d, bs = 64, 16
    g = orc.GlibcRand(42)
    Qh = g.uniform(B * H_q * N * d).reshape(B, H_q, N, d)
    K, V = g.uniform_pair(B * H_kv * N * d)
    K = K.reshape(B, H_kv, N, d)
    V = V.reshape(B, H_kv, N, d)
    nbps = (N + bs - 1) // bs
    kc = np.zeros((B * nbps, bs, H_kv, d), np.float32)
    vc = np.zeros_like(kc)
    for b in range(B):
        for t in range(N):
            kc[b * nbps + t // bs, t % bs] = K[b, :, t]
            vc[b * nbps + t // bs, t % bs] = V[b, :, t]
    table = np.arange(B * nbps, dtype=np.int32).reshape(B, nbps)
    Q = np.ascontiguousarray(Qh.transpose(0, 2, 1, 3))  # [B, N, H_q, d]
    want = oracle_prefill(orc, Q, kc, vc, table, 0, bs, H_kv)
    got = host(ie.prefill_attn(dev(Q), dev(kc), dev(vc), dev(table), 0, bs, H_kv))
    assert np.abs(got - want).max() < 1e-5
    assert rel_err(got, want) < REL
