"""GPU parity of split-K paged decode attention against the CPU oracle.

Bar (fp32 KV): max |O_gpu - O_oracle| <= 1e-5 * max |O_oracle| (relative to the
output scale), and on the reference's own six cases also its absolute bound
max |diff| < 1e-5 (tests/test_decode_attention.cu:49,132).  bf16 KV is held to
the same bar against the oracle run on the same bf16 values (only the
accumulation differs), and its distance to the fp32-input result is reported.
"""
import numpy as np
import pytest

from conftest import bf16_bits, bf16_to_f32, make_paged_cache, rng
from test_oracle_attn_support import REF_CASES, glibc_reference_case

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


def run_gpu(ie, Q, kc, vc, table, lens, max_ctx, bs, H_kv, kv_dtype=0, splits=0):
    return host(ie.decode_attn(dev(Q), dev(kc), dev(vc), dev(table), dev(lens.astype(np.int32)),
                               max_ctx, bs, H_kv, kv_dtype=kv_dtype, splits=splits))


@pytest.mark.parametrize("case", REF_CASES)
def test_reference_cases(ie, orc, case):
    B, H_q, H_kv, ctx, d, bs = case
    Q, kc, vc, table, lens, Ks, Vs = glibc_reference_case(orc, *case)
    want = orc.decode_attn(Q, kc, vc, table, lens, ctx, bs, H_kv)
    got = run_gpu(ie, Q, kc, vc, table, lens, ctx, bs, H_kv)
    assert np.abs(got - want).max() < 1e-5
    assert rel_err(got, want) < REL


def test_cfg3_mha_shuffled(ie, orc):
    # B=8, H=12, d=64, ctx=1024, block 16, shuffled physical blocks, N(0,1)
    r = rng(3)
    B, H, d, ctx = 8, 12, 64, 1024
    lens = np.full(B, ctx)
    kc, vc, table, _, _ = make_paged_cache(r, B, H, d, lens, 16)
    Q = r.standard_normal((B, H, d)).astype(np.float32)
    want = orc.decode_attn(Q, kc, vc, table, lens, ctx, 16, H)
    got = run_gpu(ie, Q, kc, vc, table, lens, ctx, 16, H)
    assert rel_err(got, want) < REL


@pytest.mark.parametrize("ctx", [4096, 8192])
@pytest.mark.parametrize("kvdt", [0, 1])
def test_cfg4_gqa_variable_lengths(ie, orc, ctx, kvdt):
    # B=32, Hq=32, Hkv=8, d=128, lengths ~U[ctx/2, ctx], shuffled table
    r = rng(ctx + kvdt)
    B, H_q, H_kv, d = 32, 32, 8, 128
    lens = r.integers(ctx // 2, ctx + 1, B)
    kc, vc, table, _, _ = make_paged_cache(r, B, H_kv, d, lens, 16)
    Q = r.standard_normal((B, H_q, d)).astype(np.float32)
    if kvdt:
        kc, vc = bf16_bits(kc), bf16_bits(vc)
    max_ctx = int(lens.max())
    want = orc.decode_attn(Q, kc, vc, table, lens, max_ctx, 16, H_kv, kv_dtype=kvdt)
    got = run_gpu(ie, Q, kc, vc, table, lens, max_ctx, 16, H_kv, kv_dtype=kvdt)
    assert rel_err(got, want) < REL


def test_ctx32768_subset(ie, orc):
    r = rng(32768)
    B, H_q, H_kv, d, ctx = 4, 32, 8, 128, 32768
    lens = r.integers(ctx // 2, ctx + 1, B)
    lens[0] = ctx
    kc, vc, table, _, _ = make_paged_cache(r, B, H_kv, d, lens, 16)
    Q = r.standard_normal((B, H_q, d)).astype(np.float32)
    for kvdt in (0, 1):
        k, v = (kc, vc) if kvdt == 0 else (bf16_bits(kc), bf16_bits(vc))
        want = orc.decode_attn(Q, k, v, table, lens, ctx, 16, H_kv, kv_dtype=kvdt)
        got = run_gpu(ie, Q, k, v, table, lens, ctx, 16, H_kv, kv_dtype=kvdt)
        assert rel_err(got, want) < REL
        got64 = run_gpu(ie, Q, k, v, table, lens, ctx, 16, H_kv, kv_dtype=kvdt, splits=64)
        assert rel_err(got64, want) < REL


@pytest.mark.parametrize("kvdt", [0, 1])
def test_cfg4_ctx32768_full_batch(ie, orc, kvdt):
    """BASELINE configs[3] at ctx 32768 and its full batch: B = 32, Hq 32 /
    Hkv 8, d 128, lengths U[16384, 32768], shuffled block table, fp32 and
    bf16 KV (~6.4 GB of fp32 K+V).  The cache is drawn on the device and
    copied to the host for the full oracle; the reference split rule (16
    splits) and a 64-split plan."""
    import torch

    r = rng(32768 + 10 * kvdt)
    B, H_q, H_kv, d, ctx, bs = 32, 32, 8, 128, 32768, 16
    lens = r.integers(ctx // 2, ctx + 1, B)
    lens[3] = ctx
    nbs = (lens + bs - 1) // bs
    P, nbps = int(nbs.sum()), int(nbs.max())
    perm = r.permutation(P).astype(np.int32)
    table = np.zeros((B, nbps), np.int32)
    off = 0
    for b in range(B):
        table[b, :nbs[b]] = perm[off:off + nbs[b]]
        off += int(nbs[b])
    g = torch.Generator(device="cuda").manual_seed(int(r.integers(1 << 30)))
    kc = torch.randn((P, bs, H_kv, d), device="cuda", generator=g)
    vc = torch.randn((P, bs, H_kv, d), device="cuda", generator=g)
    if kvdt:
        kc = kc.to(torch.bfloat16).view(torch.int16)
        vc = vc.to(torch.bfloat16).view(torch.int16)
    Q = r.standard_normal((B, H_q, d)).astype(np.float32)
    kh = kc.cpu().numpy().view(np.uint16) if kvdt else kc.cpu().numpy()
    vh = vc.cpu().numpy().view(np.uint16) if kvdt else vc.cpu().numpy()
    want = orc.decode_attn(Q, kh, vh, table, lens, ctx, bs, H_kv, kv_dtype=kvdt)
    del kh, vh
    for splits in (0, 64):
        got = host(ie.decode_attn(dev(Q), kc, vc, dev(table), dev(lens.astype(np.int32)), ctx, bs, H_kv,
                                  kv_dtype=kvdt, splits=splits))
        assert rel_err(got, want) < REL, splits


def test_bf16_vs_fp32_inputs_stated_bound(ie, orc):
    r = rng(77)
    B, H_q, H_kv, d, ctx = 4, 32, 8, 128, 2048
    lens = r.integers(ctx // 2, ctx + 1, B)
    lens[0] = ctx
    kc, vc, table, _, _ = make_paged_cache(r, B, H_kv, d, lens, 16)
    Q = r.standard_normal((B, H_q, d)).astype(np.float32)
    want32 = orc.decode_attn(Q, kc, vc, table, lens, ctx, 16, H_kv)
    got = run_gpu(ie, Q, bf16_bits(kc), bf16_bits(vc), table, lens, ctx, 16, H_kv, kv_dtype=1)
    # bf16 keeps 8 significant bits: stated bound 1e-2 of the output scale
    assert rel_err(got, want32) < 1e-2


@pytest.mark.parametrize("ctx", [385, 400, 449, 480, 513, 560, 993, 1008])
def test_engine_shapes_where_reference_reads_stale_splits(ie, orc, ctx):
    """Lengths at which the reference's pass 1 leaves split slots unwritten."""
    r = rng(ctx)
    H, d = 12, 64
    lens = np.array([ctx])
    kc, vc, table, _, _ = make_paged_cache(r, 1, H, d, lens, 16)
    Q = r.standard_normal((1, H, d)).astype(np.float32)
    want = orc.decode_attn(Q, kc, vc, table, lens, ctx, 16, H)
    got = run_gpu(ie, Q, kc, vc, table, lens, ctx, 16, H)
    assert rel_err(got, want) < REL


@pytest.mark.parametrize("bs", [1, 8, 32, 48])
@pytest.mark.parametrize("G", [1, 2, 4, 8])
def test_block_sizes_and_groups(ie, orc, bs, G):
    r = rng(bs * 10 + G)
    B, H_kv, d = 3, 2, 64 if G < 4 else 128
    H_q = H_kv * G
    lens = np.array([300, 17, 251])
    kc, vc, table, _, _ = make_paged_cache(r, B, H_kv, d, lens, bs)
    Q = r.standard_normal((B, H_q, d)).astype(np.float32)
    want = orc.decode_attn(Q, kc, vc, table, lens, 300, bs, H_kv)
    got = run_gpu(ie, Q, kc, vc, table, lens, 300, bs, H_kv)
    assert rel_err(got, want) < REL


@pytest.mark.parametrize("splits", [1, 7, 64, 256])
def test_explicit_split_counts(ie, orc, splits):
    r = rng(splits)
    B, H_q, H_kv, d = 2, 16, 4, 128
    lens = np.array([4000, 1500])
    kc, vc, table, _, _ = make_paged_cache(r, B, H_kv, d, lens, 16)
    Q = r.standard_normal((B, H_q, d)).astype(np.float32)
    want = orc.decode_attn(Q, kc, vc, table, lens, 4000, 16, H_kv)
    got = run_gpu(ie, Q, kc, vc, table, lens, 4000, 16, H_kv, splits=splits)
    assert rel_err(got, want) < REL


@pytest.mark.parametrize("kvdt", [0, 1])
@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("G", [1, 2, 4, 8])
def test_one_wave_and_four_wave_splits(ie, orc, G, d, kvdt):
    """Splits of >= 256 tokens run on one wave each, shorter ones on several
    waves that merge in LDS: both layouts for every head width, group size and
    KV type (max_context_len 700: 1 and 2 splits are one-wave, 3 and 11 are
    multi-wave; with these few (b, head, split) units, eight waves per split
    for G <= 4, four for G = 8)."""
    r = rng(1000 + 10 * G + d + kvdt)
    B, H_kv = 2, 2
    H_q = H_kv * G
    lens = np.array([700, 300])
    kc, vc, table, _, _ = make_paged_cache(r, B, H_kv, d, lens, 16)
    Q = r.standard_normal((B, H_q, d)).astype(np.float32)
    if kvdt:
        kc, vc = bf16_bits(kc), bf16_bits(vc)
    want = orc.decode_attn(Q, kc, vc, table, lens, 700, 16, H_kv, kv_dtype=kvdt)
    for splits in (1, 2, 3, 11):
        got = run_gpu(ie, Q, kc, vc, table, lens, 700, 16, H_kv, kv_dtype=kvdt, splits=splits)
        assert rel_err(got, want) < REL, splits


@pytest.mark.parametrize("kvdt", [0, 1])
@pytest.mark.parametrize("G", [1, 4])
def test_four_wave_splits_with_many_units(ie, orc, G, kvdt):
    """More than 64 (kv head, split) units per sequence of short splits
    (under 256 tokens each): four waves per split (8 KV heads x 11 splits =
    88 units); with 3 splits (24 units) eight waves.  The wave count depends
    on the sequence's units only, so the batch does not change it."""
    r = rng(1100 + G + kvdt)
    B, H_kv, d = 8, 8, 64
    lens = r.integers(100, 701, B)
    kc, vc, table, _, _ = make_paged_cache(r, B, H_kv, d, lens, 16)
    Q = r.standard_normal((B, H_kv * G, d)).astype(np.float32)
    if kvdt:
        kc, vc = bf16_bits(kc), bf16_bits(vc)
    mx = int(lens.max())
    want = orc.decode_attn(Q, kc, vc, table, lens, mx, 16, H_kv, kv_dtype=kvdt)
    for splits in (11, 3):
        got = run_gpu(ie, Q, kc, vc, table, lens, mx, 16, H_kv, kv_dtype=kvdt, splits=splits)
        assert rel_err(got, want) < REL, splits
        # each sequence alone gives the same bits as inside the batch
        for b in (0, 5):
            one = run_gpu(ie, Q[b:b + 1], kc, vc, table[b:b + 1], lens[b:b + 1], mx, 16, H_kv, kv_dtype=kvdt,
                          splits=splits)
            assert np.array_equal(one[0], got[b]), (splits, b)


def test_edges(ie, orc):
    r = rng(8)
    B, H, d = 3, 4, 64
    lens = np.array([1, 0, 40])
    kc, vc, table, Ks, Vs = make_paged_cache(r, B, H, d, lens, 16)
    Q = r.standard_normal((B, H, d)).astype(np.float32)
    got = run_gpu(ie, Q, kc, vc, table, lens, 40, 16, H)
    assert np.allclose(got[0], Vs[0][0], rtol=0, atol=1e-6)   # one token: O = V0
    assert np.all(got[1] == 0)                                   # empty sequence
    want = orc.decode_attn(Q, kc, vc, table, lens, 40, 16, H)
    assert rel_err(got[2], want[2]) < REL
    # all sequences empty, max_context_len 0
    got = run_gpu(ie, Q, kc, vc, table, np.zeros(B, np.int64), 0, 16, H)
    assert np.all(got == 0)


@pytest.mark.parametrize("d,G,kv_dtype", [(64, 1, 0), (128, 4, 0), (128, 4, 1), (128, 8, 0)])
def test_empty_table_rows(ie, d, G, kv_dtype):
    """max_context_len 0 with num_blocks_per_seq 0: a table of zero columns.
    No walk may read a table entry (every row is empty); the output is 0."""
    import torch

    B, H_kv = 5, 2
    H_q = H_kv * G
    Q = dev(rng(9).standard_normal((B, H_q, d)).astype(np.float32))
    cache = torch.zeros(16 * H_kv * d, dtype=torch.float32, device="cuda")  # one block, never read
    table = torch.zeros(1, dtype=torch.int32, device="cuda")  # a real pointer; the rows have 0 columns
    lens = torch.zeros(B, dtype=torch.int32, device="cuda")
    for splits in (0, 1, 7):
        out = torch.full_like(Q, float("nan"))
        S = ie.num_splits(0, 16, splits)
        ws = torch.empty(ie.workspace_bytes(B, H_q, d, S) // 4, device="cuda")
        P = ie._ptr
        ie.check("ie_decode_attn", B, H_q, H_kv, d, P(Q), P(cache), P(cache), kv_dtype, P(table), P(lens), 0, 16,
                 0, P(out), P(ws), ws.numel() * 4, splits, ie._stream())
        assert np.all(host(out) == 0)


def test_placement_invariance_bit_identical(ie):
    B, H_q, H_kv, d = 3, 16, 4, 128
    lens = np.array([900, 321, 1024])
    kc, vc, table, _, _ = make_paged_cache(rng(1), B, H_kv, d, lens, 16, shuffle=True)
    kc2, vc2, table2, _, _ = make_paged_cache(rng(1), B, H_kv, d, lens, 16, shuffle=False)
    Q = rng(2).standard_normal((B, H_q, d)).astype(np.float32)
    a = run_gpu(ie, Q, kc, vc, table, lens, 1024, 16, H_kv)
    b = run_gpu(ie, Q, kc2, vc2, table2, lens, 1024, 16, H_kv)
    assert np.array_equal(a, b)
    c = run_gpu(ie, Q, kc, vc, table, lens, 1024, 16, H_kv)
    assert np.array_equal(a, c)  # deterministic


def test_reference_sized_workspace(ie, orc):
    """The drop-in call shape: workspace of exactly [B, H_q, 16, d+2] floats."""
    import torch

    r = rng(10)
    B, H, d, ctx = 2, 12, 64, 1024
    lens = np.full(B, ctx)
    kc, vc, table, _, _ = make_paged_cache(r, B, H, d, lens, 16)
    Q = r.standard_normal((B, H, d)).astype(np.float32)
    ws = torch.empty(B * H * 16 * (d + 2), dtype=torch.float32, device="cuda")
    got = host(ie.decode_attn(dev(Q), dev(kc), dev(vc), dev(table), dev(lens.astype(np.int32)),
                              ctx, 16, H, workspace=ws))
    want = orc.decode_attn(Q, kc, vc, table, lens, ctx, 16, H)
    assert rel_err(got, want) < REL


@pytest.mark.parametrize("bs", [16, 8])
@pytest.mark.parametrize("kvdt", [0, 1])
@pytest.mark.parametrize("d,G", [(64, 1), (128, 4), (128, 8)])
def test_balanced_partition_ragged_lengths(ie, orc, d, G, kvdt, bs):
    """Launches with many long one-wave splits cut the batch's chunks into
    equal workgroup ranges across sequence boundaries.  Ragged lengths from 0
    to max, more than 64 sequences (two scan groups), 8 split slots.  bf16,
    d = 128, G >= 4 with block size 16 runs the bf16 MFMA walk."""
    r = rng(2000 + d + G + kvdt + bs)
    B, H_kv = 70, 2
    H_q = H_kv * G
    lens = r.integers(0, 2049, B)
    lens[[3, 40]] = 0
    lens[[5, 66]] = 2048
    kc, vc, table, _, _ = make_paged_cache(r, B, H_kv, d, lens, bs)
    Q = r.standard_normal((B, H_q, d)).astype(np.float32)
    if kvdt:
        kc, vc = bf16_bits(kc), bf16_bits(vc)
    want = orc.decode_attn(Q, kc, vc, table, lens, 2048, bs, H_kv, kv_dtype=kvdt)
    got = run_gpu(ie, Q, kc, vc, table, lens, 2048, bs, H_kv, kv_dtype=kvdt, splits=8)
    assert rel_err(got, want) < REL
    assert np.all(got[[3, 40]] == 0)


def test_balanced_partition_two_slots_and_invariance(ie, orc):
    """Two split slots (each sequence meets at most two workgroups), 300
    sequences; the partition depends on the lengths only, so block placement
    does not change the bits."""
    B, H_kv, G, d = 300, 2, 2, 64
    lens = rng(7).integers(0, 1025, B)
    kc, vc, table, _, _ = make_paged_cache(rng(8), B, H_kv, d, lens, 16, shuffle=True)
    kc2, vc2, table2, _, _ = make_paged_cache(rng(8), B, H_kv, d, lens, 16, shuffle=False)
    Q = rng(9).standard_normal((B, H_kv * G, d)).astype(np.float32)
    want = orc.decode_attn(Q, kc, vc, table, lens, 1024, 16, H_kv)
    a = run_gpu(ie, Q, kc, vc, table, lens, 1024, 16, H_kv, splits=2)
    b = run_gpu(ie, Q, kc2, vc2, table2, lens, 1024, 16, H_kv, splits=2)
    assert rel_err(a, want) < REL
    assert np.array_equal(a, b)


@pytest.mark.parametrize("kvdt", [0, 1])
@pytest.mark.parametrize("H_kv,d,G", [(4, 128, 1), (12, 64, 1), (4, 128, 4)])
def test_streamed_cache_loads_same_bits(ie, orc, H_kv, d, G, kvdt):
    """Launches whose cache reads (batch x plan context x heads x d x 2 x
    element size) pass 32 MiB load the cache with non-temporal loads in the
    multi-wave split layouts: eight waves per split at <= 64 (kv head, split)
    units per sequence (H_kv 4, 16 splits), four above (H_kv 12).  32
    sequences of 1024 tokens pass the threshold, one alone does not; the
    cache policy changes no arithmetic, so each sequence gets the same bits
    either way."""
    r = rng(3000 + H_kv + d + G + kvdt)
    B, ctx = 32, 1024
    H_q = H_kv * G
    lens = np.full(B, ctx)
    lens[7] = 999
    kc, vc, table, _, _ = make_paged_cache(r, B, H_kv, d, lens, 16)
    Q = r.standard_normal((B, H_q, d)).astype(np.float32)
    if kvdt:
        kc, vc = bf16_bits(kc), bf16_bits(vc)
    esz = 2 if kvdt else 4
    assert B * ctx * H_kv * d * 2 * esz > 32 << 20 > ctx * H_kv * d * 2 * esz
    want = orc.decode_attn(Q, kc, vc, table, lens, ctx, 16, H_kv, kv_dtype=kvdt)
    got = run_gpu(ie, Q, kc, vc, table, lens, ctx, 16, H_kv, kv_dtype=kvdt, splits=16)
    assert rel_err(got, want) < REL
    for b in (0, 7, 31):
        one = run_gpu(ie, Q[b:b + 1], kc, vc, table[b:b + 1], lens[b:b + 1], ctx, 16, H_kv, kv_dtype=kvdt,
                      splits=16)
        assert np.array_equal(one[0], got[b]), b
