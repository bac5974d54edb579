"""GPU: the device top-k selection (ie_topk) against the oracle, bit for bit,
the reference-signature sampler (sample_top_k / sample_argmax of ie_compat.h)
and sampled generation through the engine against the oracle's sampler on
the engine's own logits (seeds 42, 43, ... as src/gpt2_engine.cu:707-747)."""
import ctypes

import numpy as np
import pytest

from conftest import rng

pytestmark = pytest.mark.gpu


def run_topk(ie, rows_np, k):
    import torch

    t = torch.from_numpy(np.ascontiguousarray(rows_np, dtype=np.float32)).cuda()
    v, i = ie.topk(t, k)
    torch.cuda.synchronize()
    return v.cpu().numpy(), i.cpu().numpy()


def check(ie, orc, rows_np, k):
    v, i = run_topk(ie, rows_np, k)
    wv, wi = orc.topk(rows_np, k)
    assert np.array_equal(i, wi)
    assert np.array_equal(v, wv)


@pytest.mark.parametrize("k", [1, 40, 50, 1024])
@pytest.mark.parametrize("rows", [1, 3, 16])
def test_topk_gpt2_rows(ie, orc, rows, k):
    """GPT-2-sized rows in the range its logits take (all negative, one exponent)."""
    x = (rng(rows * 7 + k).standard_normal((rows, 50257)) * 3 - 80).astype(np.float32)
    check(ie, orc, x, k)


@pytest.mark.parametrize("n,k", [(1, 1), (2, 2), (3, 1), (5, 3), (7, 7), (100, 100), (1023, 17), (8193, 1000),
                                 (65533, 40), (65534, 40), (70001, 333)])
def test_topk_shapes(ie, orc, n, k):
    """Three rows, so rows 1 and 2 start inside a 16-byte chunk when n is not
    a multiple of 4 (n <= 5: no whole chunk at all); 65533 is the longest row
    held in registers, 65534 the shortest streamed one."""
    x = rng(n + k).standard_normal((3, n)).astype(np.float32)
    check(ie, orc, x, k)


@pytest.mark.parametrize("n", [20000, 70001])
@pytest.mark.parametrize("levels", [1, 2, 5, 300])
def test_topk_ties_take_lower_indices(ie, orc, levels, n):
    """Few distinct values: the k-th value is shared, and the lowest-index
    copies are the ones kept (levels = 1: an all-equal row).  Rows up to
    65536 are held in registers, longer ones streamed."""
    x = rng(levels + n).integers(0, levels, (3, n)).astype(np.float32)
    for k in (1, 40, 1024):
        check(ie, orc, x, k)


def test_topk_infinities_and_signed_zeros(ie, orc):
    r = rng(11)
    x = r.standard_normal((2, 5000)).astype(np.float32)
    x[0, r.integers(0, 5000, 4000)] = -np.inf
    x[1, :2500] = np.float32(0.0)
    x[1, 2500:] = np.float32(-0.0)
    x[1, 4999] = np.float32(1.0)
    check(ie, orc, x, 50)
    check(ie, orc, x, 1024)
    x[0, :] = -np.inf
    check(ie, orc, x, 7)


def test_topk_rejects_bad_k(ie):
    import torch

    t = torch.zeros((1, 10), device="cuda")
    for k in (0, 11):
        with pytest.raises(ie.IeError):
            ie.topk(t, k)
    t = torch.zeros((1, 5000), device="cuda")
    with pytest.raises(ie.IeError):
        ie.topk(t, 1025)


def fresh_seed_state(ie):
    """The draw reseeds only on a seed change (the reference's static
    last_seed): one draw with an unused seed makes the next seed a change."""
    ie.top_k_draw(np.zeros(1, np.float32), np.zeros(1, np.int32), 1.0, 987654321)


def compat_fns(ie):
    lib = ie.load()
    top_k = getattr(lib, "_Z12sample_top_kPKfiifj")
    top_k.restype = ctypes.c_int
    top_k.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_float, ctypes.c_uint]
    amax = getattr(lib, "_Z13sample_argmaxPKfi")
    amax.restype = ctypes.c_int
    amax.argtypes = [ctypes.c_void_p, ctypes.c_int]
    return top_k, amax


def test_compat_samplers_match_oracle(ie, orc):
    """sample_top_k(d_logits, V, k, T, seed) with a new seed per call, as the
    reference's generate loop calls it, and sample_argmax."""
    import torch

    top_k, amax = compat_fns(ie)
    fresh_seed_state(ie)
    r = rng(21)
    for case in range(12):
        V = int(r.choice([50257, 1000, 64]))
        k = int(r.choice([1, 40, 50, 100]))
        T = float(r.choice([0.8, 1.0, 0.5]))
        row = (r.standard_normal(V) * 2).astype(np.float32)
        d = torch.from_numpy(row).cuda()
        seed = 42 + case
        got = top_k(ctypes.c_void_p(d.data_ptr()), V, k, T, seed)
        assert got == orc.sample_top_k(row, k, T, seed), case
        assert amax(ctypes.c_void_p(d.data_ptr()), V) == orc.argmax(row)
    # k above the device limit: the whole row to the host, as the reference
    for case, (V, k) in enumerate([(50257, 2000), (3001, 3001), (1500, 5000)]):
        row = (r.standard_normal(V) * 2).astype(np.float32)
        d = torch.from_numpy(row).cuda()
        seed = 100 + case
        got = top_k(ctypes.c_void_p(d.data_ptr()), V, k, 1.3, seed)
        assert got == orc.sample_top_k(row, min(k, V), 1.3, seed), (V, k)


def test_engine_sampled_generation_matches_oracle_sampler(ie, orc):
    """generate(greedy = false) against a replay: the same engine's prefill and
    step logits, each sampled by the oracle with seeds 42, 43, ..."""
    cfg = dict(n_layers=2, n_heads=2, d_model=128, d_ff=512, vocab_size=3001, max_seq_len=128)
    prompt = rng(3).integers(0, 3001, 9).tolist()
    T, K, N = 0.8, 40, 24
    eng = ie.Engine(seed=5, **cfg)
    fresh_seed_state(ie)
    try:
        got, m = eng.generate_one(prompt, N, temperature=T, top_k=K, greedy=False)
        assert m["tokens_generated"] == len(got)
        eng.reset()
        logits = eng.prefill(np.array([prompt]))
        want = []
        seed = 42
        tok = orc.sample_top_k(logits[0], K, T, seed)
        while len(want) < N and tok != 50256:
            want.append(tok)
            if len(want) == N:
                break
            logits = eng.step(np.array([tok]))
            seed += 1
            tok = orc.sample_top_k(logits[0], K, T, seed)
    finally:
        eng.close()
    assert got == want
    assert len(set(got)) > 1  # sampling, not a repeated argmax


def test_engine_sampling_with_k_above_device_limit(ie, orc):
    """k = 2000 > IE_TOPK_MAX takes the whole-row host route with the same
    order and draw."""
    cfg = dict(n_layers=1, n_heads=1, d_model=64, d_ff=256, vocab_size=2500, max_seq_len=64)
    prompt = [1, 2, 3]
    eng = ie.Engine(seed=9, **cfg)
    fresh_seed_state(ie)
    try:
        got, _ = eng.generate_one(prompt, 6, temperature=1.3, top_k=2000, greedy=False)
        eng.reset()
        logits = eng.prefill(np.array([prompt]))
        want, seed = [], 42
        tok = orc.sample_top_k(logits[0], 2000, 1.3, seed)
        while len(want) < 6:
            want.append(tok)
            if len(want) == 6:
                break
            logits = eng.step(np.array([tok]))
            seed += 1
            tok = orc.sample_top_k(logits[0], 2000, 1.3, seed)
    finally:
        eng.close()
    assert got == want
