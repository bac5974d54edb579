"""GPU parity of the paged KV writes and the decode-step support ops."""
import numpy as np
import pytest

from conftest import bf16_bits, rng

pytestmark = pytest.mark.gpu


def dev(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    import torch

    torch.cuda.synchronize()
    return t.cpu().numpy()


@pytest.mark.parametrize("seq,start,bs", [(1, 0, 16), (1, 37, 16), (128, 0, 16), (20, 13, 8), (5, 1020, 16)])
def test_kv_write_fp32_exact(ie, orc, seq, start, bs):
    import torch

    r = rng(seq + start)
    H, dh = 12, 64
    P = (start + seq + bs - 1) // bs + 4
    table = r.permutation(P).astype(np.int32)
    K = r.standard_normal((seq, H, dh)).astype(np.float32)
    V = r.standard_normal((seq, H, dh)).astype(np.float32)
    kc = np.zeros((P, bs, H, dh), np.float32)
    vc = np.zeros_like(kc)
    kd, vd = dev(kc), dev(vc)
    ie.kv_cache_write(dev(K), dev(V), kd, vd, dev(table), start, bs)
    orc.kv_cache_write(K, V, kc, vc, table, start, bs)
    assert np.array_equal(host(kd), kc) and np.array_equal(host(vd), vc)


def test_kv_write_bf16_rounding(ie):
    import torch

    r = rng(3)
    seq, H, dh, bs = 40, 8, 128, 16
    table = np.arange(4, dtype=np.int32)[::-1].copy()
    K = (r.standard_normal((seq, H, dh)) * 10).astype(np.float32)
    V = r.standard_normal((seq, H, dh)).astype(np.float32)
    K[0, 0, :4] = [np.inf, -np.inf, 0.0, -0.0]
    kd = torch.zeros((4, bs, H, dh), dtype=torch.int16, device="cuda")
    vd = torch.zeros_like(kd)
    ie.kv_cache_write(dev(K), dev(V), kd, vd, dev(table), 0, bs, kv_dtype=ie.KV_BF16)
    got = host(kd).view(np.uint16)
    pos = np.arange(seq)
    assert np.array_equal(got[table[pos // bs], pos % bs], bf16_bits(K))  # torch RNE conversion
    assert np.array_equal(host(vd).view(np.uint16)[table[pos // bs], pos % bs], bf16_bits(V))


def test_kv_append_batch(ie):
    r = rng(4)
    B, H, dh, bs, nbps = 5, 12, 64, 16, 8
    P = B * nbps
    table = r.permutation(P).astype(np.int32).reshape(B, nbps)
    positions = np.array([0, 15, 16, 100, 127], dtype=np.int32)
    K = r.standard_normal((B, H, dh)).astype(np.float32)
    V = r.standard_normal((B, H, dh)).astype(np.float32)
    kd = dev(np.zeros((P, bs, H, dh), np.float32))
    vd = dev(np.zeros((P, bs, H, dh), np.float32))
    ie.kv_cache_append_batch(dev(K), dev(V), kd, vd, dev(table), dev(positions), bs)
    kc, vc = host(kd), host(vd)
    for b in range(B):
        p = positions[b]
        assert np.array_equal(kc[table[b, p // bs], p % bs], K[b])
        assert np.array_equal(vc[table[b, p // bs], p % bs], V[b])
    assert np.count_nonzero(kc) == np.count_nonzero(K)


@pytest.mark.parametrize("rows,cols", [(1, 768), (16, 768), (3, 3072), (2, 100)])
def test_layernorm(ie, orc, rows, cols):
    r = rng(rows + cols)
    x = (r.standard_normal((rows, cols)) * 3 + 1).astype(np.float32)
    g = r.standard_normal(cols).astype(np.float32)
    b = r.standard_normal(cols).astype(np.float32)
    want = orc.layernorm(x, g, b)
    got = host(ie.layernorm(dev(x), dev(g), dev(b)))
    assert np.abs(got - want).max() < 2e-5 * max(1.0, np.abs(want).max())
    xd = dev(x)
    ie.layernorm(xd, dev(g), dev(b), out=xd)  # in place, as the engine calls it
    assert np.array_equal(host(xd), got)


@pytest.mark.parametrize("rows,cols", [(1, 768), (128, 768), (5, 256), (3, 767), (64, 3072)])
def test_layernorm_residual(ie, orc, rows, cols):
    """ie_layernorm_residual (run_layernorm_residual): residual_out = x + res
    bit-exact, out within 1e-5 of the output scale of the oracle and equal bit
    for bit to ie_layernorm of residual_out; the same results with out and
    residual_out aliased to the inputs (cols 767: the scalar path)."""
    r = rng(rows * 7 + cols)
    x = (r.standard_normal((rows, cols)) * 2).astype(np.float32)
    res = (r.standard_normal((rows, cols)) + 0.5).astype(np.float32)
    g = (1 + 0.2 * r.standard_normal(cols)).astype(np.float32)
    b = (0.1 * r.standard_normal(cols)).astype(np.float32)
    want, want_res = orc.layernorm_residual(x, res, g, b)
    gd, bd = dev(g), dev(b)
    out, res_out = ie.layernorm_residual(dev(x), dev(res), gd, bd)
    got, got_res = host(out), host(res_out)
    assert np.array_equal(got_res, want_res)
    assert np.abs(got - want).max() <= 1e-5 * np.abs(want).max()
    assert np.array_equal(host(ie.layernorm(res_out, gd, bd)), got)
    for alias in ("out=x,res_out=res", "out=res,res_out=x", "both=x"):
        xd, rd = dev(x), dev(res)
        o, ro = {"out=x,res_out=res": (xd, rd), "out=res,res_out=x": (rd, xd), "both=x": (xd, xd)}[alias]
        if alias == "both=x":
            scratch_out, _ = ie.layernorm_residual(xd, rd, gd, bd, out=xd, residual_out=xd)
            # out written over residual_out: only out survives
            assert np.array_equal(host(scratch_out), got), alias
            continue
        ie.layernorm_residual(xd, rd, gd, bd, out=o, residual_out=ro)
        assert np.array_equal(host(o), got) and np.array_equal(host(ro), got_res), alias


def test_embedding_vocab_argmax(ie, orc):
    import torch

    r = rng(6)
    V, d, L = 50257, 768, 1024
    wte = (r.standard_normal((V, d)) * 0.02).astype(np.float32)
    wpe = (r.standard_normal((L, d)) * 0.01).astype(np.float32)
    ids = np.array([50256, 0, 1234], dtype=np.int32)
    wte_d = dev(wte)
    emb = host(ie.embedding(dev(ids), 7, wte_d, dev(wpe)))
    assert np.array_equal(emb, orc.embedding(ids, 7, wte, wpe))
    for rows in (1, 16):
        h = r.standard_normal((rows, d)).astype(np.float32)
        logits = host(ie.vocab_proj(dev(h), wte_d))
        for i in range(rows):
            want = orc.vocab_proj(h[i], wte)
            assert np.abs(logits[i] - want).max() < 1e-5 * np.abs(want).max()
        idx = host(ie.argmax(dev(logits)))
        assert idx.tolist() == [int(np.argmax(logits[i])) for i in range(rows)]
    tie = np.zeros((2, 1000), np.float32)
    tie[0, [5, 600]] = 3.0
    tie[1, :] = -1.0
    assert host(ie.argmax(dev(tie))).tolist() == [5, 0]


@pytest.mark.parametrize("n", [1, 2, 3, 5, 7, 4096, 50257, 70001])
def test_argmax_rows_and_ties(ie, orc, n):
    """First index of the maximum (std::max_element) per row: three rows, so
    rows 1 and 2 start inside a 16-byte chunk when n is not a multiple of 4;
    the maximum repeated later in a row, in the first and the last element,
    and an all -inf row."""
    r = rng(n)
    x = r.standard_normal((3, n)).astype(np.float32)
    if n > 2:
        x[0, n // 3] = x[0, n - 1] = 9.0
        x[1, 0] = 9.0
        x[1, n - 1] = 9.0
    x[2, :] = -np.inf
    got = host(ie.argmax(dev(x))).tolist()
    assert got == [orc.argmax(x[i]) for i in range(3)] == [int(np.argmax(x[i])) for i in range(3)]


@pytest.mark.parametrize("d,V", [(768, 50257), (128, 1000), (1024, 333), (100, 77)])
def test_vocab_proj_rows_bit_identical_across_batch(ie, orc, d, V):
    """Row r of a 16-row projection equals the 1-row and 5-row projections of
    the same hidden row bit for bit (the engine's batch invariance rests on
    it), for the MFMA form (d % 64 == 0) and the lane-row form (d = 100); all
    within 1e-5 of the oracle's fp64 dot products."""
    r = rng(d + V)
    wte = (r.standard_normal((V, d)) * 0.02).astype(np.float32)
    h = r.standard_normal((16, d)).astype(np.float32)
    wte_d = dev(wte)
    full = host(ie.vocab_proj(dev(h), wte_d))
    five = host(ie.vocab_proj(dev(h[:5]), wte_d))
    assert np.array_equal(full[:5], five)
    for i in (0, 3, 15):
        one = host(ie.vocab_proj(dev(h[i:i + 1]), wte_d))
        assert np.array_equal(one[0], full[i])
        want = orc.vocab_proj(h[i], wte)
        assert np.abs(full[i] - want).max() < 1e-5 * np.abs(want).max()
