"""ie_decode_attn_noalloc (split partials in the library's per-device scratch
array, no workspace, no allocation) against ie_decode_attn with a caller
workspace: same kernels and plan, so bit-identical outputs, on consecutive
calls whose second input is smaller (the scratch keeps the first call's
partials; nothing may leak into the second), and both within 1e-5 of the
oracle.  Collected last (pytest -x stops at the first failure), so a failure
here hides no other test."""
import numpy as np
import pytest

from conftest import bf16_bits, make_paged_cache, rng

pytestmark = pytest.mark.gpu


def dev(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def case(seed, B, H_q, H_kv, d, lens, kvdt):
    r = rng(seed)
    kc, vc, table, _, _ = make_paged_cache(r, B, H_kv, d, lens, 16)
    Q = r.standard_normal((B, H_q, d)).astype(np.float32)
    if kvdt:
        kc, vc = bf16_bits(kc), bf16_bits(vc)
    return Q, kc, vc, table, np.asarray(lens, np.int32)


def test_noalloc_matches_workspace_entry_point(ie, orc):
    import torch

    runs = [  # (seed, B, H_q, H_kv, d, lengths, kv dtype, splits): each input smaller than the last
        # 64 * 32 * 31 * (128 + 2) * 4 = 33,013,760 bytes of partials, 98% of
        # IE_DECODE_SCRATCH_BYTES (33,554,432): the array's far end holds the
        # last (sequence, head, split) slots; 62 blocks in 31 splits of 2, so
        # every split is non-empty (ctx >= 961)
        (5, 64, 32, 8, 128, rng(12).integers(961, 993, 64), 0, 31),
        (1, 16, 32, 8, 128, rng(11).integers(1024, 2049, 16), 0, 0),
        (2, 3, 12, 12, 64, [700, 1, 333], 0, 0),
        (3, 2, 8, 2, 128, [2048, 1500], 1, 64),
        (4, 1, 12, 12, 64, [200], 0, 0),
    ]
    for seed, B, H_q, H_kv, d, lens, kvdt, splits in runs:
        Q, kc, vc, table, lens = case(seed, B, H_q, H_kv, d, lens, kvdt)
        mx = int(lens.max())
        if seed == 5:
            need = ie.workspace_bytes(B, H_q, d, ie.num_splits(mx, 16, splits))
            assert 33_000_000 < need <= ie.DECODE_SCRATCH_BYTES, need
        args = (dev(Q), dev(kc), dev(vc), dev(table), dev(lens), mx, 16, H_kv)
        got = ie.decode_attn_noalloc(*args, kv_dtype=kvdt, splits=splits)
        want = ie.decode_attn(*args, kv_dtype=kvdt, splits=splits)
        torch.cuda.synchronize()
        g, w = got.cpu().numpy(), want.cpu().numpy()
        assert np.array_equal(g, w), (seed, np.abs(g - w).max())
        ref = orc.decode_attn(Q, kc, vc, table, lens, mx, 16, H_kv, kv_dtype=kvdt, splits=splits)
        assert np.abs(g - ref).max() <= 1e-5 * np.abs(ref).max(), seed
