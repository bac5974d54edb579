"""Engine host logic without a GPU: the random-model writer produces the
reference's on-disk format (python/export_gpt2.py:73-167) with per-row int8
weights, and invalid configurations are rejected with a status code."""
import json
import os

import numpy as np

from conftest import unpack_i8

TINY = dict(n_layers=2, n_heads=2, d_model=128, d_ff=256, vocab_size=1000, max_seq_len=64)


def test_writer_layout_and_quantization(ie, tmp_path):
    ie.write_random_model(tmp_path, seed=5, **TINY)
    cfg = json.load(open(tmp_path / "config.json"))
    assert cfg == dict(TINY, d_head=64)
    d, ff, V, S = 128, 256, 1000, 64
    assert os.path.getsize(tmp_path / "wte.bin") == V * d * 4
    assert os.path.getsize(tmp_path / "wpe.bin") == S * d * 4
    for name, N, K in [("qkv", 3 * d, d), ("out", d, d), ("ffn_up", ff, d), ("ffn_down", d, ff)]:
        w = np.fromfile(tmp_path / "layer_01" / f"{name}_weight.bin", dtype=np.int32).reshape(N, K // 4)
        s = np.fromfile(tmp_path / "layer_01" / f"{name}_scale.bin", dtype=np.float32)
        b = np.fromfile(tmp_path / "layer_01" / f"{name}_bias.bin", dtype=np.float32)
        assert s.shape == (N,) and b.shape == (N,)
        q = unpack_i8(w).astype(np.int32)
        assert np.all(np.abs(q).max(axis=1) == 127)          # row max maps to +-127
        deq = q * s[:, None]
        assert 0.015 < deq.std() < 0.025                      # N(0, 0.02) weights
        assert np.all(s > 0) and np.allclose(s, np.abs(deq).max(axis=1) / 127, rtol=1e-6)
    g = np.fromfile(tmp_path / "layer_00" / "ln1_gamma.bin", dtype=np.float32)
    assert np.all(g == 1.0)
    # same seed, same bytes
    other = tmp_path / "again"
    ie.write_random_model(other, seed=5, **TINY)
    assert open(tmp_path / "layer_00" / "qkv_weight.bin", "rb").read() == \
        open(other / "layer_00" / "qkv_weight.bin", "rb").read()


def test_writer_rejects_bad_config(ie, tmp_path):
    st = ie.call("ie_engine_write_random_model", str(tmp_path / "x").encode(), 2, 3, 128, 256, 100, 64, 1)
    assert st == ie.IE_ERR_INVALID  # d_head = 128 / 3 is not an integer head size
    st = ie.call("ie_engine_write_random_model", str(tmp_path / "y").encode(), 2, 4, 128, 256, 100, 64, 1)
    assert st == ie.IE_ERR_INVALID and "d_head" in ie.last_error()  # d_head 32 unsupported


def test_engine_c_api_rejects_bad_arguments_without_a_gpu(ie):
    """The engine's C entry points validate on the host: null handles, empty
    prompts and bad option values fail with a status before any HIP call."""
    import ctypes

    lib = ie.load()
    P = ctypes.c_void_p
    assert lib.ie_engine_prefill(None, 1, 4, P(1 << 20), None, None) == ie.IE_ERR_INVALID
    toks = (ctypes.c_int * 4)(1, 2, 3, 4)
    assert lib.ie_engine_prefill(None, 1, 4, ctypes.cast(toks, P), None, None) == ie.IE_ERR_INVALID
    assert lib.ie_engine_step(None, 1, ctypes.cast(toks, P), None, None) == ie.IE_ERR_INVALID
    assert lib.ie_engine_generate(None, 1, 4, ctypes.cast(toks, P), 2, 0, None, None) == ie.IE_ERR_INVALID
    h = P()
    # negative prefill chunk
    st = lib.ie_engine_create(ctypes.byref(h), None, 2, 2, 128, 512, 1000, 64, 1, 1, 0, 0, 1, 1, 1, -5, 0)
    assert st == ie.IE_ERR_INVALID and "prefill_chunk" in ie.last_error()
    st = lib.ie_engine_create(ctypes.byref(h), None, 2, 2, 128, 512, 1000, 64, 1, 1, 0, 0, 1, 1, 1, 0, 7)
    assert st == ie.IE_ERR_INVALID and "backend" in ie.last_error()
    assert lib.ie_engine_create(None, None, 2, 2, 128, 512, 1000, 64, 1, 1, 0, 0, 1, 1, 1, 0, 0) == ie.IE_ERR_INVALID


def test_token_id_check_rejects_out_of_range(ie):
    """ie_check_token_ids, which the engine runs on every host token before it
    is uploaded (the embedding kernels index wte rows without a bound)."""
    import ctypes

    V = 1000
    for bad, where in (([5, -1, 7], 1), ([V, 0], 0), ([0, 1, 2, V + 3], 3)):
        arr = (ctypes.c_int * len(bad))(*bad)
        st = ie.call("ie_check_token_ids", len(bad), ctypes.cast(arr, ctypes.c_void_p), V)
        assert st == ie.IE_ERR_INVALID
        assert f"index {where}" in ie.last_error() and str(bad[where]) in ie.last_error()
    ok = (ctypes.c_int * 3)(0, V - 1, 17)
    assert ie.call("ie_check_token_ids", 3, ctypes.cast(ok, ctypes.c_void_p), V) == ie.IE_OK
    assert ie.call("ie_check_token_ids", 0, None, V) == ie.IE_OK
    assert ie.call("ie_check_token_ids", 2, None, V) == ie.IE_ERR_INVALID
    assert ie.call("ie_check_token_ids", 1, ctypes.cast(ok, ctypes.c_void_p), 0) == ie.IE_ERR_INVALID


def test_writer_quantizer_and_fp32_files_pinned(ie, orc, tmp_path):
    """The writer's quantizer (quantize_rows_host, the closed form of
    python/export_gpt2.py:10-40) against the oracle's quantizer and a numpy
    restatement of the exporter, bit for bit, on the fp32 weights the writer
    also saves as {name}_weight_fp32.bin [K, N] (export_gpt2.py:48-57):
    transposed to [N, K], quantized per output row, they give exactly the
    int8 words and scales in {name}_weight.bin / _scale.bin."""
    from gpt2_model import quantize_per_row

    ie.write_random_model(tmp_path, seed=8, **TINY)
    d, ff = TINY["d_model"], TINY["d_ff"]
    for layer in ("layer_00", "layer_01"):
        for name, K, N in [("qkv", d, 3 * d), ("out", d, d), ("ffn_up", d, ff), ("ffn_down", ff, d)]:
            p = tmp_path / layer
            wf = np.fromfile(p / f"{name}_weight_fp32.bin", dtype=np.float32)
            assert wf.size == K * N
            wt = np.ascontiguousarray(wf.reshape(K, N).T)
            packed = np.fromfile(p / f"{name}_weight.bin", dtype=np.int32).reshape(N, K // 4)
            scale = np.fromfile(p / f"{name}_scale.bin", dtype=np.float32)
            op, os_ = orc.quantize(wt)
            assert np.array_equal(packed, op) and np.array_equal(scale, os_), (layer, name)
            npk, nps = quantize_per_row(wt)
            assert np.array_equal(packed, npk) and np.array_equal(scale, nps), (layer, name)
