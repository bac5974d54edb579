"""The engine's fp32 comparison backend (InferenceBackend::CUBLAS_FP32, the
reference's src/gpt2_engine.cu:530-610: vendor fp32 GEMMs on the exporter's
{name}_weight_fp32.bin [K, N] weights, python/export_gpt2.py:48-57), and the
INT8 path measured against it as the reference's --compare mode does.

Bars: the fp32 backend against TorchRefGPT2(quantized=False), an independent
float64 GPT-2 forward over the same files, within 1e-4 of the logit scale
(fp32 GEMM accumulation over K <= 3072, twelve steps); the INT8 engine against
the same float64 forward within 0.1 of the logit scale (W8A8 quantization
error, reported), and the fp32 backend much closer than the INT8 one.
"""
import numpy as np
import pytest

from gpt2_model import TorchRefGPT2, random_tensors, write_model

pytestmark = pytest.mark.gpu

CFG = dict(n_layers=3, n_heads=12, d_model=768, d_ff=3072, vocab_size=2000, max_seq_len=128)


@pytest.fixture(scope="module")
def model_dir(tmp_path_factory):
    d = tmp_path_factory.mktemp("gpt2_fp32")
    write_model(str(d), CFG, random_tensors(CFG, 61))
    return d


def rel(a, b):
    return float(np.abs(a - b).max() / np.abs(b).max())


@pytest.mark.parametrize("B", [1, 4])
def test_fp32_backend_matches_fp64_forward(ie, model_dir, B):
    rng = np.random.default_rng(70 + B)
    prompt = rng.integers(0, CFG["vocab_size"], (B, 9)).astype(np.int32)
    toks = rng.integers(0, CFG["vocab_size"], (12, B)).astype(np.int32)
    eng = ie.Engine(model_dir, max_batch=B, backend=ie.BACKEND_FP32)
    int8 = ie.Engine(model_dir, max_batch=B)
    ref = TorchRefGPT2(str(model_dir), batch=B, quantized=False)
    got = eng.prefill(prompt)        # M = B x 9 vendor GEMMs + prefill attention
    got8 = int8.prefill(prompt)
    for t in range(prompt.shape[1]):
        want = ref.step(prompt[:, t])
    errs, errs8 = [rel(got, want)], [rel(got8, want)]
    for t in toks:
        got, got8, want = eng.step(t), int8.step(t), ref.step(t)
        errs.append(rel(got, want))
        errs8.append(rel(got8, want))
    print(f"fp32 backend vs fp64: {max(errs):.2e}; INT8 engine vs fp64: {max(errs8):.2e}")
    assert max(errs) <= 1e-4, errs
    assert max(errs8) <= 0.1, errs8
    assert max(errs) * 50 < max(errs8)
    eng.close()
    int8.close()


def test_fp32_backend_generate_and_random_model(ie, model_dir):
    """generate() through the fp32 backend (prefill, decode, argmax), and a
    random model built in memory (its fp32 weights kept) agrees with the same
    model written to disk and loaded back."""
    eng = ie.Engine(model_dir, max_batch=2, backend=ie.BACKEND_FP32)
    prompts = np.random.default_rng(3).integers(0, CFG["vocab_size"], (2, 16)).astype(np.int32)
    a, m = eng.generate(prompts, 10, ignore_eos=True)
    b, _ = eng.generate(prompts, 10, ignore_eos=True)
    assert np.array_equal(a, b) and m["tps"] > 0 and (a >= 0).all()
    eng.close()
    small = dict(n_layers=2, n_heads=2, d_model=128, d_ff=512, vocab_size=500, max_seq_len=64)
    mem = ie.Engine(None, seed=9, max_batch=1, backend=ie.BACKEND_FP32, **small)
    import tempfile

    with tempfile.TemporaryDirectory() as td:
        ie.write_random_model(td, seed=9, **small)
        disk = ie.Engine(td, max_batch=1, backend=ie.BACKEND_FP32)
        for t in (5, 77, 499, 0):
            x, y = mem.step(np.array([t], np.int32)), disk.step(np.array([t], np.int32))
            assert np.array_equal(x, y)
        disk.close()
    mem.close()


def test_fp32_backend_needs_fp32_files(ie, tmp_path):
    small = dict(n_layers=1, n_heads=2, d_model=128, d_ff=256, vocab_size=300, max_seq_len=32)
    d = write_model(str(tmp_path / "nofp32"), small, random_tensors(small, 4), fp32_weights=False)
    with pytest.raises(ie.IeError) as e:
        ie.Engine(d, backend=ie.BACKEND_FP32)
    assert e.value.status == ie.IE_ERR_INVALID and "weight_fp32" in e.value.msg
