"""The C-ABI library without a GPU: it loads, exports every symbol the headers
declare, and rejects invalid arguments on the host with a status code before
any HIP call (so none of these tests touches a device)."""
import ctypes
import os
import re
import subprocess

import pytest

from conftest import PKG, ROOT

HDR = os.path.join(ROOT, "include", "ie_amd.h")
ENGINE_HDR = os.path.join(ROOT, "include", "ie_engine.h")
COMPAT = os.path.join(ROOT, "include", "ie_compat.h")
LIB = os.path.join(PKG, "libie_amd.so")


SIGS_EXPECTED = 23  # entry points declared in include/ie_amd.h


def declared_c_functions(path=HDR):
    text = open(path).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+char\s*\*|int|size_t|double)\s+(ie_\w+)\s*\(", text, re.M)))


def declared_cpp_functions():
    text = open(COMPAT).read()
    return sorted(set(re.findall(r"^\s*(?:void|int)\s+(run_\w+|sample_\w+)\s*\(", text, re.M)))


def exported():
    out = subprocess.run(["nm", "-D", "--defined-only", "-C", LIB], capture_output=True, text=True,
                         check=True).stdout
    return out


def test_library_loads_and_exports_all(ie):
    names = declared_c_functions()
    assert len(names) == SIGS_EXPECTED
    lib = ctypes.CDLL(LIB)
    for n in names:
        assert hasattr(lib, n), n
    # the ctypes tables cover exactly the headers
    assert sorted(ie.SIGNATURES) == names
    eng = declared_c_functions(ENGINE_HDR)
    assert len(eng) == 11 and sorted(ie.ENGINE_SIGNATURES) == eng
    for n in eng:
        assert hasattr(lib, n), n
    syms = exported()
    for n in declared_cpp_functions():
        assert re.search(rf"\b{n}\(", syms), n
    assert ie.load().ie_version() >= 100


def test_oracle_not_linked():
    out = subprocess.run(["ldd", LIB], capture_output=True, text=True, check=True).stdout
    assert "liborc" not in out
    assert "orc_" not in exported()


FAKE = ctypes.c_void_p(1 << 20)  # aligned, never dereferenced: validation fails first


def st(ie, name, *args):
    return ie.call(name, *args)


def test_gemm_validation(ie):
    n = None
    assert st(ie, "ie_int8_gemm_ex", 4, 4, 6, FAKE, FAKE, FAKE, FAKE, 0, n, n, FAKE, 0, n) == ie.IE_ERR_INVALID
    assert "multiple of 4" in ie.last_error()
    assert st(ie, "ie_int8_gemm_ex", -1, 4, 8, FAKE, FAKE, FAKE, FAKE, 0, n, n, FAKE, 0, n) == ie.IE_ERR_INVALID
    assert st(ie, "ie_int8_gemm_ex", 4, 4, 8, FAKE, FAKE, FAKE, FAKE, 9, n, n, FAKE, 0, n) == ie.IE_ERR_INVALID
    assert st(ie, "ie_int8_gemm_ex", 4, 4, 131072, FAKE, FAKE, FAKE, FAKE, 0, n, n, FAKE, 0, n) == ie.IE_ERR_UNSUPPORTED
    # bias epilogues need bias, residual epilogue needs residual
    for epi in (1, 2, 3):
        assert st(ie, "ie_int8_gemm_ex", 4, 4, 8, FAKE, FAKE, FAKE, FAKE, epi, n, FAKE, FAKE, 0, n) == ie.IE_ERR_INVALID
    assert st(ie, "ie_int8_gemm_ex", 4, 4, 8, FAKE, FAKE, FAKE, FAKE, 3, FAKE, n, FAKE, 0, n) == ie.IE_ERR_INVALID
    assert st(ie, "ie_int8_gemm_ex", 4, 4, 8, FAKE, FAKE, n, FAKE, 0, n, n, FAKE, 0, n) == ie.IE_ERR_INVALID
    assert st(ie, "ie_int8_gemm_ex", 4, 4, 8, n, FAKE, FAKE, FAKE, 0, n, n, FAKE, 0, n) == ie.IE_ERR_INVALID
    assert st(ie, "ie_int8_gemm_ex", 4, 4, 8, FAKE, FAKE, FAKE, FAKE, 0, n, n, FAKE, 7, n) == ie.IE_ERR_INVALID
    assert st(ie, "ie_int8_gemm_ex", 17, 4, 8, FAKE, FAKE, FAKE, FAKE, 0, n, n, FAKE, 1, n) == ie.IE_ERR_UNSUPPORTED
    # int32 output only through the _ex entry
    assert st(ie, "ie_int8_gemm", 4, 4, 8, FAKE, FAKE, FAKE, FAKE, 4, n, n, FAKE, n) == ie.IE_ERR_INVALID
    # empty problems are accepted without work
    assert st(ie, "ie_int8_gemm_ex", 0, 4, 8, n, n, n, n, 0, n, n, n, 0, n) == ie.IE_OK
    assert st(ie, "ie_int8_gemm_ex", 4, 0, 8, n, n, n, n, 0, n, n, n, 0, n) == ie.IE_OK


def test_quantize_validation(ie):
    n = None
    assert st(ie, "ie_quantize_fp32_to_int8", 2, 6, FAKE, FAKE, FAKE, n) == ie.IE_ERR_INVALID
    assert st(ie, "ie_quantize_fp32_to_int8", 2, 8, n, FAKE, FAKE, n) == ie.IE_ERR_INVALID
    assert st(ie, "ie_quantize_fp32_to_int8", 2, 8, ctypes.c_void_p((1 << 20) + 4), FAKE, FAKE, n) == ie.IE_ERR_INVALID
    assert st(ie, "ie_quantize_fp32_to_int8", 0, 8, n, n, n, n) == ie.IE_OK


def attn(ie, B=2, H_q=8, H_kv=2, d=128, kvdt=0, max_ctx=100, bs=16, nbps=7, ws=1 << 30, splits=0,
         Q=FAKE, kc=FAKE, ws_ptr=FAKE):
    return st(ie, "ie_decode_attn", B, H_q, H_kv, d, Q, kc, FAKE, kvdt, FAKE, FAKE, max_ctx, bs, nbps,
              FAKE, ws_ptr, ws, splits, None)


def test_decode_attn_validation(ie):
    assert attn(ie, d=96) == ie.IE_ERR_UNSUPPORTED          # reference: d != 64 is UB
    assert attn(ie, H_q=12, H_kv=4) == ie.IE_ERR_UNSUPPORTED  # G=3: reference is a silent no-op
    assert attn(ie, H_q=12, H_kv=5) == ie.IE_ERR_INVALID
    assert attn(ie, H_q=32, H_kv=2) == ie.IE_ERR_UNSUPPORTED  # G=16
    assert attn(ie, kvdt=2) == ie.IE_ERR_INVALID
    assert attn(ie, bs=0) == ie.IE_ERR_INVALID
    assert attn(ie, nbps=6) == ie.IE_ERR_INVALID                # 100 tokens need 7 blocks
    assert attn(ie, max_ctx=-1) == ie.IE_ERR_INVALID
    assert attn(ie, Q=None) == ie.IE_ERR_INVALID
    assert attn(ie, Q=ctypes.c_void_p((1 << 20) + 8)) == ie.IE_ERR_INVALID
    # workspace: 2*8*S*(128+2)*4 bytes for the plan's S splits
    S = ie.num_splits(100, 16)
    need = ie.workspace_bytes(2, 8, 128, S)
    assert need == 2 * 8 * S * 130 * 4
    assert attn(ie, ws=need - 4) == ie.IE_ERR_WORKSPACE
    assert attn(ie, ws=need - 4, ws_ptr=None) == ie.IE_ERR_INVALID
    assert attn(ie, B=0) == ie.IE_OK


def prefill(ie, B=2, P=40, H_q=8, H_kv=2, d=128, kvdt=0, nbps=4, bs=16, start=24, Q=FAKE, O=FAKE):
    return st(ie, "ie_prefill_attn", B, P, H_q, H_kv, d, Q, FAKE, FAKE, kvdt, FAKE, nbps, bs, start, O, None)


def test_prefill_attn_validation(ie):
    assert prefill(ie, d=96) == ie.IE_ERR_UNSUPPORTED
    assert prefill(ie, H_q=8, H_kv=3) == ie.IE_ERR_INVALID
    assert prefill(ie, kvdt=2) == ie.IE_ERR_INVALID
    assert prefill(ie, bs=0) == ie.IE_ERR_INVALID
    assert prefill(ie, start=-1) == ie.IE_ERR_INVALID
    assert prefill(ie, nbps=3) == ie.IE_ERR_INVALID       # 24 + 40 tokens need 4 blocks
    assert prefill(ie, Q=None) == ie.IE_ERR_INVALID
    assert prefill(ie, O=ctypes.c_void_p((1 << 20) + 8)) == ie.IE_ERR_INVALID
    assert prefill(ie, P=0) == ie.IE_OK
    assert prefill(ie, B=0) == ie.IE_OK
    # one workgroup per (16-query tile, head, sequence) in a 1-D grid: 2^31 of them is one too many
    assert prefill(ie, B=2048, P=16384, H_q=1024, H_kv=1, d=64, nbps=2048) == ie.IE_ERR_UNSUPPORTED
    assert "grid too large" in ie.last_error()
    fa = lambda *a: st(ie, "ie_flash_attn", *a, None)  # noqa: E731
    assert fa(2048, 1024, 16384, 64, FAKE, FAKE, FAKE, FAKE, 1) == ie.IE_ERR_UNSUPPORTED
    assert fa(1, 2, 64, 96, FAKE, FAKE, FAKE, FAKE, 1) == ie.IE_ERR_UNSUPPORTED
    assert fa(1, 2, 64, 64, FAKE, None, FAKE, FAKE, 1) == ie.IE_ERR_INVALID
    assert fa(1, 2, -1, 64, FAKE, FAKE, FAKE, FAKE, 1) == ie.IE_ERR_INVALID
    assert fa(1, 2, 0, 64, FAKE, FAKE, FAKE, FAKE, 1) == ie.IE_OK
    # O overlapping V (the reference engine's own call passes O = V)
    base = 1 << 24
    q, k, v = (ctypes.c_void_p(base + i * (1 << 20)) for i in range(3))
    assert fa(1, 2, 64, 64, q, k, v, ctypes.c_void_p(base + 2 * (1 << 20) + 256), 1) == ie.IE_ERR_INVALID
    assert "overlaps" in ie.last_error()


def test_split_plan_matches_oracle(ie, orc):
    for ctx in list(range(0, 70)) + [127, 128, 129, 400, 1000, 1024, 4096, 8192, 32768]:
        for bs in (1, 8, 16, 32):
            assert ie.num_splits(ctx, bs) == orc.decode_num_splits(ctx, bs), (ctx, bs)
    # explicit split counts are capped by the block count and IE_DA_MAX_SPLITS
    assert ie.num_splits(8192, 16, 64) == 64
    assert ie.num_splits(8192, 16, 10_000) == ie.DA_MAX_SPLITS
    assert ie.num_splits(40, 16, 64) == 3


def test_other_validation(ie):
    n = None
    assert st(ie, "ie_kv_cache_write", FAKE, FAKE, FAKE, FAKE, 0, FAKE, 1, -1, 12, 64, 16, n) == ie.IE_ERR_INVALID
    assert st(ie, "ie_kv_cache_write", FAKE, FAKE, FAKE, FAKE, 3, FAKE, 1, 0, 12, 64, 16, n) == ie.IE_ERR_INVALID
    assert st(ie, "ie_kv_cache_write", n, FAKE, FAKE, FAKE, 0, FAKE, 1, 0, 12, 64, 16, n) == ie.IE_ERR_INVALID
    assert st(ie, "ie_kv_cache_append_batch", 2, FAKE, FAKE, FAKE, FAKE, 0, FAKE, 0, FAKE, 12, 64, 16, n) == ie.IE_ERR_INVALID
    assert st(ie, "ie_layernorm", 1, 0, FAKE, FAKE, FAKE, FAKE, 1e-5, n) == ie.IE_ERR_INVALID
    assert st(ie, "ie_layernorm_residual", 1, 0, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 1e-5, n) == ie.IE_ERR_INVALID
    assert st(ie, "ie_layernorm_residual", -1, 8, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 1e-5, n) == ie.IE_ERR_INVALID
    assert st(ie, "ie_layernorm_residual", 2, 8, FAKE, n, FAKE, FAKE, FAKE, FAKE, 1e-5, n) == ie.IE_ERR_INVALID
    assert st(ie, "ie_layernorm_residual", 0, 8, n, n, n, n, n, n, 1e-5, n) == ie.IE_OK
    assert st(ie, "ie_vocab_proj", 17, FAKE, FAKE, FAKE, 768, 10, n) == ie.IE_ERR_INVALID
    assert st(ie, "ie_vocab_proj", 1, FAKE, FAKE, FAKE, 766, 10, n) == ie.IE_ERR_INVALID
    assert st(ie, "ie_argmax", 1, FAKE, 0, FAKE, n) == ie.IE_ERR_INVALID
    assert st(ie, "ie_embedding", n, 1, 0, 768, FAKE, FAKE, FAKE, n) == ie.IE_ERR_INVALID


def test_compat_wrapper_rejects_without_touching_outputs():
    """run_* (reference signatures) print the rejection and return: exercised
    through a tiny C++ program that links the library but never reaches HIP."""
    src = r"""
#include "ie_compat.h"
#include <cstdio>
#include <cstring>
int main() {
    float C[4] = {1, 2, 3, 4};
    run_int8_gemm(1, 4, 6, nullptr, nullptr, nullptr, nullptr, C);   // K % 4 != 0
    if (std::strstr(ie_last_error(), "multiple of 4") == nullptr) return 2;
    float O[64] = {7};
    run_decode_attn(1, 12, 4, 64, nullptr, nullptr, nullptr, nullptr, nullptr, 16, 16, 1, O, nullptr);
    if (std::strstr(ie_last_error(), "group size 3") == nullptr) return 3;
    return (C[0] == 1 && C[3] == 4 && O[0] == 7) ? 0 : 4;
}
"""
    import tempfile

    with tempfile.TemporaryDirectory() as td:
        cpp = os.path.join(td, "t.cpp")
        exe = os.path.join(td, "t")
        open(cpp, "w").write(src)
        subprocess.run(["g++", "-std=c++17", "-I", os.path.join(ROOT, "include"), cpp, "-o", exe, LIB,
                        f"-Wl,-rpath,{PKG}"], check=True)
        r = subprocess.run([exe], capture_output=True, text=True)
        assert r.returncode == 0, (r.returncode, r.stderr)
        assert "rejected" in r.stderr


def test_decode_attn_noalloc_rejects_plans_beyond_its_scratch(ie):
    """ie_decode_attn_noalloc validates like ie_decode_attn, then refuses a
    plan whose B * H_q * splits * (d + 2) * 4 bytes of partials exceed the
    library's scratch (IE_ERR_WORKSPACE), all before any HIP call."""
    n = None
    B, H_q, H_kv, d, ctx, splits = 64, 32, 8, 128, 8192, 64
    assert B * H_q * splits * (d + 2) * 4 > ie.DECODE_SCRATCH_BYTES
    args = (B, H_q, H_kv, d, FAKE, FAKE, FAKE, 0, FAKE, FAKE, ctx, 16, ctx // 16, FAKE)
    assert st(ie, "ie_decode_attn_noalloc", *args, splits, n) == ie.IE_ERR_WORKSPACE
    assert "scratch" in ie.last_error()
    # the same validation as ie_decode_attn: group size 3, head dim 96
    assert st(ie, "ie_decode_attn_noalloc", 1, 12, 4, 64, FAKE, FAKE, FAKE, 0, FAKE, FAKE, 16, 16, 1, FAKE, 0,
              n) == ie.IE_ERR_UNSUPPORTED
    assert st(ie, "ie_decode_attn_noalloc", 1, 4, 4, 96, FAKE, FAKE, FAKE, 0, FAKE, FAKE, 16, 16, 1, FAKE, 0,
              n) == ie.IE_ERR_UNSUPPORTED
    assert st(ie, "ie_decode_attn_noalloc", 1, 4, 4, 64, n, FAKE, FAKE, 0, FAKE, FAKE, 16, 16, 1, FAKE, 0,
              n) == ie.IE_ERR_INVALID
    # B = 0 is a no-op
    assert st(ie, "ie_decode_attn_noalloc", 0, 4, 4, 64, n, n, n, 0, n, n, 16, 16, 1, n, 0, n) == ie.IE_OK
