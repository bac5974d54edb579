"""ctypes binding of the CPU oracle (oracle/liborc.so) — TEST INFRASTRUCTURE.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use this,
as the checker (and, for cpu_baseline, as the reported CPU figure).  Takes and
returns numpy arrays.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liborc.so")

_P = ctypes.c_void_p
_I = ctypes.c_int
_L = ctypes.c_long
_F = ctypes.c_float

SIGNATURES = {
    "orc_set_threads": (None, [_I]),
    "orc_get_threads": (_I, []),
    "orc_rng_new": (_P, [ctypes.c_uint]),
    "orc_rng_free": (None, [_P]),
    "orc_rng_next": (_I, [_P]),
    "orc_rng_uniform": (None, [_P, _P, _L]),
    "orc_rng_uniform_pair": (None, [_P, _P, _P, _L]),
    "orc_quantize_fp32_to_int8": (_I, [_I, _I, _P, _P, _P]),
    "orc_int8_gemm_i32": (_I, [_I, _I, _I, _P, _P, _P]),
    "orc_int8_gemm": (_I, [_I, _I, _I, _P, _P, _P, _P, _I, _P, _P, _P]),
    "orc_gemm_f64": (None, [_I, _I, _I, _P, _P, _P]),
    "orc_decode_num_splits": (_I, [_I, _I]),
    "orc_decode_attn": (_I, [_I, _I, _I, _I, _P, _P, _P, _I, _P, _P, _I, _I, _I, _I, _P]),
    "orc_decode_attn_f32": (_I, [_I, _I, _I, _I, _P, _P, _P, _I, _P, _P, _I, _I, _I, _I, _P]),
    "orc_kv_cache_write": (_I, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I]),
    "orc_layernorm": (None, [_I, _I, _P, _P, _P, _P, _F]),
    "orc_layernorm_residual": (None, [_I, _I, _P, _P, _P, _P, _P, _P, _F]),
    "orc_embedding": (None, [_P, _I, _I, _I, _P, _P, _P]),
    "orc_vocab_proj": (None, [_P, _P, _P, _I, _I]),
    "orc_argmax": (_I, [_P, _I]),
    "orc_topk": (_I, [_I, _I, _I, _P, _P, _P]),
    "orc_rand_unit": (ctypes.c_float, [_P]),
    "orc_top_k_draw": (_I, [_P, _P, _I, ctypes.c_float, ctypes.c_float]),
}

_lib = None


def load():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise FileNotFoundError(f"{LIB_PATH} missing: run make -C oracle")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def _p(a):
    return None if a is None else ctypes.c_void_p(a.ctypes.data)


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


def set_threads(n: int) -> None:
    load().orc_set_threads(n)


def get_threads() -> int:
    return load().orc_get_threads()


class GlibcRand:
    """glibc rand() with a private state (srand(seed) then rand() ...)."""

    def __init__(self, seed: int):
        self._h = load().orc_rng_new(seed)

    def __del__(self):
        if getattr(self, "_h", None):
            load().orc_rng_free(self._h)
            self._h = None

    def next(self) -> int:
        return load().orc_rng_next(self._h)

    def uniform(self, n: int) -> np.ndarray:
        out = np.empty(n, dtype=np.float32)
        load().orc_rng_uniform(self._h, _p(out), n)
        return out

    def uniform_pair(self, n: int):
        a = np.empty(n, dtype=np.float32)
        b = np.empty(n, dtype=np.float32)
        load().orc_rng_uniform_pair(self._h, _p(a), _p(b), n)
        return a, b


def quantize(x: np.ndarray):
    x = _c(x, np.float32)
    rows, cols = x.shape
    packed = np.empty((rows, cols // 4), dtype=np.int32)
    scales = np.empty(rows, dtype=np.float32)
    st = load().orc_quantize_fp32_to_int8(rows, cols, _p(x), _p(packed), _p(scales))
    if st:
        raise ValueError("orc_quantize_fp32_to_int8 rejected its arguments")
    return packed, scales


def gemm_i32(A_packed: np.ndarray, BT_packed: np.ndarray) -> np.ndarray:
    A = _c(A_packed, np.int32)
    BT = _c(BT_packed, np.int32)
    M, K4 = A.shape
    N = BT.shape[0]
    acc = np.empty((M, N), dtype=np.int32)
    if load().orc_int8_gemm_i32(M, N, 4 * K4, _p(A), _p(BT), _p(acc)):
        raise ValueError("orc_int8_gemm_i32 rejected its arguments")
    return acc


def gemm(A_packed, BT_packed, sA, sB, epilogue=0, bias=None, residual=None) -> np.ndarray:
    A = _c(A_packed, np.int32)
    BT = _c(BT_packed, np.int32)
    M, K4 = A.shape
    N = BT.shape[0]
    sA = _c(sA, np.float32)
    sB = _c(sB, np.float32)
    bias = None if bias is None else _c(bias, np.float32)
    residual = None if residual is None else _c(residual, np.float32)
    C = np.empty((M, N), dtype=np.float32)
    if load().orc_int8_gemm(M, N, 4 * K4, _p(A), _p(BT), _p(sA), _p(sB), epilogue, _p(bias),
                            _p(residual), _p(C)):
        raise ValueError("orc_int8_gemm rejected its arguments")
    return C


def gemm_f64(A: np.ndarray, B: np.ndarray) -> np.ndarray:
    A = _c(A, np.float32)
    B = _c(B, np.float32)
    M, K = A.shape
    N = B.shape[1]
    C = np.empty((M, N), dtype=np.float64)
    load().orc_gemm_f64(M, N, K, _p(A), _p(B), _p(C))
    return C


def decode_num_splits(max_ctx: int, block_size: int) -> int:
    return load().orc_decode_num_splits(max_ctx, block_size)


def decode_attn(Q, k_cache, v_cache, block_table, context_lens, max_ctx, block_size, H_kv,
                kv_dtype=0, splits=0, f32=False) -> np.ndarray:
    """Q [B,H_q,d]; caches [P,bs,H_kv,d] float32 (kv_dtype 0) or uint16 bf16 bits (1)."""
    Q = _c(Q, np.float32)
    B, H_q, d = Q.shape
    kdt = np.float32 if kv_dtype == 0 else np.uint16
    kc = _c(k_cache, kdt)
    vc = _c(v_cache, kdt)
    bt = _c(block_table, np.int32)
    cl = _c(context_lens, np.int32)
    O = np.empty_like(Q)
    fn = load().orc_decode_attn_f32 if f32 else load().orc_decode_attn
    if fn(B, H_q, H_kv, d, _p(Q), _p(kc), _p(vc), kv_dtype, _p(bt), _p(cl), max_ctx, block_size,
          bt.shape[1], splits, _p(O)):
        raise ValueError("orc_decode_attn rejected its arguments")
    return O


def kv_cache_write(K, V, k_cache, v_cache, block_table, start_pos, block_size):
    """In-place write into numpy caches [P, bs, H, dh]."""
    K = _c(K, np.float32)
    V = _c(V, np.float32)
    seq, H, dh = K.shape
    bt = _c(block_table, np.int32)
    assert k_cache.flags.c_contiguous and v_cache.flags.c_contiguous
    if load().orc_kv_cache_write(_p(K), _p(V), _p(k_cache), _p(v_cache), _p(bt), seq, start_pos,
                                 H, dh, block_size):
        raise ValueError("orc_kv_cache_write rejected its arguments")


def layernorm(x, gamma, beta, eps=1e-5):
    x = _c(x, np.float32)
    rows, cols = x.shape
    out = np.empty_like(x)
    load().orc_layernorm(rows, cols, _p(x), _p(_c(gamma, np.float32)), _p(_c(beta, np.float32)),
                         _p(out), eps)
    return out


def layernorm_residual(x, residual, gamma, beta, eps=1e-5):
    """-> (LayerNorm(x + residual), x + residual)."""
    x = _c(x, np.float32)
    residual = _c(residual, np.float32)
    assert x.shape == residual.shape
    rows, cols = x.shape
    out = np.empty_like(x)
    res_out = np.empty_like(x)
    load().orc_layernorm_residual(rows, cols, _p(x), _p(residual), _p(_c(gamma, np.float32)),
                                  _p(_c(beta, np.float32)), _p(out), _p(res_out), eps)
    return out, res_out


def embedding(ids, start_pos, wte, wpe):
    ids = _c(ids, np.int32)
    wte = _c(wte, np.float32)
    wpe = _c(wpe, np.float32)
    d = wte.shape[1]
    out = np.empty((ids.shape[0], d), dtype=np.float32)
    load().orc_embedding(_p(ids), ids.shape[0], start_pos, d, _p(wte), _p(wpe), _p(out))
    return out


def vocab_proj(h, wte):
    h = _c(h, np.float32).reshape(-1)
    wte = _c(wte, np.float32)
    V, d = wte.shape
    out = np.empty(V, dtype=np.float32)
    load().orc_vocab_proj(_p(h), _p(wte), _p(out), d, V)
    return out


def argmax(logits) -> int:
    logits = _c(logits, np.float32)
    return load().orc_argmax(_p(logits), logits.shape[0])


def topk(logits, k):
    """logits [rows, n] -> (values [rows, k], indices [rows, k]); src/sampler.cu:20-26."""
    logits = _c(np.atleast_2d(logits), np.float32)
    rows, n = logits.shape
    vals = np.empty((rows, k), dtype=np.float32)
    idx = np.empty((rows, k), dtype=np.int32)
    if load().orc_topk(rows, n, k, _p(logits), _p(vals), _p(idx)) != 0:
        raise ValueError("orc_topk: bad arguments")
    return vals, idx


def rand_unit(seed: int, skip: int = 0) -> float:
    """(float)rand() / RAND_MAX for the (skip+1)-th rand() after srand(seed)."""
    g = GlibcRand(seed)
    for _ in range(skip):
        g.next()
    return load().orc_rand_unit(g._h)


def top_k_draw(vals, idx, temperature, r) -> int:
    """The index drawn at threshold r from sorted pairs; src/sampler.cu:27-44."""
    v = _c(vals, np.float32)
    i = _c(idx, np.int32)
    return load().orc_top_k_draw(_p(v), _p(i), len(v), ctypes.c_float(temperature), ctypes.c_float(r))


def sample_top_k(logits, k, temperature, seed, skip=0) -> int:
    """sample_top_k of one row when srand(seed) was just called (skip = rand()
    calls since), src/sampler.cu:16-45."""
    logits = np.asarray(logits, dtype=np.float32).reshape(-1)
    k = min(k, logits.shape[0])
    v, i = topk(logits, k)
    return top_k_draw(v[0], i[0], temperature, rand_unit(seed, skip))
