"""ctypes binding of libie_amd.so (include/ie_amd.h) for tests and benchmarks.

The product is the C ABI; this module only marshals torch device tensors into
it.  It never falls back to anything: if the HIP library is missing or a call
is rejected, it raises.
"""
from __future__ import annotations

import ctypes
import numbers
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libie_amd.so")

IE_OK, IE_ERR_INVALID, IE_ERR_UNSUPPORTED, IE_ERR_WORKSPACE, IE_ERR_HIP = range(5)
EPI_PLAIN, EPI_BIAS, EPI_BIAS_GELU, EPI_BIAS_RESIDUAL, EPI_I32 = range(5)
PATH_AUTO, PATH_GEMV, PATH_MFMA = range(3)
KV_F32, KV_BF16 = 0, 1
BACKEND_INT8, BACKEND_FP32 = 0, 1
DA_REF_MAX_SPLITS = 16
DA_MAX_SPLITS = 256

_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float
_Z = ctypes.c_size_t

# name -> (restype, argtypes); mirrors include/ie_amd.h one to one.
SIGNATURES = {
    "ie_last_error": (ctypes.c_char_p, []),
    "ie_version": (_I, []),
    "ie_init": (_I, []),
    "ie_quantize_fp32_to_int8": (_I, [_I, _I, _P, _P, _P, _P]),
    "ie_int8_gemm": (_I, [_I, _I, _I, _P, _P, _P, _P, _I, _P, _P, _P, _P]),
    "ie_int8_gemm_ex": (_I, [_I, _I, _I, _P, _P, _P, _P, _I, _P, _P, _P, _I, _P]),
    "ie_decode_num_splits": (_I, [_I, _I, _I]),
    "ie_decode_attn_workspace_bytes": (_Z, [_I, _I, _I, _I]),
    "ie_decode_attn": (_I, [_I, _I, _I, _I, _P, _P, _P, _I, _P, _P, _I, _I, _I, _P, _P, _Z, _I, _P]),
    "ie_prefill_attn": (_I, [_I, _I, _I, _I, _I, _P, _P, _P, _I, _P, _I, _I, _I, _P, _P]),
    "ie_flash_attn": (_I, [_I, _I, _I, _I, _P, _P, _P, _P, _I, _P]),
    "ie_kv_cache_write": (_I, [_P, _P, _P, _P, _I, _P, _I, _I, _I, _I, _I, _P]),
    "ie_kv_cache_append_batch": (_I, [_I, _P, _P, _P, _P, _I, _P, _I, _P, _I, _I, _I, _P]),
    "ie_layernorm": (_I, [_I, _I, _P, _P, _P, _P, _F, _P]),
    "ie_layernorm_residual": (_I, [_I, _I, _P, _P, _P, _P, _P, _P, _F, _P]),
    "ie_embedding": (_I, [_P, _I, _I, _I, _P, _P, _P, _P]),
    "ie_embedding_batch": (_I, [_I, _P, _P, _I, _P, _P, _P, _P]),
    "ie_vocab_proj": (_I, [_I, _P, _P, _P, _I, _I, _P]),
    "ie_argmax": (_I, [_I, _P, _I, _P, _P]),
    "ie_topk": (_I, [_I, _P, _I, _I, _P, _P, _P]),
    "ie_top_k_draw": (_I, [_P, _P, _I, _F, ctypes.c_uint, _P]),
    "ie_check_token_ids": (_I, [_I, _P, _I]),
    "ie_decode_attn_noalloc": (_I, [_I, _I, _I, _I, _P, _P, _P, _I, _P, _P, _I, _I, _I, _P, _I, _P]),
}
DECODE_SCRATCH_BYTES = 32 << 20

# include/ie_engine.h
ENGINE_SIGNATURES = {
    "ie_engine_create": (_I, [ctypes.POINTER(_P), ctypes.c_char_p, _I, _I, _I, _I, _I, _I,
                              ctypes.c_ulonglong, _I, _I, _I, _I, _I, _I, _I, _I]),
    "ie_engine_destroy": (_I, [_P]),
    "ie_engine_write_random_model": (_I, [ctypes.c_char_p, _I, _I, _I, _I, _I, _I, ctypes.c_ulonglong]),
    "ie_engine_reset": (_I, [_P]),
    "ie_engine_generate": (_I, [_P, _I, _I, _P, _I, _I, _P, _P]),
    "ie_engine_generate_one": (_I, [_P, _I, _P, _I, _F, _I, _I, _I, _P, _P, _P]),
    "ie_engine_step": (_I, [_P, _I, _P, _P, _P]),
    "ie_engine_prefill": (_I, [_P, _I, _I, _P, _P, _P]),
    "ie_engine_session_tokens": (_I, [_P]),
    "ie_engine_config": (_I, [_P, _P]),
    "ie_engine_step_bytes": (ctypes.c_double, [_P, _I]),
}


# include/ie_tokenizer.h (host code; no GPU)
TOKENIZER_SIGNATURES = {
    "ie_tokenizer_create": (_I, [_P, ctypes.c_char_p]),
    "ie_tokenizer_destroy": (_I, [_P]),
    "ie_tokenizer_encode": (_I, [_P, ctypes.c_char_p, _Z, _P, _Z, _P]),
    "ie_tokenizer_decode": (_I, [_P, _P, _Z, _P, _Z, _P]),
    "ie_tokenizer_vocab_size": (_I, [_P]),
    "ie_tokenizer_eos_token": (_I, [_P]),
}


class Metrics(ctypes.Structure):
    """ie_metrics (include/ie_engine.h): InferenceMetrics without `generating`."""
    _fields_ = [(n, ctypes.c_float) for n in ("ttft_ms", "tpot_ms", "itl_min_ms", "itl_max_ms",
                                              "itl_p95_ms", "tps")] + \
               [("tokens_generated", ctypes.c_int), ("max_tokens", ctypes.c_int)] + \
               [(n, ctypes.c_float) for n in ("kv_cache_pct", "vram_used_mb", "vram_total_mb", "mbu",
                                              "end_to_end_ms")]

    def as_dict(self):
        return {k: getattr(self, k) for k, _ in self._fields_}


class IeError(RuntimeError):
    def __init__(self, fn: str, status: int, msg: str):
        super().__init__(f"{fn} failed with status {status}: {msg}")
        self.status = status
        self.msg = msg


_lib = None


def load() -> ctypes.CDLL:
    """Loads libie_amd.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        # torch ships its own libamdhip64 (file libamdhip64.so, soname
        # libamdhip64.so.7).  Loading torch first makes the dynamic loader bind
        # our libamdhip64.so.7 dependency to that copy; the other order maps
        # two HIP/HSA runtimes into the process and the second sees no device.
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        if not os.path.exists(LIB_PATH):
            raise FileNotFoundError(
                f"{LIB_PATH} is missing: build it with __graft_entry__.build() "
                "(make -C cuda-llm-inference-engine_amd)")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in (list(SIGNATURES.items()) + list(ENGINE_SIGNATURES.items())
                                  + list(TOKENIZER_SIGNATURES.items())):
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def last_error() -> str:
    return load().ie_last_error().decode()


def call(name: str, *args) -> int:
    """Calls an ie_* entry point and returns its status without raising."""
    return getattr(load(), name)(*args)


def check(name: str, *args) -> None:
    st = call(name, *args)
    if st != IE_OK:
        raise IeError(name, st, last_error())


# ---------------------------------------------------------------- torch glue
def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(stream=None):
    import torch

    s = stream if stream is not None else torch.cuda.current_stream()
    return ctypes.c_void_p(s.cuda_stream)


def quantize(x, out_packed=None, out_scales=None, stream=None):
    """x: [rows, cols] fp32 cuda -> (packed int32 [rows, cols/4], scales [rows])."""
    import torch

    rows, cols = x.shape
    packed = out_packed if out_packed is not None else torch.empty(
        (rows, cols // 4), dtype=torch.int32, device=x.device)
    scales = out_scales if out_scales is not None else torch.empty(
        rows, dtype=torch.float32, device=x.device)
    check("ie_quantize_fp32_to_int8", rows, cols, _ptr(x), _ptr(packed), _ptr(scales), _stream(stream))
    return packed, scales


def int8_gemm(A_packed, BT_packed, sA=None, sB=None, epilogue=EPI_PLAIN, bias=None,
              residual=None, out=None, path=PATH_AUTO, stream=None):
    """Returns C [M, N] (fp32, or int32 for EPI_I32)."""
    import torch

    M, K4 = A_packed.shape
    N = BT_packed.shape[0]
    if out is None:
        dt = torch.int32 if epilogue == EPI_I32 else torch.float32
        out = torch.empty((M, N), dtype=dt, device=A_packed.device)
    check("ie_int8_gemm_ex", M, N, 4 * K4, _ptr(A_packed), _ptr(BT_packed), _ptr(sA), _ptr(sB),
          epilogue, _ptr(bias), _ptr(residual), _ptr(out), path, _stream(stream))
    return out


def num_splits(max_ctx: int, block_size: int, splits: int = 0) -> int:
    return call("ie_decode_num_splits", max_ctx, block_size, splits)


def workspace_bytes(B: int, H_q: int, d: int, splits: int) -> int:
    return call("ie_decode_attn_workspace_bytes", B, H_q, d, splits)


def decode_attn(Q, k_cache, v_cache, block_table, context_lens, max_ctx, block_size, H_kv,
                kv_dtype=KV_F32, splits=0, out=None, workspace=None, stream=None):
    """Q [B, H_q, d] fp32; caches [P, bs, H_kv, d]; returns O [B, H_q, d]."""
    import torch

    B, H_q, d = Q.shape
    nbps = block_table.shape[1]
    S = num_splits(max_ctx, block_size, splits)
    need = workspace_bytes(B, H_q, d, S)
    if workspace is None:
        workspace = torch.empty(max(need // 4, 1), dtype=torch.float32, device=Q.device)
    if out is None:
        out = torch.empty_like(Q)
    check("ie_decode_attn", B, H_q, H_kv, d, _ptr(Q), _ptr(k_cache), _ptr(v_cache), kv_dtype,
          _ptr(block_table), _ptr(context_lens), max_ctx, block_size, nbps, _ptr(out),
          _ptr(workspace), workspace.numel() * 4, splits, _stream(stream))
    return out


def decode_attn_noalloc(Q, k_cache, v_cache, block_table, context_lens, max_ctx, block_size, H_kv,
                        kv_dtype=KV_F32, splits=0, out=None, stream=None):
    """ie_decode_attn_noalloc: as decode_attn, split partials in the library's
    per-device scratch (no workspace)."""
    import torch

    B, H_q, d = Q.shape
    if out is None:
        out = torch.empty_like(Q)
    check("ie_decode_attn_noalloc", B, H_q, H_kv, d, _ptr(Q), _ptr(k_cache), _ptr(v_cache), kv_dtype,
          _ptr(block_table), _ptr(context_lens), max_ctx, block_size, block_table.shape[1], _ptr(out),
          splits, _stream(stream))
    return out


def prefill_attn(Q, k_cache, v_cache, block_table, start_pos, block_size, H_kv, kv_dtype=KV_F32,
                 out=None, stream=None):
    """Q [B, P, H_q, d] fp32 (token t at position start_pos + t, its K/V already
    cached); returns causal O [B, P, H_q, d]."""
    import torch

    B, P, H_q, d = Q.shape
    if out is None:
        out = torch.empty_like(Q)
    check("ie_prefill_attn", B, P, H_q, H_kv, d, _ptr(Q), _ptr(k_cache), _ptr(v_cache), kv_dtype,
          _ptr(block_table), block_table.shape[1], block_size, start_pos, _ptr(out), _stream(stream))
    return out


def flash_attn(Q, K, V, causal=True, out=None, stream=None):
    """Q, K, V [B, H, N, d] fp32 -> O [B, H, N, d] (run_flash_attn_v2)."""
    import torch

    B, H, N, d = Q.shape
    if out is None:
        out = torch.empty_like(Q)
    check("ie_flash_attn", B, H, N, d, _ptr(Q), _ptr(K), _ptr(V), _ptr(out), int(causal), _stream(stream))
    return out


def kv_cache_write(K, V, k_cache, v_cache, block_table, start_pos, block_size,
                   kv_dtype=KV_F32, stream=None):
    seq, H, dh = K.shape
    check("ie_kv_cache_write", _ptr(K), _ptr(V), _ptr(k_cache), _ptr(v_cache), kv_dtype,
          _ptr(block_table), seq, start_pos, H, dh, block_size, _stream(stream))


def kv_cache_append_batch(K, V, k_cache, v_cache, block_table, positions, block_size,
                          kv_dtype=KV_F32, stream=None):
    B, H, dh = K.shape
    check("ie_kv_cache_append_batch", B, _ptr(K), _ptr(V), _ptr(k_cache), _ptr(v_cache), kv_dtype,
          _ptr(block_table), block_table.shape[1], _ptr(positions), H, dh, block_size,
          _stream(stream))


def layernorm(x, gamma, beta, out=None, eps=1e-5, stream=None):
    import torch

    rows, cols = x.shape
    out = out if out is not None else torch.empty_like(x)
    check("ie_layernorm", rows, cols, _ptr(x), _ptr(gamma), _ptr(beta), _ptr(out), eps, _stream(stream))
    return out


def layernorm_residual(x, residual, gamma, beta, out=None, residual_out=None, eps=1e-5, stream=None):
    """(LayerNorm(x + residual), x + residual); out / residual_out may alias
    the inputs."""
    import torch

    rows, cols = x.shape
    out = out if out is not None else torch.empty_like(x)
    residual_out = residual_out if residual_out is not None else torch.empty_like(x)
    check("ie_layernorm_residual", rows, cols, _ptr(x), _ptr(residual), _ptr(gamma), _ptr(beta), _ptr(out),
          _ptr(residual_out), eps, _stream(stream))
    return out, residual_out


def embedding(ids, start_pos, wte, wpe, out=None, stream=None):
    import torch

    seq = ids.shape[0]
    d = wte.shape[1]
    out = out if out is not None else torch.empty((seq, d), dtype=torch.float32, device=wte.device)
    check("ie_embedding", _ptr(ids), seq, start_pos, d, _ptr(wte), _ptr(wpe), _ptr(out), _stream(stream))
    return out


def vocab_proj(h, wte, out=None, stream=None):
    import torch

    rows, d = h.shape
    V = wte.shape[0]
    out = out if out is not None else torch.empty((rows, V), dtype=torch.float32, device=h.device)
    check("ie_vocab_proj", rows, _ptr(h), _ptr(wte), _ptr(out), d, V, _stream(stream))
    return out


def argmax(logits, out=None, stream=None):
    import torch

    rows, n = logits.shape
    out = out if out is not None else torch.empty(rows, dtype=torch.int32, device=logits.device)
    check("ie_argmax", rows, _ptr(logits), n, _ptr(out), _stream(stream))
    return out


def topk(logits, k, stream=None):
    """(values [rows, k] fp32, indices [rows, k] int32) of the k largest per row,
    by value descending, equal values by index ascending."""
    import torch

    rows, n = logits.shape
    vals = torch.empty((rows, k), dtype=torch.float32, device=logits.device)
    idx = torch.empty((rows, k), dtype=torch.int32, device=logits.device)
    check("ie_topk", rows, _ptr(logits), n, k, _ptr(vals), _ptr(idx), _stream(stream))
    return vals, idx


def top_k_draw(vals, idx, temperature, seed):
    """Host draw of sample_top_k over sorted (value, index) pairs (numpy)."""
    import numpy as np

    v = np.ascontiguousarray(vals, dtype=np.float32)
    i = np.ascontiguousarray(idx, dtype=np.int32)
    tok = ctypes.c_int(-1)
    check("ie_top_k_draw", v.ctypes.data, i.ctypes.data, len(v), ctypes.c_float(temperature),
          ctypes.c_uint(seed), ctypes.addressof(tok))
    return tok.value


# ---------------------------------------------------------------- engine
GPT2_SMALL = dict(n_layers=12, n_heads=12, d_model=768, d_ff=3072, vocab_size=50257, max_seq_len=1024)


def write_random_model(path, seed=0, **cfg):
    c = dict(GPT2_SMALL, **cfg)
    check("ie_engine_write_random_model", str(path).encode(), c["n_layers"], c["n_heads"], c["d_model"],
          c["d_ff"], c["vocab_size"], c["max_seq_len"], seed)


class Engine:
    """GPT-2 decode engine (include/ie_engine.h).  model_dir=None builds a
    random model of the given shape (GPT-2 Small by default)."""

    def __init__(self, model_dir=None, seed=0, max_batch=1, kv_dtype=KV_F32, int8_lm_head=False,
                 use_graph=True, fuse=True, prefill=True, prefill_chunk=0, backend=BACKEND_INT8, **cfg):
        import numpy as np  # noqa: F401

        c = dict(GPT2_SMALL, **cfg)
        h = ctypes.c_void_p()
        check("ie_engine_create", ctypes.byref(h), None if model_dir is None else str(model_dir).encode(),
              c["n_layers"], c["n_heads"], c["d_model"], c["d_ff"], c["vocab_size"], c["max_seq_len"], seed,
              max_batch, kv_dtype, int(int8_lm_head), int(use_graph), int(fuse), int(prefill), prefill_chunk,
              backend)
        self.h = h
        v = (ctypes.c_int * 7)()
        check("ie_engine_config", h, ctypes.cast(v, ctypes.c_void_p))
        self.cfg = dict(zip(("n_layers", "n_heads", "d_model", "d_ff", "vocab_size", "max_seq_len", "d_head"),
                            list(v)))

    def close(self):
        if getattr(self, "h", None):
            load().ie_engine_destroy(self.h)
            self.h = None

    __del__ = close

    def reset(self):
        check("ie_engine_reset", self.h)

    def step(self, tokens, want_logits=True):
        import numpy as np

        toks = np.ascontiguousarray(tokens, dtype=np.int32)
        B = toks.shape[0]
        V = self.cfg["vocab_size"]
        logits = np.empty((B, V), dtype=np.float32) if want_logits else None
        check("ie_engine_step", self.h, B, toks.ctypes.data_as(ctypes.c_void_p),
              None if logits is None else logits.ctypes.data_as(ctypes.c_void_p), None)
        return logits

    def prefill(self, tokens, want_logits=True):
        """tokens [B, P] at the current position -> last-token logits [B, V]."""
        import numpy as np

        toks = np.ascontiguousarray(tokens, dtype=np.int32)
        B, P = toks.shape
        logits = np.empty((B, self.cfg["vocab_size"]), dtype=np.float32) if want_logits else None
        check("ie_engine_prefill", self.h, B, P, toks.ctypes.data_as(ctypes.c_void_p),
              None if logits is None else logits.ctypes.data_as(ctypes.c_void_p), None)
        return logits

    def generate(self, prompts, max_new, ignore_eos=False):
        """prompts [B, P] int -> (tokens [B, max_new] with -1 padding, metrics dict)."""
        import numpy as np

        p = np.ascontiguousarray(prompts, dtype=np.int32)
        B, P = p.shape
        out = np.full((B, max_new), -1, dtype=np.int32)
        m = Metrics()
        check("ie_engine_generate", self.h, B, P, p.ctypes.data_as(ctypes.c_void_p), max_new, int(ignore_eos),
              out.ctypes.data_as(ctypes.c_void_p), ctypes.byref(m))
        return out, m.as_dict()

    def generate_one(self, prompt, max_new, temperature=0.8, top_k=40, greedy=False, reset=True):
        """GPT2Engine::generate for one prompt -> (generated ids, metrics dict)."""
        import numpy as np

        p = np.ascontiguousarray(prompt, dtype=np.int32).reshape(-1)
        out = np.full(max_new, -1, dtype=np.int32)
        n = ctypes.c_int(0)
        m = Metrics()
        check("ie_engine_generate_one", self.h, len(p), p.ctypes.data_as(ctypes.c_void_p), max_new,
              ctypes.c_float(temperature), top_k, int(greedy), int(reset), out.ctypes.data_as(ctypes.c_void_p),
              ctypes.byref(n), ctypes.byref(m))
        return out[: n.value].tolist(), m.as_dict()

    def generate_text(self, tokenizer, prompt, max_new, temperature=0.8, top_k=40, greedy=False, reset=True):
        """The reference's text path (src/main.cpp:224-230, 360-367): the prompt
        encoded by the BPE tokenizer, GPT2Engine::generate, the ids decoded ->
        (generated bytes, generated ids, metrics dict)."""
        ids = tokenizer.encode(prompt)
        if not ids:
            raise ValueError("the prompt encodes to no tokens")
        toks, m = self.generate_one(ids, max_new, temperature, top_k, greedy, reset)
        return tokenizer.decode(toks), toks, m

    def session_tokens(self):
        return load().ie_engine_session_tokens(self.h)

    def step_bytes(self, batch):
        return load().ie_engine_step_bytes(self.h, batch)


class Tokenizer:
    """GPT-2 byte-level BPE tokenizer (include/ie_tokenizer.h), the reference's
    BPETokenizer (include/tokenizer.h:7-25): vocab.json and merges.txt from
    model_dir.  encode takes str or bytes; decode returns bytes, since a token
    can end inside a multi-byte character."""

    def __init__(self, model_dir):
        h = ctypes.c_void_p()
        check("ie_tokenizer_create", ctypes.byref(h), os.fsencode(model_dir))
        self.h = h

    def close(self):
        if self.h:
            load().ie_tokenizer_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def encode(self, text):
        b = text.encode("utf-8") if isinstance(text, str) else bytes(text)
        n = ctypes.c_size_t()
        check("ie_tokenizer_encode", self.h, b, len(b), None, 0, ctypes.byref(n))
        out = (ctypes.c_int * max(n.value, 1))()
        check("ie_tokenizer_encode", self.h, b, len(b), out, n.value, ctypes.byref(n))
        return list(out[:n.value])

    def decode(self, ids):
        ids = [int(i) for i in ([ids] if isinstance(ids, numbers.Integral) else ids)]
        arr = (ctypes.c_int * max(len(ids), 1))(*ids)
        n = ctypes.c_size_t()
        check("ie_tokenizer_decode", self.h, arr, len(ids), None, 0, ctypes.byref(n))
        buf = ctypes.create_string_buffer(max(n.value, 1))
        check("ie_tokenizer_decode", self.h, arr, len(ids), buf, n.value, ctypes.byref(n))
        return buf.raw[:n.value]

    @property
    def vocab_size(self):
        return load().ie_tokenizer_vocab_size(self.h)

    @property
    def eos_token(self):
        return load().ie_tokenizer_eos_token(self.h)
