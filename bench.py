#!/usr/bin/env python3
"""Measures the INT8 decode hot path on one MI355X.

Headline (`value`): INT8 GEMM throughput at M=N=K=8192 (Plain epilogue, int32
accumulate, fp32 out) in TOP/s, one "step" = one GEMM launch over resident
inputs.  Its operands are made (and quantized, untimed) first; the warm-up and
timed launches run after the other GPU legs, so the part's clock has left its
idle state (back-to-back launches on a just-woken GPU run up to ~20% slower
for the first ~30).  The same JSON line carries:
  roofline      the 8192^3 kernel against the dense i8 MFMA peak (5.0 POP/s);
                mfma_util from a SQ_VALU_MFMA_BUSY_CYCLES / GRBM_GUI_ACTIVE pass
  vendor_gemm   hipBLASLt (torch._int_mm) on the same operands, same box
  gemv          decode-M (1, 4, 16) GEMMs on the GPT-2 weight shapes, the LM
                head shape, 8192x8192 and 8192x28672, in GB/s of algorithmic
                bytes against HBM (8 TB/s), weights rotated through >= 1 GiB
                of copies so the 256 MiB MALL cannot serve them;
                gemv_roofline leads with BASELINE's M=1 K=N=8192
  gemm_m512     the GPT-2 shapes at M = 512 (prefill-sized), TOP/s
  ref_shapes    the reference's own bench shapes (INT8 GEMM 256^3..2048^3,
                incl. BASELINE cfg1 512^3; its eight decode-attention
                configurations) beside its published GTX 1650 Ti times
  decode_attn   split-K paged decode attention, BASELINE cfg3 (MHA), cfg4
                (GQA, ctx 4096/8192/32768, fp32 and bf16 KV) and G = 8 at
                d = 128, GB/s of algorithmic bytes against HBM
  e2e_gpt2      GPT-2 Small decode tok/s (BASELINE cfg5), batch 1 and 16, INT8
                and the fp32 vendor-GEMM comparison backend
  sampler       top-k sampling: device selection kernel, one sample_top_k
                call, the reference's whole-row copy, sampled decode at batch 1
  cpu_baseline  the C oracle (oracle/liborc.so) on a bounded sample of the
                8192^3 GEMM, on this host's cores; cpu_baseline_attn the same
                for decode attention cfg4 ctx 8192 fp32; cpu_baseline_detail
                1-thread and all-thread figures for cfg1, the GPT-2 shapes at
                M = 1/4/16, cfg3 and cfg4 at ctx 4096/8192, with the CPU model
  traffic       HBM bytes per launch of the dominant kernels and the BASELINE
                GEMV shapes (rocprofv3 FETCH_SIZE / WRITE_SIZE passes,
                calibrated on a 1 GiB copy)
Kernel durations come from HIP events on the stream the kernels run on.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "cuda-llm-inference-engine_amd")
for _p in (ROOT, PKG):
    if _p not in sys.path:
        sys.path.insert(0, _p)

PEAK_HBM_GBS = 8000.0      # MI355X HBM3E, GB/s
PEAK_I8_TOPS = 5000.0      # MI355X dense int8 MFMA, TOP/s
METRIC = "INT8 GEMM TOPS & decode-attn GB/s (% peak); GPT-2-124M decode tok/s, 1 GPU"
ROTATE_BYTES = 1 << 30     # rotate weight/KV copies through >= 1 GiB


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--skip", default="",
                    help="comma list of vendor,gemv,gemm512,ref,attn,cpu,e2e,sampler,mfma")
    ap.add_argument("--only-headline", action="store_true")
    ap.add_argument("--no-traffic", action="store_true", help="skip the rocprofv3 FETCH/WRITE passes")
    ap.add_argument("--pmc-child", action="store_true", help=argparse.SUPPRESS)
    ap.add_argument("--mfma-child", action="store_true", help=argparse.SUPPRESS)
    ap.add_argument("--ramp", action="store_true",
                    help="per-launch times of the headline GEMM in bursts (power transient), then exit")
    return ap.parse_args()


class Timer:
    """HIP events on the current torch stream (where the library launches)."""

    def __init__(self):
        import torch

        self.s = torch.cuda.Event(enable_timing=True)
        self.e = torch.cuda.Event(enable_timing=True)

    def __enter__(self):
        self.s.record()
        return self

    def __exit__(self, *a):
        import torch

        self.e.record()
        torch.cuda.synchronize()
        self.ms = self.s.elapsed_time(self.e)


def graph_time(launch, count, reps=3):
    """Captures `count` launches (launch(i)) into one HIP graph and returns the
    mean device time per launch in ms over `reps` replays, so host launch cost
    does not leave the GPU idle between small kernels."""
    import torch

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for i in range(min(count, 3)):  # warm up outside capture
            launch(i)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(count):
            launch(i)
    g.replay()
    torch.cuda.synchronize()
    with Timer() as t:
        for _ in range(reps):
            g.replay()
    return t.ms / (reps * count)


def roof(achieved, peak, unit, bound, traffic=None):
    return {"bound": bound, "achieved": round(achieved, 2), "peak": peak, "unit": unit,
            "frac": round(achieved / peak, 4), "traffic": traffic}


def gemm_bytes(M, N, K, bias=False, residual=False):
    b = M * K + N * K + 4 * M + 4 * N + 4 * M * N
    return b + (4 * N if bias else 0) + (4 * M * N if residual else 0)


# ------------------------------------------------------------------ headline
def headline_inputs(ie):
    """BASELINE recipe: A, B fp32 ~ N(0,1) from a seed; A quantized per row and
    B per column (= per row of B^T) with the library's quantizer (untimed)."""
    import torch

    M = N = K = 8192
    g = torch.Generator(device="cuda").manual_seed(42)
    Af = torch.randn((M, K), device="cuda", generator=g)
    Ap, sA = ie.quantize(Af)
    del Af
    BTf = torch.randn((N, K), device="cuda", generator=g)
    Bp, sB = ie.quantize(BTf)
    del BTf
    torch.cuda.empty_cache()
    torch.cuda.synchronize()
    return (Ap, Bp, sA, sB)


def bench_headline(ie, inputs, steps, warmup):
    import torch

    M = N = K = 8192
    Ap, Bp, sA, sB = inputs
    C = torch.empty((M, N), dtype=torch.float32, device="cuda")

    def launch():
        ie.int8_gemm(Ap, Bp, sA, sB, ie.EPI_PLAIN, out=C)

    for _ in range(warmup):
        launch()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    with Timer() as t:
        for _ in range(steps):
            launch()
    wall = time.perf_counter() - t0
    ops = 2.0 * M * N * K
    kern_ms = t.ms / steps
    return {
        "ms_per_step": wall * 1e3 / steps,
        "value": ops / (wall / steps) / 1e12,
        "kernel_ms": kern_ms,
        "kernel_tops": ops / (kern_ms * 1e-3) / 1e12,
        "bytes": gemm_bytes(M, N, K),
    }


def bench_vendor(ie, inputs, steps, warmup):
    """hipBLASLt's int8 GEMM (torch._int_mm) on the headline's own quantized
    operands, timed the same way: a same-box reference point for the
    power-limited MFMA rate.  It returns int32 with no dequant epilogue (our
    kernel also writes the fp32 dequant), so it does slightly less work.  Run
    just before the headline with at least 50 warm-up launches: the step into
    sustained MFMA load throttles the clock for the next ~50 launches (bench.py
    --ramp), and this leg takes both measurements past that transient."""
    import torch

    Ap, Bp, _, _ = inputs
    M, K = Ap.shape[0], Ap.shape[1] * 4
    N = Bp.shape[0]
    A8 = Ap.view(torch.int8).view(M, K)
    B8 = Bp.view(torch.int8).view(N, K)
    try:
        for _ in range(max(warmup, 50)):
            C = torch._int_mm(A8, B8.t())
        torch.cuda.synchronize()
        with Timer() as t:
            for _ in range(steps):
                C = torch._int_mm(A8, B8.t())
        del C
    except Exception as e:  # noqa: BLE001 - reported, not fatal
        return {"error": str(e)[:200]}
    ms = t.ms / steps
    return {"library": "hipBLASLt via torch._int_mm (int32 out, no dequant)",
            "TOP/s": round(2.0 * M * N * K / (ms * 1e-3) / 1e12, 1), "us": round(ms * 1e3, 1)}


# ------------------------------------------------------------------ GEMV
def bench_gemv(ie):
    import torch

    shapes = [(768, 2304), (768, 768), (768, 3072), (3072, 768), (768, 50257), (8192, 8192),
              (8192, 28672)]
    out = []
    g = torch.Generator(device="cuda").manual_seed(7)
    for K, N in shapes:
        wbytes = N * K
        R = max(8, -(-ROTATE_BYTES // wbytes))
        W = torch.randint(-127, 128, (R, N, K), dtype=torch.int8, device="cuda", generator=g)
        Wp = W.view(torch.int32)
        sB = torch.rand(N, device="cuda", generator=g) * 0.01
        bias = torch.randn(N, device="cuda", generator=g)
        for M in (1, 4, 16):
            A = torch.randint(-127, 128, (M, K), dtype=torch.int8, device="cuda", generator=g)
            Ap = A.view(torch.int32)
            sA = torch.rand(M, device="cuda", generator=g) * 0.01
            C = torch.empty((M, N), dtype=torch.float32, device="cuda")
            ms = graph_time(lambda i: ie.int8_gemm(Ap, Wp[i % R], sA, sB, ie.EPI_PLAIN, out=C), R)
            byts = gemm_bytes(M, N, K)
            gbs = byts / (ms * 1e-3) / 1e9
            out.append({"M": M, "K": K, "N": N, "us": round(ms * 1e3, 2), "GBps": round(gbs, 1),
                        "frac_hbm": round(gbs / PEAK_HBM_GBS, 3)})
            log(f"gemv M={M} K={K} N={N}: {ms * 1e3:.2f} us {gbs:.0f} GB/s")
        del W, Wp
        torch.cuda.empty_cache()
    return out


def bench_gemm512(ie):
    import torch

    out = []
    g = torch.Generator(device="cuda").manual_seed(8)
    M = 512
    for K, N in [(768, 2304), (768, 768), (768, 3072), (3072, 768), (768, 50257)]:
        A = torch.randint(-127, 128, (M, K), dtype=torch.int8, device="cuda", generator=g).view(torch.int32)
        # the launches rotate through R (weights, output) pairs totalling
        # >= 1 GiB, so neither the weights nor C stay in the 256 MiB MALL
        # between launches (the HBM claim, as the GEMV leg measures it)
        R = max(8, -(-ROTATE_BYTES // (N * K + 4 * M * N)))
        B = torch.randint(-127, 128, (R, N, K), dtype=torch.int8, device="cuda", generator=g).view(torch.int32)
        sA = torch.rand(M, device="cuda", generator=g)
        sB = torch.rand(N, device="cuda", generator=g)
        C = torch.empty((R, M, N), dtype=torch.float32, device="cuda")
        # median of three graph-timed runs: launches of the 103 MB-output
        # shape ranged 31.8-38.0 us within one traced run
        ms = sorted(graph_time(lambda i: ie.int8_gemm(A, B[i % R], sA, sB, ie.EPI_PLAIN, out=C[i % R]), R)
                    for _ in range(3))[1]
        # the hot loop beside it: one (weights, output) pair every launch
        ms_hot = sorted(graph_time(lambda i: ie.int8_gemm(A, B[0], sA, sB, ie.EPI_PLAIN, out=C[0]), 20)
                        for _ in range(3))[1]
        tops = 2.0 * M * N * K / (ms * 1e-3) / 1e12
        byt = gemm_bytes(M, N, K)
        # arithmetic intensity 2MNK / bytes is below the 629 op/B ridge for
        # every shape here: HBM is the bound
        out.append({"M": M, "K": K, "N": N, "us": round(ms * 1e3, 2), "TOPs": round(tops, 1),
                    "bytes": byt, "GBps": round(byt / (ms * 1e-3) / 1e9, 1),
                    "frac_hbm": round(byt / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 3), "bound": "hbm",
                    "rotated_pairs": R, "us_hot": round(ms_hot * 1e3, 2)})
        log(f"gemm M=512 K={K} N={N}: {ms * 1e3:.2f} us {tops:.1f} TOP/s {out[-1]['frac_hbm']} of HBM "
            f"(hot loop {ms_hot * 1e3:.2f} us)")
        del B, C
        torch.cuda.empty_cache()
    return out


# ------------------------------------------------------------------ attention
def attn_case(ie, B, H_q, H_kv, d, ctx, kv_bf16, uniform, seed, max_copies=64):
    import torch

    gen = torch.Generator().manual_seed(seed)
    if uniform:
        lens = torch.full((B,), ctx, dtype=torch.int32)
    else:
        lens = torch.randint(ctx // 2, ctx + 1, (B,), generator=gen, dtype=torch.int32)
    bs = 16
    nbs = (lens + bs - 1) // bs
    nbps = int(nbs.max())
    P = int(nbs.sum())
    kvdt = torch.bfloat16 if kv_bf16 else torch.float32
    esz = 2 if kv_bf16 else 4
    kv_bytes = int(lens.sum()) * H_kv * d * 2 * esz
    alg = kv_bytes + 2 * B * H_q * d * 4 + 4 * P + 4 * B
    copies = max(1, -(-(2 * ROTATE_BYTES) // max(kv_bytes, 1))) if kv_bytes < ROTATE_BYTES else 1
    copies = min(copies, max_copies)
    gcuda = torch.Generator(device="cuda").manual_seed(seed)
    caches = []
    for _ in range(copies):
        kc = torch.randn((P, bs, H_kv, d), device="cuda", generator=gcuda).to(kvdt)
        vc = torch.randn((P, bs, H_kv, d), device="cuda", generator=gcuda).to(kvdt)
        perm = torch.randperm(P, generator=gen).to(torch.int32)
        table = torch.zeros((B, nbps), dtype=torch.int32)
        off = 0
        for b in range(B):
            table[b, : int(nbs[b])] = perm[off: off + int(nbs[b])]
            off += int(nbs[b])
        caches.append((kc, vc, table.cuda()))
    Q = torch.randn((B, H_q, d), device="cuda", generator=gcuda)
    O = torch.empty_like(Q)
    lens_d = lens.cuda()
    max_ctx = int(lens.max())
    S = ie.num_splits(max_ctx, bs)
    ws = torch.empty(ie.workspace_bytes(B, H_q, d, S) // 4, dtype=torch.float32, device="cuda")
    dt = ie.KV_BF16 if kv_bf16 else ie.KV_F32

    def launch(i):
        kc, vc, table = caches[i % copies]
        ie.decode_attn(Q, kc, vc, table, lens_d, max_ctx, bs, H_kv, kv_dtype=dt, out=O, workspace=ws)

    n = max(copies, 8)
    # median of five captured-graph timings (single timings spread by ~3%)
    ms = sorted(graph_time(launch, n) for _ in range(5))[2]
    gbs = alg / (ms * 1e-3) / 1e9
    res = {"B": B, "H_q": H_q, "H_kv": H_kv, "d": d, "ctx": ctx, "kv": "bf16" if kv_bf16 else "fp32",
           "lengths": "uniform" if uniform else "U[ctx/2,ctx]", "sum_ctx": int(lens.sum()),
           "splits": S, "bytes": alg, "us": round(ms * 1e3, 2), "GBps": round(gbs, 1),
           "frac_hbm": round(gbs / PEAK_HBM_GBS, 3)}
    log(f"decode_attn {res}")
    del caches
    torch.cuda.empty_cache()
    return res

def bench_attn(ie):
    out = [attn_case(ie, 8, 12, 12, 64, 1024, False, True, 3)]
    for ctx in (4096, 8192, 32768):
        for bf in (False, True):
            out.append(attn_case(ie, 32, 32, 8, 128, ctx, bf, False, ctx + bf))
    # G = 8 at d = 128 (64 query heads over 8 KV heads), ctx 8192
    for bf in (False, True):
        out.append(attn_case(ie, 32, 64, 8, 128, 8192, bf, False, 88 + bf))
    return out


# ------------------------------------------------------------------ reference bench shapes
# The reference's own benchmark shapes and its published times on a GTX 1650 Ti
# (README.md:162-169, 183-186; benchmarks/int8_gemm_bench.cu:27,
# benchmarks/decode_attention_bench.cu:57-67): context only, other hardware.
REF_GEMM_US = {256: 23.7, 512: 93.2, 1024: 788.3, 2048: 5213.2}
# the same table's FP32 cuBLAS column on the reference's GPU (README.md:181-186)
REF_FP32_US = {256: 31.8, 512: 212.8, 1024: 963.2, 2048: 6619.3}
REF_ATTN_US = [((1, 8, 8, 128), 31.9), ((1, 8, 8, 256), 25.2), ((1, 8, 8, 512), 29.5), ((1, 8, 8, 1024), 51.8),
               ((4, 8, 8, 256), 49.0), ((8, 8, 8, 512), 162.6), ((1, 16, 4, 256), 34.9), ((1, 32, 8, 512), 81.5)]


def vendor_sgemm_us(A, B, C, reps=20):
    """fp32 C = A @ B on the vendor BLAS, the reference bench's cuBLAS SGEMM
    column (benchmarks/int8_gemm_bench.cu:78-96): 3 warm-ups, then `reps`
    back-to-back launches between HIP events.  rocBLAS (torch's "cublas"
    backend on ROCm) and hipBLASLt ("cublaslt")."""
    import torch

    be = torch.backends.cuda.preferred_blas_library()
    res = {}
    try:
        for name, lib in (("rocblas", "cublas"), ("hipblaslt", "cublaslt")):
            torch.backends.cuda.preferred_blas_library(lib)
            for _ in range(3):
                torch.mm(A, B, out=C)
            torch.cuda.synchronize()
            with Timer() as t:
                for _ in range(reps):
                    torch.mm(A, B, out=C)
            res[name] = t.ms * 1e3 / reps
    finally:
        torch.backends.cuda.preferred_blas_library(be)
    return res


def bench_ref_shapes(ie):
    """INT8 GEMM S^3 (U(-1,1) operands quantized by the library, Plain
    epilogue; 512^3 is BASELINE cfg1) and decode attention (d 64, block 16,
    fp32, every sequence at ctx), timed from HIP graphs.  Beside each GEMM,
    as the reference bench prints it: the fp32 vendor GEMM on the same
    operands (rocBLAS SGEMM; hipBLASLt too) and the FP32/INT8 time ratio."""
    import torch

    out = {"gemm": [], "decode_attn": [], "reference_hw": "GTX 1650 Ti (README.md:28-30)"}
    g = torch.Generator(device="cuda").manual_seed(11)
    for S, ref_us in REF_GEMM_US.items():
        A = torch.rand((S, S), device="cuda", generator=g) * 2 - 1
        BT = torch.rand((S, S), device="cuda", generator=g) * 2 - 1
        Ap, sA = ie.quantize(A)
        Bp, sB = ie.quantize(BT)
        C = torch.empty((S, S), device="cuda")
        ms = graph_time(lambda i: ie.int8_gemm(Ap, Bp, sA, sB, ie.EPI_PLAIN, out=C), 20)
        r = {"M=N=K": S, "us": round(ms * 1e3, 2), "TOPs": round(2.0 * S ** 3 / (ms * 1e-3) / 1e12, 2),
             "reference_us": ref_us}
        try:
            B = BT.t().contiguous()
            fp = vendor_sgemm_us(A, B, torch.empty((S, S), device="cuda"))
            r["fp32_rocblas_us"] = round(fp["rocblas"], 2)
            r["fp32_hipblaslt_us"] = round(fp["hipblaslt"], 2)
            r["int8_over_fp32"] = round(fp["rocblas"] / (ms * 1e3), 2)  # the reference's INT8/FP32 column
            r["reference_fp32_us"] = REF_FP32_US[S]
            r["reference_int8_over_fp32"] = round(REF_FP32_US[S] / ref_us, 2)
            del B
        except Exception as e:  # noqa: BLE001 - reported, not fatal
            r["fp32_error"] = str(e)[:200]
        out["gemm"].append(r)
        log(f"ref gemm {r}")
    for (B, H_q, H_kv, ctx), ref_us in REF_ATTN_US:
        r = attn_case(ie, B, H_q, H_kv, 64, ctx, False, True, ctx + B + H_q, max_copies=16)
        out["decode_attn"].append({"B": B, "H_q": H_q, "H_kv": H_kv, "ctx": ctx, "us": r["us"], "GBps": r["GBps"],
                                   "reference_us": ref_us})
    return out


# ------------------------------------------------------------------ end to end
def bench_e2e(ie):
    """GPT-2 Small random-init N(0, 0.02), INT8 per-row
    linears (W8A8 as the reference engine), paged KV, prompt of 128 random ids,
    greedy decode of 256 tokens at batch 1 and 16.  tok/s counts decode steps
    only (src/gpt2_engine.cu:754); MBU = bytes streamed per step (weights, LM head and the KV of
    the timed steps' mean context) x steps/s / 8 TB/s.
    ttft_ms = prompt prefill + first token; also reported with the prompt fed
    through decode steps."""
    import numpy as np

    out = []
    rng = np.random.default_rng(128)
    # fused step (4 launches per layer up to 384 tokens) for both LM heads; the unfused step
    # (every operation through the public C ABI) and the fp32 vendor-GEMM
    # backend (the reference's CUBLAS_FP32 comparison point) for comparison
    for head_i8, fuse, backend in ((False, True, 0), (True, True, 0), (False, False, 0), (False, False, 1)):
        eng = ie.Engine(None, seed=1234, max_batch=16, int8_lm_head=head_i8, fuse=fuse, backend=backend)
        for B in (1, 16):
            prompts = rng.integers(0, 50257, (B, 128)).astype(np.int32)
            eng.generate(prompts, 8, ignore_eos=True)  # warm up (graph capture)
            toks, m = eng.generate(prompts, 256, ignore_eos=True)
            step = "fp32 vendor GEMM backend" if backend else "fused" if fuse else "unfused"
            r = {"batch": B, "lm_head": "int8" if head_i8 else "fp32 (reference)",
                 "step": step, "prompt": "prefill",
                 "decode_tok_s": round(m["tps"], 1), "tpot_ms": round(m["tpot_ms"], 4),
                 "ttft_ms": round(m["ttft_ms"], 2), "itl_p95_ms": round(m["itl_p95_ms"], 4),
                 "mbu": round(m["mbu"], 4), "tokens": int((toks >= 0).sum())}
            out.append(r)
            log(f"e2e {r}")
        eng.close()
    # time to first token with the prompt fed one decode step per position
    # (the engine's path with prefill off) for comparison
    eng = ie.Engine(None, seed=1234, max_batch=16, prefill=False)
    for B in (1, 16):
        prompts = rng.integers(0, 50257, (B, 128)).astype(np.int32)
        eng.generate(prompts, 2, ignore_eos=True)
        _, m = eng.generate(prompts, 2, ignore_eos=True)
        r = {"batch": B, "lm_head": "fp32 (reference)", "step": "fused", "prompt": "decode steps",
             "ttft_ms": round(m["ttft_ms"], 2)}
        out.append(r)
        log(f"e2e {r}")
    eng.close()
    return out


def bench_sampler(ie):
    """Top-k sampling of GPT-2 logits (src/sampler.cu:16-45; k = 40, T = 0.8 as
    the reference TUI): the device selection kernel alone (rows 1 and 16), one
    whole sample_top_k call (selection, two k-pair copies, host draw), the
    201 KB row copy the reference's route starts with, and sampled decode of
    GPT-2 Small at batch 1 (prompt 128, 256 new tokens)."""
    import ctypes
    import numpy as np
    import torch

    V, k = 50257, 40
    out = {}
    g = torch.Generator(device="cuda").manual_seed(40)
    for rows in (1, 16):
        x = torch.randn((rows, V), device="cuda", generator=g) * 3 - 80
        vals = torch.empty((rows, k), device="cuda")
        idx = torch.empty((rows, k), dtype=torch.int32, device="cuda")

        def launch(i, x=x, vals=vals, idx=idx, rows=rows):  # on the capturing stream
            ie.check("ie_topk", rows, ie._ptr(x), V, k, ie._ptr(vals), ie._ptr(idx), ie._stream())

        out[f"topk_kernel_us_rows{rows}"] = round(graph_time(launch, 20) * 1e3, 2)
    lib = ie.load()
    fn = getattr(lib, "_Z12sample_top_kPKfiifj")
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_float, ctypes.c_uint]
    row = (torch.randn(V, device="cuda", generator=g) * 3 - 80).contiguous()
    for s in range(20):
        fn(ctypes.c_void_p(row.data_ptr()), V, k, 0.8, 1000 + s)
    n = 300
    t0 = time.perf_counter()
    for s in range(n):
        fn(ctypes.c_void_p(row.data_ptr()), V, k, 0.8, 2000 + s)
    out["sample_top_k_call_us"] = round((time.perf_counter() - t0) / n * 1e6, 1)
    host = np.empty(V, dtype=np.float32)
    for _ in range(20):
        host[:] = row.cpu().numpy()
    t0 = time.perf_counter()
    for _ in range(n):
        host[:] = row.cpu().numpy()
    out["reference_row_copy_us"] = round((time.perf_counter() - t0) / n * 1e6, 1)
    eng = ie.Engine(None, seed=1234, max_batch=1)
    prompt = np.random.default_rng(129).integers(0, 50257, 128).astype(np.int32)
    eng.generate_one(prompt, 8, temperature=0.8, top_k=k)
    toks, m = eng.generate_one(prompt, 256, temperature=0.8, top_k=k)
    eng.close()
    out["e2e_b1_sampled"] = {"sampling": f"top-k {k}, T 0.8, seeds 42, 43, ...", "decode_tok_s": round(m["tps"], 1),
                             "tpot_ms": round(m["tpot_ms"], 4), "ttft_ms": round(m["ttft_ms"], 2),
                             "tokens": len(toks)}
    log(f"sampler {out}")
    return out


# ------------------------------------------------------------------ HBM traffic
CALIB_BYTES = 1 << 30
# Workloads of the FETCH_SIZE / WRITE_SIZE passes, in launch order: label,
# kernel-name pattern, and for GEMVs (M, K, N).  A label's dispatches are the
# pattern's matches in launch order (one per GEMV and attention label; the
# headline GEMM's three launches are averaged).
TRAFFIC_GEMV = [("gemv_8192_m1", 1, 8192, 8192), ("gemv_8192_m16", 16, 8192, 8192),
                ("gemv_head_m1", 1, 768, 50257), ("gemv_head_m16", 16, 768, 50257),
                ("gemv_28672_m1", 1, 8192, 28672)]
TRAFFIC_M512 = (512, 768, 50257)  # (M, K, N), label gemm_m512_head


def pmc_child(ie):
    """Workload profiled by the FETCH_SIZE / WRITE_SIZE passes: a 1 GiB device
    copy (calibration: known bytes each way), three headline GEMM launches,
    one launch per TRAFFIC_GEMV shape (fresh weights) and one cfg4 ctx 8192
    fp32 attention call."""
    import torch

    src = torch.ones(CALIB_BYTES // 4, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    h = bench_headline(ie, headline_inputs(ie), 2, 1)
    del h
    torch.cuda.empty_cache()
    g = torch.Generator(device="cuda").manual_seed(9)
    for _, M, K, N in TRAFFIC_GEMV:
        W = torch.randint(-127, 128, (N, K), dtype=torch.int8, device="cuda", generator=g).view(torch.int32)
        A = torch.randint(-127, 128, (M, K), dtype=torch.int8, device="cuda", generator=g).view(torch.int32)
        sA = torch.ones(M, device="cuda")
        sB = torch.ones(N, device="cuda")
        C = torch.empty((M, N), device="cuda")
        torch.cuda.synchronize()
        ie.int8_gemm(A, W, sA, sB, ie.EPI_PLAIN, out=C)
        torch.cuda.synchronize()
        del W
    attn_case(ie, 32, 32, 8, 128, 8192, False, False, 8192, max_copies=1)
    torch.cuda.synchronize()
    # cfg2's M = 512 x 768 x 50257 GEMM (the write-dominated kernel), fresh C
    M, K, N = TRAFFIC_M512
    A = torch.randint(-127, 128, (M, K), dtype=torch.int8, device="cuda", generator=g).view(torch.int32)
    W = torch.randint(-127, 128, (N, K), dtype=torch.int8, device="cuda", generator=g).view(torch.int32)
    C = torch.empty((M, N), device="cuda")
    ie.int8_gemm(A, W, torch.ones(M, device="cuda"), torch.ones(N, device="cuda"), ie.EPI_PLAIN, out=C)
    torch.cuda.synchronize()


def _pmc_rows(counters, child_flag, extra=()):
    """Runs this script as child_flag under rocprofv3 --pmc counters; returns
    the counter rows (dicts) in dispatch order, or None."""
    import csv
    import shutil
    import subprocess
    import tempfile

    if shutil.which("rocprofv3") is None:
        return None
    with tempfile.TemporaryDirectory(dir="/tmp") as td:
        cmd = ["timeout", "-s", "KILL", "150", "rocprofv3", "--pmc", *counters, *extra, "--output-format", "csv",
               "-d", td, "-o", "run", "--", sys.executable, os.path.abspath(__file__), child_flag]
        r = subprocess.run(cmd, cwd="/tmp", env=dict(os.environ, TMPDIR="/tmp"), capture_output=True, text=True)
        found = {}
        for dp, _, fs in os.walk(td):
            for f in fs:
                if f.endswith(".csv"):
                    found[f] = os.path.join(dp, f)
        cc = [v for k, v in found.items() if k.endswith("counter_collection.csv")]
        if not cc:
            log(f"pmc pass {counters} failed rc={r.returncode}: {r.stderr[-500:]}")
            return None
        rows = list(csv.DictReader(open(cc[0])))
        kt = [v for k, v in found.items() if k.endswith("kernel_trace.csv")]
        trace = list(csv.DictReader(open(kt[0]))) if kt else []
    key = "Dispatch_Id" if rows and "Dispatch_Id" in rows[0] else None
    if key:
        rows.sort(key=lambda x: int(x[key]))
        trace.sort(key=lambda x: int(x.get(key, 0) or 0))
    return rows, trace


def measure_traffic():
    """HBM bytes per launch (FETCH_SIZE + WRITE_SIZE, KiB per dispatch, scaled
    by what the counters read for the 1 GiB calibration copy), per label."""
    out = {}
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        got = _pmc_rows([counter], "--pmc-child")
        if got is None:
            return None
        vals = {}
        gemv_i = 0
        for row in got[0]:
            if row["Counter_Name"] != counter:
                continue
            name, v = row["Kernel_Name"], float(row["Counter_Value"]) * 1024.0
            if "copy" in name.lower() or "elementwise_kernel" in name:
                vals["copy"] = max(vals.get("copy", 0.0), v)
            elif "gemm_i8_256_kernel" in name:
                vals.setdefault("gemm", []).append(v)
            elif "gemv_i8_" in name and gemv_i < len(TRAFFIC_GEMV):
                vals[TRAFFIC_GEMV[gemv_i][0]] = v
                gemv_i += 1
            elif "decode_attn_balanced_kernel" in name:
                vals["attn"] = v
            elif "gemm_i8_wide_kernel" in name:
                vals["gemm_m512_head"] = v
        if "gemm" in vals:
            vals["gemm"] = sum(vals["gemm"]) / len(vals["gemm"])
        for k, v in vals.items():
            out.setdefault(k, {})[counter] = v
    cp = out.get("copy", {})
    if not cp.get("FETCH_SIZE") or not cp.get("WRITE_SIZE"):
        return None
    f_scale = CALIB_BYTES / cp["FETCH_SIZE"]
    w_scale = CALIB_BYTES / cp["WRITE_SIZE"]
    res = {"calibration": {"copy_bytes": CALIB_BYTES, "fetch_factor": round(f_scale, 4),
                           "write_factor": round(w_scale, 4)}}
    alg = {lbl: gemm_bytes(M, N, K) for lbl, M, K, N in TRAFFIC_GEMV}
    alg["gemm"] = gemm_bytes(8192, 8192, 8192)
    alg["gemm_m512_head"] = gemm_bytes(TRAFFIC_M512[0], TRAFFIC_M512[2], TRAFFIC_M512[1])
    for k, v in out.items():
        if k != "copy" and "FETCH_SIZE" in v and "WRITE_SIZE" in v:
            fb, wb = int(v["FETCH_SIZE"] * f_scale), int(v["WRITE_SIZE"] * w_scale)
            res[k] = {"fetch_bytes": fb, "write_bytes": wb}
            if k in alg:
                res[k]["algorithmic_bytes"] = alg[k]
                res[k]["traffic_over_algorithmic"] = round((fb + wb) / alg[k], 3)
    return res


def ramp_bursts(ie):
    """Per-launch µs of the headline GEMM (HIP events around each launch):
    60 back-to-back launches on fresh operands, 30 more after 300 ms idle, 30
    into a fresh output buffer, and 30 on all-zero operands (little bit
    toggling, so little power)."""
    import torch

    Ap, Bp, sA, sB = headline_inputs(ie)
    C = torch.empty((8192, 8192), device="cuda")

    def burst(n):
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n)]
        for a, b in ev:
            a.record()
            ie.int8_gemm(Ap, Bp, sA, sB, ie.EPI_PLAIN, out=C)
            b.record()
        torch.cuda.synchronize()
        return [round(a.elapsed_time(b) * 1e3, 1) for a, b in ev]

    out = {"burst1": burst(60)}
    time.sleep(0.3)
    out["after_300ms_idle"] = burst(30)
    C = torch.empty((8192, 8192), device="cuda")
    out["fresh_output"] = burst(30)
    Ap.zero_()
    Bp.zero_()
    torch.cuda.synchronize()
    out["zero_operands"] = burst(30)
    print(json.dumps(out), flush=True)


def mfma_child(ie):
    """Workload of the MFMA-utilisation pass: the headline GEMM, 50 launches
    to bring the clock up, then 20 measured ones."""
    import torch

    inp = headline_inputs(ie)
    bench_headline(ie, inp, 20, 50)
    torch.cuda.synchronize()


def measure_mfma_util(n_last=20, simds=1024, xcds=8):
    """MfmaUtil of the headline kernel as rocprofv3 defines it
    (counter_defs.yaml: SQ_VALU_MFMA_BUSY_CYCLES summed / (GRBM_GUI_ACTIVE per
    XCD x SIMD_NUM)), the clock it implies, over the last n_last launches.
    GRBM_GUI_ACTIVE is reported summed over the XCDs, so it is divided by
    their count; the duration comes from the same run's kernel trace."""
    got = _pmc_rows(["SQ_VALU_MFMA_BUSY_CYCLES", "GRBM_GUI_ACTIVE"], "--mfma-child", extra=["--kernel-trace"])
    if got is None:
        return None
    rows, trace = got
    busy, grbm = {}, {}
    for row in rows:
        if "gemm_i8_256_kernel" not in row["Kernel_Name"]:
            continue
        did = row.get("Dispatch_Id", str(len(busy)))
        tgt = busy if row["Counter_Name"] == "SQ_VALU_MFMA_BUSY_CYCLES" else grbm
        tgt[did] = tgt.get(did, 0.0) + float(row["Counter_Value"])
    ids = sorted(set(busy) & set(grbm), key=int)[-n_last:]
    if not ids:
        return None
    dur = {}
    for t in trace:
        if "gemm_i8_256_kernel" in t.get("Kernel_Name", "") and t.get("Dispatch_Id") in ids:
            dur[t["Dispatch_Id"]] = int(t["End_Timestamp"]) - int(t["Start_Timestamp"])
    b = sum(busy[i] for i in ids) / len(ids)
    gx = sum(grbm[i] for i in ids) / len(ids) / xcds
    r = {"mfma_util": round(b / (gx * simds), 4), "sq_valu_mfma_busy_cycles": int(b),
         "grbm_gui_active_per_xcd": int(gx), "launches": len(ids)}
    if dur:
        ns = sum(dur.values()) / len(dur)
        r["kernel_us"] = round(ns / 1e3, 2)
        r["clock_mhz"] = round(gx / ns * 1e3, 1)
        r["tops_at_this_clock_peak"] = round(5000.0 * (gx / ns * 1e3) / 2400.0, 1)
    return r


# ------------------------------------------------------------------ CPU baseline
def cpu_baseline(inputs, budget_s=12.0):
    import numpy as np
    import torch

    from oracle import orc

    Ap, Bp, sA, sB = inputs
    N, K = Bp.shape[0], Bp.shape[1] * 4
    B_h = Bp.cpu().numpy()
    sB_h = sB.cpu().numpy()
    threads = min(os.cpu_count() or 1, int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1)))
    orc.set_threads(threads)
    rows = 16
    A_h = Ap[:rows].cpu().numpy()
    t0 = time.perf_counter()
    orc.gemm(A_h, B_h, sA[:rows].cpu().numpy(), sB_h, 0)
    est = (time.perf_counter() - t0) / rows
    rows = int(max(16, min(Ap.shape[0], budget_s / max(est, 1e-9))))
    A_h = Ap[:rows].cpu().numpy()
    sA_h = sA[:rows].cpu().numpy()
    t0 = time.perf_counter()
    C = orc.gemm(A_h, B_h, sA_h, sB_h, 0)
    dt = time.perf_counter() - t0
    tops = 2.0 * rows * N * K / dt / 1e12
    del C
    return {"value": round(tops, 5), "unit": "TOP/s", "cores": threads, "kind": "port",
            "sample": f"{rows} of 8192 rows of the 8192^3 INT8 GEMM (Plain), int32 triple loop "
                      f"+ dequant, OpenMP over rows, {dt:.1f} s"}


def _cpu_threads():
    return min(os.cpu_count() or 1, int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1)))


def _cpu_model():
    import platform
    import subprocess

    try:
        for ln in subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout.splitlines():
            if ln.startswith("Model name:"):
                return ln.split(":", 1)[1].strip()
    except Exception:  # noqa: BLE001 - informational only
        pass
    return platform.processor() or "unknown"


def _attn_workload(B, H_q, H_kv, d, ctx, uniform, seed):
    """Host paged cache for the CPU baselines: U(-1,1) data, shuffled block
    table, lengths ctx (uniform) or U[ctx/2, ctx]."""
    import numpy as np

    bs = 16
    r = np.random.default_rng(seed)
    lens = np.full(B, ctx, np.int32) if uniform else r.integers(ctx // 2, ctx + 1, B).astype(np.int32)
    nbs = (lens + bs - 1) // bs
    P, nbps = int(nbs.sum()), int(nbs.max())
    kc = r.random((P, bs, H_kv, d), dtype=np.float32) * 2 - 1
    vc = r.random((P, bs, H_kv, d), dtype=np.float32) * 2 - 1
    perm = r.permutation(P).astype(np.int32)
    table = np.zeros((B, nbps), np.int32)
    off = 0
    for b in range(B):
        table[b, : nbs[b]] = perm[off: off + nbs[b]]
        off += int(nbs[b])
    Q = r.random((B, H_q, d), dtype=np.float32) * 2 - 1
    return Q, kc, vc, table, lens


def _attn_bytes(lens, H_q, H_kv, d, esz=4):
    nb = int(((lens + 15) // 16).sum())
    return int(lens.sum()) * H_kv * d * 2 * esz + 2 * len(lens) * H_q * d * 4 + 4 * nb + 4 * len(lens)


def cpu_baseline_attn(B=32, ctx=8192, seed=8192, budget_s=8.0):
    """The oracle's decode attention (the reference's split-K algorithm in fp64,
    tests/test_paged_attention.cu:138-179 as the BASELINE plan restates it),
    OpenMP over (sequence, query head), on the cfg4 ctx 8192 fp32 workload
    (same shapes and length law; U(-1,1) data), repeated until budget_s of
    timed work."""
    from oracle import orc

    H_q, H_kv, d, bs = 32, 8, 128, 16
    Q, kc, vc, table, lens = _attn_workload(B, H_q, H_kv, d, ctx, False, seed)
    threads = _cpu_threads()
    orc.set_threads(threads)
    reps, t0 = 0, time.perf_counter()
    while True:
        orc.decode_attn(Q, kc, vc, table, lens, int(lens.max()), bs, H_kv)
        reps += 1
        dt = time.perf_counter() - t0
        if dt >= budget_s:
            break
    alg = _attn_bytes(lens, H_q, H_kv, d)
    return {"value": round(alg * reps / dt / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"decode attention cfg4 ctx {ctx} fp32, {B} sequences (Σctx {int(lens.sum())}), the "
                      f"oracle's fp64 split-K restatement, OpenMP over (sequence, head), {reps} calls in {dt:.1f} s"}


def _cpu_time(fn, budget_s=1.5, min_runs=5):
    """Median of >= min_runs calls after one warm-up, or of as many as budget_s
    allows (at least one)."""
    fn()
    ts, start = [], time.perf_counter()
    while len(ts) < min_runs:
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
        if time.perf_counter() - start > budget_s:
            break
    ts.sort()
    return ts[len(ts) // 2], len(ts)


def cpu_baseline_detail():
    """BASELINE's CPU plan: the oracle (C, -O3 x86-64-v3, OpenMP) on cfg1
    512^3, the GPT-2 weight shapes at M = 1, 4, 16, cfg3 and cfg4 at ctx
    4096 / 8192, each at 1 thread and at all threads; median of >= 5 runs
    after a warm-up (fewer, stated, where one run is long)."""
    import numpy as np

    from oracle import orc

    T = _cpu_threads()
    out = {"cpu_model": _cpu_model(), "nproc": os.cpu_count(), "threads_all": T, "kind": "port",
           "gemm": [], "decode_attn": []}
    r = np.random.default_rng(512)
    A = r.standard_normal((512, 512)).astype(np.float32)
    BT = r.standard_normal((512, 512)).astype(np.float32)
    Ap, sA = orc.quantize(A)
    Bp, sB = orc.quantize(BT)
    for th in (1, T):
        orc.set_threads(th)
        t, n = _cpu_time(lambda: orc.gemm(Ap, Bp, sA, sB, 0))
        out["gemm"].append({"workload": "cfg1 M=N=K=512", "threads": th, "ms": round(t * 1e3, 3),
                            "TOPs": round(2 * 512 ** 3 / t / 1e12, 5), "runs": n})
    for K, N in [(768, 2304), (768, 768), (768, 3072), (3072, 768), (768, 50257)]:
        W = r.integers(-127, 128, (N, K), dtype=np.int8).view(np.int32)
        sW = (r.random(N, dtype=np.float32) * 0.01).astype(np.float32)
        for M in (1, 4, 16):
            X = r.integers(-127, 128, (M, K), dtype=np.int8).view(np.int32)
            sX = np.ones(M, np.float32)
            for th in (1, T):
                orc.set_threads(th)
                t, n = _cpu_time(lambda: orc.gemm(X, W, sX, sW, 0), budget_s=1.0)
                out["gemm"].append({"workload": f"GPT-2 M={M} K={K} N={N}", "threads": th,
                                    "us": round(t * 1e6, 1), "GBps": round(gemm_bytes(M, N, K) / t / 1e9, 3),
                                    "runs": n})
    orc.set_threads(T)
    for name, (B, H_q, H_kv, d, ctx, uni) in (("cfg3 MHA ctx 1024", (8, 12, 12, 64, 1024, True)),
                                              ("cfg4 GQA ctx 4096", (32, 32, 8, 128, 4096, False)),
                                              ("cfg4 GQA ctx 8192", (32, 32, 8, 128, 8192, False))):
        Q, kc, vc, table, lens = _attn_workload(B, H_q, H_kv, d, ctx, uni, ctx + B)
        for th in (1, T):
            orc.set_threads(th)
            # one thread: the first two sequences of cfg4 (a bounded sample)
            nb = B if (th == T or B <= 8) else 2
            q, tb, ln = Q[:nb], table[:nb], lens[:nb]
            t, n = _cpu_time(lambda: orc.decode_attn(q, kc, vc, tb, ln, int(ln.max()), 16, H_kv), budget_s=3.0)
            out["decode_attn"].append({"workload": name, "threads": th, "sequences": nb, "ms": round(t * 1e3, 2),
                                       "GBps": round(_attn_bytes(ln, H_q, H_kv, d) / t / 1e9, 3), "runs": n})
        del Q, kc, vc
    log(f"cpu detail {out}")
    return out


def main():
    args = parse()
    if args.pmc_child or args.mfma_child or args.ramp:
        import ie_amd as ie

        ie.load()
        ie.check("ie_init")
        (pmc_child if args.pmc_child else mfma_child if args.mfma_child else ramp_bursts)(ie)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported "
              "(this build runs on a single MI355X)", file=sys.stderr)
        sys.exit(2)
    skip = set(s for s in args.skip.split(",") if s)
    import torch

    import ie_amd as ie

    ie.load()
    ie.check("ie_init")
    torch.cuda.synchronize()
    log("headline operands: 8192^3 INT8 GEMM, quantized untimed")
    inputs = headline_inputs(ie)
    legs = {}
    if not args.only_headline:
        if "gemv" not in skip:
            legs["gemv"] = bench_gemv(ie)
        if "gemm512" not in skip:
            legs["gemm_m512"] = bench_gemm512(ie)
        if "ref" not in skip:
            legs["ref_shapes"] = bench_ref_shapes(ie)
        if "attn" not in skip:
            legs["decode_attn"] = bench_attn(ie)
        if "e2e" not in skip:
            legs["e2e_gpt2"] = bench_e2e(ie)
        if "sampler" not in skip:
            legs["sampler"] = bench_sampler(ie)
    vendor = None
    if "vendor" not in skip:
        vendor = bench_vendor(ie, inputs, args.steps, args.warmup)
        log(f"vendor {vendor}")
    log("headline: 8192^3 INT8 GEMM")
    h = bench_headline(ie, inputs, args.steps, args.warmup)
    res = {
        "metric": METRIC,
        "value": round(h["value"], 2),
        "unit": "TOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(h["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "i8 (int32 accumulate, fp32 dequant)",
        "data": "synthetic: fp32 N(0,1) operands from a seed, quantized per row by the library (untimed)",
        "config": {"workload": "INT8 GEMM M=N=K=8192, NT layout, Plain epilogue (BASELINE configs[1])",
                   "M": 8192, "N": 8192, "K": 8192, "parallelism": "none (1 GPU)"},
        "roofline": roof(h["kernel_tops"], PEAK_I8_TOPS, "TOP/s", "mfma"),
        "headline_order": ("operands made first; the other GPU legs; hipBLASLt's GEMM on the same operands "
                           "(>= 50 warm-up launches, then K timed); then this kernel's W warm-up and K timed "
                           "launches" if vendor else "warm-up and timed launches right after the operands are made"),
    }
    if vendor:
        res["vendor_gemm"] = vendor
    res.update(legs)
    if "gemv" in legs:
        rows = {(r["M"], r["K"], r["N"]): r for r in legs["gemv"]}
        dom = rows[(1, 8192, 8192)]
        res["gemv_roofline"] = roof(dom["GBps"], PEAK_HBM_GBS, "GB/s", "hbm")
        res["gemv_roofline"]["kernel"] = "decode GEMV M=1 K=N=8192 (BASELINE configs[1], 67 MB of weights)"
        res["gemv_roofline"]["rows"] = [
            {"shape": f"M={M} K={K} N={N}", "frac": rows[(M, K, N)]["frac_hbm"],
             "baseline_shape": N != 28672}
            for M, K, N in [(1, 8192, 8192), (4, 8192, 8192), (16, 8192, 8192), (1, 768, 50257), (4, 768, 50257),
                            (16, 768, 50257), (1, 8192, 28672), (4, 8192, 28672), (16, 8192, 28672)]]
    if "decode_attn" in legs:
        c8 = [r for r in legs["decode_attn"] if r["ctx"] == 8192 and r["kv"] == "fp32" and r["H_q"] == 32][0]
        res["decode_attn_roofline"] = roof(c8["GBps"], PEAK_HBM_GBS, "GB/s", "hbm")
        res["decode_attn_roofline"]["kernel"] = "decode_attn cfg4 ctx 8192 fp32"
    if "cpu" not in skip:
        log("cpu baseline")
        res["cpu_baseline"] = cpu_baseline(inputs)
        res["cpu_baseline"]["cpu_model"] = _cpu_model()
        res["cpu_baseline_attn"] = cpu_baseline_attn()
        log(f"cpu attention {res['cpu_baseline_attn']}")
        res["cpu_baseline_detail"] = cpu_baseline_detail()
    if not args.no_traffic:
        if "mfma" not in skip:
            log("MFMA utilisation (rocprofv3 SQ_VALU_MFMA_BUSY_CYCLES / GRBM_GUI_ACTIVE pass)")
            res["roofline"]["mfma"] = measure_mfma_util()
            log(f"mfma {res['roofline']['mfma']}")
        log("traffic (rocprofv3 FETCH_SIZE / WRITE_SIZE passes)")
        t = measure_traffic()
        res["traffic_detail"] = t

        def traffic(k):
            return t[k]["fetch_bytes"] + t[k]["write_bytes"] if t and k in t else None

        res["roofline"]["traffic"] = traffic("gemm")
        if "gemv_roofline" in res:
            res["gemv_roofline"]["traffic"] = traffic("gemv_8192_m1")
        if "decode_attn_roofline" in res:
            res["decode_attn_roofline"]["traffic"] = traffic("attn")
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
