#!/usr/bin/env python3
"""Measures the INT8 decode hot path on one MI355X.

Headline (`value`): INT8 GEMM throughput at M=N=K=8192 (Plain epilogue, int32
accumulate, fp32 out) in TOP/s, one "step" = one GEMM launch over resident
inputs.  The same JSON line carries:
  roofline      the 8192^3 kernel against the dense i8 MFMA peak (5.0 POP/s)
  vendor_gemm   hipBLASLt (torch._int_mm) on the same operands, same box
  gemv          decode-M (1, 4, 16) GEMMs on the GPT-2 weight shapes, the LM
                head shape and 8192x8192, in GB/s of algorithmic bytes against
                HBM (8 TB/s), weights rotated through >= 1 GiB of copies so the
                256 MiB MALL cannot serve them
  gemm_m512     the GPT-2 shapes at M = 512 (prefill-sized), TOP/s
  decode_attn   split-K paged decode attention, BASELINE cfg3 (MHA) and cfg4
                (GQA, ctx 4096/8192/32768, fp32 and bf16 KV), GB/s of
                algorithmic bytes against HBM
  e2e_gpt2      GPT-2 Small decode tok/s (BASELINE cfg5), batch 1 and 16
  sampler       top-k sampling: device selection kernel, one sample_top_k
                call, the reference's whole-row copy, sampled decode at batch 1
  cpu_baseline  the C oracle (oracle/liborc.so) on a bounded sample of the
                8192^3 GEMM, on this host's cores; cpu_baseline_attn the same
                for decode attention cfg4 ctx 8192 fp32
  traffic       HBM bytes per launch of the dominant kernels (rocprofv3
                FETCH_SIZE / WRITE_SIZE passes, calibrated on a 1 GiB copy)
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
    # The first ~30 back-to-back 8192^3 launches run up to ~20% slower than the
    # steady state (measured 1772 TOP/s over launches 4-13, 2160 from ~36 on),
    # so the default warm-up is 50 launches (~30 ms).
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--skip", default="", help="comma list of vendor,gemv,gemm512,attn,cpu,e2e,sampler")
    ap.add_argument("--only-headline", action="store_true")
    ap.add_argument("--no-traffic", action="store_true", help="skip the rocprofv3 FETCH/WRITE passes")
    ap.add_argument("--pmc-child", action="store_true", help=argparse.SUPPRESS)
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
def bench_headline(ie, steps, warmup):
    import torch

    M = N = K = 8192
    # BASELINE recipe: A, B fp32 ~ N(0,1) from a seed; A quantized per row and
    # B per column (= per row of B^T) with the library's quantizer (untimed).
    g = torch.Generator(device="cuda").manual_seed(42)
    Af = torch.randn((M, K), device="cuda", generator=g)
    Ap, sA = ie.quantize(Af)
    del Af
    BTf = torch.randn((N, K), device="cuda", generator=g)
    Bp, sB = ie.quantize(BTf)
    del BTf
    torch.cuda.empty_cache()
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
        "inputs": (Ap, Bp, sA, sB),
    }


def bench_vendor(ie, inputs, steps, warmup):
    """hipBLASLt's int8 GEMM (torch._int_mm) on the headline's own quantized
    operands, timed the same way: a same-box reference point for the
    power-limited MFMA rate.  It returns int32 with no dequant epilogue (our
    kernel also writes the fp32 dequant), so it does slightly less work."""
    import torch

    Ap, Bp, _, _ = inputs
    M, K = Ap.shape[0], Ap.shape[1] * 4
    N = Bp.shape[0]
    A8 = Ap.view(torch.int8).view(M, K)
    B8 = Bp.view(torch.int8).view(N, K)
    try:
        for _ in range(warmup):
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
        B = torch.randint(-127, 128, (N, K), dtype=torch.int8, device="cuda", generator=g).view(torch.int32)
        sA = torch.rand(M, device="cuda", generator=g)
        sB = torch.rand(N, device="cuda", generator=g)
        C = torch.empty((M, N), dtype=torch.float32, device="cuda")
        ms = graph_time(lambda i: ie.int8_gemm(A, B, sA, sB, ie.EPI_PLAIN, out=C), 20)
        tops = 2.0 * M * N * K / (ms * 1e-3) / 1e12
        out.append({"M": M, "K": K, "N": N, "us": round(ms * 1e3, 2), "TOPs": round(tops, 1)})
        log(f"gemm M=512 K={K} N={N}: {ms * 1e3:.2f} us {tops:.1f} TOP/s")
    return out


# ------------------------------------------------------------------ attention
def attn_case(ie, B, H_q, H_kv, d, ctx, kv_bf16, uniform, seed):
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
    return out


# ------------------------------------------------------------------ end to end
def bench_e2e(ie):
    """GPT-2 Small random-init N(0, 0.02), INT8 per-row
    linears (W8A8 as the reference engine), paged KV, prompt of 128 random ids,
    greedy decode of 256 tokens at batch 1 and 16.  tok/s counts decode steps
    only (src/gpt2_engine.cu:754); MBU = bytes streamed per step x steps/s / 8 TB/s.
    ttft_ms = prompt prefill + first token; also reported with the prompt fed
    through decode steps."""
    import numpy as np

    out = []
    rng = np.random.default_rng(128)
    # fused step (5 launches per layer) for both LM heads; the unfused step
    # (every operation through the public C ABI) for comparison
    for head_i8, fuse in ((False, True), (True, True), (False, False)):
        eng = ie.Engine(None, seed=1234, max_batch=16, int8_lm_head=head_i8, fuse=fuse)
        for B in (1, 16):
            prompts = rng.integers(0, 50257, (B, 128)).astype(np.int32)
            eng.generate(prompts, 8, ignore_eos=True)  # warm up (graph capture)
            toks, m = eng.generate(prompts, 256, ignore_eos=True)
            r = {"batch": B, "lm_head": "int8" if head_i8 else "fp32 (reference)",
                 "step": "fused" if fuse else "unfused", "prompt": "prefill",
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
TRAFFIC_KERNELS = {"gemm": "gemm_i8_256_kernel", "gemv": "gemv_i8_parted_kernel",
                   "attn": "decode_attn_balanced_kernel"}


def pmc_child(ie):
    """Workload profiled by the FETCH_SIZE / WRITE_SIZE passes: a 1 GiB device
    copy (calibration: known bytes each way), then one launch of each dominant
    kernel on its bench shape."""
    import torch

    src = torch.ones(CALIB_BYTES // 4, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    h = bench_headline(ie, 2, 1)
    del h
    g = torch.Generator(device="cuda").manual_seed(9)
    K, N = 8192, 28672
    W = torch.randint(-127, 128, (N, K), dtype=torch.int8, device="cuda", generator=g).view(torch.int32)
    A = torch.randint(-127, 128, (1, K), dtype=torch.int8, device="cuda", generator=g).view(torch.int32)
    sA = torch.ones(1, device="cuda")
    sB = torch.ones(N, device="cuda")
    ie.int8_gemm(A, W, sA, sB, ie.EPI_PLAIN)
    torch.cuda.synchronize()
    del W
    attn_case(ie, 32, 32, 8, 128, 8192, False, False, 8192)
    torch.cuda.synchronize()


def measure_traffic():
    """Runs the PMC passes in child processes; returns per-kernel HBM bytes per
    launch (FETCH_SIZE + WRITE_SIZE, KiB, scaled by what the counters read for
    the calibration copy) or None if rocprofv3 is unavailable."""
    import csv
    import shutil
    import subprocess
    import tempfile

    if shutil.which("rocprofv3") is None:
        return None
    out = {}
    with tempfile.TemporaryDirectory(dir="/tmp") as td:
        for counter in ("FETCH_SIZE", "WRITE_SIZE"):
            d = os.path.join(td, counter)
            cmd = ["timeout", "-s", "KILL", "120", "rocprofv3", "--pmc", counter, "--output-format", "csv",
                   "-d", d, "-o", "run", "--", sys.executable, os.path.abspath(__file__), "--pmc-child"]
            r = subprocess.run(cmd, cwd="/tmp", env=dict(os.environ, TMPDIR="/tmp"), capture_output=True,
                               text=True)
            files = [os.path.join(dp, f) for dp, _, fs in os.walk(d) for f in fs
                     if f.endswith("counter_collection.csv")]
            if r.returncode != 0 and not files:
                log(f"traffic pass {counter} failed rc={r.returncode}: {r.stderr[-500:]}")
                return None
            vals = {}
            for row in csv.DictReader(open(files[0])):
                if row["Counter_Name"] != counter:
                    continue
                name = row["Kernel_Name"]
                key = "copy" if "copy" in name.lower() or "elementwise_kernel" in name else None
                for k, pat in TRAFFIC_KERNELS.items():
                    if pat in name:
                        key = k
                if key:
                    vals.setdefault(key, []).append(float(row["Counter_Value"]) * 1024.0)
            for k, v in vals.items():
                # the calibration copy is the largest "copy"-like dispatch
                out.setdefault(k, {})[counter] = max(v) if k == "copy" else sum(v) / len(v)
    cp = out.get("copy", {})
    if not cp.get("FETCH_SIZE") or not cp.get("WRITE_SIZE"):
        return None
    f_scale = CALIB_BYTES / cp["FETCH_SIZE"]
    w_scale = CALIB_BYTES / cp["WRITE_SIZE"]
    res = {"calibration": {"copy_bytes": CALIB_BYTES, "fetch_factor": round(f_scale, 4),
                           "write_factor": round(w_scale, 4)}}
    for k in TRAFFIC_KERNELS:
        if k in out and "FETCH_SIZE" in out[k] and "WRITE_SIZE" in out[k]:
            res[k] = {"fetch_bytes": int(out[k]["FETCH_SIZE"] * f_scale),
                      "write_bytes": int(out[k]["WRITE_SIZE"] * w_scale)}
    return res


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


def cpu_baseline_attn(B=32, ctx=8192, seed=8192, budget_s=8.0):
    """The oracle's decode attention (the reference's split-K algorithm in fp64,
    tests/test_paged_attention.cu:138-179 as the BASELINE plan restates it),
    OpenMP over (sequence, query head), on the cfg4 ctx 8192 fp32 workload
    (same shapes and length law; U(-1,1) data), repeated until budget_s of
    timed work."""
    import numpy as np

    from oracle import orc

    H_q, H_kv, d, bs = 32, 8, 128, 16
    r = np.random.default_rng(seed)
    lens = r.integers(ctx // 2, ctx + 1, B).astype(np.int32)
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
    threads = min(os.cpu_count() or 1, int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1)))
    orc.set_threads(threads)
    reps, t0 = 0, time.perf_counter()
    while True:
        orc.decode_attn(Q, kc, vc, table, lens, int(lens.max()), bs, H_kv)
        reps += 1
        dt = time.perf_counter() - t0
        if dt >= budget_s:
            break
    alg = int(lens.sum()) * H_kv * d * 2 * 4 + 2 * B * H_q * d * 4 + 4 * P + 4 * B
    return {"value": round(alg * reps / dt / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"decode attention cfg4 ctx {ctx} fp32, {B} sequences (Σctx {int(lens.sum())}), the "
                      f"oracle's fp64 split-K restatement, OpenMP over (sequence, head), {reps} calls in {dt:.1f} s"}


def main():
    args = parse()
    if args.pmc_child:
        import ie_amd as ie

        ie.load()
        pmc_child(ie)
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
    log("headline: 8192^3 INT8 GEMM")
    h = bench_headline(ie, args.steps, args.warmup)
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
    }
    if "vendor" not in skip:
        res["vendor_gemm"] = bench_vendor(ie, h["inputs"], args.steps, args.warmup)
        log(f"vendor {res['vendor_gemm']}")
    if not args.only_headline:
        if "gemv" not in skip:
            res["gemv"] = bench_gemv(ie)
            dom = [r for r in res["gemv"] if (r["M"], r["K"], r["N"]) == (1, 8192, 28672)][0]
            res["gemv_roofline"] = roof(dom["GBps"], PEAK_HBM_GBS, "GB/s", "hbm")
            res["gemv_roofline"]["kernel"] = "gemv M=1 K=8192 N=28672 (decode GEMV, 235 MB of weights)"
        if "gemm512" not in skip:
            res["gemm_m512"] = bench_gemm512(ie)
        if "attn" not in skip:
            res["decode_attn"] = bench_attn(ie)
            c8 = [r for r in res["decode_attn"] if r["ctx"] == 8192 and r["kv"] == "fp32"][0]
            res["decode_attn_roofline"] = roof(c8["GBps"], PEAK_HBM_GBS, "GB/s", "hbm")
            res["decode_attn_roofline"]["kernel"] = "decode_attn cfg4 ctx 8192 fp32"
        if "e2e" not in skip:
            res["e2e_gpt2"] = bench_e2e(ie)
        if "sampler" not in skip:
            res["sampler"] = bench_sampler(ie)
    if "cpu" not in skip:
        log("cpu baseline")
        res["cpu_baseline"] = cpu_baseline(h["inputs"])
        res["cpu_baseline_attn"] = cpu_baseline_attn()
        log(f"cpu attention {res['cpu_baseline_attn']}")
    if not args.no_traffic:
        log("traffic (rocprofv3 FETCH_SIZE / WRITE_SIZE passes)")
        t = measure_traffic()
        res["traffic_detail"] = t
        if t and "gemm" in t:
            res["roofline"]["traffic"] = t["gemm"]["fetch_bytes"] + t["gemm"]["write_bytes"]
        if t and "gemv" in t and "gemv_roofline" in res:
            res["gemv_roofline"]["traffic"] = t["gemv"]["fetch_bytes"] + t["gemv"]["write_bytes"]
        if t and "attn" in t and "decode_attn_roofline" in res:
            res["decode_attn_roofline"]["traffic"] = t["attn"]["fetch_bytes"] + t["attn"]["write_bytes"]
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
