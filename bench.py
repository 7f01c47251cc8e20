#!/usr/bin/env python3
"""Benchmark of the hot path on one MI355X: prints ONE JSON line.

Headline: f16 GEMM C = A . B^T, M = N = K = 8192,
A [M x K] and B [N x K] row-major f16 uniform in [-1, 1) from a seeded PRNG,
fp32 accumulation, f16 row-major C.  One "step" = one launch of the GEMM over
inputs already resident in HBM.  `value` = 2*M*N*K / mean step time
(TFLOP/s); the roofline block sets the same rate against the dense f16 MFMA
peak.  Beside it: the flash-attention forward of configs[3] (B4 H32 S4096
D128 f16, non-causal; FLOPs 4*B*H*S^2*D as the reference counts them,
wave-fa-gfx950-runner.cpp:465-467) and the CPU baseline -- the oracle's
multithreaded C++ GEMM timed on a bounded sample of output rows of the same
workload (the whole problem when it fits the CPU budget) on this host's cores.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu] [--no-fa]
                    [--no-ref-compare]

Secondary lines also run the same kernels on the input mode and shape of the
reference's own published figures (rand_int GEMM inputs; the B2 H64 S8192
bf16 attention profile; the 4096x4096x32768 MXFP4 profile) next to those
figures, for comparison.
"""

from __future__ import annotations

import argparse
import importlib
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

MFMA_PEAK_TFLOPS = 2516.6   # MI355X dense f16/bf16: 256 CU x 2.4 GHz x 4096
FP4_PEAK_TFLOPS = 10066.3  # MI355X dense fp4 MFMA: 256 CU x 2.4 GHz x 16384
FP8_PEAK_TFLOPS = 5033.2    # MI355X dense fp8: twice the f16 rate
HBM_PEAK_GBS = 8000.0
PROFILE_TRAFFIC = os.path.join(ROOT, "profiles", "gemm_f16_8192_traffic.txt")


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def read_traffic():
    """HBM bytes per GEMM launch from the committed rocprofv3 --pmc summary
    (line `traffic_bytes_per_launch: N`), or None."""
    try:
        with open(PROFILE_TRAFFIC) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return float(line.split(":", 1)[1])
    except OSError:
        pass
    return None


# The GPU lowers its clock while idle and takes a few tens of milliseconds of
# sustained load to ramp back: with 5 warmup launches (4 ms) the first timed
# launches of a 0.9 ms kernel ran 10-15 % slower than steady state on the
# same box (measured in one process: 1206 vs 1330 TFLOP/s for the GEMM, 928
# vs 1070 for the FA forward; torch vs raw hipMalloc buffers made no
# difference).  So warmup is `warmup` launches and then at least
# WARMUP_SECONDS of back-to-back launches.
WARMUP_SECONDS = 0.5


def time_launches(fn, steps, warmup, torch, warm_seconds=WARMUP_SECONDS):
    """Mean ms per launch over `steps` back-to-back launches, timed with HIP
    events on the current stream (the stream the kernels are launched on),
    after `warmup` launches and at least `warm_seconds` of untimed load."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < warm_seconds:
        for _ in range(4):
            fn()
        torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        fn()
    stop.record()
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / steps


def host_cpu():
    """The host's CPU model and core counts (for the CPU-baseline record)."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"cpu_model": model, "logical_cpus": os.cpu_count(),
            "affinity_cpus": len(os.sched_getaffinity(0))}


# Host threads for the CPU baseline: the affinity mask, capped at the CPU
# share a one-GPU job gets on the GPU boxes (16), whatever nproc shows.
CPU_THREADS_CAP = 16


def cpu_baseline(a_bits, b_bits, M, N, K, budget_s):
    """Oracle GEMM (C++, fp32 accumulate, the reference's float arithmetic)
    on this host's allowed threads: the whole M x N x K problem when three
    runs of it fit in budget_s, else a sample of whole 32-row blocks (one
    block per thread and more) of the same problem.  A run = widening and
    transposing B once (oracle gemm_prepare_bt) + the rows; for a sample the
    preparation is charged per row (its time x rows / M), as it is shared by
    all M rows of the whole problem.  Median of three runs."""
    from oracle import oracle
    threads = max(1, min(len(os.sched_getaffinity(0)), CPU_THREADS_CAP))
    t0 = time.perf_counter()
    bt = oracle.gemm_prepare_bt(b_bits, oracle.F16, threads=threads)
    t_prep = time.perf_counter() - t0
    unit = 32 * threads  # one 32-row block per thread
    out = np.zeros((M, N), dtype=np.float32)  # touched once, reused by every run
    t0 = time.perf_counter()
    oracle.gemm_nt_rows_bt(a_bits, bt, 0, unit, oracle.F16, threads=threads, out=out[:unit])
    per_row = (time.perf_counter() - t0) / unit
    whole = t_prep + per_row * M
    runs = []
    if 3 * whole <= budget_s:
        rows = M
        for _ in range(3):
            t0 = time.perf_counter()
            bt = oracle.gemm_prepare_bt(b_bits, oracle.F16, threads=threads)
            oracle.gemm_nt_rows_bt(a_bits, bt, 0, M, oracle.F16, threads=threads, out=out)
            runs.append(time.perf_counter() - t0)
        sample = f"the whole {M}x{N}x{K} f16 GEMM (B prepared inside each run)"
    else:
        rows = int((budget_s / 3 - t_prep) / per_row) // unit * unit
        rows = max(unit, min(M, rows))
        for _ in range(3):
            t0 = time.perf_counter()
            oracle.gemm_nt_rows_bt(a_bits, bt, 0, rows, oracle.F16, threads=threads,
                                   out=out[:rows])
            runs.append(time.perf_counter() - t0 + t_prep * rows / M)
        sample = (f"rows 0..{rows - 1} of C (={rows}x{N}x{K}) of the {M}x{N}x{K} f16 GEMM, "
                  f"B preparation ({t_prep:.2f} s) charged per row")
    dt = sorted(runs)[1]
    del out, bt
    return {"value": round(2.0 * rows * N * K / dt / 1e12, 6), "unit": "TFLOP/s",
            "cores": threads, "kind": "port",
            "sample": f"{sample}, median of 3 runs ({', '.join(f'{r:.2f}' for r in runs)} s), "
                      f"oracle/oracle.cpp gemm_prepare_bt + gemm_nt_rows_bt; probe-estimated "
                      f"whole problem {whole:.1f} s",
            "host": host_cpu()}


def cpu_reference_path(M, N, K, budget_s):
    """The reference runner's own CPU path (computeExpectedElement, scalar
    float accumulation; wave-matmul-calibrate-runner.cpp:1586-1597), compiled
    from the reference sources into oracle/_ref by oracle/Makefile, timed on
    a few rows of the same 8192^3 f16 problem (its own bucket inputs, which
    it generates for all of B first; generation is excluded from the timing
    by subtracting a zero-row call)."""
    import ctypes
    path = os.path.join(ROOT, "oracle", "_ref", "libref_matmul.so")
    if not os.path.exists(path):
        return None
    lib = ctypes.CDLL(path)
    f = lib.ref_gemm_expected
    f.argtypes = [ctypes.c_int] * 7 + [ctypes.c_void_p]
    f.restype = None
    rows = 1
    out = np.empty((64, N), dtype=np.float64)
    t0 = time.perf_counter()
    f(0, N, K, 1, 7, 0, 1, out.ctypes.data)  # input generation only
    gen = time.perf_counter() - t0
    t0 = time.perf_counter()
    f(rows, N, K, 1, 7, 0, 1, out.ctypes.data)
    dt = max(time.perf_counter() - t0 - gen, 1e-6)
    rows = int(max(1, min(64, rows * budget_s / dt)))
    t0 = time.perf_counter()
    f(rows, N, K, 1, 7, 0, 1, out.ctypes.data)
    dt = max(time.perf_counter() - t0 - gen, 1e-6)
    return {"value": round(2.0 * rows * N * K / dt / 1e12, 6), "unit": "TFLOP/s",
            "cores": 1, "kind": "reference",
            "sample": f"rows 0..{rows - 1} (={rows}x{N}x{K}) through the reference runner's "
                      f"computeExpectedElement, {dt:.1f} s excluding input generation"}


def rand_int_operand(rows, k, stream, torch):
    """The reference runner's rand_int inputs (hipBLASLt-style integers in
    [-2, 2]; wave-matmul-calibrate-runner.cpp:700-706, sign flip of B on
    even (row ^ col) :1176-1183), as an f16 tensor on the host."""
    idx = np.arange(rows * k, dtype=np.uint64)
    s = idx * np.uint64(1664525) + np.uint64(1013904223)
    for _ in range(3):
        s = s ^ (s << np.uint64(13)) ^ (s >> np.uint64(17)) ^ (s << np.uint64(5))
    v = (s.astype(np.uint32) % np.uint32(5)).astype(np.float32) - 2.0
    if stream == 1:
        flip = ((idx // np.uint64(k)) ^ (idx % np.uint64(k))) & np.uint64(1) == 0
        v[flip] = -v[flip]
    return torch.from_numpy(v.reshape(rows, k)).to(torch.float16)


def vendor_lines(torch, dev, a, b, steps):
    """The vendor libraries on the same box and inputs, for scale: hipBLASLt
    (torch.matmul, C = A . B^T, f16) on the headline GEMM and PyTorch's SDPA
    flash backend (forced, so nothing falls back to batched matmuls) on
    config 4.  Not this build's code; reported beside it."""
    lines = []
    c = torch.empty((a.shape[0], b.shape[0]), dtype=torch.float16, device=dev)
    ms = time_launches(lambda: torch.matmul(a, b.t(), out=c), steps, 3, torch)
    tf = 2.0 * a.shape[0] * b.shape[0] * a.shape[1] / (ms * 1e-3) / 1e12
    log(f"vendor: torch.matmul (hipBLASLt) f16 8192^3: {ms * 1e3:.1f} us/launch, {tf:.1f} TFLOP/s")
    lines.append({"workload": "vendor_hipblaslt_gemm_f16_8192x8192x8192", "value": round(tf, 2),
                  "unit": "TFLOP/s", "ms_per_step": round(ms, 4),
                  "frac_of_mfma_peak": round(tf / MFMA_PEAK_TFLOPS, 4),
                  "kernel": "torch.matmul(A, B.t()), same inputs as the headline"})
    del c
    B, H, S, D = 4, 32, 4096, 128
    g = torch.Generator(device=dev).manual_seed(11)
    q, k, v = (torch.randn((B, H, S, D), generator=g, device=dev).to(torch.float16)
               for _ in range(3))
    try:
        from torch.nn.attention import SDPBackend, sdpa_kernel
        with sdpa_kernel(SDPBackend.FLASH_ATTENTION):
            ms = time_launches(lambda: torch.nn.functional.scaled_dot_product_attention(q, k, v),
                               10, 3, torch)
        tf = 4.0 * B * H * S * S * D / (ms * 1e-3) / 1e12
        log(f"vendor: torch SDPA flash f16 B4 H32 S4096 D128: {ms * 1e3:.1f} us/launch, "
            f"{tf:.1f} TFLOP/s")
        lines.append({"workload": "vendor_torch_sdpa_flash_f16_b4_h32_s4096_d128",
                      "value": round(tf, 2), "unit": "TFLOP/s", "ms_per_step": round(ms, 4),
                      "frac_of_mfma_peak": round(tf / MFMA_PEAK_TFLOPS, 4)})
    except (RuntimeError, ImportError) as e:
        log(f"vendor: torch SDPA flash unavailable ({type(e).__name__})")
    del q, k, v
    return lines


def mxfp4_line(wave, torch, dev, steps, warmup):
    """MXFP4 scaled GEMM at the reference's MXFP4 profile shape (4096 x 4096
    x 32768, f16 column-major C): random e2m1 codes (every nibble uniform
    over the 16 codes) and e8m0 scales uniform over 124..127, the
    distribution of the runner's generator (runner.cpp:1135-1150,
    :1208-1220)."""
    Mx, Nx, Kx = 4096, 4096, 32768
    gx = torch.Generator(device=dev).manual_seed(13)
    xa = torch.randint(0, 256, (Mx, Kx // 2), generator=gx, device=dev, dtype=torch.uint8)
    xb = torch.randint(0, 256, (Nx, Kx // 2), generator=gx, device=dev, dtype=torch.uint8)
    xsa = torch.randint(124, 128, (Kx // 32, Mx), generator=gx, device=dev, dtype=torch.uint8)
    xsb = torch.randint(124, 128, (Kx // 32, Nx), generator=gx, device=dev, dtype=torch.uint8)
    xc = torch.empty((Nx, Mx), dtype=torch.float16, device=dev)
    m_ms = time_launches(lambda: wave.gemm_mxfp4(xa, xb, xsa, xsb, out_dtype=torch.float16,
                                                 layout="col", out=xc), steps, warmup, torch)
    m_tf = 2.0 * Mx * Nx * Kx / (m_ms * 1e-3) / 1e12
    log(f"gemm mxfp4 4096x4096x32768: {m_ms * 1e3:.1f} us/launch, {m_tf:.1f} TFLOP/s "
        f"({100 * m_tf / FP4_PEAK_TFLOPS:.1f}% of {FP4_PEAK_TFLOPS})")
    return {"workload": "gemm_mxfp4_4096x4096x32768_f16_col_random",
            "value": round(m_tf, 2), "unit": "TFLOP/s", "ms_per_step": round(m_ms, 4),
            "frac_of_fp4_peak": round(m_tf / FP4_PEAK_TFLOPS, 4),
            "reference_published": {
                "value": 4460.0, "unit": "TFLOP/s", "hardware": "gfx950",
                "kernel": "gfx950-mxfp4-256x256-8wave, random inputs",
                "source": "docs/Gfx950MatmulProfiles.md:57-68"}}


def mxfp8_fa_lines(wave, torch, dev, steps, warmup):
    """Block-scaled FP8 flash-attention forward (wave_fa_fwd_mxfp8_launch) on
    the f16 benchmark shape B4 H32 S4096 and on the reference's FA profile
    shape B2 H64 S8192: N(0,1) inputs quantized to MX-FP8 on the device
    (mxfp8_quantize, outside the timing), f16 O, FLOPs 4*B*H*S^2*D."""
    lines = []
    g = torch.Generator(device=dev).manual_seed(19)
    for B, H, S in ((4, 32, 4096), (2, 64, 8192)):
        D = 128
        q, k, v = (torch.randn((B, H, S, D), generator=g, device=dev) for _ in range(3))
        (qe, qs), (ke, ks), (ve, vs) = (wave.mxfp8_quantize(q), wave.mxfp8_quantize(k),
                                        wave.mxfp8_quantize(v, dim=2))
        del q, k, v
        o = torch.empty((B, H, S, D), dtype=torch.float16, device=dev)
        ms = time_launches(lambda: wave.flash_attention_mxfp8(qe, qs, ke, ks, ve, vs, out=o),
                           steps, warmup, torch)
        tf = 4.0 * B * H * S * S * D / (ms * 1e-3) / 1e12
        log(f"fa fwd mxfp8 B{B} H{H} S{S} D128 (f16 O): {ms * 1e3:.1f} us/launch, {tf:.1f} "
            f"TFLOP/s ({100 * tf / FP8_PEAK_TFLOPS:.1f}% of fp8 {FP8_PEAK_TFLOPS})")
        lines.append({"workload": f"fa_fwd_mxfp8_b{B}_h{H}_s{S}_d128_noncausal_f16out",
                      "value": round(tf, 2), "unit": "TFLOP/s", "ms_per_step": round(ms, 4),
                      "frac_of_fp8_peak": round(tf / FP8_PEAK_TFLOPS, 4),
                      "dtype": "MX-FP8 (e4m3 + e8m0 per 32) in, fp32 accumulate, f16 out"})
        del qe, qs, ke, ks, ve, vs, o
    return lines


def fa_bwd_line(wave, torch, dev, steps):
    """Flash-attention backward (no reference counterpart) on the FA forward's
    benchmark shape B4 H32 S4096 D128 f16, non-causal: delta, dK/dV and dQ
    kernels; FLOPs counted as flash-attention does, 2.5 x the forward's (five
    S x S x D products)."""
    B, H, S, D = 4, 32, 4096, 128
    g = torch.Generator(device="cpu").manual_seed(11)
    q, k, v, do = (torch.randn((B, H, S, D), generator=g).to(torch.float16).to(dev)
                   for _ in range(4))
    o, lse = wave.flash_attention_lse(q, k, v)
    bw_ms = time_launches(lambda: wave.flash_attention_bwd(q, k, v, o, do, lse), steps, 1,
                          torch)
    bw_tf = 10.0 * B * H * S * S * D / (bw_ms * 1e-3) / 1e12
    log(f"fa bwd f16 B4 H32 S4096 D128: {bw_ms * 1e3:.1f} us/launch, {bw_tf:.1f} TFLOP/s "
        f"({100 * bw_tf / MFMA_PEAK_TFLOPS:.1f}%)")
    line = {"workload": "fa_bwd_f16_b4_h32_s4096_d128_noncausal",
            "value": round(bw_tf, 2), "unit": "TFLOP/s", "ms_per_step": round(bw_ms, 4),
            "frac_of_mfma_peak": round(bw_tf / MFMA_PEAK_TFLOPS, 4),
            "flops": "10*B*H*S^2*D"}
    # PyTorch's flash-attention backward op on the same inputs, for scale
    # (its forward run once outside the timed region, as here).
    try:
        fa = torch.ops.aten._scaled_dot_product_flash_attention(q, k, v, 0.0, False, False)
        t_out, t_lse, cq, ck, mq, mk, seed, offset = fa[:8]
        vms = time_launches(
            lambda: torch.ops.aten._scaled_dot_product_flash_attention_backward(
                do, q, k, v, t_out, t_lse, cq, ck, mq, mk, 0.0, False, seed, offset),
            10, 3, torch)
        line["torch_sdpa_flash_bwd_value"] = round(10.0 * B * H * S * S * D / (vms * 1e-3) / 1e12,
                                                   2)
        log(f"vendor: torch flash-attention backward op f16 B4 H32 S4096: "
            f"{line['torch_sdpa_flash_bwd_value']:.1f} TFLOP/s")
    except (RuntimeError, TypeError, AttributeError) as e:
        log(f"vendor: torch flash-attention backward unavailable ({type(e).__name__})")
    return line


def config_lines(wave, torch, dev, steps, warmup):
    """BASELINE.json configs 3 (ragged / skinny bf16 GEMMs, entries N(0,1)
    scaled by 1/sqrt(K), bf16 in and out, fp32 accumulate) and 5 (causal GQA
    flash attention, bf16), each on inputs resident in HBM."""
    lines = []
    g = torch.Generator(device=dev).manual_seed(5)

    def operands(M, N, K):
        a = (torch.randn((M, K), generator=g, device=dev) / math.sqrt(K)).to(torch.bfloat16)
        b = (torch.randn((N, K), generator=g, device=dev) / math.sqrt(K)).to(torch.bfloat16)
        return a, b, torch.empty((M, N), dtype=torch.bfloat16, device=dev)

    for name, (M, N, K) in (("3a", (128, 8192, 8192)), ("3b", (4000, 4096, 4100)),
                            ("3c", (8192, 1024, 28672))):
        a, b, c = operands(M, N, K)
        fl = 2.0 * M * N * K
        nbytes = 2.0 * (M * K + N * K + M * N)
        ms = time_launches(lambda: wave.gemm(a, b, out_dtype=torch.bfloat16, out=c), steps,
                           warmup, torch)
        tf = fl / (ms * 1e-3) / 1e12
        line = {"workload": f"gemm_bf16_{M}x{N}x{K}_config{name}", "value": round(tf, 2),
                "unit": "TFLOP/s", "ms_per_step": round(ms, 4),
                "frac_of_mfma_peak": round(tf / MFMA_PEAK_TFLOPS, 4),
                "kernel": "wave_gemm_launch"}
        if name == "3a":  # HBM-bound: algorithmic bytes read and written once
            gbs = nbytes / (ms * 1e-3) / 1e9
            line.update({"gbps": round(gbs, 1), "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
                         "algorithmic_bytes": int(nbytes)})
        if name == "3a":  # short M: the auto dispatch's split-K short-M kernel
            ws = torch.empty(max(wave.gemm_auto_workspace_bytes(M, N, K), 1), dtype=torch.uint8,
                             device=dev)
            wrapped = time_launches(lambda: wave.gemm_auto(a, b, out_dtype=torch.bfloat16,
                                                           workspace=ws, out=c), steps, warmup,
                                    torch)
            # The same C-ABI call with its arguments bound once: the Python
            # wrapper's checks take about as long as this ~32 us launch, so
            # through it the stream can run dry between launches.
            launch = wave.runtime.lib().wave_gemm_auto_launch
            cargs = (a.data_ptr(), b.data_ptr(), c.data_ptr(), M, N, K, wave.runtime.BF16,
                     wave.runtime.BF16,
                     wave.runtime.ROW_MAJOR, ws.data_ptr(), ws.numel(),
                     torch.cuda.current_stream(dev).cuda_stream)

            def direct():
                if launch(*cargs) != 0:
                    raise RuntimeError("wave_gemm_auto_launch failed")
            ams = time_launches(direct, max(steps, 200), warmup, torch)  # ~32 us each
            atf = fl / (ams * 1e-3) / 1e12
            gbs = nbytes / (ams * 1e-3) / 1e9
            line.update({"value": round(atf, 2), "ms_per_step": round(ams, 4),
                         "frac_of_mfma_peak": round(atf / MFMA_PEAK_TFLOPS, 4),
                         "gbps": round(gbs, 1), "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
                         "kernel": "wave_gemm_auto_launch (split-K short-M kernel, + counter "
                                   "fill), called through ctypes with pre-bound arguments",
                         "ms_per_step_through_python_wrapper": round(wrapped, 4),
                         "unsplit_kernel_value": round(tf, 2)})
        if name == "3c":  # fewer 256x256 tiles (128) than CUs: the auto dispatch's Stream-K
            ws = torch.empty(max(wave.gemm_auto_workspace_bytes(M, N, K), 1), dtype=torch.uint8,
                             device=dev)
            ams = time_launches(lambda: wave.gemm_auto(a, b, out_dtype=torch.bfloat16,
                                                       workspace=ws, out=c), steps, warmup,
                                torch)
            atf = fl / (ams * 1e-3) / 1e12
            line.update({"value": round(atf, 2), "ms_per_step": round(ams, 4),
                         "frac_of_mfma_peak": round(atf / MFMA_PEAK_TFLOPS, 4),
                         "kernel": "wave_gemm_auto_launch (Stream-K, min(2*tiles, CUs) workers)",
                         "tiled_kernel_value": round(tf, 2)})
        # The vendor library on the same inputs and output, for scale (not
        # this build's code): hipBLASLt through torch.matmul, C = A . B^T.
        vms = time_launches(lambda: torch.matmul(a, b.t(), out=c), steps, warmup, torch)
        line["hipblaslt_value"] = round(fl / (vms * 1e-3) / 1e12, 2)
        log(f"config {name} gemm bf16 {M}x{N}x{K}: {line['ms_per_step'] * 1e3:.1f} us/launch, "
            f"{line['value']:.1f} TFLOP/s" + (f", {line['gbps']:.0f} GB/s" if "gbps" in line else "")
            + f" (hipBLASLt {line['hipblaslt_value']:.1f})")
        lines.append(line)
        del a, b, c

    B, Hq, Hkv, S, D = 1, 64, 8, 8192, 128
    q = torch.randn((B, Hq, S, D), generator=g, device=dev).to(torch.bfloat16)
    k = torch.randn((B, Hkv, S, D), generator=g, device=dev).to(torch.bfloat16)
    v = torch.randn((B, Hkv, S, D), generator=g, device=dev).to(torch.bfloat16)
    o = torch.empty_like(q)
    ms = time_launches(lambda: wave.flash_attention(q, k, v, causal=True, out=o), steps, warmup,
                       torch)
    tf = 2.0 * B * Hq * S * S * D / (ms * 1e-3) / 1e12
    log(f"config 5 fa fwd causal GQA bf16 B1 Hq64 Hkv8 S8192: {ms * 1e3:.1f} us/launch, "
        f"{tf:.1f} TFLOP/s (causal FLOPs)")
    line5 = {"workload": "fa_fwd_bf16_b1_hq64_hkv8_s8192_d128_causal_config5",
             "value": round(tf, 2), "unit": "TFLOP/s", "ms_per_step": round(ms, 4),
             "frac_of_mfma_peak": round(tf / MFMA_PEAK_TFLOPS, 4),
             "flops": "2*B*Hq*S^2*D (the keys a causal row attends to; the reference's "
                      "4*B*H*S^2*D non-causal count would double it)"}
    # PyTorch's SDPA flash backend on the same inputs, for scale: K and V
    # expanded to the 64 query heads (the flash backend is forced, so nothing
    # falls back to batched matmuls).
    try:
        from torch.nn.attention import SDPBackend, sdpa_kernel
        ke = k.repeat_interleave(Hq // Hkv, dim=1).contiguous()
        ve = v.repeat_interleave(Hq // Hkv, dim=1).contiguous()
        with sdpa_kernel(SDPBackend.FLASH_ATTENTION):
            vms = time_launches(
                lambda: torch.nn.functional.scaled_dot_product_attention(q, ke, ve, is_causal=True),
                10, 3, torch)
        line5["torch_sdpa_flash_value"] = round(2.0 * B * Hq * S * S * D / (vms * 1e-3) / 1e12, 2)
        log(f"vendor: torch SDPA flash causal bf16 B1 H64 S8192 (K, V expanded): "
            f"{line5['torch_sdpa_flash_value']:.1f} TFLOP/s")
        del ke, ve
    except (RuntimeError, ImportError) as e:
        log(f"vendor: torch SDPA flash unavailable for config 5 ({type(e).__name__})")
    lines.append(line5)
    del q, k, v, o
    return lines


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-fa", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=24.0)
    ap.add_argument("--no-ref-compare", action="store_true",
                    help="skip the runs on the reference's published input modes / shapes")
    ap.add_argument("--workload",
                    choices=["all", "gemm", "fa", "fabwd", "mxfp4", "mxfp8fa", "copy",
                             "configs"],
                    default="all",
                    help="gemm / fa / fabwd / mxfp4 / mxfp8fa: run only that kernel (for "
                         "profiler passes); copy: a 1 GiB device copy used to calibrate "
                         "rocprofv3 byte counters")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(the GEMM and attention would shard by output tiles and by heads, "
              "one process per GPU)", file=sys.stderr)
        sys.exit(2)

    import torch
    wave = importlib.import_module("7_amd")
    wave.runtime.lib()
    dev = torch.device("cuda:0")
    peak_dev, clock_mhz, cus = wave.runtime.device_mfma_peak(0)
    log(f"device: {torch.cuda.get_device_name(0)} CUs={cus} clock={clock_mhz:.0f} MHz "
        f"derived f16 MFMA peak={peak_dev:.1f} TFLOP/s")

    if args.workload == "copy":
        src = torch.empty(1 << 28, dtype=torch.float32, device=dev).fill_(1.0)
        dst = torch.empty_like(src)
        ms = time_launches(lambda: dst.copy_(src), args.steps, args.warmup, torch)
        log(f"copy 1 GiB: {ms:.3f} ms, {2 * 4 * src.numel() / (ms * 1e-3) / 1e9:.0f} GB/s")
        return
    if args.workload in ("fa", "fabwd", "mxfp4", "mxfp8fa", "configs"):
        args.no_cpu = True
    if args.workload == "fabwd":
        print(json.dumps(fa_bwd_line(wave, torch, dev, args.steps)), flush=True)
        return
    if args.workload == "mxfp4":
        m = mxfp4_line(wave, torch, dev, args.steps, args.warmup)
        print(json.dumps(m), flush=True)
        return
    if args.workload == "mxfp8fa":
        for m in mxfp8_fa_lines(wave, torch, dev, args.steps, args.warmup):
            print(json.dumps(m), flush=True)
        return

    M = N = K = 8192
    g = torch.Generator(device="cpu").manual_seed(7)
    a_h = (torch.rand((M, K), generator=g) * 2 - 1).to(torch.float16)
    b_h = (torch.rand((N, K), generator=g) * 2 - 1).to(torch.float16)
    a, b = a_h.to(dev), b_h.to(dev)
    c = torch.empty((M, N), dtype=torch.float16, device=dev)

    def step():
        wave.gemm(a, b, out_dtype=torch.float16, out=c)

    ms = time_launches(step, args.steps if args.workload != "fa" else 1,
                       args.warmup if args.workload != "fa" else 0, torch)
    flops = 2.0 * M * N * K
    tflops = flops / (ms * 1e-3) / 1e12
    log(f"gemm f16 8192^3: {ms * 1e3:.1f} us/launch, {tflops:.1f} TFLOP/s "
        f"({100 * tflops / MFMA_PEAK_TFLOPS:.1f}% of {MFMA_PEAK_TFLOPS})")

    secondary = []
    if args.workload in ("gemm", "configs"):
        args.no_fa = True
    if not args.no_fa:
        B, H, S, D = 4, 32, 4096, 128
        gq = torch.Generator(device="cpu").manual_seed(11)
        q = torch.randn((B, H, S, D), generator=gq).to(torch.float16).to(dev)
        k = torch.randn((B, H, S, D), generator=gq).to(torch.float16).to(dev)
        v = torch.randn((B, H, S, D), generator=gq).to(torch.float16).to(dev)
        o = torch.empty_like(q)
        fa_ms = time_launches(lambda: wave.flash_attention(q, k, v, out=o),
                              max(10, args.steps // 2), 3, torch)
        fa_tf = 4.0 * B * H * S * S * D / (fa_ms * 1e-3) / 1e12
        log(f"fa fwd f16 B4 H32 S4096 D128: {fa_ms * 1e3:.1f} us/launch, {fa_tf:.1f} TFLOP/s "
            f"({100 * fa_tf / MFMA_PEAK_TFLOPS:.1f}%)")
        secondary.append({"workload": "fa_fwd_f16_b4_h32_s4096_d128_noncausal",
                          "value": round(fa_tf, 2), "unit": "TFLOP/s",
                          "ms_per_step": round(fa_ms, 4),
                          "frac_of_mfma_peak": round(fa_tf / MFMA_PEAK_TFLOPS, 4)})
        del q, k, v, o
        if args.workload == "all":
            secondary.append(fa_bwd_line(wave, torch, dev, 5))

    if args.workload in ("all", "configs"):
        secondary.extend(config_lines(wave, torch, dev, max(10, args.steps // 2), 3))

    if args.workload == "all" and not args.no_ref_compare:
        # The same kernels on the input mode / shape of the reference's own
        # published figures (docs/PerfReferences/WaveGfx950F16Gemm4Wave.md:29-31,
        # docs/PerfReferences/WaveGfx950FlashAttention.md:5-21, MI350X): not the
        # headline metric, which uses uniform inputs.
        ra = rand_int_operand(M, K, 0, torch).to(dev)
        rb = rand_int_operand(N, K, 1, torch).to(dev)
        r_ms = time_launches(lambda: wave.gemm(ra, rb, out_dtype=torch.float16, out=c),
                             max(10, args.steps // 2), 3, torch)
        r_tf = flops / (r_ms * 1e-3) / 1e12
        log(f"gemm f16 8192^3 rand_int inputs: {r_ms * 1e3:.1f} us/launch, {r_tf:.1f} TFLOP/s")
        secondary.append({"workload": "gemm_f16_8192x8192x8192_rand_int_inputs",
                          "value": round(r_tf, 2), "unit": "TFLOP/s",
                          "ms_per_step": round(r_ms, 4),
                          "frac_of_mfma_peak": round(r_tf / MFMA_PEAK_TFLOPS, 4),
                          "reference_published": {
                              "value": 1400.4, "unit": "TFLOP/s", "hardware": "MI350X",
                              "kernel": "gfx950-f16-256x256-8wave, rand_int inputs",
                              "source": "docs/PerfReferences/WaveGfx950F16Gemm4Wave.md:29-31"}})
        del ra, rb
        B, H, S, D = 2, 64, 8192, 128
        gq = torch.Generator(device="cpu").manual_seed(12)
        q = torch.randn((B, H, S, D), generator=gq).to(torch.bfloat16).to(dev)
        k = torch.randn((B, H, S, D), generator=gq).to(torch.bfloat16).to(dev)
        v = torch.randn((B, H, S, D), generator=gq).to(torch.bfloat16).to(dev)
        o = torch.empty_like(q)
        f_ms = time_launches(lambda: wave.flash_attention(q, k, v, out=o), 10, 2, torch)
        f_tf = 4.0 * B * H * S * S * D / (f_ms * 1e-3) / 1e12
        log(f"fa fwd bf16 B2 H64 S8192 D128: {f_ms * 1e3:.1f} us/launch, {f_tf:.1f} TFLOP/s")
        secondary.append({"workload": "fa_fwd_bf16_b2_h64_s8192_d128_noncausal_online_softmax",
                          "value": round(f_tf, 2), "unit": "TFLOP/s",
                          "ms_per_step": round(f_ms, 4),
                          "frac_of_mfma_peak": round(f_tf / MFMA_PEAK_TFLOPS, 4),
                          "reference_published": {
                              "value": 1111.1, "unit": "TFLOP/s", "hardware": "MI350X",
                              "kernel": "flash_attention_bf16_gfx950 8-wave, fixed-max mode "
                                        "(qk_max_abs=1, no online max; this line runs the "
                                        "online-softmax kernel)",
                              "source": "docs/PerfReferences/WaveGfx950FlashAttention.md:5-21"}})
        # The reference's fixed-max profile itself: |Q|, |K| <= 1 declared
        # (qk_max_abs=1), Q and K uniform in [-1, 1).
        q = (torch.rand((B, H, S, D), generator=gq) * 2 - 1).to(torch.bfloat16).to(dev)
        k = (torch.rand((B, H, S, D), generator=gq) * 2 - 1).to(torch.bfloat16).to(dev)
        x_ms = time_launches(lambda: wave.flash_attention(q, k, v, qk_max_abs=1.0, out=o), 10, 2,
                             torch)
        x_tf = 4.0 * B * H * S * S * D / (x_ms * 1e-3) / 1e12
        log(f"fa fwd bf16 B2 H64 S8192 D128 fixed max (qk_max_abs=1): {x_ms * 1e3:.1f} us/launch, "
            f"{x_tf:.1f} TFLOP/s")
        secondary.append({"workload": "fa_fwd_bf16_b2_h64_s8192_d128_noncausal_qk_max_abs_1",
                          "value": round(x_tf, 2), "unit": "TFLOP/s",
                          "ms_per_step": round(x_ms, 4),
                          "frac_of_mfma_peak": round(x_tf / MFMA_PEAK_TFLOPS, 4),
                          "reference_published": {
                              "value": 1111.1, "unit": "TFLOP/s", "hardware": "MI350X",
                              "kernel": "flash_attention_bf16_gfx950 8-wave, qk_max_abs=1",
                              "source": "docs/PerfReferences/WaveGfx950FlashAttention.md:5-21"}})
        # The reference's 4-wave configuration (block 256) on the same shape.
        q = torch.randn((B, H, S, D), generator=gq).to(torch.bfloat16).to(dev)
        k = torch.randn((B, H, S, D), generator=gq).to(torch.bfloat16).to(dev)
        w_ms = time_launches(lambda: wave.flash_attention(q, k, v, waves=4, out=o), 10, 2, torch)
        w_tf = 4.0 * B * H * S * S * D / (w_ms * 1e-3) / 1e12
        log(f"fa fwd bf16 B2 H64 S8192 D128 4-wave: {w_ms * 1e3:.1f} us/launch, {w_tf:.1f} TFLOP/s")
        secondary.append({"workload": "fa_fwd_bf16_b2_h64_s8192_d128_noncausal_4wave",
                          "value": round(w_tf, 2), "unit": "TFLOP/s",
                          "ms_per_step": round(w_ms, 4),
                          "frac_of_mfma_peak": round(w_tf / MFMA_PEAK_TFLOPS, 4),
                          "reference_published": {
                              "value": 984.0, "unit": "TFLOP/s", "hardware": "gfx950",
                              "kernel": "four-wave BM=128 branch experiment (upper end of "
                                        "978-984)",
                              "source": "docs/PerfReferences/WaveGfx950FlashAttention.md:67"}})
        del q, k, v, o
        secondary.append(mxfp4_line(wave, torch, dev, 20, 3))
        secondary.extend(mxfp8_fa_lines(wave, torch, dev, 10, 2))
        secondary.extend(vendor_lines(torch, dev, a, b, max(10, args.steps // 2)))

    cpu = None
    ref_cpu = None
    if not args.no_cpu:
        a_bits = a_h.view(torch.int16).numpy().view(np.uint16)
        b_bits = b_h.view(torch.int16).numpy().view(np.uint16)
        cpu = cpu_baseline(a_bits, b_bits, M, N, K, args.cpu_budget)
        log(f"cpu baseline: {cpu['value']} TFLOP/s on {cpu['cores']} threads ({cpu['sample']})")
        ref_cpu = cpu_reference_path(M, N, K, 6.0)
        if ref_cpu:
            log(f"reference CPU path: {ref_cpu['value']} TFLOP/s on 1 thread ({ref_cpu['sample']})")

    line = {
        "metric": "TFLOP/s + % gfx950 MFMA peak: f16 GEMM 8192^3, FA fwd S=4096 D=128",
        "value": round(tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "warmup_min_seconds": WARMUP_SECONDS,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic: A, B uniform [-1, 1) f16, torch CPU generator seed 7",
        "config": {"workload": "gemm_f16_8192x8192x8192", "M": M, "N": N, "K": K,
                   "A": "M x K row-major", "B": "N x K row-major", "C": "f16 row-major",
                   "accumulate": "fp32"},
        "roofline": {"bound": "mfma", "achieved": round(tflops, 2),
                     "peak": MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(tflops / MFMA_PEAK_TFLOPS, 4),
                     "traffic": read_traffic()},
        "cpu_baseline": cpu,
        "cpu_reference_path": ref_cpu,
        "secondary": secondary,
        "device_derived_peak_tflops": round(peak_dev, 1),
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
