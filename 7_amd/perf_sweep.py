"""Performance sweep over this build's kernels, with the reference's CSV
schema (tools/wave-matmul-calibrate/wave-matmul-perf-sweep.py:798-862) and
summary table (:775-795), so results line up with the reference's sweeps.

Kernel matrix (the reference's defaults, :32-42, :150-326, :876-877):

* ``f16``         tiled GEMM, M = N = 4096, K in 512 .. 16384.
* ``f16-streamk`` the same shapes through Stream-K, 256 workers.
* ``bf16``        tiled GEMM with bf16 in/out (not in the reference).
* ``mxfp4``       MXFP4 scaled GEMM, f16 column-major C, K in 1024 .. 32768
                  (the reference's MXFP4_DOC_K_VALUES, :33, :189-197).
* ``fa``          flash-attention forward, B2 H64 S8192 D128 bf16.

Each run is one ``7_amd/wave-bench`` process with ``--check``; its
``median_per_launch_us:``, ``hw_cycles_wallclock:`` and ``output_check:``
lines are parsed with the reference's patterns (:659-679).

    python 7_amd/perf_sweep.py --csv sweep.csv [--kernels f16,fa]
        [--m 4096 --n 4096 --k 512,8192] [--input-mode rand-int] [--iters N]
"""

import argparse
import csv
import os
import re
import shlex
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
BENCH = os.path.join(HERE, "wave-bench")

F16_K_VALUES = (512, 1024, 2048, 3072, 4096, 8192, 16384)
MXFP4_K_VALUES = (1024, 2048, 3072, 4096, 8192, 16384, 32768)
FA_SHAPE = dict(batch=2, heads=64, sequence=8192, head_dim=128, xcds=8, waves=8)
PROFILES = {
    "f16": "wave-mi355x-f16-256x256-4wave",
    "f16-streamk": "wave-mi355x-f16-256x256-4wave-streamk",
    "bf16": "wave-mi355x-bf16-256x256-4wave",
    "mxfp4": "wave-mi355x-mxfp4-256x256-8wave",
    "fa": "wave-mi355x-fa-8wave-pingpong",
}
COLUMNS = ["kernel", "profile", "m", "n", "k", "variants", "iters", "warmup", "repeats", "us",
           "tflops", "cycles", "check", "returncode", "command", "workload", "batch", "heads",
           "sequence", "head_dim", "xcds", "waves"]


def runs(args):
    for kernel in args.kernels:
        if kernel == "fa":
            s = FA_SHAPE
            cmd = [BENCH, "fa", "--batch", str(s["batch"]), "--heads", str(s["heads"]),
                   "--sequence", str(s["sequence"]), "--dtype", "bf16"]
            flops = 4 * s["batch"] * s["heads"] * s["sequence"] ** 2 * s["head_dim"]
            yield kernel, None, cmd, flops
            continue
        ks = args.k
        if kernel == "mxfp4" and not args.k_given:
            ks = MXFP4_K_VALUES
        for k in ks:
            cmd = [BENCH, "gemm", "--m", str(args.m), "--n", str(args.n), "--k", str(k),
                   "--input-mode", args.input_mode]
            if kernel == "mxfp4":
                cmd += ["--input-type", "mxfp4", "--c-type", "f16", "--output-layout",
                        "column-major"]
            if kernel == "bf16":
                cmd += ["--input-type", "bf16", "--c-type", "bf16"]
            if kernel == "f16-streamk":
                cmd += ["--streamk-workers", str(args.streamk_workers)]
            yield kernel, (args.m, args.n, k), cmd, 2 * args.m * args.n * k


def parse(stdout):
    us = re.search(r"^median_per_launch_us:\s+([0-9.]+)$", stdout, re.M)
    cyc = re.search(r"^  hw_cycles_wallclock:\s+(\d+)$", stdout, re.M)
    chk = re.search(r"^output_check:\s+(\w+)", stdout, re.M)
    return (float(us.group(1)) if us else None, int(cyc.group(1)) if cyc else None,
            chk.group(1) if chk else None)


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--kernels", default="f16,f16-streamk,fa",
                    type=lambda s: [k for k in s.split(",") if k])
    ap.add_argument("--m", type=int, default=4096)
    ap.add_argument("--n", type=int, default=4096)
    ap.add_argument("--k", default=None, type=lambda s: [int(x) for x in s.split(",") if x])
    ap.add_argument("--input-mode", default="uniform")
    ap.add_argument("--streamk-workers", type=int, default=256)
    ap.add_argument("--iters", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--repeats", type=int, default=3)
    ap.add_argument("--timeout", type=int, default=300, help="seconds per run")
    ap.add_argument("--csv", default=None)
    ap.add_argument("--keep-going", action="store_true")
    args = ap.parse_args(argv)
    args.k_given = args.k is not None
    if args.k is None:
        args.k = list(F16_K_VALUES)
    unknown = set(args.kernels) - set(PROFILES)
    if unknown:
        ap.error(f"unknown kernels {sorted(unknown)}; choose from {sorted(PROFILES)}")
    if not os.path.exists(BENCH):
        sys.exit(f"{BENCH} is not built (make -C 7_amd/csrc)")

    rows = []
    for kernel, shape, cmd, flops in runs(args):
        cmd = cmd + ["--iters", str(args.iters), "--warmup", str(args.warmup), "--repeats",
                     str(args.repeats), "--check"]
        print("+ " + shlex.join(cmd), flush=True)
        try:
            proc = subprocess.run(cmd, capture_output=True, text=True, timeout=args.timeout)
            out, rc = proc.stdout, proc.returncode
            sys.stderr.write(proc.stderr)
        except subprocess.TimeoutExpired:
            out, rc = "", 124
        us, cycles, check = parse(out)
        tflops = flops / us * 1e-6 if us else None
        fa = kernel == "fa"
        rows.append({
            "kernel": kernel, "profile": PROFILES[kernel],
            "m": "" if fa else shape[0], "n": "" if fa else shape[1], "k": "" if fa else shape[2],
            "variants": "hip", "iters": args.iters, "warmup": args.warmup,
            "repeats": args.repeats, "us": us, "tflops": tflops, "cycles": cycles,
            "check": check, "returncode": rc, "command": shlex.join(cmd),
            "workload": "flash_attention" if fa else "matmul",
            **({k: FA_SHAPE[k] for k in ("batch", "heads", "sequence", "head_dim", "xcds",
                                         "waves")} if fa else
               {k: "" for k in ("batch", "heads", "sequence", "head_dim", "xcds", "waves")}),
        })
        if rc != 0 and not args.keep_going:
            break

    print("\nsummary:")
    print("kernel          shape                                    variant    us        "
          "TFLOP/s   check")
    print("--------------  ---------------------------------------  ---------  --------  "
          "--------  -------")
    for r in rows:
        shape = (f"B={r['batch']},H={r['heads']},N={r['sequence']},D={r['head_dim']}"
                 if r["workload"] == "flash_attention" else f"M={r['m']},N={r['n']},K={r['k']}")
        us = f"{r['us']:.3f}" if r["us"] is not None else "-"
        tf = f"{r['tflops']:.2f}" if r["tflops"] is not None else "-"
        check = r["check"] or ("failed" if r["returncode"] else "-")
        print(f"{r['kernel']:<14}  {shape:<39}  {r['variants']:<9}  {us:>8}  {tf:>8}  {check}")
    if args.csv:
        os.makedirs(os.path.dirname(os.path.abspath(args.csv)), exist_ok=True)
        with open(args.csv, "w", newline="") as f:
            w = csv.DictWriter(f, fieldnames=COLUMNS)
            w.writeheader()
            w.writerows(rows)
    return 0 if all(r["returncode"] == 0 and r["check"] == "passed" for r in rows) else 1


if __name__ == "__main__":
    sys.exit(main())
