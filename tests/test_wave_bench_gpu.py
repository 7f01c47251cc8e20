"""The C++ host driver 7_amd/wave-bench (the counterpart of the reference's
runners) on the GPU: every input mode and kernel family with --check, its
output lines parsed with the reference sweep's patterns (7_amd/perf_sweep.py
`parse`, tools/wave-matmul-calibrate/wave-matmul-perf-sweep.py:659-679), and
a small sweep through perf_sweep.main writing the reference's CSV schema."""

import csv
import importlib
import os
import re
import subprocess

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BENCH = os.path.join(ROOT, "7_amd", "wave-bench")


@pytest.fixture(scope="module")
def sweep():
    return importlib.import_module("7_amd.perf_sweep")


def run(args, timeout=120):
    proc = subprocess.run([BENCH] + args + ["--iters", "3", "--warmup", "1", "--repeats", "1",
                                            "--check"],
                          capture_output=True, text=True, timeout=timeout)
    assert proc.returncode == 0, proc.stderr[-2000:]
    return proc.stdout


@pytest.mark.parametrize("mode", ["uniform", "normal", "bucket", "rand-int", "hpl", "all-ones"])
@pytest.mark.parametrize("extra,shape", [
    ([], (512, 512, 512)),
    (["--input-type", "bf16", "--c-type", "bf16", "--output-layout", "column-major"],
     (300, 200, 100)),
    (["--streamk-workers", "7", "--output-layout", "column-major"], (512, 768, 1024)),
])
def test_gemm_modes(sweep, mode, extra, shape):
    M, N, K = shape
    out = run(["gemm", "--m", str(M), "--n", str(N), "--k", str(K), "--input-mode", mode] + extra)
    us, cycles, check = sweep.parse(out)
    assert check == "passed" and us > 0 and cycles > 0
    tf = float(re.search(r"^tflops:\s+([0-9.]+)$", out, re.M).group(1))
    # tflops is printed with 3 decimals (half a digit: 5e-4 absolute).
    assert tf == pytest.approx(2.0 * M * N * K / us * 1e-6, rel=1e-3, abs=5e-4)
    assert f"input_mode: {mode}" in out
    if "--streamk-workers" in extra:
        assert "gfx950_f16_streamk_gemm" in out


@pytest.mark.parametrize("mode", ["random", "all-ones"])
def test_gemm_mxfp4(sweep, mode):
    args = ["gemm", "--input-type", "mxfp4", "--m", "256", "--n", "512", "--k", "1024",
            "--c-type", "f16", "--output-layout", "column-major"]
    out = run(args + (["--all-ones"] if mode == "all-ones" else []))
    us, _, check = sweep.parse(out)
    assert check == "passed" and us > 0


@pytest.mark.parametrize("args", [
    ["--batch", "1", "--heads", "2", "--sequence", "512", "--dtype", "bf16"],
    ["--batch", "2", "--heads", "4", "--kv-heads", "2", "--sequence", "384", "--dtype", "f16",
     "--causal"],
])
def test_fa(sweep, args):
    out = run(["fa"] + args)
    us, _, check = sweep.parse(out)
    assert check == "passed" and us > 0


def test_sweep_writes_reference_csv(sweep, tmp_path, capsys):
    path = tmp_path / "sweep.csv"
    rc = sweep.main(["--kernels", "f16,f16-streamk,bf16,mxfp4", "--m", "512", "--n", "512",
                     "--k", "512,1024", "--streamk-workers", "16", "--iters", "3",
                     "--warmup", "1", "--repeats", "1",
                     "--csv", str(path)])
    assert rc == 0
    rows = list(csv.DictReader(open(path)))
    assert len(rows) == 8 and list(rows[0]) == sweep.COLUMNS
    assert all(r["check"] == "passed" and float(r["tflops"]) > 0 for r in rows)
    assert "summary:" in capsys.readouterr().out
