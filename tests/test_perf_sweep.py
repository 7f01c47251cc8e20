"""7_amd/perf_sweep.py keeps the reference's sweep CSV schema
(tools/wave-matmul-calibrate/wave-matmul-perf-sweep.py:798-825) and parses
wave-bench output with the reference's patterns (:659-679)."""

import importlib

REFERENCE_COLUMNS = ["kernel", "profile", "m", "n", "k", "variants", "iters", "warmup",
                     "repeats", "us", "tflops", "cycles", "check", "returncode", "command",
                     "workload", "batch", "heads", "sequence", "head_dim", "xcds", "waves"]


def test_csv_columns_match_reference():
    sweep = importlib.import_module("7_amd.perf_sweep")
    assert sweep.COLUMNS == REFERENCE_COLUMNS


def test_parse_wave_bench_lines():
    sweep = importlib.import_module("7_amd.perf_sweep")
    out = ("kernel: wmma_f16_matmul_tiled\nper_launch_us: 963.100\n"
           "median_per_launch_us: 963.100\n  hw_cycles_wallclock: 2311440\n"
           "tflops: 1141.6\noutput_check: passed mode=sampled elements=514\n")
    assert sweep.parse(out) == (963.1, 2311440, "passed")
    assert sweep.parse("") == (None, None, None)


def test_default_matrix_follows_reference_defaults():
    sweep = importlib.import_module("7_amd.perf_sweep")
    ns = type("A", (), dict(kernels=["f16", "fa", "mxfp4"], m=4096, n=4096,
                            k=list(sweep.F16_K_VALUES), k_given=False,
                            input_mode="uniform", streamk_workers=256))
    runs = list(sweep.runs(ns))
    gemm = [r for r in runs if r[0] == "f16"]
    assert [r[1][2] for r in gemm] == [512, 1024, 2048, 3072, 4096, 8192, 16384]
    fa = [r for r in runs if r[0] == "fa"][0]
    assert fa[3] == 4 * 2 * 64 * 8192 ** 2 * 128
    # MXFP4 rows: the reference's MXFP4_DOC_K_VALUES (wave-matmul-perf-sweep.py:33)
    mx = [r for r in runs if r[0] == "mxfp4"]
    assert [r[1][2] for r in mx] == [1024, 2048, 3072, 4096, 8192, 16384, 32768]
    assert "--input-type" in mx[0][2] and "mxfp4" in mx[0][2]
