"""bench.py's reference-comparison inputs are the reference runner's
rand_int values (runner.cpp:700-706, :1176-1183), bit for bit as the
oracle's generator (itself pinned to rand_int_test.cpp:30-33)."""

import importlib.util
import os

import numpy as np
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _bench():
    spec = importlib.util.spec_from_file_location("bench", os.path.join(ROOT, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_rand_int_operands_match_oracle(oracle):
    bench = _bench()
    for stream in (0, 1):
        got = bench.rand_int_operand(37, 50, stream, torch).view(torch.int16).numpy()
        exp = oracle.gemm_inputs(37, 50, 1, 0, stream, oracle.MODE_RAND_INT)
        assert np.array_equal(got.view(np.uint16).ravel(), exp.ravel())
