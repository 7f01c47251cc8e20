"""CPU-side checks of the drop-in boundary (no GPU needed, no compute).

* libwave_runtime.so loads and exports every function include/wave_runtime.h
  declares;
* the seven memref shims keep the reference behaviour data + offset
  (runtime/wave_runtime.cpp:27-74), per element type;
* every launch entry point rejects bad arguments on the host, before any
  HIP call, with the documented status codes (the reference runners' `die`
  paths, wave-matmul-calibrate-runner.cpp:297-455 and :424-440).
"""

import ctypes

import pytest


def test_library_exports_every_declared_symbol(wave):
    L = wave.runtime.lib()
    declared = wave.runtime.header_symbols()
    assert len(declared) >= 17
    for name in declared:
        assert hasattr(L, name), name


@pytest.mark.parametrize("tag,size", [("i32", 4), ("i8", 1), ("f32", 4), ("f16", 2),
                                      ("bf16", 2), ("i64", 8), ("f64", 8)])
def test_memref_shims_return_data_plus_offset(wave, tag, size):
    L = wave.runtime.lib()

    class MemRef(ctypes.Structure):
        _fields_ = [("base", ctypes.c_void_p), ("data", ctypes.c_void_p),
                    ("offset", ctypes.c_int64), ("sizes", ctypes.c_int64 * 1),
                    ("strides", ctypes.c_int64 * 1)]

    buf = ctypes.create_string_buffer(1024)
    base = ctypes.addressof(buf)
    for offset in (0, 1, 7, 100):
        m = MemRef(base, base + 16, offset, (ctypes.c_int64 * 1)(64), (ctypes.c_int64 * 1)(1))
        fn = getattr(L, f"_mlir_ciface_wave_memref_to_ptr_global_{tag}")
        assert fn(ctypes.byref(m)) == base + 16 + offset * size


def test_status_strings(wave):
    L = wave.runtime.lib()
    assert L.wave_status_string(0) == b"ok"
    assert L.wave_status_string(-1) == b"invalid argument"
    assert L.wave_status_string(-2) == b"unsupported configuration"


def _gemm(L, **kw):
    a = dict(A=16, B=32, C=64, M=32, N=32, K=64, i=1, o=0, lay=0)
    a.update(kw)
    return L.wave_gemm_launch(a["A"], a["B"], a["C"], a["M"], a["N"], a["K"], a["i"],
                              a["o"], a["lay"], None)


@pytest.mark.parametrize("kw,status", [
    (dict(A=None), -1), (dict(C=None), -1), (dict(M=0), -1), (dict(N=-3), -1),
    (dict(K=0), -1), (dict(i=0), -1), (dict(i=7), -1), (dict(o=5), -1), (dict(lay=2), -1),
    (dict(K=1 << 23), -2),
])
def test_gemm_rejects_bad_arguments(wave, kw, status):
    L = wave.runtime.lib()
    assert _gemm(L, **kw) == status
    assert L.wave_last_error()


def test_streamk_workspace_sizes(wave):
    # runner.cpp:393-412 and rand_int_test.cpp:216-227: 5 workers ->
    # 5*2*256*256*4 bytes of scratch; 512x768 -> 6 counters
    # (wave_matmul_streamk.py:58-59).
    w = wave
    assert w.streamk_workspace_bytes(512, 512, 5) == (5 * 2 * 256 * 256 * 4, 4 * 4)
    assert w.streamk_workspace_bytes(512, 768, 3) == (3 * 2 * 256 * 256 * 4, 6 * 4)
    assert w.streamk_workspace_bytes(8192, 8192, 256) == (134217728, 4096)
    # ragged extents round up to whole 256x256 tiles
    assert w.streamk_workspace_bytes(4000, 4096, 1)[1] == 16 * 16 * 4
    with pytest.raises(ValueError):
        w.streamk_workspace_bytes(0, 256, 1)
    with pytest.raises(ValueError):
        w.streamk_workspace_bytes(256, 256, 0)


def test_streamk_rejects_bad_arguments(wave):
    L = wave.runtime.lib()
    # 512x512x256: 4 tiles x 4 K steps = 16 work units
    args = [16, 32, 64, 512, 512, 256, 1, 1, 1, 128, 256]
    assert L.wave_gemm_streamk_launch(*args, 17, None) == -1     # workers > work
    assert L.wave_gemm_streamk_launch(*args, 0, None) == -1      # workers <= 0
    bad = list(args)
    bad[9] = None
    assert L.wave_gemm_streamk_launch(*bad, 5, None) == -1       # no scratch
    assert L.wave_gemm_streamk_workspace_reset(None, 512, 512, None) == -1
    assert L.wave_gemm_streamk_counters_check(None, 512, 512, None) == -1


def _fa(L, **kw):
    a = dict(Q=16, K=32, V=48, O=64, B=1, Hq=2, Hkv=2, S=256, D=128, dt=2, causal=0, scale=0.0)
    a.update(kw)
    return L.wave_fa_fwd_launch(a["Q"], a["K"], a["V"], a["O"], a["B"], a["Hq"], a["Hkv"],
                                a["S"], a["D"], a["dt"], a["causal"], a["scale"], None)


@pytest.mark.parametrize("kw,status", [
    (dict(Q=None), -1), (dict(B=0), -1), (dict(S=0), -1), (dict(Hq=3, Hkv=2), -1),
    (dict(dt=0), -1), (dict(causal=2), -1), (dict(scale=-1.0), -1), (dict(Q=17), -1),
    (dict(D=64), -2),
])
def test_fa_rejects_bad_arguments(wave, kw, status):
    L = wave.runtime.lib()
    assert _fa(L, **kw) == status


def test_fa_f32_rejects_bad_arguments(wave):
    L = wave.runtime.lib()
    assert L.wave_fa_f32_launch(None, 32, 48, 64, 16, 16, 32, None) == -1
    assert L.wave_fa_f32_launch(16, 32, 48, 64, 0, 16, 32, None) == -1
    assert L.wave_fa_f32_launch(16, 32, 48, 64, 16, 20000, 32, None) == -2


def test_product_does_not_import_oracle():
    """The product package never imports, links or loads the CPU checker."""
    import os
    import re
    root = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "7_amd")
    for dirpath, _, files in os.walk(root):
        for f in files:
            if f.endswith((".py", ".cpp", ".hip", ".hpp", ".h")):
                text = open(os.path.join(dirpath, f)).read()
                assert not re.search(r"liboracle|import oracle|from oracle|oracle\.h|oracle/",
                                     text), f
