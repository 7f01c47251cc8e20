"""ctypes binding of libwave_runtime.so (declared in include/wave_runtime.h).

The library is the product: every entry point here calls hand-written
gfx950 kernels through the C ABI.  There is no fallback: if the library is
missing, `lib()` raises.
"""

from __future__ import annotations

import ctypes
import os
import re

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libwave_runtime.so")
HEADER_PATH = os.path.join(os.path.dirname(_HERE), "include", "wave_runtime.h")

F32, F16, BF16 = 0, 1, 2
ROW_MAJOR, COL_MAJOR, TILE_PACKED = 0, 1, 2
OK, ERR_INVALID, ERR_UNSUPPORTED, ERR_WORKSPACE = 0, -1, -2, -3

_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float
_SZ = ctypes.c_size_t

_SIGNATURES = {
    "wave_gemm_launch": (_I, [_P, _P, _P, _I, _I, _I, _I, _I, _I, _P]),
    "wave_gemm_tile_packed_launch": (_I, [_P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I, _I,
                                          _P]),
    "wave_gemm_mxfp4_launch": (_I, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P]),
    "wave_gemm_mxfp4_aiter_launch": (_I, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P]),
    "wave_gemm_streamk_workspace_bytes": (_I, [_I, _I, _I, ctypes.POINTER(_SZ),
                                               ctypes.POINTER(_SZ)]),
    "wave_gemm_streamk_launch": (_I, [_P, _P, _P, _I, _I, _I, _I, _I, _I, _P, _P, _I, _P]),
    "wave_gemm_streamk_noalloc_launch": (_I, [_P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _P]),
    "wave_gemm_auto_workspace_bytes": (_I, [_I, _I, _I, ctypes.POINTER(_SZ)]),
    "wave_gemm_auto_launch": (_I, [_P, _P, _P, _I, _I, _I, _I, _I, _I, _P, _SZ, _P]),
    "wave_gemm_streamk_workspace_reset": (_I, [_P, _I, _I, _P]),
    "wave_gemm_streamk_counters_check": (_I, [_P, _I, _I, _P]),
    "wave_fa_fwd_launch": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _F, _P]),
    "wave_fa_fwd_bounded_launch": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _F, _F,
                                        _P]),
    "wave_fa_fwd_config_launch": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _F, _F, _I,
                                       _P]),
    "wave_fa_f32_launch": (_I, [_P, _P, _P, _P, _I, _I, _I, _P]),
    "wave_fa_fwd_lse_launch": (_I, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _F, _P]),
    "wave_fa_fwd_mxfp8_launch": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I,
                                      _I, _F, _P]),
    "wave_fa_bwd_launch": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I,
                                _I, _I, _F, _P]),
    "wave_status_string": (ctypes.c_char_p, [_I]),
    "wave_last_error": (ctypes.c_char_p, []),
    "wave_device_mfma_peak": (_I, [_I, ctypes.POINTER(ctypes.c_double),
                                   ctypes.POINTER(ctypes.c_double), ctypes.POINTER(_I)]),
}
for _t in ("i32", "i8", "f32", "f16", "bf16", "i64", "f64"):
    _SIGNATURES[f"_mlir_ciface_wave_memref_to_ptr_global_{_t}"] = (_P, [_P])

_lib = None


class WaveError(RuntimeError):
    """A HIP failure or a workspace error reported by libwave_runtime."""

    def __init__(self, status: int, message: str):
        super().__init__(f"{message} (status {status})")
        self.status = status


def lib() -> ctypes.CDLL:
    """Load libwave_runtime.so (built by `make -C 7_amd/csrc`)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is not built; run __graft_entry__.build() or "
                "make -C 7_amd/csrc")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def header_symbols() -> list[str]:
    """Function names declared in include/wave_runtime.h."""
    with open(HEADER_PATH) as f:
        text = f.read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b([A-Za-z_]\w*)\s*\(", text)) -
                  {"if", "defined"})


def check(status: int) -> int:
    """Raise for a non-OK status (ValueError for argument errors, as the
    reference's Python builders do; WaveError otherwise)."""
    if status == OK:
        return status
    msg = (lib().wave_last_error() or b"").decode() or \
        lib().wave_status_string(status).decode()
    if status == ERR_INVALID:
        raise ValueError(msg)
    if status == ERR_UNSUPPORTED:
        raise NotImplementedError(msg)
    raise WaveError(status, msg)


def device_mfma_peak(device: int = 0) -> tuple[float, float, int]:
    """(dense f16 MFMA TFLOP/s, clock MHz, CUs) from hipDeviceProp_t."""
    t, c, n = ctypes.c_double(), ctypes.c_double(), ctypes.c_int()
    check(lib().wave_device_mfma_peak(device, ctypes.byref(t), ctypes.byref(c),
                                      ctypes.byref(n)))
    return t.value, c.value, n.value
