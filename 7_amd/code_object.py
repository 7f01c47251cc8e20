"""Load and launch the reference-ABI code objects (`7_amd/hsaco/*.hsaco`).

These are the kernels of `7_amd/csrc/ref_abi.hip` compiled per shape under
the reference's symbol names and bare-pointer argument lists
(`wmma_f16_matmul_tiled`, `gfx950_f16_streamk_gemm`,
`flash_attention_bf16_gfx950`, `flash_attention_f32`).  The reference's C++
runners load them with `hipModuleLoad` + `hipModuleLaunchKernel`
(tools/wave-matmul-calibrate/wave-matmul-calibrate-runner.cpp:1852-1860,
tools/wave-fa-calibrate/wave-fa-gfx950-runner.cpp:396-428); this module does
the same from Python, in the style of the reference's ctypes helper
(test/Integration/Inputs/hip_runtime.py:20-41).  Device memory comes from
torch tensors and launches go to torch's current stream.

Build more shapes with `make -C 7_amd/csrc hsaco NAME=... DEFS=...`.
"""

import ctypes
import os

HSACO_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "hsaco")

# hipFuncAttributeMaxDynamicSharedMemorySize (hip_runtime_api.h).
_MAX_DYNAMIC_SHARED = 8

_HIP = None


def hip() -> ctypes.CDLL:
    """The HIP runtime already in this process (torch loads libamdhip64.so.7;
    opening the same soname returns that instance, so tensors and modules
    share one device context)."""
    global _HIP
    if _HIP is None:
        import torch

        torch.cuda.init()
        h = ctypes.CDLL("libamdhip64.so.7")
        h.hipModuleLoad.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_char_p]
        h.hipModuleGetFunction.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_void_p,
                                           ctypes.c_char_p]
        h.hipModuleUnload.argtypes = [ctypes.c_void_p]
        h.hipFuncSetAttribute.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int]
        h.hipModuleLaunchKernel.argtypes = [ctypes.c_void_p] + [ctypes.c_uint] * 7 + [
            ctypes.c_void_p, ctypes.POINTER(ctypes.c_void_p), ctypes.POINTER(ctypes.c_void_p)]
        h.hipGetErrorString.restype = ctypes.c_char_p
        h.hipGetErrorString.argtypes = [ctypes.c_int]
        _HIP = h
    return _HIP


def _check(err: int, what: str) -> None:
    if err != 0:
        raise RuntimeError(f"{what}: {hip().hipGetErrorString(err).decode()} ({err})")


def path(name: str) -> str:
    """Path of a built code object by name (`gemm_f16_f32_rm_32x32x64`)."""
    p = os.path.join(HSACO_DIR, name + ".hsaco")
    if not os.path.exists(p):
        raise FileNotFoundError(f"{p} is not built (make -C 7_amd/csrc hsacos)")
    return p


def arg(value):
    """A kernel argument as a ctypes value: tensors and None become bare
    device pointers, Python ints become int32."""
    if value is None:
        return ctypes.c_void_p(0)
    if hasattr(value, "data_ptr"):
        return ctypes.c_void_p(value.data_ptr())
    if isinstance(value, int):
        return ctypes.c_int32(value)
    return value


class Kernel:
    def __init__(self, module, handle, name):
        self._module = module  # keeps the module loaded
        self.handle = handle
        self.name = name

    def launch(self, grid, block, args, dynamic_lds=0, stream=None):
        """hipModuleLaunchKernel with the reference's bare-pointer arguments."""
        import torch

        vals = [arg(a) for a in args]
        params = (ctypes.c_void_p * len(vals))(
            *[ctypes.cast(ctypes.pointer(v), ctypes.c_void_p) for v in vals])
        if dynamic_lds:
            _check(hip().hipFuncSetAttribute(self.handle, _MAX_DYNAMIC_SHARED, dynamic_lds),
                   "hipFuncSetAttribute")
        if stream is None:
            stream = torch.cuda.current_stream().cuda_stream
        g = tuple(grid) + (1,) * (3 - len(grid))
        b = tuple(block) + (1,) * (3 - len(block))
        _check(hip().hipModuleLaunchKernel(self.handle, *g, *b, dynamic_lds, stream, params,
                                           None), f"hipModuleLaunchKernel {self.name}")


class CodeObject:
    """One loaded code object (hipModuleLoad)."""

    def __init__(self, name_or_path: str):
        p = name_or_path if os.path.sep in name_or_path else path(name_or_path)
        self.handle = ctypes.c_void_p()
        _check(hip().hipModuleLoad(ctypes.byref(self.handle), p.encode()), f"hipModuleLoad {p}")

    def kernel(self, symbol: str) -> Kernel:
        fn = ctypes.c_void_p()
        _check(hip().hipModuleGetFunction(ctypes.byref(fn), self.handle, symbol.encode()),
               f"hipModuleGetFunction {symbol}")
        return Kernel(self, fn, symbol)

    def close(self):
        if self.handle:
            _check(hip().hipModuleUnload(self.handle), "hipModuleUnload")
            self.handle = ctypes.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()
