"""wave-mi355x: MI355X-native (gfx950) drop-in for the reference's GEMM,
Stream-K GEMM, MXFP4 scaled GEMM and flash-attention forward kernels.

The package directory name starts with a digit, so import it with
``importlib.import_module("7_amd")``.  The compute lives in
``libwave_runtime.so`` (hand-written HIP, C ABI in include/wave_runtime.h);
``ops`` wraps it for torch tensors and ``runtime`` is the ctypes binding.
``code_object`` loads the reference-ABI code objects (``hsaco/*.hsaco``:
the reference's kernel symbols, one shape each) with hipModuleLoad.
"""

from . import code_object, runtime
from .ops import (StreamKWorkspace, flash_attention, flash_attention_bwd,
                  flash_attention_f32, flash_attention_lse, flash_attention_mxfp8, gemm,
                  gemm_auto, gemm_auto_workspace_bytes, gemm_mxfp4, gemm_streamk,
                  gemm_tile_packed, mxfp8_quantize, streamk_workspace_bytes)
from .runtime import WaveError

__all__ = [
    "runtime", "code_object", "gemm", "gemm_auto", "gemm_auto_workspace_bytes",
    "gemm_tile_packed", "gemm_mxfp4", "gemm_streamk",
    "StreamKWorkspace", "streamk_workspace_bytes",
    "flash_attention", "flash_attention_lse", "flash_attention_bwd", "flash_attention_f32",
    "flash_attention_mxfp8", "mxfp8_quantize",
    "WaveError",
]
