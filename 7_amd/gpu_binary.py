"""Splice a code object into an MLIR host module as a `gpu.binary`.

The reference's mlir-runner flow launches its GEMM with
`gpu.launch_func @kernels::@wmma_f16_matmul_tiled` (python/mlir/dialects/
wave_matmul.py:6954-6982, module and kernel names :777-778).  Its pass
`wave-attach-gpu-binary` (lib/Dialect/Wave/Transforms/WaveAttachGPUBinary.cpp
:29-89) swaps a precompiled HSACO in for the `gpu.module @kernels`: a
top-level `gpu.binary @kernels [#gpu.object<#rocdl.target<O = 3, triple = ..,
chip = .., abi = "600">, bin = "<HSACO bytes>">]`, rewriting a stub
`gpu.binary @kernels` in place or appending a new op.  This module writes the
same op as text for this build's code objects (7_amd/hsaco/*.hsaco, which
carry the reference's symbols and bare-pointer argument lists and need no
dynamic LDS), so the reference's host module can run them without the
reference's MLIR build:

    python -m 7_amd.gpu_binary 7_amd/hsaco/gemm_f16_f32_rm_32x32x64.hsaco \\
        [--symbol kernels] [--chip gfx950] [--module host.mlir] > out.mlir

Only the text transformation lives here; running the resulting module needs
an mlir-runner with the ROCm runtime wrappers.
"""

from __future__ import annotations

import argparse
import re
import sys

TRIPLE = "amdgcn-amd-amdhsa"
CHIP = "gfx950"
GPU_MODULE = "kernels"  # wave_matmul.py:778 _GPU_MODULE_NAME

_PLAIN = set(range(0x20, 0x7F)) - {ord('"'), ord("\\")}


def escape(data: bytes) -> str:
    """MLIR string-literal body for arbitrary bytes: printable ASCII as is,
    everything else (and the quote and backslash) as a two-digit hex escape
    (the lexer's \\XX form)."""
    return "".join(chr(b) if b in _PLAIN else f"\\{b:02X}" for b in data)


def object_attr(hsaco: bytes, chip: str = CHIP, triple: str = TRIPLE) -> str:
    """The #gpu.object the attach pass builds: ROCDL target with O = 3, the
    given triple and chip, no features, ABI "600", binary compilation
    target (WaveAttachGPUBinary.cpp:55-66)."""
    target = f'#rocdl.target<O = 3, triple = "{triple}", chip = "{chip}", abi = "600">'
    return f'#gpu.object<{target}, bin = "{escape(hsaco)}">'


def binary_op(hsaco: bytes, symbol: str = GPU_MODULE, chip: str = CHIP,
              triple: str = TRIPLE) -> str:
    return f"gpu.binary @{symbol} [{object_attr(hsaco, chip, triple)}]"


def attach(module_text: str, hsaco: bytes, symbol: str = GPU_MODULE, chip: str = CHIP,
           triple: str = TRIPLE) -> str:
    """Rewrite an existing `gpu.binary @<symbol>` stub, or append the op at
    the end of the top-level module body (WaveAttachGPUBinary.cpp:68-86)."""
    op = binary_op(hsaco, symbol, chip, triple)
    stub = re.compile(r"gpu\.binary\s+@" + re.escape(symbol) + r"\b[^\n]*")
    if stub.search(module_text):
        return stub.sub(lambda _: op, module_text, count=1)
    end = module_text.rstrip().rfind("}")
    if not re.match(r"\s*module\b", module_text) or end < 0:
        raise ValueError("expected a `module { ... }` to append the gpu.binary to")
    return module_text[:end] + "  " + op + "\n" + module_text[end:]


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("hsaco")
    ap.add_argument("--symbol", default=GPU_MODULE)
    ap.add_argument("--chip", default=CHIP)
    ap.add_argument("--triple", default=TRIPLE)
    ap.add_argument("--module", help="host module to splice into (default: print the op)")
    a = ap.parse_args(argv)
    with open(a.hsaco, "rb") as f:
        data = f.read()
    if data[:4] != b"\x7fELF":
        print(f"{a.hsaco}: not an ELF code object", file=sys.stderr)
        return 2
    if a.module:
        with open(a.module) as f:
            sys.stdout.write(attach(f.read(), data, a.symbol, a.chip, a.triple))
    else:
        print(binary_op(data, a.symbol, a.chip, a.triple))
    return 0


if __name__ == "__main__":
    sys.exit(main())
