"""Splice a code object into an MLIR host module as a `gpu.binary`.

The reference's mlir-runner flow launches its GEMM with
`gpu.launch_func @kernels::@wmma_f16_matmul_tiled` (python/mlir/dialects/
wave_matmul.py:6954-6982, module and kernel names :777-778).  Its pass
`wave-attach-gpu-binary` (lib/Dialect/Wave/Transforms/WaveAttachGPUBinary.cpp
:29-89) attaches a precompiled HSACO as a top-level `gpu.binary @kernels
[#gpu.object<#rocdl.target<O = 3, triple = .., chip = .., abi = "600">, bin =
"<HSACO bytes>">]`, rewriting a stub `gpu.binary @kernels` in place or
appending a new op; its compile pass (lib/Target/Wave/WaveCompileKernels.cpp
:103-124) puts the same op where the module's `gpu.module @kernels` was and
erases that module.  This module writes the op as text for this build's code
objects (7_amd/hsaco/*.hsaco, which carry the reference's symbols and
bare-pointer argument lists and need no dynamic LDS) and splices it into a
host module the way those passes do, so the reference's host module can run
them without the reference's MLIR build:

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


def _skip_string(text: str, i: int) -> int:
    """Index just past the string literal that opens at text[i] == '"'."""
    i += 1
    while i < len(text):
        if text[i] == "\\":
            i += 2
        elif text[i] == '"':
            return i + 1
        else:
            i += 1
    raise ValueError("unterminated string literal")


def _skip_group(text: str, i: int) -> int:
    """Index just past the bracket group that opens at text[i] ('{', '[',
    '(' or '<'), skipping string literals and `//` comments.  Braces,
    brackets and parentheses nest; angle brackets count only inside a group
    that opens with '<' (an attribute such as the offloading handler), and
    there a '>' that ends `->` does not close anything."""
    pairs = {"{": "}", "[": "]", "(": ")"}
    if text[i] == "<":
        pairs["<"] = ">"
    stack = [pairs[text[i]]]
    i += 1
    while i < len(text):
        c = text[i]
        if c == '"':
            i = _skip_string(text, i)
            continue
        if text.startswith("//", i):
            nl = text.find("\n", i)
            i = len(text) if nl < 0 else nl + 1
            continue
        if c in pairs:
            stack.append(pairs[c])
        elif c == stack[-1] and not (c == ">" and text[i - 1] == "-"):
            stack.pop()
            if not stack:
                return i + 1
        elif c in "}])" or (c == ">" and "<" in pairs and text[i - 1] != "-"):
            raise ValueError(f"unbalanced {c!r} at offset {i}")
        i += 1
    raise ValueError("unbalanced brackets")


def _find_gpu_module(text: str, symbol: str):
    """(start, end) of the `gpu.module @<symbol> ... { body }` op, or None.
    Between the name and the body the op may carry an offloading handler
    `<...>`, a target list `[...]` and `attributes {...}`
    (the gpu.module assembly format)."""
    m = re.search(r"gpu\.module\s+@" + re.escape(symbol) + r"(?![\w$.-])", text)
    if not m:
        return None
    i = m.end()
    while True:
        while i < len(text) and text[i].isspace():
            i += 1
        if i >= len(text):
            raise ValueError(f"gpu.module @{symbol} has no body")
        if text[i] in "[<":
            i = _skip_group(text, i)
        elif text.startswith("attributes", i):
            i += len("attributes")
            while i < len(text) and text[i].isspace():
                i += 1
            if i >= len(text) or text[i] != "{":
                raise ValueError(f"gpu.module @{symbol}: `attributes` without a dictionary")
            i = _skip_group(text, i)
        elif text[i] == "{":
            return m.start(), _skip_group(text, i)
        else:
            raise ValueError(f"gpu.module @{symbol}: unexpected {text[i]!r} before its body")


def attach(module_text: str, hsaco: bytes, symbol: str = GPU_MODULE, chip: str = CHIP,
           triple: str = TRIPLE) -> str:
    """Splice the code object into a host module as `gpu.binary @<symbol>`:
    * a `gpu.module @<symbol> { ... }` (what the reference's host builder
      emits, wave_matmul.py:11499) is replaced by the op, in its place (the
      compile pass's replace-and-erase, WaveCompileKernels.cpp:117-123);
    * else an existing `gpu.binary @<symbol>` stub is rewritten in place;
    * else the op is appended at the end of the top-level module body
      (WaveAttachGPUBinary.cpp:68-86).
    The `gpu.launch_func @<symbol>::@<kernel>` ops are left as they are: the
    binary takes over the symbol they reference.  A module holding both a
    gpu.module and a gpu.binary of that symbol is rejected (duplicate
    symbol)."""
    op = binary_op(hsaco, symbol, chip, triple)
    stub = re.compile(r"gpu\.binary\s+@" + re.escape(symbol) + r"(?![\w$.-])[^\n]*")
    span = _find_gpu_module(module_text, symbol)
    if span is not None:
        if stub.search(module_text):
            raise ValueError(f"both gpu.module @{symbol} and gpu.binary @{symbol} are defined")
        start, end = span
        return module_text[:start] + op + module_text[end:]
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
