"""The gpu.binary splice of a code object (7_amd/gpu_binary.py, the text
form of the reference's wave-attach-gpu-binary, WaveAttachGPUBinary.cpp
:29-89), and the config-1 code object's own metadata: what the reference's
`gpu.launch_func @kernels::@wmma_f16_matmul_tiled` (grid (1,1,1), block 256,
no dynamic shared memory; wave_matmul.py:6954-6982) relies on.  CPU only;
the mlir-runner run itself is not available here."""

import importlib
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CONFIG1 = os.path.join(ROOT, "7_amd", "hsaco", "gemm_f16_f32_rm_32x32x64.hsaco")


@pytest.fixture(scope="module")
def gb():
    return importlib.import_module("7_amd.gpu_binary")


def unescape(s: str) -> bytes:
    """Decode an MLIR string-literal body (\\XX hex, \\\\, \\", \\n, \\t)."""
    out, i = bytearray(), 0
    while i < len(s):
        if s[i] != "\\":
            out.append(ord(s[i]))
            i += 1
        elif s[i + 1] in "\\\"nt":
            out.append({"\\": 92, '"': 34, "n": 10, "t": 9}[s[i + 1]])
            i += 2
        else:
            out.append(int(s[i + 1:i + 3], 16))
            i += 3
    return bytes(out)


def test_binary_op_round_trips_the_code_object(gb):
    data = open(CONFIG1, "rb").read()
    op = gb.binary_op(data)
    m = re.fullmatch(r'gpu\.binary @kernels \[#gpu\.object<#rocdl\.target<O = 3, triple = '
                     r'"amdgcn-amd-amdhsa", chip = "gfx950", abi = "600">, bin = "(.*)">\]', op,
                     flags=re.S)
    assert m, op[:200]
    assert unescape(m.group(1)) == data
    assert "\n" not in op and all(0x20 <= ord(c) < 0x7F for c in op)


def test_escape_covers_every_byte(gb):
    data = bytes(range(256)) * 2
    assert unescape(gb.escape(data)) == data


def test_attach_rewrites_stub_or_appends(gb):
    data = b"\x7fELF\x00\"\\x"
    host = ('module attributes {gpu.container_module} {\n'
            '  gpu.binary @kernels [#gpu.object<#rocdl.target<chip = "gfx950">, bin = "">]\n'
            '  func.func @main() { return }\n}\n')
    out = gb.attach(host, data)
    assert out.count("gpu.binary @kernels") == 1 and 'bin = ""' not in out
    assert "func.func @main" in out
    bare = 'module attributes {gpu.container_module} {\n  func.func @main() { return }\n}\n'
    out = gb.attach(bare, data)
    assert out.rstrip().endswith("}") and out.count("gpu.binary @kernels") == 1
    assert out.index("gpu.binary") > out.index("func.func @main")
    with pytest.raises(ValueError):
        gb.attach("func.func @f() { return }", data)


# A host module with the shape of the reference's mlir-runner flow
# (wave_matmul.py:11496-11514: the memref externals, `gpu.module @kernels`
# holding the kernel, then the host main whose gpu.launch_func names
# @kernels::@wmma_f16_matmul_tiled), written here by hand: nested regions,
# a kernel attribute dictionary, strings holding braces and `->` types.
HOST_MODULE = """module attributes {gpu.container_module} {
  func.func private @_mlir_ciface_wave_memref_to_ptr_global_f16(memref<?xf16>) -> !llvm.ptr
  gpu.module @kernels [#rocdl.target<chip = "gfx950">] attributes {wave.note = "{not a brace}"} {
    gpu.func @wmma_f16_matmul_tiled(%a: !llvm.ptr, %b: !llvm.ptr, %c: !llvm.ptr, %trip: i32)
        kernel attributes {gpu.known_block_size = array<i32: 256, 1, 1>} {
      %c0 = arith.constant 0 : index
      %c1 = arith.constant 1 : index
      scf.for %i = %c0 to %c1 step %c1 {
        %m = affine.apply affine_map<(d0) -> (d0 * 2)>(%i)
        // a comment with a } brace
      }
      gpu.return
    }
  }
  func.func @main() {
    %c1 = arith.constant 1 : index
    %c256 = arith.constant 256 : index
    gpu.launch_func @kernels::@wmma_f16_matmul_tiled blocks in (%c1, %c1, %c1) threads in (%c256, %c1, %c1)
    return
  }
}
"""


def test_attach_replaces_the_kernels_module(gb):
    """The compile pass's replace-and-erase (WaveCompileKernels.cpp:117-123):
    the gpu.module @kernels goes, a gpu.binary @kernels takes its place,
    and everything else, the launch included, is unchanged."""
    data = open(CONFIG1, "rb").read()
    out = gb.attach(HOST_MODULE, data)
    assert "gpu.module" not in out and "gpu.func" not in out
    assert len(re.findall(r"@kernels\b(?!::)", out)) == 1
    assert out.count("gpu.binary @kernels") == 1
    start = HOST_MODULE.index("  gpu.module")
    end = HOST_MODULE.index("  func.func @main")
    assert out.startswith(HOST_MODULE[:start] + "  gpu.binary @kernels [")
    assert out.endswith("]\n" + HOST_MODULE[end:])
    assert "gpu.launch_func @kernels::@wmma_f16_matmul_tiled blocks in" in out
    m = re.search(r'bin = "(.*?)">\]', out, flags=re.S)
    assert unescape(m.group(1)) == data


def test_attach_rejects_a_duplicate_symbol_and_unbalanced_modules(gb):
    both = HOST_MODULE.replace("  func.func @main", '  gpu.binary @kernels [#gpu.object<'
                               '#rocdl.target<chip = "gfx950">, bin = "">]\n  func.func @main')
    with pytest.raises(ValueError):
        gb.attach(both, b"\x7fELF")
    cut = HOST_MODULE[:HOST_MODULE.index("      gpu.return")]
    with pytest.raises(ValueError):
        gb.attach(cut, b"\x7fELF")
    # Another module name is left alone (the symbol is matched whole).
    other = HOST_MODULE.replace("gpu.module @kernels", "gpu.module @kernels_v2")
    out = gb.attach(other, b"\x7fELF")
    assert "gpu.module @kernels_v2" in out and out.count("gpu.binary @kernels [") == 1


def test_cli_prints_op(gb, capsys):
    assert gb.main([CONFIG1]) == 0
    assert capsys.readouterr().out.startswith("gpu.binary @kernels [#gpu.object<")


def notes(path):
    readelf = shutil.which("llvm-readelf") or "/opt/rocm/llvm/bin/llvm-readelf"
    if not os.path.exists(readelf):
        pytest.skip("llvm-readelf not available")
    return subprocess.run([readelf, "--notes", path], capture_output=True, text=True,
                          check=True).stdout


def field(text, key):
    return int(re.search(re.escape(key) + r":\s+(\d+)", text).group(1))


@pytest.mark.parametrize("name,block", [("gemm_f16_f32_rm_32x32x64", 256),
                                        ("gemm_f16_f32_rm_64x96x64_b128", 128),
                                        ("gemm_f16_f32_rm_64x32x64_b64", 64),
                                        ("gemm_f16_f16_cm_1024x512x512_b512", 512),
                                        ("gemm_f16_f16_cm_1024x512x256_b1024", 1024)])
def test_code_object_launch_metadata(name, block):
    """The launch_func contract in the object's metadata: the LDS ring is in
    the static group segment (the launch passes no dynamic shared memory),
    the block fits the kernel's flat workgroup size, and the explicit
    kernel arguments are the bare pointers A, B, C at offsets 0, 8, 16 and
    the i32 trip at 24 (gpu-to-llvm{use-bare-pointers-for-kernels=true},
    examples/wave/common.py:279-288)."""
    text = notes(os.path.join(ROOT, "7_amd", "hsaco", name + ".hsaco"))
    kern = text.split(".name:           wmma_f16_matmul_tiled")[0]
    assert field(kern, ".group_segment_fixed_size") >= 4 * 2 * 256 * 32 * 2  # 4 stages x A, B
    assert field(kern, ".max_flat_workgroup_size") == block
    args = re.findall(r"\.offset:\s+(\d+)\s+\.size:\s+(\d+)\s+\.value_kind:\s+(\w+)", kern)
    explicit = [(int(o), int(s), k) for o, s, k in args if not k.startswith("hidden")]
    assert explicit == [(0, 8, "global_buffer"), (8, 8, "global_buffer"),
                        (16, 8, "global_buffer"), (24, 4, "by_value")]
