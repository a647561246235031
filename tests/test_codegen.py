"""Checks on the gfx950 machine code of the built library (no GPU needed).

The direct-to-LDS loads are issued from inline assembly, where the compiler
inserts no hazard wait states.  A vector memory instruction that reads an SGPR
written by a VALU instruction (the compiler reloads spilled address SGPRs with
v_readlane) needs 5 wait states; with fewer it can form its address from a stale
SGPR.  Every such load must therefore follow an s_nop of at least 4 (5 states).
"""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "sigma-0_amd", "mamba3_rocm", "libmamba3_rocm.so")
LLVM = "/opt/rocm/llvm/bin"
TARGET = "hipv4-amdgcn-amd-amdhsa--gfx950"
MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"


def _tool(name):
    path = os.path.join(LLVM, name)
    return path if os.path.exists(path) else shutil.which(name)


def _disassembly(tmp_path):
    """gfx950 disassembly of every code object bundled into the library."""
    objcopy, bundler, objdump = _tool("llvm-objcopy"), _tool("clang-offload-bundler"), _tool("llvm-objdump")
    if not (objcopy and bundler and objdump):
        pytest.skip("ROCm LLVM tools not installed")
    if not os.path.exists(LIB):
        pytest.skip("library not built")
    fat = tmp_path / "fatbin"
    subprocess.run([objcopy, "-O", "binary", "--only-section=.hip_fatbin", LIB, str(fat)], check=True)
    data = fat.read_bytes()
    starts = [m.start() for m in re.finditer(re.escape(MAGIC), data)]
    assert starts, "no offload bundle in .hip_fatbin"
    out = []
    for i, s in enumerate(starts):
        part = tmp_path / f"bundle{i}"
        part.write_bytes(data[s:starts[i + 1] if i + 1 < len(starts) else len(data)])
        co = tmp_path / f"co{i}.o"
        subprocess.run([bundler, "--unbundle", "--type=o", f"--input={part}", f"--targets={TARGET}",
                        f"--output={co}"], check=True)
        out.append(subprocess.run([objdump, "-d", str(co)], check=True, capture_output=True,
                                  text=True).stdout)
    return "\n".join(out)


def test_lds_dma_loads_carry_their_wait_states(tmp_path):
    text = _disassembly(tmp_path)
    insts = [line.split("//")[0].strip() for line in text.splitlines()]
    insts = [i for i in insts if i and not i.endswith(":") and not i.startswith("Disassembly")]
    loads = 0
    for k, inst in enumerate(insts):
        if inst.startswith("global_load_lds"):
            loads += 1
            prev = insts[k - 1].split()
            assert prev[0] == "s_nop" and int(prev[1], 0) >= 4, (inst, insts[k - 3:k])
    assert loads > 0, "the chunked scan stages its inputs with direct-to-LDS loads"
