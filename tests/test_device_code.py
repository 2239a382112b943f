"""Checks on the gfx950 machine code of this build's own lib/libom_hip.so (CPU only: the code objects are taken out of
the library's offload bundles and disassembled with the ROCm toolchain's llvm-objdump).

The direct-to-LDS GEMM loads (k_gemm_xd) are inline assembly that sets m0 right before each
global_load_lds_dwordx4: the LDS destination of that instruction comes from m0. The compiler treats m0 as reserved
and does not keep a value of its own there across such a statement, so the loads are only safe if no instruction the
compiler emits anywhere in the library reads or writes m0. This test checks exactly that on the built code: every
instruction that names m0 is an `s_mov_b32 m0, ...` immediately followed by a global_load_lds_dwordx4, and every
global_load_lds instruction immediately follows such a move.
"""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "onemodel-csharp_amd", "lib", "libom_hip.so")
LLVM = "/opt/rocm/llvm/bin"
MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"


def _code_objects(tmp):
    if not os.path.exists(LIB):
        pytest.skip("lib/libom_hip.so is not built")
    for tool in ("objcopy",):
        if not shutil.which(tool):
            pytest.skip(f"{tool} is not installed")
    for tool in ("clang-offload-bundler", "llvm-objdump"):
        if not os.path.exists(os.path.join(LLVM, tool)):
            pytest.skip(f"{tool} is not installed")
    fat = os.path.join(tmp, "fatbin")
    subprocess.run(["objcopy", "-O", "binary", "--only-section=.hip_fatbin", LIB, fat], check=True)
    data = open(fat, "rb").read()
    starts = [m.start() for m in re.finditer(re.escape(MAGIC), data)] + [len(data)]
    assert len(starts) > 1, "no offload bundle in the library"
    out = []
    for i, (a, b) in enumerate(zip(starts, starts[1:])):
        bundle, co = os.path.join(tmp, f"b{i}"), os.path.join(tmp, f"b{i}.co")
        with open(bundle, "wb") as f:
            f.write(data[a:b])
        subprocess.run([os.path.join(LLVM, "clang-offload-bundler"), "--unbundle", "--type=o",
                        "--targets=hipv4-amdgcn-amd-amdhsa--gfx950", f"--input={bundle}", f"--output={co}"],
                       check=True)
        out.append(co)
    return out


def test_only_the_lds_loads_touch_m0(tmp_path):
    cos = _code_objects(str(tmp_path))
    moves = loads = 0
    for co in cos:
        dis = subprocess.run([os.path.join(LLVM, "llvm-objdump"), "-d", "--no-show-raw-insn", co], check=True,
                             capture_output=True, text=True).stdout
        prev, func = "", ""
        for line in dis.splitlines():
            m = re.match(r"^[0-9a-f]+ <(.+)>:$", line)
            if m:
                func, prev = m.group(1), ""
                continue
            ins = line.split("//")[0].strip()
            if not ins or ins.endswith(":"):
                continue
            op = ins.split()[0]
            if re.search(r"\bm0\b", ins):
                assert op == "s_mov_b32" and ins.split()[1].rstrip(",") == "m0", (func, ins)
                moves += 1
            if op.startswith("global_load_lds"):
                assert prev.startswith("s_mov_b32 m0"), (func, prev, ins)
                loads += 1
            elif prev.startswith("s_mov_b32 m0"):
                raise AssertionError(f"{func}: m0 set but not used by the next instruction ({ins})")
            prev = ins
    assert moves == loads and loads > 0, (moves, loads)


def test_every_kernel_poisons_its_lds_first():
    """The checked build fills each workgroup's LDS with 0xFF before the kernel's own code (OM_LDS_POISON), so a read
    of LDS that nothing wrote yields NaN. That only holds if every kernel starts with the macro."""
    import glob
    srcs = sorted(glob.glob(os.path.join(ROOT, "onemodel-csharp_amd", "csrc", "*.hip")) +
                  glob.glob(os.path.join(ROOT, "onemodel-csharp_amd", "csrc", "*.hpp")))
    kernels, missing = 0, []
    for path in srcs:
        text = open(path).read()
        for m in re.finditer(r"__global__[^{;]*\{", text):
            kernels += 1
            first = text[m.end():].lstrip().split("\n", 1)[0]
            if not first.startswith("OM_LDS_POISON();"):
                name = re.findall(r"(\w+)\s*\(", text[m.start():m.end()])
                missing.append((os.path.basename(path), name[0] if name else "?"))
    assert kernels > 50 and not missing, missing
