"""Builds the two native libraries of the package in-tree:

  lib/libom_hip.so    the gfx950 HIP kernels and the C ABI of include/om.h (hipcc)
  lib/libom_train.so  the C++ training tape of include/om_train.h, linked against libom_hip.so (g++)

Run `python onemodel-csharp_amd/build.py` (or __graft_entry__.build()). Every call recompiles.
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
TRAIN = os.path.join(PKG, "train")
LIB = os.path.join(PKG, "lib")
OBJ = os.path.join(PKG, "_build")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
# gfx950 only. Packed-fp32 instructions are switched off (they have given silent wrong results on these boxes);
# -ffp-contract=off keeps every multiply and add separately rounded unless the code asks for a fused operation,
# and fp32 division/sqrt are correctly rounded, which the optimizer's bit-exactness relies on.
HIP_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
    "-fhip-fp32-correctly-rounded-divide-sqrt", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-result",
]
# OM_TUNING_KNOBS=1 at build time makes a tuning build, whose comparison knobs (OM_GEMM_X, OM_GEMM_DMA,
# OM_GROUP_BAND, OM_CONV3, OM_ATTN_PATH, OM_EMBEDDING_SORT) are read from the environment at run time; the default
# build reads none, so its kernel choices depend on the shapes alone.
if os.environ.get("OM_TUNING_KNOBS") == "1":
    HIP_FLAGS.append("-DOM_TUNING_KNOBS")
CXX_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-ffp-contract=off", "-Wall", "-Wno-unused-function"]


def _run(cmd):
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if r.returncode != 0:
        raise RuntimeError("build failed: " + " ".join(cmd) + "\n" + r.stdout)
    return r.stdout


def _obj_dir(lib: str) -> str:
    """Object files of one output directory's build (builds into different directories may run at once)."""
    return OBJ if os.path.abspath(lib) == LIB else os.path.join(OBJ + "_" + os.path.basename(os.path.abspath(lib)))


def build_hip(jobs: int = 8, lib: str = LIB, extra=()) -> str:
    os.makedirs(lib, exist_ok=True)
    obj = _obj_dir(lib)
    os.makedirs(obj, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    objs = [os.path.join(obj, os.path.basename(s) + ".o") for s in srcs]
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(lambda so: _run([HIPCC, *HIP_FLAGS, *extra, "-c", so[0], "-o", so[1]]), zip(srcs, objs)))
    out = os.path.join(lib, "libom_hip.so")
    tmp = out + ".tmp"
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs])
    os.replace(tmp, out)
    return out


def build_train(lib: str = LIB) -> str | None:
    srcs = sorted(glob.glob(os.path.join(TRAIN, "*.cpp")))
    if not srcs:
        return None
    out = os.path.join(lib, "libom_train.so")
    tmp = out + ".tmp"
    rocm_inc = "/opt/rocm/include"
    _run(["g++", *CXX_FLAGS, "-shared", "-I", os.path.join(ROOT, "include"), "-I", rocm_inc, "-o", tmp, *srcs,
          "-L", lib, "-lom_hip", "-Wl,-rpath,$ORIGIN"])
    os.replace(tmp, out)
    return out


def build_all(lib: str = LIB, checked: bool = False) -> list[str]:
    """Both libraries into `lib`. checked: the checked build (-DOM_CHECKED: LDS, arena allocations and context scratch
    handed out filled with 0xFF, a NaN for floats), for a test run that flushes out reads of memory nothing wrote."""
    built = [build_hip(lib=lib, extra=("-DOM_CHECKED",) if checked else ())]
    t = build_train(lib)
    if t:
        built.append(t)
    shutil.rmtree(_obj_dir(lib), ignore_errors=True)
    return built


if __name__ == "__main__":
    # python build.py                 the product libraries into lib/
    # python build.py --checked DIR   the checked build into DIR (copy both files over lib/ to run the tests with it)
    args = sys.argv[1:]
    if args[:1] == ["--checked"] and len(args) == 2:
        out = build_all(os.path.abspath(args[1]), checked=True)
    else:
        out = build_all()
    for p in out:
        print("built", p)
    sys.exit(0)
