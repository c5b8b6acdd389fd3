"""Builds the MI355X SpMM library and its PyTorch extension in-tree.

* ``libspmm_mi355x.so``: the HIP kernels and the C ABI (``include/spmm_mi355x.h``),
  compiled by hipcc for gfx950 only.
* ``custom_ops_lib*.so``: the PyTorch-ROCm extension imported by ``spmm_npu``,
  compiled by g++ against the torch headers and linked to the library above
  (found next to it through an ``$ORIGIN`` run path).

Run ``python ascend-spmm_amd/build.py``; objects go to ``_build/`` at the
repository root and the two shared objects land in this directory.
"""

from __future__ import annotations

import concurrent.futures
import os
import subprocess
import sys
import sysconfig

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(REPO, "_build")
LIBRARY = os.path.join(HERE, "libspmm_mi355x.so")
EXTENSION = os.path.join(HERE, "custom_ops_lib" + sysconfig.get_config_var("EXT_SUFFIX"))

HIP_SOURCES = [
    "spmm_capi.hip",
    "spmm_gather.hip",
    "spmm_block.hip",
    "permute_rows.hip",
    "spmm_cubeop.hip",
    "spmm_rowscalar.hip",
    "preprocess.hip",
]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
# Packed-FP32 instructions (v_pk_*_f32) are disabled for all device code:
# some of their forms have produced silently wrong results on MI355X boxes.
HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    # hipcc's host pass does not know the device feature flag; drop that note.
    lines = [
        ln for ln in proc.stdout.splitlines()
        if "packed-fp32-ops' is not a recognized feature" not in ln
    ]
    if proc.returncode != 0:
        sys.stderr.write("\n".join(lines) + "\n")
        raise RuntimeError(f"build step failed ({proc.returncode}): {' '.join(cmd)}")
    if lines:
        sys.stderr.write("\n".join(lines) + "\n")


def _compile_hip(src: str) -> str:
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
    _run([HIPCC, *HIPCC_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj])
    return obj


def build_library() -> str:
    os.makedirs(BUILD, exist_ok=True)
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(HIP_SOURCES))) as pool:
        objs = list(pool.map(_compile_hip, HIP_SOURCES))
    tmp = LIBRARY + ".tmp"
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", tmp,
          "-Wl,-soname,libspmm_mi355x.so"])
    os.replace(tmp, LIBRARY)
    return LIBRARY


def build_extension() -> str:
    import torch  # noqa: F401  (only for its install location)
    from torch.utils import cpp_extension

    torch_lib = cpp_extension.library_paths()[0]
    includes = cpp_extension.include_paths() + [
        sysconfig.get_paths()["include"],
        "/opt/rocm/include",
    ]
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    tmp = EXTENSION + ".tmp"
    cmd = [
        "g++", "-O2", "-std=c++17", "-fPIC", "-shared",
        f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
        "-DTORCH_EXTENSION_NAME=custom_ops_lib",
        "-DTORCH_API_INCLUDE_EXTENSION_H",
        "-D__HIP_PLATFORM_AMD__=1",
        "-DUSE_ROCM=1",
        *[f"-I{p}" for p in includes],
        os.path.join(CSRC, "torch_ext", "custom_op.cpp"),
        "-o", tmp,
        f"-L{torch_lib}", "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_python",
        f"-L{HERE}", "-lspmm_mi355x",
        "-Wl,-rpath,$ORIGIN",
        f"-Wl,-rpath,{torch_lib}",
    ]
    _run(cmd)
    os.replace(tmp, EXTENSION)
    return EXTENSION


def build() -> None:
    build_library()
    build_extension()


if __name__ == "__main__":
    build()
    print(LIBRARY)
    print(EXTENSION)
