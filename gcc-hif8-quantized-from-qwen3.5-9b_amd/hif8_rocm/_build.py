"""In-tree build of the HiF8 HIP library and its torch extension.

Produces, next to this file:
  libhif8_rocm.so                     HIP kernels + the C ABI (include/hif8_rocm.h), gfx950
  _C.cpython-*.so                     thin torch extension registering torch.ops.vllm_ascend_hif8.*

Run ``python -m hif8_rocm._build`` (or ``__graft_entry__.build()``).  hipcc
cross-compiles gfx950 code objects without a GPU present.
"""

from __future__ import annotations

import os
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR.parent / "csrc"
REPO = PKG_DIR.parent.parent
INCLUDE = REPO / "include"
BUILD_DIR = PKG_DIR.parent / "_build"
LIB_NAME = "libhif8_rocm.so"
ARCH = os.environ.get("HIF8_OFFLOAD_ARCH", "gfx950")
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))

HIP_SOURCES = ["capi.hip", "static_quant.hip", "gemv.hip", "gemm.hip", "linear_api.hip", "kv_cache.hip",
               "embedding.hip", "model_ops.hip", "prefill_attention.hip"]

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # Correctly rounded FP32 division is part of the static-quant contract.
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    # No packed FP32 instructions in any kernel.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(
        line for line in proc.stdout.splitlines() if "packed-fp32-ops" not in line
    )
    if proc.returncode != 0:
        raise RuntimeError(f"build step failed ({proc.returncode}): {' '.join(cmd)}\n{out}")


def _hipcc() -> str:
    cand = ROCM / "bin" / "hipcc"
    return str(cand) if cand.exists() else "hipcc"


def build_hip_library(jobs: int = 8) -> Path:
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    objs = []
    cmds = []
    for src in HIP_SOURCES:
        obj = BUILD_DIR / (Path(src).stem + ".o")
        objs.append(obj)
        cmds.append([_hipcc(), *HIPCC_FLAGS, "-c", str(CSRC / src), "-o", str(obj)])
    with ThreadPoolExecutor(max_workers=max(1, min(jobs, len(cmds)))) as pool:
        list(pool.map(_run, cmds))
    out = PKG_DIR / LIB_NAME
    tmp = out.with_suffix(".so.tmp")
    _run([_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)])
    os.replace(tmp, out)
    return out


def build_torch_extension() -> Path:
    import torch
    from torch.utils import cpp_extension

    suffix = sysconfig.get_config_var("EXT_SUFFIX") or ".so"
    out = PKG_DIR / f"_C{suffix}"
    tmp = out.with_suffix(".tmp")
    torch_lib = Path(torch.__file__).resolve().parent / "lib"
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cmd = [
        "g++", "-O2", "-std=c++17", "-fPIC", "-shared",
        "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
        "-DTORCH_EXTENSION_NAME=_C", "-DTORCH_API_INCLUDE_EXTENSION_H",
        f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
        *[f"-I{p}" for p in cpp_extension.include_paths()],
        f"-I{sysconfig.get_paths()['include']}",
        f"-I{ROCM / 'include'}",
        f"-I{INCLUDE}",
        str(CSRC / "torch_bridge.cpp"),
        "-o", str(tmp),
        f"-L{torch_lib}", "-lc10", "-ltorch", "-ltorch_cpu", "-ltorch_python", "-lc10_hip", "-ltorch_hip",
        f"-L{ROCM / 'lib'}", "-lamdhip64",
        f"-L{PKG_DIR}", "-l:" + LIB_NAME,
        "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{torch_lib}",
    ]
    _run(cmd)
    os.replace(tmp, out)
    return out


def build(jobs: int = 8) -> None:
    build_hip_library(jobs)
    build_torch_extension()


if __name__ == "__main__":
    build(int(sys.argv[1]) if len(sys.argv) > 1 else 8)
    print("built", PKG_DIR / LIB_NAME)
