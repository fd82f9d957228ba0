"""Build libllmik_hip.so (the gfx950 kernels + C ABI) in-tree with hipcc.

Usage: python llm-inference-kernels_amd/build_lib.py [--jobs N]

Every translation unit under csrc/ is compiled for gfx950 only, without
fast-math (the KV writers must divide exactly), and linked into
llmik_cuda/libllmik_hip.so next to the Python package that loads it.
The measurement floors (csrc_diag/, include/llmik_diag.h) are linked into
llmik_cuda/libllmik_diag.so, a library of their own.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_ROOT = Path(__file__).resolve().parent
CSRC = PKG_ROOT / "csrc"
CSRC_DIAG = PKG_ROOT / "csrc_diag"
OUT_DIR = PKG_ROOT / "llmik_cuda"
LIB_NAME = "libllmik_hip.so"
DIAG_LIB_NAME = "libllmik_diag.so"
OBJ_DIR = PKG_ROOT / "_build"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fvisibility=hidden",
    # Packed-fp32 VALU forms are kept out of the generated code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]


def sources(d: Path = CSRC) -> list[Path]:
    return sorted(list(d.glob("*.hip")) + list(d.glob("*.cpp")))


def compile_one(src: Path) -> Path:
    obj = OBJ_DIR / (src.parent.name + "_" + src.stem + ".o")
    cmd = [HIPCC, *COMMON_FLAGS, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stdout}\n{res.stderr}")
    # The host pass warns about the gfx feature flag; show anything else.
    msgs = [ln for ln in (res.stderr or "").splitlines()
            if ln.strip() and "packed-fp32-ops" not in ln and "not a recognized feature" not in ln]
    if msgs:
        print("\n".join(msgs), file=sys.stderr)
    return obj


def _link(objs: list[Path], out: Path) -> Path:
    tmp = out.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, out)
    return out


def build(jobs: int = 8) -> Path:
    """Build libllmik_hip.so and, beside it, libllmik_diag.so; returns the
    path of the product library."""
    if not Path(HIPCC).exists() and shutil.which("hipcc") is None:
        raise RuntimeError("hipcc not found; set HIPCC or install ROCm")
    OBJ_DIR.mkdir(exist_ok=True)
    srcs = sources()
    diag_srcs = sources(CSRC_DIAG)
    with cf.ThreadPoolExecutor(max_workers=max(1, min(jobs, len(srcs) + len(diag_srcs)))) as ex:
        objs = list(ex.map(compile_one, srcs + diag_srcs))
    _link(objs[len(srcs):], OUT_DIR / DIAG_LIB_NAME)
    return _link(objs[:len(srcs)], OUT_DIR / LIB_NAME)


TORCH_SRC = PKG_ROOT / "csrc_torch" / "torch_ops.cpp"


def build_torch_ext() -> Path:
    """Compile llmik_cuda/_C (csrc_torch/torch_ops.cpp, the torch-facing
    validation / allocation / stream half of the ops) with the host C++
    compiler against torch's headers, linked to libllmik_hip.so (found next
    to it through an $ORIGIN rpath)."""
    import sysconfig

    import torch
    from torch.utils import cpp_extension as ce
    cxx = os.environ.get("CXX", "g++")
    out = OUT_DIR / ("_C" + sysconfig.get_config_var("EXT_SUFFIX"))
    tmp = out.with_suffix(".tmp")
    inc = [*ce.include_paths(), sysconfig.get_paths()["include"], "/opt/rocm/include"]
    cmd = [cxx, "-O2", "-std=c++17", "-fPIC", "-shared", "-fvisibility=hidden",
           "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", "-DTORCH_EXTENSION_NAME=_C",
           "-DTORCH_API_INCLUDE_EXTENSION_H",
           f"-D_GLIBCXX_USE_CXX11_ABI={int(torch._C._GLIBCXX_USE_CXX11_ABI)}",
           *[f"-I{d}" for d in inc], str(TORCH_SRC), "-o", str(tmp),
           *[f"-L{d}" for d in ce.library_paths()], "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu",
           "-ltorch_python", f"-L{OUT_DIR}", "-lllmik_hip", "-Wl,-rpath,$ORIGIN"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"torch extension build failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, out)
    return out


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=8)
    args = ap.parse_args()
    print(build(args.jobs))
    print(build_torch_ext())


if __name__ == "__main__":
    main()
