"""Builds libslm_attn.so (HIP, gfx950) in-tree with hipcc.

Every HIP source is compiled with packed-fp32 ops disabled, no fast-math and
warnings as errors;
the RoPE/append kernels additionally switch FMA contraction off in source so
that the KV rows they write are bit-identical to the reference's f32
arithmetic.
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
HOST = PKG_DIR / "host"
REPO = PKG_DIR.parent
LIB = PKG_DIR / "libslm_attn.so"
HOST_DEMO = PKG_DIR / "slm_host_demo"
BUILD_DIR = PKG_DIR / "_build"

HIP_SOURCES = ["slm_attn.hip", "slm_layer.hip", "slm_model.hip", "rope_append.hip",
               "attn_decode.hip", "prefill_mfma.hip", "quant_gemm.hip", "norm_act.hip"]
# measurement probes of the bench, a library of their own (not the product's)
CALIB_DIR = PKG_DIR / "calib"
CALIB_LIB = CALIB_DIR / "libslm_calib.so"
# host-only C++ (no device code), compiled with the host compiler
CPP_SOURCES = ["gguf.cpp"]
CXX_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-Wall", "-Wextra", "-Werror",
             f"-I{REPO / 'include'}", f"-I{CSRC}"]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
HIP_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Werror",
    "-Wno-unused-result",
    # packed FP32 (v_pk_*_f32) is kept out of the generated code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{REPO / 'include'}",
    f"-I{CSRC}",
]
# per-source extras: the Q4_0 GEMM's MFMA results go straight to VGPRs (its
# epilogue reads every one; accumulator registers would cost a
# v_accvgpr_read per element)
HIP_SOURCE_FLAGS = {"quant_gemm.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"]}


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    # the host pass warns that it does not know the packed-fp32 feature; drop that line
    lines = [ln for ln in proc.stdout.splitlines() if "packed-fp32-ops" not in ln]
    if lines:
        sys.stdout.write("\n".join(lines) + "\n")
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}")


def build_library(jobs: int = 4) -> Path:
    BUILD_DIR.mkdir(exist_ok=True)
    objs = []
    cmds = []
    for src in HIP_SOURCES:
        obj = BUILD_DIR / (Path(src).stem + ".o")
        objs.append(obj)
        cmds.append([HIPCC, *HIP_FLAGS, *HIP_SOURCE_FLAGS.get(src, []), "-c", str(CSRC / src),
                     "-o", str(obj)])
    for src in CPP_SOURCES:
        obj = BUILD_DIR / (Path(src).stem + ".o")
        objs.append(obj)
        cmds.append(["g++", *CXX_FLAGS, "-c", str(CSRC / src), "-o", str(obj)])
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(_run, cmds))
    tmp = LIB.with_suffix(".so.tmp")
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)])
    os.replace(tmp, LIB)
    return LIB


def build_calib() -> Path:
    """The bench's measurement probes (calib/slm_calib.h) as libslm_calib.so."""
    BUILD_DIR.mkdir(exist_ok=True)
    obj = BUILD_DIR / "calib.o"
    _run([HIPCC, *HIP_FLAGS, f"-I{CALIB_DIR}", "-c", str(CALIB_DIR / "calib.hip"), "-o", str(obj)])
    tmp = CALIB_LIB.with_suffix(".so.tmp")
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", str(tmp), str(obj)])
    os.replace(tmp, CALIB_LIB)
    return CALIB_LIB


def build_host_demo() -> Path:
    """C++ host mirror of the reference interface, linked against the library."""
    _run([
        "g++", "-O2", "-std=c++17", "-Wall", "-Wextra", "-Werror",
        f"-I{REPO / 'include'}", f"-I{HOST}",
        str(HOST / "slm_host_demo.cpp"), "-o", str(HOST_DEMO),
        f"-L{PKG_DIR}", "-lslm_attn", f"-Wl,-rpath,$ORIGIN",
    ])
    return HOST_DEMO


def build_all() -> None:
    build_library()
    build_calib()
    build_host_demo()


if __name__ == "__main__":
    build_all()
    print(f"built {LIB}")
