"""Build the MI355X fused-MoE libraries in-tree.

Outputs (next to the Python package so they travel with the tree):
  vllm_xpu_kernels/libmi355moe.so       HIP kernels + C ABI (hipcc, gfx950)
  vllm_xpu_kernels/_mi355moe_torch.so   PyTorch-ROCm op registration (g++)

Usage: python vllm-xpu-kernels_amd/build.py [--jobs N]
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shlex
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
PKG = os.path.join(HERE, "vllm_xpu_kernels")
BUILD = os.path.join(HERE, "_build")
INCLUDE = os.path.join(os.path.dirname(HERE), "include")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")

HIP_SOURCES = ["routing.hip", "align.hip", "elementwise.hip", "moe_gemm.hip",
               "moe_gemm_big.hip", "moe_gemm_pipe.hip", "moe_gemm_stream.hip",
               "moe_gemm_wide.hip", "moe_gemm_wide8.hip", "moe_gemm_wide8p.hip", "moe_gemm_wide4.hip", "moe_gemm_big8.hip", "fused_moe.hip", "prologue.hip", "errors.cpp"]
HIPCC_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
    # no packed fp32 (v_pk_*_f32) code generation
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I" + INCLUDE,
]


def _run(cmd: list[str]) -> None:
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT,
                       text=True)
    out = "\n".join(l for l in r.stdout.splitlines()
                    if "packed-fp32-ops" not in l and "is not a recognized feature" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(map(shlex.quote, cmd))}\n{out}")


def build_hip(jobs: int) -> str:
    os.makedirs(BUILD, exist_ok=True)
    hipcc = os.path.join(ROCM, "bin", "hipcc")
    objs = []
    cmds = []
    for src in HIP_SOURCES:
        obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
        objs.append(obj)
        cmds.append([hipcc, *HIPCC_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj])
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(_run, cmds))
    out = os.path.join(PKG, "libmi355moe.so")
    tmp = out + ".tmp"
    _run([hipcc, "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", tmp,
          "-Wl,-soname,libmi355moe.so"])
    os.replace(tmp, out)
    return out


def build_torch_ext() -> str:
    import torch
    from torch.utils import cpp_extension as ce
    tdir = os.path.dirname(torch.__file__)
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    inc = [f"-I{p}" for p in ce.include_paths()] + [f"-I{ROCM}/include", f"-I{INCLUDE}"]
    out = os.path.join(PKG, "_mi355moe_torch.so")
    tmp = out + ".tmp"
    cmd = ["g++", "-O2", "-std=c++17", "-fPIC", "-shared",
           f"-D_GLIBCXX_USE_CXX11_ABI={abi}", "-D__HIP_PLATFORM_AMD__=1",
           "-DUSE_ROCM=1", "-w", *inc,
           os.path.join(CSRC, "torch_bindings.cpp"),
           "-o", tmp,
           f"-L{os.path.join(tdir, 'lib')}", "-lc10", "-ltorch", "-ltorch_cpu",
           "-lc10_hip", "-ltorch_hip",
           f"-L{PKG}", "-lmi355moe",
           "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{os.path.join(tdir, 'lib')}"]
    _run(cmd)
    os.replace(tmp, out)
    return out


def build(jobs: int | None = None) -> None:
    jobs = jobs or min(8, os.cpu_count() or 4)
    with cf.ThreadPoolExecutor(max_workers=2) as ex:
        f_hip = ex.submit(build_hip, jobs)
        f_hip.result()
        # the torch extension links against libmi355moe.so
        build_torch_ext()


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    args = ap.parse_args()
    build(args.jobs)
    print("built", os.path.join(PKG, "libmi355moe.so"), "and",
          os.path.join(PKG, "_mi355moe_torch.so"))
    sys.exit(0)
