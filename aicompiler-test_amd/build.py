"""Compile the gfx950 decode backend in-tree.

  libtmc_hip.so   every .hip source under csrc/, compiled by hipcc for gfx950
                  (the C ABI of include/tmc_hip.h);
  libtmc_host.so  the C++ host layer under host/ (HipRuntime, KV pools and
                  states, decoder executors, serving loop) over that ABI;
  _tmc_host*.so   its Python module (pybind11), for tests and bench.py.

  libtmc_hip_merge_launch.so  the same ABI built with TMC_ATTN_MERGE_LAUNCH=1
                  (every split-attention merge in a launch of its own, no
                  cross-block arrival counters), for the tests of that switch.
  libtmc_hip_timeline.so  the same ABI built with TMC_ATTN_TIMELINE=1 (per-wave
                  timestamps of the paged split-attention kernel, read by
                  tmc_attention_timeline; profiling.py timeline).

Objects go under _build/ (git-ignored); the libraries land next to this file
so they travel with the source tree to the GPU box.

Usage: python aicompiler-test_amd/build.py
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
OUT = os.path.join(HERE, "libtmc_hip.so")
HOST = os.path.join(HERE, "host")
HOST_OUT = os.path.join(HERE, "libtmc_host.so")
HOST_SOURCES = ["TensorIR.cpp", "HipRuntime.cpp", "KVCacheState.cpp", "DecoderLLM.cpp", "Benchmark.cpp",
                "ServingRuntime.cpp", "Tuning.cpp", "Importer.cpp", "KernelRegistry.cpp",
                "StatefulExecutor.cpp", "GraphExecutor.cpp"]
INCLUDE = os.path.join(os.path.dirname(HERE), "include")
CXX = os.environ.get("CXX", "g++")
CXXFLAGS = ["-std=c++17", "-O2", "-fPIC", "-Wall", "-Wextra", "-Wno-unused-parameter",
            f"-I{INCLUDE}", f"-I{HOST}"]

SOURCES = ["runtime.hip", "gemv.hip", "packed.hip", "elementwise.hip", "attention.hip",
           "prefill.hip", "gemm.hip"]
# The HIP runtime library of the ROCm install (rpath of the built library).
ROCM_LIB = os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "lib")

MERGE_LAUNCH_OUT = os.path.join(HERE, "libtmc_hip_merge_launch.so")
TIMELINE_OUT = os.path.join(HERE, "libtmc_hip_timeline.so")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-mcode-object-version=5",
    # Packed fp32 VALU ops are kept out of the generated code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]


# Per-source additions.  prefill.hip: keep MFMA accumulators in VGPRs (the
# online-softmax rescale multiplies them every block; from AGPRs each one is
# a read, a multiply and a write back).
SOURCE_FLAGS = {"prefill.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def _compile(src: str, variant: str = "", defines: tuple = ()) -> str:
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + variant + ".o")
    cmd = [HIPCC, *FLAGS, *SOURCE_FLAGS.get(src, []), *defines, "-c", os.path.join(CSRC, src),
           "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{res.stdout}\n{res.stderr}")
    noisy = [l for l in (res.stderr or "").splitlines()
             if l.strip() and "packed-fp32-ops" not in l]
    if noisy:
        sys.stderr.write(f"[{src}]\n" + "\n".join(noisy) + "\n")
    return obj


def _run(cmd, what):
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"{what} failed:\n{' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    if res.stderr.strip():
        sys.stderr.write(f"[{what}]\n{res.stderr}")


def _compile_host(src: str) -> str:
    obj = os.path.join(BUILD, "host_" + os.path.splitext(src)[0] + ".o")
    _run([CXX, *CXXFLAGS, "-c", os.path.join(HOST, src), "-o", obj], f"g++ {src}")
    return obj


def _module_path() -> str:
    import sysconfig
    return os.path.join(HERE, "_tmc_host" + sysconfig.get_config_var("EXT_SUFFIX"))


def _build_module() -> str:
    import sysconfig
    import pybind11
    obj = os.path.join(BUILD, "host_bindings.o")
    _run([CXX, *CXXFLAGS, f"-I{pybind11.get_include()}", f"-I{sysconfig.get_paths()['include']}",
          "-fvisibility=hidden", "-c", os.path.join(HOST, "bindings.cpp"), "-o", obj],
         "g++ bindings.cpp")
    out = _module_path()
    _run([CXX, "-shared", "-o", out + ".tmp", obj, f"-L{HERE}", "-ltmc_host", "-ltmc_hip",
          "-Wl,-rpath,$ORIGIN"], "link _tmc_host")
    shutil.move(out + ".tmp", out)
    return out


def _link_hip(objs: list, out: str) -> None:
    tmp = out + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs, f"-L{ROCM_LIB}",
           f"-Wl,-rpath,{ROCM_LIB}"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    shutil.move(tmp, out)


def build(jobs: int = 4) -> str:
    os.makedirs(BUILD, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=jobs) as pool:
        merge_launch = pool.submit(_compile, "attention.hip", "_merge_launch",
                                   ("-DTMC_ATTN_MERGE_LAUNCH=1",))
        timeline = pool.submit(_compile, "attention.hip", "_timeline", ("-DTMC_ATTN_TIMELINE=1",))
        objs = list(pool.map(_compile, SOURCES))
        host_objs = list(pool.map(_compile_host, HOST_SOURCES))
        merge_launch_obj = merge_launch.result()
        timeline_obj = timeline.result()
    _link_hip(objs, OUT)
    attention = os.path.join(BUILD, "attention.o")
    _link_hip([merge_launch_obj if o == attention else o for o in objs], MERGE_LAUNCH_OUT)
    _link_hip([timeline_obj if o == attention else o for o in objs], TIMELINE_OUT)
    _run([CXX, "-shared", "-o", HOST_OUT + ".tmp", *host_objs, f"-L{HERE}", "-ltmc_hip",
          "-Wl,-rpath,$ORIGIN"], "link libtmc_host.so")
    shutil.move(HOST_OUT + ".tmp", HOST_OUT)
    _build_module()
    return OUT


if __name__ == "__main__":
    print(build())
