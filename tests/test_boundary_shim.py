"""The drop-in boundary at the source level: with the shim
aicompiler-test_amd/host/shim/backend/metal/MetalRuntime.hpp ahead of the
reference's src/ on the include path, every reference source that uses
tensor::metal (its executors, tuners, admission, benchmark and apps)
compiles unchanged against the gfx950 runtime's headers.  Runs only where
the reference tree and g++ are present (the build container); it reads the
reference's sources as compiler input and copies nothing from them."""
import concurrent.futures as cf
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF = "/root/reference"
SHIM = os.path.join(ROOT, "aicompiler-test_amd", "host", "shim")

pytestmark = pytest.mark.skipif(not os.path.isdir(os.path.join(REF, "src")) or
                                shutil.which("g++") is None,
                                reason="needs the reference sources and g++")


def _callers():
    found = []
    for top in ("src", "apps"):
        for dirpath, _, files in os.walk(os.path.join(REF, top)):
            for name in files:
                if not name.endswith(".cpp"):
                    continue
                path = os.path.join(dirpath, name)
                with open(path, errors="replace") as f:
                    if re.search(r"MetalRuntime\.hpp|metal::", f.read()):
                        found.append(path)
    return sorted(found)


def _syntax(path):
    cmd = ["g++", "-std=c++17", "-fsyntax-only", f"-I{SHIM}", f"-I{REF}/src", f"-I{REF}",
           f"-I{ROOT}/aicompiler-test_amd/host", f"-I{ROOT}/include", path]
    res = subprocess.run(cmd, capture_output=True, text=True)
    return path, res.returncode, res.stderr


def test_reference_callers_compile_against_the_shim():
    callers = _callers()
    # the executors, tuners and admission the boundary must serve
    for required in ("runtime/DecoderLLMExecutor.cpp", "runtime/ServingRuntime.cpp",
                     "runtime/StatefulExecutor.cpp", "runtime/GraphExecutor.cpp",
                     "runtime/KVCacheState.cpp", "planner/RMSNormTuner.cpp",
                     "planner/DecodeGEMVTuner.cpp", "runtime/GeneratedKernelAdmission.cpp",
                     "benchmark/Benchmark.cpp"):
        assert any(c.endswith(required) for c in callers), required
    with cf.ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 1)) as pool:
        results = list(pool.map(_syntax, callers))
    failed = [(p, err[:2000]) for p, rc, err in results if rc != 0]
    assert not failed, "\n\n".join(f"{p}:\n{e}" for p, e in failed)
