"""Write the .tmc workload fixtures under tests/golden/ with the reference's
own exporters.

Runs in the build container only (it needs /root/reference and PyTorch on
the CPU): runs tools/export_decoder_llm.py (the decoder-only manifest and
its PyTorch prefill / per-step references, _make_workload and
_write_archive, export_decoder_llm.py:477-595) at its default small shape
with seed 11, once with --dtype fp16 and once with --dtype fp32, and
tools/export_kv_cache.py (MultiHeadAttentionKVCache prefill / decode
references, export_kv_cache.py:72-200).  The manifests and their float32
payloads are data written by the reference; tests/test_importer.py and
tests/test_importer_gpu.py read them with this build's importers.

The reference's own pipeline resolves --effective-dtype from its compiler
(run.sh:36-44); fp16 and fp32 storage are both supported here, so the
effective dtype is the requested one.

Usage: python tests/golden/make_tmc_golden.py
"""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
REFERENCE = os.environ.get("TMC_REFERENCE_ROOT", "/root/reference")

DECODER_RUNS = {  # fixture name -> requested (= effective) storage dtype
    "decoder_llm_fp16_seed11.tmc": "fp16",
    "decoder_llm_fp32_seed11.tmc": "fp32",
}
KV_CACHE = "kv_cache.tmc"


def run(args: list) -> None:
    print("+", " ".join(args), flush=True)
    subprocess.run(args, check=True, cwd=HERE)


def main() -> int:
    tools = os.path.join(REFERENCE, "tools")
    if not os.path.isdir(tools):
        print(f"{tools} is missing: the fixtures are written in the build container only",
              file=sys.stderr)
        return 1
    for name, dtype in DECODER_RUNS.items():
        run([sys.executable, os.path.join(tools, "export_decoder_llm.py"), "--output",
             os.path.join(HERE, name), "--dtype", dtype, "--effective-dtype", dtype, "--seed", "11"])
    run([sys.executable, os.path.join(tools, "export_kv_cache.py"), "--output",
         os.path.join(HERE, KV_CACHE)])
    return 0


if __name__ == "__main__":
    sys.exit(main())
