"""Build and run the gfx950 microbenchmarks behind the kernels' design rules.

    python orinmllm_amd/microbench/run.py [name ...]      (default: all of them)

Each program is a standalone HIP file in this directory; it is compiled with hipcc for
gfx950 (packed FP32 disabled, as the library is) into a temporary directory and run once,
with a time limit.  The programs print their own tables.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
PROGRAMS = ["hbm_stream", "coissue", "lds_read_rate", "lds_dma_issue", "lds_tr_layout",
            "prefill_timeline", "pingpong_coissue"]
FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
PKG = os.path.dirname(HERE)
# prefill_timeline compiles the library's fwd_pp.hip into itself with the timeline stamps on.
EXTRA = {"prefill_timeline": ["-I", os.path.join(PKG, "csrc"), "-I", os.path.join(os.path.dirname(PKG), "include"),
                              "-DORIN_PP_TIMELINE"]}


def main(argv: list[str]) -> int:
    names = argv or PROGRAMS
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    with tempfile.TemporaryDirectory() as tmp:
        for name in names:
            src = os.path.join(HERE, name + ".hip")
            exe = os.path.join(tmp, name)
            res = subprocess.run([hipcc, *FLAGS, *EXTRA.get(name, []), src, "-o", exe], capture_output=True, text=True)
            if res.returncode != 0:
                print(res.stderr, file=sys.stderr)
                return 1
            print(f"== {name}", flush=True)
            res = subprocess.run([exe], capture_output=True, text=True, timeout=120)
            print(res.stdout, end="", flush=True)
            if res.returncode != 0:
                print(res.stderr, file=sys.stderr)
                return res.returncode
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
