"""Build the C++ parity test of the host mirror (tests/cpp/test_attention_layers) in
place.  It links liborin_attn_host.so / liborin_attn.so and, as the checker only, the
CPU oracle oracle/liboracle.so; both must be built first."""
from __future__ import annotations

import os
import shutil
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
PKG = os.path.join(REPO, "orinmllm_amd")
BINARY = os.path.join(HERE, "test_attention_layers")


def build(verbose: bool = False) -> str:
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    cmd = [hipcc, "-std=c++17", "-O2", "-Wall",
           "-I", os.path.join(PKG, "cpp", "include"), "-I", os.path.join(REPO, "include"),
           os.path.join(HERE, "test_attention_layers.cpp"), "-o", BINARY + ".tmp",
           "-L", PKG, "-lorin_attn_host", "-lorin_attn",
           "-L", os.path.join(REPO, "oracle"), "-loracle",
           f"-Wl,-rpath,{PKG}:{os.path.join(REPO, 'oracle')}",
           "-Wl,-rpath,$ORIGIN/../../orinmllm_amd:$ORIGIN/../../oracle"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"building the C++ layer test failed:\n{res.stderr}")
    os.replace(BINARY + ".tmp", BINARY)
    if verbose:
        print(f"built {BINARY}")
    return BINARY


if __name__ == "__main__":
    build(verbose=True)
