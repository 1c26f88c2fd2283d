"""Host logic of the prefill's causal key split, on the CPU: tests/cpp/key_split_check.hip
compiles orinmllm_amd/csrc/fwd_pp.hip into a checker that runs the host-side chooser
(fwd_pp_key_split) and the chunk arithmetic the kernel and the merge share (pp_block_chunks,
pp_chunk_lo, pp_item) over 11,520 shapes and checks their invariants: the launch fits the
device, the bound is the smallest that does, every chunk is non-empty and starts at or before
its block's first diagonal tile, the cuts cover each block, the items run blocks last to first,
and the workspace size matches the partial rows.  No GPU is used."""
import os
import subprocess

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HIPCC = "/opt/rocm/bin/hipcc"


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="the ROCm toolchain is not installed")
def test_key_split_chunks_host(tmp_path):
    exe = tmp_path / "key_split_check"
    cmd = [HIPCC, "--offload-arch=gfx950", "-std=c++17", "-O1",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
           "-I", os.path.join(REPO, "include"), "-I", os.path.join(REPO, "orinmllm_amd", "csrc"),
           os.path.join(REPO, "tests", "cpp", "key_split_check.hip"), "-o", str(exe)]
    subprocess.run(cmd, check=True, capture_output=True, timeout=600)
    res = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert res.returncode == 0, res.stdout + res.stderr
    assert "failures 0" in res.stdout, res.stdout
    cases, splits = (int(x) for x in
                     res.stdout.split("cases ")[1].split(", failures")[0].split(", key splits "))
    assert cases == 11520 and splits > 5000, res.stdout
