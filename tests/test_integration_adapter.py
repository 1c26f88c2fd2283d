"""The kuiper-side adapter given in the integration guide at the repository root (the
kernel:: function bodies that forward to the C ABI) compiles and links: its C++ blocks are extracted, the kuiper
include lines are replaced by tests/cpp/kuiper_names.h (kuiper's type names bound to
the host mirror), and the result is built as a shared object with --no-undefined
against liborin_attn.so, so every orin_* call it makes resolves with the declared
signature.  CPU only: nothing is launched."""
import os
import re
import shutil
import subprocess

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(REPO, "orinmllm_amd")
LIB = os.path.join(PKG, "liborin_attn.so")


def adapter_source() -> str:
    text = open(os.path.join(REPO, "INTEGRATION.md")).read()
    blocks = re.findall(r"```cpp\n(.*?)```", text, flags=re.S)
    units = [b for b in blocks if "namespace kernel {" in b]
    assert len(units) == 2, "expected the attention adapter and its producer continuation"
    src = "\n".join(units)
    src = re.sub(r'#include "\.\./cuda/[^"]+"\n', "", src)
    return '#include "kuiper_names.h"\n' + src


def test_adapter_defines_the_kuiper_entry_points():
    src = adapter_source()
    for fn in ["mha_kernel_cu", "mha_kernel_cu_gpu_pos", "batched_mha_kernel_cu",
               "flash_attention_prefill_fp16_cu", "flash_attention_decode_fp16_cu",
               "flash_attention_decode_fp16_gpu_pos_cu", "vision_attention_pretransposed_cu",
               "batched_matmul_kernel_cu_pure_fp16", "copy_to_kv_cache_kernel_fp16",
               "copy_to_kv_cache_kernel", "sin_cos_cache_calc_cu",
               "fused_split_rope_transpose_cu"]:
        assert re.search(r"\bvoid " + fn + r"\(", src), fn


def test_adapter_compiles_and_links(tmp_path):
    if not os.path.exists(LIB):
        pytest.fail(f"{LIB} is missing: run __graft_entry__.build() first")
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    src = tmp_path / "attention_hip.cpp"
    src.write_text(adapter_source())
    out = tmp_path / "libkuiper_attention_adapter.so"
    cmd = [hipcc, "-std=c++17", "-O1", "-Wall", "-Werror", "-fPIC", "-shared",
           "-x", "c++", "-D__HIP_PLATFORM_AMD__",
           "-I", os.path.join(REPO, "tests", "cpp"), "-I", os.path.join(PKG, "cpp", "include"),
           "-I", os.path.join(REPO, "include"), "-I", "/opt/rocm/include", str(src), "-o", str(out),
           "-L", PKG, "-lorin_attn", "-Wl,--no-undefined",
           "-L", "/opt/rocm/lib", "-lamdhip64"]
    res = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
    assert res.returncode == 0, res.stderr[-4000:]
    nm = subprocess.run(["nm", "-DC", "--defined-only", str(out)], capture_output=True,
                        text=True).stdout
    assert "kernel::flash_attention_prefill_fp16_cu(" in nm
    assert "kernel::batched_matmul_kernel_cu_pure_fp16(" in nm
