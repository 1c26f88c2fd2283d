"""The C++ host mirror (orin::kernel functions and orin::op layers with kuiper's
signatures, over liborin_attn.so) checked by its own C++ test binary,
tests/cpp/test_attention_layers, against the CPU oracle: the host-only cases here,
the device cases on the GPU."""
import os
import subprocess

import pytest

BINARY = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cpp", "test_attention_layers")


def run(args, timeout):
    if not os.path.exists(BINARY):
        pytest.fail(f"{BINARY} is missing: run __graft_entry__.build() first")
    res = subprocess.run([BINARY, *args], capture_output=True, text=True, timeout=timeout)
    print(res.stdout)
    assert res.returncode == 0, res.stdout[-4000:] + res.stderr[-2000:]
    assert "0 failed" in res.stdout
    return res.stdout


def test_host_mirror_argument_handling():
    out = run(["--cpu-only"], 60)
    assert "4 tests ran" in out


@pytest.mark.gpu
def test_host_mirror_layers_match_oracle():
    out = run([], 110)
    assert "[  FAILED  ]" not in out
    for case in ["GpuFlashAttentionPrefillLayer.Fp16CausalFromLayerInputs",
                 "GpuFlashAttentionPrefillLayer.Bf16CausalWithPrefixDirectForward",
                 "GpuFlashAttentionDecodeLayer.Fp16HostAndDevicePosition",
                 "GpuMultiHeadAttention.Fp32C1ThroughGetMhaKernel",
                 "GpuVisionLayers.SplitRopeTransposeThenAttentionBf16",
                 "GpuCopyToKVCacheLayer.Fp16RowLandsAtDevicePosition",
                 "GpuKernels.Fp16WoProjectionMatchesFp32Reference"]:
        assert f"[       OK ] {case}" in out, case
