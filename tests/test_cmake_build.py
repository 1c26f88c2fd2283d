"""The CMake build of the library and its C++ host layer (orinmllm_amd/CMakeLists.txt)
produces both shared libraries and exports the same symbols as the in-tree build."""
import os
import shutil
import subprocess

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(REPO, "orinmllm_amd")


def _exported(lib):
    out = subprocess.run(["nm", "-D", "--defined-only", lib], capture_output=True, text=True,
                         check=True).stdout
    return {line.split()[-1] for line in out.splitlines() if " T " in line}


@pytest.mark.skipif(shutil.which("cmake") is None or not os.path.exists("/opt/rocm/bin/hipcc"),
                    reason="cmake or the ROCm toolchain is not installed")
def test_cmake_builds_both_libraries(tmp_path):
    build = tmp_path / "b"
    subprocess.run(["cmake", "-S", PKG, "-B", str(build), "-DCMAKE_PREFIX_PATH=/opt/rocm"],
                   check=True, capture_output=True, timeout=300)
    subprocess.run(["cmake", "--build", str(build), "-j8"], check=True, capture_output=True,
                   timeout=900)
    for name in ("liborin_attn.so", "liborin_attn_host.so"):
        built = build / name
        assert built.exists(), name
        ref = os.path.join(PKG, name)
        if os.path.exists(ref):
            assert _exported(str(built)) == _exported(ref), name
