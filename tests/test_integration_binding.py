"""The reference-side binding in INTEGRATION.md §1 (explicit specialisations
of the reference's GPU launcher templates, include/TensorOps.hpp:697-728,
calling include/mtgemm.h) compiles against the reference's own headers, so a
drift of either side's signatures shows here.  Build container only: it needs
the reference tree, which the GPU machines do not have."""
import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
REF_INCLUDE = Path("/root/reference/include")

pytestmark = pytest.mark.skipif(not (REF_INCLUDE / "TensorOps.hpp").exists(),
                                reason="needs the reference tree (build container only)")


def binding_source() -> str:
    text = (ROOT / "INTEGRATION.md").read_text()
    section = text[text.index("## 1."):text.index("## 2.")]
    blocks = re.findall(r"```cpp\n(.*?)```", section, re.S)
    assert blocks, "no C++ block in INTEGRATION.md section 1"
    return blocks[0]


def test_binding_compiles_against_reference_headers(tmp_path):
    cxx = shutil.which("g++")
    assert cxx, "g++ not found"
    src = tmp_path / "mtgemm_launchers.cpp"
    src.write_text(binding_source())
    names = ["matmul_gpu", "matmul_gpu_strided", "matmul_gpu_v2", "matmul_gpu_bk16",
             "conv2d_gpu", "conv2d_gpu_strided", "conv2d_backward_input_gpu",
             "conv2d_backward_weight_gpu", "conv2d_backward_bias_gpu", "fill_gpu", "sum_gpu",
             "copy_gpu_strided"]
    for n in names:   # every launcher of the path is specialised
        assert re.search(rf"template<>\s+[\w<>]+\s+{n}<float>\(", src.read_text()), n
    r = subprocess.run([cxx, "-std=c++20", "-fsyntax-only", "-DUSE_ROCM", "-D__HIP_PLATFORM_AMD__",
                        f"-I{REF_INCLUDE}", f"-I{ROOT / 'include'}", "-I/opt/rocm/include", "-w",
                        str(src)], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-4000:]
