"""Build the gfx950 GEMM library (minitensor_amd/lib/libmtgemm.so) with hipcc.

Every tile configuration is its own translation unit so the template
instantiations compile in parallel.  The library is built in-tree so it
travels with the source tree to the GPU machine; nothing is JIT-compiled.

    python -m minitensor_amd.build          # or: python minitensor_amd/build.py
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
LIBDIR = PKG / "lib"
OBJDIR = PKG / "_build"
LIB = LIBDIR / "libmtgemm.so"

ARCH = "gfx950"
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
HIPCC = os.environ.get("HIPCC", str(ROCM / "bin" / "hipcc"))

# -packed-fp32-ops: keep the compiler from emitting v_pk_{add,mul,fma}_f32.
COMMON = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++20", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{ROOT / 'include'}", f"-I{CSRC}",
    "-Wno-unused-command-line-argument",
]

N_CFG = 3      # register-staged tile configurations (TileCfg)
N_DL_CFG = 4   # gemm_f32_dl tile configurations (DlCfg 0..3; DlCfg 4 is gemm_f32_dlp)


def _units():
    units = []
    for cfg in range(N_CFG):
        units.append((CSRC / "gemm_instances.hip", OBJDIR / f"gemm_cfg{cfg}.o", [f"-DMT_CFG={cfg}"]))
    for cfg in range(N_DL_CFG):
        units.append((CSRC / "gemm_dl_instances.hip", OBJDIR / f"gemm_dl_cfg{cfg}.o",
                      [f"-DMT_CFG={cfg}"]))
    units.append((CSRC / "gemm_dlp_instances.hip", OBJDIR / "gemm_dlp.o", []))
    units.append((CSRC / "gemm_dl16_instances.hip", OBJDIR / "gemm_dl16.o", []))
    units.append((CSRC / "gemm_ksw_instances.hip", OBJDIR / "gemm_ksw.o", []))
    units.append((CSRC / "gemm_skinny_instances.hip", OBJDIR / "gemm_skinny.o", []))
    units.append((CSRC / "mtgemm_api.hip", OBJDIR / "mtgemm_api.o", []))
    return units


def _scratch_kernels(out: str) -> list:
    """(kernel, bytes per lane) of every kernel whose resource remark reports
    scratch: registers spilled to private memory (or a register array indexed
    at run time), each access a memory round trip."""
    found, name = [], None
    for line in out.splitlines():
        if "Function Name:" in line:
            name = line.split("Function Name:", 1)[1].split("[-R")[0].strip()
        elif "ScratchSize [bytes/lane]:" in line and name:
            n = int(line.split("ScratchSize [bytes/lane]:", 1)[1].split()[0])
            if n > 0:
                found.append((name, n))
    return found


def build(verbose: bool = False) -> Path:
    """Compile every unit and link libmtgemm.so; raises on any compiler error,
    and on any kernel that uses scratch memory (the compiler's resource-usage
    remarks): a spill silently costs several times the kernel's time (the
    16-deep rank-k kernel: 128 us against 22 for its neighbour at K = 17)."""
    if not shutil.which(HIPCC) and not Path(HIPCC).exists():
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    OBJDIR.mkdir(parents=True, exist_ok=True)
    LIBDIR.mkdir(parents=True, exist_ok=True)
    procs = []
    for src, obj, extra in _units():
        cmd = [HIPCC, *COMMON, *extra, "-Rpass-analysis=kernel-resource-usage", "-c", str(src),
               "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((cmd, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT,
                                            text=True)))
    failed, spills = [], []
    for cmd, p in procs:
        out, _ = p.communicate()
        lines = [l for l in out.splitlines()
                 if "packed-fp32-ops" not in l and "kernel-resource-usage" not in l]
        spills += _scratch_kernels(out)
        if p.returncode != 0:
            failed.append((cmd, "\n".join(lines)))
        elif verbose and lines:
            print("\n".join(lines))
    if failed:
        msg = "\n\n".join(f"$ {' '.join(c)}\n{o}" for c, o in failed)
        raise RuntimeError(f"hipcc failed:\n{msg}")
    if spills:
        msg = "\n".join(f"  {k}: {n} bytes/lane" for k, n in sorted(set(spills)))
        raise RuntimeError(f"kernels using scratch memory (spilled registers):\n{msg}")
    tmp = LIB.with_suffix(".so.tmp")
    link = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp),
            *[str(o) for _, o, _ in _units()]]
    if verbose:
        print(" ".join(link), flush=True)
    r = subprocess.run(link, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}")
    os.replace(tmp, LIB)
    return LIB


HOST_TESTS = LIBDIR / "mt_host_tests"


def build_host_tests(verbose: bool = False) -> Path:
    """Compile the C++ host-layer test program against libmtgemm.so (rpath $ORIGIN)."""
    src = PKG / "cpp" / "tests" / "host_tests.cpp"
    # Host-only C++ (no device code): g++ against the HIP runtime headers.
    cmd = [os.environ.get("CXX", "g++"), "-std=c++20", "-O2", "-Wall", "-D__HIP_PLATFORM_AMD__",
           f"-I{ROCM / 'include'}", f"-I{ROOT / 'include'}", f"-I{PKG / 'cpp'}", str(src),
           "-o", str(HOST_TESTS), f"-L{LIBDIR}", "-lmtgemm", f"-L{ROCM / 'lib'}", "-lamdhip64",
           "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{ROCM / 'lib'}"]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"host test build failed:\n{r.stdout}")
    return HOST_TESTS


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
    print(build_host_tests(verbose="-v" in sys.argv))
