"""Build the gfx950 library in-tree.

    python -m llm_core_amd.build          # or __graft_entry__.build()

Outputs
  llm_core_amd/lib/libaxf_hip.so          HIP kernels + C-ABI + C++ backend/decoder
  llm_core_amd/_build/test_backend_hip    C++ backend test program (tests/cpp)
  llm_core_amd/_build/test_backend_dropin the same test against the reference's own
                                          backend API (where /root/reference exists)
  oracle/liboracle.so, oracle/_ref/...    CPU checker (via oracle/Makefile)

hipcc cross-compiles for gfx950 without a GPU.  Every HIP translation unit is
compiled with packed-FP32 instruction selection disabled.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "lib"
LIBNAME = "libaxf_hip.so"

ARCH = os.environ.get("AXF_OFFLOAD_ARCH", "gfx950")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

SOURCES = [
    "kernels/gemv.hip",
    "kernels/gemm_mfma.hip",
    "kernels/ops.hip",
    "kernels/attention.hip",
    "kernels/sample.hip",
    "kernels/gemv_misc.hip",
    "capi.cpp",
    "gemm_noalloc.cpp",
    "host/synth.cpp",
    "host/llama_hip.cpp",
    "host/gguf.cpp",
    "host/sampling.cpp",
    "host/hip_backend.cpp",
]

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++20",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{ROOT / 'include'}",
]


def _run(cmd: list[str], cwd: Path | None = None) -> None:
    proc = subprocess.run(cmd, cwd=cwd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(
        ln for ln in proc.stdout.splitlines() if "packed-fp32-ops" not in ln and ln.strip()
    )
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    if out:
        print(out, file=sys.stderr)


# per-source additions: the matrix-core GEMM keeps MFMA results in VGPRs
# (the default heuristic places them in AGPRs and copies every result out)
EXTRA_FLAGS = {
    "kernels/gemm_mfma.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
}


def _compile(src: str) -> Path:
    obj = BUILD / (src.replace("/", "_") + ".o")
    _run([HIPCC, "-x", "hip", *COMMON_FLAGS, *EXTRA_FLAGS.get(src, []), "-c", str(CSRC / src),
          "-o", str(obj)])
    return obj


def build_library(jobs: int = 8) -> Path:
    BUILD.mkdir(exist_ok=True)
    LIB.mkdir(exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=max(1, min(jobs, len(SOURCES)))) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB / (LIBNAME + ".tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp),
          *map(str, objs), "-Wl,-rpath,/opt/rocm/lib", "-lpthread"])
    os.replace(tmp, LIB / LIBNAME)
    return LIB / LIBNAME


def build_cpp_tests() -> Path:
    exe = BUILD / "test_backend_hip"
    _run([HIPCC, "-std=c++20", "-O2", f"-I{ROOT / 'include'}", f"-I{CSRC / 'host'}",
          str(ROOT / "tests" / "cpp" / "test_backend_hip.cpp"), "-o", str(exe),
          f"-L{LIB}", "-laxf_hip", f"-Wl,-rpath,{LIB}", "-Wl,-rpath,/opt/rocm/lib"])
    return exe


def build_dropin_test() -> Path | None:
    """The plugin built against the reference's own headers, registry and
    Tensor where the reference tree exists (tests/cpp/build_dropin.py)."""
    import importlib.util
    spec = importlib.util.spec_from_file_location(
        "axf_build_dropin", ROOT / "tests" / "cpp" / "build_dropin.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod.build()


def build_oracle() -> None:
    make = shutil.which("make")
    if make is None:
        raise RuntimeError("make not found")
    _run([make, "-C", str(ROOT / "oracle"), "-j8"])


def build_all(jobs: int = 8) -> Path:
    lib = build_library(jobs)
    build_cpp_tests()
    build_dropin_test()
    build_oracle()
    return lib


if __name__ == "__main__":
    print(build_all())
