"""Build the plugin backend as a drop-in for the reference engine's own backend
API, from the reference tree where it lies (/root/reference), into
llm_core_amd/_build/test_backend_dropin.

    python tests/cpp/build_dropin.py        # or llm_core_amd.build.build_all()

What the reference's maintainer would do, in a scratch directory outside this
repository (deleted afterwards):
  1. copy the reference's include/ tree;
  2. write axonforge/version.hpp from its own version.hpp.in, substituting the
     @PROJECT_VERSION*@ placeholders with the version of the project() line of
     its CMakeLists.txt, as its configure_file(... @ONLY) step does
     (CMakeLists.txt:36-40); the generated text is the configured file, not a
     stand-in;
  3. apply the one documented edit: DeviceType::HIP = 5 and its name in
     device_type_name (include/axonforge/common.hpp);
then compile llm_core_amd/csrc/host/hip_backend.cpp with -DAXF_AXONFORGE_HEADERS
(the plugin's include switch takes the reference's headers), the reference's
own BackendRegistry (src/backend/backend_registry.cpp), Tensor
(src/core/tensor.cpp) and AttributeMap (src/core/graph.cpp) from source, and
tests/cpp/test_backend_hip.cpp in the same mode, and link them with
libaxf_hip.so.  Nothing of the reference is copied into this repository: the
objects and the program are build outputs (git-ignored), like oracle/_ref.

Returns the program's path, or None where the reference tree is absent (the
GPU box: there the program built here, if any, is run by the GPU test).
"""
from __future__ import annotations

import os
import re
import shutil
import subprocess
import sys
import tempfile
from pathlib import Path

ROOT = Path(__file__).resolve().parents[2]
REF = Path(os.environ.get("AXF_REFERENCE_ROOT", "/root/reference"))
HOST = ROOT / "llm_core_amd" / "csrc" / "host"
LIB = ROOT / "llm_core_amd" / "lib"
OUT = ROOT / "llm_core_amd" / "_build" / "test_backend_dropin"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
REF_SOURCES = ["src/backend/backend_registry.cpp", "src/core/tensor.cpp", "src/core/graph.cpp"]


def configured_version_header(ref: Path) -> str:
    """version.hpp as configure_file(@ONLY) writes it from version.hpp.in."""
    cm = (ref / "CMakeLists.txt").read_text()
    m = re.search(r"project\(\s*\w+\s+VERSION\s+(\d+)\.(\d+)\.(\d+)", cm)
    if not m:
        raise RuntimeError("project(... VERSION x.y.z) not found in the reference CMakeLists.txt")
    major, minor, patch = m.groups()
    text = (ref / "include" / "axonforge" / "version.hpp.in").read_text()
    for key, val in (("PROJECT_VERSION_MAJOR", major), ("PROJECT_VERSION_MINOR", minor),
                     ("PROJECT_VERSION_PATCH", patch),
                     ("PROJECT_VERSION", f"{major}.{minor}.{patch}")):
        text = text.replace(f"@{key}@", val)
    if "@" in text:
        raise RuntimeError("unsubstituted placeholder in version.hpp.in")
    return text


def add_hip_device_type(common: str) -> str:
    """The one edit of the reference: DeviceType::HIP = 5 and its name."""
    enum_end = re.search(r"(enum\s+class\s+DeviceType[^{]*\{[^}]*?)(\n\};)", common, re.S)
    if not enum_end or "HIP" in enum_end.group(1):
        raise RuntimeError("DeviceType enum not found or already has HIP")
    common = common[:enum_end.end(1)] + "\n    HIP    = 5," + common[enum_end.end(1):]
    case = re.search(r"(\n(\s*)case DeviceType::NPU:[^\n]*)", common)
    if not case:
        raise RuntimeError("device_type_name has no NPU case")
    return (common[:case.end(1)] + f'\n{case.group(2)}case DeviceType::HIP:    return "hip";'
            + common[case.end(1):])


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if proc.returncode != 0:
        out = "\n".join(ln for ln in proc.stdout.splitlines() if "packed-fp32-ops" not in ln)
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")


def build(ref: Path = REF, out: Path = OUT) -> Path | None:
    if not (ref / "include" / "axonforge" / "backend.hpp").is_file():
        return None
    if not (LIB / "libaxf_hip.so").is_file():
        raise RuntimeError("build libaxf_hip.so first")
    out.parent.mkdir(parents=True, exist_ok=True)
    with tempfile.TemporaryDirectory(prefix="axf_dropin_") as tmp:
        tmp = Path(tmp)
        inc = tmp / "include"
        shutil.copytree(ref / "include", inc)
        (inc / "axonforge" / "version.hpp").write_text(configured_version_header(ref))
        common = inc / "axonforge" / "common.hpp"
        common.write_text(add_hip_device_type(common.read_text()))
        objs = []
        # the plugin, as the library compiles it (HIP language, host side: no kernels)
        hb = tmp / "hip_backend.o"
        _run([HIPCC, "-x", "hip", "--offload-arch=gfx950", "--cuda-host-only", "-std=c++20", "-O2",
              "-fPIC", "-DAXF_AXONFORGE_HEADERS", f"-I{inc}", f"-I{ROOT / 'include'}", "-c",
              str(HOST / "hip_backend.cpp"), "-o", str(hb)])
        objs.append(hb)
        for src in REF_SOURCES:
            o = tmp / (Path(src).stem + ".o")
            _run(["g++", "-std=c++20", "-O2", "-fPIC", f"-I{inc}", "-c", str(ref / src), "-o", str(o)])
            objs.append(o)
        t = tmp / "test.o"
        _run(["g++", "-std=c++20", "-O2", "-DAXF_AXONFORGE_HEADERS", f"-I{inc}",
              f"-I{ROOT / 'include'}", "-c", str(ROOT / "tests" / "cpp" / "test_backend_hip.cpp"),
              "-o", str(t)])
        objs.append(t)
        _run(["g++", *map(str, objs), "-o", str(out), f"-L{LIB}", "-laxf_hip",
              f"-Wl,-rpath,{LIB}", "-Wl,-rpath,/opt/rocm/lib"])
    return out


if __name__ == "__main__":
    print(build() or "reference tree absent: nothing built", file=sys.stderr)
