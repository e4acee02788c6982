"""The plugin backend as a drop-in for the reference's backend API.

llm_core_amd/csrc/host/hip_backend.cpp takes its interface from one include
switch: axf_backend.hpp (namespace axf) in this tree, or, built with
AXF_AXONFORGE_HEADERS inside the reference tree, the reference's own
include/axonforge/backend.hpp (namespace axonforge, through the alias
axf_api).  Checked here (the reference parts skipped where /root/reference is
absent):

  * the real build: tests/cpp/build_dropin.py compiles the plugin in its
    drop-in mode against a copy of the reference's include tree (version.hpp
    configured from its own template, the one DeviceType::HIP edit applied),
    links it with the reference's own BackendRegistry, Tensor and AttributeMap
    compiled from source and the C++ backend test, and the program runs: the
    backend is registered under "hip", unknown ids throw std::runtime_error,
    and on a host without a GPU initialize() reports no device and device
    work throws std::runtime_error (the GPU test runs the same program's
    device checks through IKernel::execute);
  * the configured version.hpp equals what CMake's configure_file(@ONLY)
    writes from the same template and version (cmake -P);
  * against the reference's header text: every enumerator the plugin uses has
    the reference's value (DType, dtype.hpp; OpType, graph.hpp), DeviceType
    differs by exactly the one added enumerator HIP = 5 (common.hpp), IKernel
    / IBackend declare the same pure-virtual signatures (backend.hpp:18-69),
    and every Tensor member and factory the plugin calls is declared in
    tensor.hpp;
  * the drop-in mode defines none of the core types the reference supplies
    (Tensor, CpuTensorStorage, BackendRegistry).
"""
import os
import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
HOST = ROOT / "llm_core_amd" / "csrc" / "host"
REF = Path("/root/reference/include/axonforge")
OURS = (HOST / "axf_backend.hpp").read_text()
PLUGIN = (HOST / "hip_backend.cpp").read_text()

need_ref = pytest.mark.skipif(not REF.is_dir(), reason="reference headers not present")


def strip_comments(src: str) -> str:
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return re.sub(r"//[^\n]*", "", src)


def enum_values(src: str, name: str) -> dict[str, int]:
    """Enumerator -> value of `enum class name`, implicit values counted as C++ does."""
    m = re.search(r"enum\s+class\s+" + name + r"\s*(?::\s*\w+)?\s*\{(.*?)\};", strip_comments(src), re.S)
    assert m, f"enum class {name} not found"
    out, nxt = {}, 0
    for item in m.group(1).split(","):
        item = item.strip()
        if not item:
            continue
        if "=" in item:
            k, v = (t.strip() for t in item.split("=", 1))
            nxt = int(v, 0)
        else:
            k = item
        out[k] = nxt
        nxt += 1
    return out


def pure_virtuals(src: str, cls: str) -> set[str]:
    """Normalised pure-virtual declarations of `class cls`."""
    body = strip_comments(src)
    m = re.search(r"class\s+" + cls + r"\s*\{(.*?)\n\};", body, re.S)
    assert m, f"class {cls} not found"
    decls = set()
    for d in re.findall(r"virtual([^;]*?)=\s*0\s*;", m.group(1), re.S):
        d = d.replace("[[nodiscard]]", "")
        d = re.sub(r"\s+", " ", d).strip()
        d = re.sub(r"\s*([(),&*<>])\s*", r"\1", d)
        decls.add(d)
    return decls


def used(pattern: str) -> set[str]:
    return set(re.findall(pattern, PLUGIN))


@need_ref
def test_dtype_and_optype_values_match_the_reference():
    ref_dt = enum_values((REF / "dtype.hpp").read_text(), "DType")
    for name, v in enum_values(OURS, "DType").items():
        assert ref_dt.get(name) == v, f"DType::{name}: ours {v}, reference {ref_dt.get(name)}"
    ref_op = enum_values((REF / "graph.hpp").read_text(), "OpType")
    ours_op = enum_values(OURS, "OpType")
    for name in used(r"OpType::([A-Z_]+)"):
        assert ref_op[name] == ours_op[name], f"OpType::{name}"
    for name in used(r"DType::([A-Z0-9_]+)"):
        assert name in ref_dt, f"DType::{name} is not a reference enumerator"


@need_ref
def test_device_type_differs_by_the_one_hip_enumerator():
    ref = enum_values((REF / "common.hpp").read_text(), "DeviceType")
    ours = enum_values(OURS, "DeviceType")
    assert "HIP" not in ref
    assert ours == {**ref, "HIP": max(ref.values()) + 1}
    # the plugin builds its DeviceIds from DeviceType::HIP alone (no DeviceId::hip())
    assert "DeviceId::hip" not in strip_comments(PLUGIN)
    assert "DeviceId{DeviceType::HIP" in PLUGIN


@need_ref
def test_kernel_and_backend_virtuals_match_the_reference():
    ref = (REF / "backend.hpp").read_text()
    for cls in ("IKernel", "IBackend"):
        assert pure_virtuals(OURS, cls) == pure_virtuals(ref, cls), cls


@need_ref
def test_tensor_members_used_by_the_plugin_exist_in_the_reference():
    tensor = strip_comments((REF / "tensor.hpp").read_text())
    memory = strip_comments((REF / "memory.hpp").read_text())
    members = used(r"\.(raw_data|numel|nbytes|shape|dtype|device)\(") | {"data", "byte_size"}
    for m in members:
        assert re.search(r"\b" + m + r"\s*\(", tensor + memory), m
    for f in used(r"Tensor::(zeros|from_blob|from_storage)\("):
        assert re.search(r"static\s+Tensor\s+" + f + r"\s*\(", tensor), f


def test_dropin_mode_compiles_without_the_core_type_definitions(tmp_path):
    hipcc = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
    if not Path(hipcc).exists() or shutil.which("nm") is None:
        pytest.skip("hipcc / nm not available")
    inc = tmp_path / "axonforge"
    inc.mkdir()
    (inc / "backend.hpp").write_text(
        f'#pragma once\n#include "{HOST / "axf_backend.hpp"}"\nnamespace axonforge = axf;\n')
    obj = tmp_path / "dropin.o"
    # as the library build compiles it (HIP language), host side only: the file has no kernels
    cmd = [hipcc, "-x", "hip", "--offload-arch=gfx950", "--cuda-host-only", "-std=c++20", "-O0",
           "-fPIC", "-DAXF_AXONFORGE_HEADERS", f"-I{tmp_path}", f"-I{ROOT / 'include'}", "-c",
           str(HOST / "hip_backend.cpp"), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
    assert proc.returncode == 0, proc.stderr[-3000:]
    syms = subprocess.run(["nm", "-C", "--defined-only", str(obj)], capture_output=True,
                          text=True).stdout
    for core in ("BackendRegistry::instance", "Tensor::zeros", "CpuTensorStorage::CpuTensorStorage",
                 "tensor_nbytes"):
        assert core not in syms, f"drop-in mode still defines {core}"
    assert "HipBackend" in syms


def _build_dropin_module():
    import importlib.util
    spec = importlib.util.spec_from_file_location("axf_build_dropin",
                                                  ROOT / "tests" / "cpp" / "build_dropin.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


@need_ref
def test_plugin_builds_and_registers_against_the_reference_backend_api(tmp_path):
    if shutil.which("g++") is None or not Path(os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")).exists():
        pytest.skip("g++ / hipcc not available")
    if not (ROOT / "llm_core_amd" / "lib" / "libaxf_hip.so").exists():
        pytest.skip("libaxf_hip.so not built")
    exe = _build_dropin_module().build(out=tmp_path / "test_backend_dropin")
    assert exe is not None and exe.exists()
    if Path("/dev/kfd").exists():
        pytest.skip("a GPU is visible: the device checks run in the gpu test")
    proc = subprocess.run([str(exe), "--no-device"], capture_output=True, text=True, timeout=60)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    assert "no device: done" in proc.stdout and "PASSED (0 failures)" in proc.stdout


@need_ref
def test_configured_version_header_equals_cmake_configure_file(tmp_path):
    cmake = shutil.which("cmake")
    if cmake is None:
        pytest.skip("cmake not available")
    mod = _build_dropin_module()
    ref = Path("/root/reference")
    m = re.search(r"project\(\s*\w+\s+VERSION\s+([\d.]+)", (ref / "CMakeLists.txt").read_text())
    major, minor, patch = m.group(1).split(".")
    script = tmp_path / "configure.cmake"
    out = tmp_path / "version.hpp"
    script.write_text(
        f'set(PROJECT_VERSION "{m.group(1)}")\nset(PROJECT_VERSION_MAJOR {major})\n'
        f"set(PROJECT_VERSION_MINOR {minor})\nset(PROJECT_VERSION_PATCH {patch})\n"
        f'configure_file("{ref / "include" / "axonforge" / "version.hpp.in"}" "{out}" @ONLY)\n')
    subprocess.run([cmake, "-P", str(script)], check=True, capture_output=True, timeout=60)
    assert mod.configured_version_header(ref) == out.read_text()


@need_ref
def test_hip_device_type_edit_is_the_one_documented_line():
    mod = _build_dropin_module()
    ref = (REF / "common.hpp").read_text()
    edited = mod.add_hip_device_type(ref)
    assert enum_values(edited, "DeviceType") == {**enum_values(ref, "DeviceType"), "HIP": 5}
    added = [ln for ln in edited.splitlines() if ln not in ref.splitlines()]
    assert len(added) == 2 and "HIP    = 5," in added[0] and 'return "hip";' in added[1]


def test_cpp_backend_program_without_a_device():
    exe = ROOT / "llm_core_amd" / "_build" / "test_backend_hip"
    if not exe.exists():
        pytest.skip("test_backend_hip not built")
    if Path("/dev/kfd").exists():
        pytest.skip("a GPU is visible: the device checks run in the gpu test")
    proc = subprocess.run([str(exe), "--no-device"], capture_output=True, text=True, timeout=60)
    assert proc.returncode == 0, proc.stdout + proc.stderr
