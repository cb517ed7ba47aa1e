"""The drop-in binding (brisk-llm_amd/binding/hip_session.h: class HipSession : Engine) on the CPU:
it compiles against the reference's own headers (src/engine.h, src/model.h), and the test library
oracle/Makefile builds from it (oracle/_ref/libhip_engine.so, with the reference's sources and
libbrisk_hip.so) exports its entry points.  No GPU: nothing is called that touches the device."""
import ctypes as C
import os
import shutil
import subprocess

import pytest

import pyoracle

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF_SRC = "/root/reference/src"


@pytest.mark.skipif(not os.path.isdir(REF_SRC), reason="the reference tree is only in the build container")
def test_binding_compiles_against_the_reference_headers(tmp_path):
    if shutil.which("g++") is None:
        pytest.skip("no C++ compiler")
    src = tmp_path / "use.cpp"
    # a translation unit as the reference's main.cpp would write it: an Engine made from a Model
    src.write_text('#include "hip_session.h"\n'
                   "std::unique_ptr<brisk::Engine> make(const brisk::Model& m, std::span<const std::byte> f, std::size_t c) {\n"
                   "    return std::make_unique<brisk::HipSession>(m, f, c);\n}\n")
    subprocess.run(["g++", "-std=c++20", "-fsyntax-only", "-Wall", "-Werror", "-include", "memory",
                    "-I", REF_SRC, "-I", os.path.join(ROOT, "brisk-llm_amd", "binding"), "-I", os.path.join(ROOT, "include"),
                    str(src)], check=True)


def test_hip_engine_library_exports_its_entry_points():
    if not pyoracle.hip_engine_available():
        pytest.skip("oracle/_ref/libhip_engine.so is not built (__graft_entry__.build() with the reference tree)")
    so = C.CDLL(pyoracle.HIP_ENGINE_PATH)
    missing = [n for n in pyoracle.HIP_ENGINE_EXPORTS if not hasattr(so, n)]
    assert not missing, missing
