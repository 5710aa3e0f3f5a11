"""The C++ binding shown in INTEGRATION.md (fast-llm_amd/integration/
hip_backend.cpp) compiles against the reference runtime's own headers and
links against the built library: the Task / flh_task layout static_assert,
the RtShared field names (fast_kernels, i8_cpu_mask, i8k_cpu_mask,
src/runtime/runtime_internal.h:69-75) and every flh_* call it makes.

CPU only; skipped where the reference sources are absent (the GPU box)."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF = "/root/reference"
SRC = os.path.join(ROOT, "fast-llm_amd", "integration", "hip_backend.cpp")
LIB = os.path.join(ROOT, "fast-llm_amd", "libfastllm_hip.so")


@pytest.mark.skipif(not os.path.isdir(os.path.join(REF, "src", "runtime")), reason="reference sources absent")
@pytest.mark.skipif(shutil.which("g++") is None, reason="no g++")
def test_binding_compiles_and_links(tmp_path):
    inc = ["-I", os.path.join(ROOT, "include"), "-I", os.path.join(REF, "include"),
           "-I", os.path.join(REF, "src"), "-I", os.path.join(REF, "src", "runtime")]   # it lives in src/runtime
    obj = tmp_path / "hip_backend.o"
    subprocess.run(["g++", "-std=c++17", "-Wall", "-Werror", "-c", "-fPIC", SRC, "-o", str(obj)] + inc,
                   check=True, capture_output=True, text=True)
    if not os.path.exists(LIB):
        pytest.skip("library not built")
    # every flh_* symbol the binding uses resolves in the built library
    so = tmp_path / "libbinding.so"
    subprocess.run(["g++", "-shared", str(obj), "-o", str(so), "-L", os.path.dirname(LIB), "-lfastllm_hip",
                    "-Wl,--no-undefined", "-Wl,-rpath-link,/opt/rocm/lib"],
                   check=True, capture_output=True, text=True)


def test_binding_matches_integration_doc():
    """The compiled file is the code INTEGRATION.md shows."""
    md = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    i = md.index("```cpp\n") + len("```cpp\n")
    doc = md[i:md.index("```", i)]
    def code(t):
        return [l for l in t.splitlines() if l.strip() and not l.startswith("#include")]
    src = code(open(SRC).read())
    want = code(doc)
    assert src[-len(want):] == want
