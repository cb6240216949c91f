"""The boundary compiled as gemma.c's own callers would use it: a C++ caller
with the reference's call shapes (std::vector ring helpers, the runtime
state functions, the norm+RoPE launchers as function pointers of the
reference's parameter lists, the Layout-A offset in constant expressions)
built with hipcc, and a plain C caller built with gcc, both against
include/*.h and linked to libgemma4_kv.so; each runs its host-only checks
(no GPU needed)."""
import subprocess
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent
LIB_DIR = REPO / "gemma.c_amd" / "gemma_kv"
CPP = REPO / "tests" / "cpp"


def _lib():
    if not (LIB_DIR / "libgemma4_kv.so").exists():
        pytest.skip("libgemma4_kv.so not built")


def _run(cmd, cwd):
    proc = subprocess.run(cmd, cwd=cwd, capture_output=True, text=True, timeout=300)
    noise = ("packed-fp32-ops", "not a recognized feature")
    err = "\n".join(l for l in proc.stderr.splitlines() if not any(n in l for n in noise))
    assert proc.returncode == 0, f"{' '.join(map(str, cmd))}\n{proc.stdout}\n{err}"
    return proc.stdout


def test_cpp_caller_compiles_links_and_runs(tmp_path):
    _lib()
    exe = tmp_path / "boundary_caller"
    _run(["/opt/rocm/bin/hipcc", "--offload-arch=gfx950", "-std=c++17", "-Wall",
          f"-I{REPO / 'include'}", str(CPP / "boundary_caller.cpp"), f"-L{LIB_DIR}",
          "-lgemma4_kv", f"-Wl,-rpath,{LIB_DIR}", "-o", str(exe)], tmp_path)
    assert "boundary caller ok" in _run([str(exe)], tmp_path)


def test_c_caller_compiles_links_and_runs(tmp_path):
    _lib()
    exe = tmp_path / "boundary_caller_c"
    _run(["gcc", "-std=c11", "-Wall", "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include",
          f"-I{REPO / 'include'}", str(CPP / "boundary_caller.c"), f"-L{LIB_DIR}",
          "-lgemma4_kv", f"-Wl,-rpath,{LIB_DIR}", "-o", str(exe)], tmp_path)
    assert "c caller ok" in _run([str(exe)], tmp_path)
