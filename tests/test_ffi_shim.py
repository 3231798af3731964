"""The XLA FFI handler shim that INTEGRATION.md gives a maintainer (section 1),
compiled here with g++ against include/nanorts_amd.h and a declaration of the
part of XLA's FFI API it uses (tests/ffi_shim/ffi_surface.h), since jax and
its headers are absent from this image.

The compile pins the shim's calls into the C ABI (names, argument counts and
types) and each handler's parameters against its binding.  It does not pin
the declarations against XLA's own header: that takes a maintainer's build
against jax.ffi.include_dir().  The shim binds the reference's FFI targets
(src/nanorts/kernels/cuda/registry.cu:201-230)."""
from __future__ import annotations

import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
SURFACE = ROOT / "tests" / "ffi_shim"
HIP_INCLUDE = Path("/opt/rocm/include")


def _shim() -> str:
    text = (ROOT / "INTEGRATION.md").read_text()
    m = re.search(r"```cpp\n(.*?)```", text, re.S)
    assert m, "INTEGRATION.md holds no C++ block"
    code = m.group(1)
    assert code.count('#include "xla/ffi/api/ffi.h"') == 1
    return code.replace('#include "xla/ffi/api/ffi.h"', '#include "ffi_surface.h"')


def _compile(tmp_path: Path, code: str) -> subprocess.CompletedProcess:
    gxx = shutil.which("g++")
    if gxx is None or not (HIP_INCLUDE / "hip" / "hip_runtime.h").exists():
        pytest.skip("g++ or the HIP headers are missing")
    src = tmp_path / "nanorts_xla.cc"
    src.write_text(code)
    return subprocess.run([gxx, "-std=c++17", "-fsyntax-only", "-Wall", "-Wextra", "-Werror",
                           "-D__HIP_PLATFORM_AMD__", f"-I{HIP_INCLUDE}", f"-I{ROOT / 'include'}", f"-I{SURFACE}",
                           str(src)], capture_output=True, text=True, timeout=120)


def test_the_shim_compiles(tmp_path):
    done = _compile(tmp_path, _shim())
    assert done.returncode == 0, done.stderr[-4000:]


def test_the_shim_defines_each_target_it_lists():
    code = _shim()
    defined = set(re.findall(r"^NANORTS_XLA_HANDLER\((\w+),", code, re.M))
    listed = re.search(r'nanorts_targets\(\) \{\s*return ((?:"[^"]*"\s*)+);', code)
    assert listed
    names = set("".join(re.findall(r'"([^"]*)"', listed.group(1))).split(","))
    assert defined == names
    assert len(names) == 11


def test_a_binding_that_drops_an_operand_does_not_compile(tmp_path):
    """The binding check has teeth: the A* search target bound with one operand
    fewer than its handler takes is refused."""
    code = _shim()
    start = code.index("NANORTS_XLA_HANDLER(nanorts_astar_search, AstarSearch,")
    end = code.index(");", start)
    binding = code[start:end]
    assert binding.count(".Arg<ffi::AnyBuffer>()") == 4
    done = _compile(tmp_path, code[:start] + binding.replace(".Arg<ffi::AnyBuffer>()", "", 1) + code[end:])
    assert done.returncode != 0
    assert "do not match its binding" in done.stderr


def test_a_call_with_a_wrong_pointer_type_does_not_compile(tmp_path):
    code = _shim()
    call = "static_cast<int32_t*>(out->untyped_data()), extent(*out, 0)"
    assert call in code
    done = _compile(tmp_path, code.replace(call, "static_cast<float*>(out->untyped_data()), extent(*out, 0)", 1))
    assert done.returncode != 0
