"""Build recipe of the gfx950 kernel library (hipcc, in-tree).

`build()` always compiles; `library_path()` names the in-tree product.  The
library is a plain shared object with the C ABI of include/nanorts_amd.h.
"""
from __future__ import annotations

import hashlib
import os
import shutil
import subprocess
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
ROOT = PACKAGE.parent
SOURCES = (PACKAGE / "csrc" / "nanorts_amd.hip", PACKAGE / "csrc" / "engine.h", PACKAGE / "csrc" / "envstep.h", PACKAGE / "csrc" / "rollout.h",
           PACKAGE / "csrc" / "bots.h", PACKAGE / "csrc" / "gridnet.h",
           ROOT / "include" / "nanorts_amd.h")
OUTPUT = PACKAGE / "_lib" / "libnanorts_amd.so"
ARCH = "gfx950"


def source_digest() -> str:
    digest = hashlib.sha256()
    for path in SOURCES:
        digest.update(path.read_bytes())
    return digest.hexdigest()[:16]


def hipcc() -> str:
    found = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(found):
        raise RuntimeError("hipcc was not found; the nanorts_amd kernels cannot be built")
    return found


def command(output: Path = OUTPUT) -> list[str]:
    return [
        hipcc(), f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-shared",
        # packed FP32 instructions stay off: this code is integer-only and
        # does not want the compiler to form them.
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        f'-DNANORTS_BUILD_ID="{source_digest()}"',
        str(PACKAGE / "csrc" / "nanorts_amd.hip"), "-o", str(output),
    ]


def build(verbose: bool = False) -> Path:
    OUTPUT.parent.mkdir(parents=True, exist_ok=True)
    tmp = OUTPUT.with_suffix(".so.tmp")
    result = subprocess.run(command(tmp), capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"hipcc failed ({result.returncode}):\n{result.stderr}")
    if verbose and result.stderr.strip():
        print(result.stderr)
    os.replace(tmp, OUTPUT)
    return OUTPUT


def library_path() -> Path:
    return OUTPUT


if __name__ == "__main__":
    print(build(verbose=True))
