"""Build the dataplane's native libraries in-tree, for gfx950.

    python -m kvsnap_amd.build

``_native/libkvsnap_hip.so``  pinned pool + HIP kernels (hipcc, gfx950)
``_native/libkvsnap_io.so``   host CRC32C + pread/pwrite pool (g++)

Both always rebuild when asked; the loaders only use what is already built.
"""
from __future__ import annotations

import os
import shutil
import subprocess
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
CSRC = PACKAGE / "csrc"
NATIVE = PACKAGE / "_native"
HIP_LIBRARY = NATIVE / "libkvsnap_hip.so"
IO_LIBRARY = NATIVE / "libkvsnap_io.so"

ARCH = os.environ.get("KVSNAP_OFFLOAD_ARCH", "gfx950")

HIPCC_FLAGS = [
    "-std=c++17", "-O3", "-fPIC", "-shared", f"--offload-arch={ARCH}",
    # Keep the compiler from emitting packed fp32 instructions.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wextra", "-Werror",
    # the host pass does not know the gfx feature above
    "-Wno-unused-command-line-argument",
]


def _hipcc() -> str:
    for candidate in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if candidate and Path(candidate).is_file():
            return candidate
    raise RuntimeError("hipcc not found: the HIP dataplane library cannot be built")


def _run(cmd):
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode:
        raise RuntimeError(f"build failed: {' '.join(cmd)}\n{result.stdout}\n{result.stderr}")
    return result


def _atomic_output(target: Path) -> Path:
    target.parent.mkdir(parents=True, exist_ok=True)
    return target.with_name(target.name + f".tmp{os.getpid()}")


def build_hip(target: Path = HIP_LIBRARY) -> Path:
    tmp = _atomic_output(target)
    _run([_hipcc(), *HIPCC_FLAGS, "-o", str(tmp), str(CSRC / "kernels.hip"), str(CSRC / "pool.cpp")])
    os.replace(tmp, target)
    return target


def build_io(target: Path = IO_LIBRARY) -> Path:
    tmp = _atomic_output(target)
    _run(["g++", "-std=c++17", "-O3", "-fPIC", "-shared", "-pthread", "-Wall", "-Wextra", "-Werror",
          "-o", str(tmp), str(CSRC / "io.cpp")])
    os.replace(tmp, target)
    return target


def build_all() -> list[Path]:
    return [build_io(), build_hip()]


if __name__ == "__main__":
    for path in build_all():
        print(path)
