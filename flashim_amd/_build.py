"""Ahead-of-time build of the HIP library (``libflashim_amd.so``, gfx950) and of the host build of its scalar numerics
(``libfim_host.so``, used by the CPU tests), and the device probes the tests and the bench use
(``libflashim_amd_probe.so``: numerics hooks and an MFMA microbenchmark, kept out of the product library). The libraries are built in-tree so they travel with the source tree; the
ctypes loader in :mod:`flashim_amd._lib` only loads what is built and never compiles at import time.

Flags: ``-ffp-contract=off`` keeps the epilogues' separate multiply and add roundings (the reference's order) unless a
kernel asks for an FMA explicitly; ``-packed-fp32-ops`` is disabled for all device code.
"""

from __future__ import annotations

import os
import shutil
import subprocess
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
CSRC = PACKAGE / "csrc"
BUILD = PACKAGE / "_build"
LIBRARY = PACKAGE / "libflashim_amd.so"
HOST_LIBRARY = PACKAGE / "libfim_host.so"
DEVICE_SOURCES = ("quantize.hip", "igemm.hip", "depthwise.hip", "dwpw.hip", "mlp.hip", "stem.hip", "pointwise.hip", "version.hip")
PROBE_LIBRARY = PACKAGE / "libflashim_amd_probe.so"
PROBE_SOURCES = ("probe.hip",)
ARCH = os.environ.get("FLASHIM_AMD_ARCH", "gfx950")
HIP_FLAGS = (
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-ffp-contract=off", "-munsafe-fp-atomics",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", f"-I{CSRC}",
)


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found: the flashim_amd HIP library cannot be built")
    return path


def _run(cmd: list[str]) -> None:
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"build step failed ({' '.join(cmd)}):\n{result.stderr[-4000:]}")


def build(jobs: int = 4) -> Path:
    """Compile every HIP source for gfx950 and link ``libflashim_amd.so``; build ``libfim_host.so``. Always rebuilds."""
    BUILD.mkdir(exist_ok=True)
    compiler = hipcc()
    sources = DEVICE_SOURCES + PROBE_SOURCES
    objects = {src: BUILD / (src.rsplit(".", 1)[0] + ".o") for src in sources}
    commands = [[compiler, *HIP_FLAGS, "-c", str(CSRC / src), "-o", str(objects[src])] for src in sources]
    with ThreadPoolExecutor(max_workers=jobs) as pool:
        list(pool.map(_run, commands))
    for library, srcs in ((LIBRARY, DEVICE_SOURCES), (PROBE_LIBRARY, PROBE_SOURCES)):
        temporary = library.with_suffix(f".{os.getpid()}.tmp")
        _run([compiler, "-shared", "-fPIC", f"--offload-arch={ARCH}", *(str(objects[s]) for s in srcs),
              "-o", str(temporary)])
        temporary.replace(library)
    host_tmp = HOST_LIBRARY.with_suffix(f".{os.getpid()}.tmp")
    _run(["g++", "-O2", "-std=c++17", "-fPIC", "-shared", str(CSRC / "numerics_host.cpp"), "-o", str(host_tmp)])
    host_tmp.replace(HOST_LIBRARY)
    return LIBRARY


if __name__ == "__main__":
    print(build())
