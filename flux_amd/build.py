"""Build ``flux_amd/lib/libflux_amd.so`` for gfx950 with hipcc (no torch extension).

Each translation unit is compiled in parallel, then linked into one shared
library whose C ABI is ``include/flux_amd.h``.  Usage::

    python -m flux_amd.build            # or flux_amd.build.build()
    python -m flux_amd.build --trace    # also the timestamped decode library

The ``--trace`` build defines ``FLUX_TRACE`` (decode phase timestamps, read by
``flux_amd.trace_decode``) and writes ``flux_amd/lib/libflux_amd_trace.so``;
the normal library is compiled without it and carries no trace code.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PACKAGE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PACKAGE)
CSRC = os.path.join(PACKAGE, "csrc")
LIB_DIR = os.path.join(PACKAGE, "lib")
LIBRARY = os.path.join(LIB_DIR, "libflux_amd.so")
TRACE_LIBRARY = os.path.join(LIB_DIR, "libflux_amd_trace.so")
SOURCES = ("decode_kernels.hip", "prefill_kernels.hip", "eager_kernels.hip", "runtime.cpp", "capi.cpp")
ARCH = os.environ.get("FLUX_AMD_ARCH", "gfx950")


def hipcc() -> str:
    for candidate in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if candidate and os.path.exists(candidate):
            return candidate
    raise RuntimeError("hipcc not found; install ROCm or set HIPCC")


def _flags() -> list[str]:
    return [
        "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-mcode-object-version=5",
        # Packed FP32 VALU forms are disabled for every kernel in this library.
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wall", "-Wno-unused-function",
        f"-I{CSRC}", f"-I{os.path.join(ROOT, 'include')}",
    ]


def _compile(source: str, build_dir: str, defines: tuple[str, ...] = ()) -> str:
    obj = os.path.join(build_dir, os.path.splitext(source)[0] + ".o")
    cmd = [hipcc(), *_flags(), *(f"-D{d}" for d in defines)]
    if source.endswith(".cpp"):
        cmd += ["-x", "hip"]
    cmd += ["-c", os.path.join(CSRC, source), "-o", obj]
    result = subprocess.run(cmd, capture_output=True, text=True)
    messages = "\n".join(
        line for line in (result.stdout + result.stderr).splitlines()
        if "packed-fp32-ops" not in line and "not a recognized feature" not in line
    )
    if result.returncode != 0:
        raise RuntimeError(f"compiling {source} failed:\n{messages}")
    return obj


def build(verbose: bool = True, trace: bool = False) -> str:
    """Compile every HIP translation unit and link the shared library.

    ``trace=True`` builds the ``FLUX_TRACE`` variant into its own directory and
    library file; it never replaces the normal library.
    """
    build_dir = os.path.join(ROOT, "_build", "trace") if trace else os.path.join(ROOT, "_build")
    library = TRACE_LIBRARY if trace else LIBRARY
    defines = ("FLUX_TRACE",) if trace else ()
    os.makedirs(build_dir, exist_ok=True)
    os.makedirs(LIB_DIR, exist_ok=True)
    with ThreadPoolExecutor(max_workers=min(4, os.cpu_count() or 1)) as pool:
        objects = list(pool.map(lambda s: _compile(s, build_dir, defines), SOURCES))
    tmp = library + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-mcode-object-version=5", "-shared", "-fPIC", *objects, "-o", tmp]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"linking failed:\n{result.stdout}{result.stderr}")
    os.replace(tmp, library)
    if verbose:
        print(f"built {library}", flush=True)
    return library


def build_oracle(verbose: bool = True) -> str | None:
    """Build ``oracle/_ref`` from the reference's CPU sources when they are present."""
    if not os.path.isdir("/root/reference/csrc"):
        return None
    result = subprocess.run(["make", "-C", os.path.join(ROOT, "oracle")], capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"building oracle/_ref failed:\n{result.stdout}{result.stderr}")
    path = os.path.join(ROOT, "oracle", "_ref", "libfluxref.so")
    if verbose:
        print(f"built {path}", flush=True)
    return path


if __name__ == "__main__":
    build()
    build_oracle()
    if "--trace" in sys.argv[1:]:
        build(trace=True)
    sys.exit(0)
