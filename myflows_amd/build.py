"""Ahead-of-time build of libmfhip.so for gfx950 with hipcc.

The library is compiled from the HIP sources under ``csrc/`` into ``myflows_amd/libmfhip.so`` (in
tree, so that the built file travels with the package to the GPU host). Each translation unit is
compiled in its own hipcc process, in parallel, then linked. ``build()`` always recompiles;
``ensure_built()`` only builds when the library is missing or older than a source file.
Follows the role of the reference's ``ops/cuda_native/build.py:143-155`` (a build on first use),
without CMake: hipcc is the whole toolchain.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import tempfile
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
SOURCE_DIR = PACKAGE / "csrc"
INCLUDE_DIR = PACKAGE.parent / "include"
LIBRARY = PACKAGE / "libmfhip.so"
ARCH = "gfx950"
# Packed FP32 instructions are kept out of the generated code (they are avoided on this hardware);
# hipcc's host pass warns that it does not know the feature, which is harmless.
HIP_FLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-fvisibility=hidden",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-Wno-unused-command-line-argument"]


# Extra flags per translation unit. The implicit convolutions keep their MFMA accumulators in
# ordinary VGPRs: their per-stage FP32 sums then read them without v_accvgpr_read copies (measured
# on MI355X: the batch-64 layer1 products 3 % faster, the same bits).
UNIT_FLAGS = {"implicit.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


class BuildError(RuntimeError):
    pass


def sources():
    return sorted(SOURCE_DIR.glob("*.hip"))


def _inputs():
    return sources() + sorted(SOURCE_DIR.glob("*.h")) + sorted(INCLUDE_DIR.glob("*.h")) + [Path(__file__)]


def stale_reason():
    if not LIBRARY.exists():
        return "missing"
    built = LIBRARY.stat().st_mtime
    for path in _inputs():
        if path.stat().st_mtime > built:
            return f"{path.name} is newer than the library"
    return None


def _hipcc():
    for candidate in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if candidate and Path(candidate).exists():
            return candidate
    raise BuildError("hipcc not found (set HIPCC or install ROCm)")


def _run(command):
    result = subprocess.run(command, capture_output=True, text=True)
    if result.returncode != 0:
        raise BuildError(f"{' '.join(command)}\n{result.stdout}{result.stderr}")


def build(verbose=False):
    """Compile every HIP translation unit for gfx950 and link libmfhip.so (always rebuilds)."""
    hipcc = _hipcc()
    with tempfile.TemporaryDirectory(prefix="mfhip-build-") as work:
        objects = []
        commands = []
        for source in sources():
            obj = Path(work) / (source.stem + ".o")
            objects.append(obj)
            commands.append([hipcc, *HIP_FLAGS, *UNIT_FLAGS.get(source.name, []), "-c", str(source), "-o", str(obj)])
        workers = max(1, min(len(commands), int(os.environ.get("MAX_JOBS", os.cpu_count() or 1))))
        with ThreadPoolExecutor(max_workers=workers) as pool:
            for command, _ in zip(commands, pool.map(_run, commands)):
                if verbose:
                    print(" ".join(command))
        tmp = LIBRARY.with_suffix(".so.tmp")
        _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objects), "-o", str(tmp)])
        os.replace(tmp, LIBRARY)
    return LIBRARY


def ensure_built():
    if stale_reason() is not None:
        build()
    return LIBRARY


if __name__ == "__main__":
    print(build(verbose=True))
