"""Build the gfx950 HIP library ``crosspool_amd/_lib/libxpool_amd.so`` in-tree.

Each ``csrc/*.hip`` translation unit is compiled with hipcc for gfx950 only,
in parallel, then linked into one shared library exporting the C ABI declared
in ``include/xpool_amd.h``.  Packed-fp32 instruction selection is disabled
for all device code (the generated packed forms are not trusted on the target
machines); hipcc's host pass warns that it does not know that feature.
"""

from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
SOURCE_DIR = PACKAGE_DIR / "csrc"
OBJECT_DIR = PACKAGE_DIR / "_build"
LIBRARY = PACKAGE_DIR / "_lib" / "libxpool_amd.so"
# Hardware-ceiling probes launched by `bench.py --ceilings` (not part of the C ABI).
PROBE_SOURCE = PACKAGE_DIR / "probes" / "ceilings.hip"
PROBE_LIBRARY = PACKAGE_DIR / "_lib" / "libxpool_probes.so"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

COMPILE_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++20",
    "-fPIC",
    "-Wall",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
]


def sources() -> list[Path]:
    return sorted(SOURCE_DIR.glob("*.hip"))


def _compile(source: Path) -> Path:
    target = OBJECT_DIR / (source.stem + ".o")
    command = [HIPCC, *COMPILE_FLAGS, "-c", str(source), "-o", str(target)]
    result = subprocess.run(command, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"hipcc failed for {source.name}:\n{result.stderr}")
    return target


def _link(objects: list[Path], library: Path) -> None:
    temporary = library.with_name(library.name + ".tmp")
    command = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objects), "-o", str(temporary)]
    result = subprocess.run(command, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"hipcc link of {library.name} failed:\n{result.stderr}")
    temporary.replace(library)


def build(verbose: bool = False) -> Path:
    """Compile every HIP source and link the shared library (and the probe library); returns its path."""

    OBJECT_DIR.mkdir(parents=True, exist_ok=True)
    LIBRARY.parent.mkdir(parents=True, exist_ok=True)
    units = sources()
    workers = min(len(units), max(1, min(os.cpu_count() or 1, 8)))
    with ThreadPoolExecutor(max_workers=workers) as pool:
        objects = list(pool.map(_compile, [*units, PROBE_SOURCE]))
    _link(objects[:-1], LIBRARY)
    _link(objects[-1:], PROBE_LIBRARY)
    if verbose:
        print(f"built {LIBRARY}", file=sys.stderr)
    return LIBRARY


if __name__ == "__main__":
    build(verbose=True)
