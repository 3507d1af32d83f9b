"""Build recipe for the C restatement (test infrastructure only).

Compiles ``oracle/c/xpool_oracle.c`` with gcc into
``oracle/_build/libxpool_oracle.so``.  The reference's own sources for this
path are CUDA (cooperative copy) or Python/Triton (the Dense operator), so no
``oracle/_ref`` build exists: nvcc and the CUDA headers they need are absent.
"""

from __future__ import annotations

import subprocess
from pathlib import Path

ORACLE_DIR = Path(__file__).resolve().parent
SOURCE = ORACLE_DIR / "c" / "xpool_oracle.c"
LIBRARY = ORACLE_DIR / "_build" / "libxpool_oracle.so"


def build() -> Path:
    LIBRARY.parent.mkdir(parents=True, exist_ok=True)
    temporary = LIBRARY.with_suffix(".so.tmp")
    subprocess.run(
        ["gcc", "-O2", "-std=c11", "-fPIC", "-shared", "-ffp-contract=off", str(SOURCE), "-o", str(temporary), "-lm"],
        check=True,
    )
    temporary.replace(LIBRARY)
    return LIBRARY


if __name__ == "__main__":
    print(build())
