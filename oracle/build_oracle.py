"""Build the C oracle ``oracle/_build/libnqoracle.so`` with gcc (test infrastructure).

The reference itself has no buildable C/C++ source for this path: its CPU
llama.cpp operators exist only as patch hunks against a fork that is not in the
repository, so there is no ``oracle/_ref`` build.
"""

from __future__ import annotations

import subprocess
from pathlib import Path

ORACLE_DIR = Path(__file__).resolve().parent
LIBRARY = ORACLE_DIR / "_build" / "libnqoracle.so"


def build() -> Path:
    LIBRARY.parent.mkdir(parents=True, exist_ok=True)
    tmp = LIBRARY.with_name(LIBRARY.name + ".tmp")
    cmd = ["gcc", "-O2", "-std=c11", "-Wall", "-Wextra", "-shared", "-fPIC",
           str(ORACLE_DIR / "nq_oracle.c"), "-o", str(tmp)]
    subprocess.run(cmd, check=True)
    tmp.replace(LIBRARY)
    return LIBRARY


if __name__ == "__main__":
    print(build())
