"""Build the C oracle (oracle/liboracle.so) with gcc. Test infrastructure only.

    python -m oracle.build
"""

from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
SRC = HERE / "paged_attention_oracle.c"
LIB = HERE / "liboracle.so"


def build() -> Path:
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        raise RuntimeError("no C compiler for the oracle")
    tmp = LIB.with_suffix(".so.tmp")
    subprocess.run([cc, "-O2", "-std=c11", "-fPIC", "-shared", "-Wall", "-o", str(tmp), str(SRC), "-lm"], check=True)
    tmp.replace(LIB)
    return LIB


if __name__ == "__main__":
    print(build())
