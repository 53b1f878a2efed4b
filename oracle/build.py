"""Compile the oracle's C restatement (``lfilter.c``) into ``oracle/liboracle.so``.

Test infrastructure only.  Called by ``__graft_entry__.build()``; the shared
object is git-ignored and travels to the GPU box with the tree.
"""

import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
LIB = HERE / "liboracle.so"


def build(verbose: bool = False) -> Path:
    cmd = [
        "gcc",
        "-O2",
        "-fPIC",
        "-shared",
        "-std=c99",
        str(HERE / "lfilter.c"),
        "-o",
        str(LIB),
    ]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    return LIB


if __name__ == "__main__":
    build(verbose="-v" in sys.argv)
