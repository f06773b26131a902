"""Build the C parts of the CPU oracle (test infrastructure only).

Compiles ``kmeans_ref.c`` into ``oracle/_build/libkmeans_ref.so`` with plain
gcc and ``-ffp-contract=off`` so every fused multiply-add is an explicit
``fmaf`` call.  Invoked from ``__graft_entry__.build()`` and lazily by
``oracle.kmeans``.
"""

from __future__ import annotations

import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))


def build() -> str:
    out_dir = os.path.join(HERE, "_build")
    os.makedirs(out_dir, exist_ok=True)
    out = os.path.join(out_dir, "libkmeans_ref.so")
    tmp = out + ".tmp"
    cmd = ["gcc", "-O2", "-std=c11", "-ffp-contract=off", "-fno-fast-math", "-fPIC", "-shared",
           os.path.join(HERE, "kmeans_ref.c"), "-o", tmp, "-lm"]
    subprocess.run(cmd, check=True)
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    print(build())
