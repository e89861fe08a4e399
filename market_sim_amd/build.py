"""Builds the in-tree native libraries.

  market_sim_amd/lib/libmarketforge_hip.so   gfx950 kernels + C ABI (hipcc)
  market_sim_amd/bench/_build/*              benchmark programs over the C++
                                             operator layer (g++)

Run ``python -m market_sim_amd.build``.  Recompiles what changed (make), or
everything with ``force`` (the driver's build check compiles every time).
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))


def build(jobs: int = 4, force: bool = False) -> None:
    for sub in ("csrc", "bench"):
        cmd = ["make", "-s", "-j", str(jobs), "-C", os.path.join(HERE, sub)]
        if force:
            cmd.insert(1, "-B")
        subprocess.run(cmd, check=True)


if __name__ == "__main__":
    build(int(sys.argv[1]) if len(sys.argv) > 1 else 4)
