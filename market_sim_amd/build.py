"""Builds the in-tree native libraries.

  market_sim_amd/lib/libmarketforge_hip.so   gfx950 kernels + C ABI (hipcc)

Run ``python -m market_sim_amd.build``.  Always recompiles what changed
(make), so a call after editing a source rebuilds before tests or GPU runs.
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))


def build(jobs: int = 4) -> None:
    subprocess.run(["make", "-s", "-j", str(jobs), "-C", os.path.join(HERE, "csrc")],
                   check=True)


if __name__ == "__main__":
    build(int(sys.argv[1]) if len(sys.argv) > 1 else 4)
