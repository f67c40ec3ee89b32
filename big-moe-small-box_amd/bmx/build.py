"""Build libbmx.so in-tree (hipcc, gfx950). `python -m bmx.build` or bmx.build.build()."""
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(os.path.dirname(HERE), "csrc")


def build(jobs=8):
    subprocess.run(["make", "-s", f"-j{jobs}", "-C", CSRC], check=True)
    return os.path.join(HERE, "libbmx.so")


if __name__ == "__main__":
    print(build())
