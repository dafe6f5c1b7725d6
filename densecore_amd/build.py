"""Compile ``libdcattn.so`` (all HIP sources in ``csrc/``) for gfx950 with hipcc, in-tree."""
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")


def build(jobs=8, force=False):
    """Run the csrc Makefile; ``force`` rebuilds every object."""
    cmd = ["make", "-s", "-C", CSRC, f"-j{jobs}"]
    if force:
        cmd.append("-B")
    subprocess.run(cmd, check=True)
    return os.path.join(HERE, "libdcattn.so")


if __name__ == "__main__":
    print(build())
