"""Compile libqattn.so for gfx950 in-tree (telefuser_amd/lib/)."""

import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))


def build(force: bool = True) -> str:
    args = ["make", "-C", os.path.join(HERE, "csrc"), "-j4"]
    if force:
        args.insert(1, "-B")
    subprocess.run(args, check=True)
    return os.path.join(HERE, "lib", "libqattn.so")


if __name__ == "__main__":
    print(build())
