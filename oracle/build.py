"""Build the C oracle (TEST INFRASTRUCTURE ONLY): gcc -O2 dh_oracle.c -> oracle/_build/libdh_oracle.so.

The reference implementation is Python + Triton with no C/C++ sources, so there is no
oracle/_ref build of the reference itself; this compiles the oracle's own C restatement.
"""

import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "_build", "libdh_oracle.so")


def build():
    os.makedirs(os.path.dirname(OUT), exist_ok=True)
    tmp = OUT + ".tmp"
    subprocess.run(["gcc", "-O2", "-fPIC", "-shared", "-std=c11", "-Wall",
                    os.path.join(HERE, "dh_oracle.c"), "-o", tmp, "-lm"], check=True)
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build())
