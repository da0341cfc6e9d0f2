"""Build libdh_mixer.so (gfx950) in-tree from ``csrc/*.hip``.

    python -m dispatcher_hybrid._build

Compiles every translation unit with ``hipcc --offload-arch=gfx950`` in parallel, links one shared
library into ``dispatcher_hybrid/_lib/``, and replaces the old file atomically. Needs only hipcc
(no GPU): the code objects are embedded in the library.
"""

import glob
import os
import shutil
import subprocess
import sys
import tempfile

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
PROJECT_DIR = os.path.dirname(PKG_DIR)                      # dispatcher-hybrid-2_amd/
CSRC_DIR = os.path.join(PROJECT_DIR, "csrc")
REPO_DIR = os.path.dirname(PROJECT_DIR)
INCLUDE_DIRS = [os.path.join(REPO_DIR, "include"), CSRC_DIR]
OUT_DIR = os.path.join(PKG_DIR, "_lib")
LIB = os.path.join(OUT_DIR, "libdh_mixer.so")

ARCH = os.environ.get("DH_OFFLOAD_ARCH", "gfx950")
HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")

# Packed-fp32 VALU ops stay off: hipcc may only use scalar fp32 instructions.
COMMON_FLAGS = [f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
                "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
                "-Wno-unused-command-line-argument"]


def sources():
    return sorted(glob.glob(os.path.join(CSRC_DIR, "*.hip")))


def build(verbose=False):
    srcs = sources()
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC_DIR}")
    os.makedirs(OUT_DIR, exist_ok=True)
    inc = [f"-I{d}" for d in INCLUDE_DIRS]
    with tempfile.TemporaryDirectory(prefix="dh_build_") as tmp:
        procs = []
        objs = []
        for src in srcs:
            obj = os.path.join(tmp, os.path.basename(src) + ".o")
            objs.append(obj)
            cmd = [HIPCC] + COMMON_FLAGS + inc + ["-c", src, "-o", obj]
            procs.append((cmd, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)))
        failed = []
        for cmd, p in procs:
            out = p.communicate()[0].decode(errors="replace")
            out = "\n".join(l for l in out.splitlines() if "packed-fp32-ops" not in l)
            if p.returncode != 0 or "warning:" in out:
                # warnings fail the build too (an inline-asm clobber of a reserved register is one)
                failed.append(f"$ {' '.join(cmd)}\n{out}")
            elif verbose and out.strip():
                print(out)
        if failed:
            raise RuntimeError("hipcc failed:\n" + "\n".join(failed))
        tmp_lib = LIB + ".tmp"
        cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp_lib] + objs
        p = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)
        if p.returncode != 0:
            raise RuntimeError(f"link failed:\n$ {' '.join(cmd)}\n{p.stdout.decode(errors='replace')}")
        os.replace(tmp_lib, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
