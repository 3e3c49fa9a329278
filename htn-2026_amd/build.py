"""Build libqdecode.so (HIP kernels + C ABI) for gfx950 in-tree with hipcc.

    python htn-2026_amd/build.py [--jobs N]

Each csrc/*.hip is compiled to an object in csrc/_build/ (in parallel), then linked into
htn-2026_amd/libqdecode.so, next to the Python host code that loads it.
"""

import argparse
import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "libqdecode.so")
ARCH = os.environ.get("QD_OFFLOAD_ARCH", "gfx950")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17", "-Wall",
    # a variable read inside its own initialiser (e.g. a macro local named like its argument)
    # builds a garbage address: never let it through
    "-Werror=uninitialized", "-Wno-unused-function",
    "-Wno-unused-variable", "-Wno-unused-but-set-variable",
    # packed fp32 forms are kept out of the generated code (see the build notes)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(HERE, "..", "include"),
]


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def compile_one(src, objdir):
    obj = os.path.join(objdir, os.path.basename(src)[:-4] + ".o")
    cmd = [HIPCC] + FLAGS + ["-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr}")
    noise = "is not a recognized feature for this target"
    warn = "\n".join(line for line in r.stderr.splitlines() if noise not in line).strip()
    return obj, warn


def build(jobs=None, verbose=True):
    objdir = os.path.join(CSRC, "_build")
    os.makedirs(objdir, exist_ok=True)
    srcs = sources()
    jobs = jobs or min(len(srcs), os.cpu_count() or 4, 16)
    with cf.ThreadPoolExecutor(jobs) as ex:
        results = list(ex.map(lambda s: compile_one(s, objdir), srcs))
    for obj, warn in results:
        if warn and verbose:
            print(f"[build] {os.path.basename(obj)}:\n{warn}", file=sys.stderr)
    tmp = OUT + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp] + [o for o, _ in results]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, OUT)
    if verbose:
        print(f"[build] {OUT}")
    return OUT


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    a = ap.parse_args()
    build(a.jobs)
