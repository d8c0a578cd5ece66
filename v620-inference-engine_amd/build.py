"""Builds libqwq4.so (the HIP kernels + C ABI) in place, for gfx950 only.

    python v620-inference-engine_amd/build.py [-j N]

One hipcc job per source, then a shared link. The library lands next to this
file so it travels with the source tree.
"""
import argparse
import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "libqwq4.so")
OBJ = os.path.join(HERE, "_build")
SOURCES = ["q4_gemv.hip", "q4_gemv_f16.hip", "moe_gemv.hip", "q4_gemm.hip", "w16_gemv.hip", "i8_gemv.hip", "moe_w4a8.hip", "moe_route.hip", "q4_util.hip", "moe_grouped.hip", "st_loader.cpp", "wcache.cpp", "capi.cpp"]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I" + os.path.join(ROOT, "include"), "-I" + CSRC,
]


# Kernel arguments preloaded into SGPRs at wave launch (gfx950): the first
# weight request then does not wait on a scalar load of the argument block,
# which the latency-bound GEMVs feel at every launch.
PRELOAD = ["-mllvm", "-amdgpu-kernarg-preload-count=16"]
SOURCE_FLAGS = {"q4_gemv.hip": PRELOAD, "q4_gemv_f16.hip": PRELOAD, "w16_gemv.hip": PRELOAD, "i8_gemv.hip": PRELOAD}


def _compile(src):
    obj = os.path.join(OBJ, src + ".o")
    lang = ["-x", "hip"] if src.endswith(".cpp") else []
    cmd = [HIPCC] + FLAGS + SOURCE_FLAGS.get(src, []) + lang + ["-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{err}")
    return obj, err


def build(jobs=None, verbose=False):
    os.makedirs(OBJ, exist_ok=True)
    jobs = jobs or min(len(SOURCES), os.cpu_count() or 1)
    with cf.ThreadPoolExecutor(jobs) as ex:
        results = list(ex.map(_compile, SOURCES))
    for _, err in results:
        if err.strip() and verbose:
            print(err, file=sys.stderr)
    objs = [o for o, _ in results]
    tmp = OUT + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp] + objs
    subprocess.run(cmd, check=True)
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("-j", type=int, default=None)
    ap.add_argument("-v", action="store_true")
    a = ap.parse_args()
    print(build(a.j, a.v))
