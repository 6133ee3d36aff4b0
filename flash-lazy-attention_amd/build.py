"""Builds libflashlazy.so (the gfx950 HIP kernels + C ABI) in-tree with hipcc.

    python flash-lazy-attention_amd/build.py [--jobs N]

Objects go to flash-lazy-attention_amd/_build/, the library to
flash-lazy-attention_amd/adasplash/libflashlazy.so (where the Python package loads it).
"""
import argparse
import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "adasplash", "libflashlazy.so")
BUILD = os.path.join(HERE, "_build")
SOURCES = [
    "api.hip",
    "entmax.hip",
    "ada_f32.hip",
    "ada_f16.hip",
    "ada_bf16.hip",
    "lazy_f32.hip",
    "lazy_f16.hip",
    "lazy_bf16.hip",
    "lazy_dec_f32.hip",
    "lazy_dec_f16.hip",
    "lazy_dec_bf16.hip",
]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-I" + os.path.join(ROOT, "include"),
]


# Per-source flags.  The Lazy kernels produce no NaN from finite inputs (masked scores are -inf,
# every -inf - -inf is behind a select on the operand), so they are compiled without NaN
# semantics: fmaxf then needs no canonicalising v_max x, x, x per MFMA result (~30 VALU
# instructions per 64-key tile and sweep).  The AdaSplash threshold code relies on NaN
# comparisons (`!(nt > tau)`) and keeps the default.
SOURCE_FLAGS = {name: ["-fno-honor-nans"] for name in ("lazy_f32.hip", "lazy_f16.hip", "lazy_bf16.hip")}


def _compile(src):
    obj = os.path.join(BUILD, src.replace(".hip", ".o"))
    cmd = [HIPCC, *FLAGS, *SOURCE_FLAGS.get(src, []), "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{err}")
    return obj


def build(jobs=None, verbose=True):
    os.makedirs(BUILD, exist_ok=True)
    jobs = jobs or min(8, os.cpu_count() or 4)
    with cf.ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = OUT + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("link failed:\n" + r.stderr)
    os.replace(tmp, OUT)
    if verbose:
        print("built", OUT)
    return OUT


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    args = ap.parse_args()
    try:
        build(args.jobs)
    except RuntimeError as e:
        print(e, file=sys.stderr)
        sys.exit(1)
