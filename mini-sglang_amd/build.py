"""Build libmla_amd.so (gfx950) from csrc/*.hip with hipcc, in-tree.

Usage: python mini-sglang_amd/build.py [--jobs N]
The library lands in minisgl_amd/kernel/libmla_amd.so, where
minisgl_amd.kernel.lib loads it. Every call recompiles.
"""

from __future__ import annotations

import argparse
import concurrent.futures as cf
import glob
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
OUT = os.path.join(HERE, "minisgl_amd", "kernel", "libmla_amd.so")
# measured-peak kernels of the benchmark: a separate library, not part of libmla_amd's ABI
PEAKS_SRC = os.path.join(CSRC, "peaks", "mla_peaks.hip")
PEAKS_OUT = os.path.join(HERE, "minisgl_amd", "benchmark", "libmla_peaks.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
# packed-fp32 VALU forms are disabled for all device code built here.
FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


# per-source device flags: the prefill kernel's softmax needs no NaN handling in fmax (its scores
# are finite or -inf), which saves a canonicalising instruction per operand
SOURCE_FLAGS = {"mla_prefill.hip": ["-Xarch_device", "-fno-honor-nans"]}


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.basename(src) + ".o")
    cmd = [HIPCC, *FLAGS, *SOURCE_FLAGS.get(os.path.basename(src), []), "-c", src, "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "'-packed-fp32-ops' is not a recognized feature"
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{err}")
    if err.strip():
        print(err, file=sys.stderr)
    return obj


def _link(objs, out: str) -> None:
    tmp = out + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, out)


def build(jobs: int | None = None, verbose: bool = True) -> str:
    os.makedirs(BUILD, exist_ok=True)
    sources = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    jobs = jobs or min(8, len(sources) + 1)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, sources + [PEAKS_SRC]))
    _link(objs[:-1], OUT)
    _link(objs[-1:], PEAKS_OUT)
    if verbose:
        print(f"built {OUT} from {len(sources)} sources, and {PEAKS_OUT}")
    return OUT


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    build(ap.parse_args().jobs)
