"""Build libnsw.so (all HIP kernels + the C ABI) for gfx950, in-tree.

    python neural-scaling-weather_amd/build.py [--jobs N] [--verbose] [--stamps]

Each ``csrc/*.hip`` is compiled to an object with hipcc (in parallel), then
linked into ``nsw/libnsw.so``.  Always rebuilds (this is the "does it build"
check).  Packed fp32 VALU ops are disabled for all device code.  ``--stamps``
builds ``nsw/libnsw_stamps.so`` instead: the same library with the GEMM's
per-tile phase stamps compiled in (-DNSW_GEMM_STAMPS=1; read by
``bench.py --gemm-phases``).
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import glob
import os
import shutil
import subprocess
import sys
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "nsw", "libnsw.so")
OUT_STAMPS = os.path.join(HERE, "nsw", "libnsw_stamps.so")
ARCH = os.environ.get("NSW_OFFLOAD_ARCH", "gfx950")

HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(ROOT, "include"),
    "-Wno-unused-command-line-argument",
]


def _compile(src: str, obj: str, verbose: bool, defines=()) -> str:
    cmd = [HIPCC, *FLAGS, *defines, "-c", src, "-o", obj]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    # the host pass warns that it does not know the packed-fp32 feature: harmless
    err = "\n".join(l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {os.path.basename(src)}:\n{err}")
    return err


def build(jobs: int | None = None, verbose: bool = False, stamps: bool = False) -> str:
    out = OUT_STAMPS if stamps else OUT
    defines = ["-DNSW_GEMM_STAMPS=1"] if stamps else []
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    jobs = jobs or min(len(srcs), max(1, (os.cpu_count() or 4)), 16)
    with tempfile.TemporaryDirectory(prefix="nsw_build_") as tmp:
        objs = [os.path.join(tmp, os.path.basename(s).replace(".hip", ".o")) for s in srcs]
        with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
            futs = [ex.submit(_compile, s, o, verbose, defines) for s, o in zip(srcs, objs)]
            for f in futs:
                w = f.result()
                if w.strip() and verbose:
                    print(w)
        tmp_out = out + ".tmp"
        cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp_out]
        if verbose:
            print(" ".join(cmd), flush=True)
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"link failed:\n{r.stderr}")
        os.replace(tmp_out, out)
    return out


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("--verbose", action="store_true")
    ap.add_argument("--stamps", action="store_true", help="build nsw/libnsw_stamps.so with the GEMM phase stamps")
    a = ap.parse_args()
    print(build(a.jobs, a.verbose, a.stamps))
