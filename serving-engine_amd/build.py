"""Builds libkvhot.so (the C-ABI HIP library) for gfx950 with hipcc.

Usage: python serving-engine_amd/build.py [--jobs N] [--define NAME=VALUE ...]

The library lands next to this file so it travels with the source tree.
Sources compile in parallel to objects under _build/, then link into one
shared object.  Always recompiles (the "does it build" check relies on that).
"""
from __future__ import annotations

import argparse
import concurrent.futures
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB_NAME = "libkvhot.so"
LIB_PATH = os.path.join(HERE, LIB_NAME)
BUILD_DIR = os.path.join(HERE, "_build")
SOURCES = ["kvhot_cache.hip", "kvhot_attention.hip"]
ARCH = "gfx950"


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    path = os.path.join(rocm, "bin", "hipcc")
    if not os.path.exists(path):
        path = shutil.which("hipcc") or path
    return path


def common_flags(defines: list[str]) -> list[str]:
    flags = [
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        # Packed FP32 (v_pk_*_f32) stays off: plain fp32 math only.
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        # MFMA accumulators in arch VGPRs: the prefill kernel rescales its
        # output accumulators with VALU ops, which cannot read AGPRs.  (The
        # decode and merge kernels compile to the same code either way.)
        "-mllvm", "-amdgpu-mfma-vgpr-form=1",
        "-Wall",
        "-Wno-unused-command-line-argument",
    ]
    flags += [f"-D{d}" for d in defines]
    return flags


def _compile(src: str, obj: str, defines: list[str]) -> tuple[str, int, str]:
    cmd = [hipcc(), *common_flags(defines), "-c", os.path.join(CSRC, src), "-o", obj]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(
        line for line in (proc.stdout + proc.stderr).splitlines()
        if "packed-fp32-ops" not in line  # host pass does not know the feature
    )
    return src, proc.returncode, out


def build(jobs: int | None = None, defines: list[str] | None = None, verbose: bool = False) -> str:
    defines = list(defines or [])
    os.makedirs(BUILD_DIR, exist_ok=True)
    objs = [os.path.join(BUILD_DIR, os.path.splitext(s)[0] + ".o") for s in SOURCES]
    jobs = jobs or min(len(SOURCES), os.cpu_count() or 1)
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as ex:
        results = list(ex.map(lambda so: _compile(so[0], so[1], defines), zip(SOURCES, objs)))
    failed = [(s, out) for s, rc, out in results if rc != 0]
    if verbose:
        for s, rc, out in results:
            if out.strip():
                print(f"--- {s}\n{out}", file=sys.stderr)
    if failed:
        msg = "\n".join(f"--- {s}\n{out}" for s, out in failed)
        raise RuntimeError(f"hipcc failed:\n{msg}")
    tmp = LIB_PATH + ".tmp"
    cmd = [hipcc(), *common_flags(defines), "-shared", *objs, "-o", tmp]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("--define", action="append", default=[])
    ap.add_argument("-v", "--verbose", action="store_true")
    args = ap.parse_args()
    print(build(args.jobs, args.define, args.verbose))


if __name__ == "__main__":
    main()
