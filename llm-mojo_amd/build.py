"""Builds libpkv.so (HIP, gfx950) in-tree, and the CPU oracle used by the tests.

    python llm-mojo_amd/build.py            # library + oracle
    python llm-mojo_amd/build.py --lib-only

Every build compiles from scratch (no incremental cache): the sources are small and
hipcc cross-compiles gfx950 without a GPU.
"""
from __future__ import annotations

import argparse
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(PKG_DIR)
CSRC = os.path.join(PKG_DIR, "csrc")
BUILD_DIR = os.path.join(PKG_DIR, "_build")
LIB_PATH = os.path.join(PKG_DIR, "libpkv.so")
# Workload data generator (benchmark / tests only, not part of the pkv ABI).
SYNTH_PATH = os.path.join(PKG_DIR, "libpkv_synth.so")
ORACLE_DIR = os.path.join(REPO, "oracle")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
# -packed-fp32-ops: no v_pk_* fp32 instructions are generated.
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{os.path.join(REPO, 'include')}",
]
SOURCES = ["pkv_common.cpp", "pkv_state.hip", "pkv_attend.hip", "pkv_stream.hip",
           "pkv_prefill.hip", "pkv_q4.hip", "pkv_lsa.hip", "pkv_noalloc.hip"]


def _run(cmd: list[str]) -> None:
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32-ops feature.
    err = "\n".join(l for l in res.stderr.splitlines() if "packed-fp32-ops" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"command failed ({res.returncode}): {' '.join(cmd)}\n{err}")


def build_lib(verbose: bool = False) -> str:
    if shutil.which(HIPCC) is None and not os.path.exists(HIPCC):
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    os.makedirs(BUILD_DIR, exist_ok=True)
    objs = []
    cmds = []
    for src in SOURCES:
        obj = os.path.join(BUILD_DIR, os.path.splitext(src)[0] + ".o")
        lang = ["-x", "hip"] if src.endswith(".hip") else []
        cmds.append([HIPCC, *HIP_FLAGS, *lang, "-c", os.path.join(CSRC, src), "-o", obj])
        objs.append(obj)
    with ThreadPoolExecutor(max_workers=len(cmds)) as ex:
        for cmd, fut in zip(cmds, [ex.submit(_run, c) for c in cmds]):
            if verbose:
                print(" ".join(cmd))
            fut.result()
    tmp = LIB_PATH + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs])
    os.replace(tmp, LIB_PATH)
    tmp = SYNTH_PATH + ".tmp"
    _run([HIPCC, *HIP_FLAGS, "-shared", "-o", tmp, os.path.join(CSRC, "pkv_synth.hip")])
    os.replace(tmp, SYNTH_PATH)
    return LIB_PATH


def build_oracle(verbose: bool = False) -> str:
    res = subprocess.run(["make", "-B", "-C", ORACLE_DIR], capture_output=True, text=True)
    if verbose:
        print(res.stdout)
    if res.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{res.stdout}\n{res.stderr}")
    return os.path.join(ORACLE_DIR, "libpkv_oracle.so")


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--lib-only", action="store_true")
    ap.add_argument("-v", "--verbose", action="store_true")
    args = ap.parse_args()
    print(build_lib(args.verbose))
    if not args.lib_only:
        print(build_oracle(args.verbose))
    return 0


if __name__ == "__main__":
    sys.exit(main())
