"""Build the leankv_amd HIP library (gfx950) in-tree.

    python -m leankv_amd.build            # -> leankv_amd/libleankv_amd.so

Each ``csrc/*.hip`` file is compiled by ``hipcc --offload-arch=gfx950`` to an
object (in parallel) and the objects are linked into one shared library that
exports the C ABI declared in ``include/leankv_amd.h``.  No torch headers are
involved: the library is plain HIP C++ behind ``extern "C"`` entry points.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
import tempfile

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG_DIR, "csrc")
LIB_NAME = "libleankv_amd.so"
LIB_PATH = os.path.join(PKG_DIR, LIB_NAME)
ARCH = os.environ.get("LKV_OFFLOAD_ARCH", "gfx950")

# -packed-fp32-ops: hipcc must not emit packed fp32 VALU ops for this pool.
HIPCC_FLAGS = [
    "--offload-arch=" + ARCH,
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found; the leankv_amd HIP library cannot be built")


def sources() -> list[str]:
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


STAMPS_LIB_PATH = os.path.join(PKG_DIR, "libleankv_amd_stamps.so")


def build(verbose: bool = False, stamps: bool = False) -> str:
    """Compile every HIP source and link ``libleankv_amd.so``; returns its path.

    stamps=True builds ``libleankv_amd_stamps.so`` instead: the same sources with LKV_STAMPS defined, so the
    attention kernels record per-block phase times (the 100 MHz real-time clock) that
    ``lkv_debug_stamps`` copies out (bench.py --phases reads them); the product library never has them."""
    hipcc = _hipcc()
    srcs = sources()
    flags = HIPCC_FLAGS + (["-DLKV_STAMPS"] if stamps else [])
    lib_path = STAMPS_LIB_PATH if stamps else LIB_PATH
    tmp = tempfile.mkdtemp(prefix="lkv_build_")
    try:
        def compile_one(src: str) -> str:
            obj = os.path.join(tmp, os.path.basename(src) + ".o")
            cmd = [hipcc, *flags, "-c", src, "-o", obj]
            res = subprocess.run(cmd, capture_output=True, text=True)
            if res.returncode != 0:
                raise RuntimeError("hipcc failed on %s:\n%s%s" % (src, res.stdout, res.stderr))
            if verbose and res.stderr.strip():
                sys.stderr.write(res.stderr)
            return obj

        with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
            objs = list(ex.map(compile_one, srcs))
        out_tmp = lib_path + ".tmp"
        cmd = [hipcc, "--offload-arch=" + ARCH, "-shared", "-fPIC", *objs, "-o", out_tmp]
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError("link failed:\n%s%s" % (res.stdout, res.stderr))
        os.replace(out_tmp, lib_path)
    finally:
        shutil.rmtree(tmp, ignore_errors=True)
    return lib_path


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv, stamps="--stamps" in sys.argv))
