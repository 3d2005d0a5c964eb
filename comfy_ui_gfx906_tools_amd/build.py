"""Build libqlinear.so (the gfx950 HIP kernels + C ABI) in-tree with hipcc.

No torch extension machinery, no hipify: every source under csrc/ is HIP/C++ written for
gfx950 and compiled as such. The reference JIT-built a pybind11 extension for gfx906 through
torch.utils.cpp_extension.load (nodes/ComfyUI-Gfx906Int4/ops.py:17-34); this library has a
plain C ABI (include/qlinear.h) and is loaded with ctypes.

Usage: python -m comfy_ui_gfx906_tools_amd.build [--jobs N] [--verbose]
"""
from __future__ import annotations

import argparse
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG_DIR, "csrc")
BUILD_DIR = os.path.join(PKG_DIR, "_build")
LIB_NAME = "libqlinear.so"
LIB_PATH = os.path.join(PKG_DIR, LIB_NAME)
ARCH = "gfx950"

SOURCES = ["w4a16_gemm.hip", "w4a16_tile256.hip", "w4a16_gemv.hip", "w4a16_skinny.hip", "w8a8_gemm.hip", "w8a8_tile256.hip", "quant.hip", "dit_fused.hip", "w4a4_gemm.hip", "rotate.hip", "stream_read.hip", "capi.cpp"]

COMMON_FLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    f"--offload-arch={ARCH}",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-variable",
    # no implicit a*b+c -> fma: the epilogues round each step like the reference
    "-ffp-contract=off",
    # Keep the compiler from forming packed-fp32 (v_pk_*_f32) instructions.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def hipcc_path() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm under /opt/rocm)")


def _compile(hipcc: str, src: str, verbose: bool, csrc: str = CSRC, build_dir: str = BUILD_DIR,
             extra: tuple = ()) -> str:
    obj = os.path.join(build_dir, os.path.basename(src) + ".o")
    cmd = [hipcc, *COMMON_FLAGS, *extra, "-x", "hip", "-c", os.path.join(csrc, src), "-o", obj]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{res.stdout}\n{res.stderr}")
    # hipcc's host pass warns that it does not know the packed-fp32 feature: harmless
    noise = [ln for ln in res.stderr.splitlines() if ln.strip() and "packed-fp32-ops" not in ln
             and "not a recognized feature" not in ln]
    if verbose and noise:
        print("\n".join(noise), file=sys.stderr)
    return obj


def build(jobs: int | None = None, verbose: bool = False, csrc: str = CSRC, out: str = LIB_PATH,
          extra_flags: tuple = ()) -> str:
    """Compile every source for gfx950 and link libqlinear.so next to this file (or `out`, from
    the sources in `csrc`, with `extra_flags` added)."""
    hipcc = hipcc_path()
    build_dir = BUILD_DIR if out == LIB_PATH else out + ".build"
    os.makedirs(build_dir, exist_ok=True)
    jobs = jobs or min(len(SOURCES), os.cpu_count() or 1, 16)
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile(hipcc, s, verbose, csrc, build_dir, tuple(extra_flags)), SOURCES))
    tmp = out + ".tmp"
    cmd = [hipcc, "-shared", "-fPIC", f"--offload-arch={ARCH}", *objs, "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, out)
    return out


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("--verbose", action="store_true")
    ap.add_argument("--csrc", default=CSRC, help="source directory (default: the package's csrc/)")
    ap.add_argument("--out", default=LIB_PATH, help="output library path")
    ap.add_argument("-D", dest="defines", action="append", default=[], help="extra preprocessor define")
    args = ap.parse_args()
    print(build(args.jobs, args.verbose, args.csrc, args.out, tuple("-D" + d for d in args.defines)))


if __name__ == "__main__":
    main()
