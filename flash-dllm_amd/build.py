"""Builds libfdl.so, the C-ABI library of the Flash-Cache hot path, for gfx950.

    python flash-dllm_amd/build.py            # compile every source, link libfdl.so
    python flash-dllm_amd/build.py --check    # also print per-kernel register/LDS usage

HIP sources are compiled with hipcc (--offload-arch=gfx950, packed-fp32 ops disabled);
the host-only source with g++. Objects go to flash-dllm_amd/_build/, the library to
flash-dllm_amd/libfdl.so (both git-ignored).
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
BUILD_DIR = PKG_DIR / "_build"
LIB_PATH = PKG_DIR / "libfdl.so"
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
ARCH = "gfx950"

HIP_SOURCES = ["fdl_qkv.hip", "fdl_attn.hip", "fdl_rank.hip", "fdl_block.hip", "fdl_head.hip",
               "fdl_sched.hip"]
CXX_SOURCES = ["fdl_host.cpp"]

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    # keep the compiler from forming packed fp32 ops (v_pk_*_f32)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]
# Per-source additions. The QKV kernels keep their MFMA accumulators in VGPRs: with the
# accumulators in AGPRs the register allocator shuffles them between loop iterations.
HIPCC_EXTRA = {"fdl_qkv.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}
CXX_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-Wall", "-Wextra"]


def _hipcc() -> str:
    p = ROCM / "bin" / "hipcc"
    return str(p) if p.exists() else (shutil.which("hipcc") or "hipcc")


def _run(cmd: list[str]) -> str:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature; drop that line
    out = "\n".join(l for l in proc.stdout.splitlines() if "packed-fp32-ops" not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    return out


def _compile(src: str, check: bool) -> tuple[Path, str]:
    obj = BUILD_DIR / (src + ".o")
    if src.endswith(".hip"):
        cmd = [_hipcc(), *HIPCC_FLAGS, *HIPCC_EXTRA.get(src, []), "-c", str(CSRC / src),
               "-o", str(obj)]
        if check:
            cmd.append("-Rpass-analysis=kernel-resource-usage")
    else:
        cmd = ["g++", *CXX_FLAGS, "-c", str(CSRC / src), "-o", str(obj)]
    return obj, _run(cmd)


def build(check: bool = False, verbose: bool = True) -> Path:
    """Compiles every source and links libfdl.so; returns the library path."""
    BUILD_DIR.mkdir(exist_ok=True)
    sources = HIP_SOURCES + CXX_SOURCES
    with cf.ThreadPoolExecutor(max_workers=min(8, len(sources))) as ex:
        results = list(ex.map(lambda s: _compile(s, check), sources))
    for (obj, out), src in zip(results, sources):
        if verbose and out.strip():
            print(f"[{src}]\n{out}")
    tmp = LIB_PATH.with_suffix(".so.tmp")
    _run([_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp),
          *[str(o) for o, _ in results], "-Wl,-soname,libfdl.so",
          f"-Wl,-rpath,{ROCM / 'lib'}"])
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH}")
    return LIB_PATH


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--check", action="store_true", help="print kernel resource usage")
    args = ap.parse_args()
    build(check=args.check)
    return 0


if __name__ == "__main__":
    sys.exit(main())
