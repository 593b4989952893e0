"""Build libjanus_hip.so (gfx950) and the CPU oracle in-tree.

The library is compiled with hipcc for gfx950 only, one object per source
file in parallel, then linked as a shared object next to this package so the
GPU box loads it straight from the repository tree.

Usage: python -m janus_amd.build [--jobs N] [--no-oracle] [--incremental]
       python -m janus_amd.build --sanitize   (host code under AddressSanitizer and
       UndefinedBehaviorSanitizer, device code as usual, into
       _build_san/libjanus_hip_san.so for the CPU test run of tests/run_sanitizers.sh)
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libjanus_hip.so"
BUILD_SAN = PKG / "_build_san"
LIB_SAN = BUILD_SAN / "libjanus_hip_san.so"
# host-only sanitizers: each flag goes to the host compilation alone
SAN_FLAGS = [f for kind in ("address", "undefined") for f in ("-Xarch_host", f"-fsanitize={kind}")] + [
    "-Xarch_host", "-fno-omit-frame-pointer", "-Xarch_host", "-g"]
ORACLE_DIR = ROOT / "oracle"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-result",
    "-munsafe-fp-atomics",
    # Packed FP32 instructions stay off: some of their forms have given wrong
    # results on this hardware, without an error.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def _compile(src: Path, out_dir: Path = BUILD, extra: tuple = ()) -> Path:
    obj = out_dir / (src.stem + ".o")
    cmd = [HIPCC, *HIP_FLAGS, *extra, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stdout}\n{res.stderr}")
    return obj


def _stale(src: Path) -> bool:
    """An object is stale when it is missing or older than its source or any
    shared header."""
    obj = BUILD / (src.stem + ".o")
    if not obj.exists():
        return True
    deps = [src, *CSRC.glob("*.h"), *(ROOT / "include").glob("*.h")]
    return max(d.stat().st_mtime for d in deps) > obj.stat().st_mtime


def build_library(jobs: int | None = None, verbose: bool = True, incremental: bool = False) -> Path:
    """Compile every csrc/*.hip for gfx950 and link libjanus_hip.so
    (incremental: only sources whose object is stale)."""
    if shutil.which(HIPCC) is None and not Path(HIPCC).exists():
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    BUILD.mkdir(exist_ok=True)
    srcs = _sources()
    todo = [s for s in srcs if _stale(s)] if incremental else srcs
    jobs = jobs or min(8, max(1, len(todo)), os.cpu_count() or 1)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(_compile, todo))
    objs = [BUILD / (s.stem + ".o") for s in srcs]
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"[janus_amd.build] built {LIB.relative_to(ROOT)} from {len(srcs)} sources", flush=True)
    return LIB


def build_sanitized(jobs: int | None = None) -> Path:
    """The library with host code under ASan + UBSan (device code unchanged),
    for CPU runs of the host-side validation; never loaded by default."""
    BUILD_SAN.mkdir(exist_ok=True)
    srcs = _sources()
    with cf.ThreadPoolExecutor(max_workers=jobs or min(8, os.cpu_count() or 1)) as ex:
        objs = list(ex.map(lambda s: _compile(s, BUILD_SAN, tuple(SAN_FLAGS)), srcs))
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *SAN_FLAGS, "-o", str(LIB_SAN), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"sanitized link failed:\n{res.stdout}\n{res.stderr}")
    print(f"[janus_amd.build] built {LIB_SAN.relative_to(ROOT)} (host ASan + UBSan)", flush=True)
    return LIB_SAN


def build_oracle(verbose: bool = True) -> Path:
    """Compile the CPU oracle (test infrastructure) with its Makefile."""
    res = subprocess.run(["make", "-s", "-C", str(ORACLE_DIR), "-B", "liboracle.so"],
                         capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{res.stdout}\n{res.stderr}")
    if verbose:
        print("[janus_amd.build] built oracle/liboracle.so", flush=True)
    return ORACLE_DIR / "liboracle.so"


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("--no-oracle", action="store_true")
    ap.add_argument("--incremental", action="store_true", help="recompile only stale objects")
    ap.add_argument("--sanitize", action="store_true", help="build only the host-sanitised library")
    args = ap.parse_args(argv)
    if args.sanitize:
        build_sanitized(args.jobs)
        return 0
    build_library(args.jobs, incremental=args.incremental)
    if not args.no_oracle:
        build_oracle()
    return 0


if __name__ == "__main__":
    sys.exit(main())
