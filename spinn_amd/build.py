"""Build the native library and CLI in-tree.

    python -m spinn_amd.build          # incremental
    python -m spinn_amd.build --force  # rebuild everything

Outputs (git-ignored, shipped with the tree):
    spinn_amd/lib/libspinn.so   HIP kernels for gfx950 + the C host runtime
    spinn_amd/bin/spinn_run     CLI driver linked against it

HIP sources are compiled by hipcc for gfx950 only; the host runtime is plain
C11 compiled by gcc and linked into the same shared object.
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
HOST = CSRC / "host"
BUILD = PKG / "_build"
LIB = PKG / "lib" / "libspinn.so"
CLI = PKG / "bin" / "spinn_run"
INCLUDE = ROOT / "include"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
CC = os.environ.get("CC", "gcc")
ARCH = "gfx950"

HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    # packed-fp32 instructions stay off: the compiler may not form them
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}",
]
C_FLAGS = ["-O2", "-fPIC", "-std=gnu11", "-Wall", "-Wextra", "-Wno-unused-parameter", f"-I{INCLUDE}"]


def _run(cmd: list[str]) -> None:
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        print(out, file=sys.stderr)


def _stale(obj: Path, deps: list[Path]) -> bool:
    if not obj.exists():
        return True
    t = obj.stat().st_mtime
    return any(d.stat().st_mtime > t for d in deps)


def _headers() -> list[Path]:
    return sorted(CSRC.glob("*.h")) + sorted(HOST.glob("*.h")) + sorted(INCLUDE.glob("*.h"))


def build(force: bool = False, jobs: int | None = None, verbose: bool = False) -> Path:
    if shutil.which(HIPCC) is None and not Path(HIPCC).exists():
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    BUILD.mkdir(parents=True, exist_ok=True)
    LIB.parent.mkdir(parents=True, exist_ok=True)
    CLI.parent.mkdir(parents=True, exist_ok=True)
    hdrs = _headers()
    jobs_list = []
    objs = []
    for src in sorted(CSRC.glob("*.hip")):
        obj = BUILD / (src.stem + ".hip.o")
        objs.append(obj)
        if force or _stale(obj, [src] + hdrs):
            jobs_list.append([HIPCC, *HIP_FLAGS, "-c", str(src), "-o", str(obj)])
    for src in sorted(HOST.glob("*.c")):
        if src.name == "main.c":
            continue
        obj = BUILD / (src.stem + ".c.o")
        objs.append(obj)
        if force or _stale(obj, [src] + hdrs):
            jobs_list.append([CC, *C_FLAGS, "-c", str(src), "-o", str(obj)])
    n = jobs or min(8, os.cpu_count() or 4)
    with cf.ThreadPoolExecutor(max_workers=n) as ex:
        futs = [ex.submit(_run, c) for c in jobs_list]
        for f in futs:
            f.result()
    if force or jobs_list or _stale(LIB, objs):
        tmp = LIB.with_suffix(".so.tmp")
        _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)])
        os.replace(tmp, LIB)
    main_c = HOST / "main.c"
    if force or _stale(CLI, [main_c, LIB] + hdrs):
        _run([CC, *C_FLAGS, str(main_c), "-o", str(CLI), f"-L{LIB.parent}", "-lspinn",
              "-Wl,-rpath,$ORIGIN/../lib"])
    if verbose:
        print(f"built {LIB} and {CLI}")
    return LIB


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--force", action="store_true")
    ap.add_argument("-j", "--jobs", type=int, default=None)
    a = ap.parse_args()
    build(force=a.force, jobs=a.jobs, verbose=True)


if __name__ == "__main__":
    main()
