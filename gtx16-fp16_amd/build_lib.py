"""Build libg16.so (the gfx950 kernels behind gtx16_fp16) in-tree with hipcc.

    python gtx16-fp16_amd/build_lib.py [--jobs N] [--verbose]

Compiles every ``csrc/*.hip`` for gfx950 only and links ``gtx16_fp16/_lib/libg16.so``; then builds
``csrc/fastcall.c`` (host C, with gcc) into the CPython extension ``gtx16_fp16/_lib/_g16fast``. The library
lists ``libamdhip64.so.7`` as a dependency by SONAME; torch-ROCm ships a runtime with the same
SONAME, so when ``torch`` is imported first (as ``gtx16_fp16`` does) the library binds to the
runtime torch already loaded and shares its device context and streams.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
import sysconfig
from pathlib import Path

HERE = Path(__file__).resolve().parent
REPO = HERE.parent
CSRC = HERE / "csrc"
INCLUDE = REPO / "include"
OUT_DIR = HERE / "gtx16_fp16" / "_lib"
LIB = OUT_DIR / "libg16.so"
ARCH = "gfx950"

# Packed fp32 VALU ops are disabled for all device code; the host pass warns that it does not know
# the feature, which is harmless.
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-mcode-object-version=5",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: set HIPCC or install ROCm")


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in proc.stdout.splitlines() if "packed-fp32-ops" not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    if verbose and out.strip():
        print(out, flush=True)


def build(jobs: int | None = None, verbose: bool = False) -> Path:
    """Compile all sources and link the shared library; returns its path."""
    cc = hipcc()
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    obj_dir = HERE / "_build"
    obj_dir.mkdir(exist_ok=True)
    OUT_DIR.mkdir(parents=True, exist_ok=True)
    objs = [obj_dir / (s.stem + ".o") for s in sources]
    cmds = [[cc, *HIP_FLAGS, f"-I{INCLUDE}", f"-I{CSRC}", "-c", str(s), "-o", str(o)] for s, o in zip(sources, objs)]
    with cf.ThreadPoolExecutor(max_workers=jobs or min(8, len(cmds))) as ex:
        list(ex.map(lambda c: _run(c, verbose), cmds))
    tmp = LIB.with_suffix(".so.tmp")
    _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)], verbose)
    os.replace(tmp, LIB)
    build_fastcall(verbose)
    return LIB


def build_fastcall(verbose: bool = False) -> Path:
    """Compile the CPython extension _g16fast (host C only, no device code) next to libg16.so."""
    out = OUT_DIR / ("_g16fast" + sysconfig.get_config_var("EXT_SUFFIX"))
    tmp = out.with_name(out.name + ".tmp")
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        raise RuntimeError("no C compiler (gcc) for the _g16fast extension")
    _run([cc, "-O2", "-fPIC", "-shared", "-Wall", "-Wextra", "-Wno-cast-function-type",
          f"-I{sysconfig.get_paths()['include']}", str(CSRC / "fastcall.c"), "-o", str(tmp)], verbose)
    os.replace(tmp, out)
    return out


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("--verbose", action="store_true")
    args = ap.parse_args(argv)
    path = build(args.jobs, args.verbose)
    print(path)
    return 0


if __name__ == "__main__":
    sys.exit(main())
