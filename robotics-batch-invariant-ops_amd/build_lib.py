"""Build libbiops.so (the gfx950 HIP kernels + C ABI) in-tree.

    python robotics-batch-invariant-ops_amd/build_lib.py [--jobs N]

Each csrc/*.hip file is compiled to an object with hipcc for gfx950, then linked into
batch_invariant_ops/libbiops.so next to the Python package that loads it.  csrc/pyfast.c, a
CPython fast-call binding of the most frequent entry points, is compiled with the host C
compiler into batch_invariant_ops/_biops_fast (linked against libbiops.so beside it).
"""

from __future__ import annotations

import argparse
import concurrent.futures
import os
import pathlib
import shutil
import subprocess
import sys

ROOT = pathlib.Path(__file__).resolve().parent
CSRC = ROOT / "csrc"
OUT = ROOT / "batch_invariant_ops" / "libbiops.so"
BUILD = ROOT / "_build"

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # packed fp32 instructions are kept out of every kernel
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found; ROCm is required to build libbiops.so")
    return path


def _compile(src: pathlib.Path) -> pathlib.Path:
    obj = BUILD / (src.stem + ".o")
    cmd = [hipcc(), *HIPCC_FLAGS, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{proc.stdout}\n{proc.stderr}")
    return obj


def _stale(src: pathlib.Path) -> bool:
    """The object of ``src`` is missing or older than ``src`` or any csrc / include header."""
    obj = BUILD / (src.stem + ".o")
    if not obj.exists():
        return True
    deps = [src, *CSRC.glob("*.h"), *(ROOT.parent / "include").glob("*.h")]
    return obj.stat().st_mtime < max(d.stat().st_mtime for d in deps)


def build(jobs: int | None = None, verbose: bool = True, incremental: bool = False) -> pathlib.Path:
    """Compile every source (``incremental``: only those whose object is stale) and link."""
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    todo = [s for s in sources if _stale(s)] if incremental else sources
    jobs = jobs or min(max(len(todo), 1), max(1, (os.cpu_count() or 2)))
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as pool:
        list(pool.map(_compile, todo))
    objects = [BUILD / (s.stem + ".o") for s in sources]
    tmp = OUT.with_suffix(".so.tmp")
    cmd = [hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC", *map(str, objects), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, OUT)
    _build_fast()
    if verbose:
        print(f"built {OUT} from {len(sources)} sources", file=sys.stderr)
    return OUT


def _build_fast() -> pathlib.Path:
    """The CPython fast-call module next to libbiops.so (rpath $ORIGIN)."""
    import sysconfig

    out = OUT.parent / ("_biops_fast" + sysconfig.get_config_var("EXT_SUFFIX"))
    tmp = out.with_suffix(".tmp")
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        raise RuntimeError("no host C compiler for the fast-call module")
    cmd = [cc, "-O2", "-shared", "-fPIC", f"-I{sysconfig.get_paths()['include']}", str(CSRC / "pyfast.c"),
           f"-L{OUT.parent}", "-l:libbiops.so", "-Wl,-rpath,$ORIGIN", "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"fast-call module build failed:\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    parser = argparse.ArgumentParser()
    parser.add_argument("--jobs", type=int, default=None)
    parser.add_argument("--incremental", action="store_true",
                        help="recompile only sources whose object is older than the source or a header")
    args = parser.parse_args()
    build(args.jobs, incremental=args.incremental)
