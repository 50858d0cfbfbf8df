"""Build libtablemoe_hip.so (gfx950) from csrc/*.hip.

    python tablemoe-sc26_amd/build_lib.py [--jobs N]

Each source is compiled with hipcc for gfx950 in parallel, then the objects are
linked into one shared library that sits in-tree at
``table_moe/_lib/libtablemoe_hip.so``.

The library links the HIP runtime that PyTorch-ROCm ships (torch/lib/
libamdhip64.so, recorded as NEEDED "libamdhip64.so").  That copy has no SONAME,
so a process that already loaded torch resolves our dependency to the SAME
runtime instance: streams and device pointers from torch are valid in our
kernels.  Linking /opt/rocm's libamdhip64.so.7 instead would load a second HIP
runtime into the process.
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
REPO = PKG_DIR.parent
CSRC = PKG_DIR / "csrc"
INCLUDE = REPO / "include"
BUILD_DIR = PKG_DIR / "_build"
LIB_DIR = PKG_DIR / "table_moe" / "_lib"
LIB_NAME = "libtablemoe_hip.so"
ARCH = "gfx950"

ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
HIPCC = ROCM / "bin" / "hipcc"
CLANGXX = ROCM / "llvm" / "bin" / "clang++"

HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    # packed fp32 VALU forms are kept out of the generated code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]


def torch_lib_dir() -> Path:
    import importlib.util

    spec = importlib.util.find_spec("torch")
    if spec is None or spec.origin is None:
        raise RuntimeError("torch is required to locate the HIP runtime it ships")
    return Path(spec.origin).resolve().parent / "lib"


def _compile(src: Path) -> Path:
    obj = BUILD_DIR / (src.stem + ".o")
    cmd = [str(HIPCC), *HIP_FLAGS, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in (res.stderr or "").splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{err}")
    if err.strip():
        print(err, file=sys.stderr)
    return obj


def _up_to_date(src: Path) -> bool:
    """True when src's object is newer than src and every header it may include."""
    obj = BUILD_DIR / (src.stem + ".o")
    if not obj.exists():
        return False
    deps = [src, *CSRC.glob("*.h"), *INCLUDE.glob("*.h")]
    return obj.stat().st_mtime > max(d.stat().st_mtime for d in deps)


def build(jobs: int | None = None, verbose: bool = True, incremental: bool = False) -> Path:
    if not HIPCC.exists():
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    LIB_DIR.mkdir(parents=True, exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no sources under {CSRC}")
    jobs = jobs or min(len(sources), max(1, os.cpu_count() or 1), 8)
    if verbose:
        print(f"[build_lib] compiling {len(sources)} sources for {ARCH} with {jobs} jobs", flush=True)
    stale = [s for s in sources if not (incremental and _up_to_date(s))]
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(_compile, stale))
    objs = [BUILD_DIR / (s.stem + ".o") for s in sources]
    tlib = torch_lib_dir()
    if not (tlib / "libamdhip64.so").exists():
        raise RuntimeError(f"torch's HIP runtime not found in {tlib}")
    tmp = LIB_DIR / (LIB_NAME + ".tmp")
    cmd = [
        str(CLANGXX), "-shared", "-fPIC", "-o", str(tmp), *map(str, objs),
        f"-L{tlib}", "-l:libamdhip64.so", f"-Wl,-rpath,{tlib}", "-Wl,--no-undefined",
        "-lstdc++",
    ]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    out = LIB_DIR / LIB_NAME
    shutil.move(str(tmp), str(out))
    if verbose:
        print(f"[build_lib] wrote {out.relative_to(REPO)}", flush=True)
    return out


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("--incremental", action="store_true",
                    help="recompile only sources whose object is older than the source or a header")
    args = ap.parse_args()
    build(args.jobs, incremental=args.incremental)
    return 0


if __name__ == "__main__":
    sys.exit(main())
