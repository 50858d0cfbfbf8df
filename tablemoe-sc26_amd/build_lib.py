"""Build libtablemoe_hip.so (gfx950) from csrc/*.hip.

    python tablemoe-sc26_amd/build_lib.py [--jobs N]

Each source is compiled with hipcc for gfx950 in parallel, then the objects are
linked into one shared library that sits in-tree at
``table_moe/_lib/libtablemoe_hip.so``.

The library links the HIP runtime that PyTorch-ROCm ships (torch/lib/
libamdhip64.so, torch's lib/ as the run path).  Its SONAME is libamdhip64.so.7,
which becomes our NEEDED entry; in a process that already loaded torch the
loader matches it to that SAME runtime instance by SONAME, so streams and device
pointers from torch are valid in our kernels.  Loaded before torch, the name
would be looked up as a file (torch's lib/ has no libamdhip64.so.7) and could
resolve to /opt/rocm's copy, a second HIP runtime: import torch first.
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


# Kernels that issue loads from inline asm into registers (the compiler does
# not know those loads are in flight until the explicit s_waitcnt that
# retires them): their results are right only while the register allocator
# never spills, copies or reuses those registers before the wait.  The build
# fails if such a kernel uses scratch, spills VGPRs, or needs more VGPRs than
# the budget its launch bounds give (256 at two waves per SIMD), and if the
# dataflow check of its gfx950 assembly (isa_check.py) finds an instruction
# that reads or overwrites a register an outstanding load may still write.
# The pattern was first validated with the compiler VALIDATED_CLANG names;
# another compiler draws a warning (both checks still run).
ASM_LOAD_KERNELS = {"tm_project.hip": (("project_cols_pipe_kernel", 256),)}
VALIDATED_CLANG = "roc-7.2.0 26014"


def _check_asm_load_kernels(src: Path, remarks: str) -> None:
    import re

    budget = dict(ASM_LOAD_KERNELS[src.name])
    seen = 0
    for block in re.split(r"remark: Function Name: ", remarks)[1:]:
        name = block.split()[0]
        limit = next((v for k, v in budget.items() if k in name), None)
        if limit is None:
            continue
        seen += 1
        def field(label):
            m = re.search(re.escape(label) + r":\s*(\d+)", block)
            if m is None:
                raise RuntimeError(f"{src.name}: no '{label}' remark for {name}")
            return int(m.group(1))
        # SGPR spills go to lanes of compiler-allocated VGPRs (no scratch), and
        # the dataflow check sees every VGPR they write
        bad = {k: field(k) for k in ("ScratchSize [bytes/lane]", "VGPRs Spill") if field(k)}
        if field("VGPRs") > limit:
            bad["VGPRs"] = field("VGPRs")
        if bad:
            raise RuntimeError(f"{src.name}: {name} issues loads from inline asm and must not spill or exceed "
                               f"{limit} VGPRs: {bad}")
    if seen == 0:
        raise RuntimeError(f"{src.name}: no resource remarks for {sorted(budget)}")


def _device_asm(src: Path) -> Path:
    """gfx950 assembly of a source (for the dataflow check), in the build folder."""
    out = BUILD_DIR / (src.stem + ".s")
    cmd = [str(HIPCC), *HIP_FLAGS, "--cuda-device-only", "-S", str(src), "-o", str(out)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc -S failed for {src.name}:\n{res.stderr}")
    return out


def _check_asm_dataflow(src: Path, asm_path: Path) -> None:
    import isa_check

    asm = asm_path.read_text()
    for kernel, _ in ASM_LOAD_KERNELS[src.name]:
        names = isa_check.functions_named(asm, kernel)
        if not names:
            raise RuntimeError(f"{src.name}: no function named *{kernel}* in the device assembly")
        for name in names:
            issues = isa_check.check_function(asm, name)
            if issues:
                shown = "\n".join(f"  line {k}: {kind}: {line}" for k, kind, line in issues[:8])
                raise RuntimeError(f"{src.name}: {name} reads or overwrites registers of an in-flight load:\n{shown}")


def torch_lib_dir() -> Path:
    import importlib.util

    spec = importlib.util.find_spec("torch")
    if spec is None or spec.origin is None:
        raise RuntimeError("torch is required to locate the HIP runtime it ships")
    return Path(spec.origin).resolve().parent / "lib"


def _compile(src: Path) -> Path:
    obj = BUILD_DIR / (src.stem + ".o")
    checked = src.name in ASM_LOAD_KERNELS
    extra = ["-Rpass-analysis=kernel-resource-usage"] if checked else []
    cmd = [str(HIPCC), *HIP_FLAGS, *extra, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    lines = [l for l in (res.stderr or "").splitlines() if noise not in l]
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n" + "\n".join(lines))
    if checked:
        _check_asm_load_kernels(src, "\n".join(lines))
        # keep only diagnostics that are not the resource remarks
        lines = [l for l in lines if "kernel-resource-usage" not in l and not l.lstrip().startswith(("|", "^"))
                 and not l.strip().split("|")[0].strip().isdigit()]
    err = "\n".join(lines)
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
    ver = subprocess.run([str(CLANGXX), "--version"], capture_output=True, text=True).stdout
    if VALIDATED_CLANG not in ver:
        print(f"[build_lib] warning: the inline-asm load kernels were validated with {VALIDATED_CLANG}, this "
              f"compiler is: {ver.splitlines()[0] if ver else '?'}", file=sys.stderr)
    stale = [s for s in sources if not (incremental and _up_to_date(s))]
    checked = [s for s in stale if s.name in ASM_LOAD_KERNELS]
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        asm_jobs = {s: ex.submit(_device_asm, s) for s in checked}
        list(ex.map(_compile, stale))
        for src, job in asm_jobs.items():
            _check_asm_dataflow(src, job.result())
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
