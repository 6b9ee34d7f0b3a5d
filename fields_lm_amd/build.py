"""Build recipe for the gfx950 shared library ``libfields_amd.so``.

The library is compiled in-tree with ``hipcc --offload-arch=gfx950`` and loaded with ctypes
(:mod:`fields_lm_amd._native`). It links against the HIP runtime by SONAME
(``libamdhip64.so.7``), so when PyTorch-ROCm is imported first the process keeps a single HIP
runtime: PyTorch's.

Run ``python -m fields_lm_amd.build`` or call :func:`build`.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
REPO_DIR = PKG_DIR.parent
SOURCES = [PKG_DIR / "csrc" / "field_scan.hip"]
INCLUDE_DIR = REPO_DIR / "include"
LIB_PATH = PKG_DIR / "libfields_amd.so"
# measurement kernels for bench.py (the scan's access pattern without its arithmetic), kept out of
# the library behind the C ABI
BENCH_SOURCES = [PKG_DIR / "csrc" / "copy_ceiling.hip"]
BENCH_LIB_PATH = PKG_DIR / "libfields_bench.so"
ARCH = "gfx950"

# -packed-fp32-ops: keep v_pk_{add,mul,fma}_f32 out of the generated code (the compiler would
# otherwise form them from float2-shaped arithmetic).
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-ffp-contract=fast",
    "-Wall",
    "-Wno-unused-function",
]


def hipcc() -> str:
    found = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(found).exists():
        raise RuntimeError("hipcc not found; the ROCm toolchain is required to build libfields_amd.so")
    return found


def build(verbose: bool = False, extra_flags: list[str] | None = None, out: Path | None = None,
          sources: list[Path] | None = None) -> Path:
    """Compile the HIP sources into ``libfields_amd.so`` (always recompiles)."""
    target = Path(out) if out is not None else LIB_PATH
    tmp = target.with_suffix(".so.tmp")
    cmd = [hipcc(), *HIP_FLAGS, *(extra_flags or []), f"-I{INCLUDE_DIR}",
           *[str(s) for s in (sources or SOURCES)], "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    env = dict(os.environ)
    proc = subprocess.run(cmd, capture_output=True, text=True, env=env)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{proc.stdout}\n{proc.stderr}")
    if verbose and proc.stderr.strip():
        print(proc.stderr, file=sys.stderr)
    missing = unresolved_kernel_stubs(tmp)
    if missing:
        tmp.unlink()
        raise RuntimeError(f"{target.name}: hipcc left {len(missing)} kernel launch stub(s) undefined, "
                           f"so the library would not load: {missing[0]}")
    os.replace(tmp, target)
    return target


def unresolved_kernel_stubs(lib: Path) -> list[str]:
    """Undefined host-side kernel launch stubs of a built library (``nm -D --undefined-only``).
    hipcc can link a library whose launches refer to stubs it never emitted; dlopen then fails.
    Empty when nm is absent."""
    nm = shutil.which("nm")
    if nm is None:
        return []
    proc = subprocess.run([nm, "-D", "--undefined-only", str(lib)], capture_output=True, text=True)
    return [ln.split()[-1] for ln in proc.stdout.splitlines() if "__device_stub__" in ln]


def build_bench(verbose: bool = False) -> Path:
    """Compile the measurement kernels of bench.py into ``libfields_bench.so``."""
    return build(verbose=verbose, out=BENCH_LIB_PATH, sources=BENCH_SOURCES)


if __name__ == "__main__":
    print(build(verbose=True))
    print(build_bench(verbose=True))
