"""Build the gfx950 HIP library ``mstar_amd/libmstar_amd.so`` in-tree.

Every ``csrc/*.hip`` file is compiled with hipcc for gfx950 only (one process
per file, in parallel) and linked into one shared library whose C ABI is
declared in ``include/mstar_amd.h``.  The library links the HIP runtime by
its soname (``libamdhip64.so.7``); when loaded after ``import torch`` the
dynamic linker reuses torch's already-loaded runtime, so torch tensors and
our kernels share one HIP context.

Usage: ``python -m mstar_amd.build`` (or ``__graft_entry__.build()``).
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
REPO_DIR = PKG_DIR.parent
CSRC = PKG_DIR / "csrc"
INCLUDE = REPO_DIR / "include"
BUILD_DIR = PKG_DIR / "_build"
LIB_NAME = "libmstar_amd.so"
LIB_PATH = PKG_DIR / LIB_NAME

ARCH = "gfx950"

# -packed-fp32-ops: keep the compiler from forming v_pk_{add,mul,fma}_f32;
# every kernel here is written for plain fp32 VALU ops plus MFMA.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-mcode-object-version=5",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


# Per-source additions.  mi_prefill_d128.hip holds the head_dim 128 prefill
# kernels, which run faster under the backend's max-ILP scheduler (see that file).
EXTRA_FLAGS = {
    "mi_prefill_d128.hip": ["-mllvm", "-amdgpu-sched-strategy=max-ilp"],
}


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the MI355X kernels need ROCm's hipcc to build")


def _compile(src: Path, hipcc: str) -> Path:
    obj = BUILD_DIR / (src.stem + ".o")
    cmd = [hipcc, *HIPCC_FLAGS, *EXTRA_FLAGS.get(src.name, []), f"-I{INCLUDE}", f"-I{CSRC}", "-c", str(src),
           "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stdout}\n{res.stderr}")
    return obj


# The host_step extension is built twice: the module the package imports,
# and a test build forced onto the generic attribute protocol (the branch
# CPython 3.11+ compiles), which tests/test_host_step.py runs beside it.
HOST_VARIANTS = {
    "_host_step": [],
    "_host_step_generic": ["-DMI_DIRECT_DICT=0", "-DMI_HOST_STEP_MODULE=_host_step_generic"],
}


def build_host(verbose: bool = True) -> Path:
    """Compile ``csrc/host_step.c`` (the planning step's host bookkeeping) into
    the CPython extension ``mstar_amd/_host_step`` (and its generic-attribute
    test build ``_host_step_generic``)."""
    import sysconfig

    cc = os.environ.get("CC") or shutil.which("gcc") or shutil.which("cc")
    if not cc:
        raise RuntimeError("no C compiler for the host_step extension")
    main = None
    for name, defs in HOST_VARIANTS.items():
        out = PKG_DIR / (name + sysconfig.get_config_var("EXT_SUFFIX"))
        tmp = out.with_suffix(".tmp")
        cmd = [cc, "-O2", "-shared", "-fPIC", "-Wall", *defs, f"-I{sysconfig.get_paths()['include']}",
               str(CSRC / "host_step.c"), "-o", str(tmp)]
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"host_step build ({name}) failed:\n{res.stdout}\n{res.stderr}")
        os.replace(tmp, out)
        if verbose:
            print(f"built {out}", file=sys.stderr)
        main = main or out
    return main


def build(verbose: bool = True) -> Path:
    """Compile all HIP sources for gfx950 and link ``libmstar_amd.so``; build
    the host_step extension (optional: without it the package runs the same
    host loops in Python, so a failure there is reported and the HIP build
    goes on)."""
    try:
        build_host(verbose)
    except RuntimeError as e:
        print(f"warning: {e}\n(the allocation manager falls back to its Python loops)", file=sys.stderr)
    hipcc = _hipcc()
    BUILD_DIR.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    jobs = min(len(sources), int(os.environ.get("MAX_JOBS", "8")))
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, hipcc), sources))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH} from {len(sources)} sources", file=sys.stderr)
    return LIB_PATH


if __name__ == "__main__":
    build()
