"""In-tree build of ``liblemoq_hip.so`` for gfx950 with hipcc.

``python -m lemoq.build`` (with ``leanmoe-quant_amd`` on ``sys.path``) or
``build_library()`` compiles every ``csrc/*.hip`` into one shared library next
to the package (``lemoq/_lib``), which is what the ctypes loader opens.  It
always recompiles; the result is written atomically.
"""

from __future__ import annotations

import glob
import os
import subprocess
import sys

from lemoq._hip import LIB_DIR, LIB_PATH

PKG_ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))  # leanmoe-quant_amd/
REPO_ROOT = os.path.dirname(PKG_ROOT)
CSRC = os.path.join(PKG_ROOT, "csrc")
INCLUDE = os.path.join(REPO_ROOT, "include")

OFFLOAD_ARCH = "gfx950"

HIPCC_FLAGS = [
    "--offload-arch=" + OFFLOAD_ARCH,
    "-O3",
    "-std=c++17",
    "-shared",
    "-fPIC",
    "-mcode-object-version=5",
    # Never emit packed-FP32 VALU ops (v_pk_{add,mul,fma}_f32).
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    return "hipcc"


def sources() -> list[str]:
    return sorted(glob.glob(os.path.join(CSRC, "*.hip")))


_NOISE = "is not a recognized feature for this target"


def _run(cmd: list[str]) -> str:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(line for line in proc.stderr.splitlines() if _NOISE not in line)
    if proc.returncode != 0:
        raise RuntimeError("hipcc failed (%d):\n%s\n%s" % (proc.returncode, " ".join(cmd), err))
    return err


def build_library(verbose: bool = False, jobs: int | None = None) -> str:
    """Compile csrc/*.hip -> lemoq/_lib/liblemoq_hip.so; returns the path.

    Each source compiles to an object in a scratch directory (in parallel, one
    hipcc per source), then one hipcc links the shared library."""
    import concurrent.futures
    import shutil
    import tempfile

    os.makedirs(LIB_DIR, exist_ok=True)
    tmp = LIB_PATH + ".tmp%d" % os.getpid()
    work = tempfile.mkdtemp(prefix="lemoq_build_")
    compile_flags = [f for f in HIPCC_FLAGS if f != "-shared"]
    try:
        srcs = sources()
        objs = [os.path.join(work, os.path.basename(src) + ".o") for src in srcs]
        cmds = [[hipcc(), *compile_flags, "-c", "-I" + INCLUDE, "-I" + CSRC, src, "-o", obj]
                for src, obj in zip(srcs, objs)]
        n = jobs or min(len(cmds), max(1, os.cpu_count() or 1))
        with concurrent.futures.ThreadPoolExecutor(max_workers=n) as pool:
            errs = list(pool.map(_run, cmds))
        errs.append(_run([hipcc(), "--offload-arch=" + OFFLOAD_ARCH, "-shared", "-fPIC", *objs, "-o", tmp]))
        if verbose:
            text = "\n".join(e for e in errs if e.strip())
            if text:
                sys.stderr.write(text + "\n")
        os.replace(tmp, LIB_PATH)
    finally:
        shutil.rmtree(work, ignore_errors=True)
        if os.path.exists(tmp):
            os.remove(tmp)
    return LIB_PATH


if __name__ == "__main__":
    print(build_library(verbose=True))
