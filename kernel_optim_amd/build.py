"""Build recipe for libkoptim.so: every HIP source under csrc/ compiled for gfx950.

The library is built in-tree (next to this file) so it travels with the
source tree; nothing is installed. ``build()`` always recompiles.
"""

import os
import shutil
import subprocess
import tempfile
from concurrent.futures import ThreadPoolExecutor

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG_DIR, "csrc")
LIB_NAME = "libkoptim.so"
LIB_PATH = os.path.join(PKG_DIR, LIB_NAME)
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # Packed fp32 VALU ops are kept out of every kernel.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def hipcc():
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found; the HIP extension cannot be built")


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{proc.stderr[-8000:]}")


def build(verbose=False):
    """Compile csrc/*.hip into kernel_optim_amd/libkoptim.so (atomic replace): each
    source to an object in parallel, then one shared-library link."""
    srcs = sources()
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    cc = hipcc()
    fd, tmp = tempfile.mkstemp(prefix=".libkoptim.", suffix=".so.tmp", dir=PKG_DIR)
    os.close(fd)
    objdir = tempfile.mkdtemp(prefix=".koobj.", dir=PKG_DIR)
    try:
        objs = [os.path.join(objdir, os.path.basename(src) + ".o") for src in srcs]
        jobs = [[cc, *HIPCC_FLAGS, f"-I{CSRC}", "-c", src, "-o", obj]
                for src, obj in zip(srcs, objs)]
        with ThreadPoolExecutor(max_workers=min(len(jobs), os.cpu_count() or 1, 8)) as ex:
            for f in [ex.submit(_run, cmd, verbose) for cmd in jobs]:
                f.result()
        _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp], verbose)
        os.replace(tmp, LIB_PATH)
    finally:
        if os.path.exists(tmp):
            os.unlink(tmp)
        shutil.rmtree(objdir, ignore_errors=True)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
