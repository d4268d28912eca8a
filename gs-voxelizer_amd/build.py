"""Build libgsvox.so (gfx950) in-tree: ``python gs-voxelizer_amd/build.py``.

hipcc compiles every ``csrc/*.hip`` for ``--offload-arch=gfx950`` and links one
C-ABI shared library next to the Python package, where ``gs_voxelizer._lib``
loads it.  No torch headers are involved, so the library is independent of the
torch build's C++ ABI.
"""
import os
import shutil
import subprocess
import sys
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "gs_voxelizer", "libgsvox.so")
SOURCES = ["scan.hip", "project.hip", "binning.hip", "voxelize.hip"]

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    # keep the compiler from forming packed-FP32 VALU instructions
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]


def hipcc():
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found; the gfx950 library cannot be built")


def build(verbose=False):
    """Compile the library; returns its path. Always recompiles."""
    srcs = [os.path.join(CSRC, s) for s in SOURCES]
    fd, tmp = tempfile.mkstemp(suffix=".so", dir=os.path.dirname(OUT))
    os.close(fd)
    cmd = [hipcc()] + HIPCC_FLAGS + srcs + ["-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the device-only target feature; drop that noise
    noise = ("unknown target feature", "packed-fp32-ops")
    log = "\n".join(l for l in (res.stdout + res.stderr).splitlines()
                    if not any(k in l for k in noise))
    if res.returncode != 0:
        if os.path.exists(tmp):  # hipcc may already have removed it
            os.unlink(tmp)
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{log}")
    if verbose and log.strip():
        print(log, flush=True)
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
