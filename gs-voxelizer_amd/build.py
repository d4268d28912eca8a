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

# Per-source additions.  voxelize.hip runs in binary32 flush-to-zero mode: its
# forward builds exp2 values as products and relies on v_mul_f32 returning 0
# below 2^-126, the same gate v_exp_f32 applies (project.hip keeps IEEE
# denormals: its tile boxes are bit-exact with the reference).
SOURCE_FLAGS = {
    "voxelize.hip": ["-fgpu-flush-denormals-to-zero"],
}


def hipcc():
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found; the gfx950 library cannot be built")


def _clean(text):
    # hipcc's host pass does not know the device-only target feature; drop that noise
    noise = ("unknown target feature", "packed-fp32-ops")
    return "\n".join(l for l in text.splitlines() if not any(k in l for k in noise))


def build(verbose=False):
    """Compile the library; returns its path. Always recompiles.

    Each source is compiled to an object in its own hipcc process (they run
    concurrently; every translation unit is self-contained), then one link
    step writes the shared library.
    """
    flags = [f for f in HIPCC_FLAGS if f != "-shared"]
    with tempfile.TemporaryDirectory(dir=os.path.dirname(OUT)) as tmpdir:
        procs = []
        for s in SOURCES:
            obj = os.path.join(tmpdir, os.path.splitext(s)[0] + ".o")
            cmd = [hipcc()] + flags + SOURCE_FLAGS.get(s, []) + ["-c", os.path.join(CSRC, s), "-o", obj]
            if verbose:
                print(" ".join(cmd), flush=True)
            procs.append((s, obj, subprocess.Popen(cmd, stdout=subprocess.PIPE,
                                                   stderr=subprocess.STDOUT, text=True)))
        failed, objs = [], []
        for s, obj, pr in procs:
            out, _ = pr.communicate()
            log = _clean(out)
            if pr.returncode != 0:
                failed.append(f"{s} ({pr.returncode}):\n{log}")
            elif verbose and log.strip():
                print(log, flush=True)
            objs.append(obj)
        if failed:
            raise RuntimeError("hipcc failed: " + "\n".join(failed))
        tmp = os.path.join(tmpdir, "libgsvox.so")
        cmd = [hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC"] + objs + ["-o", tmp]
        if verbose:
            print(" ".join(cmd), flush=True)
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"hipcc link failed ({res.returncode}):\n{_clean(res.stdout + res.stderr)}")
        os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
