"""The package installs with pip the way the reference's does (setup.py:153-179
of PaPieta/gs-voxelizer): metadata, the package list and the compiled library
as package data.  Reading the metadata does not compile anything."""
import os
import subprocess
import sys

PKG = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "gs-voxelizer_amd")


def test_setup_metadata_lists_the_library():
    out = subprocess.run([sys.executable, "setup.py", "--name", "--version"], cwd=PKG,
                         capture_output=True, text=True, check=True).stdout.split()
    assert out[-2:] == ["gs-voxelizer-amd", "0.2.0"]
    import gs_voxelizer
    assert gs_voxelizer.__version__ == "0.2.0"
    with open(os.path.join(PKG, "setup.py")) as f:
        text = f.read()
    assert '"libgsvox.so"' in text and "build_py" in text
    assert os.path.exists(os.path.join(PKG, "pyproject.toml"))
