"""gs_voxelizer — MI355X-native drop-in for PaPieta/gs-voxelizer.

Submodules mirror the reference package: ``optim_to_render``, ``voxelize``,
``bin_and_sort_gaussians`` and the native module ``cuda`` (backed by the
gfx950 library libgsvox.so).  ``synthetic`` holds the seeded workload
generators used by the tests and the benchmark.
"""
__version__ = "0.2.0"
