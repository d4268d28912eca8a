"""CPU oracle for the Gaussian voxelization path — TEST INFRASTRUCTURE ONLY.

This package is the checker, never the thing measured or shipped. Only
``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it. The product path (``gs-voxelizer_amd/``) has no
dependency on it and fails loudly when its HIP library is missing.

``gsv_oracle.c`` restates the reference kernels (PaPieta/gs-voxelizer v0.1.0,
``gs_voxelizer/cuda/*.cu``) in binary32 C with the reference's evaluation order
and no FMA contraction; ``oracle.py`` wraps it for numpy.

Parity status of each oracle function (what pins it, in ``tests/``):

* ``project_fwd`` — closed forms (identity/90-degree quaternions, isotropic
  scales), an independent fp64 linear-algebra restatement via scipy rotations
  and ``numpy.linalg.inv``, hand-computed tile boxes, special values of the
  extent (``test_oracle_projection.py``).
* ``project_bwd`` — fp64 central finite differences of an independent fp64
  forward: dscale (rtol 1e-4 where det^2 >> 1e-7), all four dquat components
  through the unnormalised quadratic rotation polynomial (radial part
  included), dpos up to the reference's voxel-size factor; the 1e-7 det^2
  regulariser by its closed form on isotropic 0.2-0.5 voxel Gaussians
  (``test_oracle_projection.py``).
* ``bin_and_sort`` — brute force with Python ``sorted`` over (tile, gaussian)
  pairs (``test_oracle_binning.py``).
* ``voxelize_fwd`` — dense fp64 evaluation with numpy over every voxel, closed
  forms, linearity (``test_oracle_voxelize.py``).
* ``voxelize_bwd`` — torch autograd through a dense fp64 evaluation and
  central finite differences (``test_oracle_voxelize.py``).
* ``logf`` — against ``math.log`` over the binary32 range (``test_oracle_numerics.py``).

No golden vectors, fixtures or known-answer tests exist in the reference for
this path (its only value test compares live against an external CUDA
package), so nothing else can pin the oracle.
"""
from .oracle import *  # noqa: F401,F403
