"""Host-side behaviour of the drop-in Python API that needs no device: the
reference's validation errors (optim_to_render.py:67-69, bindings.h:7-12) and
the seeded workload generators."""
import pytest
import torch

from gs_voxelizer import optim_to_render, synthetic as S
import gs_voxelizer.cuda as _C


def test_invalid_pos3d_shape_raises_value_error():
    z = torch.zeros((0, 3))
    with pytest.raises(ValueError, match="Invalid shape"):
        optim_to_render.optim_to_render(z, z, torch.zeros((0, 4)), torch.zeros((0, 1)),
                                        (8, 8, 8), (1.0, 1.0, 1.0), (0.5, 0.5, 0.5))
    p = torch.zeros((4, 2))
    with pytest.raises(ValueError, match="Invalid shape"):
        optim_to_render.optim_to_render(p, p, torch.zeros((4, 4)), torch.zeros((4, 1)),
                                        (8, 8, 8), (1.0, 1.0, 1.0), (0.5, 0.5, 0.5))


def test_host_tensors_are_rejected_like_check_input():
    t = torch.zeros((4, 3))
    with pytest.raises(RuntimeError, match="must be a CUDA tensor"):
        _C.optim_to_render_forward(4, t, t, torch.zeros((4, 4)), torch.zeros((4, 1)),
                                   (8, 8, 8), (1.0, 1.0, 1.0), (0.5, 0.5, 0.5))
    with pytest.raises(RuntimeError, match="must be a CUDA tensor"):
        _C.cumsum_tiles_hit(torch.zeros((4,), dtype=torch.int32))


def test_backward_box_arguments_come_together():
    t = torch.zeros((1,))
    with pytest.raises(RuntimeError):
        _C.voxelize_backward_per_gaussian((8, 8, 8), t, t, t, t, t, t, tile_min=t)


@pytest.mark.parametrize("k", [1, 2, 3, 5])
def test_synthetic_workloads_are_seeded_and_shaped(k):
    cfg = S.CONFIGS[k]
    a = S.make_gaussians(cfg, seed=0, n=1000)
    b = S.make_gaussians(cfg, seed=0, n=1000)
    for x, y in zip((a.pos3d, a.scale3d, a.quat, a.intensities),
                    (b.pos3d, b.scale3d, b.quat, b.intensities)):
        assert torch.equal(x, y)
    assert a.intensities.shape == (1000, cfg.channels)
    assert torch.allclose(a.quat.norm(dim=1), torch.ones(1000), atol=1e-5)
    lo, hi = cfg.intensity
    assert float(a.intensities.min()) >= lo and float(a.intensities.max()) <= hi
    vs = S.voxel_size_xyz(cfg)
    s_vox = a.scale3d.double() / vs
    assert float(s_vox.min()) >= 0.5 - 1e-4
    c = S.make_gaussians(cfg, seed=1, n=1000)
    assert not torch.equal(a.pos3d, c.pos3d)


def test_phantoms_are_bounded():
    w = S.make_gaussians(S.CONFIGS[1], seed=0, n=10)
    v = S.phantom(w)
    assert v.shape == S.CONFIGS[1].vol and float(v.min()) >= 0.1 - 1e-6 and float(v.max()) <= 1.0
    cfg = S.Config("small_ellipsoids", (24, 20, 16), 10, 1, ("axis", 0.5, 2.0), "random",
                   (0.0, 1.0), "uniform", "ellipsoids")
    v = S.phantom(S.make_gaussians(cfg, seed=0))
    assert v.shape == (24, 20, 16) and float(v.max()) <= 1.0 and float(v.max()) > 0.5
