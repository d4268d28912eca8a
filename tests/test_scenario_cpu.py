"""The seeded restatement of the reference's value scenario
(test/test_gs_voxelizer.py:15-26, random_gauss_init and generate_test_volume
of test/utils.py:10-29, 91-154) has that test's shapes, constants and
intensity lookup, and is deterministic."""
import numpy as np
import torch

from gs_voxelizer import synthetic as S


def test_reference_scenario_matches_the_reference_test_setup():
    work, vol = S.reference_value_scenario(seed=0, n=5000)
    cfg = work.cfg
    assert cfg.vol == (100, 150, 80) and cfg.world == (1.0, 1.0, 1.0)
    assert cfg.center == (0.5, 0.5, 0.5) and S.REFERENCE_SCENARIO.n == 100_000
    assert vol.shape == (100, 150, 80) and vol.dtype == torch.float32
    assert float(vol.min()) >= 0.1 - 1e-7 and float(vol.max()) <= 1.0
    assert 0.05 < float((vol > 0.1).float().mean()) < 0.6  # 20 balls of radius 10-19
    np.testing.assert_array_equal(work.scale3d[0].numpy(), np.float32([0.03, 0.01, 0.02]))
    assert float(work.pos3d.min()) >= 0.0 and float(work.pos3d.max()) < 1.0
    np.testing.assert_allclose(work.quat.norm(dim=1).numpy(), 1.0, atol=1e-6)
    idx = torch.clamp((work.pos3d * torch.tensor([79.0, 149.0, 99.0])).long(), min=0)
    want = vol[idx[:, 2], idx[:, 1], idx[:, 0]] / 10
    np.testing.assert_array_equal(work.intensities[:, 0].numpy(), want.numpy())
    again, vol2 = S.reference_value_scenario(seed=0, n=5000)
    assert torch.equal(again.quat, work.quat) and torch.equal(vol2, vol)
    other, _ = S.reference_value_scenario(seed=1, n=5000)
    assert not torch.equal(other.pos3d, work.pos3d)
