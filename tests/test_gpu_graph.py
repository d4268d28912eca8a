"""The whole training step captured in one HIP graph (gs_voxelizer.graph).

Every replay is checked against the eager step bit for bit (the per-pair
reduction has a fixed summation order, so both give identical bits), with
eager steps and synchronisations between the replays; a scene that outgrows
the captured capacity is re-captured and still matches the eager result.
"""
import pytest
import torch

from gs_voxelizer import graph, optim_to_render, synthetic as S, voxelize
from helpers import small_config

pytestmark = pytest.mark.gpu


def _make(device, cfg, seed, fused=True):
    work = S.make_gaussians(cfg, seed=seed)
    target = S.phantom(work, device=device)
    gvol = (target - 0.5)[..., None].contiguous()
    w = work.to(device)
    leaves = [t.clone().requires_grad_() for t in (w.pos3d, w.scale3d, w.quat, w.intensities)]

    def step():
        for t in leaves:
            t.grad = None
        pr, cn, tmin, tmax, nt = optim_to_render.optim_to_render(*leaves, cfg.vol, cfg.world,
                                                                 cfg.center)
        if fused:
            loss, vol = voxelize.voxelize_gaussians_l1_loss(pr, cn, leaves[3], cfg.vol, tmin,
                                                           tmax, nt, target)
            loss.backward()
            return loss, vol
        # the unfused op, with a fixed volume gradient (no torch reduction in the graph)
        vol = voxelize.voxelize_gaussians(pr, cn, leaves[3], cfg.vol, tmin, tmax, nt)
        vol.backward(gvol)
        return vol, vol

    return leaves, step


def _snapshot(out, leaves):
    return [out[0].detach().clone(), out[1].detach().clone()] + [t.grad.clone() for t in leaves]


def _assert_same(a, b, what):
    for i, (x, y) in enumerate(zip(a, b)):
        assert torch.equal(x, y), f"{what}: output {i} differs"


@pytest.mark.parametrize("fused", [True, False], ids=["l1_fused", "dropin"])
def test_replays_match_eager_bitwise(device, fused):
    voxelize._capacity.pop(device.index or 0, None)
    cfg = small_config(3, 20000, vol=(96, 128, 80))
    leaves, step = _make(device, cfg, seed=3, fused=fused)
    eager = _snapshot(step(), leaves)
    g = graph.CapturedStep(step)
    for k in range(3):
        out = g.replay()
        torch.cuda.synchronize()
        _assert_same(_snapshot(out, leaves), eager, f"replay {k}")
        again = _snapshot(step(), leaves)  # eager work between the replays
        torch.cuda.synchronize()
        _assert_same(again, eager, f"eager after replay {k}")
    assert g.recaptures == 0


def test_outgrown_capacity_is_recaptured(device):
    voxelize._capacity.pop(device.index or 0, None)
    cfg = small_config(1, 3000, vol=(64, 72, 56))
    leaves, step = _make(device, cfg, seed=5)
    g = graph.CapturedStep(step)
    cap = g.capacity
    with torch.no_grad():
        leaves[1].mul_(3.0)  # larger Gaussians: several times the intersections
    out = _snapshot(g.replay(), leaves)
    torch.cuda.synchronize()
    assert g.recaptures == 1 and g.capacity > cap
    eager = _snapshot(step(), leaves)
    _assert_same(out, eager, "after re-capture")
    out2 = _snapshot(g.replay(), leaves)
    _assert_same(out2, eager, "second replay")
    assert g.recaptures == 1


def test_two_forwards_in_one_captured_step(device):
    """A step with two voxelizations: each replay checks both counts, and the
    second outgrowing its capacity is caught."""
    voxelize._capacity.pop(device.index or 0, None)
    cfg_a = small_config(3, 4000, vol=(64, 72, 56))
    cfg_b = small_config(1, 2500, vol=(56, 64, 48))
    leaves_a, step_a = _make(device, cfg_a, seed=11)
    leaves_b, step_b = _make(device, cfg_b, seed=12)

    def step():
        out_a = step_a()
        out_b = step_b()
        return out_a[0] + out_b[0], out_a[1]

    eager = _snapshot(step(), leaves_a + leaves_b)
    g = graph.CapturedStep(step)
    assert len(g.counts) == 2
    out = _snapshot(g.replay(), leaves_a + leaves_b)
    torch.cuda.synchronize()
    _assert_same(out, eager, "replay")
    with torch.no_grad():
        leaves_b[1].mul_(3.0)  # the second scene outgrows the capacity
    out = _snapshot(g.replay(), leaves_a + leaves_b)
    torch.cuda.synchronize()
    assert g.recaptures == 1
    _assert_same(out, _snapshot(step(), leaves_a + leaves_b), "after re-capture")


def test_forwards_on_concurrent_threads_and_streams(device):
    """Eager steps on two host threads, each with its own stream and scene, give
    the results of running them alone (each forward reads its own pair count)."""
    import threading
    voxelize._capacity.pop(device.index or 0, None)
    cfgs = (small_config(3, 5000, vol=(64, 64, 64)), small_config(1, 3000, vol=(72, 56, 64)))
    made = [_make(device, c, seed=20 + i) for i, c in enumerate(cfgs)]
    alone = []
    for leaves, step in made:
        alone.append(_snapshot(step(), leaves))
    torch.cuda.synchronize()
    results, errors = [None, None], []

    def run(i):
        try:
            s = torch.cuda.Stream(device=device)
            leaves, step = made[i]
            with torch.cuda.stream(s):
                for _ in range(6):
                    out = step()
                results[i] = _snapshot(out, leaves)
            s.synchronize()
        except Exception as e:  # reported after join
            errors.append(e)

    threads = [threading.Thread(target=run, args=(i,)) for i in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    torch.cuda.synchronize()
    assert not errors, errors
    for i in range(2):
        _assert_same(results[i], alone[i], f"thread {i}")
