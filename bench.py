#!/usr/bin/env python3
"""Benchmark: one full differentiable voxelization iteration on one MI355X.

A step is the reference's training iteration (README.md:28-83 of
PaPieta/gs-voxelizer): optim_to_render -> voxelize_gaussians -> torch's
l1_loss against the phantom -> loss.backward() (voxelize backward + projection
backward), on the headline workload of BASELINE.json: 256^3 volume, 200,000
Gaussians, 1 channel, synthetic seeded inputs already resident in HBM.

Prints one JSON line.  `value` is ms per iteration (lower is better) of that
step through the unchanged drop-in API, from an uninstrumented timed region.
`fused_ms_per_step` is the same step with the voxelization fused with the L1
loss (voxelize_gaussians_l1_loss: the same loss, gradients identical bit for
bit; an entry point the reference does not have), and
`fused_graph_ms_per_step` the fused step captured once in a HIP graph and
replayed (gs_voxelizer.graph).

`roofline` reports the dominant kernel of the step, the voxelize backward
(k_vox_bwd + k_vox_bwd_rest).  Its launch duration is timed live with HIP
events recorded by the library on the stream the kernel is launched on, over a
second identical timed region of drop-in steps.  `achieved` is the FP32
arithmetic the kernel executes per launch, read from rocprofv3 counters of the
same workload (profiles/valu_<workload>.json: 64 lanes x (2 FMA + ADD + MUL +
TRANS) wave instructions), divided by that duration; `peak` is MI355X's FP32
vector peak.  `ref_formulation_tflops` is the reference's flop count for the
same evaluations (E x (65 + 4C): voxelize.cu:368-574's per-evaluation terms,
delta 3, sigma 18, gate 1, 4C channel terms, dsigma 1, dconic 21, dmu 21) over the same
duration; this kernel evaluates a cheaper but equivalent formulation and skips
culled pairs, so that figure can exceed the peak and is not a utilisation.
The kernel is co-limited by VALU issue and by per-wave memory latency (a timing
build without its row loop keeps most of its time), so `bound` names both:
`frac` is the VALU side; `hbm_frac` is its HBM traffic (`traffic`, calibrated
FETCH_SIZE + WRITE_SIZE from profiles/traffic_<workload>.json) over the same
duration against the 8 TB/s peak, and `wait_inst_any_frac` / `l2_hit_rate`
(profiles/mem_<workload>.json) show the wait.
`cpu_baseline` times the C oracle (a binary32 C restatement of the reference,
OpenMP over the host cores) on the same inputs.

Usage: python bench.py [--gpus 1] [--steps 50] [--warmup 30] [--config 3]
                       [--variants dropin,fused,graph] [--no-cpu-baseline]
                       [--calibrate-copy]
"""
import argparse
import ctypes
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "gs-voxelizer_amd"))

METRIC = "voxelize fwd+bwd ms/iter @256^3,200k G; Gaussian-voxel evals/s; % FP32 peak"
FP32_PEAK_TFLOPS = 157.3   # MI355X vector FP32, AMD published
HBM_PEAK_GBS = 8000.0      # MI355X HBM3E, AMD published


def parse():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=30,
                    help="untimed steps of each variant first (the GPU needs them to reach "
                         "steady clocks)")
    ap.add_argument("--config", type=int, default=3, help="workload number 1-5 (BASELINE.json)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--variants", default="dropin,fused,graph",
                    help="comma list of steps to time besides the drop-in step `value` "
                         "times: fused (voxelize_gaussians_l1_loss), graph (the fused step "
                         "replayed from a HIP graph); `dropin` alone makes every voxelize "
                         "dispatch the one `value` times (profiling runs)")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--wave-timeline", action="store_true",
                    help="also record the forward voxelize kernel's per-workgroup start/end "
                         "over one more drop-in step (gsv_wave_timeline) and summarise its load "
                         "balance under `wave_timeline`")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="also run one elementwise kernel that reads and writes 1 GiB (a "
                         "known-size kernel that scales rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    return ap.parse_args()


class KernelTimer:
    """Wraps native entry points of gs_voxelizer.cuda and records HIP events on
    the current stream (the one the kernels are launched on) around each call."""

    def __init__(self, module, names):
        import torch
        self.torch = torch
        self.module = module
        self.names = names
        self.orig = {n: getattr(module, n) for n in names}
        self.events = {n: [] for n in names}
        self.active = False

    def install(self):
        for n in self.names:
            fn = self.orig[n]

            def wrapped(*a, __fn=fn, __n=n, **k):
                if not self.active:
                    return __fn(*a, **k)
                s = self.torch.cuda.Event(enable_timing=True)
                e = self.torch.cuda.Event(enable_timing=True)
                s.record()
                out = __fn(*a, **k)
                e.record()
                self.events[__n].append((s, e))
                return out
            setattr(self.module, n, wrapped)

    def uninstall(self):
        for n, fn in self.orig.items():
            setattr(self.module, n, fn)

    def mean_ms(self, n):
        ev = self.events[n]
        if not ev:
            return None
        return sum(s.elapsed_time(e) for s, e in ev) / len(ev)


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; multi-GPU sharding "
                                   "(z-slabs of tiles per GPU) is designed but not built",
                          "n_gpus": args.gpus}))
        sys.exit(2)
    import torch
    import torch.nn.functional as F
    if not torch.cuda.is_available():
        print(json.dumps({"error": "no HIP device visible"}))
        sys.exit(1)
    import gs_voxelizer.cuda as _C
    from gs_voxelizer import optim_to_render, synthetic as S, voxelize

    dev = torch.device("cuda:0")
    cfg = S.CONFIGS[args.config]
    work = S.make_gaussians(cfg, seed=args.seed)
    target = S.phantom(work, device=dev)
    w = work.to(dev)
    leaves = [t.clone().requires_grad_() for t in (w.pos3d, w.scale3d, w.quat, w.intensities)]
    tgt = target[..., None].expand(cfg.vol + (cfg.channels,))

    # the L1 target as the fused op takes it: (D, H, W) for one channel
    tgt_fused = target if cfg.channels == 1 else tgt.contiguous()

    def make_step(fused):
        def step():
            for t in leaves:
                t.grad = None
            pos3d, scale3d, quat, inten = leaves
            pr, cn, tmin, tmax, nt = optim_to_render.optim_to_render(
                pos3d, scale3d, quat, inten, cfg.vol, cfg.world, cfg.center)
            if fused:
                loss, vol = voxelize.voxelize_gaussians_l1_loss(
                    pr, cn, inten, cfg.vol, tmin, tmax, nt, tgt_fused,
                    use_per_gaussian_backward=True)
            else:
                vol = voxelize.voxelize_gaussians(pr, cn, inten, cfg.vol, tmin, tmax, nt,
                                                  use_per_gaussian_backward=True)
                loss = F.l1_loss(vol, tgt)
            loss.backward()
            return vol
        return step

    step_fused, step_dropin = make_step(True), make_step(False)

    def timed(step, steps):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            step()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) * 1e3 / steps

    # workload statistics (intersections, evaluations) from one untimed pass
    with torch.no_grad():
        pr, cn, tmin, tmax, nt = _C.optim_to_render_forward(cfg.n, w.pos3d, w.scale3d, w.quat,
                                                            w.intensities, cfg.vol, cfg.world,
                                                            cfg.center)
        cum, total = _C.cumsum_tiles_hit(nt)
        n_isect = int(total.item())
        ids, bins = _C.bin_and_sort_gaussians(cfg.n, n_isect, tmin, tmax, cum, cfg.vol)
        D, H, W = cfg.vol
        Tx, Ty, Tz = S.tile_grid(cfg.vol)
        t = torch.arange(Tx * Ty * Tz, device=dev)
        inside = ((torch.clamp(W - (t % Tx) * 8, max=8)) * (torch.clamp(H - ((t // Tx) % Ty) * 8, max=8))
                  * (torch.clamp(D - (t // (Tx * Ty)) * 8, max=8)))
        evals = int(((bins[:, 1] - bins[:, 0]).long() * inside).sum().item())
        tile_pairs = (bins[:, 1] - bins[:, 0]).cpu().numpy()
        del pr, cn, tmin, tmax, nt, cum, ids, bins

    variants = {v.strip() for v in args.variants.split(",") if v.strip()}
    unknown = variants - {"dropin", "fused", "graph"}
    if unknown:
        raise SystemExit(f"unknown --variants {sorted(unknown)}")
    run_fused = "fused" in variants or "graph" in variants

    for _ in range(args.warmup):
        step_dropin()
        if run_fused:
            step_fused()
    torch.cuda.synchronize()

    # `value`: the drop-in step, nothing else in the timed region.
    ms = timed(step_dropin, args.steps)
    # The same region again with the library's pooled HIP events around the
    # hot kernels, on their launch stream, for the per-kernel times (the
    # events themselves cost ~15 us of GPU time per step, kept out of `value`).
    _C._L.gsv_kernel_timing_enable(1)
    ms_events = timed(step_dropin, args.steps)
    kern = {}
    for slot, name in ((0, "k_vox_fwd"), (1, "k_vox_bwd"), (2, "k_pair_reduce")):
        tot, cnt = ctypes.c_double(0), ctypes.c_int32(0)
        _C._L.gsv_kernel_timing_collect(slot, ctypes.byref(tot), ctypes.byref(cnt))
        kern[name] = (tot.value / cnt.value) if cnt.value else None
    _C._L.gsv_kernel_timing_enable(0)
    # the step fused with the L1 loss (voxelize_gaussians_l1_loss)
    ms_fused = timed(step_fused, args.steps) if "fused" in variants else None
    # the fused step captured once in a HIP graph and replayed (gs_voxelizer.graph):
    # no host work per step beyond the replay and the check of the pair count
    ms_graph = None
    if "graph" in variants:
        from gs_voxelizer import graph as G
        captured = G.CapturedStep(step_fused)
        # as many warm replays as eager warm-up steps: the GPU idles during the
        # capture and needs a few dozen steps to reach its clocks again
        for _ in range(args.warmup):
            captured.replay()
        ms_graph = timed(captured.replay, args.steps)
        del captured

    # Per-stage times from a separate, untimed pass: torch events around each
    # native call of the drop-in API. They include the host's launch gaps inside
    # a call (the GPU waits for the host there), unlike `value`, whose steps
    # are queued back to back.
    timer = KernelTimer(_C, ["optim_to_render_forward", "cumsum_tiles_hit",
                             "bin_and_sort_gaussians", "bin_and_sort_gaussians_device_count",
                             "cumsum_bin_and_sort_device_count",
                             "voxelize_forward", "voxelize_backward_per_gaussian",
                             "optim_to_render_backward"])
    timer.install()
    timer.active = True
    for _ in range(min(args.steps, 5)):
        step_dropin()
    torch.cuda.synchronize()
    timer.active = False
    timer.uninstall()

    C = cfg.channels
    fwd_ms = kern["k_vox_fwd"]          # kernel alone
    bwd_ms = kern["k_vox_bwd"]          # kernel alone (the dominant one)
    stages = {k: round(timer.mean_ms(k), 4) for k in timer.names if timer.mean_ms(k) is not None}
    stages.update({f"kernel:{k}": round(v, 4) for k, v in kern.items() if v is not None})
    # the reference's flop count for the same evaluations (not a utilisation)
    ref_bwd_tflops = evals * (65 + 4 * C) / (bwd_ms * 1e-3) / 1e12
    ref_fwd_tflops = evals * (22 + 2 * C) / (fwd_ms * 1e-3) / 1e12
    counters = _load_profile("valu", cfg.name)
    traffic = _load_profile("traffic", cfg.name)
    # co-limited: VALU issue (frac, against the FP32 peak) and per-wave memory
    # latency (the loop-free timing build keeps most of the time; the HBM rate
    # of its traffic is hbm_frac of the peak)
    roof = {"kernel": "k_vox_bwd + k_vox_bwd_rest (voxelize backward)",
            "bound": "valu + memory latency",
            "achieved": None, "peak": FP32_PEAK_TFLOPS, "unit": "TFLOP/s", "frac": None,
            "traffic": None, "hbm_frac": None, "duration_ms": round(bwd_ms, 4)}
    if counters is not None and counters.get("evals") == evals:
        bw = counters["per_launch"]["voxelize_backward"]
        achieved = bw["fp32_flops"] / (bwd_ms * 1e-3) / 1e12
        roof.update(achieved=round(achieved, 3), frac=round(achieved / FP32_PEAK_TFLOPS, 4),
                    fp32_flops_per_launch=bw["fp32_flops"],
                    valu_insts_per_simd_cycle=bw["valu_insts_per_simd_cycle"],
                    counters=f"profiles/valu_{cfg.name}.json")
        fw = counters["per_launch"].get("voxelize_forward")
        if fw is not None:
            roof["forward"] = {"kernel": "k_vox_fwd", "duration_ms": round(fwd_ms, 4),
                               "achieved": round(fw["fp32_flops"] / (fwd_ms * 1e-3) / 1e12, 3),
                               "valu_insts_per_simd_cycle": fw["valu_insts_per_simd_cycle"]}
            roof["forward"]["frac"] = round(roof["forward"]["achieved"] / FP32_PEAK_TFLOPS, 4)
    if traffic is not None and traffic.get("evals") == evals:
        roof["traffic"] = traffic.get("voxelize_backward_hbm_bytes_per_launch")
        if roof["traffic"]:
            roof["hbm_achieved_GBps"] = round(roof["traffic"] / (bwd_ms * 1e-3) / 1e9, 1)
            roof["hbm_frac"] = round(roof["hbm_achieved_GBps"] / HBM_PEAK_GBS, 4)
    mem = _load_profile("mem", cfg.name)
    if mem is not None and mem.get("pairs") == n_isect:
        k = mem["per_kernel"].get(f"k_vox_bwd<{C}, 3>") or next(
            (v for n, v in mem["per_kernel"].items() if n.startswith("k_vox_bwd<")), None)
        if k is not None:
            roof["wait_inst_any_frac"] = k["wait_inst_any_frac"]
            roof["l2_hit_rate"] = k["tcc_hit_rate"]
    roof["ref_formulation_tflops"] = round(ref_bwd_tflops, 3)
    roof["ref_formulation_flops_per_eval"] = 65 + 4 * C

    result = {
        "metric": METRIC,
        "value": round(ms, 4),
        "unit": "ms/iter",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded CPU torch.Generator, inputs resident in HBM)",
        "config": {"workload": cfg.name, "volume_zyx": list(cfg.vol), "gaussians": cfg.n,
                   "channels": C, "intersections": n_isect, "evals": evals,
                   "loss": f"l1 vs {cfg.phantom} phantom", "seed": args.seed,
                   "step": "optim_to_render + voxelize_gaussians + torch l1_loss + backward "
                           "(the reference's API, unchanged)",
                   "fused_step": "optim_to_render + voxelize_gaussians_l1_loss (voxelization "
                                 "fused with the L1 loss; identical gradients) + backward"},
        "fused_ms_per_step": None if ms_fused is None else round(ms_fused, 4),
        "fused_graph_ms_per_step": None if ms_graph is None else round(ms_graph, 4),
        "ms_per_step_with_kernel_events": round(ms_events, 4),
        "evals_per_s": round(2 * evals / (ms * 1e-3), 1),
        "fwd_evals_per_s": round(evals / (fwd_ms * 1e-3), 1),
        "bwd_evals_per_s": round(evals / (bwd_ms * 1e-3), 1),
        "fwd_ms": round(fwd_ms, 4),
        "bwd_ms": round(bwd_ms, 4),
        "fwd_ref_formulation_tflops": round(ref_fwd_tflops, 3),
        "stage_ms": stages,
        "stage_note": "torch events around each native call of the drop-in step, one call at a time: host launch gaps included (a multi-kernel stage such as binning reads well above its kernels); kernel:* entries are the kernels alone",
        "roofline": roof,
        "cpu_baseline": None,
    }
    if args.wave_timeline:
        result["wave_timeline"] = wave_timeline(_C, step_dropin, cfg, dev, tile_pairs)
    if args.calibrate_copy:
        # an elementwise kernel that reads 1 GiB and writes 1 GiB (a plain hipMemcpy
        # D2D may run on a DMA engine, invisible to the counters); a second 1 GiB
        # fill in between evicts the source from the 256 MB last-level cache
        src = torch.ones((256 << 20,), device=dev)
        flush = torch.ones((256 << 20,), device=dev)
        dst = torch.empty_like(src)
        torch.mul(src, 2.0, out=dst)
        torch.cuda.synchronize()
        result["calibration_copy_bytes"] = src.numel() * 4
        del src, flush, dst
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(work)
    print(json.dumps(result), flush=True)


def wave_timeline(_C, step, cfg, dev, tile_pairs):
    """Per-workgroup start/end of the forward voxelize kernel (one workgroup per
    tile) over one drop-in step, summarised: the kernel span, the span an ideal
    balance would give (the summed workgroup durations over the peak number
    running at once), when the running count falls below fractions of its
    peak, and when the heaviest tiles ran."""
    import numpy as np
    import torch
    Tx, Ty, Tz = (cfg.vol[2] + 7) // 8, (cfg.vol[1] + 7) // 8, (cfg.vol[0] + 7) // 8
    T = Tx * Ty * Tz
    cap = (T + 63) // 64 * 64
    rec = torch.zeros((cap, 3), dtype=torch.int64, device=dev)
    torch.cuda.synchronize()
    assert _C._L.gsv_wave_timeline(0, ctypes.c_void_p(rec.data_ptr()), cap) == 0
    try:
        step()
        torch.cuda.synchronize()
    finally:
        _C._L.gsv_wave_timeline(0, ctypes.c_void_p(0), 0)
    r = rec.cpu().numpy()
    ok = (r[:, 0] > 0) & (r[:, 1] > 0)
    t0 = (r[ok, 0] - r[ok, 0].min()) / 100.0  # 100 MHz ticks -> microseconds
    t1 = (r[ok, 1] - r[ok, 0].min()) / 100.0
    tile = r[ok, 2]
    dur = t1 - t0
    span = float(t1.max())
    grid = np.linspace(0.0, span, 512)
    running = np.array([int(((t0 <= g) & (t1 > g)).sum()) for g in grid])
    peak = int(running.max())
    after = grid > grid[int(np.argmax(running))]
    fall = {}
    for frac in (0.75, 0.5, 0.25, 0.1):
        below = grid[(running < frac * peak) & after]
        fall[f"{int(frac * 100)}%"] = round(float(below.min()) if below.size else span, 1)
    heavy = np.argsort(-dur)[:5]
    pairs = tile_pairs[np.clip(tile, 0, tile_pairs.size - 1)]
    top = np.argsort(-pairs)[:5]
    return {"workgroups": int(ok.sum()), "span_us": round(span, 1),
            "balanced_span_us": round(float(dur.sum()) / peak, 1), "peak_running": peak,
            "running_below_peak_at_us": fall,
            "longest": [{"tile": int(tile[i]), "pairs": int(pairs[i]),
                         "start_us": round(float(t0[i]), 1), "end_us": round(float(t1[i]), 1)}
                        for i in heavy],
            "heaviest_tiles": [{"tile": int(tile[i]), "pairs": int(pairs[i]),
                                "start_us": round(float(t0[i]), 1),
                                "end_us": round(float(t1[i]), 1)} for i in top],
            "last_start_us": round(float(t0.max()), 1),
            "note": "forward voxelize kernel of one drop-in step; one workgroup (one wave) per "
                    "tile; GPU wall clock at 100 MHz"}


def _load_profile(kind, workload):
    """profiles/<kind>_<workload>.json (rocprofv3 counter summaries), or None."""
    path = os.path.join(ROOT, "profiles", f"{kind}_{workload}.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f)


def cpu_baseline(work, repeats=3):
    """The CPU oracle (test infrastructure: binary32 C restatement of the
    reference, OpenMP over all host cores) on the same inputs: one whole
    iteration (projection, binning, voxelize forward, voxelize backward,
    projection backward), median of `repeats` after one warm-up on a slice."""
    sys.path.insert(0, ROOT)
    import numpy as np
    import oracle as O
    cfg = work.cfg
    p, s, q, I = (t.numpy() for t in (work.pos3d, work.scale3d, work.quat, work.intensities))
    g = np.full(cfg.vol + (cfg.channels,), 1.0 / np.prod(cfg.vol), np.float32)

    def one(tile_range=None):
        tm = {}
        t0 = time.perf_counter()
        pr, cn, tmin, tmax, nt = O.project_fwd(p, s, q, I, cfg.vol, cfg.world, cfg.center)
        cum = O.cumsum(nt)
        ids, bins = O.bin_and_sort(cfg.n, int(cum[-1]), tmin, tmax, cum, cfg.vol)
        t1 = time.perf_counter()
        O.voxelize_fwd(cfg.vol, ids, bins, pr, cn, I, tile_range=tile_range)
        t2 = time.perf_counter()
        dpr, dcn, _ = O.voxelize_bwd(cfg.vol, ids, bins, pr, cn, I, g, tile_range=tile_range)
        t3 = time.perf_counter()
        O.project_bwd(p, s, q, cfg.vol, cfg.world, cfg.center, dpr, dcn, pr)
        t4 = time.perf_counter()
        tm.update(project_and_bin=t1 - t0, voxelize_fwd=t2 - t1, voxelize_bwd=t3 - t2,
                  project_bwd=t4 - t3, total=t4 - t0)
        return tm

    Tx, Ty, _ = O.tile_grid(cfg.vol)
    one(tile_range=(0, Tx * Ty))  # warm-up: page in, spin up the thread pool
    runs = sorted((one() for _ in range(repeats)), key=lambda r: r["total"])
    med = runs[len(runs) // 2]
    return {"value": round(med["total"] * 1e3, 1), "unit": "ms/iter", "cores": O.num_threads(),
            "kind": "port", "label": "C oracle (test infrastructure), not a dense PyTorch path",
            "sample": (f"the whole {cfg.name} iteration (no subsampling) through oracle/gsv_oracle.c, "
                       f"a binary32 C restatement of the reference (OpenMP); median of {repeats}"),
            "measured_s": {k: round(v, 3) for k, v in med.items()},
            "cpu": _cpu_model()}


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


if __name__ == "__main__":
    main()
