"""Benchmark of the MI355X tiled Gaussian-splatting rasterizer (forward + backward).

Headline workload: 1,000,000 Gaussians, SH degree 3,
1920x1080, forward + L1 loss + backward to the five Gaussian parameter arrays, one
frame per step, synthetic seeded scene (jax_gs_amd.scenes, seed 2), inputs resident
in HBM before timing.

Prints ONE JSON line (rank 0, N=1 only: this build runs on a single GPU).
"""
from __future__ import annotations

import argparse
import ctypes
import gc
import json
import math
import os
import sys
import time

_ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(_ROOT, "jax-gs_amd"))
sys.path.insert(0, _ROOT)

import numpy as np  # noqa: E402
import torch  # noqa: E402

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E
FP32_PEAK_TFLOPS = 157.3  # MI355X published FP32 vector peak (packed FP32 instructions)
# The issue rate without packed FP32, which this build disables: 256 CUs x 4 SIMDs x 16
# lanes x 2 FLOP (FMA) x 2.4 GHz.
FP32_NONPACKED_PEAK_TFLOPS = 78.6
# Estimates of the reference algorithm's arithmetic per (pixel, entry) pair it evaluates:
# ~22 FLOP + 1 exp forward, ~2.5x that backward.  The kernels skip the pairs their
# rectangle cull drops and share per-column terms between a lane's pixels, so these count
# the reference's work, not instructions issued (VALU busy, from the SQ counters, does).
COMPOSITE_FWD_FLOP_PER_PAIR = 22
COMPOSITE_BWD_FLOP_PER_PAIR = 55
PROFILES = os.path.join(_ROOT, "profiles")


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", type=int, default=2)
    ap.add_argument("--step", choices=["auto", "fwd", "fwdbwd", "fwdbwd_stats"], default="auto",
                    help="what one timed step runs; auto = the configuration's own workload in BASELINE.json: "
                         "forward only for configs 0 and 3, forward + L1 + backward for 1 and 2, and for 4 the "
                         "same plus the densification statistics (trainer.py:143-159)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-runs", type=int, default=3, help="timed CPU baseline runs (after one warm-up)")
    ap.add_argument("--stages", action="store_true", help="print per-stage timings to stderr")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="finish with a plain 256 MiB device copy (PMC byte-counter calibration)")
    return ap.parse_args()


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(json.dumps({"error": "this build runs on one GPU only (the multi-GPU path is design-only); "
                                   "run with --gpus 1"}))
        sys.exit(2)
    from jax_gs_amd import _lib, render, render_l1, scenes
    from jax_gs_amd.renderer import rasterizer
    from jax_gs_amd.renderer.projection import preprocess
    from jax_gs_amd.training.losses import l1_loss

    dev = torch.device("cuda:0")
    sc = scenes.make_scene(args.config)
    g, cam, tgt, mask = scenes.to_torch(sc, dev)
    if tgt is None:
        tgt = torch.from_numpy(np.random.default_rng(99).uniform(0, 1, (cam.H, cam.W, 3)).astype(np.float32)).to(dev)
    fields = ("means", "scales", "quaternions", "opacities", "sh_coeffs")
    for f in fields:
        getattr(g, f).requires_grad_(True)
    D = sc["sh_degree"]
    N = g.means.shape[0]
    kind = args.step if args.step != "auto" else {0: "fwd", 3: "fwd", 4: "fwdbwd_stats"}.get(args.config, "fwdbwd")
    # the densification statistics the trainer accumulates after the backward (trainer.py:143-159)
    from jax_gs_amd.training.trainer import accumulate_from_extras

    stats_state = {"grad_accum": torch.zeros(N, device=dev), "denom": torch.zeros(N, dtype=torch.int32, device=dev),
                   "max_radii": torch.zeros(N, device=dev)}

    def step(fused=True):
        if kind == "fwd":
            with torch.no_grad():
                _, extras = render(g, cam, mask=mask, sh_degree=D)
            return extras
        for f in fields:
            getattr(g, f).grad = None
        if fused:
            # render + L1 loss with the loss fused into the compositing launches
            _, loss, extras = render_l1(g, cam, tgt, mask=mask, sh_degree=D)
        else:
            image, extras = render(g, cam, mask=mask, sh_degree=D)
            loss = l1_loss(image, tgt)
        loss.backward()
        if kind == "fwdbwd_stats":
            accumulate_from_extras(stats_state, g.means.grad, g.means.detach(), cam, extras, active=mask)
        return extras

    def timed(fused):
        for _ in range(args.warmup):
            step(fused)
        torch.cuda.synchronize()
        # Python's cyclic garbage collector paused over the timed steps (as timeit does): a
        # collection triggered inside them stalled the host, and with it the GPU, for tens of
        # milliseconds (seen in a fresh process on a fresh GPU box, whose first imports
        # allocate differently).  No collection is forced first: steps timed right after a
        # gc.collect() ran 0.73-0.75 ms against 0.70 (measured; the cause was not found)
        gc.disable()
        try:
            t0 = time.perf_counter()
            for _ in range(args.steps):
                ex = step(fused)
            torch.cuda.synchronize()
            t = (time.perf_counter() - t0) / args.steps
        finally:
            gc.enable()
        return t, ex

    # ---- per-stage timing with HIP events on the launch stream (torch's current stream)
    st = torch.cuda.current_stream(dev)
    s_ = _lib.stream_handle(dev)
    ev = {}

    def mark(name):
        e = torch.cuda.Event(enable_timing=True)
        e.record(st)
        ev.setdefault(name, []).append(e)

    reps = max(3, args.steps)
    bg = torch.zeros(3, device=dev)
    one = torch.ones((), device=dev)  # dL/dloss
    W, H = cam.W, cam.H

    def stage_loop():
        """One step's stages, `reps` times, an event between stages; returns the last
        repetition's tensors."""
        for _ in range(reps):
            mark("t0")
            pre = preprocess(g, cam, mask=mask, sh_degree=D, projected=False)
            mark("t1")
            b = rasterizer.bin_gaussians(pre["means2d"], pre["radii"], pre["valid"], pre["depths"], H, W,
                                         want_tiles=False, window=True, deferred=True)
            mark("t2")
            grec = torch.empty((N, _lib.GS_REC_STRIDE), device=dev)  # cleared by the forward launch
            # the compositing forward with the L1 loss fused (its partial sums, and the
            # launch that orders the tiles for the backward finishes the loss)
            image, fT, nc, order, loss = rasterizer.composite(pre["records"], b["sorted_gids"], b["ranges"], H, W,
                                                              bg, clear_records=grec, window=b["window"], bins=b,
                                                              l1_target=tgt)
            mark("t3")
            # as in the step: the compositing VJP zeroes the five gradient arrays on the side
            # and the preprocessing VJP writes only the reached Gaussians' rows
            outs = [torch.empty_like(getattr(g, f)) for f in fields]
            cl = _lib.clear_list(*outs)
            _lib.call("gs_composite_bwd_l1", s_, N, _lib.ptr(pre["records"]), _lib.ptr(b["sorted_gids"]),
                      b["sorted_gids"].shape[0], _lib.ptr(b["ranges"]), W, H, _lib.ptr(bg), None, _lib.ptr(image),
                      _lib.ptr(tgt), _lib.ptr(one), _lib.ptr(fT), _lib.ptr(nc), _lib.ptr(order), _lib.ptr(grec),
                      None, 1, _lib.ptr(b["window"]), ctypes.byref(cl))
            mark("t4")
            _lib.call("gs_preprocess_bwd", s_, N, g.sh_coeffs.shape[1], D, *[_lib.ptr(getattr(g, f).detach())
                                                                             for f in fields],
                      _lib.ptr(cam.W2C.contiguous()), W, H, float(cam.fx), float(cam.fy), float(cam.cx),
                      float(cam.cy), _lib.ptr(grec), *[_lib.ptr(o) for o in outs], 1)
            mark("t5")
            accumulate_from_extras(stats_state, outs[0], g.means.detach(), cam,
                                   {"valid_mask": pre["valid"], "radii": pre["radii"]}, active=mask)
            mark("t6")
        return pre, b, grec, image, fT, nc, outs

    with torch.no_grad():
        # the stage tensors the side measurements below use (the stages are timed again
        # after the headline, on a warm GPU)
        pre, b, grec, image, fT, nc, outs = stage_loop()
        # the L1 loss and its VJP as separate launches (gs_l1_loss, gs_l1_loss_bwd: the unfused
        # path's loss stage) on the same image
        for _ in range(reps):
            mark("u0")
            lo1 = torch.empty((), device=dev)
            gimg = torch.empty_like(image)
            _lib.call("gs_l1_loss", s_, image.numel(), _lib.ptr(image), _lib.ptr(tgt), _lib.ptr(lo1), None)
            _lib.call("gs_l1_loss_bwd", s_, image.numel(), _lib.ptr(image), _lib.ptr(tgt), _lib.ptr(one),
                      _lib.ptr(gimg))
            mark("u1")
        # the trainer's other loss term (trainer.py:18-26): L1 + SSIM forward and VJP of
        # the same frame, timed beside the step (the headline step seeds L1 only)
        Hc, Wc, Cc = image.shape
        ws_bytes = _lib.lib().gs_l1_ssim_workspace_size(Hc, Wc, Cc)
        ws = torch.empty((ws_bytes,), dtype=torch.uint8, device=dev)
        lo = torch.empty((2,), device=dev)
        gout = torch.tensor([0.8, -0.1], device=dev)
        gss = torch.empty_like(image)
        for _ in range(reps):
            mark("s0")
            _lib.call("gs_l1_ssim", s_, Hc, Wc, Cc, _lib.ptr(image), _lib.ptr(tgt), _lib.ptr(lo), 1, _lib.ptr(ws),
                      ws_bytes)
            mark("s1")
            _lib.call("gs_l1_ssim_bwd", s_, Hc, Wc, Cc, _lib.ptr(image), _lib.ptr(tgt), _lib.ptr(gout), _lib.ptr(ws),
                      ws_bytes, _lib.ptr(gss))
            mark("s2")
        # the trainer's optimizer step (train.py:127-155, trainer.py:44-53) on the gradients
        # of the five arrays, with its moments
        from jax_gs_amd.training.optimizer import make_optimizer

        opt = make_optimizer(extent=3.0, num_iterations=30000)
        params = type(g)(*[getattr(g, f).detach().clone() for f in fields])
        grads = type(g)(*outs)
        ostate = opt.init(params)
        for _ in range(reps):
            mark("a0")
            opt.step(params, grads, ostate, mask)
            mark("a1")
        # density control (density.py:98-211) on the frame's Gaussians padded to 1.5x, with
        # the optimizer moments moving along; statistics from this frame's 2-D gradients
        from jax_gs_amd.training import density

        dstate = density.init_density_state(type(g)(*[getattr(g, f).detach() for f in fields]), opt,
                                             N + N // 2)
        dgen = torch.Generator(device=dev)
        dgen.manual_seed(0)
        base_accum = torch.rand((N + N // 2,), device=dev, generator=dgen) * 0.00025
        for _ in range(reps):
            dstate.grad_accum.copy_(base_accum)
            dstate.denom.fill_(1)
            dstate.active_mask[:N] = 1
            dstate.active_mask[N:] = 0
            mark("d0")
            density.densify_and_prune(dstate, dgen, extent=3.0)
            mark("d1")
        # PLY checkpoint records (ply.py:6-66) packed on the device: 236 B read, 248 B
        # written per Gaussian with degree-3 SH
        if g.sh_coeffs.shape[1] == 16:
            recs = torch.empty((N, 62), device=dev)
            for _ in range(reps):
                mark("p0")
                _lib.call("gs_ply_pack", s_, N, 16, *[_lib.ptr(getattr(g, f).detach()) for f in fields],
                          _lib.ptr(recs))
                mark("p1")
    # the reference's whole training step (trainer.py:55-169: render, 0.8 L1 + 0.2 D-SSIM,
    # backward, densification statistics, masked Adam) on the same frame and Gaussians,
    # timed beside the headline step (wall clock of `reps` steps between synchronisations)
    from jax_gs_amd.training.trainer import train_step

    tstate = density.init_density_state(type(g)(*[getattr(g, f).detach().clone() for f in fields]),
                                        make_optimizer(extent=3.0, num_iterations=30000), N)
    cs = (cam.W, cam.H, cam.fx, cam.fy, cam.cx, cam.cy)
    for _ in range(2):
        train_step(tstate, tgt, cam.W2C, cs, make_optimizer(extent=3.0, num_iterations=30000), sh_degree=D)
    topt = make_optimizer(extent=3.0, num_iterations=30000)
    torch.cuda.synchronize()
    t_ts = time.perf_counter()
    for _ in range(reps):
        train_step(tstate, tgt, cam.W2C, cs, topt, sh_degree=D)
    torch.cuda.synchronize()
    train_step_ms = (time.perf_counter() - t_ts) / reps * 1e3
    # The headline: W warm-up steps, then K timed steps.  It runs after the per-stage and
    # side measurements above, so that the GPU has left its idle clocks (a cold start runs
    # the first ~20 steps about 4 % slower).
    dt, extras = timed(True)
    # the same step with render and l1_loss as separate functions (the reference's call
    # structure: the loss's own launches and the image gradient in memory), for comparison
    dt_unfused = timed(False)[0] if kind != "fwd" else None
    n_int = int(extras["n_interactions"])
    for k in [k for k in ev if k.startswith("t")]:
        del ev[k]
    with torch.no_grad():
        pre, b, grec, image, fT, nc, outs = stage_loop()
    extra_ms = {nm: float(np.median([ev[a][r].elapsed_time(ev[z][r]) for r in range(reps)]))
                for nm, a, z in (("l1_ssim_fwd", "s0", "s1"), ("l1_ssim_bwd", "s1", "s2"), ("adam", "a0", "a1"),
                                 ("densify_and_prune", "d0", "d1"), ("l1_loss_unfused", "u0", "u1"))}
    if "p0" in ev:
        extra_ms["ply_pack"] = float(np.median([ev["p0"][r].elapsed_time(ev["p1"][r]) for r in range(reps)]))
    extra_ms["train_step"] = train_step_ms
    extra_counts = {"densify_and_prune": [int(v) for v in dstate.last_counts.tolist()]}
    # Adam reads parameter, gradient and both moments (16 B) and writes three (12 B) per value
    n_values = sum(getattr(g, f).numel() for f in fields)
    extra_gbs = {"adam": 28 * n_values / (extra_ms["adam"] * 1e-3) / 1e9}
    # L1 + SSIM: forward reads both images and writes 3 derivative maps (20 B per value),
    # backward reads the maps and both images and writes the gradient (24 B per value)
    n_img = image.numel()
    extra_gbs["l1_ssim_fwd"] = 20 * n_img / (extra_ms["l1_ssim_fwd"] * 1e-3) / 1e9
    extra_gbs["l1_ssim_bwd"] = 24 * n_img / (extra_ms["l1_ssim_bwd"] * 1e-3) / 1e9
    # densify-and-prune: 29 B read per slot for the flags (scales, opacity, mask, statistics,
    # radius) plus the filled slots' rows, read and written (4 B per value)
    dc = extra_counts["densify_and_prune"]
    row_vals = sum(getattr(g, f)[0].numel() for f in fields) * 3  # parameters and two moments
    den_bytes = 29 * (N + N // 2) + 8 * row_vals * (dc[0] + dc[1])
    extra_gbs["densify_and_prune"] = den_bytes / (extra_ms["densify_and_prune"] * 1e-3) / 1e9
    if "ply_pack" in extra_ms:
        extra_gbs["ply_pack"] = (236 + 248) * N / (extra_ms["ply_pack"] * 1e-3) / 1e9
    # composite_fwd and composite_bwd include the fused L1 loss and its VJP
    names = ["preprocess_fwd", "binning", "composite_fwd", "composite_bwd", "preprocess_bwd", "densify_stats"]
    stage_ms = {}
    for i, nm in enumerate(names):
        a, z = ev[f"t{i}"], ev[f"t{i + 1}"]
        stage_ms[nm] = float(np.median([a[r].elapsed_time(z[r]) for r in range(reps)]))
    K = g.sh_coeffs.shape[1]
    nb = (D + 1) ** 2
    # Algorithmic bytes per launch (what each stage must move at minimum):
    #   preprocess fwd: read means 12 + scales 12 + quats 16 + opacity 4 + (D+1)^2 SH triples
    #                   12 each; write means2d 8, radius 4, valid 1, depth 4 (binning's inputs)
    #                   and the compositing record 48 (conic and colour: the renderer writes no
    #                   separate cov2d and colour arrays).
    #   preprocess bwd: read the gradient record 48; for the Gaussians the compositing
    #                   reached (a nonzero gradient record) read the parameters and SH rows
    #                   (44 + 12 (D+1)^2) and write their rows of the 5 gradient arrays
    #                   (12 + 12 + 16 + 4 + 12 K); the other rows are zero, set by the
    #                   compositing backward's clear list while its waves compute.
    pre_fwd_bytes = N * (44 + 12 * nb) + N * (8 + 4 + 1 + 4 + 48)
    n_reached = int((grec[:, :9] != 0).any(dim=1).sum())
    pre_bwd_bytes = N * 48 + n_reached * (44 + 12 * nb + 12 + 12 + 16 + 4 + 12 * K)
    #   binning: read means2d 8 + radius 4 + valid 1 + depth 4 per Gaussian; write the tile
    #            ranges (4 B per tile), and the entry list (4 B per entry) when the binning
    #            writes it (the deferred binning leaves it to the compositing forward, which
    #            writes the entries it meets, unless the window is clamped, the capacity
    #            exceeded or the image under 2048 tiles).
    T = b["ranges"].shape[0] - 1
    st_np = b["stats"].cpu().numpy()
    deferred = bool(st_np[_lib.STAT["entries_deferred"]])
    bin_bytes = N * 17 + 4 * (T + 1) + (0 if deferred else 4 * n_int)
    # entries the compositing meets: per tile the largest n_contrib (what the backward reads)
    TXn, TYn = (W + 15) // 16, (H + 15) // 16
    ncp = torch.zeros((TYn * 16, TXn * 16), dtype=torch.int32, device=dev)
    ncp[:H, :W] = nc
    entries_met = int(ncp.view(TYn, 16, TXn, 16).amax(dim=(1, 3)).to(torch.int64).sum())
    #   densify stats: read grad_means 12 + valid 1 + active 1 + radius 4 and update the count
    #                  (4 + 4) per Gaussian; update the largest radius (4 + 4) of the visible ones;
    #                  read the mean 12 and update the gradient sum (4 + 4) of those with a
    #                  nonzero mean cotangent (a zero one adds +0).
    n_vis = int(pre["valid"].to(torch.bool).sum())
    n_gm = int((outs[0] != 0).any(dim=1).sum())
    dens_bytes = (N * (12 + 1 + (1 if mask is not None else 0) + 4 + 8) + n_vis * 8 + n_gm * (12 + 8))
    stage_gbs = {"preprocess_fwd": pre_fwd_bytes / (stage_ms["preprocess_fwd"] * 1e-3) / 1e9,
                 "binning": bin_bytes / (stage_ms["binning"] * 1e-3) / 1e9,
                 "preprocess_bwd": pre_bwd_bytes / (stage_ms["preprocess_bwd"] * 1e-3) / 1e9,
                 "densify_stats": dens_bytes / (stage_ms["densify_stats"] * 1e-3) / 1e9}
    # Compositing is VALU-bound; its unit of work is an evaluated (pixel, entry) pair,
    # i.e. sum over pixels of n_contrib, at ~22 FLOP forward and ~55 FLOP backward.
    pairs = int(nc.to(torch.int64).sum())
    stage_tflops = {"composite_fwd": pairs * COMPOSITE_FWD_FLOP_PER_PAIR / (stage_ms["composite_fwd"] * 1e-3) / 1e12,
                    "composite_bwd": pairs * COMPOSITE_BWD_FLOP_PER_PAIR / (stage_ms["composite_bwd"] * 1e-3) / 1e12}
    # The bandwidth-bound stages together (preprocessing forward and backward, binning):
    # HBM rate of this design's algorithmic bytes, and, for comparison, the traffic of the
    # key-duplication + radix-sort design the reference uses, counted as in the baseline
    # document (exclusive scan 8N, duplication 20N + 8M, LSD sort 16M per 8 key bits of
    # 13 + ceil(log2(T+1)), ranges 4M + 8T; preprocessing N(44 + 12K) + 44N forward and
    # 2N(44 + 12K) + 36N backward), over the same measured time.
    hbm_ms = stage_ms["preprocess_fwd"] + stage_ms["binning"] + stage_ms["preprocess_bwd"]
    own_bytes = pre_fwd_bytes + bin_bytes + pre_bwd_bytes
    key_bits = 13 + int(math.ceil(math.log2(T + 1)))
    ks_bytes = (N * (44 + 12 * nb) + 44 * N + 8 * N + 20 * N + 8 * n_int + 16 * n_int * int(math.ceil(key_bits / 8))
                + 4 * n_int + 8 * T + 2 * N * (44 + 12 * nb) + 36 * N)
    hbm_stages = {"stages": ["preprocess_fwd", "binning", "preprocess_bwd"], "ms": hbm_ms, "bytes": own_bytes,
                  "GBps": own_bytes / (hbm_ms * 1e-3) / 1e9,
                  "frac": own_bytes / (hbm_ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
                  # not an achieved rate: the bytes the reference's design (key duplication +
                  # radix sort of every entry) would move, over the time this design takes
                  "reference_design_bytes": ks_bytes,
                  "reference_design_bytes_over_this_time_frac": ks_bytes / (hbm_ms * 1e-3) / 1e9 / HBM_PEAK_GBS}
    # the dominant kernel of the timed step's own stages
    step_stages = {"fwd": names[:3], "fwdbwd": names[:5], "fwdbwd_stats": names}[kind]
    dominant = max(step_stages, key=stage_ms.get)
    if args.stages:
        print(json.dumps({"stage_ms": stage_ms, "stage_GBps": stage_gbs, "stage_TFLOPs": stage_tflops,
                          "n_interactions": n_int, "pairs": pairs}), file=sys.stderr)

    traffic, traffic_src = measured_traffic(dominant, args.config)
    if dominant in stage_gbs:
        ach = stage_gbs[dominant]
        roofline = {"kernel": dominant, "bound": "hbm", "achieved": ach, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": ach / HBM_PEAK_GBS, "traffic": traffic, "traffic_source": traffic_src}
    else:
        ach = stage_tflops.get(dominant, 0.0)
        busy, busy_src = measured_valu_busy(dominant, args.config)
        roofline = {"kernel": dominant, "bound": "valu", "achieved": ach, "peak": FP32_PEAK_TFLOPS,
                    "unit": "TFLOP/s", "frac": ach / FP32_PEAK_TFLOPS, "traffic": traffic,
                    "traffic_source": traffic_src, "pairs": pairs,
                    "flop_per_pair": COMPOSITE_BWD_FLOP_PER_PAIR if dominant == "composite_bwd"
                    else COMPOSITE_FWD_FLOP_PER_PAIR,
                    "flops": "estimate: the reference algorithm's FLOP per (pixel, entry) pair x sum of n_contrib",
                    # what the build can issue: non-packed FP32 (packed FP32 is disabled), and the
                    # share of SIMD cycles the kernel issues VALU work on (SQ counters)
                    "nonpacked_peak": FP32_NONPACKED_PEAK_TFLOPS, "valu_busy": busy, "valu_busy_source": busy_src}

    # after the headline (it does not disturb the timed steps), before the calibration copies
    # (the profile summaries take the run's last three copy dispatches for those)
    probe = hbm_probe(dev)

    if args.copy_calibration:
        src = torch.ones(64 * 1024 * 1024, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(sc, args.cpu_runs)

    mpix = cam.W * cam.H / 1e6
    out = {
        "metric": "fwd+bwd ms/frame & Mpix/s at 1M Gaussians 1080p SH3; % HBM roofline",
        "value": mpix / dt,
        "unit": "Mpix/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": dt * 1e3,
        "ms_per_step_unfused_loss": None if dt_unfused is None else dt_unfused * 1e3,
        "fwd_ms": stage_ms["preprocess_fwd"] + stage_ms["binning"] + stage_ms["composite_fwd"],
        "step": kind,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded scene generator, configs[%d])" % args.config,
        "config": {"workload": sc["name"] + {"fwd": " fwd", "fwdbwd": " fwd+L1+bwd",
                                             "fwdbwd_stats": " fwd+L1+bwd+densify stats"}[kind],
                   "gaussians": N, "width": cam.W, "height": cam.H,
                   "sh_degree": D, "n_interactions": n_int, "gaussians_per_s": N / dt,
                   "binning_deferred": deferred, "entries_met": entries_met, "gaussians_reached": n_reached},
        "stage_ms": stage_ms,
        "stage_GBps": stage_gbs,
        "stage_TFLOPs": stage_tflops,
        "extra_stage_ms": extra_ms,
        "extra_stage_GBps": extra_gbs,
        "extra_counts": extra_counts,
        "roofline": roofline,
        "hbm_stages": hbm_stages,
        "hbm_probe": probe,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out))


def hbm_probe(dev, mib: int = 512, reps: int = 5) -> dict:
    """This GPU's streaming rates with torch's own kernels on mib-MiB buffers (median of reps
    runs, HIP events): a fill (writes), a sum (reads) and a copy (reads + writes), in GB/s of the
    bytes each moves.  The ceiling the bandwidth-bound stages are compared with besides the
    published 8 TB/s."""
    n = mib * 2**20 // 4
    a = torch.ones(n, dtype=torch.float32, device=dev)
    b = torch.empty_like(a)
    st = torch.cuda.current_stream(dev)
    res = {"buffer_MiB": mib}
    for name, fn, nbytes in (("write", lambda: b.fill_(0.5), 4 * n), ("read", lambda: a.sum(), 4 * n),
                             ("copy", lambda: b.copy_(a), 8 * n)):
        ts = []
        for _ in range(reps):
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(st)
            fn()
            e1.record(st)
            torch.cuda.synchronize()
            ts.append(e0.elapsed_time(e1))
        res[name + "_GBps"] = nbytes / (float(np.median(ts)) * 1e-3) / 1e9
    del a, b
    torch.cuda.empty_cache()
    return res


def measured_traffic(kernel, config):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 PMC summary of the same
    configuration (FETCH_SIZE + WRITE_SIZE scaled by the copy-kernel calibration), and that
    file; (None, None) when no summary of this configuration exists."""
    path = os.path.join(PROFILES, f"hbm_traffic_cfg{config}.md")
    if not os.path.exists(path):
        return None, None
    for line in open(path):
        if line.startswith("| " + kernel + " |"):
            try:
                return float(line.split("|")[-2].strip()), os.path.relpath(path, _ROOT)
            except ValueError:
                return None, None
    return None, None


def measured_valu_busy(stage, config):
    """VALU-busy fraction of the stage's kernel from the committed SQ-counter summary of the
    same configuration, and that file; (None, None) when there is none."""
    # the builds of the bench's launches (the forward's first template argument is the pixels
    # per lane, which the image size picks): matched by prefix
    kernels = {"composite_bwd": "composite_bwd_wide_kernel<true, true>",
               "composite_fwd": "composite_fwd_kernel<"}
    path = os.path.join(PROFILES, f"composite_valu_cfg{config}.md")
    if stage not in kernels or not os.path.exists(path):
        return None, None
    col = None
    for line in open(path):
        cells = [c.strip() for c in line.strip().strip("|").split("|")]
        if col is None and "VALU busy %" in cells:
            col = cells.index("VALU busy %")
        elif col is not None and cells and cells[0].startswith(kernels[stage]):
            try:
                return float(cells[col]) / 100.0, os.path.relpath(path, _ROOT)
            except (ValueError, IndexError):
                return None, None
    return None, None


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(sc, runs):
    """The oracle (C restatement of the reference path, OpenMP over every core this
    process may run on) on the whole workload: all Gaussians, the full frame, forward +
    L1 seed + backward to the five arrays.  One warm-up, then the median of `runs`."""
    import oracle

    cores = len(os.sched_getaffinity(0))
    oracle.set_threads(cores)
    cam = sc["cam"]
    tgt = np.random.default_rng(5).uniform(0, 1, (cam["H"], cam["W"], 3)).astype(np.float32)

    def frame():
        t0 = time.perf_counter()
        img, ex, res = oracle.render(sc["params"], cam, mask=sc["mask"], sh_degree=sc["sh_degree"])
        t1 = time.perf_counter()
        _, seed = oracle.l1_loss_and_grad(img, tgt)
        oracle.render_vjp(sc["params"], cam, res, seed, sh_degree=sc["sh_degree"])
        return t1 - t0, time.perf_counter() - t0

    frame()
    times = [frame() for _ in range(max(1, runs))]
    fwd = float(np.median([t[0] for t in times]))
    tot = float(np.median([t[1] for t in times]))
    px = cam["W"] * cam["H"]
    return {"value": px / 1e6 / tot, "unit": "Mpix/s", "cores": oracle.threads(), "kind": "port",
            "ms_per_frame": tot * 1e3, "fwd_ms": fwd * 1e3, "cpu": cpu_model(),
            "sample": f"the whole workload: all {sc['params']['means'].shape[0]} Gaussians, full {cam['W']}x"
                      f"{cam['H']} frame, fwd+L1+bwd, median of {len(times)} runs after 1 warm-up "
                      f"(runs {', '.join(f'{t[1]:.2f}' for t in times)} s)"}


if __name__ == "__main__":
    main()
