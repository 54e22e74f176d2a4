#!/usr/bin/env python3
"""Benchmark: forward+backward of the splatting chain on one MI355X.

Workload (default ``sh3_1m``): 1,000,000 Gaussians, SH degree 3, one
1297x840 camera; one step = projection -> tile intersection (count, scan,
count read-back, encode, radix sort) -> tile offsets -> SH colors ->
rasterize -> L1 loss -> backward through rasterize, SH and projection to the
Gaussian parameters (autograd, as the reference training step
scanner_points_training_utils.py:2076-2123 without the optimizer). Inputs are
seeded synthetic arrays resident on the GPU before timing.

Prints ONE JSON line on stdout (diagnostics go to stderr):
  value = Mpix/s of the whole job (pixels rendered fwd+bwd per second),
  ms_per_step, roofline of the dominant kernel (per-kernel durations from HIP
  events recorded around each launch, on the launch stream, over the timed
  steps), and the CPU baseline (the oracle, single-threaded, on this host).
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "gsplat-mlx_amd"))

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E
FP32_PEAK_TFLOPS = 157.3  # MI355X FP32 (vector and matrix)

# Algorithmic work per unit (minimum read-once/write-once bytes, or flops per
# rasterizer evaluation), per kernel; units are Gaussians (G), intersections
# (M) or evaluated (pixel, list entry) pairs (E).
FWD_FLOPS_PER_EVAL = 27
BWD_FLOPS_PER_EVAL = 75


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="sh3_1m",
                    choices=["sh3_1m", "image_fit", "random_forward", "multiview_3m", "heavy_6m"])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-accutile", action="store_true", help="skip the ellipse tile list variant")
    ap.add_argument("--no-packed", action="store_true", help="skip the packed layout variant")
    ap.add_argument("--no-dssim", action="store_true", help="skip the L1 + DSSIM loss variant")
    ap.add_argument("--morton", action="store_true",
                    help="Gaussians in 3D Morton order of their means (default: the generated, random order)")
    ap.add_argument("--cpu-band-rows", type=int, default=0,
                    help="tile rows of the CPU rasterize sample (0: the whole image)")
    ap.add_argument("--cpu-repeats", type=int, default=3, help="CPU baseline runs (median per stage)")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="first run a device copy of this many MiB (counter calibration for rocprofv3 --pmc)")
    return ap.parse_args()


class Profiler:
    """ctypes view of the C ABI's opt-in kernel timing."""

    def __init__(self):
        path = os.path.join(ROOT, "gsplat-mlx_amd", "gsplat_core", "libgsplat_hip.so")
        self.lib = ctypes.CDLL(path)
        self.lib.gsplat_hip_profile_report.restype = ctypes.c_size_t
        self.lib.gsplat_hip_profile_report.argtypes = [ctypes.c_char_p, ctypes.c_size_t]

    def enable(self, on):
        self.lib.gsplat_hip_profile_enable(1 if on else 0)

    def reset(self):
        self.lib.gsplat_hip_profile_reset()

    def report(self):
        n = self.lib.gsplat_hip_profile_report(None, 0)
        buf = ctypes.create_string_buffer(n + 1)
        self.lib.gsplat_hip_profile_report(buf, n + 1)
        out = {}
        for line in buf.value.decode().splitlines():
            name, cnt, ms = line.split("\t")
            out[name] = (int(cnt), float(ms))
        return out


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the library has no multi-GPU path; "
              "run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    import gsplat_core  # noqa: F401  (loads the HIP extension; fails loudly if missing)
    from gsplat_core import render as R
    from gsplat_core.scenes import make_scene

    dev = torch.device("cuda:0")
    if args.copy_probe_mib > 0:
        n = args.copy_probe_mib * (1 << 20) // 4
        src = torch.ones(n, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"[bench] copy probe: 3 x {args.copy_probe_mib} MiB device copy (reads and writes {args.copy_probe_mib} MiB each)")
        del src, dst
    t0 = time.time()
    scene = make_scene(args.workload, seed=0)
    if args.morton:
        from gsplat_core.scenes import morton_order, permuted

        scene = permuted(scene, morton_order(scene.means))
    log(f"[bench] scene {args.workload}: N={scene.n} {scene.width}x{scene.height}"
        f"{' (Morton order)' if args.morton else ''} ({time.time() - t0:.1f}s)")

    def param(a):
        return torch.from_numpy(np.ascontiguousarray(a)).to(dev).requires_grad_(True)

    means = param(scene.means)
    quats = param(scene.quats)
    log_scales = param(scene.log_scales)
    opacity_logits = param(scene.opacity_logits)
    viewmats = torch.from_numpy(scene.viewmats).to(dev)
    Ks = torch.from_numpy(scene.Ks).to(dev)
    sh = scene.sh_degree >= 0
    if sh:
        features_dc = param(scene.features_dc)
        features_rest = param(scene.features_rest)
        params = [means, quats, log_scales, features_dc, features_rest, opacity_logits]
    else:
        colors = param(scene.colors)
        params = [means, quats, log_scales, colors, opacity_logits]
    viewspace = torch.zeros((1, scene.n_cameras, scene.n, 2), device=dev, requires_grad=True)
    target = torch.from_numpy(scene.target).to(dev) if scene.target is not None else None
    W, H, ts = scene.width, scene.height, scene.tile_size
    forward_only = target is None
    seed = torch.ones((), device=dev)

    def step(accutile=False, packed=False, loss_mode="l1"):
        for p in params + [viewspace]:
            p.grad = None
        if sh:
            out = R.render_sh_model(means, quats, log_scales, features_dc, features_rest, opacity_logits, viewmats, Ks,
                                    W, H, ts, scene.sh_degree, viewspace_points=viewspace,
                                    background=scene.background, far_plane=scene.far_plane, accutile=accutile,
                                    packed=packed)
        elif not forward_only and loss_mode == "l1":
            # the trainer's value_and_grad: loss and gradients in one call
            # (the same kernels as the render, loss and backward below)
            _, out, _ = R.render_rgb_model_l1_value_and_grad(
                means, quats, log_scales, colors, opacity_logits, viewmats, Ks, target, W, H, ts,
                background=scene.background, opacities_in_projection=scene.opacities_in_projection,
                far_plane=scene.far_plane, accutile=accutile)
            return out
        else:
            out = R.render_rgb_model(means, quats, log_scales, colors, opacity_logits, viewmats, Ks, W, H, ts,
                                     background=scene.background,
                                     opacities_in_projection=scene.opacities_in_projection,
                                     far_plane=scene.far_plane, accutile=accutile)
        if not forward_only:
            if loss_mode == "l1":
                loss = R.l1_loss(out["render_colors"], target)
            else:  # (1 - 0.2) L1 + 0.2 (1 - SSIM) / 2, window 11: the reference trainer's defaults
                loss = R.image_training_loss(out["render_colors"], target, loss_mode, 0.2, 11)
            loss.backward(seed)  # d loss / d loss = 1, allocated once
        return out

    prof = Profiler()
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    # Headline: K steps, no profiling events.
    torch.cuda.synchronize()
    t_start = time.perf_counter()
    for _ in range(args.steps):
        out = step()
    torch.cuda.synchronize()
    t_total = time.perf_counter() - t_start
    ms_per_step = 1000.0 * t_total / args.steps
    mpix = scene.n_cameras * W * H / 1e6
    value = mpix * args.steps / t_total
    log(f"[bench] {ms_per_step:.3f} ms/step, {value:.1f} Mpix/s")

    # Same K steps again with per-kernel HIP events (launch stream) for the roofline.
    prof.reset()
    prof.enable(True)
    torch.cuda.synchronize()
    tp = time.perf_counter()
    for _ in range(args.steps):
        out = step()
    torch.cuda.synchronize()
    t_prof = 1000.0 * (time.perf_counter() - tp) / args.steps
    prof.enable(False)
    kernels = prof.report()
    log(f"[bench] profiled pass: {t_prof:.3f} ms/step")
    per_step = {k: (c / args.steps, ms / args.steps) for k, (c, ms) in kernels.items()}
    for k, (c, ms) in sorted(per_step.items(), key=lambda kv: -kv[1][1]):
        log(f"[bench]   {k:28s} {c:5.1f} launches/step {ms * 1000:9.1f} us/step")

    # Work units of this step.
    N = scene.n
    n_img = scene.n_cameras
    M = int(out["isect_ids"].numel())
    offsets = out["tile_offsets"].reshape(-1).long()
    ends = torch.cat([offsets[1:], torch.tensor([M], device=dev)])
    th, tw = out["tile_offsets"].shape[-2:]
    pix_tile = (torch.arange(H, device=dev)[:, None] // ts) * tw + (torch.arange(W, device=dev)[None, :] // ts)
    pix_tile = pix_tile[None] + (torch.arange(n_img, device=dev) * (tw * th))[:, None, None]
    start_p = offsets[pix_tile]
    end_p = ends[pix_tile]
    last = out["last_ids"].reshape(n_img, H, W).long()
    e_fwd_max = int(torch.sum(end_p - start_p))  # entries examined without early termination
    e_bwd = int(torch.clamp(torch.minimum(last, end_p - 1) - start_p + 1, min=0).sum())
    e_fwd = count_forward_evals(prof.lib, torch, R, scene, means, quats, log_scales, opacity_logits, viewmats, Ks,
                                out, W, H, ts)
    K = (scene.sh_degree + 1) ** 2 if sh else 0
    NC = N * n_img  # projected (Gaussian, camera) pairs
    P = n_img * W * H
    # Algorithmic work per step of each timed kernel (all its launches):
    # bytes read once + written once, or FP32 flops for the rasterizer (the
    # reference's per-evaluation operation counts x the evaluations up to
    # each pixel's last contributor).
    blocks, grid_words = bucket_blocks(NC, N, n_img, tw, th)
    rad = out["radii"].reshape(n_img, N, 2)
    # the render skips unseen rows' SH colours with one camera only
    n_seen = int(((rad[..., 0] > 0) & (rad[..., 1] > 0)).any(dim=0).sum()) if n_img == 1 else N
    n_tiles = n_img * tw * th
    units = {
        "raster_bwd": ("flops", BWD_FLOPS_PER_EVAL * e_bwd),
        "raster_fwd": ("flops", FWD_FLOPS_PER_EVAL * e_fwd),
        # tile buckets: per (camera, Gaussian) pair 16 B of means2d and radii
        # in and 4 B of tiles_per_gauss out, plus each grid / scatter block's
        # difference grid of (tw + 1)(th + 1) words (written, scanned in place,
        # read); the tile pass reads each image's total grid and writes the
        # tile starts; the scatter also reads the depths and writes an 8-byte
        # (depth bits, flatten id) pair per entry; the tile sort reads the pairs
        # and the tile starts and writes the 64-bit ids, the flatten ids and
        # the tile offsets
        "isect_bucket_grid": ("bytes", 20 * NC + 4 * blocks * grid_words),
        "isect_bucket_scan": ("bytes", 8 * blocks * grid_words + 4 * n_img * grid_words + 4 * n_tiles),
        "isect_bucket_scatter": ("bytes", 20 * NC + 4 * blocks * grid_words + 8 * M),
        "isect_bucket_tile_sort": ("bytes", 20 * M + 8 * n_tiles),
        # the activated projection also reads the opacity logits and writes
        # the opacities (forward), reads them and the opacity cotangent and
        # writes the logits' gradient (backward)
        "projection_fwd": ("bytes", (72 + (4 if scene.opacities_in_projection else 0)) * NC + 8 * N),
        "projection_bwd": ("bytes", (80 + 40 * n_img) * N + 12 * N),
        # the camera colours' forward reads the radii (8 B per pair) and the
        # means and coefficients of the N_s rows some camera sees (the other
        # rows are in no tile list: colour 0), and writes every colour; the
        # backward reads every row and colour cotangent and writes every
        # gradient row
        "sh_camera_fwd": ("bytes", (8 * NC if n_img == 1 else 0) + (12 + 12 * K) * n_seen + 12 * NC),
        "sh_camera_bwd": ("bytes", (24 + 24 * K + 12 * n_img) * N),
        "isect_count_scan": ("bytes", 20 * NC),
        "isect_depth_keys": ("bytes", 12 * NC),
        "sort_histogram": ("bytes", 4 * (NC + M)),
        "sort_onesweep": ("bytes", 64 * NC + 40 * M),
        "isect_encode": ("bytes", 24 * NC + 8 * M),
        # one binary search per offset slot: 8 B per probed id, 4 B written
        "isect_offsets": ("bytes", n_img * tw * th * (8 * max(1, int(M).bit_length()) + 4)),
        "raster_bwd_schedule": ("bytes", 20 * P + 36 * NC),
        "l1_loss_fwd": ("bytes", 24 * P),
        "l1_loss_bwd": ("bytes", 36 * P),
        # per image value (3 per pixel): reads image and target, writes the
        # three derivative planes; the backward reads them and both images and
        # writes the image gradient
        "image_loss_fwd": ("bytes", 20 * 3 * P),
        "image_loss_bwd": ("bytes", 24 * 3 * P),
    }
    stages = {}
    for k, (calls, ms) in sorted(per_step.items()):
        if k not in units or ms <= 0:
            continue
        kind, amount = units[k]
        if kind == "flops":
            rate = amount / (ms * 1e-3) / 1e12
            stages[k] = {"us": round(ms * 1000, 1), "achieved": round(rate, 2), "unit": "TFLOP/s",
                         "frac": round(rate / FP32_PEAK_TFLOPS, 4)}
        else:
            rate = amount / (ms * 1e-3) / 1e9
            stages[k] = {"us": round(ms * 1000, 1), "achieved": round(rate, 1), "unit": "GB/s",
                         "frac": round(rate / HBM_PEAK_GBS, 4)}
    dom = max(per_step, key=lambda k: per_step[k][1])
    calls, ms_step = per_step[dom]
    avg_ms = ms_step / calls
    roofline = None
    if dom in units:
        kind, amount = units[dom]
        per_launch = amount / calls
        if kind == "flops":
            achieved = per_launch / (avg_ms * 1e-3) / 1e12
            att = valu_attainable_tflops(prof.lib, torch)
            lds = lds_broadcast_attainable(prof.lib, torch)
            roofline = {"bound": "valu", "achieved": round(achieved, 3), "peak": FP32_PEAK_TFLOPS,
                        "unit": "TFLOP/s", "frac": round(achieved / FP32_PEAK_TFLOPS, 4),
                        "traffic": measured_traffic(args.workload, dom),
                        "kernel": dom, "avg_ms": round(avg_ms, 4),
                        "note": "compute roofline: FP32 VALU (no MFMA on this path), peak = MI355X FP32 "
                                "(counts packed FP32, which these kernels do not use)",
                        "attainable": {"peak": round(att, 2), "frac": round(achieved / att, 4),
                                       "note": "measured FP32 FMA-chain probe (single, not packed, VALU "
                                               "instructions) on this GPU in this run"},
                        "lds_broadcast_attainable": lds}
            if "raster_fwd" in per_step and "raster_bwd" in per_step:
                t_fb = (per_step["raster_fwd"][1] + per_step["raster_bwd"][1]) * 1e-3
                fb = (FWD_FLOPS_PER_EVAL * e_fwd + BWD_FLOPS_PER_EVAL * e_bwd) / t_fb / 1e12
                fw = FWD_FLOPS_PER_EVAL * e_fwd / (per_step["raster_fwd"][1] * 1e-3) / 1e12
                roofline["raster_fwd_bwd"] = {"achieved": round(fb, 3), "frac_of_attainable": round(fb / att, 4),
                                              "ms": round(t_fb * 1e3, 4)}
                roofline["raster_fwd"] = {"achieved": round(fw, 3), "frac_of_attainable": round(fw / att, 4),
                                          "ms": round(per_step["raster_fwd"][1], 4), "e_fwd": e_fwd}
        else:
            achieved = per_launch / (avg_ms * 1e-3) / 1e9
            roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                        "frac": round(achieved / HBM_PEAK_GBS, 4),
                        "traffic": measured_traffic(args.workload, dom), "kernel": dom,
                        "avg_ms": round(avg_ms, 4)}
    log(f"[bench] N={N} M={M} E_fwd={e_fwd} (without termination {e_fwd_max}) E_bwd={e_bwd} dominant={dom} "
        f"{avg_ms:.4f} ms")

    # The same step with ellipse (AccuTile) tile lists: the same images from
    # fewer intersections. Reported beside the headline (which keeps the
    # reference's AABB lists), not as it.
    accutile = None
    if not args.no_accutile:
        for _ in range(args.warmup):
            step(accutile=True)
        torch.cuda.synchronize()
        ta = time.perf_counter()
        for _ in range(args.steps):
            out_a = step(accutile=True)
        torch.cuda.synchronize()
        ms_a = 1000.0 * (time.perf_counter() - ta) / args.steps
        prof.reset()
        prof.enable(True)
        for _ in range(args.steps):
            out_a = step(accutile=True)
        torch.cuda.synchronize()
        prof.enable(False)
        kern_a = {k: round(ms / args.steps * 1000, 1) for k, (c, ms) in sorted(prof.report().items())}
        M_a = int(out_a["isect_ids"].numel())
        accutile = {"ms_per_step": round(ms_a, 4), "value": round(mpix / (ms_a * 1e-3), 2), "unit": "Mpix/s",
                    "n_isects": M_a, "kernels_us_per_step": kern_a}
        log(f"[bench] accutile: {ms_a:.3f} ms/step, M={M_a} ({M_a / max(M, 1):.3f} of AABB)")

    # The same step over the packed layout (per-pair arrays hold only the
    # visible pairs; same images). Reported beside the headline.
    packed = None
    if sh and not args.no_packed:
        for _ in range(args.warmup):
            step(packed=True)
        torch.cuda.synchronize()
        tq = time.perf_counter()
        for _ in range(args.steps):
            out_p = step(packed=True)
        torch.cuda.synchronize()
        ms_p = 1000.0 * (time.perf_counter() - tq) / args.steps
        prof.reset()
        prof.enable(True)
        for _ in range(args.steps):
            out_p = step(packed=True)
        torch.cuda.synchronize()
        prof.enable(False)
        kern_p = {k: round(ms / args.steps * 1000, 1) for k, (c, ms) in sorted(prof.report().items())}
        nnz = int(out_p["camera_ids"].numel())
        packed = {"ms_per_step": round(ms_p, 4), "value": round(mpix / (ms_p * 1e-3), 2), "unit": "Mpix/s",
                  "nnz": nnz, "dense_pairs": N * n_img, "kernels_us_per_step": kern_p}
        log(f"[bench] packed: {ms_p:.3f} ms/step, nnz={nnz} of {N * n_img} pairs")

    # The same step with the reference trainer's default loss, L1 + DSSIM
    # (scanner_points_training_utils.py:1147-1172, 1773). Reported beside the
    # headline, whose workload is specified with the L1 loss.
    dssim = None
    if not forward_only and not args.no_dssim:
        for _ in range(args.warmup):
            step(loss_mode="l1_dssim")
        torch.cuda.synchronize()
        td = time.perf_counter()
        for _ in range(args.steps):
            step(loss_mode="l1_dssim")
        torch.cuda.synchronize()
        ms_d = 1000.0 * (time.perf_counter() - td) / args.steps
        prof.reset()
        prof.enable(True)
        for _ in range(args.steps):
            step(loss_mode="l1_dssim")
        torch.cuda.synchronize()
        prof.enable(False)
        kern_d = {k: (c / args.steps, ms / args.steps) for k, (c, ms) in sorted(prof.report().items())}
        loss_stages = {}
        for k in ("image_loss_fwd", "image_loss_bwd"):
            if k in kern_d and kern_d[k][1] > 0:
                rate = units[k][1] / (kern_d[k][1] * 1e-3) / 1e9
                loss_stages[k] = {"us": round(kern_d[k][1] * 1000, 1), "achieved": round(rate, 1), "unit": "GB/s",
                                  "frac": round(rate / HBM_PEAK_GBS, 4)}
        dssim = {"ms_per_step": round(ms_d, 4), "value": round(mpix / (ms_d * 1e-3), 2), "unit": "Mpix/s",
                 "loss": "0.8 L1 + 0.2 (1 - SSIM) / 2, window 11", "stages": loss_stages,
                 "kernels_us_per_step": {k: round(v[1] * 1000, 1) for k, v in kern_d.items()}}
        log(f"[bench] l1_dssim: {ms_d:.3f} ms/step {loss_stages}")

    cpu = None
    if not args.no_cpu_baseline:
        if n_img == 1:
            cpu = cpu_baseline(scene, args.cpu_band_rows, args.cpu_repeats, mpix)
        else:
            # the oracle renders one camera at a time (the reference's CPU
            # loops do): camera 0 of the batch, whose rate is the batch's
            import dataclasses

            one = dataclasses.replace(scene, viewmats=scene.viewmats[:, :1], Ks=scene.Ks[:, :1],
                                      target=None if scene.target is None else scene.target[:1])
            cpu = cpu_baseline(one, args.cpu_band_rows, args.cpu_repeats, W * H / 1e6)
            cpu["sample"] = (f"camera 0 of the {n_img} (the CPU loops render one camera at a time, so this camera's "
                             f"rate is the batch's): " + cpu["sample"])

    line = {
        "metric": "fwd+bwd ms/frame & Mpix/s, 1M Gaussians SH3 1297x840; % of HBM/VALU roofline",
        "value": round(value, 2),
        "unit": "Mpix/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded numpy scene, resident in HBM)",
        "config": {"workload": f"{args.workload}: {N} Gaussians, SH degree {scene.sh_degree}, "
                               f"{scene.n_cameras}x{W}x{H}, tile {ts}, forward+backward (L1 loss)",
                   "n_gaussians": N, "image": [W, H], "n_isects": M, "sh_degree": scene.sh_degree,
                   "gaussian_order": "morton" if args.morton else "generated"},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "stages": stages,
        "accutile": accutile,
        "packed": packed,
        "l1_dssim": dssim,
        "kernels_us_per_step": {k: round(v[1] * 1000, 1) for k, v in sorted(per_step.items())},
    }
    print(json.dumps(line), flush=True)


def bucket_blocks(pairs, n, images, tw, th):
    """Grid / scatter blocks of the tile-bucket intersection and the words of
    one difference grid, as the library sizes them (bucket.hip bucket_dims)."""
    want = (pairs + 511) // 512
    gpb = min(16, max(1, (want + 1023) // 1024)) * 1024
    return images * max(1, (n + gpb - 1) // gpb), (tw + 1) * (th + 1)


def count_forward_evals(lib, torch, R, scene, means, quats, log_scales, opacity_logits, viewmats, Ks, out, W, H,
                        ts):
    """E_f, the (pixel, list entry) evaluations of the reference's forward loop
    up to each pixel's termination, counted exactly on the GPU by the
    library's counting kernel over the step's lists (the projection is
    recomputed: it is deterministic)."""
    C = viewmats.shape[1]
    with torch.no_grad():
        proj = R.activated_projection(means, quats, log_scales, opacity_logits, viewmats, Ks, W, H, eps2d=0.3,
                                      near_plane=0.01, far_plane=scene.far_plane,
                                      opacities_in_projection=scene.opacities_in_projection)
        opac = proj["opacities"][:, None].expand(-1, C, -1).contiguous()
    th, tw = out["tile_offsets"].shape[-2:]
    evals = torch.zeros(C * th * tw, dtype=torch.int64, device="cuda")
    lib.gsplat_hip_rasterize_count_evals.restype = ctypes.c_int
    P, I64, I32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32
    lib.gsplat_hip_rasterize_count_evals.argtypes = [P, P, P, P, P, P, I64, I64, I32, I32, I32, I32, I32, I64, P, P]
    m2 = proj["means2d"].contiguous()
    co = proj["conics"].contiguous()
    to = out["tile_offsets"].contiguous()
    fl = out["flatten_ids"].contiguous()
    rc = lib.gsplat_hip_rasterize_count_evals(m2.data_ptr(), co.data_ptr(), opac.data_ptr(), None, to.data_ptr(),
                                              fl.data_ptr(), C, C * scene.n, W, H, ts, tw, th, fl.numel(),
                                              evals.data_ptr(), torch.cuda.current_stream().cuda_stream)
    if rc != 0:
        raise RuntimeError("rasterize_count_evals failed")
    return int(evals.sum())


def valu_attainable_tflops(lib, torch):
    """Attainable FP32 rate of single (not packed) VALU instructions on this
    GPU: the library's FMA-chain probe (8 independent chains per lane, 8
    workgroups per CU) timed with HIP events on the launch stream."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    blocks, iters = 8 * cus, 4096
    out = torch.empty(blocks * 256, device="cuda")
    lib.gsplat_hip_valu_probe.restype = ctypes.c_int
    lib.gsplat_hip_valu_probe.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32, ctypes.c_void_p]
    stream = torch.cuda.current_stream()

    def run():
        if lib.gsplat_hip_valu_probe(out.data_ptr(), blocks, iters, stream.cuda_stream) != 0:
            raise RuntimeError("valu probe failed")

    run()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(3):
        run()
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / 3
    return blocks * 256 * 8 * 2 * iters / (ms * 1e-3) / 1e12


def lds_broadcast_attainable(lib, torch):
    """Attainable rate of LDS broadcast reads (one 16-byte record per wave
    instruction, every lane receiving it), the rasterizers' record access:
    the library's LDS probe (4 independent ds_read_b128 per step, 8
    workgroups per CU) timed with HIP events on the launch stream. Returns
    wave-level reads per second (G/s) and per CU-cycle at the 2.4 GHz peak
    engine clock."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    blocks, iters = 8 * cus, 8192
    out = torch.empty(blocks * 256, dtype=torch.int32, device="cuda")
    lib.gsplat_hip_lds_probe.restype = ctypes.c_int
    lib.gsplat_hip_lds_probe.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32, ctypes.c_void_p]
    stream = torch.cuda.current_stream()

    def run():
        if lib.gsplat_hip_lds_probe(out.data_ptr(), blocks, iters, stream.cuda_stream) != 0:
            raise RuntimeError("lds probe failed")

    run()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(3):
        run()
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / 3
    reads = blocks * 4 * iters * 4  # waves per block x steps x reads per step
    per_s = reads / (ms * 1e-3)
    return {"reads_per_s_G": round(per_s / 1e9, 2), "per_cu_cycle": round(per_s / (cus * 2.4e9), 3),
            "note": "measured wave-level ds_read_b128 broadcast reads (LDS probe) on this GPU in this run"}


def measured_traffic(workload, kernel):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 --pmc
    summary (FETCH_SIZE and WRITE_SIZE runs, each scaled by the copy-kernel
    calibration factor), or None when none was recorded for this workload."""
    path = os.path.join(ROOT, "profiles", "pmc_traffic.json")
    try:
        with open(path) as f:
            rec = json.load(f)
    except (OSError, ValueError):
        return None
    k = rec.get("kernels", {}).get(kernel)
    if rec.get("workload") != workload or not k:
        return None
    cal = rec["calibration"]
    return int((k["fetch_kib"] * cal["FETCH_SIZE"] + k["write_kib"] * cal["WRITE_SIZE"]) * 1024)


def cpu_baseline(scene, band_rows, repeats, mpix):
    """The oracle (the reference's eval_cpu loops restated in C++) on this
    host, built here at -O3 -march=native with its OpenMP loops, on the same
    frame: every per-Gaussian and per-intersection stage on the full scene,
    and rasterize forward+backward on the whole image (band_rows <= 0) or on
    a band of tile rows through the image centre scaled to the full frame by
    its share of intersections. Each stage is the median of `repeats` runs,
    first on 1 thread (the reference's loops are single-threaded), then on
    every OpenMP thread of this process. Returns ms/frame and Mpix/s."""
    import numpy as np

    sys.path.insert(0, ROOT)
    from oracle import oracle as O

    t0 = time.perf_counter()
    libs = {False: O.build_native(openmp=False), True: O.build_native(openmp=True)}
    log(f"[bench] cpu baseline: -O3 -march=native builds ready ({time.perf_counter() - t0:.1f}s)")
    clock = time.perf_counter
    W, H, ts = scene.width, scene.height, scene.tile_size
    tw, th = (W + ts - 1) // ts, (H + ts - 1) // ts
    quats = (scene.quats / np.maximum(np.linalg.norm(scene.quats, axis=-1, keepdims=True), 1e-8)).astype(np.float32)
    scales = np.exp(scene.log_scales).astype(np.float32)
    opac = (1 / (1 + np.exp(-scene.opacity_logits))).astype(np.float32)
    sh = scene.sh_degree >= 0
    bg = np.array([scene.background], np.float32)
    if band_rows <= 0 or band_rows >= th:
        r0, r1 = 0, th
    else:
        r0 = max(0, th // 2 - band_rows // 2)
        r1 = min(th, r0 + band_rows)
    info = {}

    def run_once():
        t = {}
        c = clock()
        proj = O.projection_forward(scene.means, scene.viewmats, scene.Ks, W, H, quats=quats, scales=scales,
                                    far_plane=scene.far_plane,
                                    opacities=opac if scene.opacities_in_projection else None)
        t["projection_fwd"] = clock() - c
        c = clock()
        isect = O.isect_tile(proj["means2d"], proj["radii"], proj["depths"], 1, ts, tw, th)
        offs = O.isect_offset(isect["isect_ids"], 1, tw, th)
        t["isect+sort+offsets"] = clock() - c
        M = isect["isect_ids"].size
        if sh:
            K = (scene.sh_degree + 1) ** 2
            campos = -scene.viewmats[0, 0, :3, :3].T @ scene.viewmats[0, 0, :3, 3]
            dirs = scene.means[0] - campos
            dirs = (dirs / np.maximum(np.linalg.norm(dirs, axis=-1, keepdims=True), 1e-8)).astype(np.float32)
            coeffs = np.concatenate([scene.features_dc[0][:, None], scene.features_rest[0][:, :K - 1]], 1)
            c = clock()
            colors = O.sh_forward(scene.sh_degree, dirs, coeffs)
            t["sh_fwd"] = clock() - c
            colors = np.clip(colors + 0.5, 0, 1)[None, None]
        else:
            colors = scene.colors[:, None]
        o = offs[0].ravel()
        b_start = int(o[r0 * tw])
        b_end = int(o[r1 * tw]) if r1 < th else M
        band_offs = (offs[:, r0:r1] - b_start).astype(np.int32)
        band_ids = isect["flatten_ids"][b_start:b_end]
        m2 = proj["means2d"].copy()
        m2[..., 1] -= r0 * ts
        bh = min(H, r1 * ts) - r0 * ts
        share = M / max(1, b_end - b_start)
        info.update(M=M, share=share, band=b_end - b_start)
        c = clock()
        fwd = O.raster_forward(m2, proj["conics"], colors, opac[:, None], band_offs, band_ids, W, bh, ts,
                               backgrounds=bg)
        t["raster_fwd"] = (clock() - c) * share
        if scene.target is not None:
            tgt = scene.target[:, r0 * ts:r0 * ts + bh]
            v_rc = (np.sign(fwd["render_colors"] - tgt) / (H * W * 3)).astype(np.float32)
            c = clock()
            bwd = O.raster_backward(m2, proj["conics"], colors, opac[:, None], band_offs, band_ids, W, bh, ts,
                                    fwd["render_alphas"], fwd["last_ids"], v_rc,
                                    np.zeros_like(fwd["render_alphas"]), backgrounds=bg)
            t["raster_bwd"] = (clock() - c) * share
            if sh:
                c = clock()
                O.sh_backward(scene.sh_degree, dirs, coeffs, bwd["v_colors"][0, 0])
                t["sh_bwd"] = clock() - c
            c = clock()
            O.projection_backward(scene.means, scene.viewmats, scene.Ks, W, H, proj["radii"], proj["conics"],
                                  bwd["v_means2d"], np.zeros_like(proj["depths"]), bwd["v_conics"],
                                  quats=quats, scales=scales)
            t["projection_bwd"] = clock() - c
        return t

    def timed(openmp):
        O.use_library(libs[openmp])
        info["ftz"] = O.flush_denormals()
        got = O.set_threads(0)
        runs = [run_once() for _ in range(max(1, repeats))]
        med = {k: float(np.median([r[k] for r in runs])) for k in runs[0]}
        log(f"[bench] cpu baseline, {got} thread(s), stages (s, median of {len(runs)}): " +
            ", ".join(f"{k}={v:.3f}" for k, v in med.items()))
        return got, sum(med.values()), med

    _, one_s, one_med = timed(False)
    n_all, all_s, _ = timed(True)
    if r0 == 0 and r1 == th:
        raster = "rasterize fwd+bwd on the whole image"
    else:
        raster = (f"rasterize fwd+bwd on tile rows {r0}-{r1 - 1} ({info['band']} intersections) scaled by the "
                  f"frame's intersection share x{info['share']:.2f}")
    return {"value": round(mpix / one_s, 4), "unit": "Mpix/s", "cores": 1, "kind": "port",
            "ms_per_frame": round(1000 * one_s, 1),
            "stages_ms": {k: round(1000 * v, 1) for k, v in one_med.items()},
            "sample": (f"oracle (the reference's eval_cpu loops in C++, -O3 -march=native, 1 thread, denormals "
                       f"flushed to zero: {info['ftz']}) on this host: "
                       f"projection, SH, intersection, sort, offsets and their backwards on all {scene.n} Gaussians "
                       f"/ {info['M']} intersections; {raster}; median of {max(1, repeats)} runs per stage"),
            "all_cores": {"value": round(mpix / all_s, 4), "unit": "Mpix/s", "cores": n_all,
                          "nproc": os.cpu_count(), "ms_per_frame": round(1000 * all_s, 1),
                          "note": "the same source and frame built with its OpenMP loops over Gaussians and "
                                  "tiles (atomic gradient sums in the rasterize backward, parallel stable sort), "
                                  "on every thread this process may use (OMP_NUM_THREADS)"}}


if __name__ == "__main__":
    main()
