#!/usr/bin/env python3
"""Forward+backward benchmark of the MI355X gs3d rasterizer.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]

Default workload: 3,000,000 Gaussians, SH degree 3, four 1920x1080 cameras on
a radius-5 ring around 64 Gaussian clusters (synthetic data drawn from a
fixed seed; see dsl_splat_amd.synthetic).  A step is one gs3d.rasterize call
over all four cameras plus the backward pass of loss = sum(image * W) with W
~ N(0,1) over the RGB and alpha channels; inputs are resident in HBM before
the timed region.

Prints one JSON line: the headline ms/iter (lower is better), forward and
backward ms, the HBM roofline of the dominant HBM-bound kernel (algorithmic
bytes over its HIP-event time on the launch stream), per-stage timings and
bandwidths, and a CPU baseline (the C++ oracle on the host cores over a
bounded sample).
"""

import argparse
import json
import math
import os
import sys
import time

HBM_PEAK_GBPS = 8000.0  # MI355X HBM3E, 8 TB/s
ROOFLINE_KERNEL = "gs3d::project_fwd_kernel<true> (EWA projection + metadata of every view, one launch)"
# rocprofv3 FETCH_SIZE / WRITE_SIZE summary of that kernel on the default workload.
TRAFFIC_SUMMARY = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                               "project_fwd_kernel_traffic_3M_1080p_4view.md")


def measured_traffic(workload, n):
    """HBM bytes per launch of the projection kernel, measured with rocprofv3
    counters (committed summary; default workload only), or None."""
    if workload != "sh3_1080p_4view" or n is not None or not os.path.exists(TRAFFIC_SUMMARY):
        return None
    with open(TRAFFIC_SUMMARY) as f:
        for line in f:
            if line.startswith("traffic_bytes_per_launch:"):
                return int(line.split(":", 1)[1].strip())
    return None


def parse():
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--workload", default="sh3_1080p_4view")
    p.add_argument("--n", type=int, default=None, help="override the Gaussian count")
    p.add_argument("--stage-reps", type=int, default=5)
    p.add_argument("--cpu-baseline", choices=("on", "off"), default="on")
    p.add_argument("--tile-mode", choices=("radius", "snugbox", "accutile"), default="radius",
                   help="tile mode of the timed steps (the headline is the reference's default, radius)")
    p.add_argument("--mode-steps", type=int, default=5,
                   help="steps timed in each of the other tile modes (0 skips them)")
    p.add_argument("--copy-calibration-mib", type=int, default=0,
                   help="also run one elementwise device copy (out = in * 1) of this many MiB, the known-size "
                        "kernel that scales rocprofv3 FETCH_SIZE/WRITE_SIZE readings")
    return p.parse_args()


def log(*args):
    print(*args, file=sys.stderr, flush=True)


def make_inputs(workload, n, device):
    import torch
    from dsl_splat_amd import synthetic

    scene = synthetic.make_scene(workload, n=n)
    scene.to(device)
    leaves = dict(
        means=scene.means.clone().requires_grad_(True),
        quats=scene.quats.clone().requires_grad_(True),
        scales=scene.scales.clone().requires_grad_(True),
        opacities=scene.opacities.clone().requires_grad_(True),
    )
    colors = (scene.sh_coeffs if scene.sh_coeffs is not None else scene.features).clone().requires_grad_(True)
    extra = None if scene.extra_features is None else scene.extra_features[0].clone().requires_grad_(True)
    viewmats = scene.viewmats.clone().requires_grad_(scene.pose_grad)
    torch.cuda.synchronize()
    return scene, leaves, colors, extra, viewmats


def step_fn(scene, leaves, colors, extra, viewmats, tile_mode="radius"):
    import torch
    from dsl_splat_amd import gs3d

    sh = scene.sh_coeffs is not None
    # loss = sum(image * W) over every rendered channel, taken as one dot
    # product per output plane against contiguous slices of W prepared here,
    # outside the timed step.
    W = scene.loss_weights
    D = 3 if sh else colors.shape[-1]
    w_features = W[..., :D].contiguous().reshape(-1)
    w_extra = W[..., D:-1].contiguous().reshape(-1) if extra is not None else None
    w_alpha = W[..., -1:].contiguous().reshape(-1)

    def forward():
        res = gs3d.rasterize(leaves["means"], leaves["quats"], leaves["scales"], leaves["opacities"], viewmats,
                             scene.Ks, scene.width, scene.height, features=None if sh else colors,
                             sh_coeffs=colors if sh else None, sh_degree=scene.sh_degree,
                             extra_features=extra, absgrad=scene.absgrad, tile_mode=tile_mode)
        forward.meta = res.meta
        loss = torch.dot(res.features.reshape(-1), w_features) + torch.dot(res.alpha.reshape(-1), w_alpha)
        if res.extra_features is not None:
            loss = loss + torch.dot(res.extra_features.reshape(-1), w_extra)
        return loss

    def backward(loss):
        loss.backward()
        for t in list(leaves.values()) + [colors, extra, viewmats]:
            if t is not None:
                t.grad = None

    return forward, backward


def stage_timings(scene, reps):
    """HIP-event times (ms) and algorithmic bytes of every stage, measured on
    the launch stream with the same calls the rasterizer makes."""
    import torch
    from dsl_splat_amd.gs3d import projection as gproj, render as grender
    from dsl_splat_amd.primitives import tiling
    from dsl_splat_amd.splatting import binning, cameras

    quats = scene.quats  # raw: the projection kernels normalise them, as rasterize has them do
    sh = scene.sh_coeffs
    deg = scene.sh_degree
    views, n = scene.viewmats.shape[0], len(scene.means)
    names = ("camera", "project", "order", "bin", "render_fwd", "render_bwd", "project_bwd")
    acc = {k: 0.0 for k in names}
    info = {}
    with torch.no_grad():
        for rep in range(reps + 1):
            ev = [torch.cuda.Event(enable_timing=True) for _ in range(20)]
            ev[0].record()
            full, inverse, centers, errors = cameras.launch_prepare(scene.viewmats, scene.Ks, scene.width,
                                                                    scene.height, deg is not None and deg > 0)
            ev[1].record()
            st = gproj.project_views(scene.means, quats, scene.scales, scene.opacities, scene.viewmats, full,
                                     scene.Ks, scene.width, scene.height, 0.2, math.inf, 0.0,
                                     sh=sh, sh_degree=deg or 0, camera_centers=centers if deg else None,
                                     metadata=True, normalize_quats=True)
            ev[2].record()
            order, offsets, totals = binning.order_rows(st.centers, st.radii, st.depths, scene.width,
                                                        scene.height)
            ev[3].record()
            group_pairs, count = totals.cpu().tolist()
            ev[4].record()
            ranges, ids = binning.bin_rows(st.centers, st.radii, order, offsets, group_pairs, count, scene.width,
                                           scene.height)
            ev[8].record()
            feats = st.colors if sh is not None else scene.features
            extra = scene.extra_features  # blended after the features, before alpha
            out = grender.render_views(ranges, ids, st.centers, st.conics, feats, scene.width, scene.height,
                                       extra=extra)
            ev[9].record()
            up = scene.loss_weights
            record, gf, _ = grender.backward_views(ranges, ids, st.centers, st.conics, feats,
                                                   out.transmittance, out.contributors, up, scene.width,
                                                   scene.height, extra=extra, absgrad=scene.absgrad)
            ev[10].record()
            gproj.backward_views(scene.means, quats, scene.scales, scene.opacities, scene.viewmats, full, scene.Ks,
                                 scene.width, scene.height, st.radii, record[..., 0:2], record[..., 2:6],
                                 (True, True, True, True, False, False), sh=sh, sh_degree=deg or 0,
                                 camera_centers=centers if deg else None, grad_colors=gf if sh is not None else None,
                                 need_sh=sh is not None, normalize_quats=True)
            ev[11].record()
            torch.cuda.synchronize()
            if rep == 0:
                tiles = binning.tile_count(scene.width, scene.height, views)
                groups = views * (((scene.width + 15) // 16 + 7) // 8) * (((scene.height + 15) // 16 + 7) // 8)
                info = dict(pairs=count, group_pairs=group_pairs, groups=groups, tiles=tiles,
                            group_passes=1 if groups <= 1024 else math.ceil(int(groups - 1).bit_length() / 8),
                            rows=views * n,
                            visible=int((st.radii > 0).sum()),
                            mean_contributors=float(out.contributors.float().mean()))
                continue  # warm-up repetition
            spans = {"camera": (0, 1), "project": (1, 2), "order": (2, 3), "bin": (4, 8), "render_fwd": (8, 9),
                     "render_bwd": (9, 10), "project_bwd": (10, 11)}
            for k, (a, b) in spans.items():
                acc[k] += ev[a].elapsed_time(ev[b]) / reps
        # The roofline kernel alone, one launch at a time with HIP events
        # around it, after a 2 GiB read that evicts the L2 and the Infinity
        # Cache with clean lines: its inputs then come from HBM, as they do
        # inside a step (back-to-back launches would find the 132 MB of
        # parameters cached; a fill would leave dirty lines for the kernel to
        # write back).  The read (~0.3 ms) outlasts the host's enqueueing of
        # the launch, so no idle time falls between the events.
        launches = 10
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        flush = torch.ones(512 << 20, dtype=torch.float32, device=quats.device)
        # (without coefficients: the projection kernel only, no colour launch)
        project = lambda: gproj.project_views(scene.means, quats, scene.scales, scene.opacities, scene.viewmats, full,
                                              scene.Ks, scene.width, scene.height, 0.2, math.inf, 0.0,
                                              metadata=True, normalize_quats=True)
        project()
        acc["project_kernel"] = 0.0
        for _ in range(launches):
            flush.amax()
            e0.record()
            project()
            e1.record()
            torch.cuda.synchronize()
            acc["project_kernel"] += e0.elapsed_time(e1) / launches
        del flush
        # Contribution statistics (a masked count and a weighted sum over
        # per-view pixel maps) observed by the forward blend, against the
        # plain forward blend, both back-to-back.
        from dsl_splat_amd.statistics import PreparedStatistics
        g = torch.Generator().manual_seed(9)
        hw = scene.width * scene.height
        pv = torch.stack([(torch.rand((views, hw), generator=g) < 0.5).float(), torch.rand((views, hw), generator=g)],
                         1).to(quats.device)
        stats = PreparedStatistics((0, 1), pv, torch.zeros((views, 1, n), dtype=torch.int32, device=quats.device),
                                   torch.zeros((views, 1, n), device=quats.device))
        for key, kw in (("render_fwd_kernel", {}), ("render_fwd_stats_kernel", {"statistics": stats})):
            blend = lambda: grender.render_views(ranges, ids, st.centers, st.conics, feats, scene.width,
                                                 scene.height, **kw)
            blend()
            e0.record()
            for _ in range(5):
                blend()
            e1.record()
            torch.cuda.synchronize()
            acc[key] = e0.elapsed_time(e1) / 5
    # Algorithmic bytes of every stage: what its kernels must read and write
    # once each.
    M, S, T, R = info["pairs"], info["group_pairs"], info["tiles"], info["rows"]
    K = 0 if sh is None else sh.shape[-2]
    sh_in = 0 if sh is None else (n if sh.ndim == 3 else views * n) * K * 3 * 4
    by = {
        # params 44 B/G (+ SH once for all views) in; per view centers 8, conics+opacity 16, radii 4,
        # tiles 4, depth 4, means2d 8, meta opacity 4, meta conic 12 (+ colour 12) out
        "project": n * 44 + sh_in + views * n * (60 + (12 if sh is not None else 0)),
        # keys and records (depth 4 + centre 8 + radius 4 in, key 4 + record 8 out), 4 radix passes
        # over (key, record) (24 per pass), group counts (record 8 in, count 4 out), inclusive scan
        # (4 in, 4 out)
        "order": R * (28 + 4 * 24 + 12 + 8),
        # items: records and offsets in (12 B/row), items out (8 B/item); group sort (16 B/item/pass,
        # one 10-bit pass up to 1024 groups, whose digit scan gives the group ranges, else 8-bit
        # passes and a range search over the items, 8 B/item); count and write passes read items
        # (2 x 8 B); ids out (4 B/pair); tile totals/starts/ranges (16 B/tile)
        "bin": R * 12 + S * (8 + 16 * info["group_passes"] + (16 if info["group_passes"] == 1 else 24))
               + M * 4 + T * 16,
        # params 44 + SH 4K*3 in, per view radii 4 + centre/conic grads 24 (+ colour grads 12) in;
        # grads 44 + SH out
        "project_bwd": n * 88 + 2 * sh_in + views * n * (28 + (12 if sh is not None else 0)),
    }
    return acc, by, info


def cpu_baseline(scene):
    """The C++ oracle (fwd+bwd, OpenMP on the host cores) on one of the
    workload's cameras at full N and resolution; the per-iteration figure is
    scaled by the camera count (cameras are independent in the algorithm)."""
    import numpy as np
    import torch

    import oracle

    oracle.build()
    cores = len(os.sched_getaffinity(0))
    oracle.set_threads(cores)
    npy = lambda t: t.detach().cpu().numpy()
    qn = npy(torch.nn.functional.normalize(scene.quats, dim=-1))
    V, K = npy(scene.viewmats[:1]), npy(scene.Ks[:1])
    W, H = scene.width, scene.height
    sh = scene.sh_coeffs
    deg = scene.sh_degree
    means, scales, opac = npy(scene.means), npy(scene.scales), npy(scene.opacities)
    shn = None if sh is None else npy(sh)
    feats = None if scene.features is None else npy(scene.features)
    up = npy(scene.loss_weights[:1])
    t0 = time.perf_counter()
    full, inverse, centers, err = oracle.camera_prepare(V, K, W, H, bool(deg))
    proj = oracle.project_fwd(means, qn, scales, opac, V, full, K, W, H, sh=shn, sh_degree=deg or 0,
                              camera_centers=centers if deg else None, metadata=True)
    offsets, total = oracle.scan_i32(proj["tiles"].ravel())
    keys, vals = oracle.emit_keys(proj["centers"], proj["radii"], proj["depths"], offsets, total, W, H)
    T = ((W + 15) // 16) * ((H + 15) // 16)
    sk, sv = oracle.sort_pairs(keys, vals, 32 + int(T).bit_length())
    ranges = oracle.tile_ranges(sk, T)
    blended = proj["colors"] if shn is not None else feats
    image, final_t, contrib = oracle.render_fwd(W, H, ranges, sv, proj["centers"], proj["conics"], blended)
    t1 = time.perf_counter()
    g = oracle.render_bwd(W, H, ranges, sv, proj["centers"], proj["conics"], blended, final_t, contrib, up,
                          absgrad=scene.absgrad)
    oracle.project_bwd(means, qn, scales, opac, V, full, K, W, H, proj["radii"], g["centers"], g["conics"],
                       sh=shn, sh_degree=deg or 0, camera_centers=centers if deg else None,
                       grad_colors=g["features"] if shn is not None else None)
    t2 = time.perf_counter()
    views = scene.viewmats.shape[0]
    return dict(value=round((t2 - t0) * 1000.0 * views, 1), unit="ms", cores=cores, kind="port",
                sample=f"C++ oracle fwd+bwd on camera 1 of {views} (full N, {W}x{H}), "
                       f"{(t2 - t0):.1f} s measured, scaled x{views} to one iteration; "
                       f"fwd {(t1 - t0) * 1000 * views:.0f} ms + bwd {(t2 - t1) * 1000 * views:.0f} ms",
                fwd_ms=round((t1 - t0) * 1000.0 * views, 1), bwd_ms=round((t2 - t1) * 1000.0 * views, 1))


def main():
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}, WORLD_SIZE={world}); "
              "multi-GPU sharding of this path is a design note, not a built feature", file=sys.stderr)
        sys.exit(2)
    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        sys.exit(1)
    device = torch.device("cuda", 0)
    torch.cuda.set_device(device)
    log(f"[bench] building inputs: {args.workload}")
    scene, leaves, colors, extra, viewmats = make_inputs(args.workload, args.n, device)
    forward, backward = step_fn(scene, leaves, colors, extra, viewmats, args.tile_mode)
    log(f"[bench] warmup {args.warmup}")
    for _ in range(args.warmup):
        backward(forward())
    torch.cuda.synchronize()
    log(f"[bench] timing {args.steps} steps")
    # Steps follow each other as in a training loop: no synchronisation
    # between them (each forward synchronises once, on its pair totals), so
    # the host prepares step i+1 while step i's backward runs.  Per-step
    # forward/backward spans come from events read after the final sync.
    events = [tuple(torch.cuda.Event(enable_timing=True) for _ in range(3)) for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for e0, e1, e2 in events:
        e0.record()
        loss = forward()
        e1.record()
        backward(loss)
        e2.record()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms = (t1 - t0) * 1000.0 / args.steps
    fwd_ms = sum(e0.elapsed_time(e1) for e0, e1, _ in events)
    bwd_ms = sum(e1.elapsed_time(e2) for _, e1, e2 in events)
    modes = {args.tile_mode: dict(ms=round(ms, 3), pairs=int(forward.meta["tiles_per_gauss"].sum()))}
    for mode in ("radius", "snugbox", "accutile"):
        if mode == args.tile_mode or args.mode_steps <= 0:
            continue
        log(f"[bench] tile_mode={mode}: {args.mode_steps} steps")
        f_m, b_m = step_fn(scene, leaves, colors, extra, viewmats, mode)
        b_m(f_m())
        torch.cuda.synchronize()
        ta = time.perf_counter()
        for _ in range(args.mode_steps):
            b_m(f_m())
        torch.cuda.synchronize()
        modes[mode] = dict(ms=round((time.perf_counter() - ta) * 1000.0 / args.mode_steps, 3),
                           pairs=int(f_m.meta["tiles_per_gauss"].sum()))
    if args.copy_calibration_mib > 0:
        src = torch.ones(args.copy_calibration_mib << 18, device=device)
        dst = torch.empty_like(src)
        torch.mul(src, 1.0, out=dst)
        torch.cuda.synchronize()
        log(f"[bench] copy calibration: {src.numel() * 4} bytes read and written")
        del src, dst
    log(f"[bench] {ms:.3f} ms/iter; stage timings")
    stages, by, info = stage_timings(scene, args.stage_reps)
    s13 = ("project", "order", "bin")
    t13 = sum(stages[k] for k in s13)
    b13 = sum(by[k] for k in s13)
    kernels = ("project_kernel", "render_fwd_kernel", "render_fwd_stats_kernel")
    per_stage = {k: dict(ms=round(v, 4)) for k, v in stages.items() if k not in kernels}
    for k in by:
        per_stage[k]["gbps"] = round(by[k] / (stages[k] * 1e-3) / 1e9, 1)
        per_stage[k]["frac"] = round(by[k] / (stages[k] * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4)
        per_stage[k]["bytes"] = by[k]
    # The roofline object is the projection forward kernel: HBM-bound, one
    # launch per step, params 44 B/G in and 60 B per view out (the colour
    # kernel's bytes are in the "project" stage); every other stage's
    # bandwidth is in "stages".
    n_g, n_v = len(scene.means), scene.viewmats.shape[0]
    kernel_bytes = n_g * 44 + n_v * n_g * 60
    kernel_ms = stages["project_kernel"]
    achieved = kernel_bytes / (kernel_ms * 1e-3) / 1e9
    cpu = None
    if args.cpu_baseline == "on":
        log("[bench] CPU baseline (oracle)")
        cpu = cpu_baseline(scene)
    views = scene.viewmats.shape[0]
    result = {
        "metric": "3DGS fwd+bwd ms/iter @3M Gaussians 1080p SH3; sort/proj HBM GB/s",
        "value": round(ms, 3),
        "unit": "ms",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 3),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded)",
        "config": {
            "workload": f"{args.workload}: N={len(scene.means)}, {views} cameras, {scene.width}x{scene.height}, "
                        f"SH degree {scene.sh_degree}, fwd+bwd of sum(image*W)",
            "gaussians": len(scene.means), "cameras": views, "width": scene.width, "height": scene.height,
            "sh_degree": scene.sh_degree, "tile_mode": args.tile_mode, "pairs": info["pairs"],
            "group_pairs": info["group_pairs"],
            "visible_rows": info["visible"],
        },
        "fwd_ms": round(fwd_ms / args.steps, 3),
        "bwd_ms": round(bwd_ms / args.steps, 3),
        "roofline": {
            "bound": "hbm",
            "kernel": ROOFLINE_KERNEL,
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBPS, 4),
            "traffic": measured_traffic(args.workload, args.n),
            "ms": round(kernel_ms, 4),
            "bytes": kernel_bytes,
        },
        "stages_1_3": {"ms": round(t13, 4), "bytes": b13, "gbps": round(b13 / (t13 * 1e-3) / 1e9, 1),
                       "frac": round(b13 / (t13 * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4)},
        "stages": per_stage,
        "tile_modes": modes,
        "statistics": {"requests": "masked count + weighted sum, per-view maps",
                       "render_fwd_ms": round(stages["render_fwd_kernel"], 4),
                       "render_fwd_stats_ms": round(stages["render_fwd_stats_kernel"], 4)},
        "cpu_baseline": cpu,
    }
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
